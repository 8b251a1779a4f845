"""The pack cost models of the density-aware rank ordering against measured
attention time on the GPU: eight configs[2]-generator packs (T 16384, H 16,
D 128, bf16) are timed fwd+bwd, and the exact pair count (pack_pairs, host)
and the tile-class cost (tile_cost, from the metadata pass) must rank them as
the measurements do (Spearman rank correlation) and fit them linearly."""
import math

import numpy as np
import pytest
import torch

from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.attention import attn_bwd, attn_fwd
from tagseq2tagseq_amd.block_mask import build_block_mask
from tagseq2tagseq_amd.mask_creators import TokenLists
from tagseq2tagseq_amd.schedule import pack_pairs, tile_cost

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _ranks(x):
    return np.argsort(np.argsort(np.asarray(x)))


def _spearman(a, b):
    return float(np.corrcoef(_ranks(a), _ranks(b))[0, 1])


def test_cost_models_rank_packs_like_measured_time():
    T, H, D = 16384, 16, 128
    g = torch.Generator().manual_seed(0)
    q, k, v, do = (torch.randn(1, H, T, D, generator=g).to(torch.bfloat16).to(DEV)
                   for _ in range(4))
    scale = 1.0 / math.sqrt(D)
    # packs of different density: link probability and document length vary
    packs = [synth.linked_lognormal_docs(T, med, 1.0, 2048, p, seed=200 + i)
             for i, (med, p) in enumerate([(150, 0.05), (350, 0.15), (250, 0.3), (600, 0.1),
                                           (400, 0.4), (200, 0.15), (800, 0.3), (300, 0.6)])]
    pairs, tcost, ms = [], [], []
    for row in packs:
        lists = TokenLists(T, [row.spans], DEV, words=row.words, link_rows=[row.link_rows])
        bm = build_block_mask(*lists.build())

        def step():
            out, lse2 = attn_fwd(q, k, v, bm, scale)
            attn_bwd(q, k, v, out, do, lse2, bm, scale)

        step()
        torch.cuda.synchronize()
        times = []
        for _ in range(5):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            step()
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b))
        ms.append(float(np.median(times)))
        pairs.append(pack_pairs(T, row.spans, row.link_rows))
        tcost.append(tile_cost(bm))
    assert max(ms) > 1.5 * min(ms), f"packs too alike to test a cost model: {ms}"
    rho_p, rho_t = _spearman(pairs, ms), _spearman(tcost, ms)
    x = np.asarray(pairs, dtype=np.float64)
    A = np.stack([x, np.ones_like(x)], 1)
    y = np.asarray(ms)
    coef, *_ = np.linalg.lstsq(A, y, rcond=None)
    r2 = 1.0 - ((y - A @ coef) ** 2).sum() / ((y - y.mean()) ** 2).sum()
    assert rho_p >= 0.85, f"pair count ranks packs with rho {rho_p:.3f} (ms {ms}, pairs {pairs})"
    assert rho_t >= 0.85, f"tile cost ranks packs with rho {rho_t:.3f} (ms {ms}, costs {tcost})"
    assert r2 >= 0.8 and coef[0] > 0, f"linear fit of time on pairs: R^2 {r2:.3f}, slope {coef[0]:.3g}"
