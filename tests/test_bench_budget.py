"""bench.executed_work (the step's executed-MFMA budget) against a brute-force
count of the non-empty MFMA blocks of the dense mask (CPU)."""
import numpy as np
import pytest
import torch
from torch.nn.attention.flex_attention import create_block_mask

import bench
from oracle import mask_oracle as mo
from tagseq2tagseq_amd.block_mask import from_torch_block_mask
from tests.helpers import random_row, to_dev_words


@pytest.mark.parametrize("T,words,D,Hq", [(700, 1, 128, 3), (1024, 2, 64, 2), (129, 0, 128, 1)])
def test_executed_work_counts_nonempty_blocks(T, words, D, Hq):
    doc, qb, kb = random_row(T, np.random.default_rng(T + words), words=words, max_doc=180)
    mod = mo.torch_mask_mod(torch.from_numpy(doc), to_dev_words(qb, "cpu"), to_dev_words(kb, "cpu"))
    bm = from_torch_block_mask(create_block_mask(mod, None, None, T, T, device="cpu"))
    dense = mo.dense_mask(doc, qb, kb)
    n_pairs = int(dense.sum())
    nt = (T + 127) // 128
    pad = np.zeros((nt * 128, nt * 128), dtype=bool)
    pad[:T, :T] = dense
    blk = pad.reshape(nt * 4, 32, nt * 4, 32).any((1, 3)).sum()      # 32 x 32 blocks
    sk = 64 if D == 64 else 32                                        # forward step keys
    units = pad.reshape(nt * 4, 32, nt * 128 // sk, sk).any((1, 3)).sum()  # 32 queries x sk keys
    # per step: a score MFMA per 32-key block and 16-wide k-step over D, a
    # P V MFMA per 16-key k-step and 32-wide output column tile
    fwd_unit = (sk // 32) * (D // 16) + (sk // 16) * (D // 32)
    ew = bench.executed_work(bm, 1, Hq, D, n_pairs, config=0)
    assert ew["attn_fwd_bf16_kernel"]["mfma_per_launch"] == units * Hq * fwd_unit
    assert ew[bench.dkdv_kernel_name(D)]["mfma_per_launch"] == blk * Hq * D // 4
    assert ew["bwd_dq_kernel"]["mfma_per_launch"] == blk * Hq * 3 * D // 16
    step = ew["step"]
    useful = 14 * D * n_pairs * Hq
    executed = 32768 * (units * fwd_unit + blk * D // 4 + blk * 3 * D // 16) * Hq
    assert step["executed_over_useful"] == pytest.approx(executed / useful, abs=1e-4)
    assert step["busy_needed_for_50pct"] == pytest.approx(0.5 * executed / useful, abs=1e-4)
    assert "profile_mfma" not in ew  # no committed summary for config 0
