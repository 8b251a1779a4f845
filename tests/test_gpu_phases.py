"""GPU parity of the separately callable backward phases (t2t_attn_bwd_preprocess,
t2t_attn_bwd_dkdv, t2t_attn_bwd_dq; the reference's sdpa_dense_backward steps,
torch/_higher_order_ops/flex_attention.py:825-994) against the float64 oracle,
and against the fused t2t_attn_bwd on the same buffers.

The fused call computes Delta inside its dQ launch, the phases in a launch of
their own, with a different fp32 summation order, so the two agree to float32
rounding of Delta rather than bit for bit; dK / dV are each deterministic.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attn_oracle as ao
from oracle import mask_oracle as mo
from tagseq2tagseq_amd.attention import BwdPhases, attn_fwd
from tagseq2tagseq_amd.block_mask import build_block_mask
from tests.helpers import assert_close, random_row, to_dev_words

pytestmark = pytest.mark.gpu

TOL = 2e-2  # bf16 parity bound of this path (abs and rel)


def _case(B, Hq, Hkv, T, D, words, seed, device):
    rng = np.random.default_rng(seed)
    rows = [random_row(T, rng, words=words, uncovered=True, max_doc=150) for _ in range(B)]
    doc = torch.stack([torch.from_numpy(r[0]) for r in rows]).to(device)
    if words:
        qb = torch.stack([to_dev_words(r[1], device) for r in rows])
        kb = torch.stack([to_dev_words(r[2], device) for r in rows])
        bm = build_block_mask(doc, qb, kb)
    else:
        bm = build_block_mask(doc)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, T, D, generator=g).to(torch.bfloat16).to(device)
    k = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).to(device)
    do = torch.randn(B, Hq, T, D, generator=g).to(torch.bfloat16).to(device)
    dense = np.stack([mo.dense_mask(*r) for r in rows])
    return q, k, v, do, bm, dense


@pytest.mark.parametrize("B,Hq,Hkv,T,D,words", [(2, 4, 2, 384, 64, 2), (1, 4, 1, 333, 128, 1),
                                                 (1, 2, 2, 256, 128, 0)])
def test_phases_against_oracle_and_fused(B, Hq, Hkv, T, D, words, gpu_device):
    q, k, v, do, bm, dense = _case(B, Hq, Hkv, T, D, words, seed=T + D, device=gpu_device)
    scale = 1.0 / math.sqrt(D)
    out, lse2 = attn_fwd(q, k, v, bm, scale)
    label = f"B{B} H{Hq}/{Hkv} T{T} D{D} W{words}"

    ph = BwdPhases(q, k, v, out, do, lse2, bm, scale)
    ph.preprocess()
    # Delta = rowsum(O * dO) of the bf16 rows, accumulated in fp32
    delta_ref = (out.float() * do.float()).sum(-1)
    assert_close(ph.delta, delta_ref, 1e-4, 1e-4, f"delta {label}")
    ph.dkdv()
    ph.dq_pass()
    dq_p, dk_p, dv_p = ph.dq.clone(), ph.dk.clone(), ph.dv.clone()

    qn, kn, vn, don = (t.float().cpu().numpy() for t in (q, k, v, do))
    o_ref, lse_ref = ao.attention_fwd(qn, kn, vn, dense)
    dq_ref, dk_ref, dv_ref = ao.attention_bwd(qn, kn, vn, o_ref, don, lse_ref, dense)
    assert_close(dq_p, torch.from_numpy(dq_ref), TOL, TOL, f"phases dq {label}")
    assert_close(dk_p, torch.from_numpy(dk_ref), TOL, TOL, f"phases dk {label}")
    assert_close(dv_p, torch.from_numpy(dv_ref), TOL, TOL, f"phases dv {label}")

    # the phases again on the same buffers: bit-identical (no atomics)
    ph.preprocess()
    ph.dkdv()
    ph.dq_pass()
    assert torch.equal(ph.dq, dq_p) and torch.equal(ph.dk, dk_p) and torch.equal(ph.dv, dv_p)

    # the fused call: Delta from its dQ launch, then dK / dV
    ph.whole()
    assert_close(ph.delta, delta_ref, 1e-4, 1e-4, f"fused delta {label}")
    for name, got, want in (("dq", ph.dq, dq_p), ("dk", ph.dk, dk_p), ("dv", ph.dv, dv_p)):
        assert_close(got, want, 1e-2, 1e-2, f"fused vs phases {name} {label}")
