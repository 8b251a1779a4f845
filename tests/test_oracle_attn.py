"""CPU tests of the float64 attention oracle (oracle/attn_oracle.py).

Pins: torch's eager flex_attention on CPU (the arithmetic the reference calls,
torch/_higher_order_ops/flex_attention.py:202-294, 825-994) with the restated
mask_mod, closed forms (diagonal-only mask, fully masked rows), GQA as
repeat_interleave, and central finite differences of the backward.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attn_oracle as ao
from oracle import mask_oracle as mo
from tagseq2tagseq_amd import synth
from tests.helpers import random_row, row_arrays


def _torch_flex(q, k, v, do, doc, qb, kb, gqa=False):
    from torch.nn.attention.flex_attention import create_block_mask, flex_attention
    T = q.shape[2]
    mod = mo.torch_mask_mod(torch.from_numpy(doc),
                            None if qb is None else torch.from_numpy(qb.view(np.int64)),
                            None if kb is None else torch.from_numpy(kb.view(np.int64)))
    bm = create_block_mask(mod, None, None, T, T, device="cpu")
    qt, kt, vt = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
    out, lse = flex_attention(qt, kt, vt, block_mask=bm, enable_gqa=gqa, return_lse=True)
    out.backward(torch.from_numpy(do))
    return (out.detach().numpy(), lse.detach().numpy(), qt.grad.numpy(), kt.grad.numpy(),
            vt.grad.numpy())


def _inputs(B, Hq, Hkv, T, D, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((B, Hq, T, D)), rng.standard_normal((B, Hkv, T, D)),
            rng.standard_normal((B, Hkv, T, D)), rng.standard_normal((B, Hq, T, D)))


@pytest.mark.parametrize("name,row,Hq,Hkv", [
    ("doc_causal", lambda: row_arrays(synth.lognormal_docs(256, 40.0, 1.0, 200, seed=1)), 2, 2),
    ("cross_doc_link", lambda: row_arrays(synth.linked_lognormal_docs(300, 40.0, 1.0, 200, 0.3, seed=2)), 2, 2),
    ("gqa_ragged_words", lambda: random_row(200, np.random.default_rng(3), words=2, uncovered=True), 4, 2),
])
def test_oracle_matches_torch_eager_flex(name, row, Hq, Hkv):
    doc, qb, kb = row()
    T = doc.shape[0]
    q, k, v, do = _inputs(1, Hq, Hkv, T, 16, seed=5)
    dense = mo.dense_mask(doc, qb, kb)[None]
    o, lse = ao.attention_fwd(q, k, v, dense)
    dq, dk, dv = ao.attention_bwd(q, k, v, o, do, lse, dense)
    to, tl, tdq, tdk, tdv = _torch_flex(q, k, v, do, doc, qb, kb, gqa=Hq != Hkv)
    for a, b in ((o, to), (lse, tl), (dq, tdq), (dk, tdk), (dv, tdv)):
        np.testing.assert_allclose(a, b, rtol=1e-9, atol=1e-9)


def test_diagonal_only_mask_closed_form():
    T, D = 40, 8
    doc = np.arange(T, dtype=np.int32)  # every token its own document
    q, k, v, do = _inputs(1, 1, 1, T, D, seed=6)
    dense = mo.dense_mask(doc)[None]
    assert np.array_equal(dense[0], np.eye(T, dtype=bool))
    o, lse = ao.attention_fwd(q, k, v, dense)
    np.testing.assert_allclose(o, v, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse[0, 0], (q[0, 0] * k[0, 0]).sum(-1) / math.sqrt(D), atol=1e-12)
    dq, dk, dv = ao.attention_bwd(q, k, v, o, do, lse, dense)
    np.testing.assert_allclose(dv, do, atol=1e-12)
    assert np.abs(dq).max() < 1e-12 and np.abs(dk).max() < 1e-12


def test_fully_masked_rows_give_zero_and_neg_inf():
    T, D = 10, 4
    q, k, v, do = _inputs(1, 1, 1, T, D, seed=7)
    mask = np.tri(T, dtype=bool)
    mask[3] = False
    o, lse = ao.attention_fwd(q, k, v, mask[None])
    assert np.all(o[0, 0, 3] == 0) and lse[0, 0, 3] == -np.inf
    dq, dk, dv = ao.attention_bwd(q, k, v, o, do, lse, mask[None])
    assert np.all(dq[0, 0, 3] == 0)
    assert np.isfinite(dk).all() and np.isfinite(dv).all()


def test_softmax_rows_sum_to_one():
    doc, qb, kb = row_arrays(synth.linked_lognormal_docs(128, 20.0, 1.0, 60, 0.4, seed=9))
    T, D = 128, 8
    q, k, _, _ = _inputs(1, 1, 1, T, D, seed=8)
    dense = mo.dense_mask(doc, qb, kb)[None]
    ones = np.ones((1, 1, T, 1))
    o, _ = ao.attention_fwd(q, k, ones, dense)
    np.testing.assert_allclose(o[..., 0], 1.0, atol=1e-12)


def test_gqa_equals_repeated_heads():
    doc, qb, kb = random_row(96, np.random.default_rng(2), words=1)
    dense = mo.dense_mask(doc, qb, kb)[None]
    q, k, v, do = _inputs(1, 4, 2, 96, 8, seed=11)
    o, lse = ao.attention_fwd(q, k, v, dense)
    kr, vr = np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1)
    o2, lse2 = ao.attention_fwd(q, kr, vr, dense)
    np.testing.assert_allclose(o, o2, atol=1e-12)
    dq, dk, dv = ao.attention_bwd(q, k, v, o, do, lse, dense)
    dq2, dk2, dv2 = ao.attention_bwd(q, kr, vr, o2, do, lse2, dense)
    np.testing.assert_allclose(dq, dq2, atol=1e-12)
    np.testing.assert_allclose(dk, dk2.reshape(1, 2, 2, 96, 8).sum(2), atol=1e-12)
    np.testing.assert_allclose(dv, dv2.reshape(1, 2, 2, 96, 8).sum(2), atol=1e-12)


def test_backward_finite_differences():
    T, D = 7, 3
    doc = np.array([1, 1, 1, 2, 2, 3, 3], np.int32)
    qb = np.zeros((1, T), np.uint64); kb = np.zeros((1, T), np.uint64)
    qb[0, 5:] = 1; kb[0, :3] = 1  # doc 3 may read doc 1
    dense = mo.dense_mask(doc, qb, kb)[None]
    q, k, v, do = _inputs(1, 1, 1, T, D, seed=12)

    def loss(q_, k_, v_):
        o, _ = ao.attention_fwd(q_, k_, v_, dense)
        return float((o * do).sum())

    o, lse = ao.attention_fwd(q, k, v, dense)
    grads = ao.attention_bwd(q, k, v, o, do, lse, dense)
    eps = 1e-6
    for gi, x in enumerate((q, k, v)):
        num = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            xp = x.copy(); xp[idx] += eps
            xm = x.copy(); xm[idx] -= eps
            args_p = [q, k, v]; args_p[gi] = xp
            args_m = [q, k, v]; args_m[gi] = xm
            num[idx] = (loss(*args_p) - loss(*args_m)) / (2 * eps)
        np.testing.assert_allclose(grads[gi], num, rtol=1e-6, atol=1e-7)


def test_useful_pairs_counts_allowed_entries():
    doc, qb, kb = row_arrays(synth.config_rows(3, seed=0, T=1024)[0])
    dense = mo.dense_mask(doc, qb, kb)
    assert ao.useful_pairs(dense[None], B=2) == 2 * int(dense.sum())
    assert int(dense.sum()) == int(mo.tile_counts(doc, qb, kb).sum())
