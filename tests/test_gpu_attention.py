"""GPU parity of the masked-attention forward / backward kernels.

Small cases: against the float64 CPU oracle (oracle/attn_oracle.py).
Full-size configs: against a chunked fp32 torch reference on the GPU over
every head (every KV head's dK / dV complete).  bf16 tolerance 2e-2 (abs and rel), float32 1e-4: the
parity bounds set for this path.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attn_oracle as ao
from oracle import mask_oracle as mo
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.attention import flex_attention
from tagseq2tagseq_amd.block_mask import build_block_mask
from tests.helpers import (assert_close, random_row, row_arrays, to_dev_words,
                           torch_ref_attention)

pytestmark = pytest.mark.gpu

ATOL = RTOL = 2e-2
F32_TOL = 1e-4


def _mask_from_rows(rows_np, device):
    doc = torch.stack([torch.from_numpy(r[0]) for r in rows_np]).to(device)
    if rows_np[0][1] is None:
        return build_block_mask(doc)
    qb = torch.stack([to_dev_words(r[1], device) for r in rows_np])
    kb = torch.stack([to_dev_words(r[2], device) for r in rows_np])
    return build_block_mask(doc, qb, kb)


def _inputs(B, Hq, Hkv, T, D, seed, device, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, T, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
    do = torch.randn(B, Hq, T, D, generator=g).to(dtype)
    return [t.to(device) for t in (q, k, v, do)]


def _oracle_check(rows_np, B, Hq, Hkv, T, D, seed, device, bwd=True, dtype=torch.bfloat16):
    """Kernels vs the float64 oracle on the same inputs: 2e-2 (abs and rel)
    for bf16, 1e-4 for float32 (the parity bounds set for this path); LSE 1e-3 / 1e-4."""
    tol, lse_tol = (ATOL, 1e-3) if dtype == torch.bfloat16 else (F32_TOL, F32_TOL)
    bm = _mask_from_rows(rows_np, device)
    q, k, v, do = _inputs(B, Hq, Hkv, T, D, seed, device, dtype)
    q.requires_grad_(True); k.requires_grad_(True); v.requires_grad_(True)
    out, lse = flex_attention(q, k, v, block_mask=bm, enable_gqa=Hq != Hkv, return_lse=True)
    assert out.dtype == dtype
    dense = np.stack([mo.dense_mask(*r) for r in rows_np])
    qn, kn, vn, don = (t.detach().float().cpu().numpy() for t in (q, k, v, do))
    o_ref, lse_ref = ao.attention_fwd(qn, kn, vn, dense)
    label = f"B{B} H{Hq}/{Hkv} T{T} D{D} {dtype}"
    assert_close(out.detach(), torch.from_numpy(o_ref), tol, tol, f"out {label}")
    assert_close(lse.detach(), torch.from_numpy(lse_ref), lse_tol, lse_tol, f"lse {label}")
    if not bwd:
        return
    out.backward(do)
    dq_ref, dk_ref, dv_ref = ao.attention_bwd(qn, kn, vn, o_ref, don, lse_ref, dense)
    assert q.grad.dtype == k.grad.dtype == v.grad.dtype == dtype
    assert_close(q.grad, torch.from_numpy(dq_ref), tol, tol, f"dq {label}")
    assert_close(k.grad, torch.from_numpy(dk_ref), tol, tol, f"dk {label}")
    assert_close(v.grad, torch.from_numpy(dv_ref), tol, tol, f"dv {label}")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("T", [128, 256, 1000])
def test_doc_causal_small(T, D, gpu_device):
    rows = [row_arrays(synth.lognormal_docs(T, 60.0, 1.0, 300, seed=T + D))]
    _oracle_check(rows, 1, 2, 2, T, D, seed=1, device=gpu_device)


@pytest.mark.parametrize("D", [64, 128])
def test_cross_doc_link_small(D, gpu_device):
    rows = [row_arrays(synth.linked_lognormal_docs(512, 50.0, 1.0, 300, 0.3, seed=3))]
    _oracle_check(rows, 1, 2, 2, 512, D, seed=2, device=gpu_device)


def test_gqa_and_batch_masks(gpu_device):
    rng = np.random.default_rng(11)
    rows = [random_row(384, rng, words=2, uncovered=True, max_doc=120) for _ in range(2)]
    _oracle_check(rows, 2, 4, 2, 384, 64, seed=4, device=gpu_device)


def test_gqa_grouped_dispatch(gpu_device):
    """Hkv * tiles a multiple of 8: the forward and dQ launches place each
    KV head's query heads on one XCD (head_and_slot's grouped mapping);
    batch 2 and G = 4 so every (head, tile) work-group is checked."""
    rng = np.random.default_rng(21)
    rows = [random_row(512, rng, words=1, uncovered=False, max_doc=200) for _ in range(2)]
    _oracle_check(rows, 2, 8, 2, 512, 128, seed=21, device=gpu_device)


@pytest.mark.parametrize("B,Hq,Hkv,T,D", [
    (2, 6, 2, 512, 64),    # G = 3, Hkv * tiles = 8: grouped placement, rounds of 24 slots
    (1, 8, 1, 1024, 128),  # G = 8, Hkv * tiles = 8: grouped placement, rounds of 64 slots
    (1, 6, 2, 384, 128),   # G = 3, Hkv * tiles = 6: heads fastest
])
def test_gqa_group_sizes(B, Hq, Hkv, T, D, gpu_device):
    """Group sizes other than 2 and 4 on both of head_and_slot's paths:
    every (query head, tile) work-group must land on a distinct slot."""
    rng = np.random.default_rng(Hq * 100 + T)
    rows = [random_row(T, rng, words=2, uncovered=True, max_doc=300) for _ in range(B)]
    _oracle_check(rows, B, Hq, Hkv, T, D, seed=Hq + T, device=gpu_device)


@pytest.mark.parametrize("scale", [0.02, 0.5])
def test_explicit_scale(scale, gpu_device):
    """A non-default scale reaches the forward's score scaling and the
    backward's -LSE / scale row seeds; against the oracle at the same scale.
    At 0.5 (5.7x the default for D = 128: scores of standard deviation ~5.7)
    the softmax is sharp and the gradients span a wide range, so their bf16
    rounding (of P, dS and the outputs) is bounded relative to each tensor's
    largest entry; the element-wise bound holds at the small scale.
    Non-positive scales are refused."""
    rng = np.random.default_rng(31)
    rows = [random_row(320, rng, words=1, uncovered=True, max_doc=100)]
    bm = _mask_from_rows(rows, gpu_device)
    q, k, v, do = _inputs(1, 4, 2, 320, 128, 31, gpu_device)
    q.requires_grad_(True); k.requires_grad_(True); v.requires_grad_(True)
    out, lse = flex_attention(q, k, v, block_mask=bm, scale=scale, enable_gqa=True, return_lse=True)
    out.backward(do)
    dense = np.stack([mo.dense_mask(*r) for r in rows])
    qn, kn, vn, don = (t.detach().float().cpu().numpy() for t in (q, k, v, do))
    o_ref, lse_ref = ao.attention_fwd(qn, kn, vn, dense, scale)
    dq_ref, dk_ref, dv_ref = ao.attention_bwd(qn, kn, vn, o_ref, don, lse_ref, dense, scale)
    assert_close(out.detach(), torch.from_numpy(o_ref), ATOL, RTOL, f"out scale {scale}")
    assert_close(lse.detach(), torch.from_numpy(lse_ref), 1e-3, 1e-3, f"lse scale {scale}")
    for name, got, ref in (("dq", q.grad, dq_ref), ("dk", k.grad, dk_ref), ("dv", v.grad, dv_ref)):
        ref = torch.from_numpy(ref)
        atol = ATOL if scale < 0.1 else ATOL * float(ref.abs().max())
        assert_close(got, ref, atol, RTOL, f"{name} scale {scale}")
    with pytest.raises(ValueError, match="scale"):
        flex_attention(q, k, v, block_mask=bm, scale=-scale, enable_gqa=True)


def test_ragged_uncovered_tokens(gpu_device):
    rng = np.random.default_rng(12)
    rows = [random_row(333, rng, words=1, uncovered=True, max_doc=90)]
    _oracle_check(rows, 1, 2, 1, 333, 128, seed=5, device=gpu_device)


def test_config1_shape_bf16(gpu_device):
    rows = [row_arrays(r) for r in synth.config_rows(1, seed=0)]
    _oracle_check(rows, 1, 4, 4, 1024, 64, seed=0, device=gpu_device)


def test_config1_f32(gpu_device):
    """Config 1 as specified: float32 doc_causal B1 H4 T1024 D64 (forward,
    plus the float32 backward on the same inputs)."""
    rows = [row_arrays(r) for r in synth.config_rows(1, seed=0)]
    _oracle_check(rows, 1, 4, 4, 1024, 64, seed=0, device=gpu_device, dtype=torch.float32)


@pytest.mark.parametrize("D", [64, 128])
def test_f32_doc_causal_and_cross_doc_link(D, gpu_device):
    rows = [row_arrays(synth.lognormal_docs(384, 60.0, 1.0, 300, seed=D))]
    _oracle_check(rows, 1, 2, 2, 384, D, seed=6, device=gpu_device, dtype=torch.float32)
    rows = [row_arrays(synth.linked_lognormal_docs(512, 50.0, 1.0, 300, 0.3, seed=4))]
    _oracle_check(rows, 1, 2, 2, 512, D, seed=7, device=gpu_device, dtype=torch.float32)


def test_f32_gqa_batch_masks_and_ragged(gpu_device):
    rng = np.random.default_rng(21)
    rows = [random_row(384, rng, words=2, uncovered=True, max_doc=120) for _ in range(2)]
    _oracle_check(rows, 2, 4, 2, 384, 64, seed=8, device=gpu_device, dtype=torch.float32)
    rows = [random_row(333, rng, words=1, uncovered=True, max_doc=90)]
    _oracle_check(rows, 1, 4, 1, 333, 128, seed=9, device=gpu_device, dtype=torch.float32)


@pytest.mark.parametrize("D", [64, 128])
def test_backward_is_deterministic(D, gpu_device):
    """dQ, dK, dV bitwise equal across runs (no atomics; fixed summation
    orders), for both dK/dV kernels (D = 64 and D = 128)."""
    rows = [row_arrays(r) for r in synth.config_rows(3, seed=0, T=2048)]
    bm = _mask_from_rows(rows, gpu_device)
    q, k, v, do = _inputs(1, 4, 2, 2048, D, 7, gpu_device)
    grads = []
    for _ in range(2):
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        flex_attention(qq, kk, vv, block_mask=bm, enable_gqa=True).backward(do)
        grads.append((qq.grad.clone(), kk.grad.clone(), vv.grad.clone()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


@pytest.mark.parametrize("cfg", [2, 3, 4])
def test_full_size_against_torch_fp32(cfg, gpu_device):
    c = synth.CONFIGS[cfg]
    B, Hq, Hkv, T, D = c["B"], c["Hq"], c["Hkv"], c["T"], c["D"]
    rows = [row_arrays(r) for r in synth.config_rows(cfg, seed=0)]
    bm = _mask_from_rows(rows, gpu_device)
    q, k, v, do = _inputs(B, Hq, Hkv, T, D, cfg, gpu_device)
    q.requires_grad_(True); k.requires_grad_(True); v.requires_grad_(True)
    out, lse = flex_attention(q, k, v, block_mask=bm, enable_gqa=Hq != Hkv, return_lse=True)
    out.backward(do)
    # every query head of every batch row: each KV head then has all of its
    # query heads evaluated, so every dk / dv is complete
    heads = list(range(Hq))
    masks = []
    for r in rows:
        masks.append((torch.from_numpy(r[0]).to(gpu_device), to_dev_words(r[1], gpu_device),
                      to_dev_words(r[2], gpu_device)))
    ref = torch_ref_attention(q.detach(), k.detach(), v.detach(), do, masks, heads=heads)
    for (b, h), o_ref in ref["o"].items():
        assert_close(out[b, h].detach(), o_ref, ATOL, RTOL, f"cfg{cfg} out b{b} h{h}")
        assert_close(lse[b, h].detach(), ref["lse"][(b, h)], 1e-3, 1e-3, f"cfg{cfg} lse b{b} h{h}")
        assert_close(q.grad[b, h], ref["dq"][(b, h)], ATOL, RTOL, f"cfg{cfg} dq b{b} h{h}")
    # each checked KV head has all of its query heads evaluated -> complete dk / dv
    for (b, hk), dk_ref in ref["dk"].items():
        assert_close(k.grad[b, hk], dk_ref, ATOL, RTOL, f"cfg{cfg} dk b{b} hk{hk}")
        assert_close(v.grad[b, hk], ref["dv"][(b, hk)], ATOL, RTOL, f"cfg{cfg} dv b{b} hk{hk}")
    assert len(ref["o"]) == B * Hq and len(ref["dk"]) == B * Hkv


@pytest.mark.parametrize("seed", range(40))
def test_fuzz_shapes_and_masks(seed, gpu_device):
    """Seeded random shapes and masks against the float64 oracle: T from 1 to
    900 (ragged, below one tile included), batch 1-2 with per-row masks, GQA
    ratios 1/2/4, D 64/128, 0-3 grant words (bit 63 included), uncovered
    tokens, bf16 and float32 (at their bounds), forward and backward."""
    rng = np.random.default_rng(1000 + seed)
    T = int(rng.choice([1, 2, 31, 127, 128, 129]) if seed < 3 else rng.integers(130, 900))
    B = int(rng.integers(1, 3))
    Hkv = int(rng.integers(1, 3))
    Hq = Hkv * int(rng.choice([1, 2, 4]))
    D = int(rng.choice([64, 128]))
    words = int(rng.integers(0, 4))
    rows = [random_row(T, rng, words=words, uncovered=bool(rng.random() < 0.5),
                       max_doc=int(rng.integers(8, 300))) for _ in range(B)]
    dtype = torch.float32 if seed % 3 == 2 else torch.bfloat16
    _oracle_check(rows, B, Hq, Hkv, T, D, seed=seed, device=gpu_device, dtype=dtype)


def test_max_size_T65536(gpu_device):
    """The largest shape exercised: T = 65536 (512 tiles per side, 376
    documents, 6 grant words, ~1 GB of tile-bitmap slots) with the config-4
    generator, one GQA group (Hq 4 / Hkv 1, D 128) so dK/dV are complete;
    every output and gradient row against the chunked fp32 torch reference."""
    T, Hq, Hkv, D = 65536, 4, 1, 128
    rows = [row_arrays(r) for r in synth.config_rows(4, seed=1, T=T)]
    bm = _mask_from_rows(rows, gpu_device)
    assert bm.num_tiles == T // 128
    q, k, v, do = _inputs(1, Hq, Hkv, T, D, 11, gpu_device)
    q.requires_grad_(True); k.requires_grad_(True); v.requires_grad_(True)
    out = flex_attention(q, k, v, block_mask=bm, enable_gqa=True)
    out.backward(do)
    masks = [(torch.from_numpy(rows[0][0]).to(gpu_device), to_dev_words(rows[0][1], gpu_device),
              to_dev_words(rows[0][2], gpu_device))]
    ref = torch_ref_attention(q.detach(), k.detach(), v.detach(), do, masks)
    for (b, h), o_ref in ref["o"].items():
        assert_close(out[b, h].detach(), o_ref, ATOL, RTOL, f"T64k out h{h}")
        assert_close(q.grad[b, h], ref["dq"][(b, h)], ATOL, RTOL, f"T64k dq h{h}")
    assert_close(k.grad[0, 0], ref["dk"][(0, 0)], ATOL, RTOL, "T64k dk")
    assert_close(v.grad[0, 0], ref["dv"][(0, 0)], ATOL, RTOL, "T64k dv")


@pytest.mark.parametrize("name", ["cross_doc_link_T130_gqa", "doc_causal_T96_d128"])
def test_golden_fixture(name, gpu_device):
    import os
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", f"attn_{name}.npz"))
    qb = f["q_bits"] if "q_bits" in f else None
    kb = f["kv_bits"] if "kv_bits" in f else None
    bm = build_block_mask(torch.from_numpy(f["doc"]).to(gpu_device), to_dev_words(qb, gpu_device),
                          to_dev_words(kb, gpu_device))
    def dev(n):
        return torch.from_numpy(f[n].view(np.int16)).view(torch.bfloat16).to(gpu_device)
    q, k, v, do = dev("q"), dev("k"), dev("v"), dev("do")
    q.requires_grad_(True); k.requires_grad_(True); v.requires_grad_(True)
    out, lse = flex_attention(q, k, v, block_mask=bm, enable_gqa=q.shape[1] != k.shape[1],
                              return_lse=True)
    out.backward(do)
    for got, ref in ((out, "o"), (q.grad, "dq"), (k.grad, "dk"), (v.grad, "dv")):
        assert_close(got.detach(), torch.from_numpy(f[ref].astype(np.float32)), ATOL, RTOL, f"{name} {ref}")
    assert_close(lse.detach(), torch.from_numpy(f["lse"]), 1e-3, 1e-3, f"{name} lse")
