"""t2t_attn_bwd_noalloc (the backward whose Delta workspace is the library's
file-scope device array) against t2t_attn_bwd with a caller workspace, both
called through the C ABI: outputs bitwise equal on two calls in a row, the
second with a smaller input, in bf16 and float32; and the host-side rejection
of shapes past the array."""
import ctypes
import math

import pytest
import torch

from tagseq2tagseq_amd import _lib
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.attention import attn_fwd
from tagseq2tagseq_amd.block_mask import build_block_mask
from tagseq2tagseq_amd.mask_creators import TokenLists

DEV = torch.device("cuda:0")
DTYPES = {torch.bfloat16: _lib.T2T_DTYPE_BF16, torch.float32: _lib.T2T_DTYPE_F32}


def _case(T, Hq, Hkv, D, dtype, seed):
    row = synth.config_rows(3, seed=seed, T=T)[0]
    lists = TokenLists(T, [row.spans], DEV, words=row.words, link_rows=[row.link_rows])
    bm = build_block_mask(*lists.build())
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, Hq, T, D, generator=g).to(dtype).to(DEV)
    k = torch.randn(1, Hkv, T, D, generator=g).to(dtype).to(DEV)
    v = torch.randn(1, Hkv, T, D, generator=g).to(dtype).to(DEV)
    do = torch.randn(1, Hq, T, D, generator=g).to(dtype).to(DEV)
    out, lse2 = attn_fwd(q, k, v, bm, 1.0 / math.sqrt(D))
    return q, k, v, out.contiguous(), do, lse2, bm


def _grads(which, q, k, v, out, do, lse2, bm):
    """dq, dk, dv from t2t_attn_bwd (which='caller') or t2t_attn_bwd_noalloc."""
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    dq, dk, dv = (torch.full_like(t, float("nan")) for t in (q, k, v))
    views = [_lib.tensor_struct(t) for t in (q, k, v, out, do)]
    gviews = [_lib.tensor_struct(t) for t in (dq, dk, dv)]
    refs = [ctypes.byref(x) for x in views]
    grefs = [ctypes.byref(x) for x in gviews]
    tail = (B, Hq, Hkv, T, D, DTYPES[q.dtype], 1.0 / math.sqrt(D), ctypes.byref(bm.c_struct()),
            ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream))
    L = _lib.lib()
    if which == "caller":
        delta = torch.empty((B, Hq, T), dtype=torch.float32, device=DEV)
        rc = L.t2t_attn_bwd(*refs, lse2.data_ptr(), delta.data_ptr(), *grefs, *tail)
    else:
        rc = L.t2t_attn_bwd_noalloc(*refs, lse2.data_ptr(), *grefs, *tail)
    _lib.check(rc, which)
    torch.cuda.synchronize()
    return dq, dk, dv


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_backward_matches_caller_workspace(dtype):
    # the second call is smaller: the array keeps the first call's rows past
    # its end, which the second call must neither need nor read
    for T, Hq, Hkv, D, seed in ((1000, 4, 2, 128, 11), (300, 2, 1, 64, 12)):
        case = _case(T, Hq, Hkv, D, dtype, seed)
        want = _grads("caller", *case)
        got = _grads("noalloc", *case)
        for name, a, b in zip(("dq", "dk", "dv"), got, want):
            assert torch.isfinite(b).all(), f"{name} T={T}: reference not finite"
            assert torch.equal(a, b), (f"{name} T={T} {dtype}: max diff "
                                       f"{(a.float() - b.float()).abs().max().item():.3g}")


def test_noalloc_backward_rejects_shapes_past_the_array():
    """B * Hq * T above the 4 * 2^20 rows of the static array is refused on the
    host, before any device call (runs without a GPU)."""
    L = _lib.lib()
    t = _lib.T2TTensor(16, 128, 128, 128)
    r = ctypes.byref(t)
    rc = L.t2t_attn_bwd_noalloc(r, r, r, r, r, 16, r, r, r, 1, 64, 64, 65537, 128,
                                _lib.T2T_DTYPE_BF16, 0.1, None, None)
    assert rc == -1
    assert b"static workspace" in L.t2t_last_error()
