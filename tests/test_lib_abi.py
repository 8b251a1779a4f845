"""The C-ABI library loads, exports every symbol include/t2t_attn.h declares,
and rejects bad arguments before touching the GPU; the Python layer refuses
CPU tensors (there is no CPU fallback)."""
import ctypes
import os

import pytest
import torch

from tagseq2tagseq_amd import _lib


def test_library_built_and_loads():
    assert os.path.exists(_lib.LIB_PATH), "run python -m tagseq2tagseq_amd.build"
    assert b"gfx950" in _lib.lib().t2t_version()


def test_exports_every_header_symbol():
    names = _lib.header_functions()
    assert {"t2t_mask_meta", "t2t_attn_fwd", "t2t_attn_bwd", "t2t_attn_bwd_preprocess",
            "t2t_attn_bwd_dkdv", "t2t_attn_bwd_dq", "t2t_last_error", "t2t_version"} <= set(names)
    lib = _lib.lib()
    for n in names:
        assert hasattr(lib, n), n


# The argument-check tests pass placeholder device pointers that the library
# must reject before any launch; they run only where no GPU is visible.
no_gpu = pytest.mark.skipif(torch.cuda.is_available(),
                            reason="placeholder-pointer checks run on CPU-only hosts")


def _dummy_view():
    return _lib.T2TTensor(0x1000, 0, 0, 128)


def _err():
    return _lib.lib().t2t_last_error().decode()


@no_gpu
def test_fwd_rejects_unsupported_head_dim():
    v = _dummy_view()
    m = _lib.T2TBlockMaskC()
    rc = _lib.lib().t2t_attn_fwd(ctypes.byref(v), ctypes.byref(v), ctypes.byref(v), ctypes.byref(v),
                                 ctypes.c_void_p(0x1000), 1, 2, 2, 256, 96, 0, 0.1,
                                 ctypes.byref(m), None)
    assert rc == -2 and "head dim" in _err()


@no_gpu
def test_fwd_rejects_bad_gqa_and_dtype():
    v = _dummy_view()
    m = _lib.T2TBlockMaskC()
    lib = _lib.lib()
    rc = lib.t2t_attn_fwd(*[ctypes.byref(v)] * 4, ctypes.c_void_p(0x1000), 1, 3, 2, 256, 128, 0,
                          0.1, ctypes.byref(m), None)
    assert rc == -1 and "GQA" in _err()
    rc = lib.t2t_attn_fwd(*[ctypes.byref(v)] * 4, ctypes.c_void_p(0x1000), 1, 2, 2, 256, 128, 7,
                          0.1, ctypes.byref(m), None)
    assert rc == -2 and "dtype" in _err()


@no_gpu
def test_attention_rejects_nonpositive_scales():
    """Zero, negative, denormal, infinite and NaN scales are refused by every
    attention entry point before any launch."""
    v = _dummy_view()
    m = _lib.T2TBlockMaskC()
    lib = _lib.lib()
    P = ctypes.c_void_p(0x1000)
    for scale in (0.0, -0.125, 1e-40, float("inf"), float("nan")):
        rc = lib.t2t_attn_fwd(*[ctypes.byref(v)] * 4, P, 1, 2, 2, 256, 128, 0, scale,
                              ctypes.byref(m), None)
        assert rc == -1 and "scale" in _err(), scale
        rc = lib.t2t_attn_bwd(*[ctypes.byref(v)] * 5, P, P, *[ctypes.byref(v)] * 3,
                              1, 2, 2, 256, 128, 0, scale, ctypes.byref(m), None)
        assert rc == -1 and "scale" in _err(), scale
        rc = lib.t2t_attn_bwd_dkdv(*[ctypes.byref(v)] * 4, P, P, ctypes.byref(v), ctypes.byref(v),
                                   1, 2, 2, 256, 128, 0, scale, ctypes.byref(m), None)
        assert rc == -1 and "scale" in _err(), scale
        rc = lib.t2t_attn_bwd_dq(*[ctypes.byref(v)] * 4, P, P, ctypes.byref(v),
                                 1, 2, 2, 256, 128, 0, scale, ctypes.byref(m), None)
        assert rc == -1 and "scale" in _err(), scale
        rc = lib.t2t_attn_bwd_noalloc(*[ctypes.byref(v)] * 5, P, *[ctypes.byref(v)] * 3,
                                      1, 2, 2, 256, 128, 0, scale, ctypes.byref(m), None)
        assert rc == -1 and "scale" in _err(), scale


@no_gpu
def test_clock_probe_argument_checks():
    lib = _lib.lib()
    khz = ctypes.c_int32(0)
    assert lib.t2t_clock_probe(None, 100, ctypes.byref(khz), None) == -1
    assert lib.t2t_clock_probe(ctypes.c_void_p(0x1000), 0, ctypes.byref(khz), None) == -1
    assert "iters" in _err()
    assert lib.t2t_clock_probe(ctypes.c_void_p(0x1000), 100, None, None) == -1


@no_gpu
def test_float32_dtype_rules():
    """float32 (dtype 1) is accepted by t2t_attn_fwd / t2t_attn_bwd with
    4-byte-element alignment rules, and rejected by the separate phases."""
    lib = _lib.lib()
    m = _lib.T2TBlockMaskC()
    f32_only = _lib.T2TTensor(0x1000, 0, 0, 132)  # row stride 132: 16-byte rows only as float32
    rc = lib.t2t_attn_fwd(*[ctypes.byref(f32_only)] * 4, ctypes.c_void_p(0x1000), 1, 2, 2, 256,
                          128, 0, 0.1, ctypes.byref(m), None)
    assert rc == -1 and "view" in _err()
    rc = lib.t2t_attn_fwd(*[ctypes.byref(f32_only)] * 4, ctypes.c_void_p(0x1000), 1, 2, 2, 256,
                          128, 1, 0.1, None, None)
    assert rc == -1 and "mask" in _err()  # the view passed; the NULL mask is what fails
    rc = lib.t2t_attn_bwd(*[ctypes.byref(f32_only)] * 5, ctypes.c_void_p(0x1000),
                          ctypes.c_void_p(0x1000), *[ctypes.byref(f32_only)] * 3,
                          1, 2, 2, 256, 128, 1, 0.1, None, None)
    assert rc == -1 and "mask" in _err()
    v = _dummy_view()
    rc = lib.t2t_attn_bwd_dkdv(*[ctypes.byref(v)] * 4, ctypes.c_void_p(0x1000),
                               ctypes.c_void_p(0x1000), ctypes.byref(v), ctypes.byref(v),
                               1, 2, 2, 256, 128, 1, 0.1, ctypes.byref(m), None)
    assert rc == -2 and "dtype" in _err()
    rc = lib.t2t_attn_bwd_preprocess(ctypes.byref(v), ctypes.byref(v), ctypes.c_void_p(0x1000),
                                     1, 2, 256, 128, 1, None)
    assert rc == -2 and "dtype" in _err()


@no_gpu
def test_bwd_rejects_null_mask():
    v = _dummy_view()
    rc = _lib.lib().t2t_attn_bwd(*[ctypes.byref(v)] * 5, ctypes.c_void_p(0x1000),
                                 ctypes.c_void_p(0x1000), *[ctypes.byref(v)] * 3,
                                 1, 2, 2, 256, 128, 0, 0.1, None, None)
    assert rc == -1 and "mask" in _err()


@no_gpu
def test_mask_meta_argument_checks():
    lib = _lib.lib()
    out = _lib.T2TBlockMaskC(1, 2)
    assert lib.t2t_mask_meta(None, None, None, 1, 0, 0, None, ctypes.byref(out), None) == 0  # T = 0
    assert lib.t2t_mask_meta(None, None, None, 1, 256, 9, None, ctypes.byref(out), None) == -2
    assert "words" in _err()
    # capacity check: 2 tiles need 3 bitmap slots
    out.tile_bits_slots = 2
    rc = lib.t2t_mask_meta(ctypes.c_void_p(0x1000), None, None, 1, 256, 0, ctypes.c_void_p(0x1000),
                           ctypes.byref(out), None)
    assert rc == -1 and "slots" in _err()
    out = _lib.T2TBlockMaskC(1, 3, tile_bits_slots=100)
    rc = lib.t2t_mask_meta(ctypes.c_void_p(0x1000), None, None, 1, 256, 0, ctypes.c_void_p(0x1000),
                           ctypes.byref(out), None)
    assert rc == -1 and "nt=" in _err()
    # bitmap slots are int32 indices: 65536 tiles a side need 2^31 + 2^15 slots
    nt = 65536
    out = _lib.T2TBlockMaskC(1, nt, tile_bits_slots=1 << 40)
    rc = lib.t2t_mask_meta(ctypes.c_void_p(0x1000), None, None, 1, nt * 128, 0,
                           ctypes.c_void_p(0x1000), ctypes.byref(out), None)
    assert rc == -2 and "int32" in _err()


def test_python_layer_refuses_cpu_tensors():
    from tagseq2tagseq_amd.block_mask import build_block_mask
    from tagseq2tagseq_amd.mask_creators import create_doc_causal_block_mask
    with pytest.raises(RuntimeError, match="GPU"):
        build_block_mask(torch.zeros(256, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="GPU"):
        create_doc_causal_block_mask(torch.zeros((1, 256), dtype=torch.long), [])


def test_flex_attention_validation_on_cpu():
    from tagseq2tagseq_amd.attention import flex_attention
    q = torch.zeros(1, 2, 256, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="block_mask is required"):
        flex_attention(q, q, q)
    with pytest.raises(NotImplementedError):
        flex_attention(q, q, q, score_mod=lambda s, b, h, i, j: s, block_mask=object())


@no_gpu
def test_token_inputs_argument_checks():
    lib = _lib.lib()
    P = ctypes.c_void_p(0x1000)
    # empty work is a no-op
    assert lib.t2t_token_inputs(None, None, 0, None, None, 0, None, 0, 16, 0, None, None, None,
                                None) == 0
    assert lib.t2t_token_inputs(P, P, 4, None, None, 0, None, 1, -1, 0, P, None, None, None) == -1
    assert "negative" in _err()
    assert lib.t2t_token_inputs(P, P, 4, None, None, 0, None, 1, 64, 9, P, P, P, None) == -2
    assert "words" in _err()
    assert lib.t2t_token_inputs(P, P, 4, None, None, 0, None, 1, 64, 0, None, None, None,
                                None) == -1
    assert "doc" in _err()
    # grants without their count, and grant words without words
    assert lib.t2t_token_inputs(P, P, 4, P, None, 8, None, 1, 64, 1, P, P, P, None) == -1
    assert "both" in _err()
    assert lib.t2t_token_inputs(P, P, 4, P, P, 8, None, 1, 64, 0, P, None, None, None) == -1
    assert "words > 0" in _err()
    assert lib.t2t_token_inputs(P, P, 4, None, None, 0, None, 1, 64, 2, P, None, P, None) == -1
    assert "q_bits" in _err()


def test_qkv_rope_argument_checks():
    lib = _lib.lib()
    P = ctypes.c_void_p(0x1000)
    view = _lib.T2TTensor(0x1000, 0, 64 * 32, 64)
    bad = _lib.T2TTensor(0x1008, 0, 64 * 32, 64)  # misaligned
    v = ctypes.byref(view)
    # empty work is a no-op
    assert lib.t2t_qkv_rope(None, 0, 0, 0, 32, 4, 64, None, None, 0, 0, None, None, None, None) == 0
    assert lib.t2t_qkv_rope(P, 0, 768, 1, -1, 4, 64, P, P, 32, 0, v, v, v, None) == -1
    assert "negative" in _err()
    assert lib.t2t_qkv_rope(P, 0, 768, 1, 32, 4, 40, P, P, 32, 0, v, v, v, None) == -2
    assert "multiple of 16" in _err()
    # positions past the table
    assert lib.t2t_qkv_rope(P, 0, 768, 1, 32, 4, 64, P, P, 40, 9, v, v, v, None) == -1
    assert "table rows" in _err()
    # token rows overlap (stride below 3 H D)
    assert lib.t2t_qkv_rope(P, 0, 512, 1, 32, 4, 64, P, P, 32, 0, v, v, v, None) == -1
    assert "3*H*D" in _err()
    assert lib.t2t_qkv_rope(P, 0, 768, 1, 32, 4, 64, P, P, 32, 0, v, ctypes.byref(bad), v,
                            None) == -1
    assert "view" in _err()
    assert lib.t2t_qkv_rope(P, 0, 768, 1, 32, 4, 64, None, P, 32, 0, v, v, v, None) == -1
    assert "NULL" in _err()
    assert lib.t2t_qkv_rope_backward(v, v, v, P, P, 32, 0, 1, 32, 4, 64, ctypes.c_void_p(0x1004),
                                     0, 768, None) == -1
    assert "aligned" in _err()
    assert lib.t2t_qkv_rope_backward(v, v, None, P, P, 32, 0, 1, 32, 4, 64, P, 0, 768,
                                     None) == -1
    assert "view" in _err()


def test_attn_decode_argument_checks():
    lib = _lib.lib()
    P = ctypes.c_void_p(0x1000)
    view = _lib.T2TTensor(0x1000, 0, 64 * 128, 64)
    v = ctypes.byref(view)
    ws = lib.t2t_attn_decode_workspace(1, 4, 1, 1000, 64)
    assert ws == 4 * 1 * 4 * 1 * 4 * (64 + 2)  # ceil(1000 / 256) chunks of (D + 2) floats

    def call(**kw):
        a = dict(q=v, k=v, v=v, o=v, lse2=P, key_doc=P, key_bits=None, key_stride=1000, q_pos=P,
                 q_doc=P, q_bits=None, mask_batch=1, words=0, B=1, Hq=4, Hkv=4, Tq=1,
                 Tkv=1000, D=64, dtype=0, scale=0.125, ws=P, ws_bytes=ws, stream=None)
        a.update(kw)
        return lib.t2t_attn_decode(*a.values())

    assert call(Tq=0) == 0  # no rows: no-op
    assert call(D=96) == -2 and "head dim" in _err()
    assert call(dtype=1) == -2
    assert call(Hq=6) == -1 and "multiple" in _err()
    assert call(Hq=8, Hkv=1, Tq=2) == -2 and "exceeds" in _err()
    assert call(mask_batch=2) == -1 and "broadcast" in _err()
    assert call(key_stride=999) == -1 and "key_stride" in _err()
    assert call(words=1) == -1 and "NULL" in _err()
    assert call(ws_bytes=ws - 4) == -1 and "workspace" in _err()
    assert call(words=9) == -2


def test_rows_linear_argument_checks():
    """t2t_rows_linear / t2t_rows_qkv_rope reject bad shapes and pointers
    before any launch (no GPU needed)."""
    lib = _lib.lib()
    P = ctypes.c_void_p(0x1000)

    def lin(M=1, K=768, N=768, x=P, xs=768, w=P, nw=None, ndt=0, ep=0, res=None, rs=0, y=P,
            ys=768, sk=None, sks=0, sw=None, swdt=0):
        return lib.t2t_rows_linear(x, xs, M, K, w, N, nw, ndt, 1e-6, ep, res, rs, sk, sks, sw,
                                   swdt, y, ys, None)

    assert lin(M=9) == -2 and "rows" in _err()
    assert lin(M=-1) == -2
    assert lin(K=0, xs=16) == -2 and "outside" in _err()
    assert lin(K=4104, xs=4104) == -2
    assert lin(N=0) == -1
    assert lin(x=None) == -1 and "NULL" in _err()
    assert lin(x=ctypes.c_void_p(0x1001)) == -1 and "aligned" in _err()
    assert lin(nw=ctypes.c_void_p(0x1002), ndt=1) == -1 and "misaligned" in _err()
    assert lin(xs=760) == -1 and "stride" in _err()
    assert lin(nw=P, ndt=2) == -2 and "dtype" in _err()
    assert lin(ep=3) == -2 and "epilogue" in _err()
    assert lin(y=None) == -1
    assert lin(ys=700) == -1 and "stride" in _err()
    assert lin(ep=1) == -1 and "res" in _err()
    assert lin(ep=1, res=P, rs=100) == -1
    assert lin(M=0) == 0  # nothing to do, nothing launched
    assert lin(sw=P) == -1 and "add epilogue" in _err()
    assert lin(ep=1, res=P, rs=768, sk=P, sks=768) == -1 and "without a skip weight" in _err()
    assert lin(ep=1, res=P, rs=768, sw=P, swdt=2) == -2 and "dtype" in _err()
    assert lin(ep=1, res=P, rs=768, sk=P, sks=700, sw=P) == -1 and "skip row stride" in _err()
    assert lin(M=0, ep=1, res=P, rs=768, sk=P, sks=768, sw=P) == 0

    v = _dummy_view()

    def qkv(M=1, K=768, H=12, D=64, pos=None, pos0=0, rows=128, cache=128, views=(v, v, v)):
        return lib.t2t_rows_qkv_rope(P, K, M, K, P, None, 0, 1e-6, H, D, P, P, rows, pos, pos0,
                                     *[ctypes.byref(t) for t in views], cache, None)

    assert qkv(D=63) == -2
    assert qkv(H=0) == -2
    assert qkv(M=9) == -2
    assert qkv(pos0=127, M=2) == -1 and "exceed" in _err()
    assert qkv(pos0=126, M=2, cache=127) == -1 and "cache rows" in _err()
    bad = _lib.T2TTensor(0, 0, 0, 64)
    assert qkv(views=(v, bad, v)) == -1 and "view" in _err()
    assert qkv(M=0) == 0


def test_first_input_diff_argument_checks():
    lib = _lib.lib()
    P = ctypes.c_void_p(0x1000)
    args = lambda words=1, n=16, out=P, sa=16, sb=16, q=P: (  # noqa: E731
        P, P, P, P, q, q, q, q, sa, sb, words, n, out, None)
    assert lib.t2t_first_input_diff(*args(words=9)) == -1 and "words" in _err()
    assert lib.t2t_first_input_diff(*args(n=-1)) == -1
    assert lib.t2t_first_input_diff(*args(out=None)) == -1 and "out" in _err()
    assert lib.t2t_first_input_diff(*args(q=None)) == -1 and "grant-word" in _err()
    assert lib.t2t_first_input_diff(*args(sa=8)) == -1 and "stride" in _err()


def test_ce_rows_argument_checks():
    lib = _lib.lib()
    P = ctypes.c_void_p(0x1000)
    args = lambda rows=4, V=10, ld=16, lg=P, sc=P: (  # noqa: E731
        lg, lg, rows, V, ld, P, -100, sc, P, None)
    assert lib.t2t_ce_rows(*args(ld=12)) == -1 and "ld" in _err()
    assert lib.t2t_ce_rows(*args(V=0)) == -1
    assert lib.t2t_ce_rows(*args(V=17)) == -1
    assert lib.t2t_ce_rows(*args(rows=-1)) == -1
    assert lib.t2t_ce_rows(*args(sc=None)) == -1 and "NULL" in _err()
    assert lib.t2t_ce_rows(*args(lg=ctypes.c_void_p(0x1002))) == -1 and "aligned" in _err()
    assert lib.t2t_ce_rows(*args(rows=0)) == 0


def test_swiglu_argument_checks():
    lib = _lib.lib()
    P = ctypes.c_void_p(0x1000)
    assert lib.t2t_swiglu(P, 32, P, 16, 4, 12, None) == -1 and "H" in _err()
    assert lib.t2t_swiglu(P, 24, P, 16, 4, 16, None) == -1 and "stride" in _err()
    assert lib.t2t_swiglu(None, 32, P, 16, 4, 16, None) == -1 and "NULL" in _err()
    assert lib.t2t_swiglu(ctypes.c_void_p(0x1008), 32, P, 16, 4, 16, None) == -1
    assert lib.t2t_swiglu_backward(P, 32, P, 8, P, 32, 4, 16, None) == -1 and "stride" in _err()
    assert lib.t2t_swiglu(P, 32, P, 16, 0, 16, None) == 0


def test_wgrad_argument_checks():
    lib = _lib.lib()
    P = ctypes.c_void_p(0x1000)
    ws = lib.t2t_wgrad_workspace(768, 768, 16384)
    assert ws > 0 and ws % (768 * 768 * 4) == 0
    assert lib.t2t_wgrad_workspace(100, 768, 64) == 0
    assert lib.t2t_wgrad_workspace(128, 128, 32) == 0
    args = lambda M=128, N=128, K=64, lda=128, ldb=128, dt=0, ws=1 << 20, a=P: (  # noqa: E731
        a, lda, P, ldb, P, dt, M, N, K, P, ws, None)
    assert lib.t2t_wgrad(*args(M=100)) == -2 and "128" in _err()
    assert lib.t2t_wgrad(*args(K=96)) == -2
    assert lib.t2t_wgrad(*args(dt=3)) == -1
    assert lib.t2t_wgrad(*args(lda=120)) == -1 and "lda" in _err()
    assert lib.t2t_wgrad(*args(ws=16)) == -1 and "workspace" in _err()
    assert lib.t2t_wgrad(*args(a=None)) == -1 and "NULL" in _err()
