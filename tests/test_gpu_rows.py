"""GPU parity of the fused few-row linear maps (t2t_rows_linear,
t2t_rows_qkv_rope) against a float32 torch restatement of the unfused
sequence they replace: RMSNorm (rounded to bf16), nn.Linear (products summed
in float32 from the bf16 operands, rounded to bf16), then the residual add,
SwiGLU or rotary embedding with the same rounding points.

The kernels sum over K in an order of their own, so a product can differ
from the float32 reference's by one bf16 rounding; the bound is 1e-2
relative to the output scale (about 2.5 bf16 ulps) plus 1e-3 absolute.
"""
import math

import pytest
import torch

from tagseq2tagseq_amd.modules import RMSNorm
from tagseq2tagseq_amd.rope import qkv_rope, rope_tables
from tagseq2tagseq_amd.rows import rows_linear, rows_qkv_rope

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 1e-2


def _norm_ref(x, norm):
    if norm is None:
        return x
    xf = x.float()
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + norm.eps)
    return (xf * r * norm.weight.float()).to(torch.bfloat16)


def _lin_ref(x, w):
    return (x.float() @ w.float().t()).to(torch.bfloat16)


def _assert_close(got, ref, what):
    got, ref = got.float(), ref.float()
    scale = ref.abs().max().item()
    err = (got - ref).abs().max().item()
    assert err <= TOL * scale + 1e-3, f"{what}: max err {err:.4g} (scale {scale:.3g})"


def _norm(K, dtype, seed):
    n = RMSNorm(K).to(DEV)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        n.weight.copy_(1.0 + 0.1 * torch.randn(K, generator=g))
    return n.to(dtype)


@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("K,N", [(64, 40), (768, 768), (768, 1001), (2048, 768), (4096, 264),
                                 (682, 256), (1365, 512), (7, 9)])
@pytest.mark.parametrize("epilogue", ["store", "add", "swiglu"])
def test_rows_linear_matches_torch(M, K, N, epilogue):
    g = torch.Generator().manual_seed(M * 7 + K + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    rows_w = 2 * N if epilogue == "swiglu" else N
    w = (torch.randn(rows_w, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(DEV)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    for norm in (None, _norm(K, torch.bfloat16, 1), _norm(K, torch.float32, 2)):
        got = rows_linear(x, w, norm=norm, epilogue=epilogue,
                          res=res if epilogue == "add" else None)
        xin = _norm_ref(x, norm)
        if epilogue == "store":
            ref = _lin_ref(xin, w)
        elif epilogue == "add":
            ref = (res.float() + _lin_ref(xin, w).float()).to(torch.bfloat16)
        else:
            gate, up = _lin_ref(xin, w).chunk(2, dim=-1)
            ref = (torch.nn.functional.silu(gate) * up)
        what = f"{epilogue} M{M} K{K} N{N} norm={None if norm is None else norm.weight.dtype}"
        assert got.shape == (M, N)
        _assert_close(got, ref, what)


def test_rows_linear_strided_rows_and_in_place_add():
    """Input rows with a row stride above K (a column slice of a wider
    tensor), 3-D leading shape, and the residual add written in place."""
    g = torch.Generator().manual_seed(5)
    wide = torch.randn(1, 4, 1024, generator=g).to(torch.bfloat16).to(DEV)
    x = wide[..., :768]
    w = (torch.randn(512, 768, generator=g) / 28).to(torch.bfloat16).to(DEV)
    res = torch.randn(1, 4, 512, generator=g).to(torch.bfloat16).to(DEV)
    ref = (res.float() + _lin_ref(x, w).float()).to(torch.bfloat16)
    out = rows_linear(x, w, epilogue="add", res=res, out=res)
    assert out.data_ptr() == res.data_ptr() and out.shape == (1, 4, 512)
    _assert_close(res, ref, "in-place add")


@pytest.mark.parametrize("M", [1, 3])
@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
def test_rows_linear_add_with_skip(M, wdt):
    """The add epilogue with the backbone's weighted skip connection folded in:
    t = res + W x, then t + w * skip (skip rows), or t + w * t (no rows), each
    step rounded to bf16 as the unfused torch ops round it."""
    g = torch.Generator().manual_seed(11 + M)
    K, N = 2048, 768
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(DEV)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    sk = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    sw = torch.tensor([0.0, 0.75, 1.3], dtype=wdt, device=DEV)[1:]  # a view at an offset
    t = (res.float() + _lin_ref(x, w).float()).to(torch.bfloat16)
    got = rows_linear(x, w, epilogue="add", res=res, skip=(sk, sw[1]))
    ref = (t.float() + (sw[1].float() * sk.float()).to(torch.bfloat16).float()).to(torch.bfloat16)
    _assert_close(got, ref, "skip rows")
    got = rows_linear(x, w, epilogue="add", res=res, skip=(None, sw[0]))
    ref = (t.float() + (sw[0].float() * t.float()).to(torch.bfloat16).float()).to(torch.bfloat16)
    _assert_close(got, ref, "self skip")


def test_rows_linear_lm_head_width():
    """A vocabulary-wide product (N = 50257, the bench model's LM head) with
    the final norm fused in."""
    g = torch.Generator().manual_seed(6)
    x = torch.randn(1, 1, 768, generator=g).to(torch.bfloat16).to(DEV)
    w = (0.02 * torch.randn(50257, 768, generator=g)).to(torch.bfloat16).to(DEV)
    norm = _norm(768, torch.bfloat16, 3)
    got = rows_linear(x, w, norm=norm)
    _assert_close(got, _lin_ref(_norm_ref(x, norm), w), "lm head")


def _qkv_case(M, H, D, cap, seed):
    C = H * D
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, M, C, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(3 * C, C, generator=g) / math.sqrt(C)).to(torch.bfloat16).to(DEV)
    kc = torch.randn(1, H, cap, D, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(1, H, cap, D, generator=g).to(torch.bfloat16).to(DEV)
    return x, w, kc, vc


@pytest.mark.parametrize("M,H,D", [(1, 12, 64), (3, 4, 64), (8, 8, 128), (2, 2, 128)])
def test_rows_qkv_rope_matches_unfused(M, H, D):
    """q rows and the cache rows written at pos0 .. pos0 + M - 1 equal the
    unfused norm -> Linear -> qkv_rope sequence; every other cache row is
    untouched."""
    cap, p0 = 96, 37
    x, w, kc, vc = _qkv_case(M, H, D, cap, seed=M + H + D)
    norm = _norm(H * D, torch.bfloat16, 4)
    cos, sin = rope_tables(D, 128, DEV)
    k0, v0 = kc.clone(), vc.clone()
    q = rows_qkv_rope(x, w, H, cos, sin, p0, kc, vc, norm=norm)
    qr, kr, vr = qkv_rope(_lin_ref(_norm_ref(x, norm), w), cos, sin, H, p0)
    _assert_close(q, qr, "q")
    _assert_close(kc[:, :, p0:p0 + M], kr, "k cache rows")
    _assert_close(vc[:, :, p0:p0 + M], vr, "v cache rows")
    keep = torch.ones(cap, dtype=torch.bool, device=DEV)
    keep[p0:p0 + M] = False
    assert torch.equal(kc[:, :, keep], k0[:, :, keep])
    assert torch.equal(vc[:, :, keep], v0[:, :, keep])


def test_rows_qkv_rope_device_positions():
    """Positions from a device tensor (as the captured decode step passes
    them), in any order; a row whose position is at or past the cache
    capacity writes nothing."""
    H, D, cap = 4, 64, 64
    x, w, kc, vc = _qkv_case(3, H, D, cap, seed=9)
    cos, sin = rope_tables(D, 128, DEV)
    pos = torch.tensor([40, 5, 100], dtype=torch.int64, device=DEV)
    k0 = kc.clone()
    q = rows_qkv_rope(x, w, H, cos, sin, pos, kc, vc)
    proj = _lin_ref(x, w)
    for m, p in enumerate([40, 5]):
        qr, kr, vr = qkv_rope(proj[:, m:m + 1], cos, sin, H, p)
        _assert_close(q[:, :, m:m + 1], qr, f"q row {m}")
        _assert_close(kc[:, :, p:p + 1], kr, f"k row {m}")
        _assert_close(vc[:, :, p:p + 1], vr, f"v row {m}")
    keep = torch.ones(cap, dtype=torch.bool, device=DEV)
    keep[[40, 5]] = False
    assert torch.equal(kc[:, :, keep], k0[:, :, keep])


def test_rows_qkv_rope_rejects_positions_past_tables():
    H, D = 4, 64
    x, w, kc, vc = _qkv_case(2, H, D, 64, seed=10)
    cos, sin = rope_tables(D, 128, DEV)
    with pytest.raises(RuntimeError, match="exceed"):
        rows_qkv_rope(x, w, H, cos, sin, 63, kc, vc)
