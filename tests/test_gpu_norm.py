"""GPU checks of the RMS-normalisation kernels (t2t_rms_norm and its
gradient) against an fp64 restatement of y = x / sqrt(mean(x^2) + eps) * w on
the same bf16 inputs: y within one bf16 rounding, 1/rms within fp32
rounding, dx and dweight against fp64 autograd; a bitwise-deterministic
weight gradient; padded rows; opcheck.  (tunalab's RMSNorm itself is absent,
so parity with it is unpinned; the definition is the textbook one.)"""
import pytest
import torch

from tagseq2tagseq_amd.modules import RMSNorm
from tagseq2tagseq_amd.norm import rms_norm_op

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
EPS = 1e-6


def _ref(x, w):
    xd = x.double()
    r = torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + EPS)
    return xd * r * w.double(), r.squeeze(-1)


def _inputs(N, C, wdtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(N, C, generator=g) * 3).to(torch.bfloat16).to(DEV)
    w = (1 + 0.5 * torch.randn(C, generator=g)).to(wdtype).to(DEV)
    return x, w


@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N,C", [(1, 8), (3, 256), (1000, 768), (257, 1000), (64, 2048),
                                 (16, 4096), (16384, 768)])
def test_forward(N, C, wdtype):
    x, w = _inputs(N, C, wdtype, N + C)
    y, rstd = rms_norm_op(x, w, EPS)
    ry, rr = _ref(x, w)
    err = (y.double() - ry).abs()
    assert bool((err <= ry.abs() * 2.0 ** -8 + 1e-6).all()), f"max excess {(err - ry.abs() * 2.0 ** -8).max()}"
    assert torch.allclose(rstd.double(), rr, rtol=2e-6, atol=0)


@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N,C", [(5, 64), (1000, 768), (300, 1024), (33, 4096)])
def test_backward(N, C, wdtype):
    x, w = _inputs(N, C, wdtype, 7 * N + C)
    g = torch.Generator().manual_seed(N)
    dy = torch.randn(N, C, generator=g).to(torch.bfloat16).to(DEV)
    xg = x.clone().requires_grad_(True)
    wg = w.clone().requires_grad_(True)
    y, _ = rms_norm_op(xg, wg, EPS)
    y.backward(dy)
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    ry, _ = _ref(xd, wd)
    ry.backward(dy.double())
    dx_err = (xg.grad.double() - xd.grad).abs().max() / xd.grad.abs().max()
    dw_err = (wg.grad.double() - wd.grad).abs().max() / wd.grad.abs().max()
    assert dx_err < 1e-2, f"dx rel err {dx_err}"
    assert dw_err < 1e-2, f"dw rel err {dw_err}"
    assert wg.grad.dtype == wdtype


def test_weight_gradient_is_deterministic():
    x, w = _inputs(4096, 768, torch.bfloat16, 1)
    dy = torch.randn(4096, 768, device=DEV).to(torch.bfloat16)
    _, rstd = rms_norm_op(x, w, EPS)
    a = torch.ops.t2t.rms_norm_backward(dy, x, w, rstd)
    b = torch.ops.t2t.rms_norm_backward(dy, x, w, rstd)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_padded_rows_and_3d_input():
    g = torch.Generator().manual_seed(3)
    big = torch.randn(2, 100, 800, generator=g).to(torch.bfloat16).to(DEV)
    x = big[:, :, :768]  # rows 800 apart
    w = torch.ones(768, dtype=torch.bfloat16, device=DEV)
    y, _ = rms_norm_op(x, w, EPS)
    ry, _ = _ref(x, w)
    assert y.shape == x.shape
    assert bool(((y.double() - ry).abs() <= ry.abs() * 2.0 ** -8 + 1e-6).all())


def test_module_uses_kernel_and_matches_formula():
    m = RMSNorm(768).to(DEV, torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_(torch.linspace(0.5, 1.5, 768))
    x = torch.randn(4, 33, 768, device=DEV).to(torch.bfloat16)
    y = m(x)
    ry, _ = _ref(x, m.weight)
    assert bool(((y.double() - ry).abs() <= ry.abs() * 2.0 ** -8 + 1e-6).all())


def test_opcheck():
    x, w = _inputs(64, 256, torch.bfloat16, 9)
    torch.library.opcheck(torch.ops.t2t.rms_norm.default,
                          (x.requires_grad_(True), w.requires_grad_(True), EPS),
                          test_utils=("test_schema", "test_faketensor",
                                      "test_autograd_registration"))
