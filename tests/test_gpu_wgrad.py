"""GPU parity of the split-K weight gradient (t2t_wgrad, linear.Linear)
against a float32 torch reference of dY^T X, and determinism."""
import ctypes

import pytest
import torch

from tagseq2tagseq_amd import _lib
from tagseq2tagseq_amd.linear import Linear, WGradLinearFn, wgrad

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("K,M,N,pad_a,pad_b", [(64, 128, 128, 0, 0), (192, 256, 384, 8, 16),
                                               (16384, 768, 768, 0, 0), (2048, 2304, 768, 0, 8),
                                               (16384, 4096, 768, 0, 0), (4096, 768, 2048, 16, 0)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_wgrad_against_float32(K, M, N, pad_a, pad_b, out_dtype):
    g = torch.Generator().manual_seed(K + M + N)
    dy = torch.randn(K, M + pad_a, generator=g).to(torch.bfloat16).to(DEV)[:, :M]
    x = torch.randn(K, N + pad_b, generator=g).to(torch.bfloat16).to(DEV)[:, :N]
    got = wgrad(dy, x, out_dtype)
    ref = dy.float().t() @ x.float()
    tol = 1e-4 * K ** 0.5 if out_dtype == torch.float32 else 8e-3 * float(ref.abs().max())
    torch.testing.assert_close(got.float(), ref, rtol=1e-3 if out_dtype == torch.float32 else 8e-3,
                               atol=tol)
    assert torch.equal(wgrad(dy, x, out_dtype), got)  # fixed summation order


def test_linear_gradients_match_nn_linear():
    torch.manual_seed(0)
    lin = Linear(256, 384, bias=False).to(DEV).to(torch.bfloat16)
    ref = torch.nn.Linear(256, 384, bias=False).to(DEV)
    ref.weight.data.copy_(lin.weight.data.float())
    x = torch.randn(2, 64, 256, device=DEV).to(torch.bfloat16)
    dy = torch.randn(2, 64, 384, device=DEV).to(torch.bfloat16)
    xa = x.clone().requires_grad_()
    y = lin(xa)
    assert type(y.grad_fn).__name__ == "WGradLinearFnBackward"
    y.backward(dy)
    xr = x.float().requires_grad_()
    ref(xr).backward(dy.float())
    torch.testing.assert_close(y.float(), ref(xr).detach(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(xa.grad.float(), xr.grad, rtol=2e-2, atol=5e-2)
    torch.testing.assert_close(lin.weight.grad.float(), ref.weight.grad, rtol=2e-2, atol=5e-2)


def test_rows_not_multiple_of_64_use_the_library_product():
    lin = Linear(128, 128, bias=False).to(DEV).to(torch.bfloat16)
    x = torch.randn(33, 128, device=DEV).to(torch.bfloat16).requires_grad_()
    lin(x).float().sum().backward()
    ref = torch.ones(33, 128, device=DEV).t() @ x.detach().float()
    torch.testing.assert_close(lin.weight.grad.float(), ref, rtol=2e-2, atol=5e-2)
