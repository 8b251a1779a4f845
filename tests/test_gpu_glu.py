"""GPU parity of the fused SwiGLU (t2t_swiglu and its gradient) against a
float32 torch reference of silu(g) * u and its autograd gradient."""
import pytest
import torch
import torch.nn.functional as F

from tagseq2tagseq_amd.glu import swiglu
from tagseq2tagseq_amd.modules import GLU

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("shape", [(1, 8, 32), (3, 77, 2 * 2048), (5, 16)])
def test_swiglu_against_float32(shape):
    g = torch.Generator().manual_seed(sum(shape))
    gu0 = (torch.randn(*shape, generator=g) * 4).to(torch.bfloat16).to(DEV)
    H = shape[-1] // 2
    dh = torch.randn(*shape[:-1], H, generator=g).to(torch.bfloat16).to(DEV)

    gu = gu0.clone().requires_grad_()
    h = swiglu(gu)
    h.backward(dh)

    ref_in = gu0.float().requires_grad_()
    a, b = ref_in.chunk(2, dim=-1)
    ref = F.silu(a) * b
    ref.backward(dh.float())
    # one bf16 rounding of fp32 results
    torch.testing.assert_close(h.float(), ref, rtol=8e-3, atol=1e-5)
    torch.testing.assert_close(gu.grad.float(), ref_in.grad, rtol=8e-3, atol=1e-5)


def test_swiglu_strided_rows_and_saturation():
    # rows of a wider buffer (row stride > 2H) and saturated sigmoid inputs
    base = torch.zeros(6, 96, dtype=torch.bfloat16, device=DEV)
    gu = base[:, :64]
    gu[:, :32] = torch.tensor([-100.0, -20.0, 0.0, 20.0, 100.0, 1e30, -1e30, 3.0] * 4,
                              dtype=torch.bfloat16, device=DEV)
    gu[:, 32:] = 2.0
    h = swiglu(gu)
    ref = F.silu(gu[:, :32].float()) * 2.0
    torch.testing.assert_close(h.float(), ref, rtol=8e-3, atol=1e-5)
    assert torch.isfinite(h).all()


def test_swiglu_unaligned_view_is_copied():
    """Rows whose stride is a multiple of 8 elements but whose first element
    is not 16-byte aligned (a buffer viewed from its second element) take the
    copy path, forward and backward, and match the float32 reference."""
    g = torch.Generator().manual_seed(7)
    buf = torch.randn(9 * 72 + 1, generator=g).to(torch.bfloat16).to(DEV)
    gu0 = buf[1:].view(9, 72)[:, :64]  # starts 2 bytes past the allocation
    assert gu0.stride(0) % 8 == 0 and gu0.data_ptr() % 16 != 0
    dh = torch.randn(9, 32, generator=g).to(torch.bfloat16).to(DEV)
    leaf = gu0.detach().requires_grad_()
    h = swiglu(leaf)
    h.backward(dh)
    ref_in = gu0.float().requires_grad_()
    a, b = ref_in.chunk(2, dim=-1)
    ref = F.silu(a) * b
    ref.backward(dh.float())
    torch.testing.assert_close(h.float(), ref, rtol=8e-3, atol=1e-5)
    torch.testing.assert_close(leaf.grad.float(), ref_in.grad, rtol=8e-3, atol=1e-5)


def _graph_nodes(fn):
    seen, stack = set(), [fn]
    while stack:
        f = stack.pop()
        if f is None or type(f).__name__ in seen:
            continue
        seen.add(type(f).__name__)
        stack.extend(n for n, _ in f.next_functions)
    return seen


def test_glu_module_uses_fused_path_and_matches_torch():
    torch.manual_seed(0)
    m = GLU(64, 64, 160).to(DEV).to(torch.bfloat16)
    x = torch.randn(2, 33, 64, device=DEV).to(torch.bfloat16).requires_grad_()
    y = m(x)
    assert "SwiGLUFnBackward" in _graph_nodes(y.grad_fn)
    y.float().sum().backward()
    xr = x.detach().float().requires_grad_()
    wg = m.gate_up.weight.detach().float()
    wd = m.down.weight.detach().float()
    gur = xr @ wg.t()
    a, b = gur.chunk(2, dim=-1)
    yr = (F.silu(a) * b) @ wd.t()
    yr.sum().backward()
    torch.testing.assert_close(y.float(), yr, rtol=3e-2, atol=3e-2)
    torch.testing.assert_close(x.grad.float(), xr.grad, rtol=3e-2, atol=3e-2)
