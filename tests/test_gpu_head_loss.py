"""GPU parity of the fused linear-head cross-entropy (t2t_ce_rows and
head_loss.HeadCEFn) against plain torch: the kernel against float64
logsumexp / softmax on the same bf16 logits, and the whole head loss against
torch's own chunk path (bf16 product, float32 cross-entropy, autograd) and a
float32 reference."""
import ctypes
import math

import pytest
import torch
import torch.nn.functional as F

from tagseq2tagseq_amd import _lib
from tagseq2tagseq_amd.head_loss import head_cross_entropy
from tagseq2tagseq_amd.modules import LinearCELoss

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _ce_rows(logits, V, target, ignore, scale, grad=None):
    rows, ld = logits.shape
    grad = logits if grad is None else grad
    loss = torch.empty(rows, dtype=torch.float32, device=DEV)
    sc = torch.tensor([scale], dtype=torch.float32, device=DEV)
    rc = _lib.lib().t2t_ce_rows(logits.data_ptr(), grad.data_ptr(), rows, V, ld,
                                target.data_ptr(), ignore, sc.data_ptr(), loss.data_ptr(),
                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "t2t_ce_rows")
    torch.cuda.synchronize()
    return loss, grad


@pytest.mark.parametrize("rows,V,ld", [(5, 1, 8), (33, 1000, 1000), (64, 1003, 1008),
                                       (17, 50257, 50264), (3, 70001, 70008)])
def test_ce_rows_against_float64(rows, V, ld):
    g = torch.Generator().manual_seed(rows + V)
    x = (torch.randn(rows, ld, generator=g) * 3).to(torch.bfloat16).to(DEV)
    t = torch.randint(0, V, (rows,), generator=g)
    t[::4] = -100  # ignored rows
    t = t.to(DEV)
    src = x.clone()
    out = torch.full_like(x, 7.0)
    loss, grad = _ce_rows(src, V, t, -100, 0.25, grad=out)
    assert torch.equal(src, x)  # out of place: logits untouched

    xf = x[:, :V].double()
    lse = torch.logsumexp(xf, dim=1)
    tc = t.clamp(min=0)
    ref_loss = torch.where(t == -100, torch.zeros_like(lse), lse - xf.gather(1, tc[:, None])[:, 0])
    torch.testing.assert_close(loss.double(), ref_loss, rtol=1e-5, atol=1e-5)
    p = torch.softmax(xf, dim=1)
    onehot = torch.zeros_like(p)
    onehot.scatter_(1, tc[:, None], 1.0)
    ref_grad = (p - onehot) * 0.25
    ref_grad[t == -100] = 0
    # one bf16 rounding of the gradient
    torch.testing.assert_close(grad[:, :V].double(), ref_grad, rtol=8e-3, atol=1e-6)
    assert (grad[:, V:] == 0).all()

    # in place: the same bits
    inplace = x.clone()
    loss2, _ = _ce_rows(inplace, V, t, -100, 0.25)
    assert torch.equal(loss2, loss) and torch.equal(inplace, grad)


def test_ce_rows_out_of_range_target_is_nan():
    x = torch.randn(3, 16, device=DEV).to(torch.bfloat16)
    t = torch.tensor([2, 16, -5], device=DEV)
    loss, grad = _ce_rows(x.clone(), 16, t, -100, 1.0)
    assert torch.isfinite(loss[0]) and torch.isnan(loss[1]) and torch.isnan(loss[2])
    assert (grad[1:] == 0).all()


@pytest.mark.parametrize("N,D,V,wdtype,chunk", [(257, 64, 1003, torch.float32, None),
                                                (300, 128, 1000, torch.bfloat16, 64),
                                                (96, 64, 8, torch.float32, 7)])
def test_head_loss_against_torch(N, D, V, wdtype, chunk):
    g = torch.Generator().manual_seed(N + D + V)
    x0 = torch.randn(N, D, generator=g).to(torch.bfloat16).to(DEV)
    w0 = (torch.randn(V, D, generator=g) * D ** -0.5).to(wdtype).to(DEV)
    t = torch.randint(0, V, (N,), generator=g)
    t[3::7] = -100
    t = t.to(DEV)

    x = x0.clone().requires_grad_()
    w = w0.clone().requires_grad_()
    loss = head_cross_entropy(x, w, t, -100, chunk)
    loss.backward()

    # torch's path on the same bf16 product: bf16 logits -> float32 cross-entropy
    xr = x0.clone().requires_grad_()
    wr = w0.clone().requires_grad_()
    ref = F.cross_entropy(F.linear(xr, wr.to(torch.bfloat16)).float(), t, ignore_index=-100)
    ref.backward()
    torch.testing.assert_close(loss, ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(x.grad.float(), xr.grad.float(), rtol=2e-2, atol=2e-4)
    torch.testing.assert_close(w.grad.float(), wr.grad.float(), rtol=2e-2, atol=2e-4)

    # and a float32 reference of the whole head
    xf = x0.float().requires_grad_()
    wf = w0.float().requires_grad_()
    reff = F.cross_entropy(xf @ wf.t(), t, ignore_index=-100)
    reff.backward()
    torch.testing.assert_close(loss, reff, rtol=5e-3, atol=5e-3)
    scale = xf.grad.abs().max()
    torch.testing.assert_close(x.grad.float(), xf.grad, rtol=3e-2, atol=3e-2 * float(scale))


def test_head_loss_scales_by_incoming_gradient_and_ignores_all():
    x = torch.randn(40, 64, device=DEV).to(torch.bfloat16).requires_grad_()
    w = torch.randn(100, 64, device=DEV).requires_grad_()
    t = torch.randint(0, 100, (40,), device=DEV)
    loss = head_cross_entropy(x, w, t)
    (3.0 * loss).backward()
    gx3 = x.grad.clone()
    x.grad = None
    head_cross_entropy(x, w, t).backward()
    torch.testing.assert_close(gx3.float(), 3.0 * x.grad.float(), rtol=1e-2, atol=1e-6)

    x.grad = None
    w.grad = None
    t_all = torch.full((40,), -100, device=DEV)
    loss0 = head_cross_entropy(x, w, t_all)
    loss0.backward()
    # torch's mean cross-entropy over no counted row is 0 / 0 = NaN; no row
    # has a gradient
    ref0 = F.cross_entropy(F.linear(x.detach(), w.detach().to(torch.bfloat16)).float(),
                           t_all, ignore_index=-100)
    assert math.isnan(float(loss0)) and math.isnan(float(ref0))
    assert (x.grad == 0).all() and (w.grad == 0).all()


def test_head_loss_without_grad_skips_gradient_products():
    """Under no_grad, and for inputs that need no gradient, the loss comes from
    the loss-only pass: the same value as the gradient pass, no autograd node,
    and no [V, D] fp32 weight-gradient buffer allocated."""
    torch.manual_seed(5)
    V, D, N = 5000, 256, 300
    x = torch.randn(N, D, device=DEV).to(torch.bfloat16)
    w = (torch.randn(V, D, device=DEV) * D ** -0.5).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), device=DEV)
    t[:7] = -100
    w_req = w.clone().requires_grad_()

    def peak_of(fn):
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated(DEV)
        torch.cuda.reset_peak_memory_stats(DEV)
        out = fn()
        torch.cuda.synchronize()
        return out, torch.cuda.max_memory_allocated(DEV) - base

    with_grad, peak_grad = peak_of(lambda: head_cross_entropy(x, w_req, t))
    assert with_grad.grad_fn is not None
    with_grad = float(with_grad)  # frees the graph and its dx / dW
    with torch.no_grad():
        no_grad, peak_nograd = peak_of(lambda: head_cross_entropy(x, w_req, t))
    plain, peak_plain = peak_of(lambda: head_cross_entropy(x, w, t))  # no input requires grad
    assert no_grad.grad_fn is None and plain.grad_fn is None
    assert float(no_grad) == with_grad == float(plain)
    # the gradient pass also holds the fp32 dW (V * D * 4 bytes, padded) and dx
    for peak in (peak_nograd, peak_plain):
        assert peak + 4 * V * D <= peak_grad, (peak, peak_grad)
    head = LinearCELoss(D, V, weight=torch.nn.Parameter(w.float()))
    with torch.no_grad():
        assert head(x[None], t[None]).grad_fn is None


def test_module_uses_fused_path_and_matches_cpu_chunks():
    torch.manual_seed(3)
    emb = torch.nn.Embedding(500, 64)
    head = LinearCELoss(64, 500, weight=emb.weight, chunk=50)
    x = torch.randn(1, 130, 64).to(torch.bfloat16)
    t = torch.randint(0, 500, (1, 130))
    t[0, :5] = -100
    cpu = head(x.float(), t)
    emb.to(DEV)
    gpu = head(x.to(DEV), t.to(DEV))
    assert gpu.grad_fn is not None and type(gpu.grad_fn).__name__ == "HeadCEFnBackward"
    torch.testing.assert_close(gpu.cpu(), cpu, rtol=5e-3, atol=5e-3)


def test_head_loss_takes_host_targets_and_checks_shapes():
    x = torch.randn(16, 64, device=DEV).to(torch.bfloat16)
    w = torch.randn(40, 64, device=DEV)
    t = torch.randint(0, 40, (16,))  # host tensor: moved to the rows' device
    ref = F.cross_entropy(F.linear(x, w.to(torch.bfloat16)).float(), t.to(DEV))
    torch.testing.assert_close(head_cross_entropy(x, w, t), ref, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError):
        head_cross_entropy(x, w, t[:15])
    with pytest.raises(ValueError):
        head_cross_entropy(x, torch.randn(40, 32, device=DEV), t)
