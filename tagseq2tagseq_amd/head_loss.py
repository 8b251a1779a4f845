"""Linear head + mean cross-entropy with the logit gradient computed in the
forward, on the gfx950 ``t2t_ce_rows`` kernel.

Replaces the reference's FusedLinearCELoss (tunalab, a Liger-style fused
linear cross-entropy; constructed at model/modules/training_module.py:127-133
and called at :209; the package is absent, so the definition followed is the
textbook one: loss = mean over rows whose target is not ignore_index of
logsumexp(x W^T) - (x W^T)[target]).  Per chunk of rows:

  1. logits = x_chunk W^T                     (bf16 product, hipBLASLt)
  2. t2t_ce_rows: the rows' losses and, over the logits in place,
     (softmax - onehot) / n_counted           (one kernel, fp32 arithmetic)
  3. dx_chunk = grad W,  dW += grad^T x_chunk (bf16 products, dW summed in fp32)
     -- only when autograd needs a gradient; evaluation stops after step 2

so the backward only scales dx and dW by the incoming gradient: the logits
are never recomputed and never exist in fp32.  The vocabulary is padded to a
multiple of 8 columns (zero weight rows) so that every logit row starts on a
16-byte boundary; padded columns get no probability and a zero gradient.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

# rows per chunk when the caller gives none: the whole batch while the bf16
# logits stay under this many bytes
AUTO_CHUNK_BYTES = 2 << 30


def fused_head_applies(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """bf16 rows on a ROCm device and a bf16 / float32 head weight."""
    return (x.is_cuda and x.dtype == torch.bfloat16 and weight.is_cuda
            and weight.dtype in (torch.bfloat16, torch.float32) and x.dim() == 2)


def _mm_f32(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a @ b of bf16 operands with a float32 result."""
    try:
        return torch.mm(a, b, out_dtype=torch.float32)
    except (RuntimeError, TypeError):
        return torch.mm(a, b).float()


def _head_pass(x, weight, targets, ignore_index: int, chunk: Optional[int], grads: bool):
    """Per chunk of rows: logits, t2t_ce_rows (row losses, and the logit
    gradient in place over the logits), then -- when ``grads`` -- dx and the
    fp32 dW from that gradient.  Returns (row_loss, n counted, dx, dw); dx and
    dw are None without ``grads``."""
    N, D = x.shape
    V = weight.shape[0]
    ld = (V + 7) // 8 * 8
    dev = x.device
    t = targets.reshape(-1).to(device=dev, dtype=torch.int64).contiguous()
    if t.numel() != N:
        raise ValueError(f"{t.numel()} targets for {N} rows")
    if weight.shape[1] != D:
        raise ValueError(f"weight {tuple(weight.shape)} does not match rows of width {D}")
    w = torch.zeros((ld, D), dtype=torch.bfloat16, device=dev)
    w[:V].copy_(weight)
    n = (t != ignore_index).sum()
    # gradient scale 1 / n; with every row ignored no row has a gradient, so
    # the scale only has to be finite
    scale = (1.0 / n.clamp(min=1).to(torch.float32)).reshape(1)
    row_loss = torch.empty((N,), dtype=torch.float32, device=dev)
    dx = torch.empty((N, D), dtype=x.dtype, device=dev) if grads else None
    dw = torch.zeros((ld, D), dtype=torch.float32, device=dev) if grads else None
    if chunk is None:
        chunk = max(1, AUTO_CHUNK_BYTES // (2 * ld))
    rows = max(1, min(chunk, N))
    buf = torch.empty((rows, ld), dtype=torch.bfloat16, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    L = _lib.lib()
    with torch.cuda.device(dev):
        for r0 in range(0, N, rows):
            xs = x[r0:r0 + rows]
            m = xs.shape[0]
            logits = buf[:m]
            torch.mm(xs, w.t(), out=logits)
            rc = L.t2t_ce_rows(logits.data_ptr(), logits.data_ptr(), m, V, ld,
                               t[r0:r0 + m].data_ptr(), ignore_index, scale.data_ptr(),
                               row_loss[r0:r0 + m].data_ptr(), stream)
            _lib.check(rc, "t2t_ce_rows")
            if grads:
                torch.mm(logits, w, out=dx[r0:r0 + m])
                dw += _mm_f32(logits.t(), xs)
    return row_loss, n, dx, dw


def _mean(row_loss: torch.Tensor, n: torch.Tensor) -> torch.Tensor:
    """Sum of the row losses over the counted rows, as torch's mean
    cross-entropy: 0 / 0 = NaN when every target is ignore_index."""
    return row_loss.sum() / n.to(torch.float32)


class HeadCEFn(torch.autograd.Function):
    """forward(x [N, D] bf16, weight [V, D], targets [N] int64, ignore_index,
    chunk) -> mean loss (float32 scalar); gradients for x and weight."""

    @staticmethod
    def forward(ctx, x, weight, targets, ignore_index: int, chunk: Optional[int]):
        row_loss, n, dx, dw = _head_pass(x, weight, targets, ignore_index, chunk, grads=True)
        ctx.save_for_backward(dx, dw)
        ctx.V, ctx.wdtype = weight.shape[0], weight.dtype
        return _mean(row_loss, n)

    @staticmethod
    def backward(ctx, g):
        dx, dw = ctx.saved_tensors
        gx = dx * g.to(dx.dtype)
        gw = (dw[:ctx.V] * g).to(ctx.wdtype)
        return gx, gw, None, None, None


def head_loss_needs_grad(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """True when autograd will ask for a gradient of x or weight."""
    return torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad)


def head_loss_value(x: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                    ignore_index: int = -100, chunk: Optional[int] = None) -> torch.Tensor:
    """The mean loss alone (evaluation, no_grad): the logits and one
    t2t_ce_rows pass per chunk, without the dx / dW products or their buffers."""
    with torch.no_grad():
        row_loss, n, _, _ = _head_pass(x, weight, targets, int(ignore_index), chunk, grads=False)
        return _mean(row_loss, n)


def head_cross_entropy(x: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                       ignore_index: int = -100, chunk: Optional[int] = None) -> torch.Tensor:
    """Mean cross-entropy of x W^T against targets (rows equal to
    ignore_index not counted; NaN when every row is, as torch's mean
    cross-entropy) on the fused kernel; x [N, D] bf16 on the GPU.  The
    gradient products run only when autograd needs them."""
    if not fused_head_applies(x, weight):
        raise RuntimeError("head_cross_entropy needs bf16 rows and a bf16 / float32 weight "
                           "on a ROCm device")
    if not head_loss_needs_grad(x, weight):
        return head_loss_value(x, weight, targets, ignore_index, chunk)
    return HeadCEFn.apply(x, weight, targets, int(ignore_index), chunk)
