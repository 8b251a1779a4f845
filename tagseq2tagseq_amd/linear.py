"""nn.Linear whose weight gradient runs on the gfx950 split-K kernel
(``t2t_wgrad``).

The layers' projections (tunalab FlexSelfAttention's qkv / out projections
and GLU's gate_up / down, called from model/modules/layer.py:33-35) are
bias-free nn.Linear maps over all T tokens.  Their forward and input
gradient stay library products (hipBLASLt / rocBLAS through torch); the
weight gradient dW = dY^T X contracts K = T rows into a small output
(768 x 768 ... 4096 x 768 at configs[4]), which the library runs on 36-192
output tiles, a fraction of the 256 CUs.  ``t2t_wgrad`` splits K across
work-groups into fp32 partials and sums them in a fixed order.
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib

_OUT_DTYPE = {torch.bfloat16: 0, torch.float32: 1}


def wgrad_applies(dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor) -> bool:
    """bf16 rows on a ROCm device, M and N multiples of 128, K of 64."""
    M, N = weight.shape
    K = x.numel() // max(N, 1)
    return (x.is_cuda and x.dtype == torch.bfloat16 and dy.dtype == torch.bfloat16
            and weight.dtype in _OUT_DTYPE and M % 128 == 0 and N % 128 == 0
            and K > 0 and K % 64 == 0)


def _rows(t: torch.Tensor) -> torch.Tensor:
    t = t.reshape(-1, t.shape[-1])
    ok = t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0
    return t if ok else t.contiguous()


def wgrad(dy: torch.Tensor, x: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """dY^T X of [K, M] and [K, N] bf16 rows -> [M, N] (out_dtype)."""
    d2, x2 = _rows(dy), _rows(x)
    K, M = d2.shape
    N = x2.shape[1]
    L = _lib.lib()
    ws = torch.empty((L.t2t_wgrad_workspace(M, N, K),), dtype=torch.uint8, device=x.device)
    out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    with torch.cuda.device(x.device):
        rc = L.t2t_wgrad(d2.data_ptr(), d2.stride(0), x2.data_ptr(), x2.stride(0),
                         out.data_ptr(), _OUT_DTYPE[out_dtype], M, N, K, ws.data_ptr(),
                         ws.numel(), stream)
    _lib.check(rc, "t2t_wgrad")
    return out


class WGradLinearFn(torch.autograd.Function):
    """y = x W^T (bias-free); dX = dY W by the library, dW by t2t_wgrad."""

    @staticmethod
    def forward(ctx, x, weight):
        ctx.save_for_backward(x, weight)
        return F.linear(x, weight)

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        dx = dw = None
        if ctx.needs_input_grad[0]:
            dx = (dy.reshape(-1, dy.shape[-1]) @ weight.to(dy.dtype)).view(x.shape)
        if ctx.needs_input_grad[1]:
            if wgrad_applies(dy, x, weight):
                dw = wgrad(dy, x, weight.dtype)
            else:
                d2, x2 = dy.reshape(-1, dy.shape[-1]), x.reshape(-1, x.shape[-1])
                dw = (d2.t() @ x2).to(weight.dtype)
        return dx, dw


class Linear(nn.Linear):
    """nn.Linear (same parameters and state dict); bias-free bf16 maps on the
    GPU take their weight gradient from t2t_wgrad."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # (graphs being compiled keep torch's own linear: the Function's
        # backward calls the library through ctypes)
        if (self.bias is None and x.is_cuda and x.dtype == torch.bfloat16
                and self.weight.dtype == torch.bfloat16 and not torch.compiler.is_compiling()):
            return WGradLinearFn.apply(x, self.weight)
        return super().forward(x)
