"""RMS normalisation on the gfx950 kernels (``t2t_rms_norm`` and its
gradient) as a ``torch.library`` custom op with registered autograd.

Replaces the RMSNorm of the reference's layers and head
(model/modules/layer.py:14,19; model/modules/training_module.py:122-123; the
module itself comes from the absent tunalab package, so its definition here
is the textbook one: y = x / sqrt(mean(x^2) + eps) * weight, fp32 arithmetic,
one rounding to the row dtype).  One launch forward, two backward (dx per row;
the weight gradient reduced across work-groups in a fixed order).
"""
from __future__ import annotations

import ctypes
from typing import Tuple

import torch

from . import _lib

_WDT = {torch.bfloat16: 0, torch.float32: 1}


def _stream_ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _rows(t: torch.Tensor) -> torch.Tensor:
    t = t.reshape(-1, t.shape[-1])
    return t if t.stride(1) == 1 and t.stride(0) % 8 == 0 else t.contiguous()


def _fwd_impl(x, weight, eps):
    C = x.shape[-1]
    xr = _rows(x)
    N = xr.shape[0]
    y = torch.empty((N, C), dtype=x.dtype, device=x.device)
    rstd = torch.empty((N,), dtype=torch.float32, device=x.device)
    w = weight.contiguous()
    with torch.cuda.device(x.device):
        rc = _lib.lib().t2t_rms_norm(xr.data_ptr(), xr.stride(0), w.data_ptr(), _WDT[w.dtype],
                                     y.data_ptr(), y.stride(0), rstd.data_ptr(), N, C,
                                     float(eps), _stream_ptr(x))
    _lib.check(rc, "t2t_rms_norm")
    return y.view(x.shape), rstd


@torch.library.custom_op("t2t::rms_norm", mutates_args=())
def rms_norm_op(x: torch.Tensor, weight: torch.Tensor,
                eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """(y like x, rstd float32 [N]) over the last dimension of x (bf16)."""
    return _fwd_impl(x, weight, eps)


@rms_norm_op.register_fake
def _rms_norm_fake(x, weight, eps):
    n = x.numel() // max(1, x.shape[-1])
    return x.new_empty(x.shape), x.new_empty((n,), dtype=torch.float32)


def _bwd_impl(dy, x, weight, rstd):
    C = x.shape[-1]
    xr, dyr = _rows(x), _rows(dy)
    N = xr.shape[0]
    dx = torch.empty((N, C), dtype=x.dtype, device=x.device)
    w = weight.contiguous()
    dw = torch.empty_like(w)
    L = _lib.lib()
    ws = torch.empty(max(1, L.t2t_rms_norm_backward_workspace(N, C) // 4), dtype=torch.float32,
                     device=x.device)
    with torch.cuda.device(x.device):
        rc = L.t2t_rms_norm_backward(dyr.data_ptr(), dyr.stride(0), xr.data_ptr(), xr.stride(0),
                                     w.data_ptr(), _WDT[w.dtype], rstd.data_ptr(), dx.data_ptr(),
                                     dx.stride(0), dw.data_ptr(), ws.data_ptr(), ws.numel() * 4,
                                     N, C, _stream_ptr(x))
    _lib.check(rc, "t2t_rms_norm_backward")
    return dx.view(x.shape), dw


@torch.library.custom_op("t2t::rms_norm_backward", mutates_args=())
def rms_norm_backward_op(dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor,
                         rstd: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(dx like x, dweight like weight)."""
    return _bwd_impl(dy, x, weight, rstd)


@rms_norm_backward_op.register_fake
def _rms_norm_backward_fake(dy, x, weight, rstd):
    return x.new_empty(x.shape), torch.empty_like(weight)


def _setup(ctx, inputs, output):
    x, weight, _ = inputs
    _, rstd = output
    ctx.save_for_backward(x, weight, rstd)


def _backward(ctx, dy, _drstd):
    x, weight, rstd = ctx.saved_tensors
    dx, dw = rms_norm_backward_op(dy, x, weight, rstd)
    return dx, dw, None


rms_norm_op.register_autograd(_backward, setup_context=_setup)


def kernel_applies(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """bf16 rows on a ROCm device with a bf16 / float32 weight and C % 8 == 0."""
    C = x.shape[-1]
    return (x.is_cuda and x.dtype == torch.bfloat16 and weight.dtype in _WDT
            and C % 8 == 0 and 0 < C <= 4096)


class RMSNormFn(torch.autograd.Function):
    """The same kernels as t2t::rms_norm for eager execution: a plain
    autograd.Function costs tens of microseconds of host time per call, the
    registered custom-op autograd several hundred (the custom op is what
    compiled graphs trace)."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        y, rstd = _fwd_impl(x, weight, eps)
        ctx.save_for_backward(x, weight, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, weight, rstd = ctx.saved_tensors
        dx, dw = _bwd_impl(dy, x, weight, rstd)
        return dx, dw, None


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    if torch.compiler.is_compiling():
        return rms_norm_op(x, weight, float(eps))[0]
    return RMSNormFn.apply(x, weight, float(eps))
