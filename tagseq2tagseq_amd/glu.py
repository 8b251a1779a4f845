"""SwiGLU of the layers' MLP on the gfx950 kernels (``t2t_swiglu`` and its
gradient): h = silu(g) * u from the gate / up product [g | u], one pass
forward, one pass backward writing the product's gradient [dg | du] whole.

Replaces the activation and product of tunalab's GLU(activation="silu") in
the reference's layers (model/modules/layer.py:23-28; textbook definition,
parity with tunalab unpinned), which torch runs as chunk + silu + multiply
and, backward, four elementwise kernels and a concatenation.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _rows(t: torch.Tensor) -> torch.Tensor:
    """[N, C] rows as the kernels read them: unit column stride, rows 16-byte
    aligned (row stride a multiple of 8 elements, 16-byte aligned start);
    anything else is copied."""
    t = t.reshape(-1, t.shape[-1])
    ok = t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0
    return t if ok else t.contiguous()


def swiglu_applies(gu: torch.Tensor) -> bool:
    """bf16 rows [..., 2H] on a ROCm device with H % 8 == 0."""
    return gu.is_cuda and gu.dtype == torch.bfloat16 and gu.shape[-1] % 16 == 0


class SwiGLUFn(torch.autograd.Function):
    """forward(gu [..., 2H]) -> silu(gu[..., :H]) * gu[..., H:] ([..., H])."""

    @staticmethod
    def forward(ctx, gu):
        H = gu.shape[-1] // 2
        g2 = _rows(gu)
        N = g2.shape[0]
        h = torch.empty((N, H), dtype=gu.dtype, device=gu.device)
        with torch.cuda.device(gu.device):
            rc = _lib.lib().t2t_swiglu(g2.data_ptr(), g2.stride(0), h.data_ptr(), h.stride(0),
                                       N, H, _stream(gu))
        _lib.check(rc, "t2t_swiglu")
        ctx.save_for_backward(g2)
        ctx.shape = gu.shape
        return h.view(*gu.shape[:-1], H)

    @staticmethod
    def backward(ctx, dh):
        (g2,) = ctx.saved_tensors
        N, H2 = g2.shape
        H = H2 // 2
        d2 = _rows(dh)
        dgu = torch.empty((N, H2), dtype=g2.dtype, device=g2.device)
        with torch.cuda.device(g2.device):
            rc = _lib.lib().t2t_swiglu_backward(g2.data_ptr(), g2.stride(0), d2.data_ptr(),
                                                d2.stride(0), dgu.data_ptr(), dgu.stride(0), N,
                                                H, _stream(g2))
        _lib.check(rc, "t2t_swiglu_backward")
        return dgu.view(ctx.shape)


def swiglu(gu: torch.Tensor) -> torch.Tensor:
    """silu(g) * u of [g | u] rows on the fused kernels (bf16, ROCm device)."""
    if not swiglu_applies(gu):
        raise RuntimeError("swiglu needs bf16 rows on a ROCm device with H % 8 == 0")
    return SwiGLUFn.apply(gu)
