"""Attention-module prologue on the gfx950 kernels: QKV split + rotary
embedding in one pass, as a ``torch.library`` custom op with registered
autograd (the gradient is one pass too).

Replaces the head split and rotary embedding inside the reference's attention
module (tunalab ``FlexSelfAttention``, constructed and called at
model/modules/layer.py:16-21,33; the package is not part of the reference, so
the rotary variant -- half-split pairs, base 10000, position = token index --
is the textbook form and its parity with tunalab is unpinned).

    q, k, v = qkv_rope(qkv, cos, sin, num_heads)       # qkv: [B, T, 3 C]
    cos, sin = rope_tables(head_dim, rows, device)      # float32 [rows, D/2]

Kernels: libt2t_attn.so ``t2t_qkv_rope`` / ``t2t_qkv_rope_backward``.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Tuple

import torch

from . import _lib

_TABLES: Dict[Tuple[int, int, float, str], Tuple[torch.Tensor, torch.Tensor]] = {}


def _stream_ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def rope_tables(head_dim: int, rows: int, device, base: float = 10000.0):
    """(cos, sin) float32 [rows, head_dim / 2]: angle[p][i] = p * base^(-i / (D/2)).
    Cached per (head_dim, rows, base, device)."""
    key = (head_dim, rows, float(base), str(torch.device(device)))
    if key not in _TABLES:
        half = head_dim // 2
        inv = base ** (-torch.arange(0, half, dtype=torch.float32) / half)
        ang = torch.outer(torch.arange(rows, dtype=torch.float32), inv)
        _TABLES[key] = (ang.cos().to(device), ang.sin().to(device))
    return _TABLES[key]


def _split_dims(qkv: torch.Tensor, num_heads: int):
    if qkv.dim() != 3:
        raise ValueError(f"qkv must be [B, T, 3 C], got shape {tuple(qkv.shape)}")
    B, T, C3 = qkv.shape
    if C3 % (3 * num_heads) != 0:
        raise ValueError(f"last dim {C3} is not 3 * num_heads * head_dim (num_heads={num_heads})")
    return B, T, C3 // (3 * num_heads)


def _qkv_rope_impl(qkv, cos, sin, num_heads, pos0):
    B, T, D = _split_dims(qkv, num_heads)
    H = num_heads
    if qkv.dtype != torch.bfloat16:
        raise NotImplementedError(f"qkv dtype {qkv.dtype} is not supported (bfloat16 only)")
    if not qkv.is_cuda:
        raise RuntimeError("the prologue kernel needs ROCm GPU tensors")
    if qkv.stride(2) != 1:
        qkv = qkv.contiguous()
    cos, sin = cos.contiguous(), sin.contiguous()
    q, k, v = (torch.empty((B, H, T, D), dtype=qkv.dtype, device=qkv.device) for _ in range(3))
    views = [_lib.tensor_struct(t) for t in (q, k, v)]
    with torch.cuda.device(qkv.device):
        rc = _lib.lib().t2t_qkv_rope(qkv.data_ptr(), qkv.stride(0), qkv.stride(1), B, T, H, D,
                                     cos.data_ptr(), sin.data_ptr(), cos.shape[0], pos0,
                                     *[ctypes.byref(x) for x in views], _stream_ptr(qkv))
    _lib.check(rc, "t2t_qkv_rope")
    return q, k, v


def _qkv_rope_bwd_impl(dq, dk, dv, cos, sin, pos0):
    B, H, T, D = dq.shape
    grads = [g if g.stride(3) == 1 else g.contiguous() for g in (dq, dk, dv)]
    cos, sin = cos.contiguous(), sin.contiguous()
    dqkv = torch.empty((B, T, 3 * H * D), dtype=dq.dtype, device=dq.device)
    views = [_lib.tensor_struct(g) for g in grads]
    with torch.cuda.device(dq.device):
        rc = _lib.lib().t2t_qkv_rope_backward(*[ctypes.byref(x) for x in views], cos.data_ptr(),
                                              sin.data_ptr(), cos.shape[0], pos0, B, T, H, D,
                                              dqkv.data_ptr(), dqkv.stride(0), dqkv.stride(1),
                                              _stream_ptr(dq))
    _lib.check(rc, "t2t_qkv_rope_backward")
    return dqkv


@torch.library.custom_op("t2t::qkv_rope", mutates_args=())
def qkv_rope_op(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, num_heads: int,
                pos0: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(q, k, v) [B, H, T, D] from qkv [B, T, 3 H D]; q and k rotated."""
    return _qkv_rope_impl(qkv, cos, sin, num_heads, pos0)


@qkv_rope_op.register_fake
def _qkv_rope_fake(qkv, cos, sin, num_heads, pos0):
    B, T, D = _split_dims(qkv, num_heads)
    return tuple(qkv.new_empty((B, num_heads, T, D)) for _ in range(3))


@torch.library.custom_op("t2t::qkv_rope_backward", mutates_args=())
def qkv_rope_backward_op(dq: torch.Tensor, dk: torch.Tensor, dv: torch.Tensor, cos: torch.Tensor,
                         sin: torch.Tensor, pos0: int) -> torch.Tensor:
    """dqkv [B, T, 3 H D]: transposed rotation of dq, dk; dv copied."""
    return _qkv_rope_bwd_impl(dq, dk, dv, cos, sin, pos0)


@qkv_rope_backward_op.register_fake
def _qkv_rope_backward_fake(dq, dk, dv, cos, sin, pos0):
    B, H, T, D = dq.shape
    return dq.new_empty((B, T, 3 * H * D))


def _qkv_rope_setup(ctx, inputs, output):
    _, cos, sin, _, pos0 = inputs
    ctx.save_for_backward(cos, sin)
    ctx.pos0 = pos0


def _qkv_rope_bwd(ctx, dq, dk, dv):
    # Unused outputs arrive as materialised zero gradients.
    cos, sin = ctx.saved_tensors
    return qkv_rope_backward_op(dq, dk, dv, cos, sin, ctx.pos0), None, None, None, None


qkv_rope_op.register_autograd(_qkv_rope_bwd, setup_context=_qkv_rope_setup)


class QKVRopeFn(torch.autograd.Function):
    """The same kernels as t2t::qkv_rope for eager execution (a plain
    autograd.Function has a fraction of the host cost of the custom op's
    registered autograd; compiled graphs trace the custom op)."""

    @staticmethod
    def forward(ctx, qkv, cos, sin, num_heads, pos0):
        ctx.save_for_backward(cos, sin)
        ctx.pos0 = pos0
        return _qkv_rope_impl(qkv, cos, sin, num_heads, pos0)

    @staticmethod
    def backward(ctx, dq, dk, dv):
        cos, sin = ctx.saved_tensors
        return _qkv_rope_bwd_impl(dq, dk, dv, cos, sin, ctx.pos0), None, None, None, None


def qkv_rope_torch(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, num_heads: int,
                   pos0: int = 0):
    """The same split and rotation composed from torch ops in qkv's dtype, for
    modules whose dtype the prologue kernel does not take (float32)."""
    B, T, D = _split_dims(qkv, num_heads)
    x = qkv.view(B, T, 3, num_heads, D).permute(2, 0, 3, 1, 4)  # [3, B, H, T, D]
    c = cos[pos0:pos0 + T].to(qkv.dtype)
    s = sin[pos0:pos0 + T].to(qkv.dtype)
    h = D // 2

    def rot(t):
        t1, t2 = t[..., :h], t[..., h:]
        return torch.cat((t1 * c + t2 * s, t2 * c - t1 * s), dim=-1)

    return rot(x[0]).contiguous(), rot(x[1]).contiguous(), x[2].contiguous()


def qkv_rope(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, num_heads: int,
             pos0: int = 0):
    """Split qkv [B, T, 3 C] into rotated q, k and v, each [B, H, T, D]
    (contiguous), with positions pos0 .. pos0 + T - 1 (table rows).  bf16 runs
    the kernel; float32 (module not cast to bf16) the torch composition."""
    if qkv.dtype == torch.float32:
        return qkv_rope_torch(qkv, cos, sin, num_heads, pos0)
    if torch.compiler.is_compiling():
        return qkv_rope_op(qkv, cos, sin, int(num_heads), int(pos0))
    return QKVRopeFn.apply(qkv, cos, sin, int(num_heads), int(pos0))
