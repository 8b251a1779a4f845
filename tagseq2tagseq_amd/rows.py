"""Fused linear maps of a few token rows for generation steps
(``t2t_rows_linear``, ``t2t_rows_qkv_rope``).

A generation step sends one to eight new rows through each layer
(model/modules/layer.py:32-35).  Per layer the unfused sequence is an RMSNorm,
the qkv nn.Linear, the head split and rotation, two cache writes, the
out-projection and its residual add, a second RMSNorm, gate_up, SwiGLU (a
chunk, silu and a product), down and its residual add; at one row every one
of these is a separate launch whose cost is latency, not bytes.  Here the
layer is four launches around the decode attention:

    rows_qkv_rope(x, qkv, ln_1)          -> q rows, k / v cache rows
    rows_linear(y, proj, add=x)          -> x
    rows_linear(x, gate_up, ln_2, swiglu)-> h
    rows_linear(h, down, add=x)          -> x

with the rounding points of the unfused sequence (see the kernel source,
csrc/rows_linear.hip).  Only bf16 rows and weights on the GPU are served;
callers check ``applies`` and keep the torch sequence otherwise.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Union

import torch

from . import _lib

_EPILOGUES = {"store": _lib.T2T_ROWS_STORE, "add": _lib.T2T_ROWS_ADD,
              "swiglu": _lib.T2T_ROWS_SWIGLU}
_WDT = {torch.bfloat16: 0, torch.float32: 1}


def applies(x: torch.Tensor, *weights: torch.Tensor) -> bool:
    """bf16 rows on a GPU, at most ``ROWS_MAX`` of them and at most 4096 wide,
    bf16 weights."""
    rows = x.numel() // max(1, x.shape[-1])
    return (x.is_cuda and x.dtype == torch.bfloat16 and 0 < rows <= _lib.ROWS_MAX
            and 0 < x.shape[-1] <= 4096
            and all(w.dtype == torch.bfloat16 and w.is_cuda for w in weights))


def _rows(t: torch.Tensor) -> torch.Tensor:
    t = t.reshape(-1, t.shape[-1])
    return t if t.stride(1) == 1 and t.stride(0) >= t.shape[1] else t.contiguous()


def _norm_args(norm):
    if norm is None:
        return None, 0, 0.0
    w = norm.weight
    if not w.is_contiguous():
        raise ValueError("the norm weight must be contiguous")
    return w.data_ptr(), _WDT[w.dtype], float(norm.eps)


def _stream(x: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)


def rows_linear(x: torch.Tensor, weight: torch.Tensor, *, norm=None, epilogue: str = "store",
                res: Optional[torch.Tensor] = None, skip=None,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``epilogue(W · norm(x))`` for the rows of x [..., K] (at most 8 rows).

    weight: nn.Linear weight [N, K] ([2N, K] for "swiglu": gate rows then up
    rows); norm: an RMSNorm module (its ``weight`` and ``eps``) applied to x
    first, or None; res: rows [..., N] added for "add" (``out`` may be
    ``res``); skip: for "add", ``(rows or None, w)`` with w a one-element
    device tensor: the sum t then becomes t + w * rows (rows None: t + w * t),
    the backbone's weighted skip connection.  Returns [..., N] bf16."""
    if not weight.is_contiguous():
        raise ValueError("weight must be contiguous ([N, K] row-major)")
    K = x.shape[-1]
    xr = _rows(x)
    M = xr.shape[0]
    N = weight.shape[0] // 2 if epilogue == "swiglu" else weight.shape[0]
    if weight.shape[-1] != K:
        raise ValueError(f"weight {tuple(weight.shape)} does not take rows of {K}")
    y = out.reshape(M, N) if out is not None else torch.empty((M, N), dtype=x.dtype,
                                                                device=x.device)
    rr = res.reshape(M, N) if res is not None else None
    if rr is not None and rr.stride(1) != 1:
        raise ValueError("res rows must have unit stride")
    if y.stride(1) != 1:
        raise ValueError("out rows must have unit stride")
    nw, ndt, eps = _norm_args(norm)
    sk = sw = None
    if skip is not None:
        sk, sw = skip
        if sw.numel() != 1 or sw.dtype not in _WDT or not sw.is_cuda:
            raise ValueError("the skip weight must be a one-element bf16 / float32 device tensor")
        if sk is not None:
            sk = sk.reshape(M, N)
            if sk.stride(1) != 1:
                raise ValueError("skip rows must have unit stride")
    with torch.cuda.device(x.device):
        rc = _lib.lib().t2t_rows_linear(
            xr.data_ptr(), xr.stride(0), M, K, weight.data_ptr(), N, nw, ndt, eps,
            _EPILOGUES[epilogue], rr.data_ptr() if rr is not None else None,
            rr.stride(0) if rr is not None else 0, sk.data_ptr() if sk is not None else None,
            sk.stride(0) if sk is not None else 0, sw.data_ptr() if sw is not None else None,
            _WDT[sw.dtype] if sw is not None else 0, y.data_ptr(), y.stride(0), _stream(x))
    _lib.check(rc, "t2t_rows_linear")
    return y.view(*x.shape[:-1], N)


def rows_qkv_rope(x: torch.Tensor, weight: torch.Tensor, num_heads: int, cos: torch.Tensor,
                  sin: torch.Tensor, pos: Union[int, torch.Tensor], k_cache: torch.Tensor,
                  v_cache: torch.Tensor, *, norm=None) -> torch.Tensor:
    """qkv projection of the rows of x [..., C] (at most 8 rows) with the
    rotary embedding: returns q [1, H, M, D] and writes the rotated k and the
    v rows into k_cache / v_cache [1, H, capacity, D] at their positions.

    pos: the first row's position (rows at pos .. pos + M - 1) or a device
    int64 tensor [M] of positions (read by the kernel; rows outside the
    tables or the cache are not written).  cos, sin: the rotary tables
    [rows, D / 2] (float32, contiguous)."""
    C = x.shape[-1]
    H = int(num_heads)
    D = C // H
    if weight.shape != (3 * C, C) or not weight.is_contiguous():
        raise ValueError(f"qkv weight {tuple(weight.shape)} is not a contiguous [3C, C]")
    for t in (cos, sin):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.shape[-1] != D // 2:
            raise ValueError("cos / sin must be contiguous float32 [rows, D / 2]")
    if k_cache.shape != v_cache.shape or k_cache.shape[1] != H or k_cache.shape[3] != D:
        raise ValueError("k_cache / v_cache must both be [1, H, capacity, D]")
    xr = _rows(x)
    M = xr.shape[0]
    q = torch.empty((1, H, M, D), dtype=x.dtype, device=x.device)
    if isinstance(pos, torch.Tensor):
        if pos.dtype != torch.int64 or pos.numel() != M or not pos.is_cuda:
            raise ValueError("pos must be a device int64 tensor with one entry per row")
        pos = pos.contiguous()
        pos_ptr, pos0 = pos.data_ptr(), 0
    else:
        pos_ptr, pos0 = None, int(pos)
    nw, ndt, eps = _norm_args(norm)
    qv, kv, vv = (_lib.tensor_struct(t) for t in (q, k_cache, v_cache))
    with torch.cuda.device(x.device):
        rc = _lib.lib().t2t_rows_qkv_rope(
            xr.data_ptr(), xr.stride(0), M, C, weight.data_ptr(), nw, ndt, eps, H, D,
            cos.data_ptr(), sin.data_ptr(), cos.shape[0], pos_ptr, pos0, ctypes.byref(qv),
            ctypes.byref(kv), ctypes.byref(vv), k_cache.shape[2], _stream(x))
    _lib.check(rc, "t2t_rows_qkv_rope")
    return q
