"""Decode-step attention on the gfx950 kernels: a few new query rows against
a key/value cache, the mask evaluated per key from the per-token mask inputs
(doc ids and q / kv words, the layout ``T2TBlockMask`` carries).

Replaces, for generation, the full recompute the reference does per token
(model/generation_loop.py:90-92 -> TS2TSModel.forward_inference,
model/model.py:214-237).  Kernel: libt2t_attn.so ``t2t_attn_decode``.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from . import _lib

MAX_ROWS = 8  # (Hq / Hkv) * Tq per call


def _stream_ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _view(t: torch.Tensor) -> _lib.T2TTensor:
    return _lib.tensor_struct(t)


def attn_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, n_keys: int,
                key_doc: torch.Tensor, key_bits: Optional[torch.Tensor], q_pos: torch.Tensor,
                q_doc: torch.Tensor, q_bits: Optional[torch.Tensor],
                scale: Optional[float] = None, out: Optional[torch.Tensor] = None):
    """Attention of the new rows q [B, Hq, Tq, D] over cache positions
    0 .. n_keys - 1 of k_cache / v_cache [B, Hkv, cap, D].

    key_doc int32 [Bm, cap], key_bits int64 [Bm, W, cap] (or None for W = 0);
    q_pos / q_doc int32 [Bm, Tq], q_bits int64 [Bm, W, Tq].  Key j is allowed
    for row t iff j <= q_pos[t] and (key_doc[j] == q_doc[t] or the rows share a
    word bit).  Returns (o [B, Hq, Tq, D] bf16, lse2 float32 [B, Hq, Tq], log2
    domain).  (Hq / Hkv) * Tq must be at most 8."""
    B, Hq, Tq, D = q.shape
    Hkv = k_cache.shape[1]
    if q.dtype != torch.bfloat16 or k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise NotImplementedError("bfloat16 only")
    if not (q.is_cuda and k_cache.is_cuda and v_cache.is_cuda):
        raise RuntimeError("the decode kernel needs ROCm GPU tensors")
    W = 0 if key_bits is None else int(key_bits.shape[1])
    if (q_bits is None) != (key_bits is None) or (q_bits is not None and q_bits.shape[1] != W):
        raise ValueError("q_bits and key_bits must both be given with the same word count")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    for name, t in (("key_doc", key_doc), ("q_pos", q_pos), ("q_doc", q_doc)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int32 tensor")
    for name, t in (("key_bits", key_bits), ("q_bits", q_bits)):
        if t is not None and (t.dtype != torch.int64 or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous int64 tensor")
    Bm, cap = key_doc.shape
    if Bm not in (1, B):
        raise ValueError(f"mask batch {Bm} does not broadcast to B={B}")
    if k_cache.shape != v_cache.shape or k_cache.shape[0] != B or k_cache.shape[3] != D:
        raise ValueError(f"caches {tuple(k_cache.shape)} / {tuple(v_cache.shape)} do not fit "
                         f"q {tuple(q.shape)}")
    if not 0 <= n_keys <= min(cap, k_cache.shape[2]):
        raise ValueError(f"n_keys={n_keys} exceeds the cache ({k_cache.shape[2]} rows, "
                         f"{cap} mask slots)")
    if tuple(q_pos.shape) != (Bm, Tq) or tuple(q_doc.shape) != (Bm, Tq):
        raise ValueError(f"q_pos / q_doc must be [{Bm}, {Tq}]")
    if key_bits is not None and (tuple(key_bits.shape) != (Bm, W, cap)
                                 or tuple(q_bits.shape) != (Bm, W, Tq)):
        raise ValueError(f"key_bits must be [{Bm}, {W}, {cap}] and q_bits [{Bm}, {W}, {Tq}]")
    if q.stride(3) != 1:
        q = q.contiguous()
    o = out if out is not None else torch.empty((B, Hq, Tq, D), dtype=q.dtype, device=q.device)
    lse2 = torch.empty((B, Hq, Tq), dtype=torch.float32, device=q.device)
    L = _lib.lib()
    nbytes = L.t2t_attn_decode_workspace(B, Hq, Tq, n_keys, D)
    ws = torch.empty(max(1, nbytes // 4), dtype=torch.float32, device=q.device)
    qs, ks, vs, os_ = _view(q), _view(k_cache), _view(v_cache), _view(o)
    with torch.cuda.device(q.device):
        rc = L.t2t_attn_decode(ctypes.byref(qs), ctypes.byref(ks), ctypes.byref(vs),
                               ctypes.byref(os_), lse2.data_ptr(), key_doc.data_ptr(),
                               key_bits.data_ptr() if key_bits is not None else None,
                               key_doc.shape[1], q_pos.data_ptr(), q_doc.data_ptr(),
                               q_bits.data_ptr() if q_bits is not None else None,
                               key_doc.shape[0], W, B, Hq, Hkv, Tq, n_keys, D,
                               _lib.T2T_DTYPE_BF16, float(scale), ws.data_ptr(), ws.numel() * 4,
                               _stream_ptr(q))
    _lib.check(rc, "t2t_attn_decode")
    return o, lse2
