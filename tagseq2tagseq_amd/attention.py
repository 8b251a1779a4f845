"""Masked attention entry points: the ``flex_attention`` seam, its autograd
Function and a ``FlexSelfAttention``-shaped module.

Seams replaced (reference file:line):
  * ``flex_attention(q, k, v, block_mask=..., scale=None, enable_gqa=False)`` --
    the module-global symbol the reference's attention module calls
    (model/modules/layer.py:16-21,33; monkey-patched at generate.py:167-178),
    i.e. torch/nn/attention/flex_attention.py:1396-1676.
  * FlexAttentionAutogradOp (torch/_higher_order_ops/flex_attention.py:628-767)
    -- twice, over the same kernels: ``T2TFlexAttentionFn``, a plain
    autograd.Function that eager calls use (saves q, k, v, out and the
    log2-domain LSE; backward = atomic-free dK/dV + dQ kernels), and
    ``torch.ops.t2t.masked_attention`` / ``t2t::masked_attention_backward``,
    ``torch.library`` custom ops with fake implementations and registered
    autograd that compiled graphs trace.  ``flex_attention`` picks the custom
    op while torch.compile traces and the Function otherwise: the custom op's
    registered autograd costs several hundred microseconds of host time per
    call, the Function tens.
  * ``FlexSelfAttention(dim, num_heads, max_seq_len, fp8_out_proj)`` with
    ``forward(x, block_mask)`` -- the constructor / call signature the
    reference's Layer uses (model/modules/layer.py:16-21,33).

All compute runs in libt2t_attn.so on the current ROCm stream.
"""
from __future__ import annotations

import ctypes
import math
import warnings
from typing import Optional

import torch
import torch.nn as nn

from . import _lib
from typing import List, Tuple

from .block_mask import T2TBlockMask, from_torch_block_mask, tables_c_struct
from .linear import Linear

LN2 = math.log(2.0)
_DTYPE_CODES = {torch.bfloat16: _lib.T2T_DTYPE_BF16, torch.float32: _lib.T2T_DTYPE_F32}


def _stream_ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _view(t: torch.Tensor) -> _lib.T2TTensor:
    s = _lib.tensor_struct(t)
    # size-1 dims may carry arbitrary strides; they are never stepped
    if t.shape[0] == 1:
        s.stride_b = 0
    if t.shape[1] == 1:
        s.stride_h = 0
    return s


def as_t2t_block_mask(block_mask):
    """A T2TBlockMask, or a torch BlockMask converted once
    (block_mask.from_torch_block_mask) and kept on the BlockMask object, so
    that every layer of a step reuses the conversion."""
    if isinstance(block_mask, T2TBlockMask):
        return block_mask
    from torch.nn.attention.flex_attention import BlockMask
    if not isinstance(block_mask, BlockMask):
        raise TypeError(f"block_mask must be a T2TBlockMask or a torch BlockMask, "
                        f"got {type(block_mask).__name__}")
    conv = getattr(block_mask, "_t2t_block_mask", None)
    if conv is None:
        conv = from_torch_block_mask(block_mask)
        block_mask._t2t_block_mask = conv
    return conv


def _validate(q, k, v, block_mask, enable_gqa):
    """Shape rules of torch/nn/attention/flex_attention.py:1473-1541."""
    if not isinstance(block_mask, T2TBlockMask):
        raise TypeError("block_mask must be a T2TBlockMask (build one with the mask creators "
                        "in tagseq2tagseq_amd.mask_creators, or pass a torch BlockMask to "
                        "flex_attention)")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("query, key, value must be 4-D [B, H, T, D]")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"dtype mismatch: {q.dtype}, {k.dtype}, {v.dtype}")
    if q.dtype not in _DTYPE_CODES:
        raise NotImplementedError(f"dtype {q.dtype} is not supported (bfloat16 or float32)")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("the masked-attention kernels need ROCm GPU tensors")
    B, Hq, T, D = q.shape
    if k.shape[0] != B or v.shape[0] != B:
        raise ValueError("batch sizes of query, key, value differ")
    if k.shape[2] != T or v.shape[2] != T:
        raise ValueError("query and key/value sequence lengths must match (self-attention)")
    if k.shape[3] != D or v.shape[3] != D:
        raise ValueError("query, key and value head dims must match")
    if k.shape[1] != v.shape[1]:
        raise ValueError("key and value head counts differ")
    Hkv = k.shape[1]
    if Hq != Hkv:
        if not enable_gqa:
            raise ValueError(f"Expect query and key/value to have the same number of heads but got "
                             f"Hq={Hq} and Hkv={Hkv}. Try setting enable_gqa=True for GQA.")
        if Hq % Hkv != 0:
            raise ValueError(f"Expect number of query heads to be a multiple of kv heads for GQA "
                             f"but got Hq={Hq} and Hkv={Hkv}.")
    if block_mask.seq_len != T:
        raise ValueError(f"block_mask was built for T={block_mask.seq_len} but inputs have T={T}")
    if block_mask.mask_batch not in (1, B):
        raise ValueError(f"block_mask batch {block_mask.mask_batch} does not broadcast to B={B}")
    if D not in (64, 128):
        raise NotImplementedError(f"head dim {D} is not supported (64 or 128)")
    return B, Hq, Hkv, T, D


def _mask_struct(block_mask):
    """struct t2t_block_mask of a T2TBlockMask or of its list of tables."""
    if isinstance(block_mask, T2TBlockMask):
        return block_mask.c_struct()
    return tables_c_struct(block_mask)


def attn_fwd(q, k, v, block_mask, scale: float):
    """Kernel call: returns (out [B,Hq,T,D] in q.dtype, lse2 float32 [B,Hq,T]).
    ``block_mask``: a T2TBlockMask or its ``tables()`` list."""
    B, Hq, Hkv, T, D = q.shape[0], q.shape[1], k.shape[1], q.shape[2], q.shape[3]
    # [B, T, Hq, D] storage seen as [B, Hq, T, D]: the module's output
    # projection then reads token rows without a transpose copy.
    out = torch.empty((B, T, Hq, D), dtype=q.dtype, device=q.device).transpose(1, 2)
    lse2 = torch.empty((B, Hq, T), dtype=torch.float32, device=q.device)
    qs, ks, vs, os_ = _view(q), _view(k), _view(v), _view(out)
    with torch.cuda.device(q.device):
        rc = _lib.lib().t2t_attn_fwd(ctypes.byref(qs), ctypes.byref(ks), ctypes.byref(vs),
                                     ctypes.byref(os_), lse2.data_ptr(), B, Hq, Hkv, T, D,
                                     _DTYPE_CODES[q.dtype], float(scale),
                                     ctypes.byref(_mask_struct(block_mask)), _stream_ptr(q))
    _lib.check(rc, "t2t_attn_fwd")
    return out, lse2


def attn_bwd(q, k, v, out, dout, lse2, block_mask, scale: float):
    """Kernel call: returns (dq, dk, dv).  ``block_mask`` as in attn_fwd."""
    B, Hq, Hkv, T, D = q.shape[0], q.shape[1], k.shape[1], q.shape[2], q.shape[3]
    if dout.stride(3) != 1:
        dout = dout.contiguous()
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    delta = torch.empty((B, Hq, T), dtype=torch.float32, device=q.device)
    views = [_view(t) for t in (q, k, v, out, dout)]
    gviews = [_view(t) for t in (dq, dk, dv)]
    with torch.cuda.device(q.device):
        rc = _lib.lib().t2t_attn_bwd(*[ctypes.byref(x) for x in views], lse2.data_ptr(),
                                     delta.data_ptr(), *[ctypes.byref(x) for x in gviews],
                                     B, Hq, Hkv, T, D, _DTYPE_CODES[q.dtype], float(scale),
                                     ctypes.byref(_mask_struct(block_mask)), _stream_ptr(q))
    _lib.check(rc, "t2t_attn_bwd")
    return dq, dk, dv


class BwdPhases:
    """The three backward launches bound to fixed buffers (t2t_attn_bwd_preprocess,
    t2t_attn_bwd_dkdv, t2t_attn_bwd_dq), for callers that schedule or time
    them separately, and ``whole`` = t2t_attn_bwd on the same buffers (its dQ
    launch computes Delta itself, then dK/dV)."""

    def __init__(self, q, k, v, out, dout, lse2, block_mask: T2TBlockMask, scale: float):
        self.B, self.Hq, self.T, self.D = q.shape
        self.Hkv = k.shape[1]
        self.dq = torch.empty_like(q, memory_format=torch.contiguous_format)
        self.dk = torch.empty_like(k, memory_format=torch.contiguous_format)
        self.dv = torch.empty_like(v, memory_format=torch.contiguous_format)
        self.delta = torch.empty((self.B, self.Hq, self.T), dtype=torch.float32, device=q.device)
        self._keep = (q, k, v, out, dout, lse2, block_mask)
        self._v = {n: _view(t) for n, t in dict(q=q, k=k, v=v, o=out, do=dout, dq=self.dq,
                                                 dk=self.dk, dv=self.dv).items()}
        self._lse2 = lse2.data_ptr()
        self._mask = block_mask.c_struct()
        self._dtype = _DTYPE_CODES[q.dtype]
        self._scale = float(scale)
        self._dev = q.device

    def preprocess(self):
        v = self._v
        rc = _lib.lib().t2t_attn_bwd_preprocess(ctypes.byref(v["o"]), ctypes.byref(v["do"]),
                                                self.delta.data_ptr(), self.B, self.Hq, self.T,
                                                self.D, self._dtype, _stream_ptr(self.delta))
        _lib.check(rc, "t2t_attn_bwd_preprocess")

    def dkdv(self):
        v = self._v
        rc = _lib.lib().t2t_attn_bwd_dkdv(
            ctypes.byref(v["q"]), ctypes.byref(v["k"]), ctypes.byref(v["v"]), ctypes.byref(v["do"]),
            self._lse2, self.delta.data_ptr(), ctypes.byref(v["dk"]), ctypes.byref(v["dv"]),
            self.B, self.Hq, self.Hkv, self.T, self.D, self._dtype, self._scale,
            ctypes.byref(self._mask), _stream_ptr(self.delta))
        _lib.check(rc, "t2t_attn_bwd_dkdv")

    def dq_pass(self):
        v = self._v
        rc = _lib.lib().t2t_attn_bwd_dq(
            ctypes.byref(v["q"]), ctypes.byref(v["k"]), ctypes.byref(v["v"]), ctypes.byref(v["do"]),
            self._lse2, self.delta.data_ptr(), ctypes.byref(v["dq"]),
            self.B, self.Hq, self.Hkv, self.T, self.D, self._dtype, self._scale,
            ctypes.byref(self._mask), _stream_ptr(self.delta))
        _lib.check(rc, "t2t_attn_bwd_dq")

    def whole(self):
        v = self._v
        rc = _lib.lib().t2t_attn_bwd(
            *[ctypes.byref(v[n]) for n in ("q", "k", "v", "o", "do")], self._lse2,
            self.delta.data_ptr(), *[ctypes.byref(v[n]) for n in ("dq", "dk", "dv")],
            self.B, self.Hq, self.Hkv, self.T, self.D, self._dtype, self._scale,
            ctypes.byref(self._mask), _stream_ptr(self.delta))
        _lib.check(rc, "t2t_attn_bwd")


class T2TFlexAttentionFn(torch.autograd.Function):
    """autograd.Function over the gfx950 kernels (in place of
    FlexAttentionAutogradOp, torch/_higher_order_ops/flex_attention.py:628-767)."""

    @staticmethod
    def forward(ctx, q, k, v, block_mask, scale):
        out, lse2 = attn_fwd(q, k, v, block_mask, scale)
        ctx.save_for_backward(q, k, v, out, lse2)
        ctx.block_mask = block_mask
        ctx.scale = scale
        ctx.mark_non_differentiable(lse2)
        return out, lse2

    @staticmethod
    def backward(ctx, dout, _dlse2):
        q, k, v, out, lse2 = ctx.saved_tensors
        dq, dk, dv = attn_bwd(q, k, v, out, dout, lse2, ctx.block_mask, ctx.scale)
        return dq, dk, dv, None, None


@torch.library.custom_op("t2t::masked_attention", mutates_args=())
def masked_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     tables: List[torch.Tensor], scale: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """Masked attention forward on the gfx950 kernels: (out, lse2).  ``tables``
    = T2TBlockMask.tables() (the mask as tensors, so the op has a schema)."""
    return attn_fwd(q, k, v, tables, scale)


@masked_attention.register_fake
def _masked_attention_fake(q, k, v, tables, scale):
    B, Hq, T, D = q.shape
    return (q.new_empty((B, T, Hq, D)).transpose(1, 2),
            q.new_empty((B, Hq, T), dtype=torch.float32))


@torch.library.custom_op("t2t::masked_attention_backward", mutates_args=())
def masked_attention_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                              out: torch.Tensor, dout: torch.Tensor, lse2: torch.Tensor,
                              tables: List[torch.Tensor],
                              scale: float) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dq, dk, dv) on the gfx950 kernels (Delta, dK/dV, dQ launches)."""
    return attn_bwd(q, k, v, out, dout, lse2, tables, scale)


@masked_attention_backward.register_fake
def _masked_attention_backward_fake(q, k, v, out, dout, lse2, tables, scale):
    return (torch.empty_like(q, memory_format=torch.contiguous_format),
            torch.empty_like(k, memory_format=torch.contiguous_format),
            torch.empty_like(v, memory_format=torch.contiguous_format))


def _masked_attention_setup(ctx, inputs, output):
    q, k, v, tables, scale = inputs
    out, lse2 = output
    ctx.save_for_backward(q, k, v, out, lse2, *tables)
    ctx.scale = scale


def _masked_attention_bwd(ctx, dout, _dlse2):
    q, k, v, out, lse2, *tables = ctx.saved_tensors
    dq, dk, dv = masked_attention_backward(q, k, v, out, dout.contiguous(), lse2, tables, ctx.scale)
    return dq, dk, dv, [None] * len(tables), None


masked_attention.register_autograd(_masked_attention_bwd, setup_context=_masked_attention_setup)


def flex_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                   score_mod=None, block_mask: Optional[T2TBlockMask] = None,
                   scale: Optional[float] = None, enable_gqa: bool = False,
                   return_lse: bool = False, kernel_options=None):
    """Drop-in for torch's flex_attention on the doc_causal / cross_doc_link
    path (torch/nn/attention/flex_attention.py:1396-1676).

    ``block_mask`` is a T2TBlockMask from this package's mask creators or a
    torch BlockMask (128 x 128 tiles, one mask for every head, e.g. from
    create_block_mask); the latter is converted once and the conversion kept
    on it (as_t2t_block_mask).

    ``score_mod`` must be None (the reference passes none).  The returned LSE is
    in natural log, as torch's (internal log2 value times ln 2, :1575-1600).
    """
    if score_mod is not None:
        raise NotImplementedError("score_mod is not supported by the gfx950 masked-attention path")
    if block_mask is None:
        raise ValueError("block_mask is required (build it with tagseq2tagseq_amd.mask_creators)")
    if not query.is_cuda:
        raise RuntimeError("the masked-attention kernels need ROCm GPU tensors")
    block_mask = as_t2t_block_mask(block_mask)
    _, _, _, _, D = _validate(query, key, value, block_mask, enable_gqa)
    if scale is None:
        scale = 1.0 / math.sqrt(D)  # torch/nn/attention/flex_attention.py:1544
    if not (math.isfinite(scale) and scale > 0.0):
        raise ValueError(f"scale={scale!r}: the gfx950 kernels need a positive finite scale")
    if torch.compiler.is_compiling():
        # compiled graphs trace the custom op (schema + fake implementation)
        out, lse2 = masked_attention(query, key, value, block_mask.tables(), float(scale))
    else:
        # eager: the same kernels through a plain autograd.Function, whose host
        # cost per call is a fraction of the custom op's registered autograd
        out, lse2 = T2TFlexAttentionFn.apply(query, key, value, block_mask, float(scale))
    if return_lse:
        return out, lse2 * LN2
    return out


class Rotary(nn.Module):
    """Rotary-embedding tables for [B, H, T, D] heads: half-split pairs, base
    10000, position = token index (float32 [max_seq_len, D/2] cos / sin, kept
    in float32 whatever dtype the module is cast to)."""

    def __init__(self, head_dim: int, max_seq_len: int, base: float = 10000.0):
        super().__init__()
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.base = base

    def tables(self, device):
        from .rope import rope_tables
        return rope_tables(self.head_dim, self.max_seq_len, device, self.base)


class FlexSelfAttention(nn.Module):
    """Self-attention with the constructor and call signature the reference's
    Layer uses (model/modules/layer.py:16-21, 33): QKV projection, rotary
    embedding, masked attention on the gfx950 kernels, output projection.

    The head split and rotation run as one prologue kernel (t2t::qkv_rope);
    the attention output is produced in [B, T, H, D] order, so the output
    projection reads it without a transpose copy.  The reference's module
    comes from the absent ``tunalab`` package; its internal details (RoPE
    variant, QK-norm, fp8 out-projection) are not available here, so
    ``fp8_out_proj=True`` is accepted for signature compatibility, warned
    about once, and the output projection stays in the module's dtype.
    """

    def __init__(self, dim: int, num_heads: int, max_seq_len: int, fp8_out_proj: bool = False):
        super().__init__()
        if dim % num_heads != 0:
            raise ValueError("dim must be divisible by num_heads")
        self.dim = dim
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.qkv = Linear(dim, 3 * dim, bias=False)
        self.proj = Linear(dim, dim, bias=False)
        self.rotary = Rotary(self.head_dim, max_seq_len)
        self.fp8_out_proj = fp8_out_proj
        if fp8_out_proj:
            warnings.warn("FlexSelfAttention(fp8_out_proj=True): the fp8 output projection is not "
                          "implemented; the projection runs in the module's dtype", stacklevel=2)

    def forward(self, x: torch.Tensor, block_mask: T2TBlockMask) -> torch.Tensor:
        from .rope import qkv_rope
        B, T, C = x.shape
        cos, sin = self.rotary.tables(x.device)
        q, k, v = qkv_rope(self.qkv(x), cos, sin, self.num_heads)
        y = flex_attention(q, k, v, block_mask=block_mask)
        return self.proj(y.transpose(1, 2).reshape(B, T, C))
