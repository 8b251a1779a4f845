"""Device-side BlockMask for the gfx950 masked-attention path.

``T2TBlockMask`` carries the per-token mask inputs of the reference's
``mask_mod`` (document ids and grant words, model/graph_traversal/
cross_doc_mask.py:348-357) together with the BlockMask tables torch's
``create_block_mask`` derives from them (torch/nn/attention/flex_attention.py:
1144-1225): 128 x 128 tile classes and the eight ordered index tables
(kv_num_blocks, kv_indices, full_kv_num_blocks, full_kv_indices, q_num_blocks,
q_indices, full_q_num_blocks, full_q_indices; shapes [Bm, 1, nt] and
[Bm, 1, nt, nt] as in torch's BlockMask).  The tables are computed on the GPU
by ``t2t_mask_meta`` without materialising the [T, T] mask.

``to_block_mask()`` rebuilds a torch ``BlockMask`` from the same tables (via
``BlockMask.from_kv_blocks``) for interoperability with torch's own
flex_attention.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _lib

TILE = _lib.TILE


@dataclass
class T2TBlockMask:
    seq_len: int
    doc_ids: torch.Tensor          # int32 [Bm, T]
    q_bits: torch.Tensor           # int64 [Bm, W, T] (bit patterns of uint64 words)
    kv_bits: torch.Tensor          # int64 [Bm, W, T]
    tile_class: torch.Tensor       # int8  [Bm, nt, nt]: 0 skip, 1 partial, 2 full
    kv_num_blocks: torch.Tensor    # int32 [Bm, 1, nt]
    kv_indices: torch.Tensor       # int32 [Bm, 1, nt, nt]
    full_kv_num_blocks: torch.Tensor
    full_kv_indices: torch.Tensor
    q_num_blocks: torch.Tensor
    q_indices: torch.Tensor
    full_q_num_blocks: torch.Tensor
    full_q_indices: torch.Tensor
    BLOCK_SIZE: tuple = (TILE, TILE)
    _c: Optional[_lib.T2TMask] = field(default=None, repr=False)

    @property
    def mask_batch(self) -> int:
        return int(self.doc_ids.shape[0])

    @property
    def words(self) -> int:
        return int(self.q_bits.shape[1])

    @property
    def num_tiles(self) -> int:
        return int(self.tile_class.shape[-1])

    @property
    def shape(self):
        return (self.mask_batch, 1, self.seq_len, self.seq_len)

    @property
    def seq_lengths(self):
        return (self.seq_len, self.seq_len)

    def c_struct(self) -> _lib.T2TMask:
        if self._c is None:
            w = self.words
            self._c = _lib.T2TMask(
                self.doc_ids.data_ptr(),
                self.q_bits.data_ptr() if w else None,
                self.kv_bits.data_ptr() if w else None,
                w, self.mask_batch,
                self.kv_num_blocks.data_ptr(), self.kv_indices.data_ptr(),
                self.full_kv_num_blocks.data_ptr(), self.full_kv_indices.data_ptr(),
                self.q_num_blocks.data_ptr(), self.q_indices.data_ptr(),
                self.full_q_num_blocks.data_ptr(), self.full_q_indices.data_ptr())
        return self._c

    def mask_mod(self):
        """The reference's mask_mod over this mask's per-token tensors
        (cross_doc_mask.py:348-357; doc_causal when there are no words)."""
        doc, qb, kb = self.doc_ids, self.q_bits, self.kv_bits
        W = self.words

        def t2t_mask_mod(b, h, q_idx, kv_idx):
            bb = b if doc.shape[0] > 1 else 0
            same = doc[bb, q_idx] == doc[bb, kv_idx]
            for w in range(W):
                same = same | ((qb[bb, w, q_idx] & kb[bb, w, kv_idx]) != 0)
            return (q_idx >= kv_idx) & same

        return t2t_mask_mod

    def to_block_mask(self):
        """torch BlockMask with identical tables (for torch's flex_attention)."""
        from torch.nn.attention.flex_attention import BlockMask
        return BlockMask.from_kv_blocks(
            self.kv_num_blocks, self.kv_indices, self.full_kv_num_blocks, self.full_kv_indices,
            BLOCK_SIZE=self.BLOCK_SIZE, mask_mod=self.mask_mod(),
            seq_lengths=(self.seq_len, self.seq_len))

    def sparsity(self) -> float:
        """Percentage of tiles that are skipped (torch BlockMask.sparsity)."""
        tc = self.tile_class
        return 100.0 * float((tc == 0).sum().item()) / max(1, tc.numel())


def _as_words(bits: Optional[torch.Tensor], Bm: int, T: int, device) -> torch.Tensor:
    if bits is None:
        return torch.zeros((Bm, 0, T), dtype=torch.int64, device=device)
    if bits.dtype not in (torch.int64, torch.uint64):
        raise TypeError(f"grant words must be int64/uint64, got {bits.dtype}")
    if bits.dim() == 2:
        bits = bits.unsqueeze(0)
    return bits.to(device=device).view(torch.int64).contiguous()


def build_block_mask(doc_ids: torch.Tensor, q_bits: Optional[torch.Tensor] = None,
                     kv_bits: Optional[torch.Tensor] = None,
                     stream: Optional[torch.cuda.Stream] = None) -> T2TBlockMask:
    """Run the metadata pass on the GPU.

    doc_ids: int32 [T] or [Bm, T] on a ROCm device.
    q_bits / kv_bits: int64 (or uint64) [W, T] or [Bm, W, T] grant words, or None.
    """
    if not doc_ids.is_cuda:
        raise RuntimeError("build_block_mask needs doc_ids on a ROCm GPU device "
                           "(the masked-attention path has no CPU implementation)")
    device = doc_ids.device
    if doc_ids.dim() == 1:
        doc_ids = doc_ids.unsqueeze(0)
    doc_ids = doc_ids.to(torch.int32).contiguous()
    Bm, T = doc_ids.shape
    qb = _as_words(q_bits, Bm, T, device)
    kb = _as_words(kv_bits, Bm, T, device)
    if qb.shape != kb.shape or qb.shape[0] != Bm or qb.shape[2] != T:
        raise ValueError(f"q_bits {tuple(qb.shape)} / kv_bits {tuple(kb.shape)} do not match "
                         f"doc_ids {tuple(doc_ids.shape)}")
    W = qb.shape[1]
    if W > _lib.MAX_WORDS:
        raise ValueError(f"{W} grant words exceed the supported {_lib.MAX_WORDS}")
    nt = (T + TILE - 1) // TILE
    i32 = dict(dtype=torch.int32, device=device)
    tile_class = torch.empty((Bm, nt, nt), dtype=torch.int8, device=device)
    tabs = {}
    for name in ("kv", "full_kv", "q", "full_q"):
        tabs[name + "_num"] = torch.empty((Bm, 1, nt), **i32)
        tabs[name + "_idx"] = torch.empty((Bm, 1, nt, nt), **i32)
    s = stream if stream is not None else torch.cuda.current_stream(device)
    with torch.cuda.device(device):
        rc = _lib.lib().t2t_mask_meta(
            doc_ids.data_ptr(), qb.data_ptr() if W else None, kb.data_ptr() if W else None,
            Bm, T, W, tile_class.data_ptr(),
            tabs["kv_num"].data_ptr(), tabs["kv_idx"].data_ptr(),
            tabs["full_kv_num"].data_ptr(), tabs["full_kv_idx"].data_ptr(),
            tabs["q_num"].data_ptr(), tabs["q_idx"].data_ptr(),
            tabs["full_q_num"].data_ptr(), tabs["full_q_idx"].data_ptr(),
            ctypes.c_void_p(s.cuda_stream))
    _lib.check(rc, "t2t_mask_meta")
    return T2TBlockMask(
        seq_len=T, doc_ids=doc_ids, q_bits=qb, kv_bits=kb, tile_class=tile_class,
        kv_num_blocks=tabs["kv_num"], kv_indices=tabs["kv_idx"],
        full_kv_num_blocks=tabs["full_kv_num"], full_kv_indices=tabs["full_kv_idx"],
        q_num_blocks=tabs["q_num"], q_indices=tabs["q_idx"],
        full_q_num_blocks=tabs["full_q_num"], full_q_indices=tabs["full_q_idx"])
