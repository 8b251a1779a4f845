"""Device-side BlockMask for the gfx950 masked-attention path.

``T2TBlockMask`` carries the per-token mask inputs of the reference's
``mask_mod`` (document ids and grant words, model/graph_traversal/
cross_doc_mask.py:348-357) together with the BlockMask tables torch's
``create_block_mask`` derives from them (torch/nn/attention/flex_attention.py:
1144-1225): 128 x 128 tile classes and the eight ordered index tables
(kv_num_blocks, kv_indices, full_kv_num_blocks, full_kv_indices, q_num_blocks,
q_indices, full_q_num_blocks, full_q_indices; shapes [Bm, 1, nt] and
[Bm, 1, nt, nt] as in torch's BlockMask).  The metadata kernel computes them on
the GPU without materialising the [T, T] mask, plus launch orders and a
128 x 128 allowed-pair bitmap per partial tile that the attention kernels use
for element masking.

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
    row_order: torch.Tensor        # int32 [Bm, nt]
    col_order: torch.Tensor        # int32 [Bm, nt]
    kv_bits_off: torch.Tensor      # int32 [Bm, nt]
    q_bits_slot: torch.Tensor      # int32 [Bm, nt, nt]
    tile_bits: torch.Tensor        # int32 [slots, 2, 128, 4]
    BLOCK_SIZE: tuple = (TILE, TILE)
    _c: Optional[_lib.T2TBlockMaskC] = field(default=None, repr=False)

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

    def tables(self):
        """The 13 device tables the kernels read, in t2t_block_mask order."""
        return [self.kv_num_blocks, self.kv_indices, self.full_kv_num_blocks,
                self.full_kv_indices, self.q_num_blocks, self.q_indices, self.full_q_num_blocks,
                self.full_q_indices, self.row_order, self.col_order, self.kv_bits_off,
                self.q_bits_slot, self.tile_bits]

    def c_struct(self) -> _lib.T2TBlockMaskC:
        if self._c is None:
            self._c = tables_c_struct(self.tables())
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


def tables_c_struct(tables) -> _lib.T2TBlockMaskC:
    """struct t2t_block_mask over the 13 tables of T2TBlockMask.tables()."""
    kv_num = tables[0]
    Bm, nt = int(kv_num.shape[0]), int(kv_num.shape[-1])
    return _lib.T2TBlockMaskC(Bm, nt, *[t.data_ptr() for t in tables], tables[-1].shape[0])


def _as_words(bits: Optional[torch.Tensor], Bm: int, T: int, device) -> torch.Tensor:
    if bits is None:
        return torch.zeros((Bm, 0, T), dtype=torch.int64, device=device)
    if bits.dtype not in (torch.int64, torch.uint64):
        raise TypeError(f"grant words must be int64/uint64, got {bits.dtype}")
    if bits.dim() == 2:
        bits = bits.unsqueeze(0)
    return bits.to(device=device).view(torch.int64).contiguous()


@dataclass
class MaskInputs:
    """The per-token inputs of a mask without its tile tables: what the
    decode-step kernel reads (doc ids and q / kv words per position)."""
    seq_len: int
    doc_ids: torch.Tensor          # int32 [Bm, T]
    q_bits: torch.Tensor           # int64 [Bm, W, T]
    kv_bits: torch.Tensor          # int64 [Bm, W, T]

    @property
    def mask_batch(self) -> int:
        return int(self.doc_ids.shape[0])

    @property
    def words(self) -> int:
        return int(self.q_bits.shape[1])


def mask_inputs(doc_ids: torch.Tensor, q_bits: Optional[torch.Tensor] = None,
                kv_bits: Optional[torch.Tensor] = None) -> MaskInputs:
    """The inputs build_block_mask takes, normalised to [Bm, T] / [Bm, W, T]."""
    if doc_ids.dim() == 1:
        doc_ids = doc_ids.unsqueeze(0)
    doc_ids = doc_ids.to(torch.int32).contiguous()
    Bm, T = doc_ids.shape
    qb = _as_words(q_bits, Bm, T, doc_ids.device)
    kb = _as_words(kv_bits, Bm, T, doc_ids.device)
    if qb.shape != kb.shape or qb.shape[0] != Bm or qb.shape[2] != T:
        raise ValueError(f"q_bits {tuple(qb.shape)} / kv_bits {tuple(kb.shape)} do not match "
                         f"doc_ids {tuple(doc_ids.shape)}")
    return MaskInputs(T, doc_ids, qb, kb)


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
    t = {}
    for name in ("kv", "full_kv", "q", "full_q"):
        t[name + "_num"] = torch.empty((Bm, 1, nt), **i32)
        t[name + "_idx"] = torch.empty((Bm, 1, nt, nt), **i32)
    row_order = torch.empty((Bm, nt), **i32)
    col_order = torch.empty((Bm, nt), **i32)
    kv_bits_off = torch.empty((Bm, nt), **i32)
    q_bits_slot = torch.empty((Bm, nt, nt), **i32)
    slots = max(1, Bm * nt * (nt + 1) // 2)
    tile_bits = torch.empty((slots, 2, TILE, 4), **i32)
    tabs = (t["kv_num"], t["kv_idx"], t["full_kv_num"], t["full_kv_idx"], t["q_num"], t["q_idx"],
            t["full_q_num"], t["full_q_idx"], row_order, col_order, kv_bits_off, q_bits_slot,
            tile_bits)
    cs = tables_c_struct(tabs)
    s = stream if stream is not None else torch.cuda.current_stream(device)
    with torch.cuda.device(device):
        rc = _lib.lib().t2t_mask_meta(
            doc_ids.data_ptr(), qb.data_ptr() if W else None, kb.data_ptr() if W else None,
            Bm, T, W, tile_class.data_ptr(), ctypes.byref(cs), ctypes.c_void_p(s.cuda_stream))
    _lib.check(rc, "t2t_mask_meta")
    return T2TBlockMask(
        seq_len=T, doc_ids=doc_ids, q_bits=qb, kv_bits=kb, tile_class=tile_class,
        kv_num_blocks=t["kv_num"], kv_indices=t["kv_idx"],
        full_kv_num_blocks=t["full_kv_num"], full_kv_indices=t["full_kv_idx"],
        q_num_blocks=t["q_num"], q_indices=t["q_idx"],
        full_q_num_blocks=t["full_q_num"], full_q_indices=t["full_q_idx"],
        row_order=row_order, col_order=col_order, kv_bits_off=kv_bits_off,
        q_bits_slot=q_bits_slot, tile_bits=tile_bits, _c=cs)
