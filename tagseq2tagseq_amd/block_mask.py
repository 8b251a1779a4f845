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
flex_attention, and ``from_torch_block_mask()`` goes the other way: a torch
``BlockMask`` (128 x 128 tiles, one mask for every head) becomes a
``T2TBlockMask`` over its own KV tables, with the partial tiles' bitmaps
evaluated from its ``mask_mod``.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Callable, Optional

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
    # mask_mod of the torch BlockMask this mask was converted from (its
    # per-token inputs are then unknown: doc_ids are zeros and words 0)
    source_mask_mod: Optional[Callable] = field(default=None, repr=False)

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
        (cross_doc_mask.py:348-357; doc_causal when there are no words), or
        the source BlockMask's own mask_mod for a converted mask."""
        if self.source_mask_mod is not None:
            return self.source_mask_mod
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


def _ordered(flags: torch.Tensor):
    """(count, order) of a [..., n] bool tensor: the number of set entries and
    their indices ascending followed by the unset ones ascending (torch's
    _dense_to_ordered convention, torch/nn/attention/flex_attention.py:429-436)."""
    n = flags.shape[-1]
    key = (~flags).to(torch.int64) * n + torch.arange(n, device=flags.device)
    return flags.sum(-1, dtype=torch.int32), key.argsort(-1).to(torch.int32)


ORDER_BUCKET = 2  # non-skip tiles per launch-order bucket (mask_meta.hip)


def _launch_order(count: torch.Tensor, index_desc: bool) -> torch.Tensor:
    """Indices by descending count // ORDER_BUCKET, within a bucket by
    descending (rows) or ascending (columns) index: the launch orders of the
    metadata pass."""
    n = count.shape[-1]
    idx = torch.arange(n, device=count.device)
    key = (count.to(torch.int64) // ORDER_BUCKET) * n + (idx if index_desc else n - 1 - idx)
    return key.argsort(-1, descending=True).to(torch.int32)


def _pack_bits(m: torch.Tensor) -> torch.Tensor:
    """[P, 128, 128] bool -> int32 [P, 128, 4]: bit j of word w of row r is
    m[r, 32 w + j]."""
    P = m.shape[0]
    w = m.reshape(P, TILE, 4, 32).to(torch.int64) << torch.arange(32, device=m.device)
    return w.sum(-1).to(torch.int32)


def from_torch_block_mask(bm, tile_chunk: int = 256) -> T2TBlockMask:
    """A T2TBlockMask over a torch BlockMask's own tables (kv_num_blocks,
    kv_indices, full_kv_num_blocks, full_kv_indices define the tile classes;
    torch/nn/attention/flex_attention.py:586-657), for the flex_attention seam
    when the caller brings a mask made by torch's create_block_mask.  The
    column tables, launch orders and bitmap slots are derived with torch ops
    on the mask's device, and the allowed-pair bitmap of every partial tile is
    evaluated from ``bm.mask_mod`` at head 0 over the tile's valid positions
    (positions past the sequence are masked, as create_block_mask pads).
    Masks with partial tiles above the diagonal (not causal) are accepted:
    their bitmaps take one slot per tile of the square.
    Requires 128 x 128 tiles, equal query and key lengths and one mask for
    every head (a head dimension of 1)."""
    if tuple(bm.BLOCK_SIZE) != (TILE, TILE):
        raise ValueError(f"BlockMask tiles {tuple(bm.BLOCK_SIZE)} are not {TILE} x {TILE}")
    Tq, Tk = bm.seq_lengths
    if Tq != Tk:
        raise ValueError(f"self-attention masks only (Q_LEN {Tq} != KV_LEN {Tk})")
    kvn = bm.kv_num_blocks
    if kvn.dim() != 3 or kvn.shape[1] != 1:
        raise ValueError("per-head block masks are not supported (the head dimension must be 1)")
    T, dev = int(Tq), kvn.device
    Bm, nt = int(kvn.shape[0]), int(kvn.shape[-1])
    if nt != (T + TILE - 1) // TILE:
        raise ValueError(f"BlockMask has {nt} tile columns for length {T}")
    i32 = dict(dtype=torch.int32, device=dev)
    ar = torch.arange(nt, device=dev)
    cls = torch.zeros((Bm, nt, nt), dtype=torch.int8, device=dev)

    def mark(num, idx, value):
        if num is None:
            return
        num, idx = num[:, 0].to(torch.int64), idx[:, 0, :, :nt].to(torch.int64)
        live = ar[None, None, :] < num[:, :, None]
        rows = ar[None, :, None].expand(Bm, nt, nt)
        bsel = torch.arange(Bm, device=dev)[:, None, None].expand(Bm, nt, nt)
        cls[bsel[live], rows[live], idx[live]] = value

    mark(bm.kv_num_blocks, bm.kv_indices, 1)
    mark(bm.full_kv_num_blocks, bm.full_kv_indices, 2)
    part, full = cls == 1, cls == 2
    kv_num, kv_idx = _ordered(part)
    fkv_num, fkv_idx = _ordered(full)
    q_num, q_idx = _ordered(part.transpose(1, 2))
    fq_num, fq_idx = _ordered(full.transpose(1, 2))
    row_order = _launch_order(kv_num + fkv_num, True)
    col_order = _launch_order(q_num + fq_num, False)
    # bitmap slot of partial tile (b, r, c): kv_bits_off[b, r] + c.  A causal
    # mask has partial tiles on or below the diagonal only (c <= r), and the
    # slots are the tile's position in the lower triangle, b nt (nt + 1) / 2 +
    # r (r + 1) / 2 + c (the metadata pass's layout).  Any other mask (a
    # bidirectional or sliding-window mask_mod, say) gets the square layout,
    # b nt^2 + r nt + c, so that no two partial tiles share a slot.
    upper = part & (ar[None, None, :] > ar[None, :, None])
    per_row = nt * nt if bool(upper.any()) else nt * (nt + 1) // 2
    row_start = ar * nt if per_row == nt * nt else ar * (ar + 1) // 2
    kv_bits_off = (torch.arange(Bm, device=dev)[:, None] * per_row
                   + row_start[None, :]).to(torch.int32)
    slot_grid = kv_bits_off[:, :, None].to(torch.int64) + ar[None, None, :]
    q_bits_slot = torch.gather(slot_grid.transpose(1, 2), 2, q_idx.to(torch.int64))
    q_bits_slot = torch.where(ar[None, None, :] < q_num[:, :, None], q_bits_slot,
                              torch.zeros_like(q_bits_slot)).to(torch.int32)
    # bitmaps of the partial tiles
    pb, pr, pc = part.nonzero(as_tuple=True)
    P = int(pb.numel())
    tile_bits = torch.zeros((max(1, Bm * per_row), 2, TILE, 4), **i32)
    t = torch.arange(TILE, device=dev)
    for s0 in range(0, P, tile_chunk):
        b_, r_, c_ = (x[s0:s0 + tile_chunk] for x in (pb, pr, pc))
        qpos = r_[:, None, None] * TILE + t[None, :, None]
        kpos = c_[:, None, None] * TILE + t[None, None, :]
        ok = (qpos < T) & (kpos < T)
        m = bm.mask_mod(b_[:, None, None], torch.zeros_like(b_)[:, None, None],
                        qpos.clamp(max=T - 1), kpos.clamp(max=T - 1))
        m = torch.as_tensor(m, device=dev).expand(ok.shape) & ok
        slots = slot_grid[b_, r_, c_]
        tile_bits[slots, 0] = _pack_bits(m)
        tile_bits[slots, 1] = _pack_bits(m.transpose(1, 2))
    out = T2TBlockMask(
        seq_len=T, doc_ids=torch.zeros((Bm, T), **i32),
        q_bits=torch.zeros((Bm, 0, T), dtype=torch.int64, device=dev),
        kv_bits=torch.zeros((Bm, 0, T), dtype=torch.int64, device=dev), tile_class=cls,
        kv_num_blocks=kv_num[:, None].contiguous(), kv_indices=kv_idx[:, None].contiguous(),
        full_kv_num_blocks=fkv_num[:, None].contiguous(),
        full_kv_indices=fkv_idx[:, None].contiguous(),
        q_num_blocks=q_num[:, None].contiguous(), q_indices=q_idx[:, None].contiguous(),
        full_q_num_blocks=fq_num[:, None].contiguous(),
        full_q_indices=fq_idx[:, None].contiguous(),
        row_order=row_order.contiguous(), col_order=col_order.contiguous(),
        kv_bits_off=kv_bits_off.contiguous(), q_bits_slot=q_bits_slot.contiguous(),
        tile_bits=tile_bits, source_mask_mod=bm.mask_mod)
    return out
