"""Shared test helpers: synthetic rows -> per-token mask arrays, torch fp32
reference attention (chunked, for full-size GPU checks)."""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import mask_oracle as mo
from oracle import tile_oracle
from tagseq2tagseq_amd import synth


def row_arrays(row: synth.SynthRow):
    """(doc_ids int32[T], q_bits uint64[W,T] | None, kv_bits | None) of a row,
    doc ids taken from the spans (global ids) like the reference."""
    doc = mo.document_ids(row.seq_len, row.spans)
    if row.link_rows is None:
        return doc, None, None
    qb, kb = mo.doc_link_token_bits(row.doc_index, row.link_rows)
    return doc, qb, kb


def random_row(T: int, rng: np.random.Generator, words: int = 0, uncovered: bool = False,
               max_doc: int = 200):
    """Random doc runs plus random grant words (exercises bit 63 and gaps)."""
    doc = np.empty(T, dtype=np.int32)
    pos = 0
    d = 0
    while pos < T:
        n = int(rng.integers(1, max_doc))
        doc[pos:pos + n] = (d * 13 + 5) if not (uncovered and rng.random() < 0.2) else -1
        pos += n
        d += 1
    if words == 0:
        return doc, None, None
    qb = np.zeros((words, T), dtype=np.uint64)
    kb = np.zeros((words, T), dtype=np.uint64)
    for _ in range(int(rng.integers(1, 12))):
        w = int(rng.integers(0, words))
        bit = np.uint64(63 if rng.random() < 0.3 else int(rng.integers(0, 64)))
        a = int(rng.integers(0, T))
        bq = int(rng.integers(a, T + 1))
        c = int(rng.integers(0, T))
        ck = int(rng.integers(c, min(T, c + 300) + 1))
        qb[w, a:bq] |= np.uint64(1) << bit
        kb[w, c:ck] |= np.uint64(1) << bit
    return doc, qb, kb


def to_dev_words(bits, device):
    if bits is None:
        return None
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int64)).to(device)


def dense_mask_torch(doc: torch.Tensor, qb, kb, r0: int, r1: int) -> torch.Tensor:
    """Rows [r0, r1) of the reference mask_mod as a bool tensor on doc's device."""
    T = doc.shape[0]
    q = torch.arange(r0, r1, device=doc.device)[:, None]
    kv = torch.arange(T, device=doc.device)[None, :]
    m = doc[r0:r1, None] == doc[None, :]
    if qb is not None:
        for w in range(qb.shape[0]):
            m |= (qb[w, r0:r1, None] & kb[w][None, :]) != 0
    return m & (q >= kv)


def torch_ref_attention(q, k, v, do, masks, scale=None, heads=None, chunk=2048):
    """fp32 masked attention fwd + bwd on the GPU, chunked over query rows.

    masks: list (len Bm) of (doc int32[T], qb int64[W,T] | None, kb) device tensors.
    heads: iterable of query heads to evaluate (default all).  Returns dicts
    keyed by (b, h) for o / lse(natural) / dq and by (b, hk) partial dk / dv
    accumulated over the evaluated heads only.
    """
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    heads = range(Hq) if heads is None else heads
    out = {"o": {}, "lse": {}, "dq": {}, "dk": {}, "dv": {}}
    for b in range(B):
        doc, qb, kb = masks[b if len(masks) > 1 else 0]
        for h in heads:
            hk = h // G
            qh, kh, vh = q[b, h].float(), k[b, hk].float(), v[b, hk].float()
            doh = do[b, h].float() if do is not None else None
            o = torch.empty_like(qh)
            lse = torch.empty(T, device=q.device)
            dq = torch.zeros_like(qh)
            dk = out["dk"].setdefault((b, hk), torch.zeros_like(kh))
            dv = out["dv"].setdefault((b, hk), torch.zeros_like(vh))
            for r0 in range(0, T, chunk):
                r1 = min(T, r0 + chunk)
                m = dense_mask_torch(doc, qb, kb, r0, r1)
                s = (qh[r0:r1] @ kh.T) * scale
                s = s.masked_fill(~m, float("-inf"))
                lse_c = torch.logsumexp(s, dim=1)
                p = torch.exp(s - lse_c[:, None])
                p = torch.nan_to_num(p, nan=0.0)
                o[r0:r1] = p @ vh
                lse[r0:r1] = lse_c
                if doh is not None:
                    dp = doh[r0:r1] @ vh.T
                    delta = (o[r0:r1] * doh[r0:r1]).sum(1, keepdim=True)
                    ds = p * (dp - delta)
                    dq[r0:r1] = ds @ kh * scale
                    dk += ds.T @ qh[r0:r1] * scale
                    dv += p.T @ doh[r0:r1]
            out["o"][(b, h)] = o
            out["lse"][(b, h)] = lse
            out["dq"][(b, h)] = dq
    return out


def assert_close(actual, expected, atol, rtol, what=""):
    a = actual.float() if isinstance(actual, torch.Tensor) else torch.as_tensor(actual).float()
    e = expected.float() if isinstance(expected, torch.Tensor) else torch.as_tensor(expected).float()
    e = e.to(a.device)
    both_inf = torch.isinf(a) & torch.isinf(e) & (torch.sign(a) == torch.sign(e))
    err = (a - e).abs()
    tol = atol + rtol * e.abs()
    bad = ~(both_inf | (err <= tol))
    if bad.any():
        idx = bad.nonzero()[:5].tolist()
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.numel()} elements out of tolerance "
                             f"(atol={atol}, rtol={rtol}); max err {float(err[~both_inf].max()):.4g}; "
                             f"first at {idx}")


# -- block-mask tables against the oracle ------------------------------------

TABLES = ["kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
          "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices"]


def _pack_bits(tile: np.ndarray) -> np.ndarray:
    """bool [128, 128] -> uint32 [128, 4], bit j of word w = tile[r, 32 w + j]."""
    return np.packbits(tile, axis=1, bitorder="little").view("<u4").reshape(128, 4)


def _check_extras(bm, b, doc, qb, kb, label):
    """Launch orders, bitmap slots and partial-tile bitmaps against the oracle."""
    T = doc.shape[0]
    nt = (T + 127) // 128
    kv_num = bm.kv_num_blocks[b, 0].cpu().numpy()
    full_num = bm.full_kv_num_blocks[b, 0].cpu().numpy()
    kv_idx = bm.kv_indices[b, 0].cpu().numpy()
    q_num = bm.q_num_blocks[b, 0].cpu().numpy()
    q_full = bm.full_q_num_blocks[b, 0].cpu().numpy()
    q_idx = bm.q_indices[b, 0].cpu().numpy()
    row_order = bm.row_order[b].cpu().numpy()
    col_order = bm.col_order[b].cpu().numpy()
    off = bm.kv_bits_off[b].cpu().numpy()
    slot_col = bm.q_bits_slot[b].cpu().numpy()
    bits = bm.tile_bits.cpu().numpy()
    assert sorted(row_order.tolist()) == list(range(nt)), f"{label}: row_order not a permutation"
    assert sorted(col_order.tolist()) == list(range(nt)), f"{label}: col_order not a permutation"
    # launch orders: non-skip counts in buckets of two, longest first; within a
    # bucket rows by descending index, columns by ascending index
    idx = np.arange(nt)
    exp_rows = np.lexsort((-idx, -((kv_num + full_num) // 2)))
    exp_cols = np.lexsort((idx, -((q_num + q_full) // 2)))
    np.testing.assert_array_equal(row_order, exp_rows, err_msg=f"{label}: row_order")
    np.testing.assert_array_equal(col_order, exp_cols, err_msg=f"{label}: col_order")
    # bitmap slot of tile (b, r, c): its position in the lower triangle
    exp_off = b * (nt * (nt + 1) // 2) + np.arange(nt) * (np.arange(nt) + 1) // 2
    np.testing.assert_array_equal(off, exp_off, err_msg=f"{label}: kv_bits_off")
    row_slot = {}
    pad = nt * 128 - T
    for qt in range(nt):
        if kv_num[qt] == 0:
            continue
        rows = mo.dense_mask(doc, qb, kb, (qt * 128, min(T, qt * 128 + 128)))
        rows = np.pad(rows, ((0, 128 - rows.shape[0]), (0, pad)))
        for i in range(kv_num[qt]):
            kt = kv_idx[qt, i]
            slot = off[qt] + kt
            row_slot[(qt, kt)] = slot
            tile = rows[:, kt * 128:(kt + 1) * 128]
            np.testing.assert_array_equal(bits[slot, 0].view("<u4"), _pack_bits(tile),
                                          err_msg=f"{label}: row bits tile ({qt},{kt})")
            np.testing.assert_array_equal(bits[slot, 1].view("<u4"), _pack_bits(tile.T.copy()),
                                          err_msg=f"{label}: column bits tile ({qt},{kt})")
    for kt in range(nt):
        for i in range(q_num[kt]):
            assert slot_col[kt, i] == row_slot[(q_idx[kt, i], kt)], f"{label}: q_bits_slot ({kt},{i})"


def check_block_mask(bm, rows_np, label):
    """Tile classes, the eight BlockMask tables, launch orders, bitmap slots
    and partial-tile bitmaps of ``bm`` against the oracle."""
    tc = bm.tile_class.cpu().numpy()
    got = {name: getattr(bm, name).cpu().numpy() for name in TABLES}
    for b, (doc, qb, kb) in enumerate(rows_np):
        counts = tile_oracle.tile_counts(doc, qb, kb)
        ref = mo.block_mask_tables(doc, qb, kb, counts=counts)
        exp_cls = ref["partial"] + 2 * ref["full"]
        np.testing.assert_array_equal(tc[b], exp_cls, err_msg=f"{label} b={b}: tile classes")
        for name in TABLES:
            np.testing.assert_array_equal(got[name][b, 0], ref[name], err_msg=f"{label} b={b}: {name}")
        _check_extras(bm, b, doc, qb, kb, f"{label} b={b}")
