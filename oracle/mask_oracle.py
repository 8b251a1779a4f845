"""Mask-semantics oracle (numpy).  TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

Restates, for CPU checking:

* ``document_ids``          -- model/graph_traversal/block_mask_creator.py:107-117
* ``find_link_span`` / ``find_target_span``
                            -- cross_doc_mask.py:170-188 and :258-272 (first match wins)
* ``build_cross_doc_dense`` -- cross_doc_mask.py:151-208 (dense O(T^2) grant mask)
* ``build_grant_bitmasks``  -- cross_doc_mask.py:210-300 (chunk k//64, bit k%64,
                               bit 63 stored as INT64_MIN, truncation at ``cap``)
* ``dense_mask``            -- the ``mask_mod`` of cross_doc_mask.py:348-357, which
                               reduces to ``doc_causal_mod`` (block_mask_creator.py:121-129)
                               when there are no grant words
* ``doc_link_token_bits``   -- the per-sequence doc x doc link bitmask form, expressed in
                               the reference's (q_bitmask, kv_bitmask) encoding
* ``classify_tiles``        -- torch/nn/attention/flex_attention.py:979-1022
                               (pad with False to a multiple of 128; full iff the tile sum
                               is 128*128, partial iff 0 < sum < 128*128)
* ``dense_to_ordered`` / ``transpose_ordered``
                            -- torch/nn/attention/flex_attention.py:429-441
                               (stable descending argsort of the 0/1 tile rows)

Bitmasks are carried as ``uint64`` arrays; the bit patterns equal the reference's
signed ``int64`` tensors (INT64_MIN == 1 << 63).
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

BLOCK = 128  # torch/nn/attention/flex_attention.py:395 (_DEFAULT_SPARSE_BLOCK_SIZE)


def document_ids(seq_len: int, doc_spans: Sequence) -> np.ndarray:
    """block_mask_creator.py:107-117: -1 everywhere, then span.doc_id on
    [max(0,start), min(T,end)) for each span in order (later spans overwrite)."""
    ids = np.full(seq_len, -1, dtype=np.int32)
    for span in doc_spans:
        start = max(0, span.start)
        end = min(seq_len, span.end)
        if start < end:
            ids[start:end] = span.doc_id
    return ids


def find_link_span(doc_spans: Sequence, link_pos: int):
    """cross_doc_mask.py:171-175 / :259-263: first span with start < link_pos <= end."""
    for span in doc_spans:
        if span.start < link_pos <= span.end:
            return span
    return None


def find_target_span(doc_spans: Sequence, doc_id: int):
    """cross_doc_mask.py:184-188 / :268-272: first span whose doc_id matches."""
    for span in doc_spans:
        if span.doc_id == doc_id:
            return span
    return None


def build_cross_doc_dense(seq_len: int, doc_spans: Sequence,
                          link_to_target: Dict[int, List[int]]) -> np.ndarray:
    """cross_doc_mask.py:151-208: dense [T,T] grant mask (no same-doc, no causal)."""
    m = np.zeros((seq_len, seq_len), dtype=bool)
    for link_pos, targets in sorted(link_to_target.items()):
        for tgt in targets:
            src = find_link_span(doc_spans, link_pos)
            if src is None:
                continue
            tspan = find_target_span(doc_spans, tgt)
            if tspan is None:
                continue
            gs, ge = link_pos, min(seq_len, src.end)
            ts, te = max(0, tspan.start), min(seq_len, tspan.end)
            if gs < ge and ts < te:
                m[gs:ge, ts:te] = True
    return m


def build_grant_bitmasks(seq_len: int, doc_spans: Sequence,
                         link_to_target: Dict[int, List[int]], n_chunks: int,
                         cap: int) -> Tuple[np.ndarray, np.ndarray, int]:
    """cross_doc_mask.py:210-300.

    Returns (q_bits uint64[n_chunks, T], kv_bits uint64[n_chunks, T], n_grants).
    Grant k -> chunk k // 64, bit k % 64 (:282-287).  Once ``grant_idx >= cap`` the
    remaining grants are dropped (:251-257).  Unresolvable links and empty ranges
    do not consume a grant index (:258-277, :283-294).
    """
    qb = np.zeros((n_chunks, seq_len), dtype=np.uint64)
    kb = np.zeros((n_chunks, seq_len), dtype=np.uint64)
    grant_idx = 0
    truncated = False
    for link_pos, targets in sorted(link_to_target.items()):
        if truncated:
            break
        for tgt in targets:
            if grant_idx >= cap:
                truncated = True
                break
            src = find_link_span(doc_spans, link_pos)
            if src is None:
                continue
            tspan = find_target_span(doc_spans, tgt)
            if tspan is None:
                continue
            gs, ge = link_pos, min(seq_len, src.end)
            ts, te = max(0, tspan.start), min(seq_len, tspan.end)
            if gs < ge and ts < te:
                chunk, bit = grant_idx // 64, grant_idx % 64
                b = np.uint64(1) << np.uint64(bit)
                qb[chunk, gs:ge] |= b
                kb[chunk, ts:te] |= b
                grant_idx += 1
    return qb, kb, grant_idx


def bitmask_to_dense(q_bits: np.ndarray, kv_bits: np.ndarray) -> np.ndarray:
    """tests/model/graph_traversal/test_grant_bitmask_equivalence.py:50-63:
    OR over chunks of (q_bm[:,None] & kv_bm[None,:]) != 0."""
    T = q_bits.shape[-1]
    out = np.zeros((T, T), dtype=bool)
    for c in range(q_bits.shape[0]):
        out |= (q_bits[c][:, None] & kv_bits[c][None, :]) != 0
    return out


def dense_mask(doc_ids: np.ndarray, q_bits: Optional[np.ndarray] = None,
               kv_bits: Optional[np.ndarray] = None, q_range=None) -> np.ndarray:
    """mask_mod of cross_doc_mask.py:348-357 evaluated densely (rows ``q_range``):

        causal & (doc[q] == doc[kv] | OR_c (q_bm[c][q] & kv_bm[c][kv]) != 0)

    With no bit words this is doc_causal_mod (block_mask_creator.py:121-129).
    """
    T = doc_ids.shape[0]
    q0, q1 = (0, T) if q_range is None else q_range
    q = np.arange(q0, q1)[:, None]
    kv = np.arange(T)[None, :]
    m = doc_ids[q0:q1, None] == doc_ids[None, :]
    if q_bits is not None:
        for c in range(q_bits.shape[0]):
            m |= (q_bits[c, q0:q1, None] & kv_bits[c][None, :]) != 0
    return m & (q >= kv)


def doc_link_token_bits(doc_index: np.ndarray, link_rows: np.ndarray
                        ) -> Tuple[np.ndarray, np.ndarray]:
    """Per-sequence doc-link bitmask -> reference (q_bitmask, kv_bitmask) words.

    ``doc_index[t]`` in [0, n_docs) (or -1 for an uncovered token) and
    ``link_rows[d]`` = uint64[W] row d of the lower-triangular doc x doc bitmask
    (bit j set: doc d may read doc j; diagonal set).  Grant "bit j" is "target doc
    j", so kv_bits[t] = 1 << doc(t) and q_bits[t] = link_rows[doc(t)]; then
    (q_bits[q] & kv_bits[kv]) != 0 iff doc(q) links doc(kv) -- the same mask_mod
    formula as cross_doc_mask.py:348-357.
    """
    T = doc_index.shape[0]
    W = link_rows.shape[1]
    qb = np.zeros((W, T), dtype=np.uint64)
    kb = np.zeros((W, T), dtype=np.uint64)
    cov = doc_index >= 0
    d = doc_index[cov]
    qb[:, cov] = link_rows[d].T
    kb[d // 64, np.nonzero(cov)[0]] = np.uint64(1) << (d % 64).astype(np.uint64)
    return qb, kb


def tile_counts(doc_ids: np.ndarray, q_bits=None, kv_bits=None,
                block: int = BLOCK) -> np.ndarray:
    """Per-tile allowed-pair counts over the False-padded mask
    (torch/nn/attention/flex_attention.py:990-1013).  int64[nQ, nK]."""
    T = doc_ids.shape[0]
    n = (T + block - 1) // block
    counts = np.zeros((n, n), dtype=np.int64)
    for qt in range(n):
        q0, q1 = qt * block, min(T, (qt + 1) * block)
        rows = dense_mask(doc_ids, q_bits, kv_bits, (q0, q1))
        pad = n * block - T
        if pad:
            rows = np.pad(rows, ((0, 0), (0, pad)))
        counts[qt] = rows.reshape(q1 - q0, n, block).sum(axis=(0, 2))
    return counts


def classify_tiles(counts: np.ndarray, block: int = BLOCK) -> Tuple[np.ndarray, np.ndarray]:
    """torch/nn/attention/flex_attention.py:1014-1018: (partial, full) int8."""
    full_sum = block * block
    full = (counts == full_sum).astype(np.int8)
    partial = ((counts > 0) & (counts < full_sum)).astype(np.int8)
    return partial, full


def dense_to_ordered(blocks: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """torch/nn/attention/flex_attention.py:429-436: row sums and the stable
    descending argsort of each 0/1 row (set columns ascending, then unset ones)."""
    b = blocks.astype(np.int32)
    num = b.sum(axis=-1).astype(np.int32)
    idx = np.argsort(-b, axis=-1, kind="stable").astype(np.int32)
    return num, idx


def transpose_ordered(blocks: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """torch/nn/attention/flex_attention.py:439-441 applied to the dense 0/1 grid."""
    return dense_to_ordered(np.swapaxes(blocks, -1, -2))


def block_mask_tables(doc_ids: np.ndarray, q_bits=None, kv_bits=None,
                      counts: Optional[np.ndarray] = None) -> Dict[str, np.ndarray]:
    """Everything ``create_block_mask`` derives for one mask row (B = H = 1)."""
    if counts is None:
        counts = tile_counts(doc_ids, q_bits, kv_bits)
    partial, full = classify_tiles(counts)
    out = {"partial": partial, "full": full, "counts": counts}
    out["kv_num_blocks"], out["kv_indices"] = dense_to_ordered(partial)
    out["full_kv_num_blocks"], out["full_kv_indices"] = dense_to_ordered(full)
    out["q_num_blocks"], out["q_indices"] = transpose_ordered(partial)
    out["full_q_num_blocks"], out["full_q_indices"] = transpose_ordered(full)
    return out


def torch_mask_mod(doc_ids, q_bits=None, kv_bits=None):
    """The reference's mask_mod (cross_doc_mask.py:348-357; doc_causal_mod of
    block_mask_creator.py:121-129 when there are no grant words) as a closure
    over torch tensors, for torch's create_block_mask / flex_attention.

    doc_ids int32 [T]; q_bits / kv_bits int64 [W, T] (uint64 bit patterns) or None.
    """
    W = 0 if q_bits is None else int(q_bits.shape[0])
    q_list = [q_bits[w] for w in range(W)]
    kv_list = [kv_bits[w] for w in range(W)]

    def reference_mask_mod(b, h, q_idx, kv_idx):
        causal = q_idx >= kv_idx
        same_doc = doc_ids[q_idx] == doc_ids[kv_idx]
        if W:
            in_grant = (q_list[0][q_idx] & kv_list[0][kv_idx]) != 0
            for i in range(1, W):
                in_grant = in_grant | ((q_list[i][q_idx] & kv_list[i][kv_idx]) != 0)
            return causal & (same_doc | in_grant)
        return causal & same_doc

    return reference_mask_mod
