"""Seeded synthetic packed sequences for the masked-attention workloads.

The reference trains on packed document sequences (data/collate.py:79-182): one
row of T tokens holds consecutive documents described by ``DocSpan`` records
(data/collate.py:16-33).  These generators produce the same structure without a
corpus: document lengths from a stated distribution, packed until the row is
full with the last document truncated, plus (for cross-document links) a
lower-triangular doc x doc link bitmask with the diagonal set.

``doc_id`` values are deliberately *not* 0..n-1 (the reference's doc ids are
global graph ids, data/collate.py:28), so consumers cannot confuse them with
the in-row document index.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np


@dataclass
class DocSpan:
    """Field-compatible with the reference's DocSpan (data/collate.py:16-33)."""
    doc_id: int
    start: int
    end: int
    normed_identifier: str = ""
    truncated: bool = False
    outgoing_identifiers: List[str] = field(default_factory=list)
    raw_identifier: str = ""


@dataclass
class SynthRow:
    """One packed row: spans, per-token document index, optional link rows."""
    seq_len: int
    spans: List[DocSpan]
    doc_index: np.ndarray            # int32[T], in-row document index (0..n-1)
    link_rows: Optional[np.ndarray]  # uint64[n_docs, W] or None (doc_causal)

    @property
    def n_docs(self) -> int:
        return len(self.spans)

    @property
    def words(self) -> int:
        return 0 if self.link_rows is None else int(self.link_rows.shape[1])


def _pack(lengths_fn, T: int, rng: np.random.Generator, id_base: int) -> List[DocSpan]:
    spans: List[DocSpan] = []
    pos = 0
    while pos < T:
        n = int(lengths_fn(rng))
        n = max(1, n)
        end = min(T, pos + n)
        i = len(spans)
        spans.append(DocSpan(doc_id=id_base + 7 * i + 3, start=pos, end=end,
                             truncated=end < pos + n, raw_identifier=f"doc{i}",
                             normed_identifier=f"doc{i}"))
        pos = end
    return spans


def _doc_index(spans: List[DocSpan], T: int) -> np.ndarray:
    idx = np.full(T, -1, dtype=np.int32)
    for i, s in enumerate(spans):
        idx[s.start:s.end] = i
    return idx


def _link_rows(n: int, prob: np.ndarray, rng: np.random.Generator) -> np.ndarray:
    """Lower-triangular bitmask rows: bit j of row i set with prob[i, j] (j < i),
    diagonal always set."""
    W = max(1, (n + 63) // 64)
    rows = np.zeros((n, W), dtype=np.uint64)
    u = rng.random((n, n))
    for i in range(n):
        for j in range(i + 1):
            if j == i or u[i, j] < prob[i, j]:
                rows[i, j // 64] |= np.uint64(1) << np.uint64(j % 64)
    return rows


def uniform_docs(T: int, lo: int, hi: int, seed: int, id_base: int = 1000) -> SynthRow:
    """Config 1: doc lengths ~ U[lo, hi], packed, last doc truncated."""
    rng = np.random.default_rng(seed)
    spans = _pack(lambda r: r.integers(lo, hi + 1), T, rng, id_base)
    return SynthRow(T, spans, _doc_index(spans, T), None)


def lognormal_docs(T: int, median: float, sigma: float, cap: int, seed: int,
                   id_base: int = 1000) -> SynthRow:
    """Config 2: doc lengths log-normal(median, sigma) capped at ``cap``."""
    rng = np.random.default_rng(seed)
    mu = np.log(median)
    spans = _pack(lambda r: min(cap, round(r.lognormal(mu, sigma))), T, rng, id_base)
    return SynthRow(T, spans, _doc_index(spans, T), None)


def linked_lognormal_docs(T: int, median: float, sigma: float, cap: int, p_link: float,
                          seed: int, id_base: int = 1000) -> SynthRow:
    """Config 3: log-normal docs in BFS (= index) order; doc i links each earlier
    doc j independently with probability ``p_link``; diagonal set."""
    row = lognormal_docs(T, median, sigma, cap, seed, id_base)
    rng = np.random.default_rng(seed + 7919)
    n = row.n_docs
    prob = np.full((n, n), p_link)
    row.link_rows = _link_rows(n, prob, rng)
    return row


def clustered_pareto_docs(T: int, alpha: float, min_len: int, cap: int,
                          clusters=(3, 8), p_intra: float = 0.4, p_inter: float = 0.02,
                          seed: int = 0, id_base: int = 1000) -> SynthRow:
    """Config 4: Pareto(alpha, min_len) doc lengths capped at ``cap``; docs split
    into 3-8 contiguous clusters; link prob p_intra within a cluster, p_inter across."""
    rng = np.random.default_rng(seed)
    spans = _pack(lambda r: min(cap, int(min_len * (1.0 + r.pareto(alpha)))), T, rng, id_base)
    n = len(spans)
    k = int(rng.integers(clusters[0], clusters[1] + 1))
    k = min(k, n)
    cuts = np.sort(rng.choice(np.arange(1, n), size=k - 1, replace=False)) if n > 1 and k > 1 else np.array([], int)
    cluster = np.zeros(n, dtype=np.int64)
    for c in cuts:
        cluster[c:] += 1
    prob = np.where(cluster[:, None] == cluster[None, :], p_intra, p_inter)
    row = SynthRow(T, spans, _doc_index(spans, T), None)
    row.link_rows = _link_rows(n, prob, rng)
    return row


# Parameters of BASELINE.json's configs (index 0..4 <-> configs[0..4]).
CONFIGS = {
    1: dict(kind="doc_causal", dtype="float32", B=1, Hq=4, Hkv=4, T=1024, D=64, fwd_only=True),
    2: dict(kind="doc_causal", dtype="bfloat16", B=2, Hq=12, Hkv=12, T=8192, D=64),
    3: dict(kind="cross_doc_link", dtype="bfloat16", B=1, Hq=16, Hkv=16, T=16384, D=128),
    4: dict(kind="cross_doc_link", dtype="bfloat16", B=1, Hq=16, Hkv=4, T=32768, D=128),
}


def config_rows(cfg: int, seed: int, T: Optional[int] = None) -> List[SynthRow]:
    """The per-row document structure of config ``cfg`` (optionally at a smaller T)."""
    c = CONFIGS[cfg]
    T = c["T"] if T is None else T
    if cfg == 1:
        return [uniform_docs(T, 32, 256, seed)]
    if cfg == 2:
        return [lognormal_docs(T, 300.0, 1.0, 2048, seed * 1000 + b, id_base=1000 + 100000 * b)
                for b in range(c["B"])]
    if cfg == 3:
        return [linked_lognormal_docs(T, 350.0, 1.0, 2048, 0.15, seed)]
    if cfg == 4:
        return [clustered_pareto_docs(T, 1.5, 64, 4096, seed=seed)]
    raise ValueError(f"unknown config {cfg}")
