"""Density-aware ordering of packed batches across data-parallel ranks.

The reference trains with one pack sampler per rank, seeded base_seed + rank
(main.py:164-179), so at every step each rank runs a different mask, and the
backward of the densest one sets the pace of the gradient all-reduce
(configs/baseline.yaml:37-46: "some ranks get dense masks -> slow FlexAttention
backward ... fast ranks stall at the NCCL barrier").  Its README lists the fix
as a TODO (README.md:151: "batch mask density pre-computation system to ensure
ranks spend less time waiting for whichever rank has the densest mask").

Here every rank draws a window of packs from its own sampler, predicts each
pack's attention cost from its mask inputs, and yields the window in
descending cost order.  All ranks apply the same rule to windows of the same
length, so at each step the ranks run packs of the same cost rank within
their windows: the per-step maximum over ranks moves towards the mean without
moving any data between ranks (for two ranks, pairing both windows in the
same order minimises the summed per-step maximum: sum max(a, b) =
sum (a + b) / 2 + sum |a - b| / 2, and equal ordering minimises the second sum).
With gradient accumulation the all-reduce waits on sums of accum_steps
consecutive micro-batches, which the same ordering balances.

Cost models:
  * ``pack_pairs``: exact number of allowed (q, kv) pairs of a pack from its
    spans and doc-link rows (host, O(T + links)) -- the work of every
    attention kernel that skips masked blocks;
  * ``tile_cost``: full + partial 128 x 128 tiles of a T2TBlockMask (the
    metadata pass on the device), for masks given as per-token words.
"""
from __future__ import annotations

from typing import Any, Callable, Dict, Iterable, Iterator, List, Optional, Sequence

import numpy as np
import torch

from .mask_creators import document_ids_host


def _span_index(T: int, doc_spans: Sequence) -> np.ndarray:
    """Index of the span covering each token (later spans overwrite, -1 none)."""
    idx = np.full(T, -1, dtype=np.int64)
    for i, s in enumerate(doc_spans):
        a, b = max(0, int(s.start)), min(T, int(s.end))
        if a < b:
            idx[a:b] = i
    return idx


def pack_pairs(seq_len: int, doc_spans: Sequence, doc_links: Optional[np.ndarray] = None) -> int:
    """Allowed (q, kv) pairs, q >= kv, of the doc_causal mask (doc_links None) or
    of the doc-link cross_doc_link mask (create_doc_link_block_mask's form: bit j
    of doc_links[i] lets span i read span j).

    Same-document pairs: for every doc id (uncovered tokens share id -1, as in
    block_mask_creator.py:121-129) m (m + 1) / 2 for its m tokens.  Link pairs:
    for every set bit j of span i whose tokens carry a different doc id, the
    (q in span i, kv in span j, kv < q) pairs, counted with a sorted search."""
    T = int(seq_len)
    doc = document_ids_host(T, doc_spans).astype(np.int64)
    _, counts = np.unique(doc, return_counts=True)
    total = int(np.sum(counts * (counts + 1) // 2))
    if doc_links is None:
        return total
    links = np.asarray(doc_links, dtype=np.uint64)
    span = _span_index(T, doc_spans)
    n = len(doc_spans)
    # Every token of span i carries span i's doc id (the last covering span sets
    # both), so a linked pair of spans with equal doc ids adds nothing new.
    members = [np.nonzero(span == i)[0] for i in range(n)]
    for i in range(min(n, links.shape[0])):
        qi = members[i]
        if qi.size == 0:
            continue
        for w in range(links.shape[1]):
            word = int(links[i, w])
            while word:
                low = word & -word
                j = 64 * w + low.bit_length() - 1
                word ^= low
                if j >= n or members[j].size == 0 or \
                        int(doc_spans[j].doc_id) == int(doc_spans[i].doc_id):
                    continue
                total += int(np.searchsorted(members[j], qi, side="right").sum())
    return total


def tile_cost(block_mask, partial_weight: float = 0.63) -> float:
    """full + partial_weight * partial non-skip 128 x 128 tiles (all mask rows).
    The default weight is the ratio fitted on measured attention fwd+bwd times
    of config-3 packs on MI355X (a partial tile's fully masked 32 x 32 blocks
    are skipped, so it costs about 0.63 of a full one)."""
    tc = block_mask.tile_class
    full = int((tc == 2).sum().item())
    partial = int((tc == 1).sum().item())
    return full + partial_weight * partial


def straggler_fraction(costs: np.ndarray) -> float:
    """Idle share of a lockstep run: costs [ranks, steps]; per step every rank
    waits for the slowest.  sum_k (max_r - mean_r) / sum_k max_r."""
    c = np.asarray(costs, dtype=np.float64)
    mx = c.max(axis=0)
    return float((mx - c.mean(axis=0)).sum() / max(mx.sum(), 1e-30))


class DensityOrderedBatches:
    """Iterable over ``batches`` that yields each window of ``window`` batches
    in descending predicted cost (stable for ties).  ``cost_fn(batch)`` -> float;
    every rank must use the same window length (and accumulation grouping) so
    that step k pairs the k-th costliest packs of all ranks.  The last, partial
    window is yielded in the same order.  ``last_costs`` holds the yielded
    window's costs, in yield order."""

    def __init__(self, batches: Iterable[Dict[str, Any]], cost_fn: Callable[[Dict[str, Any]], float],
                 window: int = 16):
        if window <= 0:
            raise ValueError(f"window must be positive, got {window}")
        self.batches = batches
        self.cost_fn = cost_fn
        self.window = window
        self.last_costs: List[float] = []

    def __iter__(self) -> Iterator[Dict[str, Any]]:
        it = iter(self.batches)
        while True:
            buf = []
            for _ in range(self.window):
                try:
                    buf.append(next(it))
                except StopIteration:
                    break
            if not buf:
                return
            costs = [float(self.cost_fn(b)) for b in buf]
            order = sorted(range(len(buf)), key=lambda k: (-costs[k], k))
            self.last_costs = [costs[k] for k in order]
            for k in order:
                yield buf[k]


def gather_costs(costs: Sequence[float], group=None) -> np.ndarray:
    """All ranks' per-step costs [world, steps] (a CPU all_gather; with the
    gloo backend the tensors stay in host memory)."""
    import torch.distributed as dist
    t = torch.tensor(list(costs), dtype=torch.float64)
    world = dist.get_world_size(group)
    out = [torch.empty_like(t) for _ in range(world)]
    dist.all_gather(out, t, group=group)
    return torch.stack(out).numpy()
