"""Density-aware batch ordering (CPU): the exact pair-count cost model
against the oracle's dense mask, the window ordering invariants, the
straggler measure, and a two-rank gloo run."""
import os
import random
import socket

import numpy as np
import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

from oracle import mask_oracle as mo
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.schedule import (DensityOrderedBatches, gather_costs, pack_pairs,
                                        straggler_fraction, tile_cost)


def _doc_link_bits(T, spans, links):
    """Per-token words of create_doc_link_block_mask (span index bits)."""
    idx = np.full(T, -1, dtype=np.int64)
    for i, s in enumerate(spans):
        a, b = max(0, s.start), min(T, s.end)
        if a < b:
            idx[a:b] = i
    W = links.shape[1]
    qb = np.zeros((W, T), dtype=np.uint64)
    kb = np.zeros((W, T), dtype=np.uint64)
    cov = idx >= 0
    qb[:, cov] = links[idx[cov]].T
    kb[idx[cov] // 64, np.nonzero(cov)[0]] = np.uint64(1) << (idx[cov] % 64).astype(np.uint64)
    return qb, kb


def _random_layout(rng, T, n, W):
    spans = []
    for i in range(n):
        a = rng.randint(-20, T)
        spans.append(synth.DocSpan(doc_id=rng.randint(0, n // 2), start=a, end=a + rng.randint(0, T // 3)))
    links = np.zeros((n, W), dtype=np.uint64)
    for i in range(n):
        for _ in range(rng.randint(0, 4)):
            j = rng.randint(0, n - 1)
            links[i, j // 64] |= np.uint64(1) << np.uint64(j % 64)
    return spans, links


@pytest.mark.parametrize("seed", range(10))
def test_pack_pairs_matches_dense_mask(seed):
    """Overlapping, unsorted, out-of-range spans; repeated doc ids; uncovered
    tokens; 2 words (more than 64 spans)."""
    rng = random.Random(seed)
    T = rng.choice([1, 97, 300, 777])
    n = rng.choice([3, 20, 70])
    spans, links = _random_layout(rng, T, n, 2)
    doc = mo.document_ids(T, spans)
    qb, kb = _doc_link_bits(T, spans, links)
    assert pack_pairs(T, spans, links) == int(mo.dense_mask(doc, qb, kb).sum())
    assert pack_pairs(T, spans) == int(mo.dense_mask(doc).sum())


def test_pack_pairs_config_rows():
    for seed in range(3):
        row = synth.config_rows(3, seed=seed, T=4096)[0]
        doc = mo.document_ids(4096, row.spans)
        qb, kb = mo.doc_link_token_bits(row.doc_index, row.link_rows)
        assert pack_pairs(4096, row.spans, row.link_rows) == int(mo.dense_mask(doc, qb, kb).sum())


def test_window_order_invariants():
    items = [{"id": i, "c": c} for i, c in enumerate([3, 9, 1, 9, 4, 7, 2, 8, 5, 6, 0])]
    sched = DensityOrderedBatches(items, lambda b: b["c"], window=4)
    out = list(sched)
    assert sorted(b["id"] for b in out) == list(range(11))  # a permutation
    windows = [out[0:4], out[4:8], out[8:11]]
    for w, src in zip(windows, [items[0:4], items[4:8], items[8:11]]):
        assert {b["id"] for b in w} == {b["id"] for b in src}
        cs = [b["c"] for b in w]
        assert cs == sorted(cs, reverse=True)
    assert [b["id"] for b in windows[0]] == [1, 3, 0, 2]  # ties keep arrival order
    with pytest.raises(ValueError):
        DensityOrderedBatches(items, lambda b: 0, window=0)


def test_straggler_fraction_closed_form():
    assert straggler_fraction(np.array([[1.0, 1.0], [1.0, 1.0]])) == 0.0
    # step 1: max 3 mean 2; step 2: max 1 mean 1 -> (1 + 0) / (3 + 1)
    assert straggler_fraction(np.array([[3.0, 1.0], [1.0, 1.0]])) == pytest.approx(0.25)


def _packs(seed, n, T=16384):
    """Pack costs of the configs[2] generator (lognormal docs, random links)."""
    rows = [synth.linked_lognormal_docs(T, 350.0, 1.0, 2048, 0.15, seed=seed * 1000 + k)
            for k in range(n)]
    return [{"seed": seed * 1000 + k, "cost": pack_pairs(T, r.spans, r.link_rows)}
            for k, r in enumerate(rows)]


def test_ordering_reduces_stragglers_8_ranks():
    ranks, steps = 8, 32
    packs = [_packs(r, steps, T=4096) for r in range(ranks)]
    raw = np.array([[p["cost"] for p in ps] for ps in packs], dtype=np.float64)
    ordered = np.array([[b["cost"] for b in DensityOrderedBatches(ps, lambda b: b["cost"], 8)]
                        for ps in packs], dtype=np.float64)
    f_raw, f_ord = straggler_fraction(raw), straggler_fraction(ordered)
    assert f_ord < 0.6 * f_raw, (f_raw, f_ord)


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _worker(rank, world, port, q):
    os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        packs = _packs(rank, 16, T=4096)
        sched = DensityOrderedBatches(packs, lambda b: b["cost"], window=8)
        got = list(sched)
        raw = gather_costs([p["cost"] for p in packs])
        ordered = gather_costs([b["cost"] for b in got])
        q.put((rank, sorted(b["seed"] for b in got), sorted(p["seed"] for p in packs),
               straggler_fraction(raw), straggler_fraction(ordered)))
    finally:
        dist.destroy_process_group()


def test_two_rank_gloo():
    ctx = mp.get_context("spawn")
    q = ctx.Queue()
    port = _free_port()
    procs = [ctx.Process(target=_worker, args=(r, 2, port, q)) for r in range(2)]
    for p in procs:
        p.start()
    res = [q.get(timeout=120) for _ in procs]
    for p in procs:
        p.join(60)
        assert p.exitcode == 0
    for rank, got, want, f_raw, f_ord in res:
        assert got == want  # each rank keeps exactly its own packs
        assert f_ord <= f_raw
    assert res[0][3] == res[1][3] and res[0][4] == res[1][4]  # same gathered view


def test_tile_cost_counts_full_and_weighted_partial_tiles():
    """tile_cost = full + w * partial over every mask row (skip tiles free)."""
    import types
    tc = torch.tensor([[[2, 1, 0], [1, 1, 2], [0, 0, 1]]], dtype=torch.int8)  # 2 full, 4 partial
    bm = types.SimpleNamespace(tile_class=tc)
    assert tile_cost(bm, partial_weight=1.0) == 6.0
    assert tile_cost(bm, partial_weight=0.5) == 4.0
    assert abs(tile_cost(bm) - (2 + 0.63 * 4)) < 1e-12
