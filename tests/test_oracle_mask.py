"""CPU tests of the mask oracle and of the host-side mask logic.

Pins (no reference import is possible here: model.* needs the absent tunalab
package and tiktoken's network download):
  * the known-answer scenarios, fuzz and grant-capacity matrix of
    tests/model/graph_traversal/test_grant_bitmask_equivalence.py:109-408
    (restated: dense grant mask == bitmask form, spot values, truncation);
  * the dense-mask invariants of tests/model/graph_traversal/test_cross_doc_mask.py:103-125;
  * tile classification and ordered index lists against torch's own
    create_block_mask run on the restated mask_mod (torch is the library the
    reference calls, torch/nn/attention/flex_attention.py:1144-1225);
  * closed forms (single document = plain causal grid) and brute force (C oracle).
"""
import random
from dataclasses import dataclass, field
from typing import Dict, List

import numpy as np
import pytest
import torch

from oracle import mask_oracle as mo
from oracle import tile_oracle
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.mask_creators import CrossDocLinkMaskCreator, document_ids_host
from tests.helpers import random_row, row_arrays


@dataclass
class MockDocSpan:
    doc_id: int
    raw_identifier: str
    start: int
    end: int
    truncated: bool = False
    outgoing_identifiers: List[str] = field(default_factory=list)


def _both(seq_len, spans, link_to_target, n_chunks=1, cap=64):
    dense = mo.build_cross_doc_dense(seq_len, spans, link_to_target)
    qb, kb, _ = mo.build_grant_bitmasks(seq_len, spans, link_to_target, n_chunks, cap)
    return dense, mo.bitmask_to_dense(qb, kb)


def _spans(*triples):
    return [MockDocSpan(d, chr(65 + i), s, e) for i, (d, s, e) in enumerate(triples)]


# --- known-answer scenarios (test_grant_bitmask_equivalence.py:109-240) ---------

def test_empty_no_links():
    dense, bm = _both(20, _spans((0, 0, 10), (1, 10, 20)), {})
    assert not dense.any() and np.array_equal(dense, bm)


def test_single_grant_spot_values():
    dense, bm = _both(16, _spans((0, 0, 5), (1, 5, 16)), {8: [0]})
    assert np.array_equal(dense, bm)
    assert dense[8, 2] and bm[8, 2]
    assert not dense[5, 2] and not bm[5, 2]


def test_two_nonoverlapping_grants():
    dense, bm = _both(30, _spans((0, 0, 5), (1, 5, 15), (2, 15, 30)), {10: [0], 20: [1]})
    assert np.array_equal(dense, bm)


def test_overlapping_q_ranges():
    dense, bm = _both(30, _spans((0, 0, 5), (1, 5, 10), (2, 10, 30)), {15: [0], 18: [1]})
    assert np.array_equal(dense, bm)
    assert dense[20, 3] and dense[20, 7]


def test_overlapping_kv_ranges():
    dense, bm = _both(30, _spans((0, 0, 5), (1, 5, 15), (2, 15, 30)), {10: [0], 20: [0]})
    assert np.array_equal(dense, bm)


def test_link_at_span_end_is_empty():
    dense, bm = _both(20, _spans((0, 0, 5), (1, 5, 12)), {12: [0]})
    assert np.array_equal(dense, bm) and not dense.any()


def test_link_just_before_span_end():
    dense, bm = _both(20, _spans((0, 0, 5), (1, 5, 12)), {11: [0]})
    assert np.array_equal(dense, bm)
    assert dense[11, 2] and not dense[10, 2]


def test_three_doc_chain():
    dense, bm = _both(30, _spans((0, 0, 8), (1, 8, 18), (2, 18, 30)), {12: [0], 22: [0], 25: [1]})
    assert np.array_equal(dense, bm)


def test_link_outside_every_span_is_dropped():
    dense, bm = _both(20, _spans((0, 0, 5), (1, 5, 10)), {15: [0]})
    assert np.array_equal(dense, bm) and not dense.any()


# --- fuzz (test_grant_bitmask_equivalence.py:247-291) ---------------------------

def _random_scenario(rng: random.Random):
    n_docs = rng.randint(2, 8)
    widths = [rng.randint(2, 20) for _ in range(n_docs)]
    seq_len = sum(widths)
    spans, pos = [], 0
    for doc_id, w in enumerate(widths):
        spans.append(MockDocSpan(doc_id, f"doc_{doc_id}", pos, pos + w))
        pos += w
    link_to_target: Dict[int, List[int]] = {}
    for _ in range(rng.randint(1, 10)):
        src = rng.randint(1, n_docs - 1)
        link_pos = rng.randint(spans[src].start + 1, spans[src].end)
        link_to_target.setdefault(link_pos, []).append(rng.randint(0, src - 1))
    return seq_len, spans, link_to_target


@pytest.mark.parametrize("seed", range(20))
def test_fuzz_equivalence(seed):
    seq_len, spans, l2t = _random_scenario(random.Random(seed))
    dense, bm = _both(seq_len, spans, l2t)
    assert np.array_equal(dense, bm)


# --- capacity and truncation (test_grant_bitmask_equivalence.py:360-408) --------

def _n_grant_scenario(n):
    spans = [MockDocSpan(0, "target", 0, 4)]
    pos = 4
    for i in range(1, n + 1):
        spans.append(MockDocSpan(i, f"src_{i}", pos, pos + 4))
        pos += 4
    return pos, spans, {s.start + 1: [0] for s in spans[1:]}


@pytest.mark.parametrize("n_grants,max_grants,expect_equal", [
    (64, 64, True), (128, 128, True), (256, 256, True),
    (65, 64, False), (129, 128, False), (257, 256, False),
    (65, 128, True), (129, 256, True)])
def test_truncation_boundary(n_grants, max_grants, expect_equal):
    seq_len, spans, l2t = _n_grant_scenario(n_grants)
    n_chunks = max(1, (max_grants + 63) // 64)
    dense, bm = _both(seq_len, spans, l2t, n_chunks=n_chunks, cap=max_grants)
    assert np.array_equal(dense, bm) == expect_equal


def test_bit63_is_int64_min_pattern():
    """Grant 63 sets bit 63 (the reference stores it as INT64_MIN)."""
    seq_len, spans, l2t = _n_grant_scenario(64)
    qb, kb, n = mo.build_grant_bitmasks(seq_len, spans, l2t, 1, 64)
    assert n == 64
    assert (qb[0].view(np.int64) == np.iinfo(np.int64).min).any()


# --- product host logic against the oracle --------------------------------------

class _NoDetector:
    def detect_links(self, ids):
        return []

    def index_doc_span(self, span):
        return span.raw_identifier


def _paint(seq_len, ranges, words):
    """Grant ranges -> uint64 [words, T] words (bit k of word k // 64)."""
    qb = np.zeros((words, seq_len), dtype=np.uint64)
    kb = np.zeros((words, seq_len), dtype=np.uint64)
    for bit, qs, qe, ks, ke in ranges:
        m = np.uint64(1) << np.uint64(bit % 64)
        qb[bit // 64, max(0, qs):min(seq_len, qe)] |= m
        kb[bit // 64, max(0, ks):min(seq_len, ke)] |= m
    return qb, kb


@pytest.mark.parametrize("seed", range(20))
def test_host_grant_ranges_match_oracle(seed):
    seq_len, spans, l2t = _random_scenario(random.Random(100 + seed))
    creator = CrossDocLinkMaskCreator(_NoDetector(), max_grants=128)
    ranges = creator._grant_ranges(seq_len, spans, l2t)
    assert [r[0] for r in ranges] == list(range(len(ranges)))  # consecutive grant indices
    qb, kb = _paint(seq_len, ranges, 2)
    oq, ok, on = mo.build_grant_bitmasks(seq_len, spans, l2t, 2, 128)
    assert len(ranges) == on and np.array_equal(qb, oq) and np.array_equal(kb, ok)


@pytest.mark.parametrize("n_grants,max_grants", [(65, 64), (257, 256), (129, 256)])
def test_host_grant_ranges_truncate_like_oracle(n_grants, max_grants):
    seq_len, spans, l2t = _n_grant_scenario(n_grants)
    creator = CrossDocLinkMaskCreator(_NoDetector(), max_grants=max_grants)
    ranges = creator._grant_ranges(seq_len, spans, l2t)
    qb, kb = _paint(seq_len, ranges, creator._n_chunks)
    oq, ok, on = mo.build_grant_bitmasks(seq_len, spans, l2t, creator._n_chunks, max_grants)
    assert len(ranges) == on == min(n_grants, max_grants)
    assert np.array_equal(qb, oq) and np.array_equal(kb, ok)


def test_max_grants_cosine_warmup():
    c = CrossDocLinkMaskCreator(_NoDetector(), max_grants=256, max_grants_start=64,
                                max_grants_warmup_steps=10)
    assert c._current_max_grants() == 64
    c._step = 5
    assert c._current_max_grants() == 160  # 64 + 192 * (1 - cos(pi/2)) / 2
    c._step = 10
    assert c._current_max_grants() == 256
    assert c._n_chunks == 4


def test_link_matching_dag_rule():
    from types import SimpleNamespace as NS
    spans = [MockDocSpan(7, "A", 0, 10), MockDocSpan(9, "B", 10, 30)]
    links = [NS(link_end_pos=15, target_str="A"), NS(link_end_pos=5, target_str="B"),
             NS(link_end_pos=20, target_str="missing")]
    c = CrossDocLinkMaskCreator(_NoDetector())
    assert c._match_links_to_docs(links, spans) == {15: [7]}


def test_document_ids_known_answer():
    """Explicit expected maps (block_mask_creator.py:107-117 semantics): doc 5
    on [-3, 4) is clipped at 0; doc 7 on [8, 40) is clipped at T = 20 and
    overwrites token 8 of doc 6; doc 9 on [12, 14) overwrites the middle of
    doc 7; doc 2 on [30, 35) lies past T and writes nothing.  The second case
    leaves gaps, which stay -1."""
    spans = _spans((5, -3, 4), (6, 4, 9), (7, 8, 40), (9, 12, 14), (2, 30, 35))
    want = np.array([5, 5, 5, 5, 6, 6, 6, 6, 7, 7, 7, 7, 9, 9, 7, 7, 7, 7, 7, 7], np.int32)
    assert np.array_equal(mo.document_ids(20, spans), want)
    gap = _spans((1, 0, 3), (2, 5, 7))  # tokens 3, 4 and 7.. uncovered: -1
    want_gap = np.array([1, 1, 1, -1, -1, 2, 2, -1, -1], np.int32)
    assert np.array_equal(mo.document_ids(9, gap), want_gap)
    assert np.array_equal(document_ids_host(9, gap), want_gap)


def test_document_ids_host_matches_oracle():
    spans = _spans((5, -3, 4), (6, 4, 9), (7, 8, 40))  # clipped, overlapping, overflow
    assert np.array_equal(document_ids_host(20, spans), mo.document_ids(20, spans))


# --- dense-mask invariants (test_cross_doc_mask.py:103-125) ---------------------

@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_dense_mask_invariants(cfg):
    for row in synth.config_rows(cfg, seed=1, T=512):
        doc, qb, kb = row_arrays(row)
        dense = mo.dense_mask(doc, qb, kb)
        assert not np.triu(dense, 1).any(), "no future attention"
        assert dense.diagonal().all(), "every position attends to itself"


def test_doc_link_form_equals_grant_form():
    """Doc-level link rows expressed as grants reproduce the dense mask built
    from explicit per-document grants."""
    row = synth.linked_lognormal_docs(600, 40.0, 1.0, 200, 0.3, seed=4)
    doc, qb, kb = row_arrays(row)
    dense = mo.dense_mask(doc, qb, kb)
    idx = row.doc_index
    expect = np.zeros_like(dense)
    for i in range(row.n_docs):
        for j in range(i + 1):
            if int(row.link_rows[i, j // 64]) >> (j % 64) & 1:
                expect |= (idx[:, None] == i) & (idx[None, :] == j)
    expect &= np.tri(600, dtype=bool)
    assert np.array_equal(dense, expect)


# --- tile classification against torch's create_block_mask ----------------------

def _torch_block_mask(doc, qb, kb):
    from torch.nn.attention.flex_attention import create_block_mask
    T = doc.shape[0]
    mod = mo.torch_mask_mod(torch.from_numpy(doc),
                            None if qb is None else torch.from_numpy(qb.view(np.int64)),
                            None if kb is None else torch.from_numpy(kb.view(np.int64)))
    return create_block_mask(mod, None, None, T, T, device="cpu")


CASES = [("c1", lambda: row_arrays(synth.config_rows(1, seed=0)[0])),
         ("c3_1k", lambda: row_arrays(synth.config_rows(3, seed=2, T=1024)[0])),
         ("c4_1k", lambda: row_arrays(synth.config_rows(4, seed=3, T=1024)[0])),
         ("ragged_777_w2", lambda: random_row(777, np.random.default_rng(7), words=2, uncovered=True)),
         ("ragged_300_w0", lambda: random_row(300, np.random.default_rng(8), words=0, uncovered=True))]


@pytest.mark.parametrize("name,make", CASES, ids=[c[0] for c in CASES])
def test_oracle_tables_match_torch_create_block_mask(name, make):
    doc, qb, kb = make()
    ref = mo.block_mask_tables(doc, qb, kb)
    bm = _torch_block_mask(doc, qb, kb)
    np.testing.assert_array_equal(ref["kv_num_blocks"], bm.kv_num_blocks[0, 0].numpy())
    np.testing.assert_array_equal(ref["kv_indices"], bm.kv_indices[0, 0].numpy())
    np.testing.assert_array_equal(ref["full_kv_num_blocks"], bm.full_kv_num_blocks[0, 0].numpy())
    np.testing.assert_array_equal(ref["full_kv_indices"], bm.full_kv_indices[0, 0].numpy())
    np.testing.assert_array_equal(ref["q_num_blocks"], bm.q_num_blocks[0, 0].numpy())
    np.testing.assert_array_equal(ref["q_indices"], bm.q_indices[0, 0].numpy())
    np.testing.assert_array_equal(ref["full_q_num_blocks"], bm.full_q_num_blocks[0, 0].numpy())
    np.testing.assert_array_equal(ref["full_q_indices"], bm.full_q_indices[0, 0].numpy())


@pytest.mark.parametrize("name,make", CASES, ids=[c[0] for c in CASES])
def test_c_tile_oracle_matches_numpy(name, make):
    doc, qb, kb = make()
    np.testing.assert_array_equal(tile_oracle.tile_counts(doc, qb, kb), mo.tile_counts(doc, qb, kb))


def test_single_document_closed_form():
    T = 1000
    counts = tile_oracle.tile_counts(np.zeros(T, np.int32))
    partial, full = mo.classify_tiles(counts)
    nt = 8
    assert np.array_equal(full, np.tril(np.ones((nt, nt), np.int8), -1) * (np.arange(nt) < 7)[:, None])
    # diagonal tiles and the padded last row are partial; nothing above the diagonal
    assert (np.diag(partial) == 1).all() and not np.triu(partial, 1).any()
    assert partial[7, :7].all()
    # exact counts: causal pairs
    assert counts.sum() == T * (T + 1) // 2


def test_dense_to_ordered_matches_torch():
    from torch.nn.attention.flex_attention import _dense_to_ordered
    rng = np.random.default_rng(0)
    grid = (rng.random((9, 9)) < 0.4).astype(np.int8)
    num, idx = mo.dense_to_ordered(grid)
    tn, ti = _dense_to_ordered(torch.from_numpy(grid))
    assert np.array_equal(num, tn.numpy()) and np.array_equal(idx, ti.numpy())
