"""GPU parity of the device-side per-token input builder (t2t_token_inputs)
against the oracle's restatement of the reference's span and grant loops
(block_mask_creator.py:107-117, cross_doc_mask.py:210-300) and of the doc-link
bitmask encoding; bit-exact."""
import random

import numpy as np
import pytest
import torch

from oracle import mask_oracle as mo
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.block_mask import build_block_mask
from tagseq2tagseq_amd.mask_creators import (CrossDocLinkMaskCreator, TokenLists,
                                             create_doc_causal_block_mask,
                                             create_doc_link_block_mask, token_inputs)
from tests.test_oracle_mask import (MockDocSpan, _NoDetector, _n_grant_scenario,
                                    _random_scenario)

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _u64(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint64)


def _random_spans(rng: random.Random, T: int):
    """Overlapping, unsorted, partly out-of-range and empty spans."""
    spans = []
    for i in range(rng.randint(0, 300)):
        s = rng.randint(-50, T + 20)
        e = s + rng.randint(-5, 400)
        spans.append(MockDocSpan(rng.randint(-3, 10 ** 6), f"d{i}", s, e))
    return spans


@pytest.mark.parametrize("seed", range(8))
def test_doc_ids_match_oracle(seed):
    rng = random.Random(seed)
    T = rng.choice([1, 100, 257, 1024, 4099])
    spans = _random_spans(rng, T)
    doc, qb, kb = token_inputs(T, spans, DEV)
    assert qb is None and kb is None
    assert np.array_equal(doc[0].cpu().numpy(), mo.document_ids(T, spans)), f"seed {seed}"


@pytest.mark.parametrize("seed", range(12))
def test_grant_words_match_oracle(seed):
    seq_len, spans, l2t = _random_scenario(random.Random(500 + seed))
    creator = CrossDocLinkMaskCreator(_NoDetector(), max_grants=128)
    qb, kb, n = creator._build_grant_bitmasks(seq_len, spans, l2t, device=DEV)
    oq, ok, on = mo.build_grant_bitmasks(seq_len, spans, l2t, 2, 128)
    assert n == on
    assert np.array_equal(_u64(qb[0]), oq) and np.array_equal(_u64(kb[0]), ok)


@pytest.mark.parametrize("n_grants,max_grants", [(64, 64), (65, 64), (257, 256), (300, 512)])
def test_grant_capacity_and_bit63(n_grants, max_grants):
    seq_len, spans, l2t = _n_grant_scenario(n_grants)
    creator = CrossDocLinkMaskCreator(_NoDetector(), max_grants=max_grants)
    qb, kb, n = creator._build_grant_bitmasks(seq_len, spans, l2t, device=DEV)
    oq, ok, on = mo.build_grant_bitmasks(seq_len, spans, l2t, creator._n_chunks, max_grants)
    assert n == on == min(n_grants, max_grants)
    assert np.array_equal(_u64(qb[0]), oq) and np.array_equal(_u64(kb[0]), ok)
    # grant 63 sets the sign bit, the INT64_MIN pattern of cross_doc_mask.py:285-287
    assert (qb[0, 0].cpu().numpy() == np.iinfo(np.int64).min).any()


@pytest.mark.parametrize("cfg", [3, 4])
def test_doc_link_words_match_oracle(cfg):
    for row in synth.config_rows(cfg, seed=2, T=4096):
        doc, qb, kb = token_inputs(row.seq_len, row.spans, DEV, words=row.words,
                                   links=row.link_rows)
        oq, ok = mo.doc_link_token_bits(row.doc_index, row.link_rows)
        assert np.array_equal(doc[0].cpu().numpy(), mo.document_ids(row.seq_len, row.spans))
        assert np.array_equal(_u64(qb[0]), oq) and np.array_equal(_u64(kb[0]), ok)


def test_batched_rows_match_per_row_builds():
    rows = synth.config_rows(2, seed=3, T=2048)
    lists = TokenLists(2048, [r.spans for r in rows], DEV)
    doc, _, _ = lists.build()
    for b, r in enumerate(rows):
        assert np.array_equal(doc[b].cpu().numpy(), mo.document_ids(2048, r.spans))


def test_grants_and_links_combine():
    """Grant words OR onto the doc-link words (both forms in one launch)."""
    row = synth.config_rows(3, seed=4, T=1024)[0]
    grants = [(0, 100, 300, 700, 900), (63, 0, 50, 1000, 1024)]
    doc, qb, kb = token_inputs(1024, row.spans, DEV, words=row.words, grants=grants,
                               links=row.link_rows)
    oq, ok = mo.doc_link_token_bits(row.doc_index, row.link_rows)
    for bit, qs, qe, ks, ke in grants:
        m = np.uint64(1) << np.uint64(bit)
        oq[0, qs:qe] |= m
        ok[0, ks:ke] |= m
    assert np.array_equal(_u64(qb[0]), oq) and np.array_equal(_u64(kb[0]), ok)


def test_creators_end_to_end():
    """The mask creators built on the device builder give the oracle's tables."""
    row = synth.config_rows(3, seed=5, T=2048)[0]
    tokens = torch.zeros((1, 2048), dtype=torch.int64, device=DEV)
    bm = create_doc_link_block_mask(tokens, row.spans, row.link_rows)
    oq, ok = mo.doc_link_token_bits(row.doc_index, row.link_rows)
    ref = mo.block_mask_tables(mo.document_ids(2048, row.spans), oq, ok)
    assert np.array_equal(bm.kv_num_blocks[0, 0].cpu().numpy(), ref["kv_num_blocks"])
    assert np.array_equal(bm.full_kv_num_blocks[0, 0].cpu().numpy(), ref["full_kv_num_blocks"])
    bm2 = create_doc_causal_block_mask(tokens, row.spans)
    ref2 = mo.block_mask_tables(mo.document_ids(2048, row.spans))
    assert np.array_equal(bm2.kv_num_blocks[0, 0].cpu().numpy(), ref2["kv_num_blocks"])
    assert np.array_equal(bm2.full_kv_num_blocks[0, 0].cpu().numpy(), ref2["full_kv_num_blocks"])
