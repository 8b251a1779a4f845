"""Synthetic workload generators match the configurations they stand for."""
import numpy as np
import pytest

from tagseq2tagseq_amd import synth


@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_rows_cover_the_sequence(cfg):
    c = synth.CONFIGS[cfg]
    rows = synth.config_rows(cfg, seed=0)
    assert len(rows) == (c["B"] if cfg == 2 else 1)
    for r in rows:
        assert r.seq_len == c["T"]
        assert r.spans[0].start == 0 and r.spans[-1].end == c["T"]
        assert all(a.end == b.start for a, b in zip(r.spans, r.spans[1:]))
        assert (r.doc_index >= 0).all()
        ids = [s.doc_id for s in r.spans]
        assert len(set(ids)) == len(ids) and ids != list(range(len(ids)))


def test_config1_lengths_uniform():
    r = synth.config_rows(1, seed=0)[0]
    lens = [s.end - s.start for s in r.spans]
    assert all(32 <= n <= 256 for n in lens[:-1]) and lens[-1] <= 256


@pytest.mark.parametrize("cfg", [3, 4])
def test_link_rows_lower_triangular_with_diagonal(cfg):
    r = synth.config_rows(cfg, seed=0)[0]
    n, W = r.n_docs, r.words
    assert W == (n + 63) // 64
    for i in range(n):
        bits = [(int(r.link_rows[i, j // 64]) >> (j % 64)) & 1 for j in range(W * 64)]
        assert bits[i] == 1
        assert not any(bits[i + 1:])


def test_config3_shape_and_density():
    r = synth.config_rows(3, seed=0)[0]
    assert 20 <= r.n_docs <= 64 and r.words == 1
    n = r.n_docs
    links = sum(bin(int(r.link_rows[i, 0])).count("1") - 1 for i in range(n))
    frac = links / (n * (n - 1) / 2)
    assert 0.05 < frac < 0.3  # p = 0.15


def test_config4_needs_several_words():
    r = synth.config_rows(4, seed=0)[0]
    assert r.n_docs > 64 and r.words >= 2
