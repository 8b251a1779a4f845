"""The committed golden fixtures (tests/golden/, written by make_golden.py
from the oracle after a cross-check against torch's eager flex_attention)
still match the oracle: a regression pin of oracle/ itself."""
import glob
import os

import numpy as np
import pytest
import torch

from oracle import attn_oracle as ao
from oracle import mask_oracle as mo

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TABLES = ["kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
          "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices"]


def bf16_bits_to_f64(b):
    return torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).float().numpy().astype(np.float64)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(HERE, "mask_*.npz"))),
                         ids=lambda p: os.path.basename(p))
def test_mask_fixture(path):
    f = np.load(path)
    qb = f["q_bits"] if "q_bits" in f else None
    kb = f["kv_bits"] if "kv_bits" in f else None
    ref = mo.block_mask_tables(f["doc"], qb, kb)
    assert np.array_equal(ref["partial"] + 2 * ref["full"], f["tile_class"])
    for n in TABLES:
        assert np.array_equal(ref[n], f[n]), n


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(HERE, "attn_*.npz"))),
                         ids=lambda p: os.path.basename(p))
def test_attn_fixture(path):
    f = np.load(path)
    qb = f["q_bits"] if "q_bits" in f else None
    kb = f["kv_bits"] if "kv_bits" in f else None
    q, k, v, do = (bf16_bits_to_f64(f[n]) for n in ("q", "k", "v", "do"))
    dense = mo.dense_mask(f["doc"], qb, kb)[None]
    o, lse = ao.attention_fwd(q, k, v, dense)
    dq, dk, dv = ao.attention_bwd(q, k, v, o, do, lse, dense)
    for name, got in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        np.testing.assert_allclose(got, f[name].astype(np.float64), rtol=1e-3, atol=1e-3, err_msg=name)
