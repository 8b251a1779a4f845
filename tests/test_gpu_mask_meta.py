"""GPU parity of the metadata kernel (t2t_mask_meta) against the CPU oracle:
tile classes and all eight BlockMask tables must be bit-identical."""
import numpy as np
import pytest
import torch

from oracle import mask_oracle as mo
from oracle import tile_oracle
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.block_mask import build_block_mask
from tests.helpers import TABLES
from tests.helpers import check_block_mask as _check
from tests.helpers import random_row, row_arrays, to_dev_words

pytestmark = pytest.mark.gpu

def _run(rows_np, device, label):
    doc = torch.stack([torch.from_numpy(r[0]) for r in rows_np]).to(device)
    if rows_np[0][1] is None:
        qb = kb = None
    else:
        qb = torch.stack([to_dev_words(r[1], device) for r in rows_np])
        kb = torch.stack([to_dev_words(r[2], device) for r in rows_np])
    bm = build_block_mask(doc, qb, kb)
    torch.cuda.synchronize()
    _check(bm, rows_np, label)
    return bm


@pytest.mark.parametrize("cfg,T", [(1, None), (2, 2048), (3, 4096), (4, 8192)])
def test_config_rows_reduced(cfg, T, gpu_device):
    rows = [row_arrays(r) for r in synth.config_rows(cfg, seed=0, T=T)]
    _run(rows, gpu_device, f"config{cfg} T={T}")


@pytest.mark.parametrize("cfg", [2, 3, 4])
def test_config_rows_full_size(cfg, gpu_device):
    rows = [row_arrays(r) for r in synth.config_rows(cfg, seed=0)]
    _run(rows, gpu_device, f"config{cfg} full")


@pytest.mark.parametrize("T", [1, 7, 64, 127, 128, 129, 255, 1000, 1537])
@pytest.mark.parametrize("words", [0, 1, 3])
def test_ragged_random(T, words, gpu_device):
    rng = np.random.default_rng(T * 31 + words)
    rows = [random_row(T, rng, words=words, uncovered=True, max_doc=150)]
    _run(rows, gpu_device, f"ragged T={T} W={words}")


@pytest.mark.parametrize("T,words", [(300, 0), (1000, 2), (2100, 8)])
def test_many_short_runs(T, words, gpu_device):
    # documents of 1-2 tokens: 60-120 runs per 128-token tile side, so the
    # run-pair loop takes many passes and run starts fall in both 64-token halves
    rng = np.random.default_rng(T + words)
    rows = [random_row(T, rng, words=words, uncovered=True, max_doc=3) for _ in range(2)]
    _run(rows, gpu_device, f"short runs T={T} W={words}")


def test_max_words_and_batch(gpu_device):
    rng = np.random.default_rng(5)
    rows = [random_row(777, rng, words=8, uncovered=True) for _ in range(3)]
    _run(rows, gpu_device, "W=8 Bm=3")


def test_single_document_is_causal(gpu_device):
    T = 1024
    doc = np.zeros(T, dtype=np.int32)
    bm = _run([(doc, None, None)], gpu_device, "causal")
    tc = bm.tile_class.cpu().numpy()[0]
    nt = T // 128
    # closed form: strictly lower tiles full, diagonal partial, upper skip
    exp = np.tril(np.full((nt, nt), 2, np.int8), -1) + np.eye(nt, dtype=np.int8)
    np.testing.assert_array_equal(tc, exp)


def test_deterministic(gpu_device):
    rows = [row_arrays(r) for r in synth.config_rows(3, seed=1, T=4096)]
    a = _run(rows, gpu_device, "det a")
    b = _run(rows, gpu_device, "det b")
    for name in TABLES + ["tile_class", "row_order", "col_order", "kv_bits_off"]:
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    # q_bits_slot is defined for the first q_num_blocks entries of each column
    nt = a.num_tiles
    valid = torch.arange(nt, device=a.q_num_blocks.device)[None, None, :] < a.q_num_blocks[:, 0, :, None]
    assert torch.equal(a.q_bits_slot[valid], b.q_bits_slot[valid])


@pytest.mark.parametrize("name", ["config1_T1024", "config3_T4096", "config4_T4096"])
def test_golden_fixture(name, gpu_device):
    import os
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", f"mask_{name}.npz"))
    qb = f["q_bits"] if "q_bits" in f else None
    kb = f["kv_bits"] if "kv_bits" in f else None
    bm = build_block_mask(torch.from_numpy(f["doc"]).to(gpu_device), to_dev_words(qb, gpu_device),
                          to_dev_words(kb, gpu_device))
    np.testing.assert_array_equal(bm.tile_class[0].cpu().numpy(), f["tile_class"])
    for n in TABLES:
        np.testing.assert_array_equal(getattr(bm, n)[0, 0].cpu().numpy(), f[n], err_msg=n)
