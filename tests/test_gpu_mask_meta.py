"""GPU parity of the metadata kernel (t2t_mask_meta) against the CPU oracle:
tile classes and all eight BlockMask tables must be bit-identical."""
import numpy as np
import pytest
import torch

from oracle import mask_oracle as mo
from oracle import tile_oracle
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.block_mask import build_block_mask
from tests.helpers import random_row, row_arrays, to_dev_words

pytestmark = pytest.mark.gpu

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
    rc = (kv_num + full_num)[row_order]
    cc = (q_num + q_full)[col_order]
    assert (np.diff(rc) <= 0).all() and (np.diff(cc) <= 0).all(), f"{label}: orders not longest-first"
    base = int(bm.kv_num_blocks[:b].sum().item())
    exp_off = base + np.concatenate([[0], np.cumsum(kv_num)[:-1]])
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
            slot = off[qt] + i
            row_slot[(qt, kt)] = slot
            tile = rows[:, kt * 128:(kt + 1) * 128]
            np.testing.assert_array_equal(bits[slot, 0].view("<u4"), _pack_bits(tile),
                                          err_msg=f"{label}: row bits tile ({qt},{kt})")
            np.testing.assert_array_equal(bits[slot, 1].view("<u4"), _pack_bits(tile.T.copy()),
                                          err_msg=f"{label}: column bits tile ({qt},{kt})")
    for kt in range(nt):
        for i in range(q_num[kt]):
            assert slot_col[kt, i] == row_slot[(q_idx[kt, i], kt)], f"{label}: q_bits_slot ({kt},{i})"


def _check(bm, rows_np, label):
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
