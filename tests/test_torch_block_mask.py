"""A torch BlockMask (create_block_mask with the reference's mask_mod) as the
flex_attention seam's mask: the conversion's tables, launch orders, bitmap
slots and partial-tile bitmaps against the oracle (CPU), and on the GPU the
attention outputs and gradients bitwise equal to those under the library's own
metadata pass for the same mask."""
import math

import numpy as np
import pytest
import torch
from torch.nn.attention.flex_attention import create_block_mask

from oracle import mask_oracle as mo
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.block_mask import build_block_mask, from_torch_block_mask
from tests.helpers import check_block_mask, random_row, row_arrays, to_dev_words


def _torch_mask(doc, qb, kb, device):
    mod = mo.torch_mask_mod(torch.from_numpy(doc).to(device),
                            None if qb is None else to_dev_words(qb, device),
                            None if kb is None else to_dev_words(kb, device))
    T = doc.shape[0]
    return create_block_mask(mod, None, None, T, T, device=device)


CASES = [
    ("config1", lambda: row_arrays(synth.config_rows(1, seed=0)[0])),
    ("config3 T1024", lambda: row_arrays(synth.config_rows(3, seed=2, T=1024)[0])),
    ("config4 T1024", lambda: row_arrays(synth.config_rows(4, seed=1, T=1024)[0])),
    ("ragged T300 words", lambda: random_row(300, np.random.default_rng(5), words=2, uncovered=True)),
    ("T129", lambda: random_row(129, np.random.default_rng(6), words=1)),
]


@pytest.mark.parametrize("name,make", CASES, ids=[c[0] for c in CASES])
def test_conversion_matches_oracle(name, make):
    doc, qb, kb = make()
    bm = from_torch_block_mask(_torch_mask(doc, qb, kb, "cpu"))
    check_block_mask(bm, [(doc, qb, kb)], name)
    assert bm.mask_mod() is not None


def _doc_bidirectional(doc, device):
    d = torch.from_numpy(doc).to(device)

    def mod(b, h, q, k):
        return d[q] == d[k]
    return mod


def _sliding_window(w, device):
    def mod(b, h, q, k):
        return (q - k).abs() <= w
    return mod


NON_CAUSAL = [
    ("doc bidirectional T384", 384, lambda dev: _doc_bidirectional(
        random_row(384, np.random.default_rng(8), max_doc=150)[0], dev)),
    ("doc bidirectional T1000", 1000, lambda dev: _doc_bidirectional(
        row_arrays(synth.config_rows(3, seed=4, T=1000)[0])[0], dev)),
    ("sliding window 100 T700", 700, lambda dev: _sliding_window(100, dev)),
]


def _dense(mod, T):
    q = torch.arange(T)[:, None]
    k = torch.arange(T)[None, :]
    return torch.as_tensor(mod(torch.zeros(()), torch.zeros(()), q, k)).expand(T, T).numpy()


def check_any_mask(bm, dense, label):
    """Tables of a converted mask with tiles on either side of the diagonal:
    the tile classes from the dense mask (torch's padding with False), every
    partial tile's two bitmaps, and distinct slots for distinct partial tiles."""
    T = dense.shape[0]
    nt = (T + 127) // 128
    pad = np.zeros((nt * 128, nt * 128), dtype=bool)
    pad[:T, :T] = dense
    tiles = pad.reshape(nt, 128, nt, 128).transpose(0, 2, 1, 3)
    cnt = tiles.sum((2, 3))
    exp_cls = np.where(cnt == 128 * 128, 2, np.where(cnt > 0, 1, 0))
    np.testing.assert_array_equal(bm.tile_class[0].cpu().numpy(), exp_cls, err_msg=label)
    off = bm.kv_bits_off[0].cpu().numpy().astype(np.int64)
    bits = bm.tile_bits.cpu().numpy()
    slots = {}
    for r, c in zip(*np.nonzero(exp_cls == 1)):
        slot = off[r] + c
        assert slot not in slots, f"{label}: tiles {slots.get(slot)} and {(r, c)} share slot {slot}"
        slots[slot] = (r, c)
        assert slot < bits.shape[0], f"{label}: slot {slot} past the {bits.shape[0]} slots"
        tile = tiles[r, c]
        np.testing.assert_array_equal(
            bits[slot, 0].view("<u4"), np.packbits(tile, axis=1, bitorder="little").view("<u4"),
            err_msg=f"{label}: row bits ({r},{c})")
        np.testing.assert_array_equal(
            bits[slot, 1].view("<u4"),
            np.packbits(tile.T.copy(), axis=1, bitorder="little").view("<u4"),
            err_msg=f"{label}: column bits ({r},{c})")
    q_num = bm.q_num_blocks[0, 0].cpu().numpy()
    q_idx = bm.q_indices[0, 0].cpu().numpy()
    q_slot = bm.q_bits_slot[0].cpu().numpy()
    for c in range(nt):
        for i in range(q_num[c]):
            assert q_slot[c, i] == off[q_idx[c, i]] + c, f"{label}: q_bits_slot ({c},{i})"
    assert any(c > r for r, c in slots.values()), f"{label}: no partial tile above the diagonal"


@pytest.mark.parametrize("name,T,make", NON_CAUSAL, ids=[c[0] for c in NON_CAUSAL])
def test_conversion_of_non_causal_masks(name, T, make):
    mod = make("cpu")
    bm = from_torch_block_mask(create_block_mask(mod, None, None, T, T, device="cpu"))
    check_any_mask(bm, _dense(mod, T), name)


def test_conversion_rejects_unsupported_masks():
    def causal(b, h, q, k):
        return q >= k
    with pytest.raises(ValueError, match="tiles"):
        from_torch_block_mask(create_block_mask(causal, None, None, 256, 256, device="cpu",
                                                BLOCK_SIZE=64))
    with pytest.raises(ValueError, match="head"):
        from_torch_block_mask(create_block_mask(causal, None, 2, 256, 256, device="cpu"))
    with pytest.raises(ValueError, match="self-attention"):
        from_torch_block_mask(create_block_mask(causal, None, None, 256, 384, device="cpu"))


@pytest.mark.gpu
@pytest.mark.parametrize("name,make", CASES[1:], ids=[c[0] for c in CASES[1:]])
def test_torch_block_mask_attention_equals_own_mask(name, make):
    from tagseq2tagseq_amd.attention import flex_attention
    dev = torch.device("cuda:0")
    doc, qb, kb = make()
    T = doc.shape[0]
    tbm = _torch_mask(doc, qb, kb, dev)
    own = build_block_mask(torch.from_numpy(doc).to(dev), to_dev_words(qb, dev),
                           to_dev_words(kb, dev))
    g = torch.Generator().manual_seed(T)
    q, k, v, do = (torch.randn(1, 4, T, 128, generator=g).to(torch.bfloat16).to(dev)
                   for _ in range(4))
    res = []
    for mask in (tbm, own):
        qq, kk, vv = (x.clone().requires_grad_(True) for x in (q, k, v))
        out, lse = flex_attention(qq, kk, vv, block_mask=mask, return_lse=True)
        out.backward(do)
        res.append([out, lse, qq.grad, kk.grad, vv.grad])
    for what, a, b in zip(("out", "lse", "dq", "dk", "dv"), *res):
        assert torch.equal(a, b), f"{name}: {what} differs (max {(a.float() - b.float()).abs().max():.3g})"
    assert getattr(tbm, "_t2t_block_mask", None) is not None  # converted once, kept


@pytest.mark.gpu
@pytest.mark.parametrize("name,T,make", NON_CAUSAL, ids=[c[0] for c in NON_CAUSAL])
def test_non_causal_torch_block_mask_against_oracle(name, T, make):
    """Attention under a converted non-causal torch BlockMask (partial tiles
    above the diagonal, square slot layout) against the float64 oracle on
    the dense mask: 2e-2 abs and rel for bf16."""
    from oracle import attn_oracle as ao
    from tagseq2tagseq_amd.attention import flex_attention
    from tests.helpers import assert_close
    dev = torch.device("cuda:0")
    dense = _dense(make("cpu"), T)
    tbm = create_block_mask(make(dev), None, None, T, T, device=dev)
    g = torch.Generator().manual_seed(T + 1)
    q, k, v, do = (torch.randn(1, 2, T, 64, generator=g).to(torch.bfloat16).to(dev)
                   for _ in range(4))
    qq, kk, vv = (x.clone().requires_grad_(True) for x in (q, k, v))
    out, lse = flex_attention(qq, kk, vv, block_mask=tbm, return_lse=True)
    out.backward(do)
    qn, kn, vn, don = (x.float().cpu().numpy() for x in (q, k, v, do))
    o_ref, lse_ref = ao.attention_fwd(qn, kn, vn, dense[None])
    dq_ref, dk_ref, dv_ref = ao.attention_bwd(qn, kn, vn, o_ref, don, lse_ref, dense[None])
    for what, got, ref in (("out", out, o_ref), ("dq", qq.grad, dq_ref), ("dk", kk.grad, dk_ref),
                           ("dv", vv.grad, dv_ref)):
        assert_close(got.detach(), torch.from_numpy(ref), 2e-2, 2e-2, f"{name} {what}")
    assert_close(lse.detach(), torch.from_numpy(lse_ref), 1e-3, 1e-3, f"{name} lse")
