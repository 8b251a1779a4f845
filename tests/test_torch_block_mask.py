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
