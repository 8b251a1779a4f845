"""Modules on the GPU: a Layer against the same Layer with the attention
replaced by an fp32 dense masked reference, and a small training-module step."""
import math

import numpy as np
import pytest
import torch

import tagseq2tagseq_amd.attention as attn_mod
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.block_mask import build_block_mask
from tagseq2tagseq_amd.mask_creators import TokenLists
from tagseq2tagseq_amd.modules import Layer, TS2TSTrainingModule
from tests.helpers import assert_close, dense_mask_torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _dense_flex(bm):
    """flex_attention stand-in: fp32 dense attention under the mask's mask_mod."""
    def fa(q, k, v, block_mask=None, **kw):
        T = q.shape[2]
        m = dense_mask_torch(bm.doc_ids[0], bm.q_bits[0] if bm.words else None,
                             bm.kv_bits[0] if bm.words else None, 0, T)
        s = (q.float() @ k.float().transpose(-1, -2)) / math.sqrt(q.shape[-1])
        s = s.masked_fill(~m, float("-inf"))
        p = torch.softmax(s, -1).nan_to_num(0.0)
        return (p @ v.float()).to(q.dtype)
    return fa


@pytest.mark.parametrize("n_embd,n_head", [(512, 8), (512, 4)])
def test_layer_matches_dense_reference(n_embd, n_head, monkeypatch):
    T = 512
    row = synth.linked_lognormal_docs(T, 120.0, 1.0, 512, 0.3, seed=3)
    lists = TokenLists(T, [row.spans], DEV, words=row.words, link_rows=[row.link_rows])
    bm = build_block_mask(*lists.build())
    torch.manual_seed(0)
    layer = Layer(n_embd, n_head, 0.0, T, False, 0.0).to(DEV, torch.bfloat16)
    x = torch.randn(1, T, n_embd, device=DEV, dtype=torch.bfloat16)
    got = layer(x, bm).float()
    monkeypatch.setattr(attn_mod, "flex_attention", _dense_flex(bm))
    ref = layer(x, bm).float()
    assert_close(got, ref, 2e-2, 2e-2, "layer output")


def test_float32_layer_forward_and_backward(monkeypatch):
    """A Layer left in float32 runs the float32 attention kernels (and the
    torch QKV rotation); output and input gradient against the same Layer
    with fp32 dense attention, at the float32 bound 1e-4."""
    T = 384
    row = synth.linked_lognormal_docs(T, 90.0, 1.0, 384, 0.3, seed=5)
    lists = TokenLists(T, [row.spans], DEV, words=row.words, link_rows=[row.link_rows])
    bm = build_block_mask(*lists.build())
    torch.manual_seed(1)
    layer = Layer(256, 4, 0.0, T, False, 0.0).to(DEV)
    x = torch.randn(1, T, 256, device=DEV)
    g = torch.randn(1, T, 256, device=DEV)
    xa = x.clone().requires_grad_(True)
    got = layer(xa, bm)
    got.backward(g)
    monkeypatch.setattr(attn_mod, "flex_attention", _dense_flex(bm))
    xb = x.clone().requires_grad_(True)
    ref = layer(xb, bm)
    ref.backward(g)
    assert got.dtype == torch.float32
    assert_close(got.detach(), ref.detach(), 1e-4, 1e-4, "float32 layer output")
    assert_close(xa.grad, xb.grad, 1e-4, 1e-4, "float32 layer input gradient")


def test_training_module_step():
    T = 1024
    row = synth.config_rows(3, seed=1, T=T)[0]
    lists = TokenLists(T, [row.spans], DEV, words=row.words, link_rows=[row.link_rows])
    torch.manual_seed(0)
    m = TS2TSTrainingModule.from_config(
        vocab_size=1000, num_layers=4, model_dim=256, num_heads=4, max_seq_len=T, dropout=0.0,
        drop_path_rate=0.0, block_mask_creator=lambda tokens, **kw: build_block_mask(*lists.build())
    ).to(DEV, torch.bfloat16)
    opt = torch.optim.AdamW(m.parameters(), lr=1e-3, foreach=True)
    tokens = torch.randint(0, 1000, (1, T + 1), device=DEV)
    losses = []
    for _ in range(3):
        loss = m({"tokens": tokens})
        loss.backward()
        assert all(p.grad is None or torch.isfinite(p.grad).all() for p in m.parameters())
        opt.step()
        opt.zero_grad(set_to_none=True)
        losses.append(float(loss))
    assert all(math.isfinite(l) for l in losses)
    assert losses[-1] < losses[0]  # memorising one batch


def test_backbone_activation_checkpointing_matches_plain():
    """TS2TSBackbone(activation_checkpointing=True) (backbone.py:99-102: each
    layer's forward, attention included, re-runs inside the backward) on a
    cross_doc_link mask against the same weights without checkpointing: the
    output bitwise equal, the input and parameter gradients within 2e-2; the
    attention forward runs twice per layer with checkpointing, once without."""
    from tagseq2tagseq_amd.modules import TS2TSBackbone
    T, L = 1024, 4
    row = synth.config_rows(3, seed=2, T=T)[0]
    lists = TokenLists(T, [row.spans], DEV, words=row.words, link_rows=[row.link_rows])
    bm = build_block_mask(*lists.build())
    assert bm.words > 0
    torch.manual_seed(4)
    plain = TS2TSBackbone(L, 256, 4, T, 0.0, 0.0).to(DEV, torch.bfloat16)
    ckpt = TS2TSBackbone(L, 256, 4, T, 0.0, 0.0, activation_checkpointing=True).to(
        DEV, torch.bfloat16)
    ckpt.load_state_dict(plain.state_dict())
    calls = {"n": 0}

    def count(*_):
        calls["n"] += 1
    for m in (plain, ckpt):
        for layer in m.layers:
            layer.attn.register_forward_hook(count)
    x = torch.randn(1, T, 256, device=DEV, dtype=torch.bfloat16)
    g = torch.randn(1, T, 256, device=DEV, dtype=torch.bfloat16)
    res = []
    for m in (plain, ckpt):
        calls["n"] = 0
        xi = x.clone().requires_grad_(True)
        y = m(xi, bm)
        y.backward(g)
        res.append((y.detach(), xi.grad, {n: p.grad for n, p in m.named_parameters()},
                    calls["n"]))
    (y0, gx0, gp0, n0), (y1, gx1, gp1, n1) = res
    assert (n0, n1) == (L, 2 * L)
    assert torch.equal(y0, y1)
    assert_close(gx1, gx0, 2e-2, 2e-2, "checkpointed input gradient")
    for name, ref in gp0.items():
        assert gp1[name] is not None, name
        scale = float(ref.float().abs().max())
        assert_close(gp1[name], ref, 2e-2 * max(scale, 1.0), 2e-2, f"checkpointed grad {name}")
