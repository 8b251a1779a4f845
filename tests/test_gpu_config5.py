"""configs[4] on the GPU: the 12-layer backbone training step at its workload
(12 layers, d_model 768, 12 heads of 64, SwiGLU 4x, RMSNorm, RoPE, vocab
50257, T = 16384 random token ids, the configs[2] cross_doc_link generator;
model/modules/training_module.py:177-211, backbone.py:70-109), and a reduced
backbone of the same width whose loss and input gradient are compared with
the same modules on dense float32 masked attention."""
import math

import pytest
import torch

import tagseq2tagseq_amd.attention as attn_mod
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.block_mask import build_block_mask
from tagseq2tagseq_amd.mask_creators import TokenLists
from tagseq2tagseq_amd.modules import TS2TSTrainingModule
from tests.helpers import dense_mask_torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
VOCAB = 50257


def _module(T, layers, seed, lists):
    torch.manual_seed(seed)
    return TS2TSTrainingModule.from_config(
        vocab_size=VOCAB, num_layers=layers, model_dim=768, num_heads=12, max_seq_len=T,
        dropout=0.0, drop_path_rate=0.0,
        block_mask_creator=lambda tokens, **kw: build_block_mask(*lists.build()),
    ).to(DEV, torch.bfloat16)


def test_config5_training_steps():
    """Three AdamW steps of the full configs[4] workload on one packed row:
    finite loss and gradients, and the loss falls (one batch is memorised)."""
    T = 16384
    row = synth.config_rows(3, seed=0)[0]
    assert row.seq_len == T
    lists = TokenLists(T, [row.spans], DEV, words=row.words, link_rows=[row.link_rows])
    m = _module(T, 12, 0, lists)
    assert sum(p.numel() for p in m.parameters()) > 1.2e8
    opt = torch.optim.AdamW(m.parameters(), lr=1e-3, foreach=True)
    g = torch.Generator().manual_seed(0)
    tokens = torch.randint(0, VOCAB, (1, T + 1), generator=g).to(DEV)
    losses = []
    for step in range(3):
        loss = m({"tokens": tokens})
        loss.backward()
        for name, p in m.named_parameters():
            assert p.grad is not None, f"step {step}: no gradient for {name}"
            assert torch.isfinite(p.grad).all(), f"step {step}: non-finite gradient in {name}"
        opt.step()
        opt.zero_grad(set_to_none=True)
        losses.append(float(loss.detach()))
    # (nn.Embedding's N(0, 1) init tied to the head, as in the reference's
    # from_config, training_module.py:120, puts the first loss far above ln V)
    assert all(math.isfinite(x) for x in losses), losses
    assert losses[2] < losses[1] < losses[0], losses


def _dense_flex(bm):
    """flex_attention stand-in: float32 dense attention under the mask's
    mask_mod (doc ids and grant words of the block mask)."""
    def fa(q, k, v, block_mask=None, **kw):
        T = q.shape[2]
        msk = dense_mask_torch(bm.doc_ids[0], bm.q_bits[0] if bm.words else None,
                               bm.kv_bits[0] if bm.words else None, 0, T)
        s = (q.float() @ k.float().transpose(-1, -2)) / math.sqrt(q.shape[-1])
        p = torch.softmax(s.masked_fill(~msk, float("-inf")), -1).nan_to_num(0.0)
        return (p @ v.float()).to(q.dtype)
    return fa


def test_reduced_backbone_matches_dense_attention(monkeypatch):
    """Two layers of the configs[4] width at T = 2048 under a cross_doc_link
    mask: the loss and the gradient at the backbone's input (the embedded
    tokens) against the same module with dense float32 attention, within 2e-2
    of the reference's scale."""
    T = 2048
    row = synth.config_rows(3, seed=2, T=T)[0]
    assert row.words >= 1 and row.n_docs > 2
    lists = TokenLists(T, [row.spans], DEV, words=row.words, link_rows=[row.link_rows])
    bm = build_block_mask(*lists.build())
    m = _module(T, 2, 1, lists)
    g = torch.Generator().manual_seed(1)
    tokens = torch.randint(0, VOCAB, (1, T + 1), generator=g).to(DEV)
    seen = {}

    def keep(mod, inp, out):
        out.retain_grad()
        seen["x"] = out

    m.embedding.register_forward_hook(keep)

    def run():
        loss = m({"tokens": tokens})
        loss.backward()
        grad = seen["x"].grad.float().clone()
        m.zero_grad(set_to_none=True)
        return float(loss.detach()), grad

    loss_k, grad_k = run()
    monkeypatch.setattr(attn_mod, "flex_attention", _dense_flex(bm))
    loss_r, grad_r = run()
    assert abs(loss_k - loss_r) <= 2e-2 * abs(loss_r), (loss_k, loss_r)
    scale = grad_r.abs().max().item()
    err = (grad_k - grad_r).abs().max().item()
    assert scale > 0 and err <= 2e-2 * scale, f"input gradient: max err {err:.3g} (scale {scale:.3g})"
