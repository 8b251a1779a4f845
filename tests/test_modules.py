"""Model modules (reference signatures) on the CPU: norms, GLU, the chunked
linear + cross-entropy loss and the backbone's skip wiring."""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from tagseq2tagseq_amd.modules import (GLU, DropPath, LinearCELoss, RMSNorm, TS2TSBackbone,
                                       TS2TSTrainingModule)


def test_rmsnorm_closed_form():
    n = RMSNorm(8)
    with torch.no_grad():
        n.weight.copy_(torch.arange(1, 9, dtype=torch.float32))
    x = torch.tensor([[3.0, -4.0, 0, 0, 0, 0, 0, 0]])
    rms = math.sqrt((9 + 16) / 8 + 1e-6)
    assert torch.allclose(n(x), x / rms * n.weight, atol=1e-6)


def test_glu_is_swiglu():
    torch.manual_seed(0)
    m = GLU(6, 5, 4)
    x = torch.randn(3, 6)
    g, u = (x @ m.gate_up.weight.T).chunk(2, -1)
    assert torch.allclose(m(x), (F.silu(g) * u) @ m.down.weight.T, atol=1e-6)


def test_drop_path_identity_at_zero_and_eval():
    x = torch.randn(4, 3)
    assert torch.equal(DropPath(0.0)(x), x)
    d = DropPath(0.5).eval()
    assert torch.equal(d(x), x)


def test_chunked_loss_matches_full_cross_entropy():
    torch.manual_seed(1)
    emb = nn.Embedding(50, 16)
    loss = LinearCELoss(16, 50, weight=emb.weight, chunk=7)
    x = torch.randn(1, 33, 16, requires_grad=True)
    t = torch.randint(0, 50, (1, 33))
    t[0, 5] = -100
    got = loss(x, t)
    ref = F.cross_entropy((x[0] @ emb.weight.T), t[0], ignore_index=-100)
    assert torch.allclose(got, ref, atol=1e-5)
    got.backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()


class _Add(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.c = c

    def forward(self, x, block_mask):
        return x + self.c


def test_backbone_skip_wiring():
    """backbone.py:93-120: outputs of layers 0..n/2-1 re-enter, weighted, before
    layers n/2.. in reverse order."""
    bb = TS2TSBackbone.__new__(TS2TSBackbone)
    nn.Module.__init__(bb)
    bb.layers = nn.ModuleList([_Add(10.0 ** i) for i in range(4)])
    bb.skip_weights = nn.Parameter(torch.tensor([2.0, 3.0]))
    bb.activation_checkpointing = False
    x0 = torch.zeros(1)
    # l0: 1; l1: 1 + 10 = 11; before l2 (weight[0] = 2, last pushed = 11):
    # 11 + 2 * 11 = 33, l2: 133; before l3 (weight[1] = 3, first pushed = 1):
    # 133 + 3 * 1 = 136, l3: 1136
    assert bb(x0, None).item() == 1136.0


def test_training_module_signature():
    m = TS2TSTrainingModule.from_config(vocab_size=100, num_layers=2, model_dim=64, num_heads=1,
                                        max_seq_len=32, dropout=0.0, drop_path_rate=0.0,
                                        block_mask_creator=lambda **kw: None)
    assert m.loss_fn.weight is m.embedding.weight  # weight tying
    assert len(m.backbone.layers) == 2 and m.backbone.skip_weights.numel() == 1
