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


def test_chunked_loss_all_ignored_is_nan_like_torch():
    """Every target ignore_index: torch's mean cross-entropy is 0 / 0 = NaN,
    and no row has a gradient."""
    emb = nn.Embedding(20, 8)
    loss = LinearCELoss(8, 20, weight=emb.weight, chunk=3)
    x = torch.randn(1, 10, 8, requires_grad=True)
    t = torch.full((1, 10), -100)
    got = loss(x, t)
    ref = F.cross_entropy(x[0] @ emb.weight.T, t[0], ignore_index=-100)
    assert math.isnan(float(got)) and math.isnan(float(ref))
    got.backward()
    assert (x.grad == 0).all()


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


def test_token_lists_packing_clips_bounds_and_wraps_doc_ids():
    """TokenLists packs each row's spans and grants as int32 with bounds
    clipped to [-1, T + 1] (same coverage of [0, T)) and doc ids wrapped to
    int32; rows with bounds beyond int64 take the per-entry path."""
    import random
    import numpy as np
    from tagseq2tagseq_amd import mask_creators as mc, synth
    rng = random.Random(0)
    T = 1000
    for _ in range(50):
        B = rng.randint(1, 3)
        spans = [[synth.DocSpan(doc_id=rng.randint(-5, 2 ** 40), start=rng.randint(-50, 1100),
                                end=rng.randint(-50, 1100)) for _ in range(rng.randint(0, 6))]
                 for _ in range(B)]
        grants = [[(rng.randint(0, 127), *[rng.randint(-50, 1100) for _ in range(4)])
                   for _ in range(rng.randint(0, 5))] for _ in range(B)]
        if rng.random() < 0.2 and spans[0]:
            spans[0][0] = synth.DocSpan(doc_id=1, start=-2 ** 70, end=2 ** 70)
        got = mc.TokenLists(T, spans, torch.device("cpu"), 2, grants, None).lists.numpy()
        ms = max(1, max(len(r) for r in spans))
        mg = max(1, max(len(r) for r in grants))
        sp = np.zeros((B, ms, 3), np.int64)
        gr = np.zeros((B, mg, 5), np.int64)
        for b, row in enumerate(spans):
            for i, s in enumerate(row):
                sp[b, i] = (min(max(s.start, -1), T + 1), min(max(s.end, -1), T + 1),
                            (s.doc_id + 2 ** 31) % 2 ** 32 - 2 ** 31)
        for b, row in enumerate(grants):
            for i, (bit, *bounds) in enumerate(row):
                gr[b, i] = (bit, *[min(max(x, -1), T + 1) for x in bounds])
        cnt = np.array([[len(r) for r in spans], [len(r) for r in grants]])
        ref = np.concatenate([sp.ravel(), gr.ravel(), cnt.ravel()]).astype(np.int32)
        assert np.array_equal(got, ref)


def test_fp8_out_proj_is_warned_about():
    import warnings
    from tagseq2tagseq_amd.attention import FlexSelfAttention
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        FlexSelfAttention(64, 2, 128)
        assert not w
        m = FlexSelfAttention(64, 2, 128, fp8_out_proj=True)
    assert m.fp8_out_proj and any("fp8" in str(x.message) for x in w)


def test_model_weights_state_tracks_edits_and_mode():
    """TS2TSModel drops its generation cache when this state changes."""
    from tagseq2tagseq_amd.model import TS2TSModel
    torch.manual_seed(0)
    m = TS2TSModel.from_config(vocab_size=50, num_layers=2, model_dim=64, num_heads=2,
                               max_seq_len=64, dropout=0.0, drop_path_rate=0.0,
                               block_mask_creator=None).eval()
    s0 = m._weights_state()
    assert m._weights_state() == s0
    with torch.no_grad():
        m.backbone.layers[0].mlp.down.weight.add_(1.0)
    s1 = m._weights_state()
    assert s1 != s0
    m.backbone.load_state_dict(m.backbone.state_dict())
    s2 = m._weights_state()
    assert s2 != s1
    m.train()
    assert m._weights_state() != s2
    m.eval()
    assert m._weights_state() == s2


def test_gemm_tuning_file_has_validators_and_gfx950_shapes():
    from tagseq2tagseq_amd import gemm_tuning
    lines = open(gemm_tuning.TUNED_FILE).read().splitlines()
    validators = {l.split(",")[1] for l in lines if l.startswith("Validator,")}
    assert {"PT_VERSION", "HIP_VERSION", "HIPBLASLT_VERSION", "GCN_ARCH_NAME"} <= validators
    assert any("gfx950" in l for l in lines if l.startswith("Validator,GCN_ARCH_NAME"))
    shapes = [l.split(",")[1] for l in lines if l.startswith("GemmTunableOp")]
    # the head (vocabulary padded to 50264) and the four layer projections
    assert any("50264" in s for s in shapes) and len(shapes) >= 10
    if not torch.cuda.is_available():
        assert gemm_tuning.use_tuned_gemms() is False
