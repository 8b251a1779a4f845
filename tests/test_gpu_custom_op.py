"""The custom ops on the GPU: torch.library.opcheck (schema, fake tensor,
autograd registration, AOT dispatch) and a fully compiled fwd+bwd graph that
matches eager bit for bit."""
import math

import pytest
import torch

from tagseq2tagseq_amd.attention import flex_attention
from tagseq2tagseq_amd.block_mask import build_block_mask
import numpy as np

from tests.helpers import random_row, to_dev_words

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _inputs(T=384, Hq=4, Hkv=2, D=64, seed=0):
    doc, qb, kb = random_row(T, np.random.default_rng(seed), words=1)
    bm = build_block_mask(torch.from_numpy(doc).to(DEV), to_dev_words(qb, DEV),
                          to_dev_words(kb, DEV))
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, Hq, T, D, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(1, Hkv, T, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(1, Hkv, T, D, generator=g).to(torch.bfloat16).to(DEV)
    return q, k, v, bm


def test_opcheck():
    q, k, v, bm = _inputs()
    for t in (q, k, v):
        t.requires_grad_(True)
    torch.library.opcheck(torch.ops.t2t.masked_attention.default,
                          (q, k, v, bm.tables(), 1.0 / math.sqrt(64)))


def test_compiled_graph_matches_eager():
    q, k, v, bm = _inputs(seed=1)
    do = torch.randn_like(q)

    def fn(q, k, v):
        return flex_attention(q, k, v, block_mask=bm, enable_gqa=True)

    grads = []
    for f in (fn, torch.compile(fn, backend="aot_eager", fullgraph=True)):
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        out = f(qq, kk, vv)
        out.backward(do)
        grads.append([out.detach(), qq.grad, kk.grad, vv.grad])
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_compiled_layer_matches_eager():
    """A whole Layer (RMSNorm, QKV projection, rotary prologue, attention,
    out-projection, GLU) compiled with the aot_eager backend: the prologue,
    norm and attention kernels enter the graph as custom ops and give the
    eager results."""
    from tagseq2tagseq_amd.modules import Layer
    T, C, H = 256, 256, 4
    doc, qb, kb = random_row(T, np.random.default_rng(3), words=1)
    bm = build_block_mask(torch.from_numpy(doc).to(DEV), to_dev_words(qb, DEV),
                          to_dev_words(kb, DEV))
    torch.manual_seed(0)
    layer = Layer(C, H, 0.0, T, False, 0.0).to(DEV, torch.bfloat16)
    x = torch.randn(1, T, C, device=DEV).to(torch.bfloat16)
    gy = torch.randn(1, T, C, device=DEV).to(torch.bfloat16)

    def fn(x):
        return layer(x, bm)

    results = []
    for f in (fn, torch.compile(fn, backend="aot_eager", fullgraph=True)):
        layer.zero_grad(set_to_none=True)
        xx = x.detach().clone().requires_grad_(True)
        y = f(xx)
        y.backward(gy)
        results.append([y.detach(), xx.grad, layer.ln_1.weight.grad,
                        layer.attn.qkv.weight.grad])
    for a, b in zip(*results):
        assert torch.allclose(a.float(), b.float(), atol=2e-2, rtol=2e-2)
