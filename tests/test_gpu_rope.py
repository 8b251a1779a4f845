"""GPU checks of the attention-module prologue (t2t_qkv_rope and its
gradient) and of the module around it.

The rotary variant of the reference's module (tunalab FlexSelfAttention) is
not available, so parity with it is unpinned; these tests pin the kernels to
the half-split rotation they implement, through:
  * an fp64 restatement of the rotation on the same bf16 inputs (within one
    bf16 rounding of the output);
  * the transpose identity: the gradient pass applied to the forward's output
    gives the input back (the rotation is orthogonal), so a sign or index slip
    in either pass fails;
  * the relative-position property: <R(m) q, R(n) k> depends on m - n only,
    checked through the pos0 offset;
  * torch autograd of the fp32 restatement for the backward;
  * a FlexSelfAttention forward + backward against an all-torch fp32 module.
"""
import math

import pytest
import torch

import tagseq2tagseq_amd.attention as attn_mod
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.block_mask import build_block_mask
from tagseq2tagseq_amd.mask_creators import TokenLists
from tagseq2tagseq_amd.rope import qkv_rope, rope_tables
from tests.helpers import dense_mask_torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _rotate_ref(x, cos, sin):
    """x [..., T, D] (float64) rotated by table rows [T, D/2] (float64)."""
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    return torch.cat((x1 * cos + x2 * sin, x2 * cos - x1 * sin), dim=-1)


def _split_ref(qkv, H, cos, sin):
    """fp64 restatement: [B, T, 3 H D] -> rotated q, k and v, each [B, H, T, D]."""
    B, T, C3 = qkv.shape
    D = C3 // (3 * H)
    x = qkv.double().view(B, T, 3, H, D).permute(2, 0, 3, 1, 4)
    c, s = cos.double(), sin.double()
    return _rotate_ref(x[0], c, s), _rotate_ref(x[1], c, s), x[2]


def _bf16_close(got, ref, what):
    """Within one bf16 rounding (2^-8 relative) of the fp64 value."""
    err = (got.double() - ref).abs()
    bound = ref.abs() * 2.0 ** -8 + 1e-6
    assert bool((err <= bound).all()), f"{what}: max excess {(err - bound).max().item():.3g}"


@pytest.mark.parametrize("B,T,H,D,pos0", [(1, 300, 12, 64, 0), (2, 128, 4, 128, 17),
                                          (1, 1, 2, 64, 5), (1, 77, 3, 32, 0)])
def test_forward_matches_fp64_rotation(B, T, H, D, pos0):
    g = torch.Generator().manual_seed(B * 1000 + T)
    qkv = torch.randn(B, T, 3 * H * D, generator=g).to(torch.bfloat16).to(DEV)
    cos, sin = rope_tables(D, pos0 + T + 3, DEV)
    q, k, v = qkv_rope(qkv, cos, sin, H, pos0)
    rq, rk, rv = _split_ref(qkv, H, cos[pos0:pos0 + T], sin[pos0:pos0 + T])
    assert q.shape == (B, H, T, D) and q.is_contiguous()
    _bf16_close(q, rq, "q")
    _bf16_close(k, rk, "k")
    assert torch.equal(v.double(), rv)  # v is copied bit-exactly


def test_strided_input_rows():
    """Token rows with padding (stride > 3 H D) and a batch stride."""
    B, T, H, D = 2, 200, 6, 64
    g = torch.Generator().manual_seed(7)
    big = torch.randn(B, T, 3 * H * D + 64, generator=g).to(torch.bfloat16).to(DEV)
    qkv = big[:, :, 32:32 + 3 * H * D]
    assert qkv.stride(1) == 3 * H * D + 64
    cos, sin = rope_tables(D, T, DEV)
    q, k, v = qkv_rope(qkv, cos, sin, H)
    rq, rk, rv = _split_ref(qkv, H, cos, sin)
    _bf16_close(q, rq, "q")
    _bf16_close(k, rk, "k")
    assert torch.equal(v.double(), rv)


def test_backward_inverts_forward():
    """dqkv = R^T applied to (q, k, v) returns qkv: R^T R = I."""
    B, T, H, D = 1, 257, 8, 128
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn(B, T, 3 * H * D, generator=g).to(torch.bfloat16).to(DEV)
    cos, sin = rope_tables(D, T, DEV)
    q, k, v = qkv_rope(qkv, cos, sin, H)
    back = torch.ops.t2t.qkv_rope_backward(q, k, v, cos, sin, 0)
    # Two bf16 roundings between qkv and back, each relative to the rotated
    # pair (x[i], x[i + D/2]), whose norm the rotation preserves.
    x = qkv.float().view(B, T, 3, H, D)
    h = D // 2
    r = torch.sqrt(x[..., :h] ** 2 + x[..., h:] ** 2).repeat(1, 1, 1, 1, 2).view_as(qkv)
    err = (back.float() - qkv.float()).abs()
    assert bool((err <= r * 2.0 ** -7 + 1e-6).all())
    assert torch.equal(back.view(B, T, 3, H, D)[:, :, 2], qkv.view(B, T, 3, H, D)[:, :, 2])


def test_relative_position_property():
    """<R(m) q, R(n) k> is the same for (m, n) and (m + s, n + s)."""
    H, D, T = 4, 64, 64
    g = torch.Generator().manual_seed(11)
    qkv = torch.randn(1, T, 3 * H * D, generator=g).to(torch.bfloat16).to(DEV)
    cos, sin = rope_tables(D, 4096, DEV)
    dots = []
    for shift in (0, 100, 3000):
        q, k, _ = qkv_rope(qkv, cos, sin, H, shift)
        dots.append((q.float() @ k.float().transpose(-1, -2)))
    scale = dots[0].abs().max().item()
    for d in dots[1:]:
        assert (d - dots[0]).abs().max().item() < 0.05 * scale


def test_backward_matches_autograd_of_fp32_rotation():
    B, T, H, D = 2, 150, 4, 64
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(B, T, 3 * H * D, generator=g).to(torch.bfloat16).to(DEV)
    gq, gk, gv = (torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(DEV)
                  for _ in range(3))
    cos, sin = rope_tables(D, T, DEV)
    x = qkv.clone().requires_grad_(True)
    q, k, v = qkv_rope(x, cos, sin, H)
    ((q.float() * gq.float()).sum() + (k.float() * gk.float()).sum()
     + (v.float() * gv.float()).sum()).backward()
    xr = qkv.double().requires_grad_(True)
    rq, rk, rv = _split_ref(xr, H, cos, sin)
    ((rq * gq.double()).sum() + (rk * gk.double()).sum() + (rv * gv.double()).sum()).backward()
    _bf16_close(x.grad, xr.grad, "dqkv")


def test_table_bounds_raise():
    qkv = torch.zeros(1, 64, 3 * 2 * 64, dtype=torch.bfloat16, device=DEV)
    cos, sin = rope_tables(64, 64, DEV)
    with pytest.raises(RuntimeError, match="table rows"):
        qkv_rope(qkv, cos, sin, 2, 1)


def test_opcheck():
    B, T, H, D = 1, 64, 2, 64
    qkv = torch.randn(B, T, 3 * H * D, device=DEV).to(torch.bfloat16).requires_grad_(True)
    cos, sin = rope_tables(D, T, DEV)
    torch.library.opcheck(torch.ops.t2t.qkv_rope.default, (qkv, cos, sin, H, 0),
                          test_utils=("test_schema", "test_faketensor",
                                      "test_autograd_registration"))


class _TorchAttention(torch.nn.Module):
    """All-torch fp32 restatement of FlexSelfAttention: linear QKV, half-split
    rotation, dense masked softmax attention, output projection."""

    def __init__(self, mod, bm):
        super().__init__()
        self.mod, self.bm = mod, bm

    def forward(self, x):
        m = self.mod
        B, T, C = x.shape
        H, D = m.num_heads, m.head_dim
        qkv = x.float() @ m.qkv.weight.float().t()
        cos, sin = rope_tables(D, T, x.device)
        x5 = qkv.view(B, T, 3, H, D).permute(2, 0, 3, 1, 4)
        q, k, v = _rotate_ref(x5[0], cos, sin), _rotate_ref(x5[1], cos, sin), x5[2]
        bm = self.bm
        mask = dense_mask_torch(bm.doc_ids[0], bm.q_bits[0] if bm.words else None,
                                bm.kv_bits[0] if bm.words else None, 0, T)
        s = (q @ k.transpose(-1, -2)) / math.sqrt(D)
        p = torch.softmax(s.masked_fill(~mask, float("-inf")), -1).nan_to_num(0.0)
        y = (p @ v).transpose(1, 2).reshape(B, T, C)
        return y @ m.proj.weight.float().t()


@pytest.mark.parametrize("C,H", [(768, 12), (512, 4)])
def test_attention_module_forward_backward(C, H):
    T = 512
    row = synth.linked_lognormal_docs(T, 120.0, 1.0, 512, 0.3, seed=4)
    lists = TokenLists(T, [row.spans], DEV, words=row.words, link_rows=[row.link_rows])
    bm = build_block_mask(*lists.build())
    torch.manual_seed(1)
    mod = attn_mod.FlexSelfAttention(C, H, T).to(DEV, torch.bfloat16)
    x = torch.randn(1, T, C, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    gy = torch.randn(1, T, C, device=DEV, dtype=torch.bfloat16)
    y = mod(x, bm)
    y.backward(gy)
    xr = x.detach().float().requires_grad_(True)
    ref = _TorchAttention(mod, bm)
    yr = ref(xr)
    wq = mod.qkv.weight
    yr.backward(gy.float())
    err = (y.float() - yr).abs().max().item() / yr.abs().max().item()
    assert err < 2e-2, f"output rel err {err}"
    gerr = (x.grad.float() - xr.grad).abs().max().item() / xr.grad.abs().max().item()
    assert gerr < 3e-2, f"dx rel err {gerr}"
    assert wq.grad is not None and torch.isfinite(wq.grad).all()
