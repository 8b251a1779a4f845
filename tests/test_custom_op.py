"""The torch.library custom ops over the kernels have schemas and fake
(meta) implementations, so compiled models trace them without a GPU."""
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import tagseq2tagseq_amd.attention  # noqa: F401  (registers torch.ops.t2t.*)


def test_fake_shapes_forward_and_backward():
    with FakeTensorMode():
        q = torch.empty(2, 8, 384, 128, dtype=torch.bfloat16)
        kv = torch.empty(2, 2, 384, 128, dtype=torch.bfloat16)
        tables = [torch.empty(1, 1, 3, dtype=torch.int32) for _ in range(13)]
        out, lse2 = torch.ops.t2t.masked_attention(q, kv, kv, tables, 0.088)
        assert out.shape == q.shape and out.dtype == torch.bfloat16
        assert lse2.shape == (2, 8, 384) and lse2.dtype == torch.float32
        dq, dk, dv = torch.ops.t2t.masked_attention_backward(q, kv, kv, out, out, lse2, tables,
                                                             0.088)
        assert dq.shape == q.shape and dk.shape == kv.shape and dv.shape == kv.shape


def test_schemas():
    s = str(torch.ops.t2t.masked_attention.default._schema)
    assert "Tensor[] tables" in s and "float scale" in s
    s = str(torch.ops.t2t.masked_attention_backward.default._schema)
    assert s.count("Tensor") >= 7


def test_qkv_rope_fake_shapes_and_schema():
    import tagseq2tagseq_amd.rope  # noqa: F401  (registers torch.ops.t2t.qkv_rope*)
    with FakeTensorMode():
        qkv = torch.empty(2, 96, 3 * 12 * 64, dtype=torch.bfloat16)
        cos = torch.empty(128, 32)
        q, k, v = torch.ops.t2t.qkv_rope(qkv, cos, cos, 12, 0)
        assert q.shape == k.shape == v.shape == (2, 12, 96, 64)
        dqkv = torch.ops.t2t.qkv_rope_backward(q, k, v, cos, cos, 0)
        assert dqkv.shape == qkv.shape and dqkv.dtype == torch.bfloat16
    s = str(torch.ops.t2t.qkv_rope.default._schema)
    assert "num_heads" in s and "pos0" in s


def test_attention_output_is_token_major():
    """The forward's output is [B, T, H, D] storage seen as [B, H, T, D], so the
    module's transpose + reshape to [B, T, C] is a view."""
    with FakeTensorMode():
        q = torch.empty(1, 4, 256, 64, dtype=torch.bfloat16)
        tables = [torch.empty(1, 1, 2, dtype=torch.int32) for _ in range(13)]
        out, _ = torch.ops.t2t.masked_attention(q, q, q, tables, 0.125)
        y = out.transpose(1, 2)
        assert y.is_contiguous()
        assert y.reshape(1, 256, 256).data_ptr() == out.data_ptr()
