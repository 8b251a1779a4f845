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
