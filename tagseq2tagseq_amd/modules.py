"""Model modules around the masked attention, with the reference's
constructors and call signatures, for the layer / backbone / training-step
measurements (the 12-layer training-step workload) and as the drop-in host of
the attention.

Mirrors (reference file:line):
  * ``Layer`` -- model/modules/layer.py:11-35 (RMSNorm -> FlexSelfAttention ->
    residual; RMSNorm -> GLU(silu, hidden 8/3 n_embd) -> residual; DropPath)
  * ``TS2TSBackbone`` -- model/modules/backbone.py:11-120 (layer stack with
    skip connections from the first half of the layers to the second half,
    optional activation checkpointing)
  * ``TS2TSTrainingModule`` -- model/modules/training_module.py:12-230 (embedding
    -> backbone -> RMSNorm -> linear + cross-entropy, weight tying, the mask
    built once per step by ``block_mask_creator`` from the batch)

``RMSNorm``, ``GLU``, ``DropPath`` and the fused linear-cross-entropy loss
come from the absent ``tunalab`` package in the reference; they are written
here from their textbook definitions (parity with tunalab unpinned; the
attention kernels do not depend on them).  fp8 projections are accepted and
ignored (bf16 only).
"""
from __future__ import annotations

from typing import Any, Callable, Dict, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
import torch.utils.checkpoint

from . import norm
from .attention import FlexSelfAttention
from .glu import SwiGLUFn, swiglu_applies
from .head_loss import HeadCEFn, fused_head_applies, head_loss_needs_grad, head_loss_value
from .linear import Linear


class RMSNorm(nn.Module):
    """y = x / sqrt(mean(x^2) + eps) * weight (computed in fp32).  bf16 rows on
    the GPU run the one-pass kernels (t2t::rms_norm, with its gradient); other
    dtypes and CPU tensors use the same formula in torch."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if norm.kernel_applies(x, self.weight):
            return norm.rms_norm(x, self.weight, self.eps)
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


class GLU(nn.Module):
    """Gated linear unit: out(act(gate(x)) * up(x)) (SwiGLU for silu; bf16 rows
    on the GPU run the fused SwiGLU kernels of ``glu``)."""

    def __init__(self, in_dim: int, out_dim: int, hidden_dim: int, activation: str = "silu",
                 dropout: float = 0.0, fp8: bool = False):
        super().__init__()
        self.gate_up = Linear(in_dim, 2 * hidden_dim, bias=False)
        self.down = Linear(hidden_dim, out_dim, bias=False)
        self.act = {"silu": F.silu, "gelu": F.gelu, "relu": F.relu}[activation]
        self.dropout = nn.Dropout(dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gu = self.gate_up(x)
        if self.act is F.silu and swiglu_applies(gu) and not torch.compiler.is_compiling():
            # one fused pass each way (t2t_swiglu), the gradient of [g | u] whole
            return self.dropout(self.down(SwiGLUFn.apply(gu)))
        g, u = gu.chunk(2, dim=-1)
        return self.dropout(self.down(self.act(g) * u))


class DropPath(nn.Module):
    """Stochastic depth: zero a sample's residual branch with probability p."""

    def __init__(self, p: float = 0.0):
        super().__init__()
        self.p = p

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.p == 0.0 or not self.training:
            return x
        keep = torch.rand((x.shape[0],) + (1,) * (x.dim() - 1), device=x.device) >= self.p
        return x * keep.to(x.dtype) / (1.0 - self.p)


class Layer(nn.Module):
    """model/modules/layer.py:11-35."""

    def __init__(self, n_embd: int, n_head: int, dropout: float, max_seq_len: int, fp8: bool,
                 drop_path_rate: float):
        super().__init__()
        self.drop_path = DropPath(drop_path_rate)
        self.ln_1 = RMSNorm(n_embd)
        self.attn = FlexSelfAttention(dim=n_embd, num_heads=n_head, max_seq_len=max_seq_len,
                                      fp8_out_proj=fp8)
        self.ln_2 = RMSNorm(n_embd)
        self.mlp = GLU(in_dim=n_embd, out_dim=n_embd, hidden_dim=int(8 / 3 * n_embd),
                       activation="silu", dropout=dropout, fp8=fp8)

    def forward(self, x: torch.Tensor, block_mask) -> torch.Tensor:
        x = x + self.drop_path(self.attn(self.ln_1(x), block_mask=block_mask))
        x = x + self.drop_path(self.mlp(self.ln_2(x)))
        return x


class TS2TSBackbone(nn.Module):
    """model/modules/backbone.py:11-120: the layer stack; the outputs of the
    first num_layers // 2 layers are added (weighted) to the inputs of the
    last ones in reverse order."""

    def __init__(self, num_layers: int, model_dim: int, num_heads: int, max_seq_len: int,
                 dropout: float, drop_path_rate: float, fp8: bool = False,
                 activation_checkpointing: bool = False, **kwargs):
        super().__init__()
        self.model_dim = model_dim
        self.max_seq_len = max_seq_len
        self.layers = nn.ModuleList([
            Layer(n_embd=model_dim, n_head=num_heads, max_seq_len=max_seq_len, dropout=dropout,
                  drop_path_rate=drop_path_rate, fp8=fp8) for _ in range(num_layers)])
        self.skip_weights = nn.Parameter(torch.ones(num_layers // 2))
        self.activation_checkpointing = activation_checkpointing

    def forward(self, x: torch.Tensor, block_mask: Any) -> torch.Tensor:
        skips = []
        n_skip = len(self.skip_weights)
        for i, layer in enumerate(self.layers):
            if i >= n_skip and skips:
                x = x + self.skip_weights[i - n_skip] * skips.pop()
            if self.activation_checkpointing:
                x = torch.utils.checkpoint.checkpoint(layer, x, block_mask, use_reentrant=False)
            else:
                x = layer(x, block_mask)
            if i < n_skip:
                skips.append(x)
        return x


class LinearCELoss(nn.Module):
    """Linear head + mean cross-entropy (the role of tunalab's FusedLinearCELoss,
    model/modules/training_module.py:127-133, 209).  bf16 rows on the GPU run
    the fused path of ``head_loss`` (the logit gradient produced in the
    forward by the ``t2t_ce_rows`` kernel, no recomputation, no fp32 logits;
    ``gpu_chunk`` rows per chunk, None = as many as 2 GiB of bf16 logits
    hold); other inputs are evaluated in row chunks of ``chunk`` with
    recomputation, so the full [T, V] logits never exist at once.  ``weight``
    ties the head to the embedding."""

    def __init__(self, D: int, V: int, dtype: torch.dtype = torch.bfloat16,
                 ignore_index: int = -100, weight: Optional[nn.Parameter] = None,
                 chunk: int = 4096, gpu_chunk: Optional[int] = None):
        super().__init__()
        self.weight = weight if weight is not None else nn.Parameter(torch.empty(V, D))
        if weight is None:
            nn.init.normal_(self.weight, std=D ** -0.5)
        self.ignore_index = ignore_index
        self.chunk = chunk
        self.gpu_chunk = gpu_chunk

    def forward(self, x: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
        x = x.reshape(-1, x.shape[-1])
        t = targets.reshape(-1)
        if fused_head_applies(x, self.weight) and not torch.compiler.is_compiling():
            if not head_loss_needs_grad(x, self.weight):
                return head_loss_value(x, self.weight, t, self.ignore_index, self.gpu_chunk)
            return HeadCEFn.apply(x, self.weight, t, int(self.ignore_index), self.gpu_chunk)
        # mean over the counted rows; 0 / 0 = NaN when every row is ignored,
        # as torch's mean cross-entropy
        n = (t != self.ignore_index).sum()
        total = x.new_zeros((), dtype=torch.float32)
        for r0 in range(0, x.shape[0], self.chunk):
            xs, ts = x[r0:r0 + self.chunk], t[r0:r0 + self.chunk]
            total = total + torch.utils.checkpoint.checkpoint(
                self._chunk_loss, xs, ts, use_reentrant=False)
        return total / n

    def _chunk_loss(self, xs: torch.Tensor, ts: torch.Tensor) -> torch.Tensor:
        logits = F.linear(xs, self.weight.to(xs.dtype)).float()
        return F.cross_entropy(logits, ts, ignore_index=self.ignore_index, reduction="sum")


class TS2TSTrainingModule(nn.Module):
    """model/modules/training_module.py:12-230: batch in, loss out."""

    def __init__(self, backbone: TS2TSBackbone, embedding: nn.Embedding, norm: RMSNorm,
                 loss_fn: LinearCELoss, block_mask_creator: Callable, vocab_size: int,
                 ignore_index: int = -100):
        super().__init__()
        self.backbone = backbone
        self.embedding = embedding
        self.norm = norm
        self.loss_fn = loss_fn
        self.block_mask_creator = block_mask_creator
        self.vocab_size = vocab_size
        self.ignore_index = ignore_index

    @classmethod
    def from_config(cls, vocab_size: int, num_layers: int, model_dim: int, num_heads: int,
                    max_seq_len: int, dropout: float, drop_path_rate: float,
                    block_mask_creator: Callable, fp8: bool = False, weight_tying: bool = True,
                    ignore_index: int = -100, dtype: torch.dtype = torch.bfloat16,
                    activation_checkpointing: bool = False) -> "TS2TSTrainingModule":
        backbone = TS2TSBackbone(num_layers=num_layers, model_dim=model_dim, num_heads=num_heads,
                                 max_seq_len=max_seq_len, dropout=dropout,
                                 drop_path_rate=drop_path_rate, fp8=fp8,
                                 activation_checkpointing=activation_checkpointing)
        embedding = nn.Embedding(vocab_size, model_dim)
        norm = RMSNorm(model_dim)
        loss_fn = LinearCELoss(D=model_dim, V=vocab_size, dtype=dtype, ignore_index=ignore_index,
                               weight=embedding.weight if weight_tying else None)
        return cls(backbone, embedding, norm, loss_fn, block_mask_creator, vocab_size,
                   ignore_index)

    def forward(self, batch: Dict[str, Any]) -> torch.Tensor:
        tokens = batch["tokens"]
        input_ids = tokens[:, :-1].contiguous()
        target_ids = tokens[:, 1:].contiguous()
        block_mask = self.block_mask_creator(**{**batch, "tokens": input_ids})
        x = self.embedding(input_ids)
        x = self.backbone(x, block_mask=block_mask)
        x = self.norm(x)
        return self.loss_fn(x, target_ids)
