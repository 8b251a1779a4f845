"""Inference wrapper with the reference's ``TS2TSModel`` interface, plus a
cached forward for generation.

Mirrors (reference file:line):
  * ``TS2TSModel.__init__`` / ``from_config`` / ``eval`` / ``train`` / ``to``
    (model/model.py:17-211): backbone, embedding / LM-head weights (tied by
    default), final norm, mask creator;
  * ``forward_inference(tokens, doc_spans, **kwargs)`` (model/model.py:214-237):
    mask, embedding, backbone, norm, LM head over the whole sequence.

Added for generation: ``forward_inference_last`` returns the logits of the
last position only -- the single row the generation loop reads
(model/generation_loop.py:90-97) -- and reuses the keys / values of every
position whose inputs are unchanged since the previous call (``KVCache``).
The reusable prefix is the longest one over which the token ids and all mask
inputs (doc id, q words, kv words) agree: a position's hidden states depend
only on the positions before it and on its own mask row, so they are exact
for that prefix.  The cache also records the weights it was filled with --
each parameter's storage address and version counter, and the train / eval
mode -- and is dropped when any of them changes (an optimizer step,
load_state_dict, an in-place edit, train() / eval()).  Writes through a
parameter's ``.data`` bypass its version counter; call ``reset_cache()`` after
such an edit.  New rows go through each layer with the decode-step kernel
(``t2t_attn_decode``, up to 8 rows per kv head per launch); when more than
``prefill_rows`` rows are new, the whole sequence is recomputed through the
block-mask kernels and the cache refilled.
"""
from __future__ import annotations

import ctypes
from typing import Any, Callable, List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .attention import flex_attention
from .block_mask import T2TBlockMask, build_block_mask
from .decode import MAX_ROWS, attn_decode
from .modules import RMSNorm, TS2TSBackbone
from .rope import qkv_rope
from .rows import applies as rows_apply, rows_linear, rows_qkv_rope


class KVCache:
    """Keys and values of every layer for the cached positions of one
    sequence (batch 1), with the token ids and mask inputs they were computed
    under.  Storage: k, v bf16 [L][1][H][cap][D]; doc int32 [1][cap]; q / kv
    words int64 [1][W][cap]."""

    def __init__(self, num_layers: int, num_heads: int, head_dim: int, capacity: int,
                 words: int, device, dtype=torch.bfloat16):
        shape = (num_layers, 1, num_heads, capacity, head_dim)
        self.k = torch.empty(shape, dtype=dtype, device=device)
        self.v = torch.empty(shape, dtype=dtype, device=device)
        self.tokens = torch.full((1, capacity), -1, dtype=torch.int64, device=device)
        self.doc = torch.empty((1, capacity), dtype=torch.int32, device=device)
        self.q_bits = torch.zeros((1, words, capacity), dtype=torch.int64, device=device)
        self.kv_bits = torch.zeros((1, words, capacity), dtype=torch.int64, device=device)
        self.capacity = capacity
        self.words = words
        self.length = 0

    def first_diff(self, tokens: torch.Tensor, bm, n: int) -> torch.Tensor:
        """Device int32 [1]: the first of positions 0 .. n - 1 whose token id
        or mask inputs (doc id, q / kv words) differ from the cached ones, or n
        (``t2t_first_input_diff`` lowering a fill of n; no host sync)."""
        out = torch.full((1,), n, dtype=torch.int32, device=self.tokens.device)

        def row(t):
            t = t[0]
            return t if t.stride(-1) == 1 else t.contiguous()

        tok, doc = row(tokens.to(torch.int64)), row(bm.doc_ids.to(torch.int32))
        qa = ka = qb = kb = None
        if self.words:
            qa, ka, qb, kb = (row(t) for t in (self.q_bits, self.kv_bits, bm.q_bits, bm.kv_bits))
            if qb.stride(0) != kb.stride(0):
                qb, kb = qb.contiguous(), kb.contiguous()
        ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
        with torch.cuda.device(out.device):
            rc = _lib.lib().t2t_first_input_diff(
                self.tokens.data_ptr(), tok.data_ptr(), self.doc.data_ptr(), doc.data_ptr(),
                ptr(qa), ptr(qb), ptr(ka), ptr(kb), qa.stride(0) if qa is not None else 0,
                qb.stride(0) if qb is not None else 0, self.words, n, out.data_ptr(),
                ctypes.c_void_p(torch.cuda.current_stream(out.device).cuda_stream))
        _lib.check(rc, "t2t_first_input_diff")
        return out

    def reusable_prefix(self, tokens: torch.Tensor, bm) -> int:
        """Length of the longest prefix whose token ids and mask inputs match."""
        n = min(self.length, tokens.shape[1])
        return int(self.first_diff(tokens, bm, n).item()) if n else 0

    def store_inputs(self, tokens: torch.Tensor, bm, p0: int, p1: int) -> None:
        self.tokens[0, p0:p1] = tokens[0, p0:p1]
        self.doc[0, p0:p1] = bm.doc_ids[0, p0:p1]
        if self.words:
            self.q_bits[0, :, p0:p1] = bm.q_bits[0, :, p0:p1]
            self.kv_bits[0, :, p0:p1] = bm.kv_bits[0, :, p0:p1]


class TS2TSModel:
    """model/model.py:17-237 (generation / evaluation helpers that need the
    absent tokenizer stack are not provided)."""

    def __init__(self, backbone: TS2TSBackbone, embedding_weight: torch.Tensor,
                 lm_head_weight: torch.Tensor, norm: nn.Module, block_mask_creator: Callable,
                 vocab_size: int, ignore_index: int = -100, tokenizer=None, link_detector=None,
                 layout_policy=None):
        self.backbone = backbone
        self.embedding_weight = embedding_weight
        self.lm_head_weight = lm_head_weight
        self.norm = norm
        self.block_mask_creator = block_mask_creator
        self.vocab_size = vocab_size
        self.ignore_index = ignore_index
        self.tokenizer = tokenizer
        self.link_detector = link_detector
        self.layout_policy = layout_policy
        self.kv_cache: Optional[KVCache] = None
        self.prefill_rows = 64
        self.use_graphs = True
        self.fuse_rows = True  # few-row steps on the fused row kernels (rows.py)
        self._graph: Optional[_DecodeGraph] = None
        self._weights_seen = None  # _weights_state() the cache was filled under
        self._param_slots = None   # (module, name) of every backbone / norm parameter

    @classmethod
    def from_config(cls, vocab_size: int, num_layers: int, model_dim: int, num_heads: int,
                    max_seq_len: int, dropout: float, drop_path_rate: float,
                    block_mask_creator: Callable, fp8: bool = False, weight_tying: bool = True,
                    ignore_index: int = -100, tokenizer=None, link_detector=None,
                    layout_policy=None) -> "TS2TSModel":
        backbone = TS2TSBackbone(num_layers=num_layers, model_dim=model_dim, num_heads=num_heads,
                                 max_seq_len=max_seq_len, dropout=dropout,
                                 drop_path_rate=drop_path_rate, fp8=fp8)
        embedding = nn.Embedding(vocab_size, model_dim)
        norm = RMSNorm(model_dim)
        if weight_tying:
            lm_head_weight = embedding.weight
        else:
            lm_head_weight = nn.Parameter(torch.empty(vocab_size, model_dim))
            nn.init.normal_(lm_head_weight, mean=0.0, std=0.02)
        return cls(backbone, embedding.weight, lm_head_weight, norm, block_mask_creator,
                   vocab_size, ignore_index, tokenizer, link_detector, layout_policy)

    def eval(self):
        self.backbone.eval()
        return self

    def train(self, mode: bool = True):
        self.backbone.train(mode)
        return self

    def to(self, device, dtype=None):
        self.backbone.to(device, dtype)
        self.norm.to(device, dtype)
        tied = self.lm_head_weight is self.embedding_weight
        self.embedding_weight = self.embedding_weight.to(device=device, dtype=dtype)
        self.lm_head_weight = (self.embedding_weight if tied else
                               self.lm_head_weight.to(device=device, dtype=dtype))
        self.kv_cache = None
        self._graph = None
        return self

    def reset_cache(self) -> None:
        self.kv_cache = None
        self._graph = None
        self._weights_seen = None
        self._param_slots = None

    def _weights_state(self):
        """What the cached keys / values depend on besides the inputs: the mode
        and, per parameter, its storage address and version counter (bumped by
        every in-place write through the parameter, optimizer steps and
        load_state_dict included).  The (module, attribute) slots that hold
        the parameters are listed once (walking the module tree per token cost
        ~0.2 ms of host time before each step); each call reads the slots
        again, so a parameter assigned anew is seen.  Submodules replaced
        after the first cached call need reset_cache()."""
        if self._param_slots is None:
            self._param_slots = [(m, name) for owner in (self.backbone, self.norm)
                                 for m in owner.modules()
                                 for name, prm in m._parameters.items() if prm is not None]
        params = [m._parameters.get(name) for m, name in self._param_slots]
        params += (self.embedding_weight, self.lm_head_weight)
        return self.backbone.training, tuple(None if p is None else (p.data_ptr(), p._version)
                                             for p in params)

    @torch.no_grad()
    def forward_inference(self, tokens: torch.Tensor, doc_spans: Optional[List[Any]] = None,
                          **kwargs) -> torch.Tensor:
        """model/model.py:214-237: logits [1, T, V] over the whole sequence."""
        block_mask = self.block_mask_creator(tokens=tokens, doc_spans=doc_spans or [], **kwargs)
        x = F.embedding(tokens, self.embedding_weight)
        x = self.backbone(x, block_mask=block_mask)
        x = self.norm(x)
        return F.linear(x, self.lm_head_weight)

    # -- cached path -------------------------------------------------------

    def _layers(self):
        return self.backbone.layers

    def _new_cache(self, words: int, device) -> KVCache:
        attn = self._layers()[0].attn
        return KVCache(len(self._layers()), attn.num_heads, attn.head_dim,
                       self._layers()[0].attn.rotary.max_seq_len, words, device,
                       self.embedding_weight.dtype)

    @torch.no_grad()
    def forward_inference_last(self, tokens: torch.Tensor,
                               doc_spans: Optional[List[Any]] = None, **kwargs) -> torch.Tensor:
        """Logits [1, 1, V] of the last position of ``tokens`` [1, T]; equal
        (to bf16 rounding) to ``forward_inference(tokens, doc_spans)[:, -1:]``."""
        if tokens.shape[0] != 1:
            raise ValueError("the cached path serves one sequence (batch 1)")
        if self.embedding_weight.dtype != torch.bfloat16:
            # The key/value cache and the decode kernel are bf16; a float32
            # model recomputes the sequence on the float32 attention kernels.
            return self.forward_inference(tokens, doc_spans, **kwargs)[:, -1:]
        # Per-token mask inputs only; the tile tables are built below if the
        # whole sequence has to be recomputed.
        bm = self.block_mask_creator(tokens=tokens, doc_spans=doc_spans or [], inputs_only=True,
                                     **kwargs)
        T = tokens.shape[1]
        state = self._weights_state()
        if state != self._weights_seen:
            self.reset_cache()
            self._weights_seen = state
        cache = self.kv_cache
        if cache is None or cache.words != bm.words or T > cache.capacity:
            cache = self.kv_cache = self._new_cache(bm.words, tokens.device)
            self._graph = None
        p = T - 1
        if self.use_graphs and p >= 1 and cache.length >= p:
            # The generation case: the cached prefix covers every position but
            # the last.  Launch the single-row step at once and check the
            # prefix on the device beside it; the check is read back after the
            # step's launches, so the step costs one host synchronisation.
            cache.store_inputs(tokens, bm, p, T)
            logits = self._graph_step(cache, tokens, bm, p)
            first = cache.first_diff(tokens, bm, p)  # reads positions < p only
            if int(first.item()) == p:
                cache.length = T
                return logits
            # an earlier input changed: recompute from the first difference
            cache.length = int(first.item())
        p0 = min(cache.reusable_prefix(tokens, bm), T - 1)
        full = T - p0 > self.prefill_rows
        if full:
            p0 = 0
            if not isinstance(bm, T2TBlockMask):
                bm = build_block_mask(bm.doc_ids, bm.q_bits, bm.kv_bits)
        cache.length = p0  # positions >= p0 are rewritten below
        cache.store_inputs(tokens, bm, p0, T)
        if self.use_graphs and not full and T - p0 == 1:
            logits = self._graph_step(cache, tokens, bm, p0)
            cache.length = T
            return logits
        x = F.embedding(tokens[:, p0:], self.embedding_weight)
        x = self._backbone_rows(x, bm, cache, p0, full)
        cache.length = T
        x = x[:, -1:]
        if self._rows_fusable(x):
            return rows_linear(x, self.lm_head_weight, norm=self.norm)
        return F.linear(self.norm(x), self.lm_head_weight)

    def _graph_step(self, cache: KVCache, tokens: torch.Tensor, bm, p: int) -> torch.Tensor:
        """One new row at position p through the captured decode step."""
        if (self._graph is None or self._graph.cache is not cache
                or self._graph.fused != self.fuse_rows):
            self._graph = _DecodeGraph(self, cache)
        return self._graph.run(p)

    def _step_body(self, cache: KVCache, buf: "_DecodeGraph") -> torch.Tensor:
        """The single-row step over static buffers (no host values in any
        launch): embedding, every layer with its cache write and decode
        attention over the whole cache capacity (slots past the new row are
        excluded by the causal test), final norm and LM head."""
        # The new row's token id and mask inputs, written into the cache at
        # position pos before every replay, are gathered inside the graph.
        tok = cache.tokens.index_select(1, buf.pos)
        qdoc = cache.doc.index_select(1, buf.pos)
        qbits = cache.q_bits.index_select(2, buf.pos) if cache.words else None
        qpos = buf.pos.to(torch.int32).view(1, 1)
        x = F.embedding(tok, self.embedding_weight)
        cos_t, sin_t = self._layers()[0].attn.rotary.tables(x.device)
        fused = self._rows_fusable(x)
        if not fused:
            cos = cos_t.index_select(0, buf.pos)
            sin = sin_t.index_select(0, buf.pos)
        bb = self.backbone
        skips = []
        n_skip = len(bb.skip_weights)
        carried = False  # this layer's skip add was folded into the previous layer
        for i, layer in enumerate(bb.layers):
            if i >= n_skip and skips and not carried:
                x = x + bb.skip_weights[i - n_skip] * skips.pop()
            attn = layer.attn
            C = x.shape[-1]
            nxt = self._next_skip(i, skips) if fused else None
            if fused:
                q = rows_qkv_rope(x, attn.qkv.weight, attn.num_heads, cos_t, sin_t, buf.pos,
                                  cache.k[i], cache.v[i], norm=layer.ln_1)
            else:
                q, k, v = qkv_rope(attn.qkv(layer.ln_1(x)), cos, sin, attn.num_heads, 0)
                cache.k[i].index_copy_(2, buf.pos, k)
                cache.v[i].index_copy_(2, buf.pos, v)
            y, _ = attn_decode(q, cache.k[i], cache.v[i], cache.capacity, cache.doc,
                               cache.kv_bits if cache.words else None, qpos, qdoc, qbits)
            x = self._layer_tail(layer, y.transpose(1, 2).reshape(1, 1, C), x, fused, nxt)
            carried = nxt is not None
            if i < n_skip and not carried:
                skips.append(x)
        if fused:
            return rows_linear(x, self.lm_head_weight, norm=self.norm)
        return F.linear(self.norm(x), self.lm_head_weight)

    def _rows_fusable(self, x) -> bool:
        """Whether the layers of a few-row step can run on the fused row
        kernels (rows.py): bf16 rows and weights on the GPU, at most 8 rows,
        SwiGLU GLUs, and dropout / drop-path that are the identity."""
        if (not self.fuse_rows or not rows_apply(x, self.lm_head_weight)
                or not self.lm_head_weight.is_contiguous()):
            return False
        for layer in self._layers():
            mlp = layer.mlp
            if (mlp.act is not F.silu or not isinstance(layer.ln_1, RMSNorm)
                    or not isinstance(layer.ln_2, RMSNorm)):
                return False
            if layer.training and (layer.drop_path.p > 0 or mlp.dropout.p > 0):
                return False
            ws = (layer.attn.qkv.weight, layer.attn.proj.weight, mlp.gate_up.weight,
                  mlp.down.weight)
            if not all(w.dtype == torch.bfloat16 and w.is_contiguous() for w in ws):
                return False
            if mlp.down.weight.shape[1] > 4096:
                return False
        return isinstance(self.norm, RMSNorm)

    def _next_skip(self, i: int, skips: list):
        """The skip add that starts layer i + 1 (model/modules/backbone.py:93-104:
        x + skip_weights[j - n_skip] * skips.pop() for layers j >= n_skip),
        to be folded into layer i's down-projection: (rows, weight), rows None
        when layer i + 1 pops layer i's own output; None when layer i + 1 adds
        nothing."""
        bb = self.backbone
        n_skip, j = len(bb.skip_weights), i + 1
        if j >= len(bb.layers) or j < n_skip:
            return None
        if i == n_skip - 1:
            return None, bb.skip_weights[0]
        if not skips:
            return None
        return skips.pop(), bb.skip_weights[j - n_skip]

    @staticmethod
    def _layer_tail(layer, y, x, fused: bool, skip=None):
        """Out-projection + residual, norm + GLU + residual of Layer.forward
        (model/modules/layer.py:33-34) on the attention rows y; ``skip``: the
        next layer's skip add, folded into the last product (fused only)."""
        if fused:
            mlp = layer.mlp
            x = rows_linear(y, layer.attn.proj.weight, epilogue="add", res=x)
            h = rows_linear(x, mlp.gate_up.weight, norm=layer.ln_2, epilogue="swiglu")
            return rows_linear(h, mlp.down.weight, epilogue="add", res=x, skip=skip)
        x = x + layer.drop_path(layer.attn.proj(y))
        return x + layer.drop_path(layer.mlp(layer.ln_2(x)))

    def _backbone_rows(self, x, bm, cache: KVCache, p0: int, full: bool):
        """TS2TSBackbone.forward (skip wiring of model/modules/backbone.py:93-104)
        over rows p0 .. T - 1 with cached attention."""
        bb = self.backbone
        skips = []
        n_skip = len(bb.skip_weights)
        fused = not full and self._rows_fusable(x)
        carried = False  # this layer's skip add was folded into the previous layer
        for i, layer in enumerate(bb.layers):
            if i >= n_skip and skips and not carried:
                x = x + bb.skip_weights[i - n_skip] * skips.pop()
            nxt = self._next_skip(i, skips) if fused else None
            x = self._layer_rows(i, layer, x, bm, cache, p0, full, fused, nxt)
            carried = nxt is not None
            if i < n_skip and not carried:
                skips.append(x)
        return x

    def _layer_rows(self, i: int, layer, x, bm, cache: KVCache, p0: int, full: bool,
                    fused: bool, skip=None):
        """Layer.forward (model/modules/layer.py:32-35) over the new rows."""
        attn = layer.attn
        B, n, C = x.shape
        T = p0 + n
        cos, sin = attn.rotary.tables(x.device)
        if fused:
            q = rows_qkv_rope(x, attn.qkv.weight, attn.num_heads, cos, sin, p0, cache.k[i],
                              cache.v[i], norm=layer.ln_1)
        else:
            q, k, v = qkv_rope(attn.qkv(layer.ln_1(x)), cos, sin, attn.num_heads, p0)
            cache.k[i, :, :, p0:T] = k
            cache.v[i, :, :, p0:T] = v
        if full:
            y = flex_attention(q, k, v, block_mask=bm)
        else:
            y = torch.empty_like(q)
            rows = MAX_ROWS  # one query head per kv head in this model
            pos = torch.arange(p0, T, dtype=torch.int32, device=x.device)[None]
            for c0 in range(0, n, rows):
                c1 = min(n, c0 + rows)
                qb = bm.q_bits[:, :, p0 + c0:p0 + c1].contiguous() if bm.words else None
                attn_decode(q[:, :, c0:c1], cache.k[i], cache.v[i], p0 + c1, cache.doc,
                            cache.kv_bits if bm.words else None, pos[:, c0:c1].contiguous(),
                            bm.doc_ids[:, p0 + c0:p0 + c1].contiguous(), qb,
                            out=y[:, :, c0:c1])
        return self._layer_tail(layer, y.transpose(1, 2).reshape(B, n, C), x, fused, skip)


class _DecodeGraph:
    """The single-row decode step of a TS2TSModel captured as a HIP graph
    (torch.cuda.graph) over one static buffer, the row's position: the step
    gathers the row's token id and mask inputs from the cache, where
    ``store_inputs`` has written them before the replay.  Replays cost two
    launches from the host (the position and the graph) instead of the
    launches of the eager step (six per layer on the fused row kernels, ~15
    without them); the recorded kernels (the row kernels and the decode
    kernels, or hipBLASLt GEMMs, torch elementwise / reduction kernels and
    the prologue kernel) write no memset nodes of their own."""

    def __init__(self, model: TS2TSModel, cache: KVCache):
        self.cache = cache
        self.pos = torch.zeros((1,), dtype=torch.int64, device=cache.k.device)
        self.model = model
        self.fused = model.fuse_rows
        self.graph = None
        self.logits = None

    def _capture(self):
        """Warm up on a side stream (default priority), then capture.  The
        buffers already hold the first step's values, so the warm-up run writes
        exactly what the first replay writes."""
        dev = self.pos.device
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            self.model._step_body(self.cache, self)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = self.model._step_body(self.cache, self)

    def run(self, p: int) -> torch.Tensor:
        """Logits of the row at position p, whose inputs are in the cache."""
        self.pos.fill_(p)
        if self.graph is None:
            self._capture()
        self.graph.replay()
        return self.logits.clone()

