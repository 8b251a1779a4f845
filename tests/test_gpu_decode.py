"""GPU parity of the decode step (t2t_attn_decode) and of the cached
generation forward built on it.

Kernel: the rows of the float64 oracle attention (oracle/attn_oracle.py, the
restatement of torch's math attention under the reference mask_mod) at the
new rows' positions, bf16 tolerance 2e-2 abs+rel on o and 1e-3 on the LSE;
GQA, per-row masks, grant words, uncovered tokens, ragged key counts, cache
slots past the filled length holding NaN (never read), fully masked rows.
Model: TS2TSModel.forward_inference_last against the last row of the full
recompute forward_inference (the reference's per-token path) while tokens are
appended one and several at a time, after an early token changes, and under a
cross-document link mask.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attn_oracle as ao
from oracle import mask_oracle as mo
from tagseq2tagseq_amd import synth
from tagseq2tagseq_amd.decode import attn_decode
from tagseq2tagseq_amd.mask_creators import (create_doc_causal_block_mask,
                                             create_doc_link_block_mask)
from tagseq2tagseq_amd.model import TS2TSModel
from tests.helpers import assert_close, random_row, to_dev_words

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
LOG2E = 1.0 / math.log(2.0)


def _decode_case(rows_np, B, Hq, Hkv, T, D, Tq, cap, seed, positions=None):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, T, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    pos = np.arange(T - Tq, T) if positions is None else np.asarray(positions)
    # caches with NaN past the filled length
    kc = torch.full((B, Hkv, cap, D), float("nan"), dtype=torch.bfloat16)
    vc = torch.full((B, Hkv, cap, D), float("nan"), dtype=torch.bfloat16)
    kc[:, :, :T] = k
    vc[:, :, :T] = v
    Bm = len(rows_np)
    W = 0 if rows_np[0][1] is None else rows_np[0][1].shape[0]
    key_doc = torch.full((Bm, cap), -7, dtype=torch.int32)
    key_doc[:, :T] = torch.from_numpy(np.stack([r[0] for r in rows_np]))
    key_bits = q_bits = None
    if W:
        key_bits = torch.zeros((Bm, W, cap), dtype=torch.int64)
        key_bits[:, :, :T] = torch.stack([to_dev_words(r[2], "cpu") for r in rows_np])
        q_bits = torch.stack([to_dev_words(r[1][:, pos], "cpu") for r in rows_np])
    q_doc = torch.from_numpy(np.stack([r[0][pos] for r in rows_np])).int()
    q_pos = torch.from_numpy(np.tile(pos.astype(np.int32), (Bm, 1)))
    dev = lambda t: None if t is None else t.to(DEV).contiguous()
    o, lse2 = attn_decode(dev(q[:, :, pos]), dev(kc), dev(vc), T, dev(key_doc), dev(key_bits),
                          dev(q_pos), dev(q_doc), dev(q_bits))
    dense = np.stack([mo.dense_mask(*r) for r in rows_np])
    o_ref, lse_ref = ao.attention_fwd(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                      dense)
    label = f"B{B} H{Hq}/{Hkv} T{T} D{D} Tq{Tq}"
    assert_close(o, torch.from_numpy(o_ref[:, :, pos]), 2e-2, 2e-2, f"o {label}")
    assert_close(lse2, torch.from_numpy(lse_ref[:, :, pos] * LOG2E), 1e-3, 1e-3, f"lse {label}")
    return o, lse2


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("T", [1, 200, 1000, 4099])
def test_single_row_doc_causal(T, D):
    rows = [random_row(T, np.random.default_rng(T + D), max_doc=600)]
    _decode_case(rows, 1, 2, 2, T, D, 1, T + 37, seed=T)


@pytest.mark.parametrize("D", [64, 128])
def test_gqa_rows_words_and_batch_masks(D):
    """R = (Hq / Hkv) * Tq = 8 rows per kv head; per-row masks with 2 words."""
    rng = np.random.default_rng(21)
    T = 777
    rows = [random_row(T, rng, words=2, uncovered=True, max_doc=150) for _ in range(2)]
    _decode_case(rows, 2, 8, 2, T, D, 2, 1024, seed=3)


def test_rows_at_arbitrary_positions():
    rng = np.random.default_rng(5)
    T = 600
    rows = [random_row(T, rng, words=1, max_doc=100)]
    _decode_case(rows, 1, 4, 4, T, 128, 2, 640, seed=4, positions=[17, 402])


def test_cross_doc_link_rows():
    row = synth.config_rows(3, seed=1, T=2048)[0]
    doc = mo.document_ids(2048, row.spans)
    qb, kb = mo.doc_link_token_bits(row.doc_index, row.link_rows)
    _decode_case([(doc, qb, kb)], 1, 4, 4, 2048, 128, 2, 2048, seed=6)


def test_fully_masked_row():
    T, D = 300, 64
    kc = torch.randn(1, 1, T, D, device=DEV).to(torch.bfloat16)
    key_doc = torch.zeros(1, T, dtype=torch.int32, device=DEV)
    q = torch.randn(1, 1, 1, D, device=DEV).to(torch.bfloat16)
    o, lse2 = attn_decode(q, kc, kc, T, key_doc, None,
                          torch.tensor([[T - 1]], dtype=torch.int32, device=DEV),
                          torch.tensor([[5]], dtype=torch.int32, device=DEV), None)
    assert torch.equal(o.float(), torch.zeros_like(o.float()))
    assert torch.isneginf(lse2).all()


def test_too_many_rows_raises():
    q = torch.zeros(1, 4, 3, 64, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(1, 1, 16, 64, dtype=torch.bfloat16, device=DEV)
    i32 = torch.zeros(1, 16, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="exceeds"):
        attn_decode(q, kc, kc, 16, i32, None, i32[:, :3].contiguous(), i32[:, :3].contiguous(),
                    None)


# -- cached model path ------------------------------------------------------

def _distinct_skip_weights(m):
    """Skip weights 0.5, 1.5, 0.75, ... instead of the all-ones init, so that a
    skip add that takes the wrong weight or the wrong popped row changes the
    logits (model/modules/backbone.py:93-104)."""
    vals = [0.5, 1.5, 0.75, 1.25, 0.625, 1.375]
    with torch.no_grad():
        sw = m.backbone.skip_weights
        sw.copy_(torch.tensor(vals[:sw.numel()], dtype=sw.dtype))


def _model(creator, T_max=1024, num_layers=4):
    # model_dim 384: GLU hidden width 1024, a multiple of 8, so the row
    # kernels read every operand in 16-byte vectors
    torch.manual_seed(0)
    m = TS2TSModel.from_config(vocab_size=500, num_layers=num_layers, model_dim=384, num_heads=6,
                               max_seq_len=T_max, dropout=0.0, drop_path_rate=0.0,
                               block_mask_creator=creator)
    with torch.no_grad():
        m.embedding_weight.mul_(0.05)  # keeps logits in a range where bf16 rounding is small
    _distinct_skip_weights(m)
    return m.to(DEV, torch.bfloat16).eval()


def _check_last(m, tokens, spans, what, **kw):
    got = m.forward_inference_last(tokens, spans, **kw).float()
    ref = m.forward_inference(tokens, spans, **kw)[:, -1:].float()
    scale = ref.abs().max().item()
    err = (got - ref).abs().max().item()
    assert err <= 2e-2 * scale + 1e-3, f"{what}: max err {err:.4g} (logit scale {scale:.3g})"


def _grow(spans, n):
    """Extend the last document by n tokens."""
    last = spans[-1]
    return spans[:-1] + [synth.DocSpan(doc_id=last.doc_id, start=last.start, end=last.end + n)]


@pytest.mark.parametrize("graphs,layers", [(True, 4), (False, 4), (True, 5)])
def test_cached_generation_matches_full_recompute(graphs, layers):
    """Single-row steps run through the captured HIP graph (graphs=True, replayed
    with eager work and host synchronisation between replays) or eagerly; five
    layers leave the last layer with no skip row to pop."""
    m = _model(create_doc_causal_block_mask, num_layers=layers)
    m.use_graphs = graphs
    g = torch.Generator().manual_seed(1)
    vocab = torch.randint(0, 500, (1, 1024), generator=g).to(DEV)
    spans = [synth.DocSpan(doc_id=7, start=0, end=120), synth.DocSpan(doc_id=3, start=120, end=300)]
    T = 300
    _check_last(m, vocab[:, :T], spans, "prefill")
    assert m.kv_cache.length == T
    for step in range(8):  # one token at a time: decode path
        spans = _grow(spans, 1)
        T += 1
        _check_last(m, vocab[:, :T], spans, f"decode step {step}")
    # one token appended while an earlier one changed: the single-row step
    # launched at once is discarded and the rows from the change recomputed
    spans = _grow(spans, 1)
    T += 1
    tok = vocab[:, :T].clone()
    tok[0, T - 10] = (tok[0, T - 10] + 7) % 500
    _check_last(m, tok, spans, "appended + changed")
    spans = _grow(spans, 5)  # five new rows at once
    T += 5
    _check_last(m, vocab[:, :T], spans, "5-row step")
    # an earlier token changes: rows from there on are recomputed (40 rows, decode chunks)
    tok = vocab[:, :T].clone()
    tok[0, T - 40] = (tok[0, T - 40] + 1) % 500
    _check_last(m, tok, spans, "changed token")
    # a new document appended after the generated one
    spans2 = spans + [synth.DocSpan(doc_id=11, start=T, end=T + 3)]
    _check_last(m, torch.cat([tok, vocab[:, T:T + 3]], 1), spans2, "new doc")


def test_float32_model_inference(monkeypatch):
    """A model left in float32 (the cache and decode kernel are bf16): the
    last-row call recomputes on the float32 attention kernels and equals
    forward_inference's last row; forward_inference itself matches the same
    model with dense float32 masked attention within 1e-4."""
    import math
    import tagseq2tagseq_amd.attention as attn_mod
    from tests.helpers import dense_mask_torch
    torch.manual_seed(0)
    m = TS2TSModel.from_config(vocab_size=500, num_layers=2, model_dim=256, num_heads=4,
                               max_seq_len=512, dropout=0.0, drop_path_rate=0.0,
                               block_mask_creator=create_doc_causal_block_mask).to(DEV).eval()
    g = torch.Generator().manual_seed(2)
    tokens = torch.randint(0, 500, (1, 300), generator=g).to(DEV)
    spans = [synth.DocSpan(doc_id=7, start=0, end=120), synth.DocSpan(doc_id=3, start=120, end=300)]
    full = m.forward_inference(tokens, spans)
    assert full.dtype == torch.float32
    assert torch.equal(m.forward_inference_last(tokens, spans), full[:, -1:])

    def dense(q, k, v, block_mask=None, **kw):
        T = q.shape[2]
        msk = dense_mask_torch(block_mask.doc_ids[0], None, None, 0, T)
        sc = (q @ k.transpose(-1, -2)) / math.sqrt(q.shape[-1])
        return torch.softmax(sc.masked_fill(~msk, float("-inf")), -1).nan_to_num(0.0) @ v

    monkeypatch.setattr(attn_mod, "flex_attention", dense)
    ref = m.forward_inference(tokens, spans)
    err = (full - ref).abs().max().item()
    assert err <= 1e-4 * ref.abs().max().item() + 1e-5, f"float32 logits: max err {err:.3g}"


@pytest.mark.parametrize("graphs", [True, False])
def test_cached_generation_cross_doc_links(graphs):
    m = _model(create_doc_link_block_mask)
    m.use_graphs = graphs
    g = torch.Generator().manual_seed(2)
    vocab = torch.randint(0, 500, (1, 1024), generator=g).to(DEV)
    spans = [synth.DocSpan(doc_id=i, start=100 * i, end=100 * i + 100) for i in range(4)]
    links = np.zeros((4, 1), dtype=np.uint64)
    for i in range(4):
        links[i, 0] |= np.uint64(1) << np.uint64(i)
    links[3, 0] |= np.uint64(1 << 1)
    T = 400
    _check_last(m, vocab[:, :T], spans, "prefill", doc_links=links)
    for step in range(3):
        spans = _grow(spans, 1)
        T += 1
        _check_last(m, vocab[:, :T], spans, f"decode {step}", doc_links=links)
    links2 = links.copy()
    links2[3, 0] |= np.uint64(1)  # the generated doc gains a link: its rows change
    _check_last(m, vocab[:, :T], spans, "link added", doc_links=links2)


@pytest.mark.parametrize("graphs", [True, False])
@pytest.mark.parametrize("dim,heads,layers", [(384, 6, 4), (256, 4, 4), (384, 6, 5)])
def test_fused_row_kernels_match_unfused_layers(graphs, dim, heads, layers, monkeypatch):
    """Decode steps on the fused row kernels (norm + qkv + rotation + cache
    write, out-projection + residual, norm + gate_up + SwiGLU, down +
    residual, norm + LM head) against the same steps through the unfused torch
    layer sequence, one and five rows at a time.  dim 256 has a GLU hidden
    width of 682, not a multiple of 8: its down-projection reads its rows
    element by element instead of in 16-byte vectors."""
    import tagseq2tagseq_amd.model as model_mod
    calls = []
    real = model_mod.rows_linear
    monkeypatch.setattr(model_mod, "rows_linear",
                        lambda *a, **kw: calls.append(1) or real(*a, **kw))
    torch.manual_seed(0)
    m = TS2TSModel.from_config(vocab_size=500, num_layers=layers, model_dim=dim, num_heads=heads,
                               max_seq_len=1024, dropout=0.0, drop_path_rate=0.0,
                               block_mask_creator=create_doc_causal_block_mask)
    with torch.no_grad():
        m.embedding_weight.mul_(0.05)
    _distinct_skip_weights(m)
    m = m.to(DEV, torch.bfloat16).eval()
    m.use_graphs = graphs
    g = torch.Generator().manual_seed(3)
    vocab = torch.randint(0, 500, (1, 1024), generator=g).to(DEV)
    spans = [synth.DocSpan(doc_id=1, start=0, end=200)]
    T = 200
    m.forward_inference_last(vocab[:, :T], spans)
    for n in (1, 1, 5, 1):
        spans = _grow(spans, n)
        T += n
        m.fuse_rows = True
        fused = m.forward_inference_last(vocab[:, :T], spans).float()
        m.fuse_rows = False
        m.kv_cache.length = T - n  # recompute the same rows unfused
        m.kv_cache.tokens[0, T - n:T] = -1
        plain = m.forward_inference_last(vocab[:, :T], spans).float()
        scale = plain.abs().max().item()
        err = (fused - plain).abs().max().item()
        assert err <= 2e-2 * scale + 1e-3, f"{n} rows: max err {err:.4g} (scale {scale:.3g})"
    assert calls, "the fused row kernels did not run"


@pytest.mark.parametrize("graphs", [True, False])
def test_cache_dropped_when_weights_change(graphs):
    """The cached keys / values and the captured step are rebuilt after an
    in-place weight edit, load_state_dict, an optimizer step, a train() /
    eval() switch and a parameter assigned anew: each following call equals the full recompute under the
    new weights (the reference recomputes every call, model/model.py:214-237)."""
    m = _model(create_doc_causal_block_mask)
    m.use_graphs = graphs
    g = torch.Generator().manual_seed(4)
    vocab = torch.randint(0, 500, (1, 1024), generator=g).to(DEV)
    spans = [synth.DocSpan(doc_id=2, start=0, end=250)]
    T = 250
    _check_last(m, vocab[:, :T], spans, "prefill")

    def step(what):
        nonlocal spans, T
        spans = _grow(spans, 1)
        T += 1
        _check_last(m, vocab[:, :T], spans, what)

    step("decode")  # the single-row step exists now (captured when graphs=True)
    with torch.no_grad():
        m.backbone.layers[1].attn.qkv.weight.mul_(1.5)
    step("after an in-place edit")
    sd = {k: v * 0.9 for k, v in m.backbone.state_dict().items()}
    m.backbone.load_state_dict(sd)
    step("after load_state_dict")
    opt = torch.optim.SGD(m.backbone.parameters(), lr=1.0)
    for p_ in m.backbone.parameters():
        p_.grad = torch.full_like(p_, 1e-3)
    opt.step()
    step("after an optimizer step")
    m.train()
    m.eval()
    step("after train() / eval()")
    down = m.backbone.layers[0].mlp.down
    down.weight = torch.nn.Parameter(down.weight.detach() * 1.1)
    step("after a parameter is assigned anew")


@pytest.mark.parametrize("words", [0, 1, 3])
def test_first_input_diff_kernel(words):
    """t2t_first_input_diff (the cache check) against numpy: the first position
    whose token id, doc id or any q / kv word differs, or n; a difference
    planted in each array in turn, at positions across the work-group's
    steps, n = 0 and n not a multiple of the group size; bits rows with a
    stride above n."""
    from tagseq2tagseq_amd.model import KVCache
    rng = np.random.default_rng(words)
    cap, n_tot = 9000, 8195
    cache = KVCache(1, 1, 64, cap, words, DEV)
    tok = rng.integers(0, 500, (1, n_tot))
    doc = rng.integers(0, 9, (1, n_tot)).astype(np.int32)
    qb = rng.integers(0, 2 ** 62, (1, words, n_tot))
    kb = rng.integers(0, 2 ** 62, (1, words, n_tot))

    class Inputs:
        pass

    cache.tokens[0, :n_tot] = torch.from_numpy(tok[0]).to(DEV)
    cache.doc[0, :n_tot] = torch.from_numpy(doc[0]).to(DEV)
    if words:
        cache.q_bits[0, :, :n_tot] = torch.from_numpy(qb[0]).to(DEV)
        cache.kv_bits[0, :, :n_tot] = torch.from_numpy(kb[0]).to(DEV)
    arrays = ["tok", "doc"] + (["q", "kv"] if words else [])
    cases = [(None, None)] + [(a, p) for a in arrays for p in (0, 1023, 1024, 4097, 8194)]
    for which, p in cases:
        t2, d2, q2, k2 = tok.copy(), doc.copy(), qb.copy(), kb.copy()
        if which == "tok":
            t2[0, p] += 1
        elif which == "doc":
            d2[0, p] += 1
        elif which == "q":
            q2[0, words - 1, p] ^= 1 << 40
        elif which == "kv":
            k2[0, 0, p] ^= 1
        bm = Inputs()
        bm.doc_ids = torch.from_numpy(d2).to(DEV)
        bm.q_bits = torch.from_numpy(q2).to(DEV)
        bm.kv_bits = torch.from_numpy(k2).to(DEV)
        toks = torch.from_numpy(t2).to(DEV)
        for n in (n_tot, 4096, 1, 0):
            want = p if p is not None and p < n else n
            got = int(cache.first_diff(toks, bm, n).item())
            assert got == want, f"{which} at {p}, n={n}: got {got}, want {want}"
