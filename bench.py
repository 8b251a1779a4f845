"""Benchmark of the gfx950 masked-attention hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3]

One step = one pass of the hot path over one batch: the per-token mask
inputs rebuilt from the device-resident span / link lists (t2t_token_inputs),
the metadata pass (tile classification + BlockMask tables), the forward
kernel and the three backward launches, with every input already resident in
HBM.  Prints one JSON line.

metric  : BASELINE.json's "masked attn fwd+bwd useful TFLOP/s", quoted on
          configs[2] (cross_doc_link, B1 H16 T16384 D128, bf16) by default.
useful FLOPs per step = 14 * D * N_pairs * Hq (fwd 4, bwd 10: the FA2
          convention), N_pairs = exact number of allowed (b, q, kv) pairs.
roofline: the dominant kernel's algorithmic FLOPs per launch / its mean
          duration (HIP events on the launch stream) vs the MI355X dense bf16
          MFMA peak.
cpu_baseline: the reference's CPU path -- torch eager flex_attention +
          create_block_mask with the reference's mask_mod -- on a bounded
          sample (one head), scaled to the whole step.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from tagseq2tagseq_amd import synth  # noqa: E402
from tagseq2tagseq_amd.attention import BwdPhases, attn_bwd, attn_fwd  # noqa: E402
from tagseq2tagseq_amd.block_mask import build_block_mask  # noqa: E402
from tagseq2tagseq_amd.mask_creators import TokenLists  # noqa: E402

METRIC = "masked attn fwd+bwd useful TFLOP/s + % bf16 MFMA peak, cross_doc_link T=16k"
PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA: 256 CU x 2.4 GHz x 4096 FLOP/clk
PEAK_HBM_GBS = 8000.0
PEAK_F32_TFLOPS = 157.3     # MI355X dense fp32 MFMA

WORKLOAD_NAMES = {
    2: "doc_causal fwd+bwd bf16 B2 H12 T8192 D64 (configs[1])",
    3: "cross_doc_link fwd+bwd bf16 B1 H16 T16384 D128 (configs[2])",
    4: "cross_doc_link GQA fwd+bwd bf16 B1 Hq16/Hkv4 T32768 D128 (configs[3])",
}


def per_token_arrays(row: synth.SynthRow):
    """doc ids (span ids) and grant words of one synthetic row, host numpy."""
    from tagseq2tagseq_amd.mask_creators import document_ids_host
    T = row.seq_len
    doc = document_ids_host(T, row.spans)
    if row.link_rows is None:
        return doc, None, None
    W = row.link_rows.shape[1]
    qb = np.zeros((W, T), dtype=np.uint64)
    kb = np.zeros((W, T), dtype=np.uint64)
    cov = row.doc_index >= 0
    d = row.doc_index[cov].astype(np.int64)
    qb[:, cov] = row.link_rows[d].T
    kb[d // 64, np.nonzero(cov)[0]] = np.uint64(1) << (d % 64).astype(np.uint64)
    return doc, qb, kb


def count_pairs(doc, qb, kb, chunk=1024) -> int:
    """Exact allowed-pair count of one mask row, on the GPU (chunked rows)."""
    T = doc.shape[0]
    total = 0
    kv = torch.arange(T, device=doc.device)[None, :]
    for r0 in range(0, T, chunk):
        r1 = min(T, r0 + chunk)
        m = doc[r0:r1, None] == doc[None, :]
        if qb is not None:
            for w in range(qb.shape[0]):
                m |= (qb[w, r0:r1, None] & kb[w][None, :]) != 0
        m &= torch.arange(r0, r1, device=doc.device)[:, None] >= kv
        total += int(m.sum().item())
    return total


def measured_traffic(config: int, kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 summary
    (profiles/hbm_traffic_config<N>.txt: FETCH_SIZE / WRITE_SIZE passes scaled
    by the copy calibration), or None when no summary exists."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_config{config}.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith(kernel + ":"):
                for tok in line.split():
                    if tok.startswith("traffic_bytes="):
                        return int(tok.split("=", 1)[1])
    return None


def profile_mfma_busy(config: int):
    """MFMA-busy fraction per kernel from the committed instruction-mix summary
    (profiles/instruction_mix_config<N>.txt: SQ_VALU_MFMA_BUSY_CYCLES over the
    chip's SIMD-cycles in the kernel's duration, from rocprofv3 runs of this
    bench), or None when no summary exists."""
    from tagseq2tagseq_amd.rocprof_summary import read_mfma_busy
    path = os.path.join(ROOT, "profiles", f"instruction_mix_config{config}.txt")
    got = read_mfma_busy(path)
    return {"source": os.path.relpath(path, ROOT), **got} if got else None


def dkdv_kernel_name(D: int) -> str:
    """The dK/dV kernel t2t_attn_bwd runs at head dim D (the pair-split,
    two-work-groups-per-CU kernel at D = 64)."""
    return "bwd_dkdv_pair_kernel" if D == 64 else "bwd_dkdv_kernel"


def fwd_step_keys(D: int) -> int:
    """Keys per step of the bf16 forward kernel at head dim D (64-key halves
    at D = 64, 32-key quarters at D = 128; launch_attn_fwd_bf16)."""
    return 64 if D == 64 else 32


def executed_work(bm, B: int, Hq: int, D: int, n_pairs: int, config: int):
    """MFMA work the attention kernels execute for one step, counted from the
    block mask, against the useful work of the metric.

    The kernels compute whole MFMA blocks: the forward a 32-query x SK-key
    step of a non-skip tile (SK = fwd_step_keys(D)) when any pair in it is
    allowed (SK D / 256 MFMAs: the scores and P V), dK/dV and dQ a 32 x 32
    block when any pair in it is allowed (D / 4 MFMAs: S, dP, dV, dK;
    3 D / 16: S, dP, dQ).  An MFMA
    (32 x 32 x 16) is 32768 FLOP.  Useful work is 4 D (forward), 8 D (dK/dV,
    which recomputes S and dP) and 6 D (dQ, the same recompute) FLOP per
    allowed pair, and 14 D per pair for the step (the metric's convention,
    S and dP once).  `busy_needed_for_50pct`: the share of the chip's MFMA
    cycles (at the 2.4 GHz of the published peak) the executed work would
    have to fill for the step to reach 50 % of peak on useful FLOPs, were
    the step nothing but these three kernels.  `profile_mfma` repeats the
    per-dispatch MFMA counts of the committed instruction-mix summary, which
    come from the counters (SQ_INSTS_MFMA) of a profiled run of this bench."""
    dkdv = dkdv_kernel_name(D)
    tc = bm.tile_class
    Bm, nt = tc.shape[0], tc.shape[-1]
    rows_per_mask = B // Bm if Bm < B else 1
    n_full = int((tc == 2).sum())
    # row-major bitmaps of the partial tiles: [P, 128 queries, 4 words of 32 keys]
    b_, r_, c_ = (tc == 1).nonzero(as_tuple=True)
    slots = (bm.kv_bits_off[b_, r_].to(torch.int64) + c_.to(torch.int64))
    words = bm.tile_bits[slots, 0] != 0 if slots.numel() else torch.zeros(
        (0, 128, 4), dtype=torch.bool, device=tc.device)
    blocks32 = words.view(-1, 4, 32, 4).any(2)                        # [P, q blk, k blk]
    sk = fwd_step_keys(D)
    units_fwd = words.view(-1, 4, 32, 128 // sk, sk // 32).any(4).any(2)  # [P, q blk, k step]
    n_blk = (16 * n_full + int(blocks32.sum())) * rows_per_mask * Hq
    n_fwd = (4 * (128 // sk) * n_full + int(units_fwd.sum())) * rows_per_mask * Hq
    mf = {"attn_fwd_bf16_kernel": n_fwd * sk * D // 256,
          dkdv: n_blk * D // 4,
          "bwd_dq_kernel": n_blk * 3 * D // 16}
    useful = {"attn_fwd_bf16_kernel": 4.0, dkdv: 8.0, "bwd_dq_kernel": 6.0}
    out = {}
    executed = 0.0
    for k, n in mf.items():
        fl = 32768.0 * n
        executed += fl
        out[k] = {"mfma_per_launch": int(n), "executed_gflop": round(fl / 1e9, 2),
                  "executed_over_useful": round(fl / (useful[k] * D * n_pairs * Hq), 4)}
    step_useful = 14.0 * D * n_pairs * Hq
    out["step"] = {"executed_gflop": round(executed / 1e9, 2),
                   "useful_gflop": round(step_useful / 1e9, 2),
                   "executed_over_useful": round(executed / step_useful, 4),
                   "busy_needed_for_50pct": round(0.5 * executed / step_useful, 4),
                   "allowed_share_fwd_units": round(n_pairs * Hq / (32.0 * sk * n_fwd), 4),
                   "allowed_share_bwd_blocks": round(n_pairs * Hq / (1024.0 * n_blk), 4)}
    from tagseq2tagseq_amd.rocprof_summary import read_mfma_counts
    path = os.path.join(ROOT, "profiles", f"instruction_mix_config{config}.txt")
    prof = {k: v for k, v in read_mfma_counts(path).items() if k in mf}
    if prof:
        out["profile_mfma"] = {"source": os.path.relpath(path, ROOT), **prof}
    return out


def time_launches(fn, reps: int) -> float:
    """Mean duration (ms) of fn()'s launches, HIP events on the current stream."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / reps


def median_ms(fn, reps: int = 50, warmup: int = 10):
    """(median, min, max) duration in ms of fn() over `reps` calls after
    `warmup` discarded ones, each call bracketed by its own HIP events."""
    for _ in range(warmup):
        fn()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]
    torch.cuda.synchronize()
    for e0, e1 in evs:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    t = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
    return t[len(t) // 2], t[0], t[-1]


def engine_clock(dev, iters: int = 40000, reps: int = 5):
    """Engine clock (MHz) while every SIMD runs MFMA chains (t2t_clock_probe:
    shader cycles over wall-clock ticks of one wave), median of `reps`
    probes, and the bf16 MFMA peak at that clock (the published 2516.6
    TFLOP/s is the same product at 2400 MHz)."""
    import ctypes
    from tagseq2tagseq_amd import _lib
    L = _lib.lib()
    out = torch.zeros(2, dtype=torch.int64, device=dev)
    khz = ctypes.c_int32(0)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    mhz = []
    for _ in range(reps):
        _lib.check(L.t2t_clock_probe(ctypes.c_void_p(out.data_ptr()), iters, ctypes.byref(khz),
                                     stream), "t2t_clock_probe")
        cyc, ticks = (int(x) for x in out.tolist())
        mhz.append(cyc / ticks * khz.value / 1e3)
    mhz.sort()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    clk = mhz[len(mhz) // 2]
    return {"engine_mhz_under_mfma_load": round(clk, 1), "wall_clock_khz": khz.value,
            "probes_mhz": [round(m, 1) for m in mhz],
            "bf16_peak_at_clock_tflops": round(cus * 4096 * clk * 1e6 / 1e12, 1)}


def host_cores():
    """(CPUs this process may run on, CPUs the host reports)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return avail, os.cpu_count() or avail


def _median_spread(fn, reps: int):
    """One untimed warm-up call, then `reps` timed calls: (median, min, max) s."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], ts[0], ts[-1]


def cpu_baseline(rows_np, c, seed, threads, reps=5):
    """Reference CPU path on one head of batch row 0, each phase timed on its
    own (one warm-up, median of `reps`): create_block_mask with the reference's
    mask_mod (restated in oracle/mask_oracle.py), eager flex_attention forward,
    and forward + backward (torch/_higher_order_ops/flex_attention.py:202-294,
    825-994).  Returns the per-phase statistics and the scaled step time."""
    from oracle.mask_oracle import torch_mask_mod
    from torch.nn.attention.flex_attention import create_block_mask, flex_attention
    torch.set_num_threads(threads)
    T, D = c["T"], c["D"]
    doc, qb, kb = rows_np[0]
    mod = torch_mask_mod(torch.from_numpy(doc),
                         None if qb is None else torch.from_numpy(qb.view(np.int64)),
                         None if kb is None else torch.from_numpy(kb.view(np.int64)))
    bm = create_block_mask(mod, None, None, T, T, device="cpu")
    g = torch.Generator().manual_seed(seed)
    dt = torch.bfloat16
    q = torch.randn(1, 1, T, D, generator=g).to(dt).requires_grad_(True)
    k = torch.randn(1, 1, T, D, generator=g).to(dt).requires_grad_(True)
    v = torch.randn(1, 1, T, D, generator=g).to(dt).requires_grad_(True)
    do = torch.randn(1, 1, T, D, generator=g).to(dt)

    def fwd():
        with torch.no_grad():
            flex_attention(q, k, v, block_mask=bm)

    def fwd_bwd():
        q.grad = k.grad = v.grad = None
        flex_attention(q, k, v, block_mask=bm).backward(do)

    phases = {
        "mask": _median_spread(lambda: create_block_mask(mod, None, None, T, T, device="cpu"), reps),
        "fwd_head": _median_spread(fwd, reps),
        "fwd_bwd_head": _median_spread(fwd_bwd, reps),
    }
    # Cost is linear in heads and in independent batch rows.
    t_step = len(rows_np) * (phases["mask"][0] + c["Hq"] * phases["fwd_bwd_head"][0])
    return t_step, phases


def prologue_stats(dev, T: int, C: int, H: int, reps: int):
    """HIP-event timing of the attention-module prologue (t2t_qkv_rope and its
    gradient pass) at one layer's shape.  Algorithmic bytes per launch: the
    bf16 qkv rows read once and the q, k, v rows written once (2 x 3 C T x 2 B),
    plus the float32 cos / sin rows of the T positions (2 x T x D/2 x 4 B)."""
    import ctypes
    from tagseq2tagseq_amd import _lib
    from tagseq2tagseq_amd.rope import rope_tables
    D = C // H
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn(1, T, 3 * C, generator=g).to(torch.bfloat16).to(dev)
    dqkv = torch.empty_like(qkv)
    cos, sin = rope_tables(D, T, dev)
    ops = [torch.empty(1, H, T, D, dtype=torch.bfloat16, device=dev) for _ in range(3)]
    views = [ctypes.byref(_lib.tensor_struct(t)) for t in ops]
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    L = _lib.lib()
    # Launch through the C ABI with preallocated buffers, so the loop times the
    # kernels rather than the Python dispatch around them.
    calls = {
        "fwd": lambda: L.t2t_qkv_rope(qkv.data_ptr(), qkv.stride(0), qkv.stride(1), 1, T, H, D,
                                      cos.data_ptr(), sin.data_ptr(), T, 0, *views, stream),
        "bwd": lambda: L.t2t_qkv_rope_backward(*views, cos.data_ptr(), sin.data_ptr(), T, 0, 1,
                                               T, H, D, dqkv.data_ptr(), dqkv.stride(0),
                                               dqkv.stride(1), stream),
    }
    nbytes = 2 * 3 * C * T * 2 + 2 * T * (D // 2) * 4
    out = {"shape": {"T": T, "C": C, "H": H, "D": D}, "bytes_per_launch": nbytes}
    for name, fn in calls.items():
        _lib.check(fn(), "t2t_qkv_rope " + name)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        us = 1e3 * e0.elapsed_time(e1) / reps
        gbps = nbytes / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "GBps": round(gbps, 1),
                     "frac_of_hbm_peak": round(gbps / PEAK_HBM_GBS, 3)}
    return out


def schedule_bench(args, dev):
    """Density-aware ordering of packs across data-parallel ranks
    (tagseq2tagseq_amd.schedule).
      * cost model: 16 packs of the configs[2] generator (T 16384), attention
        fwd+bwd (H 16, D 128) timed per pack; R^2 of a linear fit of the step
        time on the exact pair count (pack_pairs, host);
      * straggler share (idle time of lockstep ranks waiting for the slowest,
        sum over steps of max - mean over sum of max) of 8 ranks x 64 steps,
        each rank drawing its own packs, with and without the ordering
        (window 16), costs = measured-model times of the packs."""
    from tagseq2tagseq_amd.schedule import DensityOrderedBatches, pack_pairs, straggler_fraction
    T, H, D = 16384, 16, 128
    g = torch.Generator().manual_seed(args.seed)
    q, k, v, do = (torch.randn(1, H, T, D, generator=g).to(torch.bfloat16).to(dev)
                   for _ in range(4))
    scale = 1.0 / math.sqrt(D)
    pairs, ms, tiles = [], [], []
    for s in range(16):
        row = synth.linked_lognormal_docs(T, 350.0, 1.0, 2048, 0.15, seed=100 + s)
        rows_np = [per_token_arrays(row)]
        doc = torch.from_numpy(rows_np[0][0]).to(dev)[None]
        qb = torch.from_numpy(rows_np[0][1].view(np.int64)).to(dev)[None]
        kb = torch.from_numpy(rows_np[0][2].view(np.int64)).to(dev)[None]
        bm = build_block_mask(doc, qb, kb)

        def step():
            out, lse2 = attn_fwd(q, k, v, bm, scale)
            attn_bwd(q, k, v, out, do, lse2, bm, scale)

        ms.append(time_launches(step, max(3, args.reps // 4)))
        pairs.append(pack_pairs(T, row.spans, row.link_rows))
        tc = bm.tile_class
        tiles.append((int((tc == 2).sum()), int((tc == 1).sum())))
    x, y = np.array(pairs, dtype=np.float64), np.array(ms)
    A = np.stack([x, np.ones_like(x)], 1)
    coef, *_ = np.linalg.lstsq(A, y, rcond=None)
    r2 = 1.0 - ((y - A @ coef) ** 2).sum() / ((y - y.mean()) ** 2).sum()
    # tile-class model (masks given only as per-token grant words): time =
    # a full + b partial + c; b / a is the partial-tile weight of tile_cost
    tf = np.array(tiles, dtype=np.float64)
    At = np.stack([tf[:, 0], tf[:, 1], np.ones(len(tf))], 1)
    ct, *_ = np.linalg.lstsq(At, y, rcond=None)
    r2t = 1.0 - ((y - At @ ct) ** 2).sum() / ((y - y.mean()) ** 2).sum()
    # 8 ranks x 64 steps of independent packs, costs from the fitted model
    ranks, steps, window = 8, 64, 16
    raw, ordered = [], []
    for r in range(ranks):
        packs = [{"ms": float(coef[0] * pack_pairs(T, row.spans, row.link_rows) + coef[1])}
                 for row in (synth.linked_lognormal_docs(T, 350.0, 1.0, 2048, 0.15,
                                                         seed=10000 * (r + 1) + k)
                             for k in range(steps))]
        raw.append([p["ms"] for p in packs])
        ordered.append([p["ms"] for p in DensityOrderedBatches(packs, lambda b: b["ms"], window)])
    f_raw, f_ord = straggler_fraction(np.array(raw)), straggler_fraction(np.array(ordered))
    print(json.dumps({
        "metric": "lockstep straggler share at 8 ranks (attention fwd+bwd time model)",
        "value": round(f_ord, 4), "unit": "fraction of step time idle",
        "higher_is_better": False, "n_gpus": 1, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "configs[2] packs, T 16384, H 16, D 128", "ranks": ranks,
                   "steps": steps, "window": window},
        "unordered": round(f_raw, 4),
        "cost_model": {"packs_timed": len(ms), "ms_per_mpair": round(coef[0] * 1e6, 5),
                       "ms_fixed": round(coef[1], 4), "r2": round(float(r2), 4),
                       "ms_range": [round(float(y.min()), 4), round(float(y.max()), 4)]},
        "tile_cost_model": {"ms_per_full_tile": round(float(ct[0]), 6),
                            "ms_per_partial_tile": round(float(ct[1]), 6),
                            "partial_weight": round(float(ct[1] / ct[0]), 3) if ct[0] else None,
                            "r2": round(float(r2t), 4)},
    }))


def decode_bench(args, dev):
    """Generation on the configs[4] model (12 layers, d768, H12, D64, vocab
    50257, random init) over a T = 16384 - 64 token context packed with the
    configs[2] cross_doc_link generator: after one prefill, each step appends a
    token to the last document and asks for the last position's logits.
      * cached: TS2TSModel.forward_inference_last (key/value cache, decode
        kernel over the new row), `--steps` steps after `--warmup`;
      * full recompute: TS2TSModel.forward_inference over the whole sequence,
        the reference's per-token path (model/generation_loop.py:90-92), 3 steps;
      * the decode attention kernel alone at one layer's shape (Tq 1, H 12,
        D 64, all context keys): algorithmic bytes = allowed keys x H x 4 D
        (K and V rows) + H x Tkv x (4 + 8 W) (mask inputs read per head).
    With --no-graphs nothing is captured as a HIP graph: the steps run eagerly
    and the kernel loop launches directly (the form for rocprofv3 counter
    passes, which serialise and instrument every dispatch)."""
    import numpy as np
    from tagseq2tagseq_amd.decode import attn_decode
    from tagseq2tagseq_amd.mask_creators import create_doc_link_block_mask
    from tagseq2tagseq_amd.model import TS2TSModel
    T_max, V, H, D = 16384, 50257, 12, 64
    row = synth.config_rows(3, seed=args.seed)[0]
    T0 = T_max - 64
    spans = [s for s in row.spans if s.start < T0]
    last = spans[-1]
    spans[-1] = synth.DocSpan(doc_id=last.doc_id, start=last.start, end=T0)
    links = np.asarray(row.link_rows, dtype=np.uint64)[:len(spans)]
    torch.manual_seed(args.seed)
    model = TS2TSModel.from_config(vocab_size=V, num_layers=12, model_dim=768, num_heads=H,
                                   max_seq_len=T_max, dropout=0.0, drop_path_rate=0.0,
                                   block_mask_creator=create_doc_link_block_mask)
    model = model.to(dev, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(args.seed)
    stream = torch.randint(0, V, (1, T_max), generator=g).to(dev)

    def grown(n):
        sp = list(spans)
        sp[-1] = synth.DocSpan(doc_id=last.doc_id, start=last.start, end=T0 + n)
        return stream[:, :T0 + n], sp

    graphs = not args.no_graphs
    model.use_graphs = graphs
    tok, sp = grown(0)
    model.forward_inference_last(tok, sp, doc_links=links)  # prefill
    n_steps = min(args.steps, 60 - args.warmup)
    for i in range(1, args.warmup + 1):
        tok, sp = grown(i)
        model.forward_inference_last(tok, sp, doc_links=links)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.warmup + 1, args.warmup + 1 + n_steps):
        tok, sp = grown(i)
        logits = model.forward_inference_last(tok, sp, doc_links=links)
        logits.argmax().item()  # the sampler needs the row on the host
    cached_ms = 1e3 * (time.perf_counter() - t0) / n_steps
    # the same steps without the captured graph (eager launches)
    model.use_graphs = False
    t0 = time.perf_counter()
    for i in range(args.warmup + 1, args.warmup + 1 + n_steps):
        tok, sp = grown(i)
        model.forward_inference_last(tok, sp, doc_links=links).argmax().item()
    eager_ms = 1e3 * (time.perf_counter() - t0) / n_steps
    model.use_graphs = graphs

    def replay_us(reps=50):
        if not graphs:
            return None
        # GPU time of one captured step (the graph alone, no host work)
        g = model._graph.graph
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return 1e3 * e0.elapsed_time(e1) / reps

    step_us = replay_us()
    # the same steps with the unfused layer sequence (torch GEMMs and
    # elementwise kernels around the prologue and decode kernels)
    model.fuse_rows = False
    for i in range(args.warmup + 1, args.warmup + 1 + n_steps):
        tok, sp = grown(i)
        model.forward_inference_last(tok, sp, doc_links=links).argmax().item()
    unfused_step_us = replay_us()
    model.fuse_rows = True
    tok, sp = grown(args.warmup + n_steps)
    ref = model.forward_inference(tok, sp, doc_links=links)[:, -1:].float()
    err = (logits.float() - ref).abs().max().item() / ref.abs().max().item()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        model.forward_inference(tok, sp, doc_links=links)[0, -1].argmax().item()
    full_ms = 1e3 * (time.perf_counter() - t0) / 3

    # the decode kernel alone at one layer's shape
    bm = create_doc_link_block_mask(tok, sp, doc_links=links)
    T = tok.shape[1]
    cache = model.kv_cache
    q = torch.randn(1, H, 1, D, device=dev).to(torch.bfloat16)
    pos = torch.tensor([[T - 1]], dtype=torch.int32, device=dev)
    qd = bm.doc_ids[:, T - 1:T].contiguous()
    qb = bm.q_bits[:, :, T - 1:T].contiguous()
    kc, vc = cache.k[0], cache.v[0]
    out = torch.empty(1, H, 1, D, dtype=torch.bfloat16, device=dev)
    attn_decode(q, kc, vc, T, cache.doc, cache.kv_bits, pos, qd, qb, out=out)  # validates
    # Launch through the C ABI with preallocated buffers so the loop times the
    # kernels (partial + combine), not the Python wrapper.
    import ctypes
    from tagseq2tagseq_amd import _lib
    L = _lib.lib()
    lse2 = torch.empty(1, H, 1, dtype=torch.float32, device=dev)
    wsb = L.t2t_attn_decode_workspace(1, H, 1, T, D)
    ws = torch.empty(wsb // 4, dtype=torch.float32, device=dev)
    views = [ctypes.byref(_lib.tensor_struct(t)) for t in (q, kc, vc, out)]
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    call_args = (*views, lse2.data_ptr(), cache.doc.data_ptr(), cache.kv_bits.data_ptr(),
                 cache.doc.shape[1], pos.data_ptr(), qd.data_ptr(), qb.data_ptr(), 1, bm.words,
                 1, H, H, 1, T, D, _lib.T2T_DTYPE_BF16, 1.0 / math.sqrt(D), ws.data_ptr(), wsb,
                 stream)
    _lib.check(L.t2t_attn_decode(*call_args), "t2t_attn_decode")
    torch.cuda.synchronize()
    # The pair of launches is ~15 us of GPU time, less than the host cost of
    # one ctypes call with two dozen arguments: the calls are captured into a
    # HIP graph on a side stream and the replays are timed, so the figure is
    # the kernels' time, not the host's.
    if graphs:
        side = torch.cuda.Stream(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            cap_args = call_args[:-1] + (ctypes.c_void_p(side.cuda_stream),)
            for _ in range(args.reps):
                _lib.check(L.t2t_attn_decode(*cap_args), "t2t_attn_decode")
        run_reps = graph.replay
    else:
        def run_reps():
            for _ in range(args.reps):
                _lib.check(L.t2t_attn_decode(*call_args), "t2t_attn_decode")
    run_reps()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    run_reps()
    e1.record()
    torch.cuda.synchronize()
    k_us = 1e3 * e0.elapsed_time(e1) / args.reps
    doc = bm.doc_ids[0]
    allowed = (doc == doc[T - 1]) | ((bm.kv_bits[0] & bm.q_bits[0, :, T - 1:T]) != 0).any(0)
    n_allowed = int(allowed.sum())
    W = bm.words
    k_bytes = n_allowed * H * 4 * D + H * T * (4 + 8 * W)
    gbps = k_bytes / (k_us * 1e-6) / 1e9
    print(json.dumps({
        "metric": "generation tokens/s with the key/value cache (12L d768 H12 D64, "
                  "cross_doc_link, T=16k context)",
        "value": round(1e3 / cached_ms, 2), "unit": "tokens/s", "n_gpus": 1, "steps": n_steps,
        "warmup": args.warmup, "ms_per_step": round(cached_ms, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random token ids, seeded packed documents, random-init weights)",
        "config": {"workload": "decode steps on the configs[4] model", "context": T0,
                   "vocab": V, "n_docs": len(spans), "grant_words": W},
        "graph_step_gpu_us": None if step_us is None else round(step_us, 1),
        "graph_step_gpu_us_unfused_layers": (None if unfused_step_us is None
                                             else round(unfused_step_us, 1)),
        "graphs": graphs,
        "eager_cached_ms_per_token": round(eager_ms, 3),
        "full_recompute_ms_per_token": round(full_ms, 2),
        "speedup_vs_full_recompute": round(full_ms / cached_ms, 1),
        "last_logits_rel_err_vs_full": round(err, 5),
        "decode_kernel": {"us": round(k_us, 2), "Tkv": T, "allowed_keys": n_allowed,
                          "bytes": k_bytes, "GBps": round(gbps, 1),
                          "frac_of_hbm_peak": round(gbps / PEAK_HBM_GBS, 3)},
    }))


def rows_bench(args, dev):
    """The fused few-row linear kernels of a decode step at the configs[4]
    model's layer shapes (one row, d768, GLU hidden 2048, vocab 50257): each
    kernel timed alone, algorithmic bytes = the weight matrix read once
    (2 N K; the rows, norm weights and outputs are < 0.1 % of it).  Timed as
    replays of a HIP graph of `--reps` calls (a ctypes call costs more host
    time than one kernel takes); `--rows-eager` launches the calls directly
    instead (no graph), e.g. for counter passes."""
    from tagseq2tagseq_amd.modules import RMSNorm
    from tagseq2tagseq_amd.rope import rope_tables
    from tagseq2tagseq_amd.rows import rows_linear, rows_qkv_rope
    C, hid, V, H, T = 768, 2048, 50257, 12, 16384
    D = C // H
    g = torch.Generator().manual_seed(args.seed)

    def w(n, k):
        return (torch.randn(n, k, generator=g) / math.sqrt(k)).to(torch.bfloat16).to(dev)

    x = torch.randn(1, C, generator=g).to(torch.bfloat16).to(dev)
    h = torch.randn(1, hid, generator=g).to(torch.bfloat16).to(dev)
    norm = RMSNorm(C).to(dev).to(torch.bfloat16)
    wqkv, wproj, wgu, wdown, whead = w(3 * C, C), w(C, C), w(2 * hid, C), w(C, hid), w(V, C)
    cos, sin = rope_tables(D, T, dev)
    kc = torch.zeros(1, H, T, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    pos = torch.tensor([T - 1], dtype=torch.int64, device=dev)
    calls = {
        "qkv_rope (norm + qkv + rotation + cache write)":
            (lambda: rows_qkv_rope(x, wqkv, H, cos, sin, pos, kc, vc, norm=norm), 3 * C * C),
        "add (out-projection + residual)":
            (lambda: rows_linear(x, wproj, epilogue="add", res=x), C * C),
        "swiglu (norm + gate_up + SwiGLU)":
            (lambda: rows_linear(x, wgu, norm=norm, epilogue="swiglu"), 2 * hid * C),
        "add (down + residual)": (lambda: rows_linear(h, wdown, epilogue="add", res=x), C * hid),
        "store (norm + LM head)": (lambda: rows_linear(x, whead, norm=norm), V * C),
    }
    out = {}
    for name, (fn, n_weights) in calls.items():
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        if args.rows_eager:
            e0.record()
            for _ in range(args.reps):
                fn()
            e1.record()
        else:
            side = torch.cuda.Stream(dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                for _ in range(args.reps):
                    fn()
            graph.replay()
            torch.cuda.synchronize()
            e0.record()
            graph.replay()
            e1.record()
        torch.cuda.synchronize()
        us = 1e3 * e0.elapsed_time(e1) / args.reps
        nbytes = 2 * n_weights
        gbps = nbytes / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "weight_bytes": nbytes, "GBps": round(gbps, 1),
                     "frac_of_hbm_peak": round(gbps / PEAK_HBM_GBS, 3)}
    print(json.dumps({
        "metric": "fused few-row linear kernels of a decode step (1 row, configs[4] layer shapes)",
        "unit": "us per launch", "timing": "eager launches" if args.rows_eager else "graph replays",
        "reps": args.reps, "dtype": "bf16", "data": "synthetic (random weights and rows)",
        "kernels": out}))


def config1_bench(args, dev):
    """doc_causal forward only, float32, B1 H4 T1024 D64 -- the
    reference's CPU-runnable case.  A step = per-token inputs from the span
    lists + metadata pass + float32 forward; value = 4 D N_pairs H / step time
    (forward-only useful FLOPs).  Next to it, the reference's own CPU path on
    the same inputs (torch eager create_block_mask + flex_attention forward in
    float32, every head) and the torch.compile(flex_attention) CPU forward."""
    from oracle.mask_oracle import torch_mask_mod
    from torch.nn.attention.flex_attention import create_block_mask
    from torch.nn.attention.flex_attention import flex_attention as torch_flex
    c = synth.CONFIGS[1]
    B, Hq, Hkv, T, D = c["B"], c["Hq"], c["Hkv"], c["T"], c["D"]
    rows = synth.config_rows(1, seed=args.seed)
    rows_np = [per_token_arrays(r) for r in rows]
    doc = torch.from_numpy(rows_np[0][0]).to(dev)[None]
    n_pairs = count_pairs(doc[0], None, None)
    useful = 4.0 * D * n_pairs * Hq
    g = torch.Generator().manual_seed(args.seed)
    qc, kc, vc = (torch.randn(B, h, T, D, generator=g) for h in (Hq, Hkv, Hkv))
    q, k, v = (t.to(dev) for t in (qc, kc, vc))
    scale = 1.0 / math.sqrt(D)
    lists = TokenLists(T, [r.spans for r in rows], dev)

    def step():
        bm = build_block_mask(*lists.build())
        return attn_fwd(q, k, v, bm, scale)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    bm = build_block_mask(*lists.build())
    t_fwd = time_launches(lambda: attn_fwd(q, k, v, bm, scale), args.reps)
    achieved = useful / (t_fwd * 1e-3) / 1e12
    result = {
        "metric": "masked attn fwd useful TFLOP/s, doc_causal float32 T=1k (configs[0])",
        "value": round(useful / (ms * 1e-3) / 1e12, 4), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded packed documents, Q/K/V ~ N(0,1))",
        "config": {"workload": "doc_causal fwd float32 B1 H4 T1024 D64 (configs[0])", "B": B,
                   "Hq": Hq, "Hkv": Hkv, "T": T, "D": D, "seed": args.seed,
                   "n_docs": [r.n_docs for r in rows], "n_pairs": n_pairs},
        "roofline": {"bound": "mfma", "kernel": "attn_fwd_f32_kernel", "achieved": round(achieved, 3),
                     "peak": PEAK_F32_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_F32_TFLOPS, 4), "traffic": None},
        "kernels_ms": {"attn_fwd_f32_kernel": round(t_fwd, 4)},
    }
    if not args.no_cpu_baseline:
        torch.set_num_threads(args.cpu_threads)
        mod = torch_mask_mod(torch.from_numpy(rows_np[0][0]), None, None)

        def cpu_step():
            m = create_block_mask(mod, None, None, T, T, device="cpu")
            return m, torch_flex(qc, kc, vc, block_mask=m)

        t_eager, t_lo, t_hi = _median_spread(cpu_step, args.cpu_reps)
        cbm, out = cpu_step()
        # same inputs: the GPU float32 forward against the reference's CPU output
        got = attn_fwd(q, k, v, bm, scale)[0].float().cpu()
        max_err = float((got - out).abs().max())
        avail, reported = host_cores()
        result["cpu_baseline"] = {
            "value": round(useful / t_eager / 1e12, 6), "unit": "TFLOP/s",
            "cores": args.cpu_threads, "host_cpus": {"os_cpu_count": reported, "affinity": avail},
            "kind": "reference", "reps": args.cpu_reps,
            "phases_s": {"mask+fwd": {"median": round(t_eager, 4), "min": round(t_lo, 4),
                                      "max": round(t_hi, 4)}},
            "sample": (f"torch {torch.__version__} eager create_block_mask + flex_attention "
                       f"forward, float32, all {Hq} heads, on CPU (median of {args.cpu_reps} after "
                       f"1 warm-up: {t_eager:.3f} s)"),
            "max_abs_diff_vs_gpu": max_err,
        }
        try:
            cf = torch.compile(torch_flex)
            cf(qc, kc, vc, block_mask=cbm)  # compile
            t_comp, _, _ = _median_spread(lambda: cf(qc, kc, vc, block_mask=cbm), args.cpu_reps)
            result["cpu_compiled_fwd"] = {"s": round(t_comp, 4),
                                          "TFLOPs": round(useful / t_comp / 1e12, 6),
                                          "sample": "torch.compile(flex_attention) forward on CPU, "
                                                    f"block mask prebuilt, median of {args.cpu_reps} "
                                                    "after the compiling call and 1 warm-up"}
        except Exception as e:  # inductor's CPU path needs a host C++ toolchain
            result["cpu_compiled_fwd"] = {"error": f"{type(e).__name__}: {str(e)[:200]}"}
    print(json.dumps(result))


def backbone_step(args, dev):
    """one training step (mask creation from the device-resident
    span / link lists, embedding, 12 layers, RMSNorm, tied linear + CE loss,
    backward, AdamW) of the 12-layer d768 H12 (D 64) backbone on a packed
    T = 16384 row of random token ids with the configs[2] cross_doc_link
    generator; random-init weights (tagseq2tagseq_amd.train_step).  The
    library products use the committed TunableOp selections
    (tagseq2tagseq_amd.gemm_tuning) when this software stack matches them.
    Prints one JSON line (tokens/s)."""
    from tagseq2tagseq_amd.gemm_tuning import TUNED_FILE, use_tuned_gemms
    from tagseq2tagseq_amd.train_step import VOCAB, configs4_step
    tuned = False if args.no_gemm_tuning else use_tuned_gemms()
    step = configs4_step(dev, seed=args.seed)
    model, row, T, V = step.model, step.row, step.T, VOCAB

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(args.steps):
        loss = step()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    n_params = sum(p.numel() for p in model.parameters())
    prologue = prologue_stats(dev, T, 768, 12, args.reps)
    print(json.dumps({
        "metric": "backbone training tokens/s (12L d768 H12 D64, cross_doc_link T=16k)",
        "value": round(T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random token ids, seeded packed documents)",
        "config": {"workload": "12-layer backbone training step (configs[4])", "T": T,
                   "vocab": V, "params": n_params, "n_docs": row.n_docs,
                   "optimizer": "AdamW (fused)"},
        "gemm_tuning": {"file": os.path.relpath(TUNED_FILE, ROOT), "loaded": tuned},
        "final_loss": round(float(loss.item()), 4),
        "prologue": prologue,
    }))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--no-gemm-tuning", action="store_true",
                    help="with --config 5: the library products' default heuristics instead of "
                         "the committed TunableOp selections")
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5],
                    help="3 (default): the metric's workload; 2, 4: other attention "
                         "workloads; 1: float32 forward-only case; 5: 12-layer backbone "
                         "training step (tokens/s)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--reps", type=int, default=20, help="launches per per-kernel timing")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=host_cores()[0],
                    help="CPU-baseline threads (default: every CPU this process may use)")
    ap.add_argument("--cpu-reps", type=int, default=5,
                    help="timed repetitions per CPU-baseline phase (after one warm-up)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (HBM-counter calibration)")
    ap.add_argument("--schedule", action="store_true",
                    help="density-aware ordering across ranks: cost-model check on the GPU "
                         "and the simulated straggler share at 8 ranks")
    ap.add_argument("--decode", action="store_true",
                    help="generation with the key/value cache on the configs[4] model "
                         "(per-token latency, cached vs full recompute, decode kernel roofline)")
    ap.add_argument("--no-graphs", action="store_true",
                    help="with --decode: run every step eagerly and launch the kernel loop "
                         "directly, capturing no HIP graph")
    ap.add_argument("--rows", action="store_true",
                    help="the fused few-row linear kernels of a decode step, each timed alone")
    ap.add_argument("--rows-eager", action="store_true",
                    help="with --rows: time direct launches instead of graph replays")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")

    if args.rows:
        rows_bench(args, dev)
        return
    if args.decode:
        decode_bench(args, dev)
        return
    if args.schedule:
        schedule_bench(args, dev)
        return
    if args.config == 5:
        backbone_step(args, dev)
        return
    if args.config == 1:
        config1_bench(args, dev)
        return

    if args.copy_calibration:
        x = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": x.numel(), "launches": 5}))
        return

    c = synth.CONFIGS[args.config]
    B, Hq, Hkv, T, D = c["B"], c["Hq"], c["Hkv"], c["T"], c["D"]
    rows = synth.config_rows(args.config, seed=args.seed)
    rows_np = [per_token_arrays(r) for r in rows]

    doc = torch.stack([torch.from_numpy(r[0]) for r in rows_np]).to(dev)
    if rows_np[0][1] is not None:
        qb = torch.stack([torch.from_numpy(r[1].view(np.int64)) for r in rows_np]).to(dev)
        kb = torch.stack([torch.from_numpy(r[2].view(np.int64)) for r in rows_np]).to(dev)
    else:
        qb = kb = None
    g = torch.Generator().manual_seed(args.seed)
    q = torch.randn(B, Hq, T, D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).to(dev)
    do = torch.randn(B, Hq, T, D, generator=g).to(torch.bfloat16).to(dev)
    scale = 1.0 / math.sqrt(D)

    W = 0 if qb is None else qb.shape[1]
    n_pairs = 0
    for b in range(B):
        bb = b if len(rows_np) > 1 else 0
        n_pairs += count_pairs(doc[bb], None if qb is None else qb[bb], None if kb is None else kb[bb])
    causal_pairs = B * T * (T + 1) // 2
    useful_flops = 14.0 * D * n_pairs * Hq

    # Span / link lists resident on the device; each step rebuilds the
    # per-token inputs from them (t2t_token_inputs), then the metadata pass.
    lists = TokenLists(T, [r.spans for r in rows], dev, words=W,
                       link_rows=None if W == 0 else [r.link_rows for r in rows])
    doc_d, qb_d, kb_d = lists.build()
    assert torch.equal(doc_d, doc) and (qb is None or (torch.equal(qb_d, qb) and torch.equal(kb_d, kb)))

    def step():
        d_, q_, k_ = lists.build()
        bm = build_block_mask(d_, q_, k_)
        out, lse2 = attn_fwd(q, k, v, bm, scale)
        return attn_bwd(q, k, v, out, do, lse2, bm, scale)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = ev0.elapsed_time(ev1) / args.steps
    value = useful_flops / (ms_per_step * 1e-3) / 1e12

    # Per-kernel mean durations on fixed buffers.
    bm = build_block_mask(doc, qb, kb)
    out, lse2 = attn_fwd(q, k, v, bm, scale)
    ph = BwdPhases(q, k, v, out, do, lse2, bm, scale)
    ph.preprocess()
    # The small launches are timed through their C entry points on fixed
    # buffers, so the loop measures the kernels rather than the Python around
    # them (tensor allocation, argument marshalling).
    import ctypes
    from tagseq2tagseq_amd import _lib
    tok_bufs = lists.build()
    t_tok = time_launches(lambda: lists.build(out=tok_bufs), args.reps)
    cs = bm.c_struct()
    meta_args = (bm.doc_ids.data_ptr(), bm.q_bits.data_ptr() if bm.words else None,
                 bm.kv_bits.data_ptr() if bm.words else None, bm.mask_batch, T, bm.words,
                 bm.tile_class.data_ptr(), ctypes.byref(cs),
                 ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    L = _lib.lib()
    t_meta = time_launches(lambda: L.t2t_mask_meta(*meta_args), args.reps)
    t_fwd = time_launches(lambda: attn_fwd(q, k, v, bm, scale), args.reps)
    t_pre = time_launches(ph.preprocess, args.reps)
    t_dkdv = time_launches(ph.dkdv, args.reps)
    t_dq = time_launches(ph.dq_pass, args.reps)
    t_bwd = time_launches(ph.whole, args.reps)
    # The measurement plan's form: medians of >= 50 timed calls after 10
    # discarded ones, forward alone and forward + backward, on the prebuilt
    # mask (the metadata pass is timed separately above).
    fwd_med = median_ms(lambda: attn_fwd(q, k, v, bm, scale))

    def fwd_bwd():
        o_, l_ = attn_fwd(q, k, v, bm, scale)
        return attn_bwd(q, k, v, o_, do, l_, bm, scale)

    fb_med = median_ms(fwd_bwd)

    base = D * n_pairs * Hq
    kernels = {
        "attn_fwd_bf16_kernel": (t_fwd, 4.0 * base),
        dkdv_kernel_name(D): (t_dkdv, 8.0 * base),
        "bwd_dq_kernel": (t_dq, 6.0 * base),
    }
    dom = max(kernels, key=lambda n: kernels[n][0])
    dom_ms, dom_flops = kernels[dom]
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12

    nt = (T + 127) // 128
    Bm = doc.shape[0]
    tc = bm.tile_class
    tiles = {"full": int((tc == 2).sum()), "partial": int((tc == 1).sum()), "skip": int((tc == 0).sum())}
    # the engine clock this box sustains under MFMA load, and the metric and
    # the roofline kernel against the peak at that clock (the line's own
    # `peak` stays the published figure)
    clock = engine_clock(dev)
    peak_clk = clock["bf16_peak_at_clock_tflops"]
    clock["pct_of_peak_at_clock"] = round(100.0 * value / peak_clk, 2)
    clock["roofline_frac_at_clock"] = round(achieved / peak_clk, 4)
    # metadata pass, algorithmic bytes: per-token reads + every table written once
    meta_bytes = (Bm * T * 4 + 2 * 8 * W * Bm * T          # doc ids, q / kv grant words
                  + Bm * nt * nt                           # tile classes
                  + 4 * (5 * Bm * nt * nt + 7 * Bm * nt)   # 4 index + q_bits_slot, 4 counts + 3
                  + 4096 * tiles["partial"])               # two 128x128-bit maps per partial tile

    # token-input builder, algorithmic bytes: the span / grant lists read, the
    # per-token doc ids and grant words written
    tok_bytes = (lists.lists.numel() * 4 + (0 if lists.links is None else lists.links.numel() * 8)
                 + Bm * T * 4 + 2 * 8 * W * Bm * T)

    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded packed documents, Q/K/V/dO ~ N(0,1))",
        "config": {
            "workload": WORKLOAD_NAMES[args.config],
            "B": B, "Hq": Hq, "Hkv": Hkv, "T": T, "D": D, "seed": args.seed,
            "n_docs": [r.n_docs for r in rows], "grant_words": W,
            "n_pairs": n_pairs, "density_vs_causal": round(n_pairs / causal_pairs, 4),
            "tiles_128": tiles,
        },
        "pct_of_bf16_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "roofline": {
            "bound": "mfma",
            "kernel": dom,
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": measured_traffic(args.config, dom),
            "traffic_source": f"profiles/hbm_traffic_config{args.config}.txt",
        },
        "mfma_busy": profile_mfma_busy(args.config),
        "executed_work": executed_work(bm, B, Hq, D, n_pairs, args.config),
        "clock": clock,
        "kernels_ms": {
            "token_inputs_kernel": round(t_tok, 4),
            "mask_meta (3 launches)": round(t_meta, 4),
            "attn_fwd_bf16_kernel": round(t_fwd, 4),
            "bwd_delta_kernel": round(t_pre, 4),
            dkdv_kernel_name(D): round(t_dkdv, 4),
            "bwd_dq_kernel": round(t_dq, 4),
        },
        # The step's backward is t2t_attn_bwd: dQ computing Delta itself, then
        # dK/dV (bwd_delta above is the separate-phase entry point's launch).
        "attn_bwd_ms": {"t2t_attn_bwd (dQ+Delta, dK/dV)": round(t_bwd, 4)},
        "median_of_50": {
            "fwd_ms": [round(x, 4) for x in fwd_med],
            "fwd_TFLOPs": round(4.0 * base / (fwd_med[0] * 1e-3) / 1e12, 2),
            "fwd_bwd_ms": [round(x, 4) for x in fb_med],
            "fwd_bwd_TFLOPs": round(useful_flops / (fb_med[0] * 1e-3) / 1e12, 2),
            "method": "median, min, max of 50 calls after 10 warm-ups, each bracketed by HIP "
                      "events; mask prebuilt; useful FLOPs 4 D N_pairs Hq (fwd), 14 D N_pairs Hq",
        },
        "mask_meta": {"us": round(t_meta * 1e3, 2), "bytes": int(meta_bytes),
                      "GBps": round(meta_bytes / (t_meta * 1e-3) / 1e9, 2)},
        "token_inputs": {"us": round(t_tok * 1e3, 2), "bytes": int(tok_bytes),
                         "GBps": round(tok_bytes / (t_tok * 1e-3) / 1e9, 2)},
        "wall_s_timed": round(wall, 3),
    }

    if not args.no_cpu_baseline:
        t_step, ph_cpu = cpu_baseline(rows_np, c, args.seed, args.cpu_threads, args.cpu_reps)
        avail, reported = host_cores()
        result["cpu_baseline"] = {
            "value": round(useful_flops / t_step / 1e12, 6),
            "unit": "TFLOP/s",
            "cores": args.cpu_threads,
            "host_cpus": {"os_cpu_count": reported, "affinity": avail},
            "kind": "reference",
            "reps": args.cpu_reps,
            "phases_s": {n: {"median": round(m, 4), "min": round(lo, 4), "max": round(hi, 4)}
                         for n, (m, lo, hi) in ph_cpu.items()},
            "sample": (f"torch {torch.__version__} on CPU, reference mask_mod: create_block_mask, "
                       f"eager flex_attention fwd and fwd+bwd on 1 of {Hq} heads of batch row 0, "
                       f"median of {args.cpu_reps} after 1 warm-up each; step = rows x (mask + "
                       f"{Hq} x fwd+bwd head) = {len(rows_np)} x ({ph_cpu['mask'][0]:.2f} + {Hq} x "
                       f"{ph_cpu['fwd_bwd_head'][0]:.2f}) s"),
            "s_per_step": round(t_step, 2),
        }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
