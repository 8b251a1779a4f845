"""Layer benchmark: the reference's benchmarks/bench_layer.py sweep, extended.

    python -m tagseq2tagseq_amd.bench_layer [--masks causal,doc_causal,cross_doc_link]
                                            [--reps 20] [--csv layer_bench.csv]

The reference times its ``Layer`` (RMSNorm -> FlexSelfAttention -> GLU,
model/modules/layer.py:11-35) fwd and fwd+bwd over n_embd {256, 512, 1024} x
n_head {4, 8} x max_seq_len {512, 1024, 2048} with a causal BlockMask
(benchmarks/bench_layer.py:16-41).  This harness runs the same sweep on the
gfx950 attention (bf16; the fp8 variants are not built) and adds, per
configuration and mask kind:
  * the metadata pass time and its GB/s (algorithmic bytes, as in bench.py),
  * useful attention TFLOP/s counted over unmasked pairs only (fwd 4 D N H,
    fwd+bwd 14 D N H) and as a fraction of the MI355X dense bf16 peak.
Head dims other than 64 / 128 (n_embd / n_head) are reported as unsupported.
Prints one JSON line per configuration and writes a CSV.

MFMA utilisation per point and attention kernel:

    python -m tagseq2tagseq_amd.bench_layer --profile-mfma profiles/layer_mfma.txt

runs the sweep again in a child process under ``rocprofv3 --pmc
SQ_VALU_MFMA_BUSY_CYCLES`` (this process never touches the GPU) and writes,
per point, each attention kernel's MFMA-busy cycles over the chip's
SIMD-cycles during its dispatches (1024 SIMDs at 2.4 GHz; the dispatch
durations come from the same counter records).  A normal run attaches the
committed figures of profiles/layer_mfma.txt to each point as ``mfma_busy``.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import math
import os
import statistics
import subprocess
import sys
import tempfile

import numpy as np
import torch

from . import synth
from .block_mask import build_block_mask
from .mask_creators import TokenLists
from .modules import Layer

PEAK_BF16_TFLOPS = 2516.6
SIMDS, CLOCK_HZ = 1024, 2.4e9
ATTN_KERNELS = ("attn_fwd_bf16_kernel", "bwd_dq_kernel", "bwd_dkdv_kernel", "bwd_dkdv_pair_kernel")
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROFILE = os.path.join(ROOT, "profiles", "layer_mfma.txt")
PASS_CALLS = 3  # layer fwd+bwd calls per point in the counter pass


def _point_key(rec) -> str:
    return f"{rec['mask']} n_embd={rec['n_embd']} n_head={rec['n_head']} T={rec['max_seq_len']}"


def load_profile(path: str = PROFILE):
    """{point key: {kernel: busy fraction}} from a --profile-mfma summary."""
    out = {}
    if not os.path.exists(path):
        return out
    with open(path) as f:
        for line in f:
            if line.startswith("#") or "|" not in line:
                continue
            key, vals = line.split("|", 1)
            out[key.strip()] = {k: float(v) for k, v in (t.split("=") for t in vals.split())}
    return out


def _mask_inputs(kind: str, T: int, seed: int, dev):
    if kind == "causal":
        return TokenLists(T, [[synth.DocSpan(doc_id=0, start=0, end=T)]], dev)
    if kind == "doc_causal":
        row = synth.lognormal_docs(T, 300.0, 1.0, 2048, seed)
        return TokenLists(T, [row.spans], dev)
    row = synth.linked_lognormal_docs(T, 350.0, 1.0, 2048, 0.15, seed)
    return TokenLists(T, [row.spans], dev, words=row.words, link_rows=[row.link_rows])


def _pairs(bm) -> int:
    """Exact allowed-pair count of the mask (GPU, chunked rows)."""
    doc = bm.doc_ids[0]
    T = doc.shape[0]
    kv = torch.arange(T, device=doc.device)[None, :]
    total = 0
    for r0 in range(0, T, 1024):
        r1 = min(T, r0 + 1024)
        m = doc[r0:r1, None] == doc[None, :]
        for w in range(bm.words):
            m |= (bm.q_bits[0, w, r0:r1, None] & bm.kv_bits[0, w][None, :]) != 0
        m &= torch.arange(r0, r1, device=doc.device)[:, None] >= kv
        total += int(m.sum().item())
    return total


def _median_ms(fn, reps: int) -> float:
    fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b))
    return statistics.median(times)


def run(masks, reps: int, seed: int = 0, counter_pass: bool = False):
    """The sweep.  ``counter_pass``: per point only PASS_CALLS layer fwd+bwd
    calls after the mask build (3 attention dispatches each: forward, dQ,
    dK/dV), so that a profiler's dispatch list splits by point."""
    dev = torch.device("cuda:0")
    prof = {} if counter_pass else load_profile()
    rows = []
    for kind in masks:
        for n_embd in (256, 512, 1024):
            for n_head in (4, 8):
                for T in (512, 1024, 2048):
                    D = n_embd // n_head
                    rec = {"mask": kind, "n_embd": n_embd, "n_head": n_head, "max_seq_len": T,
                           "head_dim": D, "fp8": False}
                    if D not in (64, 128):
                        rec["status"] = f"unsupported head dim {D}"
                        rows.append(rec)
                        print(json.dumps(rec), flush=True)
                        continue
                    torch.manual_seed(seed)
                    layer = Layer(n_embd, n_head, 0.0, T, False, 0.0).to(dev, torch.bfloat16)
                    x = torch.randn(1, T, n_embd, device=dev, dtype=torch.bfloat16,
                                    requires_grad=True)
                    lists = _mask_inputs(kind, T, seed, dev)
                    bm = build_block_mask(*lists.build())
                    g = torch.randn(1, T, n_embd, device=dev, dtype=torch.bfloat16)
                    if counter_pass:
                        for _ in range(PASS_CALLS):
                            layer(x, bm).backward(g)
                        torch.cuda.synchronize()
                        rec.update({"status": "ok", "attn_dispatches": 3 * PASS_CALLS})
                        rows.append(rec)
                        print(json.dumps(rec), flush=True)
                        del layer, x, bm, lists
                        continue
                    n_pairs = _pairs(bm)
                    t_meta = _median_ms(lambda: build_block_mask(*lists.build()), reps)
                    t_fwd = _median_ms(lambda: layer(x, bm), reps)

                    def fwd_bwd():
                        layer(x, bm).backward(g)

                    t_fb = _median_ms(fwd_bwd, reps)
                    nt = (T + 127) // 128
                    W = bm.words
                    meta_bytes = (4 * T + 16 * W * T + nt * nt + 4 * (5 * nt * nt + 7 * nt)
                                  + 4096 * int((bm.tile_class == 1).sum()))
                    att_fwd = 4.0 * D * n_pairs * n_head
                    att_fb = 14.0 * D * n_pairs * n_head
                    rec.update({
                        "status": "ok", "n_pairs": n_pairs,
                        "density_vs_causal": round(n_pairs / (T * (T + 1) / 2), 4),
                        "meta_us": round(1e3 * t_meta, 2),
                        "meta_GBps": round(meta_bytes / (t_meta * 1e-3) / 1e9, 2),
                        "layer_fwd_ms": round(t_fwd, 4), "layer_fwd_bwd_ms": round(t_fb, 4),
                        "attn_useful_TFLOPs_in_layer_fwd": round(att_fwd / (t_fwd * 1e-3) / 1e12, 2),
                        "attn_useful_TFLOPs_in_layer_fwd_bwd": round(att_fb / (t_fb * 1e-3) / 1e12, 2),
                        "pct_of_bf16_peak_fwd_bwd": round(
                            100 * att_fb / (t_fb * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 3),
                        "mfma_busy": prof.get(_point_key(rec)),
                    })
                    rows.append(rec)
                    print(json.dumps(rec), flush=True)
                    del layer, x, bm, lists
    return rows


def profile_mfma(masks: str, seed: int, out_path: str) -> None:
    """The sweep's counter pass in a child process under rocprofv3, then the
    per-point MFMA-busy fractions written to out_path."""
    with tempfile.TemporaryDirectory(prefix="layer_mfma_") as work:
        cmd = ["rocprofv3", "--pmc", "SQ_VALU_MFMA_BUSY_CYCLES", "--output-format", "csv",
               "-d", work, "-o", "layer", "--", sys.executable, "-u", "-m",
               "tagseq2tagseq_amd.bench_layer", "--masks", masks, "--seed", str(seed),
               "--counter-pass"]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        points = [json.loads(l) for l in proc.stdout.splitlines() if l.startswith("{")]
        if proc.returncode != 0 and not points:
            raise SystemExit(f"counter pass failed ({proc.returncode}):\n{proc.stderr[-2000:]}")
        files = glob.glob(os.path.join(work, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            raise SystemExit("the counter pass wrote no counter_collection.csv")
        disp = {}
        with open(files[0]) as f:
            for r in csv.DictReader(f):
                name = r["Kernel_Name"]
                kern = next((k for k in ATTN_KERNELS if k in name), None)
                if kern is None:
                    continue
                d = disp.setdefault(int(r["Dispatch_Id"]), [kern, 0.0, 0.0])
                d[1] += float(r["Counter_Value"])
                d[2] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9
    order = [disp[i] for i in sorted(disp)]
    ok = [p for p in points if p.get("status") == "ok"]
    want = sum(p["attn_dispatches"] for p in ok)
    if len(order) != want:
        raise SystemExit(f"{len(order)} attention dispatches profiled, {want} expected")
    lines = ["# MFMA-busy fraction of the attention kernels per bench_layer point (MI355X, bf16):",
             "# SQ_VALU_MFMA_BUSY_CYCLES summed over a kernel's dispatches / (1024 SIMDs x 2.4 GHz x",
             f"# their summed durations), {PASS_CALLS} layer fwd+bwd calls per point after the mask build.",
             "# command (repo root, GPU box):",
             f"#   python -m tagseq2tagseq_amd.bench_layer --masks {masks} --seed {seed} "
             f"--profile-mfma {os.path.relpath(out_path, ROOT)}",
             ""]
    i = 0
    for p in ok:
        chunk = order[i:i + p["attn_dispatches"]]
        i += p["attn_dispatches"]
        busy = {}
        for k in ATTN_KERNELS:
            cyc = sum(c for n, c, _ in chunk if n == k)
            dur = sum(t for n, _, t in chunk if n == k)
            if dur > 0:
                busy[k] = cyc / (SIMDS * CLOCK_HZ * dur)
        lines.append(f"{_point_key(p)} | " + " ".join(f"{k}={v:.4f}" for k, v in busy.items()))
    with open(out_path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(f"wrote {out_path} ({len(ok)} points)")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--masks", default="causal,doc_causal,cross_doc_link")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--csv", default=None)
    ap.add_argument("--profile-mfma", metavar="OUT", default=None,
                    help="measure the per-point MFMA utilisation under rocprofv3 and write OUT")
    ap.add_argument("--counter-pass", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args(argv)
    if args.profile_mfma:
        profile_mfma(args.masks, args.seed, os.path.abspath(args.profile_mfma))
        return
    rows = run(args.masks.split(","), args.reps, args.seed, counter_pass=args.counter_pass)
    if args.csv:
        keys = sorted({k for r in rows for k in r})
        with open(args.csv, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=keys)
            w.writeheader()
            w.writerows(rows)


if __name__ == "__main__":
    main()
