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
MFMA busy cycles of the attention kernels come from rocprofv3 counters
(SQ_VALU_MFMA_BUSY_CYCLES) in a separate run: profiles/ holds the summary.
Prints one JSON line per configuration and writes a CSV.
"""
from __future__ import annotations

import argparse
import csv
import json
import math
import statistics

import numpy as np
import torch

from . import synth
from .block_mask import build_block_mask
from .mask_creators import TokenLists
from .modules import Layer

PEAK_BF16_TFLOPS = 2516.6


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


def run(masks, reps: int, seed: int = 0):
    dev = torch.device("cuda:0")
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
                    n_pairs = _pairs(bm)
                    t_meta = _median_ms(lambda: build_block_mask(*lists.build()), reps)
                    t_fwd = _median_ms(lambda: layer(x, bm), reps)
                    g = torch.randn(1, T, n_embd, device=dev, dtype=torch.bfloat16)

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
                    })
                    rows.append(rec)
                    print(json.dumps(rec), flush=True)
                    del layer, x, bm, lists
    return rows


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--masks", default="causal,doc_causal,cross_doc_link")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--csv", default=None)
    args = ap.parse_args(argv)
    rows = run(args.masks.split(","), args.reps, args.seed)
    if args.csv:
        keys = sorted({k for r in rows for k in r})
        with open(args.csv, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=keys)
            w.writeheader()
            w.writerows(rows)


if __name__ == "__main__":
    main()
