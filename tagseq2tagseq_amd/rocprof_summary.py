"""Text summaries of rocprofv3 runs of bench.py (kernel durations, HBM traffic).

    python -m tagseq2tagseq_amd.rocprof_summary trace  <kt_dir> <bench_json> <config> [bench args] > kernel_trace.txt
    python -m tagseq2tagseq_amd.rocprof_summary traffic <fetch_dir> <write_dir> \
        <copy_fetch_dir> <copy_write_dir> <config> > hbm_traffic.txt
    python -m tagseq2tagseq_amd.rocprof_summary insts <sq_dir> <kt_dir> <config> [bench args] > insts.txt

`insts` reads one `--pmc` pass of SQ instruction counters (SQ_INSTS_VALU,
SQ_INSTS_MFMA, SQ_INSTS_LDS, SQ_INSTS_SALU, SQ_INSTS_VALU_TRANS_F32,
SQ_INSTS_VMEM, SQ_VALU_MFMA_BUSY_CYCLES, SQ_BUSY_CYCLES) and lists, per
kernel, the instructions issued per MFMA and the MFMA-busy fraction:
SQ_VALU_MFMA_BUSY_CYCLES per dispatch (summed over the chip) over the
machine's SIMD-cycles in the kernel's mean duration from the kernel-trace
run of the same session (1024 SIMDs at 2.4 GHz).  bench.py attaches the
`mfma_busy` lines of this file to its JSON line.

`trace` reads a `rocprofv3 --kernel-trace` database and lists, per kernel,
the number of dispatches and their mean / median / min / max duration next to
bench.py's own HIP-event means (the `kernels_ms` of its JSON line).

`traffic` reads the `--pmc FETCH_SIZE` and `--pmc WRITE_SIZE` databases of a
bench.py run and of `bench.py --copy-calibration` (1 GiB device copies), and
scales each counter so that the copy reads as its known size.  bench.py's
roofline `traffic` field reads the resulting file.
"""
from __future__ import annotations

import glob
import json
import sqlite3
import statistics
import sys
from collections import defaultdict
from typing import Dict, List

WORKLOADS = {
    "2": "doc_causal B2 H12 T8192 D64 bf16",
    "3": "cross_doc_link B1 H16 T16384 D128 bf16",
    "4": "cross_doc_link GQA B1 Hq16 Hkv4 T32768 D128 bf16",
    "5": "12-layer d768 H12 D64 backbone training step, cross_doc_link T16384 bf16",
    "decode": "generation on the config-5 model, T~16k context, one token per step",
    "rows": "fused few-row linear kernels of a decode step, one row, config-5 layer shapes",
}
DEFAULT_ARGS = "--config {cfg} --no-cpu-baseline --steps 10 --warmup 3"


def _label(cfg) -> str:
    return f"config {cfg}" if str(cfg).isdigit() else str(cfg)


def _short(name: str) -> str:
    """Kernel name without the namespace / template / argument decoration."""
    base = name.replace("(anonymous namespace)", "").split("(")[0]
    tmpl = ""
    if "<" in base:
        base, tmpl = base.split("<", 1)
    base = base.split("::")[-1].replace("void ", "").strip()
    if base == "rows_linear_kernel":  # <K chunks per lane, rows, epilogue>: one line per shape
        mode = ("store", "add", "swiglu", "qkv_rope")[int(tmpl.rstrip(">").split(",")[-1])]
        kv, mt = (int(t) for t in tmpl.split(",")[:2])
        return f"rows_linear[K<={512 * kv},M<={mt},{mode}]"
    return base


def _db(path: str) -> sqlite3.Connection:
    dbs = glob.glob(f"{path}/**/*.db", recursive=True)
    if not dbs:
        raise SystemExit(f"no rocprofv3 database under {path}")
    return sqlite3.connect(dbs[0])


def kernel_durations(path: str) -> Dict[str, List[float]]:
    """Dispatch durations (us) per t2t kernel of a kernel-trace database."""
    out: Dict[str, List[float]] = defaultdict(list)
    for name, dur in _db(path).execute("select name, duration from kernels"):
        if "t2t::" in name:
            out[_short(name)].append(dur / 1000.0)
    return out


def counter_means(path: str, counter: str, match: str = "t2t::") -> Dict[str, float]:
    """Mean per-dispatch value of one counter (summed over its instances)."""
    per_dispatch: Dict[tuple, float] = defaultdict(float)
    con = _db(path)
    rows = con.execute("select kernel_name, dispatch_id, counter_name, value from counters_collection")
    for kname, disp, cname, val in rows:
        if cname == counter and match in kname:
            per_dispatch[(_short(kname), disp)] += val
    sums: Dict[str, List[float]] = defaultdict(list)
    for (k, _), v in per_dispatch.items():
        sums[k].append(v)
    return {k: sum(v) / len(v) for k, v in sums.items()}


def copy_counter(path: str, counter: str) -> float:
    """Mean per-dispatch counter value of the calibration copy kernel."""
    vals = counter_means(path, counter, match="copy")
    if not vals:
        raise SystemExit(f"no copy kernel with {counter} under {path}")
    return max(vals.values())


def trace(kt_dir: str, bench_json: str, cfg: str, bench_args: str = "") -> str:
    durs = kernel_durations(kt_dir)
    dbs = glob.glob(f"{kt_dir}/**/*_results.db", recursive=True)
    out_name = dbs[0].rsplit("/", 1)[-1][:-len("_results.db")] if dbs else "kt"
    bench_args = bench_args or DEFAULT_ARGS.format(cfg=cfg)
    with open(bench_json) as f:
        bench = json.loads(f.read().strip().splitlines()[-1])
    ev = bench.get("kernels_ms", {})
    lines = [
        f"# rocprofv3 kernel trace -- {_label(cfg)} ({WORKLOADS.get(str(cfg), '?')}), MI355X",
        "#",
        "# command (repo root, GPU box):",
        f"#   rocprofv3 --kernel-trace --stats -d {kt_dir} -o {out_name} -- \\",
        f"#       python3 -u bench.py {bench_args}",
        "# durations in microseconds over every dispatch of the run (warm-up, timed steps and",
        "# bench.py's per-kernel timing loops); the last column is bench.py's own HIP-event",
        "# mean per call from the JSON line of the same profiled run (token_inputs: the whole",
        "# TokenLists.build() call, host side included).",
        "",
        f"{'kernel':36s} {'calls':>6s} {'mean':>8s} {'median':>8s} {'min':>8s} {'max':>8s}   bench.py HIP events",
    ]
    for k, v in sorted(durs.items(), key=lambda kv: -statistics.mean(kv[1])):
        evk = next((ev[e] for e in ev if e.startswith(k)), None)
        evs = f"{1000 * evk:10.1f}" if evk is not None else "         -"
        lines.append(f"{k:36s} {len(v):6d} {statistics.mean(v):8.1f} {statistics.median(v):8.1f} "
                     f"{min(v):8.1f} {max(v):8.1f}   {evs}")
    lines.append("")
    lines.append(f"# bench.py line of that run: value {bench.get('value')} {bench.get('unit')}, "
                 f"ms_per_step {bench.get('ms_per_step')}")
    for key in ("prologue", "decode_kernel"):
        if key in bench:
            lines.append(f"# bench.py {key}: {json.dumps(bench[key])}")
    return "\n".join(lines) + "\n"


def traffic(fetch_dir: str, write_dir: str, cfetch_dir: str, cwrite_dir: str, cfg: str,
            bench_args: str = "") -> str:
    bench_args = bench_args or f"--config {cfg} --no-cpu-baseline --steps 2 --warmup 1 --reps 2"
    copy_kib = 1024.0 * 1024.0  # bench.py --copy-calibration copies 1 GiB
    ff = copy_kib / copy_counter(cfetch_dir, "FETCH_SIZE")
    wf = copy_kib / copy_counter(cwrite_dir, "WRITE_SIZE")
    fetch = counter_means(fetch_dir, "FETCH_SIZE")
    write = counter_means(write_dir, "WRITE_SIZE")
    lines = [
        f"# HBM traffic per launch -- {_label(cfg)} ({WORKLOADS.get(str(cfg), '?')}), MI355X",
        "#",
        "# commands (repo root, GPU box), one counter per pass:",
        f"#   rocprofv3 --pmc FETCH_SIZE -d {fetch_dir} -o f -- python3 -u bench.py {bench_args}",
        f"#   rocprofv3 --pmc WRITE_SIZE -d {write_dir} -o w -- python3 -u bench.py {bench_args}",
        "# calibration: the same counters on bench.py --copy-calibration (1 GiB device copies):",
        f"#   rocprofv3 --pmc FETCH_SIZE -d {cfetch_dir} -o cf -- python3 -u bench.py --copy-calibration",
        f"#   rocprofv3 --pmc WRITE_SIZE -d {cwrite_dir} -o cw -- python3 -u bench.py --copy-calibration",
        f"# copy of {copy_kib:.0f} KiB: factors fetch {ff:.4f}, write {wf:.4f}",
        "# traffic_bytes = (FETCH_SIZE * fetch_factor + WRITE_SIZE * write_factor) * 1024, mean per dispatch",
        "",
        f"fetch_factor={ff:.4f}",
        f"write_factor={wf:.4f}",
    ]
    for k in sorted(fetch, key=lambda k: -fetch[k]):
        w = write.get(k, 0.0)
        tb = (fetch[k] * ff + w * wf) * 1024
        lines.append(f"{k}: fetch_kib={fetch[k]:.1f} write_kib={w:.1f} traffic_bytes={tb:.0f}")
    return "\n".join(lines) + "\n"


INST_COUNTERS = ["SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_INSTS_SALU",
                 "SQ_INSTS_VALU_TRANS_F32", "SQ_INSTS_VMEM", "SQ_VALU_MFMA_BUSY_CYCLES",
                 "SQ_BUSY_CYCLES"]


SIMDS = 1024          # MI355X: 256 CUs x 4 SIMDs
CLOCK_HZ = 2.4e9      # peak engine clock (the dense-peak figure uses the same)


def insts(sq_dir: str, kt_dir: str, cfg: str, bench_args: str = "") -> str:
    bench_args = bench_args or f"--config {cfg} --no-cpu-baseline --steps 2 --warmup 1 --reps 2"
    means = {c: counter_means(sq_dir, c) for c in INST_COUNTERS}
    durs = {k: statistics.mean(v) for k, v in kernel_durations(kt_dir).items()}
    lines = [
        f"# SQ instruction counters per dispatch -- {_label(cfg)} ({WORKLOADS.get(str(cfg), '?')}), MI355X",
        "#",
        "# command (repo root, GPU box), one pass:",
        f"#   rocprofv3 --pmc {' '.join(INST_COUNTERS)} -d {sq_dir} -o sq -- \\",
        f"#       python3 -u bench.py {bench_args}",
        "# instructions issued per MFMA: SQ_INSTS_VALU as counted (whether it includes the",
        "# MFMA instructions themselves is not separated here), transcendental VALU, LDS,",
        "# SALU and vector-memory instructions; MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES summed",
        "# over the dispatch; busy frac = that / (1024 SIMDs x 2.4 GHz x the kernel's mean",
        f"# duration in the kernel-trace run {kt_dir} of the same session).",
        "",
        f"{'kernel':28s} {'MFMA':>10s} {'VALU/MFMA':>10s} {'TRANS/MFMA':>11s} {'LDS/MFMA':>9s} "
        f"{'SALU/MFMA':>10s} {'VMEM/MFMA':>10s} {'MFMA busy':>12s} {'mean us':>9s} {'busy frac':>9s}",
    ]
    fracs = {}
    kernels = sorted(means["SQ_INSTS_MFMA"], key=lambda k: -means["SQ_INSTS_MFMA"][k])
    for k in kernels:
        mf = means["SQ_INSTS_MFMA"].get(k, 0.0)
        if mf <= 0:
            continue
        g = lambda c: means[c].get(k, 0.0) / mf
        lines.append(f"{k:28s} {mf:10.0f} {g('SQ_INSTS_VALU'):10.2f} "
                     f"{g('SQ_INSTS_VALU_TRANS_F32'):11.2f} {g('SQ_INSTS_LDS'):9.2f} "
                     f"{g('SQ_INSTS_SALU'):10.2f} {g('SQ_INSTS_VMEM'):10.2f} "
                     f"{means['SQ_VALU_MFMA_BUSY_CYCLES'].get(k, 0.0):12.0f} "
                     f"{durs.get(k, float('nan')):9.1f} {_busy_frac(means, durs, k):9.4f}")
        if k in durs:
            fracs[k] = _busy_frac(means, durs, k)
    lines.append("")
    for k, f in fracs.items():
        lines.append(f"mfma_busy {k}={f:.4f}")
    return "\n".join(lines) + "\n"


def _busy_frac(means, durs, k) -> float:
    d = durs.get(k)
    if not d:
        return float("nan")
    return means["SQ_VALU_MFMA_BUSY_CYCLES"].get(k, 0.0) / (SIMDS * CLOCK_HZ * d * 1e-6)


def read_mfma_busy(path: str) -> Dict[str, float]:
    """The `mfma_busy <kernel>=<frac>` lines of an `insts` summary."""
    out: Dict[str, float] = {}
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("mfma_busy "):
                    k, v = line[len("mfma_busy "):].strip().split("=")
                    out[k] = float(v)
    except FileNotFoundError:
        pass
    return out


def read_mfma_counts(path: str) -> Dict[str, int]:
    """MFMA instructions per dispatch, per kernel, from the table of an
    `insts` summary (the first two columns: kernel, MFMA)."""
    out: Dict[str, int] = {}
    try:
        with open(path) as f:
            for line in f:
                tok = line.split()
                if len(tok) >= 2 and not line.startswith("#") and tok[1].isdigit():
                    out[tok[0]] = int(tok[1])
    except FileNotFoundError:
        pass
    return out


def main(argv: List[str]) -> None:
    if len(argv) >= 4 and argv[0] == "trace":
        sys.stdout.write(trace(argv[1], argv[2], argv[3], " ".join(argv[4:])))
    elif len(argv) >= 4 and argv[0] == "insts":
        sys.stdout.write(insts(argv[1], argv[2], argv[3], " ".join(argv[4:])))
    elif len(argv) >= 6 and argv[0] == "traffic":
        sys.stdout.write(traffic(argv[1], argv[2], argv[3], argv[4], argv[5], " ".join(argv[6:])))
    else:
        raise SystemExit(__doc__)


if __name__ == "__main__":
    main(sys.argv[1:])
