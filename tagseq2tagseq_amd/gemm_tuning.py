"""Tuned GEMM selections for the library products of the training step.

The layers' and the head's plain products (qkv / out / gate_up / down
projections and the tied head, forward and both gradients) run in hipBLASLt /
rocBLAS through torch.  torch's TunableOp can time every candidate kernel of
both libraries for each product shape once and keep the fastest; the
selections for the configs[4] step (T = 16384, d 768, H 12, hidden 2048,
vocabulary 50257 padded to 50264) on MI355X are committed in
``gemm_tuning_gfx950.csv`` next to this file, together with the validators
TunableOp checks before it uses them (torch, HIP, hipBLASLt and rocBLAS
versions, GPU architecture): on any other software stack the file is refused
and the default heuristics run.

    use_tuned_gemms()          # before the first product: load, never tune
    python -m tagseq2tagseq_amd.gemm_tuning --out FILE
                               # re-tune on this box (about two minutes)
"""
from __future__ import annotations

import argparse
import os
import tempfile

import torch

TUNED_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_tuning_gfx950.csv")


def use_tuned_gemms(path: str = TUNED_FILE) -> bool:
    """Enable TunableOp with tuning off and the selections of `path`; True
    when the file was read and its validators match this stack."""
    if not (torch.cuda.is_available() and os.path.exists(path)):
        return False
    tun = torch.cuda.tunable
    # results are never written back over the committed file
    tun.set_filename(os.path.join(tempfile.gettempdir(), f"t2t_tunableop_{os.getpid()}.csv"))
    tun.enable(True)
    tun.tuning_enable(False)
    ok = bool(tun.read_file(path))
    if not ok:
        tun.enable(False)
    return ok


def tune(step, path: str, steps: int = 2, max_ms: int = 30) -> int:
    """Run `step` with tuning on and write the selections to `path`; returns
    the number of tuned product shapes."""
    tun = torch.cuda.tunable
    tun.set_filename(path)
    tun.set_max_tuning_duration(max_ms)
    tun.enable(True)
    tun.tuning_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    tun.tuning_enable(False)
    n = len(tun.get_results())
    # TunableOp writes the file when the process ends
    return n


def _main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", required=True)
    args = ap.parse_args()
    from .train_step import configs4_step
    step = configs4_step(torch.device("cuda:0"), seed=0)
    print(f"{tune(step, args.out)} product shapes tuned -> {args.out} (written at exit)")


if __name__ == "__main__":
    _main()
