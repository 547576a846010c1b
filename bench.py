"""Decode-throughput benchmark of the MI355X plane-codec path.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]``

One "step" restores one batch of synthetic tensors from their compressed
planes, resident in HBM, through the library's tensor-level entry point
(``ptwm_hardware_backend_v1_dispatch_decode_cuda``).  Prints one JSON line
(the driver's contract) with ``roofline`` (dominant kernel, HIP-event
timing on the library stream) and ``cpu_baseline`` (the C restatement of
the reference CPU decoder on a bounded sample, timed on this host).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_bf16(shape, seed, std=0.02):
    import torch

    g = torch.Generator(device="cuda:0").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda:0") * std).to(torch.bfloat16)


class Workload:
    """Compressed tensors in HBM plus their decode plan."""

    def __init__(self, name, blob, plan_bytes, out_len, comp_bytes, restored, codecs, check):
        self.name, self.blob, self.plan_bytes = name, blob, plan_bytes
        self.out_len, self.comp_bytes, self.restored = out_len, comp_bytes, restored
        self.codecs, self.check = codecs, check


def build_identity_bf16(total_bytes: int) -> Workload:
    """bf16 tensors with Identity-coded planes: decode = fused inverse chain
    (merge + bit revert) only.  Planes come from the library's own split."""
    import torch

    from ptwm_amd import api, plan

    rows = total_bytes // (4096 * 2)
    x = make_bf16((rows, 4096), 11)
    raw = x.view(torch.uint8).reshape(-1)
    n = raw.numel() // 2
    blob = torch.empty(2 * n, dtype=torch.uint8, device="cuda:0")
    api.split_cuda(plan.CHAIN_IEEE16_SPLIT2, raw, [blob[:n], blob[n:]])
    t = plan.TensorPlan(plan.CHAIN_IEEE16_SPLIT2, 0, raw.numel(), [
        plan.PlanePlan(0, 0, n, n), plan.PlanePlan(0, n, n, n)])
    return Workload(f"bf16 {rows}x4096 N(0,0.02), split2, identity planes (inverse chain only)", blob,
                    plan.encode_plan([t]), raw.numel(), blob.numel(), raw.numel(), "identity", raw)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="identity_bf16")
    ap.add_argument("--size-mb", type=int, default=2048)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import ctypes as C

    import torch

    from ptwm_amd import api, ids
    from ptwm_amd._native import lib

    log(f"[bench] building workload {args.workload}")
    wl = build_identity_bf16(args.size_mb << 20)
    out = torch.empty(wl.out_len, dtype=torch.uint8, device="cuda:0")
    L = lib()

    def step():
        return api.hardware_backend_dispatch_decode_cuda(ids.HARDWARE_BACKEND_LABEL, ids.DECODE_PLAN_LABEL,
                                                         wl.plan_bytes, wl.blob, out, 0)

    log("[bench] warmup")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ok = bool(torch.equal(out, wl.check))
    log(f"[bench] bit-exact check: {ok}")
    if not ok:
        raise SystemExit("decode mismatch")

    L.ptwm_mi355x_set_profiling(0, 1)
    ms = (C.c_float * 3)()
    kern_ms = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
        L.ptwm_mi355x_last_kernel_ms(0, ms)
        kern_ms.append((ms[0], ms[1], ms[2]))
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    L.ptwm_mi355x_set_profiling(0, 0)
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    value = wl.restored / (ms_per_step * 1e-3) / 1e9
    merge_ms = sum(k[1] for k in kern_ms) / len(kern_ms)
    traffic = wl.comp_bytes + wl.restored
    achieved = traffic / (merge_ms * 1e-3) / 1e9
    res = {
        "metric": "decode GB/s (restored bytes) per MI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded torch.randn on device)",
        "config": {"workload": wl.name, "restored_bytes": wl.restored, "compressed_bytes": wl.comp_bytes,
                   "codecs": wl.codecs, "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "kernel": "merge_ieee16_kernel", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "kernel_ms": round(merge_ms, 4), "traffic": None},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res), flush=True)


def cpu_baseline():
    """The oracle's inverse chain (C restatement of fusion.rs:127-194) on a
    bounded sample, single thread, on this host."""
    import numpy as np

    import oracle as O

    n = 128 << 20
    rng = np.random.default_rng(0)
    p0 = rng.integers(0, 256, n // 2, dtype=np.uint8).tobytes()
    p1 = rng.integers(0, 256, n // 2, dtype=np.uint8).tobytes()
    t0 = time.perf_counter()
    reps = 0
    while True:
        O.chain_inverse(O.CHAIN_IEEE16_SPLIT2, [p0, p1])
        reps += 1
        if time.perf_counter() - t0 > 3.0:
            break
    dt = time.perf_counter() - t0
    return {"value": round(n * reps / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{reps} x 128 MiB bf16 inverse chain (identity planes), oracle C restatement"}


if __name__ == "__main__":
    main()
