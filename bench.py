"""Benchmark of the SunnyNet token loop on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload scan]

Workload (the headline): the standalone gated prefill scan, B=16, D=2048
channels, T=4096, fp32, inputs resident in HBM (``sunnynet_amd.workloads``).
A step is one full scan. ``value`` is algorithmic HBM GB/s (read a and b,
write s: 3*B*T*D*4 bytes per step) over the K timed steps. The ``roofline``
object times each launch with HIP events on the stream the kernel runs on;
``cpu_baseline`` times the reference C runtime's ``sn_recur_scan`` (built
from the reference sources into oracle/_ref) on the host cores on the same
inputs.

Prints exactly one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from sunnynet_amd import runtime  # noqa: E402
from sunnynet_amd.workloads import SCAN_B, SCAN_D, SCAN_T, scan_bytes, scan_inputs  # noqa: E402

HBM_PEAK_GBS = 8000.0
# HBM bytes per scan launch on this workload from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE, each scaled by the counter's reading for a plain copy of known
# size (FETCH x2.0, WRITE x1.0): profiles/scan_gated_B16_D2048_T4096.md.
SCAN_TRAFFIC_BYTES = 1_611_150_336
METRIC = "decode tok/s @B=1,B=64 (SunnyNet-100M); gated-scan HBM GB/s % of peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def physical_cores() -> int:
    try:
        seen = set()
        phys = core = None
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("physical id"):
                    phys = line.split(":")[1].strip()
                elif line.startswith("core id"):
                    core = line.split(":")[1].strip()
                elif not line.strip():
                    if core is not None:
                        seen.add((phys, core))
                    phys = core = None
        n = len(seen)
    except OSError:
        n = 0
    return n or (os.cpu_count() or 1)


def bench_scan(steps: int, warmup: int, cpu: bool):
    dev = torch.device("cuda:0")
    B, T, D = SCAN_B, SCAN_T, SCAN_D
    log(f"[bench] generating scan inputs B={B} T={T} D={D}")
    a, b, s0 = scan_inputs(B, T, D, gated=True)
    da, db, d0 = (torch.from_numpy(x).to(dev) for x in (a, b, s0))
    torch.cuda.synchronize()
    for _ in range(warmup):
        runtime.scan(da, db, d0, gated=True)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1 in evs:
        e0.record(stream)
        runtime.scan(da, db, d0, gated=True)
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = [e0.elapsed_time(e1) for e0, e1 in evs]
    nbytes = scan_bytes(B, T, D)
    value = nbytes * steps / wall / 1e9
    avg_ms = float(np.mean(kern_ms))
    achieved = nbytes / (avg_ms * 1e-3) / 1e9
    log(f"[bench] scan: wall {wall*1e3/steps:.3f} ms/step, kernel avg {avg_ms*1e3:.1f} us "
        f"(min {min(kern_ms)*1e3:.1f}), {achieved:.1f} GB/s")
    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "ms_per_step": round(wall * 1e3 / steps, 4),
        "dtype": "f32",
        "config": {"workload": f"gated scan B={B} D={D} T={T} fp32 (bit-exact vs reference)",
                   "B": B, "D": D, "T": T, "bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": SCAN_TRAFFIC_BYTES, "kernel": "k_recur_scan_buf",
                     "kernel_avg_us": round(avg_ms * 1e3, 2)},
    }
    if cpu:
        res["cpu_baseline"] = cpu_scan_baseline(a, b, s0)
    return res


def cpu_scan_baseline(a, b, s0):
    """Reference sn_recur_scan on host cores; falls back to the oracle port."""
    import oracle
    B, T, D = a.shape
    out = np.empty_like(a)
    send = np.empty_like(s0)
    f = oracle._f
    threads = min(16, physical_cores(), B)
    if oracle.ref_available():
        lib = oracle.ref_lib("recur")
        lib.sn_set_threads(threads)
        run = lambda: lib.sn_recur_scan(f(a), f(b), f(s0), f(out), f(send), B, T, D, 1)
        kind = "reference"
    else:
        run = lambda: oracle.load().orc_recur_scan(f(a), f(b), f(s0), f(out), f(send), B, T, D, 1)
        kind = "port"
        os.environ["OMP_NUM_THREADS"] = str(threads)
    run()
    times = []
    deadline = time.perf_counter() + 15.0
    while len(times) < 5 and time.perf_counter() < deadline:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    gbs = scan_bytes(B, T, D) / med / 1e9
    log(f"[bench] cpu {kind} sn_recur_scan: {med*1e3:.1f} ms, {gbs:.2f} GB/s, {threads} threads")
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": f"full workload B={B} D={D} T={T}, median of {len(times)} runs "
                      f"({med*1e3:.1f} ms each)"}


def pmc_probe():
    """A short fixed sequence for `rocprofv3 --pmc` runs: 3 scans of the
    workload, then 3 plain device copies of one 537 MB input array (the copy
    calibrates FETCH_SIZE / WRITE_SIZE against a known byte count)."""
    dev = torch.device("cuda:0")
    a, b, s0 = scan_inputs(SCAN_B, SCAN_T, SCAN_D, gated=True)
    da, db, d0 = (torch.from_numpy(x).to(dev) for x in (a, b, s0))
    for _ in range(3):
        runtime.scan(da, db, d0, gated=True)
    y = torch.empty_like(da)
    for _ in range(3):
        y.copy_(da)
    torch.cuda.synchronize()
    log(f"[pmc] scan bytes/launch {scan_bytes(SCAN_B, SCAN_T, SCAN_D)}; copy bytes/launch "
        f"read {da.numel() * 4} write {da.numel() * 4}")
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="scan", choices=["scan"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run the fixed launch sequence used for rocprofv3 --pmc and exit")
    args = ap.parse_args(argv)
    if args.pmc_probe:
        return pmc_probe()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        log("bench.py measures one GPU only: this build has no multi-GPU path "
            "(each channel / sequence shards with no communication; see DESIGN.md).")
        return 2
    res = bench_scan(args.steps, args.warmup, cpu=not args.no_cpu)
    line = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": res["dtype"], "data": "synthetic (seeded numpy PCG64)",
            "config": res["config"], "roofline": res["roofline"]}
    if "cpu_baseline" in res:
        line["cpu_baseline"] = res["cpu_baseline"]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
