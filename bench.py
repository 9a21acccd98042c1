"""Benchmark of the SunnyNet token loop on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|scan|core|decode]

Headline (``value``): the standalone gated prefill scan, B=16, D=2048
channels, T=4096, fp32, inputs resident in HBM (``sunnynet_amd.workloads``).
A step is one full scan; ``value`` is algorithmic HBM GB/s (read a and b,
write s: 3*B*T*D*4 bytes per step) over the K timed steps. ``roofline``
times each launch with HIP events on the stream the kernel runs on;
``cpu_baseline`` times the reference C runtime's ``sn_recur_scan`` (built
from the reference sources into oracle/_ref) on host cores, same inputs.

``core`` (same JSON line): the fused block core (compete gate + decay gate +
gated scan, core_avx2.c:34-149) forward and backward on the same B, T, D
(q is (B,T,2D)), each launch timed with HIP events, HBM roofline of its
algorithmic bytes, the reference core_fwd_f32 / core_bwd_f32 beside them.

``decode`` (same JSON line): SunnyNet-100M (L=12, D=1024, V=32000, seed-1
random init), chunked prefill of a T=1024 random prompt, then 256 greedy
steps on the device at B=1 and B=64, fp32; and the same shape with INT4 g32
weights (matmuls ~ N(0, 0.02)) after a T=2048 prefill at B=1, 8, 32. Each
case gives tokens/s, us/step and a ``roofline`` of the step (HBM bytes for
the weight-streaming cases; fp32 MFMA flops for fp32 B=64 and INT4 B=32).
CPU legs: the reference ``sn_step`` (fp32 B=1), the fp32 torch
``forward_step`` restatement at B=64 (the reference has no batched C step),
and the reference ``sn_gemv_i4`` over one step's INT4 matrices.
``decode.small``: SunnyNet small (seed 0), prefill 256 then 64 greedy steps
at B=1, with the reference ``sn_prefill`` / ``sn_step`` beside it.
``decode.rwkv7``: the RWKV-7 configuration (12 layers, D=768, vocab 65536,
INT4 g32), 512-token prompt, 128 greedy steps at B=1 and B=64, with the
reference ``sn_rk_step`` timed on its INT4 blob. Every CPU leg states the
host's sockets, physical cores and logical CPUs.

Modes that run a fixed sequence and exit: ``--pmc-probe [scan|decode]`` (for
``rocprofv3 --pmc`` counter runs), ``--profile b1|batch|rwkv|small`` (for
``rocprofv3 --kernel-trace`` summaries of the decode paths) and
``--hbm-probe`` (the bandwidth plain streaming kernels reach over the scan's
byte pattern, beside the nominal peak; one JSON line).

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
from sunnynet_amd.config import SUNNY_100M, matmul_params  # noqa: E402

HBM_PEAK_GBS = 8000.0
# HBM bytes per scan launch on this workload from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE, each scaled by the counter's reading for a plain copy of known
# size (FETCH x2.0, WRITE x1.0): profiles/scan_gated_B16_D2048_T4096.md.
SCAN_TRAFFIC_BYTES = 1_611_150_336
# HBM bytes per decode step, by (weights, B), from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE over the dispatches of one greedy call of `bench.py --pmc-probe
# decode`, calibrated like the scan's and divided by the call's steps. Filled
# from the tables of profiles/decode_pmc_traffic.md.
DECODE_TRAFFIC: dict = {
    ("int4", 1): 96_525_699, ("int4", 8): 155_992_914, ("int4", 32): 174_590_113,
    ("fp32", 1): 517_375_353, ("fp32", 64): 627_634_736, ("fp16", 1): 285_576_898,
    ("small", 1): 1_386_042, ("rwkv7-exact", 1): 457_100_727, ("rwkv7", 64): 1_047_303_436,
    ("rwkv7-persist", 1): 149_502_529,
}
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


def host_cpu() -> dict:
    """The host's CPU counts (lscpu's sockets / cores / logical CPUs), read
    from /proc/cpuinfo, for every CPU baseline."""
    sockets, model = set(), ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("physical id"):
                    sockets.add(line.split(":")[1].strip())
                elif line.startswith("model name") and not model:
                    model = line.split(":", 1)[1].strip()
    except OSError:
        pass
    return {"sockets": len(sockets) or 1, "physical_cores": physical_cores(),
            "logical_cpus": os.cpu_count() or 1, "model": model}


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
    # The timed region: K scans back to back, nothing else on the stream,
    # bracketed by HIP events on the kernel's stream (the launches' average
    # duration behind the roofline figure) inside the host wall clock.
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        runtime.scan(da, db, d0, gated=True)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    avg_ms = ev0.elapsed_time(ev1) / steps
    # Then K more, each alone between two HIP events (each launch then also
    # pays the event records around it): the spread of single launches.
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for e0, e1 in evs:
        e0.record(stream)
        runtime.scan(da, db, d0, gated=True)
        e1.record(stream)
    torch.cuda.synchronize()
    kern_ms = [e0.elapsed_time(e1) for e0, e1 in evs]
    nbytes = scan_bytes(B, T, D)
    value = nbytes * steps / wall / 1e9
    achieved = nbytes / (avg_ms * 1e-3) / 1e9
    log(f"[bench] scan: wall {wall*1e3/steps:.3f} ms/step, timed-region events {avg_ms*1e3:.1f} us/launch, "
        f"{achieved:.1f} GB/s; single launches avg {np.mean(kern_ms)*1e3:.1f} (min {min(kern_ms)*1e3:.1f}) us")
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
                     "kernel_avg_us": round(avg_ms * 1e3, 2),
                     "single_launch_avg_us": round(float(np.mean(kern_ms)) * 1e3, 2)},
    }
    if cpu:
        res["cpu_baseline"] = cpu_scan_baseline(a, b, s0)
    res["host_pointer_abi"] = bench_scan_host_abi(a, b, s0)
    res["scan_bwd"] = bench_scan_bwd(da, db, d0, steps, warmup, cpu)
    return res


def bench_scan_host_abi(a, b, s0, reps: int = 3):
    """The stable ABI's host-pointer scan (snhip_abi_recur_scan, the entry a
    caller of the reference's sn_abi_recur_scan binds, sn_abi.c:63-71) on the
    same host arrays: device buffers, the copies in, the scan and the copies
    out, PCIe included. A reported figure beside the device-resident
    headline, never the headline."""
    from sunnynet_amd import _native
    L = _native.lib()
    B, T, N = a.shape
    out = np.empty_like(a)
    send = np.empty_like(s0)
    f = lambda x: x.ctypes.data

    def call():
        _native.check(L.snhip_abi_recur_scan(f(a), f(b), f(s0), f(out), f(send), B, T, N, 1),
                      "snhip_abi_recur_scan")
    call()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        call()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    nbytes = scan_bytes(B, T, N)
    log(f"[bench] host-pointer ABI scan: {med*1e3:.1f} ms/call, {nbytes/med/1e9:.1f} GB/s (PCIe included)")
    return {"entry": "snhip_abi_recur_scan", "ms_per_call": round(med * 1e3, 2),
            "GB/s": round(nbytes / med / 1e9, 2),
            "note": f"host numpy arrays in and out (pageable), median of {reps} calls; includes "
                    "device allocation and the PCIe copies; the headline is device-resident"}


def bench_scan_bwd(dp_, dnu_, ds0_, steps, warmup, cpu):
    """The gated scan's backward (scan_avx2.c:50-99) on the same workload:
    read p, nu, the forward states and dout, write dp and dnu (6 x B*T*D*4
    bytes per launch), timed per launch with HIP events on the kernel's
    stream; the reference scan_bwd_f32 (single-threaded, as it ships) on the
    same arrays beside it."""
    B, T, D = dp_.shape
    out, _ = runtime.scan(dp_, dnu_, ds0_, gated=True)
    g = torch.Generator(device="cpu").manual_seed(2)
    dout = torch.randn(B, T, D, generator=g).to(dp_.device)
    for _ in range(warmup):
        runtime.scan_bwd(dp_, dnu_, ds0_, out, dout)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dp_.device)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for e0, e1 in evs:
        e0.record(stream)
        runtime.scan_bwd(dp_, dnu_, ds0_, out, dout)
        e1.record(stream)
    torch.cuda.synchronize()
    avg_ms = float(np.mean([e0.elapsed_time(e1) for e0, e1 in evs]))
    nbytes = 6 * B * T * D * 4 + 2 * B * D * 4
    gbs = nbytes / (avg_ms * 1e-3) / 1e9
    log(f"[bench] scan_bwd: kernel avg {avg_ms*1e3:.1f} us, {gbs:.1f} GB/s")
    res = {"kernel": "k_scan_bwd_buf", "kernel_avg_us": round(avg_ms * 1e3, 2),
           "bytes_per_launch": nbytes,
           "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    if cpu:
        import oracle
        if oracle.ref_available():
            hp = [x.cpu().numpy() for x in (dp_, dnu_, ds0_, out, dout)]
            o = [np.empty_like(hp[0]), np.empty_like(hp[0]), np.empty_like(hp[2])]
            f = oracle._f
            lib = oracle.ref_lib("scan")
            t0 = time.perf_counter()
            lib.scan_bwd_f32(f(hp[0]), f(hp[1]), f(hp[2]), f(hp[3]), f(hp[4]), f(o[0]), f(o[1]),
                             f(o[2]), B, T, D)
            sec = time.perf_counter() - t0
            log(f"[bench] cpu reference scan_bwd_f32: {sec*1e3:.1f} ms, {nbytes/sec/1e9:.2f} GB/s")
            res["cpu_baseline"] = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1,
                                   "kind": "reference",
                                   "sample": f"full workload B={B} D={D} T={T}, one run "
                                             f"({sec*1e3:.0f} ms; scan_bwd_f32 is single-threaded)"}
    return res


def _event_avg_ms(fn, steps, stream):
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for e0, e1 in evs:
        e0.record(stream)
        fn()
        e1.record(stream)
    torch.cuda.synchronize()
    return float(np.mean([e0.elapsed_time(e1) for e0, e1 in evs]))


def bench_core(steps, warmup, cpu, B=SCAN_B, T=SCAN_T, D=SCAN_D):
    """The fused block core (core_avx2.c:34-149) on the scan's workload shape:
    q (B,T,2D), D channels. Forward reads q and writes states, u, p (20 bytes
    per channel-step); backward reads q, u, p, the previous states, dstate,
    du_in and writes dq (36 bytes per channel-step). Each launch is timed with
    HIP events on the kernel's stream; the reference core_fwd_f32 /
    core_bwd_f32 on host cores beside them on a T/16 slice."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(9)
    q = torch.randn(B, T, 2 * D, generator=g, device=dev) * 0.6
    delta = 0.01 + 0.4 * torch.rand(D, generator=g, device=dev)
    s0 = torch.randn(B, D, generator=g, device=dev) * 0.1
    dstate = torch.randn(B, T, D, generator=g, device=dev)
    du_in = torch.randn(B, T, D, generator=g, device=dev)
    fwd = runtime.core_fwd(q, delta, s0)
    for _ in range(warmup):
        runtime.core_fwd(q, delta, s0)
        runtime.core_bwd(q, delta, s0, *fwd, dstate, du_in)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    fms = _event_avg_ms(lambda: runtime.core_fwd(q, delta, s0), steps, stream)
    bms = _event_avg_ms(lambda: runtime.core_bwd(q, delta, s0, *fwd, dstate, du_in), steps, stream)
    n = B * T * D
    fbytes, bbytes = 20 * n + 8 * B * D + 4 * D, 36 * n + 12 * B * D + 8 * D
    fg, bg = fbytes / (fms * 1e-3) / 1e9, bbytes / (bms * 1e-3) / 1e9
    log(f"[bench] core fwd: {fms*1e3:.1f} us, {fg:.1f} GB/s; bwd: {bms*1e3:.1f} us, {bg:.1f} GB/s")
    res = {"workload": f"fused core B={B} D={D} T={T} fp32",
           "fwd": {"kernel": "k_core_fwd_buf", "kernel_avg_us": round(fms * 1e3, 2), "bytes_per_launch": fbytes,
                   "roofline": {"bound": "hbm", "achieved": round(fg, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(fg / HBM_PEAK_GBS, 4)}},
           "bwd": {"kernel": "k_core_bwd_buf", "kernel_avg_us": round(bms * 1e3, 2), "bytes_per_launch": bbytes,
                   "roofline": {"bound": "hbm", "achieved": round(bg, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(bg / HBM_PEAK_GBS, 4)}}}
    if cpu:
        import oracle
        if oracle.ref_available():
            Ts = T // 16
            hq = q[:, :Ts].cpu().numpy().copy()
            hd, hs = delta.cpu().numpy(), s0.cpu().numpy()
            hds, hdu = dstate[:, :Ts].cpu().numpy().copy(), du_in[:, :Ts].cpu().numpy().copy()
            st, u, p = (np.empty((B, Ts, D), np.float32) for _ in range(3))
            dq, dd, ds0 = np.empty_like(hq), np.zeros(D, np.float32), np.empty_like(hs)
            f = oracle._f
            lib = oracle.ref_lib("core")
            threads = min(16, physical_cores())
            lib.sn_set_threads(threads)
            t0 = time.perf_counter()
            lib.core_fwd_f32(f(hq), f(hd), f(hs), f(st), f(u), f(p), B, Ts, D)
            t1 = time.perf_counter()
            lib.core_bwd_f32(f(hq), f(hd), f(hs), f(st), f(u), f(p), f(hds), f(hdu), f(dq), f(dd), f(ds0),
                             B, Ts, D)
            t2 = time.perf_counter()
            ns = B * Ts * D
            cf, cb = (20 * ns) / (t1 - t0) / 1e9, (36 * ns) / (t2 - t1) / 1e9
            log(f"[bench] cpu reference core_fwd_f32 {cf:.2f} GB/s, core_bwd_f32 {cb:.2f} GB/s, {threads} threads")
            smp = f"B={B} D={D} T={Ts} (a T/16 slice), one run each"
            res["fwd"]["cpu_baseline"] = {"value": round(cf, 3), "unit": "GB/s", "cores": threads, "host": host_cpu(),
                                          "kind": "reference", "sample": smp}
            res["bwd"]["cpu_baseline"] = {"value": round(cb, 3), "unit": "GB/s", "cores": threads, "host": host_cpu(),
                                          "kind": "reference", "sample": smp}
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
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "host": host_cpu(), "kind": kind,
            "sample": f"full workload B={B} D={D} T={T}, median of {len(times)} runs "
                      f"({med*1e3:.1f} ms each)"}


def decode_bytes(cfg, fmt: str, block: int = 32) -> int:
    """Weight bytes one decode step must read: every matmul and the head
    (fp32: 4 B per weight; fp16: 2 B; INT4: 0.5 B + one fp32 scale per group)."""
    n = matmul_params(cfg)
    if fmt == "int4":
        return int(n // 2 + (n // block) * 4)
    return int(n * (2 if fmt == "fp16" else 4))


def decode_step_bytes(cfg, fmt: str, B: int) -> int:
    """Algorithmic HBM bytes of one decode step: the weights, the per-layer
    vectors (norm gains and centres, conv taps, delta; 4 B each) and per
    sequence the embedding row, the state and history read and written, and
    the logits written."""
    D, I, K, L, V = cfg.dim, cfg.inner, cfg.taps, cfg.layers, cfg.vocab_size
    small = (L * (2 * D + 2 * I + K * D + D) + 2 * D) * 4
    per_seq = D * 4 + 2 * L * K * D * 4 + V * 4
    return decode_bytes(cfg, fmt) + small + B * per_seq


FP32_MFMA_TFLOPS = 157.3


def step_roofline(nbytes: int, flops: int, us_per_step: float, kernel: str, traffic) -> dict:
    """Roofline of a decode step from its measured time, against whichever
    floor is higher: its algorithmic HBM bytes at 8 TB/s or its fp32 matrix
    flops at the fp32 MFMA peak (the products run as fp32 MFMA or FMA on
    dequantized weights). The other floor's fraction is kept beside it.
    ``traffic``: HBM bytes per step measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, calibrated), or None."""
    sec = us_per_step * 1e-6
    hbm_floor_us = nbytes / (HBM_PEAK_GBS * 1e9) * 1e6
    mfma_floor_us = flops / (FP32_MFMA_TFLOPS * 1e12) * 1e6
    gbs = nbytes / sec / 1e9
    tfs = flops / sec / 1e12
    if mfma_floor_us > hbm_floor_us:
        return {"bound": "mfma", "achieved": round(tfs, 2), "peak": FP32_MFMA_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tfs / FP32_MFMA_TFLOPS, 4), "traffic": traffic,
                "kernel": kernel, "flops_per_step": flops, "bytes_per_step": nbytes,
                "floor_us": round(mfma_floor_us, 2), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": kernel,
            "bytes_per_step": nbytes, "flops_per_step": flops, "floor_us": round(hbm_floor_us, 2),
            "mfma_frac": round(tfs / FP32_MFMA_TFLOPS, 4)}


def decode_roofline(cfg, fmt: str, B: int, us_per_step: float, kernel: str, traffic=None) -> dict:
    """SunnyNet decode step: 2 flops per matrix weight per sequence."""
    return step_roofline(decode_step_bytes(cfg, fmt, B), 2 * matmul_params(cfg) * B, us_per_step,
                         kernel, traffic)


def rwkv7_step_bytes(cfg, B: int) -> int:
    """Algorithmic HBM bytes of one RWKV-7 INT4 g32 decode step: the weights
    (0.5 B per weight and an fp32 scale per 32), and per sequence the 64 x 64
    head states read and written."""
    n = cfg.matmul_params()
    return n // 2 + (n // 32) * 4 + B * 2 * cfg.layers * cfg.n_head * cfg.head_size ** 2 * 4


def rwkv7_step_flops(cfg, B: int) -> int:
    """Matrix flops of one RWKV-7 decode step: 2 per matrix weight per
    sequence, plus the head-state update and read-out (about 6 flops per state
    entry: decay, rank-1 removal, k v write, S r) per sequence."""
    return 2 * cfg.matmul_params() * B + 6 * B * cfg.layers * cfg.n_head * cfg.head_size ** 2


def _time_ms(fn):
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def _write_blob(tmp, name, buf):
    path = os.path.join(tmp, name)
    with open(path, "wb") as f:
        f.write(buf)
    return path


def bench_decode_small(cpu: bool):
    """SunnyNet small (4 layers, D=256, I=384, R=128, V=4096, seed 0): a
    256-token random prompt through the chunked prefill, then 64 greedy steps
    on the device, B=1, fp32. Launch- and latency-bound: its 9.96 MB of weights
    stay in the caches. The reference ``sn_prefill`` + ``sn_step`` on the same
    blob beside it."""
    import tempfile

    from sunnynet_amd.blob import pack_sunny_blob
    from sunnynet_amd.config import SMALL
    from sunnynet_amd.runtime.model import HipModel
    from sunnynet_amd.weights import init_sunnynet
    cfg = SMALL
    dev = torch.device("cuda:0")
    tmp = tempfile.mkdtemp(prefix="snhip_bench_small_")
    path = _write_blob(tmp, "small.bin", pack_sunny_blob(init_sunnynet(cfg, 0)))
    prompt = torch.from_numpy(np.random.default_rng(256).integers(0, cfg.vocab_size, (1, 256))
                              .astype(np.int32)).to(dev)
    hm = HipModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers)
    tok = hm.prefill_batch(prompt).argmax(1).int()       # warm: prefill path and step graph
    hm.decode_greedy(tok, 8)
    hm.reset()
    torch.cuda.synchronize()
    lg = None

    def pre():
        nonlocal lg
        lg = hm.prefill_batch(prompt)
    pms = _time_ms(pre)
    tok = lg.argmax(1).int()
    n = 64
    ms = _time_ms(lambda: hm.decode_greedy(tok, n)) / n
    grid = hm.persistent_grid
    hm.close()
    us = ms * 1e3
    case = {"workload": "SunnyNet small B=1 fp32: prefill 256 then 64 greedy steps",
            "prefill_ms": round(pms, 3), "us_per_step": round(us, 2), "tok_s": round(1e3 / ms, 1),
            "roofline": decode_roofline(cfg, "fp32", 1, us, "k_decode_persist<0>" if grid else
                                        "per-kernel step", DECODE_TRAFFIC.get(("small", 1)))}
    case["roofline"]["bound"] = "latency"
    case["roofline"]["note"] = ("launch- and latency-bound: the step's 9.96 MB of weights stay in "
                                "L2/MALL; frac is against the HBM peak")
    log(f"[bench] decode small B=1: {case['us_per_step']} us/step, {case['tok_s']} tok/s, "
        f"prefill 256 {pms:.2f} ms")
    if cpu:
        case["cpu_baseline"] = cpu_decode_small_baseline(path, cfg, prompt.cpu().numpy()[0])
    return case


def cpu_decode_small_baseline(path, cfg, prompt):
    """The reference sn_prefill over the 256-token prompt, then 64 greedy
    sn_step calls, on host cores (the reference's OpenMP GEMVs)."""
    import oracle
    threads = min(16, physical_cores())
    if not oracle.ref_available():
        return {"value": None, "unit": "tok/s (B=1)", "cores": threads, "host": host_cpu(),
                "kind": "reference", "sample": "reference build absent"}
    oracle.ref_lib("model").sn_set_threads(threads)
    m = oracle.RefSnModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers)
    t0 = time.perf_counter()
    lg = m.prefill(prompt.tolist())
    pre = time.perf_counter() - t0
    times = []
    for _ in range(64):
        t = int(np.argmax(lg))
        t0 = time.perf_counter()
        lg = m.step(t)
        times.append(time.perf_counter() - t0)
    m.close()
    med = float(np.median(times))
    log(f"[bench] cpu reference sn_step small: {med*1e3:.3f} ms/token, prefill {pre*1e3:.1f} ms, "
        f"{threads} threads")
    return {"value": round(1.0 / med, 1), "unit": "tok/s (B=1)", "cores": threads, "host": host_cpu(),
            "kind": "reference", "ms_per_token": round(med * 1e3, 4), "prefill_ms": round(pre * 1e3, 2),
            "sample": "the whole workload: sn_prefill of the 256-token prompt, then the median of "
                      "64 greedy sn_step calls"}


def bench_decode(cpu: bool):
    import tempfile

    from sunnynet_amd.blob import pack_sunny_blob
    from sunnynet_amd.runtime.model import HipModel
    from sunnynet_amd.weights import gaussian_matmuls, init_sunnynet
    cfg = SUNNY_100M
    dev = torch.device("cuda:0")
    tmp = tempfile.mkdtemp(prefix="snhip_bench_")
    log("[bench] SunnyNet-100M weights (seed 1)")
    w = init_sunnynet(cfg, 1)
    p32 = _write_blob(tmp, "m100_fp32.bin", pack_sunny_blob(w))
    w4 = gaussian_matmuls(init_sunnynet(cfg, 1), seed=3)
    p4 = _write_blob(tmp, "m100_gauss.bin", pack_sunny_blob(w4))
    out = {"model": "SunnyNet-100M L=12 D=1024 I=1536 R=512 V=32000",
           "steps": 256, "cases": []}
    g = torch.Generator(device="cpu").manual_seed(123)
    for fmt, path, T, batches in (("fp32", p32, 1024, (1, 64)), ("fp16", p32, 1024, (1,)),
                                  ("int4", p4, 2048, (1, 8, 32))):
        for B in batches:
            hm = HipModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers,
                          max_batch=B, weights=fmt, block=32)
            prompts = torch.randint(0, cfg.vocab_size, (B, T), generator=g, dtype=torch.int32).to(dev)
            hm.prefill_batch(prompts[:, :32])          # warm the prefill graph-free path
            hm.reset()
            torch.cuda.synchronize()
            lg = None

            def pre():
                nonlocal lg
                lg = hm.prefill_batch(prompts)
            pms = _time_ms(pre)
            tok = lg.argmax(1).int()
            # prefill flops: the layers' products for every token (the head
            # runs on the last token only: 2 V D per sequence)
            layer_w = matmul_params(cfg) - cfg.vocab_size * cfg.dim
            pf_flops = 2 * layer_w * B * T + 2 * cfg.vocab_size * cfg.dim * B
            extra = {}
            if fmt == "fp32" and B == 64:
                # the reference's forward: logits at every position (B, T, V)
                st_s, st_h = hm.get_state(B)
                hm.reset()
                lall = None

                def pre_all():
                    nonlocal lall
                    lall = hm.prefill_all(prompts)
                ams = _time_ms(pre_all)
                all_flops = 2 * matmul_params(cfg) * B * T
                extra = {"prefill_all_ms": round(ams, 2),
                         "prefill_all_tflops": round(all_flops / ams / 1e9, 1),
                         "prefill_all_note": "every position's logits (B, T, V), the head GEMM over "
                                             "all B T rows included"}
                del lall
                hm.set_state(st_s, st_h)
                log(f"[bench] prefill fp32 B=64 T={T} with every position's logits: {ams:.1f} ms, "
                    f"{all_flops / ams / 1e9:.1f} TFLOP/s")
            hm.decode_greedy(tok, 8)                    # capture + warm the step graph
            torch.cuda.synchronize()
            n = out["steps"]
            ms = _time_ms(lambda: hm.decode_greedy(tok, n)) / n
            blk = {'int4': 32, 'fp16': 16}.get(fmt, 0)
            slices = hm.persistent_grid_for(B) if B > 1 else 0
            kernel = (f"k_decode_persist<{blk}> (the whole step)" if B == 1 and hm.persistent_grid else
                      f"k_decode_persist<{blk}> on {B} grid slices of {slices // B} workgroups "
                      f"(the whole step)" if slices else
                      "k_decode_batch (layers) + head GEMM + greedy argmax" if hm.batch_grid else
                      "per-kernel step")
            hm.close()
            us = ms * 1e3
            case = {"weights": fmt, "B": B, "prefill_T": T, "prefill_ms": round(pms, 2),
                    "prefill_tok_s": round(B * T / pms * 1e3, 1),
                    "prefill_tflops": round(pf_flops / pms / 1e9, 2), **extra,
                    "us_per_step": round(us, 2),
                    "tok_s": round(B / ms * 1e3, 1),
                    "roofline": decode_roofline(cfg, fmt, B, us, kernel,
                                                DECODE_TRAFFIC.get((fmt, B)))}
            log(f"[bench] decode {fmt} B={B}: {case['us_per_step']} us/step, {case['tok_s']} tok/s, "
                f"prefill T={T} {pms:.1f} ms, {case['roofline']['frac']:.4f} of {case['roofline']['bound']}")
            out["cases"].append(case)
    if cpu:
        out["cpu_baseline"] = cpu_decode_baseline(p32, cfg)
        out["cpu_baseline_f16"] = cpu_decode_baseline(p32, cfg, half=True)
        out["cpu_baseline_b64"] = cpu_decode_b64_baseline(w)
        out["cpu_baseline_int4_gemv"] = cpu_gemv_i4_baseline(w4)
    out["small"] = bench_decode_small(cpu)
    out["rwkv7"] = bench_rwkv7(cpu)
    return out


def cpu_decode_b64_baseline(w):
    """B=64 on host cores: the reference C runtime steps one sequence per
    handle, so the batched figure is the fp32 torch restatement of
    ``forward_step`` (the oracle, same operation sequence as the reference's
    torch path) at B=64 with one torch thread per physical core."""
    from oracle.torch_ref import TorchSunny
    threads = min(16, physical_cores())
    old = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        tr = TorchSunny(w, torch.float32)
        st = tr.init_state(64)
        idx = torch.from_numpy(np.random.default_rng(64).integers(0, w.cfg.vocab_size, 64))
        with torch.no_grad():
            _, st = tr.forward_step(idx, st)
            times = []
            deadline = time.perf_counter() + 15.0
            while len(times) < 8 and time.perf_counter() < deadline:
                t0 = time.perf_counter()
                _, st = tr.forward_step(idx, st)
                times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(old)
    med = float(np.median(times))
    log(f"[bench] cpu port forward_step B=64 fp32: {med*1e3:.1f} ms/step, {threads} threads")
    return {"value": round(64 / med, 1), "unit": "tok/s (B=64)", "cores": threads, "host": host_cpu(),
            "kind": "port", "ms_per_step": round(med * 1e3, 2),
            "sample": f"SunnyNet-100M fp32, torch forward_step restatement at B=64, one warm-up "
                      f"step then the median of {len(times)} steps"}


def cpu_gemv_i4_baseline(w4):
    """The reference's INT4 GEMV ``sn_gemv_i4`` (W4A8, group 32,
    quant.c:89-154, OpenMP over rows) over one decode step's matrices: per
    layer V, U, W_z, W_c, W_eff, then the head, quantized with the reference's
    ``sn_quant_i4``. There is no INT4 SunnyNet step in the reference, so this
    times the products alone."""
    import ctypes

    import oracle
    from sunnynet_amd.blob import layer_matrices
    threads = min(16, physical_cores())
    if not oracle.ref_available():
        return {"value": None, "unit": "tok/s (B=1)", "cores": threads, "host": host_cpu(),
                "kind": "reference", "sample": "reference build absent"}
    oracle.ref_lib("model").sn_set_threads(threads)
    q4 = oracle.ref_lib("quant")
    mats = []
    for l in range(w4.cfg.layers):
        M = layer_matrices(w4, l)
        mats += [M.V, M.U, M.W_z, M.W_c, M.W_s_eff]
    mats.append(np.ascontiguousarray(w4.embed.numpy(), np.float32))
    packed = []
    for W in mats:
        W = np.ascontiguousarray(W, np.float32)
        out, inn = W.shape
        q = np.empty((out, inn // 2), np.uint8)
        sc = np.empty((out, inn // 32), np.float32)
        q4.sn_quant_i4(W.ctypes.data, q.ctypes.data, sc.ctypes.data, out, inn, 32)
        x = np.random.default_rng(out + inn).standard_normal(inn).astype(np.float32)
        y = np.empty(out, np.float32)
        packed.append((q, sc, x, y, inn, out))

    def step():
        for q, sc, x, y, inn, out in packed:
            q4.sn_gemv_i4(y.ctypes.data, x.ctypes.data, q.ctypes.data, sc.ctypes.data, inn, out, 32)
    step()
    times = []
    deadline = time.perf_counter() + 10.0
    while len(times) < 32 and time.perf_counter() < deadline:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    nbytes = sum(q.nbytes + sc.nbytes for q, sc, *_ in packed)
    log(f"[bench] cpu reference sn_gemv_i4 step products: {med*1e3:.2f} ms, {threads} threads")
    return {"value": round(1.0 / med, 2), "unit": "tok/s (B=1, products only)", "cores": threads,
            "host": host_cpu(), "kind": "reference", "ms_per_step": round(med * 1e3, 3),
            "gbs": round(nbytes / med / 1e9, 2),
            "sample": f"SunnyNet-100M INT4 g32 weights: the 61 products of one step (12 x V, U, W_z, "
                      f"W_c, W_eff and the head) through sn_gemv_i4, median of {len(times)} steps"}


def bench_rwkv7(cpu: bool):
    """RWKV-7 12 layers, D=768, 12 heads of 64, F=3072, vocab 65536 (seed-2
    synthetic weights), INT4 g32 quantized at load: a 512-token random prompt
    by stepping, then 128 greedy steps on the device at B=1 and B=64 (the
    default steps, both bit-exact: the exact one-launch kernel at B=1, the
    per-kernel step at B=64), and at B=1 on the opt-in fast one-launch
    kernel."""
    import tempfile

    from sunnynet_amd.runtime.rwkv7 import HipRwkv7
    from sunnynet_amd.rwkv7 import RWKV_CFG4, init_rwkv7, pack_rwkv7_blob
    cfg = RWKV_CFG4
    dev = torch.device("cuda:0")
    tmp = tempfile.mkdtemp(prefix="snhip_bench_rk_")
    log("[bench] RWKV-7 weights (seed 2)")
    w = init_rwkv7(cfg, 2)
    p32 = os.path.join(tmp, "rk_fp32.bin")
    with open(p32, "wb") as f:
        f.write(pack_rwkv7_blob(w))
    out = {"model": "RWKV-7 L=12 D=768 H=12x64 F=3072 V=65536 ranks (64,64,32,128), INT4 g32",
           "steps": 128, "prompt": 512, "cases": []}
    g = torch.Generator(device="cpu").manual_seed(321)
    # The default (bit-exact) steps at B=1 and B=64, then the opt-in fast
    # one-launch step at B=1 (SNHIP_RK_PERSIST=1: not bit-exact, measured up
    # to 1.3e-4 from sn_rk_step), reported beside it.
    for B, persist in ((1, False), (64, False), (1, True)):
        if persist:
            os.environ["SNHIP_RK_PERSIST"] = "1"
        hm = HipRwkv7(p32, weights="int4", block=32, max_batch=B)
        os.environ.pop("SNHIP_RK_PERSIST", None)
        if persist and not hm.persist_grid:
            hm.close()
            continue
        prompts = torch.randint(0, cfg.vocab, (out["prompt"], B), generator=g, dtype=torch.int32).to(dev)
        lg = torch.empty(B, cfg.vocab, device=dev)
        for t in range(out["prompt"]):
            hm.step_batch(prompts[t], out=lg)
        tok = lg.argmax(1).int()
        hm.decode_greedy(tok, 4)
        torch.cuda.synchronize()
        steps = out["steps"]
        ms = _time_ms(lambda: hm.decode_greedy(tok, steps)) / steps
        exact = bool(hm.persist_grid) and hm.persist_exact and B == 1
        kernel = ("k_rk_exact (the whole step)" if exact else
                  "k_rk_persist (the whole step)" if hm.persist_grid and B == 1 else
                  "per-kernel step: k_rkq_ln, k_rkq_mm_w4 (tiled fp32 copies), k_rkq_heads")
        hm.close()
        key = ("rwkv7-persist" if persist else "rwkv7-exact" if exact else "rwkv7", B)
        rl = step_roofline(rwkv7_step_bytes(cfg, B), rwkv7_step_flops(cfg, B), ms * 1e3, kernel,
                           DECODE_TRAFFIC.get(key))
        rl["note"] = "bytes: weights plus the 64x64 head states read and written per sequence"
        if exact:
            rl["note"] += ("; this kernel reads fp32 copies of the layer matrices (each output one "
                           "sequential FMA chain in the reference's order), and its floor is those "
                           "chains' latency, not HBM")
        case = {"weights": "int4-g32", "B": B, "us_per_step": round(ms * 1e3, 2),
                "tok_s": round(B / ms * 1e3, 1), "roofline": rl,
                "parity": ("opt-in (SNHIP_RK_PERSIST=1): logits within 2e-4 of sn_rk_step, not bit-exact"
                           if persist else "bit-exact to sn_rk_step")}
        log(f"[bench] rwkv7 B={B}{' opt-in fast one-launch' if persist else ''}: {case['us_per_step']} us/step, "
            f"{case['tok_s']} tok/s")
        out["cases"].append(case)
    if cpu:
        out["cpu_baseline"] = cpu_rwkv7_baseline(w, tmp)
    return out


def cpu_rwkv7_baseline(w, tmp):
    """The reference sn_rk_step (B = 1) on the INT4 v3 blob (group 64, its
    W4A8 path; quant.c's INT4 GEMV runs OpenMP threads, fixed here to the
    physical-core count capped at 16); bounded to ~10 s."""
    import oracle
    from sunnynet_amd.rwkv7 import pack_rwkv7_blob
    threads = min(16, physical_cores())
    if not oracle.ref_available():
        return {"value": None, "unit": "tok/s (B=1)", "cores": threads, "host": host_cpu(), "kind": "reference",
                "sample": "reference build absent"}
    oracle.ref_lib("model").sn_set_threads(threads)     # process-wide OpenMP thread count
    p4 = os.path.join(tmp, "rk_q4.bin")
    with open(p4, "wb") as f:
        f.write(pack_rwkv7_blob(w, int4=True))
    m = oracle.RefRk(p4, w.cfg.vocab)
    for t in range(4):
        m.step(t)
    times = []
    deadline = time.perf_counter() + 10.0
    while len(times) < 20 and time.perf_counter() < deadline:
        t0 = time.perf_counter()
        m.step(len(times) + 100)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    log(f"[bench] cpu reference sn_rk_step int4: {med*1e3:.2f} ms/token, {threads} threads")
    return {"value": round(1.0 / med, 2), "unit": "tok/s (B=1)", "cores": threads, "host": host_cpu(), "kind": "reference",
            "ms_per_token": round(med * 1e3, 3),
            "sample": f"RWKV-7 same shape, INT4 group-64 blob (W4A8), 4 warm-up steps then median "
                      f"of {len(times)} single steps"}


def cpu_decode_baseline(path, cfg, half: bool = False):
    """The reference sn_step on the fp32 blob (B = 1, host cores), after a
    16-token prefill by stepping; bounded to a few seconds. half: the
    reference's sn_load_h handle (matrices held as fp16, sunnynet.c:455-579)."""
    import oracle
    threads = min(16, physical_cores())
    if oracle.ref_available():
        lib = oracle.ref_lib("model")
        lib.sn_set_threads(threads)
        m = oracle.RefSnModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers,
                              half=half)
        kind = "reference"
    else:
        m = None
        kind = "port"
    if m is None:
        if half:
            return {"value": None, "unit": "tok/s (B=1)", "cores": threads, "host": host_cpu(),
                    "kind": "reference", "sample": "reference build absent"}
        blob = np.fromfile(path, np.uint8)
        orc = oracle.SnOracle(blob)
        os.environ["OMP_NUM_THREADS"] = str(threads)
        step = lambda t: orc.step([t])
    else:
        step = m.step
    for t in range(16):
        step(t)
    times = []
    deadline = time.perf_counter() + 10.0
    while len(times) < 16 and time.perf_counter() < deadline:
        t0 = time.perf_counter()
        step(len(times) + 100)
        times.append(time.perf_counter() - t0)
    if m is not None:
        m.close()
    med = float(np.median(times))
    log(f"[bench] cpu {kind} sn_step 100M {'fp16 (sn_load_h)' if half else 'fp32'}: {med*1e3:.2f} ms/token, "
        f"{threads} threads")
    return {"value": round(1.0 / med, 2), "unit": "tok/s (B=1)", "cores": threads, "host": host_cpu(), "kind": kind,
            "ms_per_token": round(med * 1e3, 3),
            "sample": f"SunnyNet-100M {'fp16 weights (sn_load_h)' if half else 'fp32'}, 16-token prefill "
                      f"then median of {len(times)} single steps"}


def pmc_probe():
    """A short fixed sequence for `rocprofv3 --pmc` runs: 3 scans of the
    workload, then 3 plain device copies of one 537 MB input array (the copy
    calibrates FETCH_SIZE / WRITE_SIZE against a known byte count), then 3 each
    of the scan backward, the core forward and the core backward."""
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
    # Then 3 scan backwards, 3 core forwards and 3 core backwards on the same
    # shape (each kernel is named in the trace).
    out, _ = runtime.scan(da, db, d0, gated=True)
    dout = torch.randn_like(da)
    for _ in range(3):
        runtime.scan_bwd(da, db, d0, out, dout)
    del y, out, dout
    B, T, D = SCAN_B, SCAN_T, SCAN_D
    g = torch.Generator(device=dev).manual_seed(9)
    q = torch.randn(B, T, 2 * D, generator=g, device=dev) * 0.6
    delta = 0.01 + 0.4 * torch.rand(D, generator=g, device=dev)
    s0 = torch.randn(B, D, generator=g, device=dev) * 0.1
    for _ in range(3):
        fwd = runtime.core_fwd(q, delta, s0)
    dstate, du_in = torch.randn_like(fwd[0]), torch.randn_like(fwd[0])
    for _ in range(3):
        runtime.core_bwd(q, delta, s0, *fwd, dstate, du_in)
    torch.cuda.synchronize()
    log(f"[pmc] scan_bwd bytes/launch {6 * B * T * D * 4}; core fwd {20 * B * T * D}, "
        f"core bwd {36 * B * T * D}")
    return 0


def hbm_probe(reps: int = 10) -> int:
    """Achievable-bandwidth calibration on the scan's arrays (three fp32
    arrays of 16 x 4096 x 2048): plain grid-stride streaming kernels
    (snhip_abi_hbm_probe_dev) for c = a + b (the scan's two reads and one
    write) and for the two reads alone, over a sweep of grid sizes, and
    torch's device copy of one array; HIP events around `reps` launches after
    3 warm-ups. Prints one JSON line of GB/s figures."""
    from sunnynet_amd import _native
    dev = torch.device("cuda:0")
    n = SCAN_B * SCAN_T * SCAN_D
    a = torch.ones(n, device=dev)
    b = torch.ones(n, device=dev)
    c = torch.empty(n, device=dev)
    L = _native.lib()
    stream = torch.cuda.current_stream().cuda_stream

    def timed(fn):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    out = {"arrays": f"3 x fp32 {SCAN_B}x{SCAN_T}x{SCAN_D} ({n * 4} B each)", "reps": reps, "cases": []}
    for kind, name, nbytes in ((0, "c = a + b (2 reads + 1 write)", 3 * n * 4), (1, "read a and b", 2 * n * 4)):
        for grid in (1024, 2048, 4096, 16384):
            def launch():
                _native.check(L.snhip_abi_hbm_probe_dev(kind, a.data_ptr(), b.data_ptr(), c.data_ptr(), n, grid,
                                                        stream), "snhip_abi_hbm_probe_dev")
            us = timed(launch)
            out["cases"].append({"kernel": name, "grid": grid, "us": round(us, 2),
                                 "GB/s": round(nbytes / us / 1e3, 1)})
            log(f"[hbm] {name} grid {grid}: {us:.1f} us {nbytes / us / 1e3:.1f} GB/s")
    us = timed(lambda: c.copy_(a))
    out["cases"].append({"kernel": "torch copy (1 read + 1 write)", "us": round(us, 2),
                         "GB/s": round(2 * n * 4 / us / 1e3, 1)})
    print(json.dumps(out), flush=True)
    return 0


def _m100_blobs(tmp):
    from sunnynet_amd.blob import pack_sunny_blob
    from sunnynet_amd.weights import gaussian_matmuls, init_sunnynet
    w = init_sunnynet(SUNNY_100M, 1)
    return {"fp32": _write_blob(tmp, "m100_fp32.bin", pack_sunny_blob(w)),
            "int4": _write_blob(tmp, "m100_int4.bin", pack_sunny_blob(gaussian_matmuls(w, seed=3)))}


def profile_sequence(which: str) -> int:
    """Fixed launch sequences for rocprofv3 kernel-trace summaries:

    b1: SunnyNet-100M (seed 1; INT4 g32 on N(0, 0.02) matmuls), a chunked
        prefill of 1024 random ids, then 256 greedy steps at B=1, fp32 then INT4.
    batch: 64 greedy steps from random tokens at fp32 B=64, INT4 B=8, INT4 B=32.
    rwkv: RWKV-7 (12 layers, D=768, vocab 65536, seed-2 weights, INT4 g32 at
        load), 8 warm-up then 64 greedy steps at B=1 (the exact one-launch
        kernel) and at B=64, then at B=1 on the opt-in fast one-launch kernel.
    small: SunnyNet small (seed 0), prefill of 256 random ids, 64 greedy steps.
    """
    import tempfile

    from sunnynet_amd.runtime.model import HipModel
    dev = torch.device("cuda:0")
    tmp = tempfile.mkdtemp(prefix="snhip_prof_")
    g = torch.Generator(device="cpu").manual_seed(5)
    if which == "rwkv":
        from sunnynet_amd.runtime.rwkv7 import HipRwkv7
        from sunnynet_amd.rwkv7 import RWKV_CFG4, init_rwkv7, pack_rwkv7_blob
        cfg = RWKV_CFG4
        path = _write_blob(tmp, "rk.bin", pack_rwkv7_blob(init_rwkv7(cfg, 2)))
        for B, persist in ((1, False), (64, False), (1, True)):
            if persist:
                os.environ["SNHIP_RK_PERSIST"] = "1"
            hm = HipRwkv7(path, weights="int4", block=32, max_batch=B)
            os.environ.pop("SNHIP_RK_PERSIST", None)
            tok = torch.randint(0, cfg.vocab, (B,), generator=g, dtype=torch.int32).to(dev)
            hm.decode_greedy(tok, 8)
            hm.decode_greedy(tok, 64)
            torch.cuda.synchronize()
            log(f"[profile] rwkv7 int4 B={B}: 64 greedy steps (one-launch grid {hm.persist_grid}, "
                f"exact {hm.persist_exact})")
            hm.close()
        return 0
    if which == "small":
        from sunnynet_amd.blob import pack_sunny_blob
        from sunnynet_amd.config import SMALL
        from sunnynet_amd.weights import init_sunnynet
        cfg = SMALL
        path = _write_blob(tmp, "small.bin", pack_sunny_blob(init_sunnynet(cfg, 0)))
        hm = HipModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers)
        ids = torch.randint(0, cfg.vocab_size, (1, 256), generator=g, dtype=torch.int32).to(dev)
        tok = hm.prefill_batch(ids).argmax(1).int()
        hm.decode_greedy(tok, 64)
        torch.cuda.synchronize()
        hm.close()
        log("[profile] small fp32 B=1: prefill 256, 64 greedy steps")
        return 0
    cfg = SUNNY_100M
    paths = _m100_blobs(tmp)
    cases = [("fp32", 1), ("int4", 1)] if which == "b1" else [("fp32", 64), ("int4", 8), ("int4", 32)]
    for fmt, B in cases:
        hm = HipModel(paths[fmt], cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers,
                      max_batch=B, weights=fmt, block=32)
        if B == 1:
            ids = torch.randint(0, cfg.vocab_size, (1, 1024), generator=g, dtype=torch.int32).to(dev)
            tok = hm.prefill_batch(ids).argmax(1).int()
            n = 256
        else:
            tok = torch.randint(0, cfg.vocab_size, (B,), generator=g, dtype=torch.int32).to(dev)
            n = 64
        hm.decode_greedy(tok, n)
        torch.cuda.synchronize()
        hm.close()
        log(f"[profile] {fmt} B={B}: {n} greedy steps")
    return 0


def pmc_probe_decode() -> int:
    """A fixed sequence for `rocprofv3 --pmc` runs on every decode case. It
    starts with 3 plain device copies of a 512 MiB array (calibrating
    FETCH_SIZE / WRITE_SIZE against a known byte count). Then, per case, a
    handle is built and warmed up, and one measured call runs n greedy steps.
    Every measured call is bracketed by marker launches of `k_hbm_read2`
    (snhip_abi_hbm_probe_dev over 4 KiB), so a case's dispatches are the ones
    between its two markers. The cases, in order, with steps per call:
    SunnyNet-100M INT4 g32 B=1 (16), B=8 (8), B=32 (8); fp32 B=1 (16), B=64
    (8); fp16 B=1 (16); SunnyNet small fp32 B=1 (16); RWKV-7 INT4 g32 B=1
    (16), B=64 (4), B=1 on the opt-in persistent step (16). Each case's line on
    stderr names its order, steps and algorithmic bytes per step."""
    import tempfile

    from sunnynet_amd import _native
    from sunnynet_amd.blob import pack_sunny_blob
    from sunnynet_amd.config import SMALL
    from sunnynet_amd.runtime.model import HipModel
    from sunnynet_amd.runtime.rwkv7 import HipRwkv7
    from sunnynet_amd.rwkv7 import RWKV_CFG4, init_rwkv7, pack_rwkv7_blob
    from sunnynet_amd.weights import init_sunnynet
    dev = torch.device("cuda:0")
    x = torch.randn(128 << 20, device=dev)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    log(f"[pmc] copy bytes/launch read {x.numel() * 4} write {x.numel() * 4}")
    del x, y
    mk = torch.zeros(3, 1024, device=dev)
    L = _native.lib()

    nmark = 0

    def marker():
        nonlocal nmark
        torch.cuda.synchronize()
        _native.check(L.snhip_abi_hbm_probe_dev(1, mk[0].data_ptr(), mk[1].data_ptr(), mk[2].data_ptr(),
                                                1024, 1, torch.cuda.current_stream().cuda_stream),
                      "marker")
        torch.cuda.synchronize()
        nmark += 1

    tmp = tempfile.mkdtemp(prefix="snhip_pmc_")
    paths = _m100_blobs(tmp)
    paths["fp16"] = paths["fp32"]
    g = torch.Generator(device="cpu").manual_seed(11)
    order = 0

    def measured(name, hm, vocab, B, n, nbytes):
        nonlocal order
        tok = torch.randint(0, vocab, (B,), generator=g, dtype=torch.int32).to(dev)
        hm.decode_greedy(tok, n)
        marker()
        hm.decode_greedy(tok, n)
        marker()
        log(f"[pmc] case {order}: {name}: {n} greedy steps between markers {nmark - 2} and "
            f"{nmark - 1} (counting from 0); algorithmic bytes/step {nbytes}")
        order += 1

    marker()
    cfg = SUNNY_100M
    for fmt, B, n in (("int4", 1, 16), ("int4", 8, 8), ("int4", 32, 8), ("fp32", 1, 16),
                      ("fp32", 64, 8), ("fp16", 1, 16)):
        hm = HipModel(paths[fmt], cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers,
                      max_batch=B, weights=fmt, block=32)
        marker()
        measured(f"SunnyNet-100M {fmt} B={B}", hm, cfg.vocab_size, B, n, decode_step_bytes(cfg, fmt, B))
        hm.close()
    sc = SMALL
    ps = _write_blob(tmp, "small.bin", pack_sunny_blob(init_sunnynet(sc, 0)))
    hm = HipModel(ps, sc.vocab_size, sc.dim, sc.inner, sc.rank, sc.taps, sc.layers)
    marker()
    measured("SunnyNet small fp32 B=1", hm, sc.vocab_size, 1, 16, decode_step_bytes(sc, "fp32", 1))
    hm.close()
    rc = RWKV_CFG4
    path = _write_blob(tmp, "rk.bin", pack_rwkv7_blob(init_rwkv7(rc, 2)))
    nw = rc.matmul_params()
    for B, n, persist in ((1, 16, False), (64, 4, False), (1, 16, True)):
        if persist:
            os.environ["SNHIP_RK_PERSIST"] = "1"
        hm = HipRwkv7(path, weights="int4", block=32, max_batch=B)
        os.environ.pop("SNHIP_RK_PERSIST", None)
        marker()
        label = (" fast one-launch (opt-in)" if persist else
                 " exact one-launch" if hm.persist_grid and hm.persist_exact and B == 1 else "")
        measured(f"RWKV-7 int4 B={B}{label}", hm, rc.vocab, B, n,
                 rwkv7_step_bytes(rc, B))
        hm.close()
    torch.cuda.synchronize()
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="all", choices=["all", "scan", "core", "decode"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--pmc-probe", nargs="?", const="scan", choices=["scan", "decode"],
                    help="run the fixed launch sequence used for rocprofv3 --pmc and exit")
    ap.add_argument("--profile", choices=["b1", "batch", "rwkv", "small"],
                    help="run a fixed decode launch sequence for rocprofv3 --kernel-trace and exit")
    ap.add_argument("--hbm-probe", action="store_true",
                    help="time plain streaming kernels over the scan's arrays and exit")
    args = ap.parse_args(argv)
    if args.hbm_probe:
        return hbm_probe()
    if args.pmc_probe == "scan":
        return pmc_probe()
    if args.pmc_probe == "decode":
        return pmc_probe_decode()
    if args.profile:
        return profile_sequence(args.profile)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        log("bench.py measures one GPU only: this build has no multi-GPU path "
            "(the scan shards by channel and decode by sequence, with no communication, "
            "so N GPUs would run N independent copies).")
        return 2
    res = None
    if args.workload in ("all", "scan"):
        # The headline scan runs first, on a cold allocator and clean caches.
        res = bench_scan(args.steps, args.warmup, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
    core = None
    if args.workload in ("all", "core"):
        core = bench_core(args.steps, args.warmup, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        if args.workload == "core":
            print(json.dumps({"core": core}), flush=True)
            return 0
    dec = None
    if args.workload in ("all", "decode"):
        dec = bench_decode(cpu=not args.no_cpu)
    if args.workload == "decode":
        # Decode-only run: the headline is the B=1 fp32 decode rate.
        c = dec["cases"][0]
        line = {"metric": METRIC, "value": c["tok_s"], "unit": "tok/s", "n_gpus": 1,
                "steps": dec["steps"], "warmup": 8, "ms_per_step": c["us_per_step"] / 1e3,
                "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
                "data": "synthetic (seeded random ids, random-init weights)",
                "config": {"workload": "SunnyNet-100M greedy decode B=1 fp32"}, "decode": dec}
        print(json.dumps(line), flush=True)
        return 0
    line = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": res["dtype"], "data": "synthetic (seeded numpy PCG64)",
            "config": res["config"], "roofline": res["roofline"]}
    if "cpu_baseline" in res:
        line["cpu_baseline"] = res["cpu_baseline"]
    if "scan_bwd" in res:
        line["scan_bwd"] = res["scan_bwd"]
    if core is not None:
        line["core"] = core
    if dec is not None:
        line["decode"] = dec
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
