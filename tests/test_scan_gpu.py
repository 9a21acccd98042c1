"""GPU parity of the gated scan against the oracle: bit-exact, every shape.

The kernel follows recur.c's rounding (separate (1-a)*u, one FMA per step,
two roundings in the reference's scalar channel tail), so the comparison is
``np.array_equal``, not a tolerance. Shapes cover ragged N (tails), T not a
multiple of the time tile, T = 1, tiny and large channel counts, non-zero s0,
both forms, the device and host-pointer entry points, and the full
B=16, D=2048, T=4096 workload.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from sunnynet_amd import runtime
from sunnynet_amd.workloads import scan_inputs

pytestmark = pytest.mark.gpu


def _rand(B, T, N, seed):
    rng = np.random.default_rng(seed)
    a = rng.random((B, T, N), dtype=np.float32)
    b = rng.standard_normal((B, T, N)).astype(np.float32)
    s0 = rng.standard_normal((B, N)).astype(np.float32)
    return a, b, s0


SHAPES = [(1, 1, 8), (3, 50, 29), (2, 7, 64), (4, 129, 130), (2, 300, 2048),
          (1, 1000, 96), (5, 257, 1000), (16, 64, 2048), (3, 17, 4096)]


@pytest.mark.parametrize("gated", [True, False])
@pytest.mark.parametrize("B,T,N", SHAPES)
def test_scan_bitexact_device(gpu, B, T, N, gated):
    print(f"scan dev B={B} T={T} N={N} gated={gated}", flush=True)
    a, b, s0 = _rand(B, T, N, B * 7 + T + N)
    ro, rs = oracle.recur_scan(a, b, s0, gated)
    da, db, d0 = (torch.from_numpy(x).to(gpu) for x in (a, b, s0))
    out, send = runtime.scan(da, db, d0, gated=gated)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), ro)
    assert np.array_equal(send.cpu().numpy(), rs)


@pytest.mark.parametrize("gated", [True, False])
def test_scan_bitexact_host_pointers(gpu, gated):
    a, b, s0 = _rand(3, 77, 130, 11)
    ro, rs = oracle.recur_scan(a, b, s0, gated)
    out, send = runtime.scan(*(torch.from_numpy(x) for x in (a, b, s0)), gated=gated)
    assert np.array_equal(out.numpy(), ro) and np.array_equal(send.numpy(), rs)


def test_scan_pinned_shapes(gpu, monkeypatch):
    """Every compiled launch shape gives the same bits."""
    a, b, s0 = _rand(4, 333, 1024, 5)   # T not a multiple of any tile
    ro, rs = oracle.recur_scan(a, b, s0, True)
    da, db, d0 = (torch.from_numpy(x).to(gpu) for x in (a, b, s0))
    for shape in ("gen,1,8,16", "gen,2,8,16", "gen,2,2,32", "gen,4,4,16", "buf,1,4,32",
                  "buf,1,4,64", "buf,2,2,32", "buf,2,2,64", "buf,2,4,32", "buf,2,4,64",
                  "buf,2,8,32", "buf,4,2,32"):
        print("shape", shape, flush=True)
        monkeypatch.setenv("SNHIP_SCAN_SHAPE", shape)
        out, send = runtime.scan(da, db, d0, gated=True)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), ro), shape
        assert np.array_equal(send.cpu().numpy(), rs), shape


@pytest.mark.parametrize("gated", [True, False])
def test_step_bitexact(gpu, gated):
    a, b, s0 = _rand(3, 1, 131, 3)
    ref = oracle.recur_step(a[:, 0], b[:, 0], s0, gated)
    s = torch.from_numpy(s0).to(gpu)
    runtime.step(torch.from_numpy(a[:, 0].copy()).to(gpu), torch.from_numpy(b[:, 0].copy()).to(gpu),
                 s, gated=gated)
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy(), ref)


def test_step_loop_equals_scan(gpu):
    a, b, s0 = _rand(2, 40, 64, 9)
    da, db = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    s = torch.from_numpy(s0).to(gpu)
    out, _ = runtime.scan(da, db, s.clone(), gated=True)
    for t in range(40):
        runtime.step(da[:, t].contiguous(), db[:, t].contiguous(), s, gated=True)
        assert torch.equal(s, out[:, t])


@pytest.mark.parametrize("gated", [True, False])
def test_scan_full_workload_bitexact(gpu, gated):
    """B=16, D=2048, T=4096 (the measured workload), both forms."""
    print(f"full scan gated={gated}", flush=True)
    a, b, s0 = scan_inputs(gated=gated)
    ro, rs = oracle.recur_scan(a, b, s0, gated)
    da, db, d0 = (torch.from_numpy(x).to(gpu) for x in (a, b, s0))
    out, send = runtime.scan(da, db, d0, gated=gated)
    torch.cuda.synchronize()
    assert np.array_equal(send.cpu().numpy(), rs)
    assert np.array_equal(out.cpu().numpy(), ro)
