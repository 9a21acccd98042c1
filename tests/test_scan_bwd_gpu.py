"""Gated-scan backward on the GPU (scan_avx2.c:50-99): bit-identical to the
oracle (itself pinned bit-exact to the reference's scan_bwd_f32 in
tests/test_oracle.py) on the buffer path (N a multiple of 128, T with and
without a partial time tile) and the generic path; and the autograd function
against float64 torch autograd of the recurrence."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from sunnynet_amd import runtime

pytestmark = pytest.mark.gpu


def _inputs(B, T, N, seed):
    rng = np.random.default_rng(seed)
    p = rng.uniform(0.3, 1.0, (B, T, N)).astype(np.float32)
    nu = rng.standard_normal((B, T, N)).astype(np.float32)
    s0 = rng.standard_normal((B, N)).astype(np.float32)
    dout = rng.standard_normal((B, T, N)).astype(np.float32)
    return p, nu, s0, dout


@pytest.mark.parametrize("B,T,N", [(16, 64, 2048), (16, 200, 2048), (8, 33, 4096), (2, 37, 21), (3, 50, 640)])
def test_scan_bwd_matches_oracle(gpu, B, T, N):
    print(f"scan_bwd B={B} T={T} N={N}", flush=True)
    p, nu, s0, dout = _inputs(B, T, N, T + N)
    out, _ = oracle.recur_scan(p, nu, s0, gated=True)
    ref = oracle.scan_bwd(p, nu, s0, out, dout)
    d = [torch.from_numpy(x).to(gpu) for x in (p, nu, s0, out, dout)]
    got = runtime.scan_bwd(*d)
    for g, r in zip(got, ref):
        assert np.array_equal(g.cpu().numpy(), r)


def test_gated_scan_autograd(gpu):
    B, T, N = 2, 20, 256
    p, nu, s0, dout = _inputs(B, T, N, 9)
    dsend = np.random.default_rng(10).standard_normal((B, N)).astype(np.float32)
    tp, tn, ts = (torch.from_numpy(x).to(gpu).requires_grad_() for x in (p, nu, s0))
    out, send = runtime.gated_scan(tp, tn, ts)
    ((out * torch.from_numpy(dout).to(gpu)).sum() + (send * torch.from_numpy(dsend).to(gpu)).sum()).backward()
    # float64 reference of the same recurrence on the CPU
    rp, rn, rs = (torch.from_numpy(x).double().requires_grad_() for x in (p, nu, s0))
    s = rs
    outs = []
    for t in range(T):
        s = rp[:, t] * s + (1 - rp[:, t]) * rn[:, t]
        outs.append(s)
    ro = torch.stack(outs, 1)
    ((ro * torch.from_numpy(dout).double()).sum() + (ro[:, -1] * torch.from_numpy(dsend).double()).sum()).backward()
    for g, r in ((tp.grad, rp.grad), (tn.grad, rn.grad), (ts.grad, rs.grad)):
        err = (g.double().cpu() - r).abs().max().item()
        assert err < 1e-4 * max(1.0, r.abs().max().item()), err
