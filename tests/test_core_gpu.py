"""The fused block core (compete gate + decay gate + gated scan) and its
backward on the device, against the oracle (itself bit-identical to the
reference's core_fwd_f32 / core_bwd_f32, core_avx2.c:34-149) and against the
closed form in float64.

Bar: the reference's own (tests/test_architecture.py:738-740, 803-805): 1e-5
on states, u and p and 1e-4 on dq, ddelta and ds0, here against the oracle
(the device's expf is within 1 ulp of glibc's, every other operation is the
reference's in its order) and, on the reference's test inputs, against
float64 autograd. Shapes cover the ring kernels (D % 128 == 0 and T a multiple
of their time tile) and the one-lane-per-channel kernels (any D % 8 == 0, any T).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from sunnynet_amd import _native, runtime

pytestmark = pytest.mark.gpu

FWD_TOL, BWD_TOL = 1e-5, 1e-4
SHAPES = [(2, 128, 128), (3, 192, 256), (1, 512, 384), (2, 96, 128), (2, 80, 128), (2, 48, 32),
          (2, 37, 40), (4, 100, 128)]


def _inputs(B, T, D, seed, gate_scale=0.6):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((B, T, 2 * D)) * 0.6).astype(np.float32)
    q[..., D:] *= gate_scale / 0.6
    delta = (0.01 + 0.4 * rng.random(D)).astype(np.float32)
    s0 = (rng.standard_normal((B, D)) * 0.1).astype(np.float32)
    dstate = rng.standard_normal((B, T, D)).astype(np.float32)
    du_in = rng.standard_normal((B, T, D)).astype(np.float32)
    return q, delta, s0, dstate, du_in


def _dev(*xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in xs]


@pytest.mark.parametrize("B,T,D", SHAPES)
def test_core_fwd_bwd_match_oracle(gpu, B, T, D):
    print(f"core fwd/bwd B={B} T={T} D={D}", flush=True)
    q, delta, s0, dstate, du_in = _inputs(B, T, D, B * 1000 + T + D)
    ref = oracle.core_fwd(q, delta, s0)
    got = runtime.core_fwd(*_dev(q, delta, s0))
    torch.cuda.synchronize()
    for name, a, b in zip(("states", "u", "p"), got, ref):
        a = a.cpu().numpy()
        assert np.abs(a - b).max() < FWD_TOL, name
    # The backward from the oracle's forward outputs, so both sides see
    # identical inputs.
    rb = oracle.core_bwd(q, delta, s0, *ref, dstate, du_in)
    gb = runtime.core_bwd(*_dev(q, delta, s0, *ref, dstate, du_in))
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "ddelta", "ds0"), gb, rb):
        a = a.cpu().numpy()
        assert np.abs(a - b).max() < BWD_TOL * max(1.0, float(np.abs(b).max())), name


def test_core_matches_float64_closed_form(gpu):
    """The reference's own test inputs and bars (test_architecture.py:707-805),
    through the autograd seam: loss = sum(states dstate) + sum(u du_in)."""
    B, T, D, G = 2, 40, 32, 8
    for shape in ((B, T, D), (2, 64, 128)):
        B, T, D = shape
        q, delta, s0, dstate, du_in = _inputs(B, T, D, 12)
        qd, dd, sd = (x.requires_grad_(True) for x in _dev(q, delta, s0))
        u, st = runtime.core_forward(qd, dd, sd)
        ((st * torch.from_numpy(dstate).cuda()).sum() + (u * torch.from_numpy(du_in).cuda()).sum()).backward()
        qt = torch.from_numpy(q).double().requires_grad_(True)
        dt = torch.from_numpy(delta).double().requires_grad_(True)
        s0t = torch.from_numpy(s0).double().requires_grad_(True)
        ur, gt = qt[..., :D], qt[..., D:]
        gg = gt.view(B, T, D // G, G)
        w = torch.sigmoid(gg - torch.roll(gg, -1, dims=-1)) * torch.sigmoid(gg - torch.roll(gg, -2, dims=-1))
        ut = ur * w.reshape(B, T, D)
        pt = 1.0 - dt.view(1, 1, -1) * (1.0 - torch.sigmoid(gt))
        s = s0t
        sts = []
        for t in range(T):
            s = pt[:, t] * s + (1 - pt[:, t]) * ut[:, t]
            sts.append(s)
        stt = torch.stack(sts, 1)
        ((stt * torch.from_numpy(dstate).double()).sum() + (ut * torch.from_numpy(du_in).double()).sum()).backward()
        assert float((u.detach().cpu().double() - ut.detach()).abs().max()) < FWD_TOL
        assert float((st.detach().cpu().double() - stt.detach()).abs().max()) < FWD_TOL
        assert float((qd.grad.cpu().double() - qt.grad).abs().max()) < BWD_TOL
        assert float((dd.grad.cpu().double() - dt.grad).abs().max()) < BWD_TOL
        assert float((sd.grad.cpu().double() - s0t.grad).abs().max()) < BWD_TOL


def test_core_bwd_deterministic_and_accumulates_ddelta(gpu):
    """Fixed summation orders: two backward calls agree bit for bit. Through
    the C-ABI, ddelta is added to (the reference's `ddelta[d] += ...`)."""
    B, T, D = 4, 256, 256
    q, delta, s0, dstate, du_in = _inputs(B, T, D, 7)
    dv = _dev(q, delta, s0)
    fwd = runtime.core_fwd(*dv)
    a = runtime.core_bwd(*dv, *fwd, *_dev(dstate, du_in))
    b = runtime.core_bwd(*dv, *fwd, *_dev(dstate, du_in))
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    acc = torch.full((D,), 1.5, device="cuda")
    dq, ds0 = torch.empty_like(dv[0]), torch.empty_like(dv[2])
    ds, di = _dev(dstate, du_in)
    ptrs = [t.data_ptr() for t in (*dv, *fwd, ds, di, dq, acc, ds0)]
    rc = _native.lib().snhip_abi_core_bwd_dev(*ptrs, B, T, D, _native.stream_handle(dq.device))
    _native.check(rc, "snhip_abi_core_bwd_dev")
    torch.cuda.synchronize()
    assert torch.equal(dq, a[0]) and torch.equal(ds0, a[2])
    assert torch.equal(acc, torch.full_like(acc, 1.5) + a[1])


def test_core_saturated_gates_match_oracle(gpu):
    """Gates far outside expf's range (|g| = 100: e overflows to inf or
    underflows to 0, e_i / e_j becomes inf, 0 or NaN) give the reference's
    non-finite pattern and its finite values."""
    B, T, D = 2, 64, 128
    q, delta, s0, dstate, du_in = _inputs(B, T, D, 3)
    rng = np.random.default_rng(4)
    mask = rng.random((B, T, D)) < 0.1
    q[..., D:][mask] = rng.choice([-100.0, 100.0, -50.0, 50.0], size=int(mask.sum())).astype(np.float32)
    ref = oracle.core_fwd(q, delta, s0)
    got = [x.cpu().numpy() for x in runtime.core_fwd(*_dev(q, delta, s0))]
    for a, b in zip(got, ref):
        assert np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(np.isinf(a), np.isinf(b))
        fin = np.isfinite(b)
        assert np.abs(a[fin] - b[fin]).max() < FWD_TOL


def test_core_abi_rejects_bad_shapes(gpu):
    lib = _native.lib()
    x = torch.zeros(64, device="cuda")
    p = x.data_ptr()
    bad = lib.snhip_abi_core_fwd_dev(p, p, p, p, p, p, 1, 1, 12, None)      # D % 8 != 0
    assert bad != 0
    assert lib.snhip_abi_core_fwd_dev(None, p, p, p, p, p, 1, 1, 8, None) != 0
    assert lib.snhip_abi_core_bwd_dev(p, p, p, p, p, p, p, p, p, p, p, 1, 0, 8, None) != 0
