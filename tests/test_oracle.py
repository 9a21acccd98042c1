"""Pins the CPU oracle before anything is compared against it.

* bit-exact against the reference's own C compiled from its sources
  (oracle/_ref), where that was built;
* against closed forms, invariants and fp64 restatements that a plausible
  mistake (dropped term, swapped operand, wrong index) would break;
* against the known-answer formulas of the reference's tests
  (tests/test_quant_i4.py:32-70, tests/test_architecture.py:871-915).
"""
from __future__ import annotations

import ctypes
import os
import tempfile

import numpy as np
import pytest
import torch

import oracle
from oracle.torch_ref import TorchSunny, forward_hist_to_step
from sunnynet_amd.blob import pack_sunny_blob, parse_sunny_blob
from sunnynet_amd.config import SMALL, TINY
from sunnynet_amd.weights import init_sunnynet

f = oracle._f


# ------------------------------------------------------------------- scan
@pytest.mark.parametrize("gated", [0, 1])
@pytest.mark.parametrize("B,T,N", [(3, 50, 29), (2, 7, 64), (1, 1, 8), (4, 33, 130)])
def test_scan_bitexact_vs_reference(ref_built, gated, B, T, N):
    rng = np.random.default_rng(B * 100 + T + N)
    a = rng.random((B, T, N), dtype=np.float32)
    b = rng.standard_normal((B, T, N)).astype(np.float32)
    s0 = rng.standard_normal((B, N)).astype(np.float32)
    o1, e1 = oracle.recur_scan(a, b, s0, gated)
    lib = oracle.ref_lib("recur")
    o2, e2 = np.empty_like(a), np.empty_like(s0)
    lib.sn_recur_scan(f(a), f(b), f(s0), f(o2), f(e2), B, T, N, gated)
    assert np.array_equal(o1, o2) and np.array_equal(e1, e2)
    # The stable-ABI wrapper and, for the gated form, scan_f32 agree too.
    abi = oracle.ref_lib("abi")
    o3, e3 = np.empty_like(a), np.empty_like(s0)
    assert abi.sn_abi_recur_scan(f(a), f(b), f(s0), f(o3), f(e3), B, T, N, gated) == 0
    assert np.array_equal(o1, o3) and np.array_equal(e1, e3)
    if gated and N % 8 == 0:
        sl = oracle.ref_lib("scan")
        o4, e4 = np.empty_like(a), np.empty_like(s0)
        sl.scan_f32(f(a), f(b), f(s0), f(o4), f(e4), B, T, N)
        assert np.array_equal(o1, o4) and np.array_equal(e1, e4)


def test_scan_matches_fp64_loop():
    """tests/test_architecture.py:871-896: within 1e-5 of an fp64 loop."""
    rng = np.random.default_rng(21)
    B, T, N = 3, 128, 96
    a = (rng.random((B, T, N)) * 0.8 + 0.1).astype(np.float32)
    b = rng.standard_normal((B, T, N)).astype(np.float32)
    s0 = np.zeros((B, N), np.float32)
    for gated in (0, 1):
        A, Bb = a.astype(np.float64), b.astype(np.float64)
        s = s0.astype(np.float64)
        ref = np.empty((B, T, N))
        for t in range(T):
            bt = (1.0 - A[:, t]) * Bb[:, t] if gated else Bb[:, t]
            s = A[:, t] * s + bt
            ref[:, t] = s
        o, e = oracle.recur_scan(a, b, s0, gated)
        assert np.abs(o - ref).max() < 1e-5
        assert np.abs(e - ref[:, -1]).max() < 1e-5


def test_scan_invariants():
    rng = np.random.default_rng(5)
    B, T, N = 2, 200, 40
    u = rng.standard_normal((B, T, N)).astype(np.float32)
    s0 = rng.standard_normal((B, N)).astype(np.float32)
    # p = 1 => the state never moves.
    o, e = oracle.recur_scan(np.ones((B, T, N), np.float32), u, s0, 1)
    assert np.array_equal(o, np.broadcast_to(s0[:, None], o.shape))
    # p = 0 => the state is the input.
    o, _ = oracle.recur_scan(np.zeros((B, T, N), np.float32), u, s0, 1)
    assert np.array_equal(o, u)
    # Convex combination: |s_t| <= max(|s_{t-1}|, |u_t|) (README.md:25).
    p = rng.random((B, T, N), dtype=np.float32)
    o, _ = oracle.recur_scan(p, u, s0, 1)
    prev = np.concatenate([s0[:, None], o[:, :-1]], axis=1)
    bound = np.maximum(np.abs(prev), np.abs(u)) * (1 + 1e-6)
    assert np.all(np.abs(o) <= bound)
    # Constant input converges geometrically: |s_T - c| = prod(p) |s0 - c|.
    pc = np.full((1, T, N), 0.9, np.float32)
    o, _ = oracle.recur_scan(pc, np.full((1, T, N), 3.0, np.float32), np.zeros((1, N), np.float32), 1)
    assert np.allclose(o[0, -1], 3.0 * (1 - 0.9 ** T), rtol=1e-5)


def test_step_equals_scan():
    """tests/test_architecture.py:899-915, bit-exact."""
    rng = np.random.default_rng(22)
    B, T, N = 2, 96, 67
    a = (rng.random((B, T, N)) * 0.6 + 0.3).astype(np.float32)
    b = rng.standard_normal((B, T, N)).astype(np.float32)
    s = np.zeros((B, N), np.float32)
    o_scan, _ = oracle.recur_scan(a, b, s, 1)
    for t in range(T):
        s = oracle.recur_step(a[:, t], b[:, t], s, 1)
        assert np.array_equal(s, o_scan[:, t])


# ------------------------------------------------------------------- INT4
@pytest.mark.parametrize("block", [32, 64, 128])
def test_quant_i4_bitexact_vs_reference(ref_built, block):
    rng = np.random.default_rng(block)
    x = (rng.standard_normal((16, 1024)) * 0.05).astype(np.float32)
    x[3, :block] = 0.0                      # an all-zero group -> scale 1
    q1, s1 = oracle.quant_i4(x, block)
    lib = oracle.ref_lib("quant")
    q2, s2 = np.empty_like(q1), np.empty_like(s1)
    lib.sn_quant_i4(f(x), f(q2), f(s2), 16, 1024, block)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
    assert s1[3, 0] == 1.0
    d1 = oracle.dequant_i4(q1, s1, 1024, block)
    d2 = np.empty_like(x)
    lib.sn_dequant_i4(f(q1), f(s1), f(d2), 16, 1024, block)
    assert np.array_equal(d1, d2)


@pytest.mark.parametrize("block", [32, 64])
def test_quant_i4_known_answer(block):
    """Packing per tests/test_quant_i4.py:32-70 and error bound per :22-29."""
    rng = np.random.default_rng(1)
    out, n = 24, 256
    W = (rng.standard_normal((out, n)) * 2.0).astype(np.float32)
    q, s = oracle.quant_i4(W, block)
    half, nb = block // 2, n // block
    Wint = np.empty((out, n), np.int32)
    for o in range(out):
        for g in range(nb):
            for k in range(half):
                byte = int(q[o, g * half + k])
                Wint[o, g * block + k] = (byte & 0x0F) - 8
                Wint[o, g * block + half + k] = (byte >> 4) - 8
    # Independent restatement of the quantizer: scale = amax/7, q = rint(w/scale).
    amax = np.abs(W.reshape(out, nb, block)).max(-1)
    sc = (amax / np.float32(7.0)).astype(np.float32)
    assert np.array_equal(s, sc)
    inv = (np.float32(1.0) / sc).astype(np.float32)
    qq = np.clip(np.rint(W.reshape(out, nb, block) * inv[..., None]), -8, 7).astype(np.int32)
    assert np.array_equal(Wint, qq.reshape(out, n))
    deq = oracle.dequant_i4(q, s, n, block)
    assert np.array_equal(deq, (Wint.reshape(out, nb, block) * s[..., None]).reshape(out, n).astype(np.float32))
    assert np.all(np.abs(W - deq).reshape(out, nb, block) <= s[..., None] / 2 + 1e-6)


# ------------------------------------------------------------ decode step
def _blob_file(buf):
    f_ = tempfile.NamedTemporaryFile(suffix=".bin", delete=False)
    f_.write(buf)
    f_.close()
    return f_.name


@pytest.mark.parametrize("cfg", [TINY, SMALL], ids=["tiny", "small"])
def test_sn_step_bitexact_vs_reference(ref_built, cfg):
    w = init_sunnynet(cfg, 0)
    buf = pack_sunny_blob(w)
    path = _blob_file(buf)
    orc = oracle.SnOracle(buf)
    ref = oracle.RefSnModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps,
                            cfg.layers)
    toks = np.random.default_rng(3).integers(0, cfg.vocab_size, 24)
    for t in toks:
        assert np.array_equal(orc.step([t])[0], ref.step(int(t)))
    # Prefill is a step loop (sunnynet.c:347-349).
    ref.reset()
    orc.reset()
    last = ref.prefill(toks)
    for t in toks:
        lo = orc.step([t])[0]
    assert np.array_equal(lo, last)


def test_sn_dbg_layer_bitexact_vs_reference(ref_built):
    cfg = TINY
    w = init_sunnynet(cfg, 4)
    buf = pack_sunny_blob(w)
    path = _blob_file(buf)
    orc = oracle.SnOracle(buf)
    ref = oracle.RefSnModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps,
                            cfg.layers)
    for tok in (5, 77, 300):
        d1 = orc.dbg_layer(0, tok, 1)
        d2 = ref.dbg_layer(tok, 1, cfg.dim, cfg.inner, cfg.rank)
        mine = np.concatenate(list(d1.values()))
        assert np.array_equal(mine, d2[:mine.size])


def test_oracle_state_roundtrip_and_batch():
    cfg = TINY
    w = init_sunnynet(cfg, 1)
    buf = pack_sunny_blob(w)
    one = oracle.SnOracle(buf, batch=1)
    two = oracle.SnOracle(buf, batch=3)
    toks = np.random.default_rng(2).integers(0, cfg.vocab_size, (10, 3))
    for row in toks:
        l3 = two.step(row)
        assert np.array_equal(l3[1], one.step([row[1]])[0])
        assert np.array_equal(l3[0], l3[0])
    s, h = two.get_state()
    other = oracle.SnOracle(buf, batch=3)
    other.set_state(s, h)
    assert np.array_equal(other.step([1, 2, 3]), two.step([1, 2, 3]))


def test_blob_layout_roundtrip():
    cfg = TINY
    w = init_sunnynet(cfg, 2)
    p = parse_sunny_blob(pack_sunny_blob(w))
    assert p["cfg"].dim == cfg.dim and p["group"] == 8 and p["tied"] == 1 and p["clamp"] == 0
    assert np.array_equal(p["layers"][1]["U"], w.layers[1].U.numpy())
    assert np.array_equal(p["layers"][0]["W_s_eff"], w.ws_eff(0).numpy())
    assert np.array_equal(p["head"], w.embed.numpy())
    assert abs(p["eps"] - 4.1e-4) < 1e-9 and p["p_floor"] == np.float32(1 / 8192)


def test_oracle_step_matches_fp64_torch_forward_step():
    """The C oracle (fp32) against an independent fp64 torch restatement of
    forward_step: a dropped term or wrong index would break 1e-4."""
    cfg = TINY
    w = init_sunnynet(cfg, 9)
    orc = oracle.SnOracle(pack_sunny_blob(w))
    tr = TorchSunny(w, torch.float64)
    st = tr.init_state(1)
    toks = np.random.default_rng(4).integers(0, cfg.vocab_size, 40)
    worst = 0.0
    for t in toks:
        lg, st = tr.forward_step(torch.tensor([int(t)]), st)
        lo = orc.step([t])[0]
        worst = max(worst, float(np.abs(lg[0].numpy() - lo).max()))
    assert worst < 1e-5, worst
    s, h = orc.get_state()
    assert np.abs(s - st[0].numpy()).max() < 1e-5
    assert np.abs(h - st[1].numpy()).max() < 1e-5


def test_torch_ref_step_equals_forward_fp64():
    """tests/test_architecture.py:357-377 and :380-393 on the restatement:
    stepping equals the chunked prefill to 1e-10 in fp64, also when a segment
    continues from a carried state."""
    cfg = TINY
    w = init_sunnynet(cfg, 11)
    tr = TorchSunny(w, torch.float64)
    idx = torch.randint(0, cfg.vocab_size, (2, 70), generator=torch.Generator().manual_seed(0))
    full, (s_f, h_f) = tr.forward(idx)
    st = tr.init_state(2)
    outs = []
    for t in range(idx.shape[1]):
        lg, st = tr.forward_step(idx[:, t], st)
        outs.append(lg)
    step = torch.stack(outs, 1)
    assert float((step - full).abs().max()) < 1e-10
    assert float((st[0] - s_f).abs().max()) < 1e-10
    assert float((st[1] - forward_hist_to_step(h_f)).abs().max()) < 1e-10
    o1, s1 = tr.forward(idx[:, :29])
    o2, _ = tr.forward(idx[:, 29:], s1)
    assert float((torch.cat([o1, o2], 1) - full).abs().max()) < 1e-10


def test_weight_init_is_deterministic_and_orthogonal():
    """Same seed -> same weights, orthogonal rows scaled by rho (rho/2 for
    W_s), embedding std 0.02. The values themselves are pinned against the
    reference's SunnyNet(cfg) in test_weights_golden.py."""
    a = init_sunnynet(TINY, 0)
    b = init_sunnynet(TINY, 0)
    assert torch.equal(a.layers[1].W_s, b.layers[1].W_s)
    q = a.layers[0].V
    assert torch.allclose(q @ q.T, torch.eye(q.shape[0]), atol=1e-5)      # orthogonal rows
    Ws = a.layers[0].W_s
    assert torch.allclose(Ws @ Ws.T, 0.25 * torch.eye(Ws.shape[0]), atol=1e-5)   # rho/2
    assert abs(float(a.embed.std()) - 0.02) < 2e-3


@pytest.mark.parametrize("B,T,N", [(2, 37, 21), (3, 64, 64)])
def test_scan_bwd_bitexact_vs_reference(ref_built, B, T, N):
    """orc_scan_bwd against the reference's scan_bwd_f32 (scan_avx2.c:50-99):
    widths with and without the scalar tail, bit for bit."""
    rng = np.random.default_rng(B * 1000 + N)
    p = rng.uniform(0.3, 1.0, (B, T, N)).astype(np.float32)
    nu = rng.standard_normal((B, T, N)).astype(np.float32)
    s0 = rng.standard_normal((B, N)).astype(np.float32)
    out, _ = oracle.recur_scan(p, nu, s0, gated=True)
    dout = rng.standard_normal((B, T, N)).astype(np.float32)
    got = oracle.scan_bwd(p, nu, s0, out, dout)
    ref = [np.empty_like(p), np.empty_like(p), np.empty_like(s0)]
    f = oracle._f
    oracle.ref_lib("scan").scan_bwd_f32(f(p), f(nu), f(s0), f(out), f(dout), f(ref[0]), f(ref[1]),
                                        f(ref[2]), B, T, N)
    for a, b in zip(got, ref):
        assert np.array_equal(a, b)


def _core_inputs(B, T, D, seed):
    """The reference's own core test inputs (tests/test_architecture.py:714-719)."""
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((B, T, 2 * D)) * 0.6).astype(np.float32)
    delta = (0.01 + 0.4 * rng.random(D)).astype(np.float32)
    s0 = (rng.standard_normal((B, D)) * 0.1).astype(np.float32)
    return rng, q, delta, s0


def _ref_core(q, delta, s0, dstate=None, du_in=None):
    lib = oracle.ref_lib("core")
    f = oracle._f
    B, T, D2 = q.shape
    D = D2 // 2
    st, u, p = (np.empty((B, T, D), np.float32) for _ in range(3))
    lib.core_fwd_f32(f(q), f(delta), f(s0), f(st), f(u), f(p), B, T, D)
    if dstate is None:
        return st, u, p
    dq = np.empty_like(q)
    dd = np.zeros(D, np.float32)
    ds0 = np.empty((B, D), np.float32)
    lib.sn_set_threads(1)          # ddelta's per-row atomics then add in row order
    try:
        lib.core_bwd_f32(f(q), f(delta), f(s0), f(st), f(u), f(p), f(dstate), f(du_in), f(dq), f(dd),
                         f(ds0), B, T, D)
    finally:
        lib.sn_set_threads(os.cpu_count() or 1)
    return (st, u, p), (dq, dd, ds0)


@pytest.mark.parametrize("B,T,D", [(2, 48, 32), (3, 37, 64), (5, 16, 8)])
def test_core_fwd_bwd_bitexact_vs_reference(ref_built, B, T, D):
    """orc_core_fwd / orc_core_bwd against the reference's core_fwd_f32 /
    core_bwd_f32 (core_avx2.c:34-149), bit for bit (the reference run on one
    OpenMP thread so that its ddelta sums the rows in order)."""
    rng, q, delta, s0 = _core_inputs(B, T, D, 11 + B)
    dstate = rng.standard_normal((B, T, D)).astype(np.float32)
    du_in = rng.standard_normal((B, T, D)).astype(np.float32)
    fwd, bwd = _ref_core(q, delta, s0, dstate, du_in)
    got = oracle.core_fwd(q, delta, s0)
    for a, b in zip(got, fwd):
        assert np.array_equal(a, b)
    gb = oracle.core_bwd(q, delta, s0, *got, dstate, du_in)
    for a, b in zip(gb, bwd):
        assert np.array_equal(a, b)


def test_core_oracle_matches_float64_autograd():
    """The closed form the kernel implements, in float64 torch: the compete
    gate sigma(g_i - g_{i+1}) sigma(g_i - g_{i+2}) within groups of 8, p = 1 -
    delta (1 - sigma(g)), the gated scan; gradients by autograd of
    sum(states * dstate) + sum(u * du_in). The reference's own bars
    (tests/test_architecture.py:738-740, 803-805): 1e-5 forward, 1e-4 backward."""
    B, T, D, G = 2, 40, 32, 8
    rng, q, delta, s0 = _core_inputs(B, T, D, 12)
    st, u, p = oracle.core_fwd(q, delta, s0)
    dstate = rng.standard_normal((B, T, D)).astype(np.float32)
    du_in = rng.standard_normal((B, T, D)).astype(np.float32)
    dq, dd, ds0 = oracle.core_bwd(q, delta, s0, st, u, p, dstate, du_in)
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
    assert float((torch.from_numpy(u).double() - ut).abs().max()) < 1e-5
    assert float((torch.from_numpy(p).double() - pt).abs().max()) < 1e-5
    assert float((torch.from_numpy(st).double() - stt).abs().max()) < 1e-5
    ((stt * torch.from_numpy(dstate).double()).sum() + (ut * torch.from_numpy(du_in).double()).sum()).backward()
    assert float(np.abs(dq - qt.grad.numpy()).max()) < 1e-4
    assert float(np.abs(dd - dt.grad.numpy()).max()) < 1e-4
    assert float(np.abs(ds0 - s0t.grad.numpy()).max()) < 1e-4
