"""GPU parity of the RWKV-7 decode handle against the oracle.

Bar: logits within 2e-5 absolute of the C oracle, which is bit-identical to
the reference's sn_rk_step on fp32 blobs (tests/test_rwkv7_oracle.py); the
greedy argmax equal on every token. INT4: the oracle runs the fp32 path on the
bit-identically dequantized weights (W4A32).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from sunnynet_amd import _native
from sunnynet_amd.runtime.rwkv7 import HipRwkv7
from sunnynet_amd.rwkv7 import (RWKV_CFG4, RWKV_TINY, RwkvConfig, dequant_i4_np, init_rwkv7,
                                pack_rwkv7_blob, quant_i4_np)

pytestmark = pytest.mark.gpu
TOL = 2e-5
# Batches of 8 or more run the matrix products on the MFMA GEMM (blocked
# accumulation, split-K partials summed in a fixed order). On the 12-layer,
# 65536-vocab model its logits (|logit| up to ~5) differ from the sequential
# oracle by up to 3.0e-5 on the first step (GEMV path: 1.7e-5), 6e-6 relative.
TOL_MM = 5e-5


def dequant_weights(w, block):
    """Copy of `w` whose matrices (input length a multiple of block) hold their
    INT4-dequantized values."""
    import copy
    d = copy.deepcopy(w)

    def dq(M):
        if M.shape[1] % block:
            return M
        q, s = quant_i4_np(M, block)
        return dequant_i4_np(q, s, M.shape[1], block)

    for L in d.layers:
        for k in ("r", "k", "v", "o", "w1", "w2", "a1", "a2", "v1", "v2", "g1", "g2", "cmk", "cmv"):
            L[k] = dq(L[k])
    d.head = dq(d.head)
    return d


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    w = init_rwkv7(RWKV_TINY, 2)
    d = tmp_path_factory.mktemp("rk")
    p32 = d / "tiny.bin"
    p32.write_bytes(pack_rwkv7_blob(w))
    p4 = d / "tiny_q4.bin"
    p4.write_bytes(pack_rwkv7_blob(w, int4=True))
    return w, p32, p4


def _check_steps(hm, orc, toks, B=1, tol=TOL):
    worst = 0.0
    for t in toks:
        if B == 1:
            a = np.asarray(hm.step(int(t)), np.float32)
            b = orc.step([t])[0]
        else:
            tt = np.asarray(t, np.int32)
            a = hm.step_batch(torch.from_numpy(tt).cuda()).cpu().numpy()
            b = orc.step(tt)
        worst = max(worst, float(np.abs(a - b).max()))
        assert np.array_equal(np.argmax(a, -1), np.argmax(b, -1))
    print("worst |dlogit|", worst, flush=True)
    assert worst < tol, worst
    return worst


def test_tiny_fp32_b1(gpu, tiny):
    w, p32, _ = tiny
    print("rwkv7 tiny fp32 B=1", flush=True)
    hm = HipRwkv7(p32)
    orc = oracle.RkOracle(p32.read_bytes())
    _check_steps(hm, orc, np.random.default_rng(1).integers(0, RWKV_TINY.vocab, 32))
    S, sh = hm.get_state(1)
    So, sho = orc.get_state()
    assert np.abs(S.cpu().numpy() - So).max() < 1e-4 and np.abs(sh.cpu().numpy() - sho).max() < 1e-5


def test_reference_class_surface(gpu, tiny):
    """Constructed and driven like the reference's SnRWKV7(path, vocab)
    (rwkv7_c.py:65-104): step_raw advances the state, logits() returns the
    last step's logits, prefill feeds tokens in order; a vocab that does not
    match the blob is rejected."""
    w, p32, _ = tiny
    print("rwkv7 tiny reference class surface", flush=True)
    hm = HipRwkv7(p32, RWKV_TINY.vocab)
    orc = oracle.RkOracle(p32.read_bytes())
    toks = [5, 77, 300, 2]
    for t in toks[:-1]:
        hm.step_raw(t)
        orc.step([t])
    a = np.asarray(hm.step(toks[-1]), np.float32)
    b = orc.step([toks[-1]])[0]
    assert np.abs(a - b).max() < TOL
    assert np.array_equal(np.asarray(hm.logits(), np.float32), a)
    hm.reset()
    c = np.asarray(hm.prefill(toks), np.float32)
    assert np.array_equal(c, a)
    with pytest.raises(ValueError):
        HipRwkv7(p32, RWKV_TINY.vocab + 1)


@pytest.mark.parametrize("B", [3, 9])
def test_tiny_batched(gpu, tiny, B):
    """B=9 runs the matrix products on the MFMA GEMM."""
    w, p32, _ = tiny
    print(f"rwkv7 tiny fp32 B={B}", flush=True)
    hm = HipRwkv7(p32, max_batch=16)
    orc = oracle.RkOracle(p32.read_bytes(), batch=B)
    rng = np.random.default_rng(B)
    _check_steps(hm, orc, [rng.integers(0, RWKV_TINY.vocab, B) for _ in range(10)], B=B,
                 tol=TOL_MM if B >= 8 else TOL)


def test_int4_blob_stored(gpu, tiny):
    """INT4 (group 64) matrices of the v3 blob run as stored."""
    w, _, p4 = tiny
    print("rwkv7 tiny int4 blob", flush=True)
    hm = HipRwkv7(p4)
    orc = oracle.RkOracle(p4.read_bytes())   # dequantizes at load
    _check_steps(hm, orc, np.random.default_rng(2).integers(0, RWKV_TINY.vocab, 24))


def test_int4_g32_at_load(gpu, tiny, tmp_path):
    w, p32, _ = tiny
    print("rwkv7 tiny fp32 blob quantized to int4 g32 at load", flush=True)
    hm = HipRwkv7(p32, weights="int4", block=32, max_batch=4)
    orc = oracle.RkOracle(pack_rwkv7_blob(dequant_weights(w, 32)), batch=4)
    rng = np.random.default_rng(3)
    _check_steps(hm, orc, [rng.integers(0, RWKV_TINY.vocab, 4) for _ in range(12)], B=4)


def test_state_roundtrip_and_greedy(gpu, tiny):
    w, p32, _ = tiny
    B = 2
    hm = HipRwkv7(p32, max_batch=B)
    orc = oracle.RkOracle(p32.read_bytes(), batch=B)
    g = torch.Generator().manual_seed(0)
    S = torch.randn(B, RWKV_TINY.layers, RWKV_TINY.n_head, 64, 64, generator=g) * 0.1
    sh = torch.randn(B, RWKV_TINY.layers, 2, RWKV_TINY.dim, generator=g)
    hm.set_state(S.cuda(), sh.cuda())
    orc.set_state(S.numpy(), sh.numpy())
    start = np.array([5, 300], np.int32)
    out = hm.decode_greedy(torch.from_numpy(start).cuda(), 12).cpu().numpy()
    cur = start
    for i in range(12):
        nxt = orc.step(cur).argmax(1).astype(np.int32)
        assert np.array_equal(out[i], nxt), i
        cur = nxt


def test_abi_mirror(gpu, tiny):
    w, p32, _ = tiny
    L = _native.lib()
    h = L.snhip_abi_rwkv7_load(str(p32).encode())
    assert h
    V = L.snhip_abi_rwkv7_vocab(h)
    assert V == RWKV_TINY.vocab
    out = np.empty(V, np.float32)
    orc = oracle.RkOracle(p32.read_bytes())
    toks = np.array([3, 9, 27, 81], np.int32)
    assert L.snhip_abi_rwkv7_prefill(h, toks.ctypes.data, 4, out.ctypes.data) == 0
    for t in toks:
        ref = orc.step([t])[0]
    assert np.abs(out - ref).max() < TOL
    assert L.snhip_abi_rwkv7_step(h, -1, out.ctypes.data) == -1
    assert L.snhip_abi_rwkv7_reset(h) == 0
    L.snhip_abi_rwkv7_free(h)


def test_cfg4_int4_b1_and_b64(gpu, tmp_path_factory):
    """12 layers, D=768, 12 heads, vocab 65536, INT4 g32 at load (seed 2):
    B=1 for 3 steps, then B=64 with sequences 0, 17, 63 checked."""
    cfg = RWKV_CFG4
    print("rwkv7 cfg4: generating weights", flush=True)
    w = init_rwkv7(cfg, 2)
    p = tmp_path_factory.mktemp("rk4") / "cfg4.bin"
    p.write_bytes(pack_rwkv7_blob(w))
    dq = pack_rwkv7_blob(dequant_weights(w, 32))
    print("rwkv7 cfg4 int4 g32 B=1", flush=True)
    hm = HipRwkv7(p, weights="int4", block=32, max_batch=64)
    orc = oracle.RkOracle(dq)
    _check_steps(hm, orc, np.random.default_rng(4).integers(0, cfg.vocab, 3))
    print("rwkv7 cfg4 int4 g32 B=64", flush=True)
    hm.reset()
    pick = [0, 17, 63]
    orc3 = oracle.RkOracle(dq, batch=len(pick))
    rng = np.random.default_rng(64)
    for _ in range(2):
        toks = rng.integers(0, cfg.vocab, 64).astype(np.int32)
        a = hm.step_batch(torch.from_numpy(toks).cuda()).cpu().numpy()
        b = orc3.step(toks[pick])
        print("B=64 worst |dlogit|", float(np.abs(a[pick] - b).max()), flush=True)
        assert np.abs(a[pick] - b).max() < TOL_MM
        assert np.array_equal(a[pick].argmax(1), b.argmax(1))
