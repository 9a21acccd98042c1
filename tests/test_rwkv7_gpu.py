"""GPU parity of the RWKV-7 decode handle against the oracle.

The oracle is bit-identical to the reference's sn_rk_step on fp32 blobs
(tests/test_rwkv7_oracle.py). INT4: the oracle runs the fp32 path on the
bit-identically dequantized weights (W4A32).

Bars. Both default paths follow the reference's rounding order everywhere,
so their logits and states must EQUAL the oracle's, bit for bit, step after
step: the one-launch exact kernel (rkexact.hip: one sequence, and 2..8 on
grid slices; tests/test_rkexact_gpu.py covers it in depth) and the
per-kernel step (larger batches, ragged LoRA ranks, or every step with
SNHIP_RK_EXACT=0). The opt-in fast one-launch kernel (rkpersist.hip, summing
in parallel) has its own bar in tests/test_rkpersist_gpu.py.
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
EXACT = 0.0


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
    """tol = EXACT asks for identical logits."""
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
        if tol == EXACT:
            assert np.array_equal(a, b), worst
    print("worst |dlogit|", worst, flush=True)
    assert worst <= tol if tol == EXACT else worst < tol, worst
    return worst


def _per_kernel(path, monkeypatch, **kw):
    """A handle whose steps all take the per-kernel step (SNHIP_RK_EXACT=0)."""
    monkeypatch.setenv("SNHIP_RK_EXACT", "0")
    h = HipRwkv7(path, **kw)
    monkeypatch.delenv("SNHIP_RK_EXACT")
    assert h.persist_grid == 0
    return h


def test_tiny_fp32_b1(gpu, tiny):
    """A handle as loaded (B=1 on the default exact one-launch kernel): exact."""
    w, p32, _ = tiny
    print("rwkv7 tiny fp32 B=1", flush=True)
    hm = HipRwkv7(p32)
    assert hm.persist_grid > 0 and hm.persist_exact
    orc = oracle.RkOracle(p32.read_bytes())
    _check_steps(hm, orc, np.random.default_rng(1).integers(0, RWKV_TINY.vocab, 32), tol=EXACT)
    S, sh = hm.get_state(1)
    So, sho = orc.get_state()
    assert np.array_equal(S.cpu().numpy(), So) and np.array_equal(sh.cpu().numpy(), sho)


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


def test_tiny_per_kernel_b1_exact(gpu, tiny, monkeypatch):
    w, p32, _ = tiny
    print("rwkv7 tiny fp32 B=1 per-kernel step, exact", flush=True)
    hm = _per_kernel(p32, monkeypatch)
    orc = oracle.RkOracle(p32.read_bytes())
    _check_steps(hm, orc, np.random.default_rng(1).integers(0, RWKV_TINY.vocab, 32), tol=EXACT)
    S, sh = hm.get_state(1)
    So, sho = orc.get_state()
    assert np.array_equal(S.cpu().numpy(), So) and np.array_equal(sh.cpu().numpy(), sho)


@pytest.mark.parametrize("B", [2, 3, 9, 16])
def test_tiny_batched_exact(gpu, tiny, B):
    w, p32, _ = tiny
    print(f"rwkv7 tiny fp32 B={B}, exact", flush=True)
    hm = HipRwkv7(p32, max_batch=16)
    assert (hm.persist_grid_for(B) > 0) == (B <= 8)   # grid slices up to 8 sequences
    orc = oracle.RkOracle(p32.read_bytes(), batch=B)
    rng = np.random.default_rng(B)
    _check_steps(hm, orc, [rng.integers(0, RWKV_TINY.vocab, B) for _ in range(10)], B=B, tol=EXACT)
    S, sh = hm.get_state(B)
    So, sho = orc.get_state()
    assert np.array_equal(S.cpu().numpy(), So) and np.array_equal(sh.cpu().numpy(), sho)


def test_int4_blob_stored(gpu, tiny, monkeypatch):
    """INT4 (group 64) matrices of the v3 blob run as stored; the 32-input
    V_2 stays fp32. B=1 (per-kernel and one-launch) and B=3 exact."""
    w, _, p4 = tiny
    print("rwkv7 tiny int4 blob", flush=True)
    toks = np.random.default_rng(2).integers(0, RWKV_TINY.vocab, 24)
    hg = _per_kernel(p4, monkeypatch)
    _check_steps(hg, oracle.RkOracle(p4.read_bytes()), toks, tol=EXACT)   # dequantizes at load
    _check_steps(HipRwkv7(p4), oracle.RkOracle(p4.read_bytes()), toks, tol=EXACT)
    h3 = HipRwkv7(p4, max_batch=3)
    assert h3.persist_grid_for(3) > 0
    rng = np.random.default_rng(22)
    _check_steps(h3, oracle.RkOracle(p4.read_bytes(), batch=3),
                 [rng.integers(0, RWKV_TINY.vocab, 3) for _ in range(8)], B=3, tol=EXACT)


def test_int4_g32_at_load(gpu, tiny, tmp_path):
    """INT4 g32 quantized at load, B=4: exact."""
    w, p32, _ = tiny
    print("rwkv7 tiny fp32 blob quantized to int4 g32 at load, exact", flush=True)
    hm = HipRwkv7(p32, weights="int4", block=32, max_batch=4)
    assert hm.persist_grid_for(4) > 0
    orc = oracle.RkOracle(pack_rwkv7_blob(dequant_weights(w, 32)), batch=4)
    rng = np.random.default_rng(3)
    _check_steps(hm, orc, [rng.integers(0, RWKV_TINY.vocab, 4) for _ in range(12)], B=4, tol=EXACT)


def test_ragged_ranks_and_tail_columns_exact(gpu, tmp_path, monkeypatch):
    """LoRA ranks that differ per layer and are not multiples of 8 (12, 20):
    the products' last columns take the reference's two-rounding scalar tail."""
    w = init_rwkv7(RWKV_TINY, 13)
    rng = np.random.default_rng(13)
    D = w.cfg.dim
    ranks = [w.cfg.ranks, (20, 64, 12, 36)]
    for k, r in zip(("w", "a", "v", "g"), ranks[1]):
        w.layers[1][k + "1"] = (rng.standard_normal((r, D)) / np.sqrt(D)).astype(np.float32)
        w.layers[1][k + "2"] = (rng.standard_normal((D, r)) * 0.5 / np.sqrt(r)).astype(np.float32)
    p = tmp_path / "ragged.bin"
    p.write_bytes(pack_rwkv7_blob(w, ranks=ranks))
    print("rwkv7 ragged ranks B=1 and B=5, exact", flush=True)
    toks = np.random.default_rng(5).integers(0, RWKV_TINY.vocab, 12)
    _check_steps(_per_kernel(p, monkeypatch), oracle.RkOracle(p.read_bytes()), toks, tol=EXACT)
    h5 = HipRwkv7(p, max_batch=5)
    assert h5.persist_grid == 0       # the one-launch kernels take power-of-two ranks only
    rng = np.random.default_rng(55)
    _check_steps(h5, oracle.RkOracle(p.read_bytes(), batch=5),
                 [rng.integers(0, RWKV_TINY.vocab, 5) for _ in range(6)], B=5, tol=EXACT)


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


@pytest.fixture(scope="module")
def cfg4(tmp_path_factory):
    cfg = RWKV_CFG4
    print("rwkv7 cfg4: generating weights", flush=True)
    w = init_rwkv7(cfg, 2)
    p = tmp_path_factory.mktemp("rk4") / "cfg4.bin"
    p.write_bytes(pack_rwkv7_blob(w))
    return p, pack_rwkv7_blob(dequant_weights(w, 32))


def test_cfg4_int4_b1(gpu, cfg4):
    """12 layers, D=768, 12 heads, vocab 65536, INT4 g32 at load (seed 2),
    B=1 on the handle as loaded (the exact one-launch kernel): exact."""
    p, dq = cfg4
    toks = np.random.default_rng(4).integers(0, RWKV_CFG4.vocab, 4)
    print("rwkv7 cfg4 int4 g32 B=1, exact", flush=True)
    hm = HipRwkv7(p, weights="int4", block=32)
    assert hm.persist_grid > 0 and hm.persist_exact
    _check_steps(hm, oracle.RkOracle(dq), toks, tol=EXACT)


def _w4(monkeypatch, w4):
    """SNHIP_RKQ_W4 for the next handle: "1" (default) multiplies the per-kernel
    products on input-blocked fp32 copies made at load (one independent wave
    per tile), "0" on the INT4 codes (producer waves dequantizing into LDS)."""
    monkeypatch.setenv("SNHIP_RKQ_W4", w4)


@pytest.mark.parametrize("w4,fuse", [("1", "1"), ("0", "1"), ("1", "0")])
def test_cfg4_int4_b64_exact(gpu, cfg4, monkeypatch, w4, fuse):
    """B=64 (the benchmark's batched configuration): five sequences replayed
    on the oracle, four steps, logits identical; with the LoRA up-projections
    inside the heads kernel (default) and in their own launch
    (SNHIP_RKQ_FUSE_UPS=0)."""
    p, dq = cfg4
    cfg = RWKV_CFG4
    print(f"rwkv7 cfg4 int4 g32 B=64, exact, SNHIP_RKQ_W4={w4} SNHIP_RKQ_FUSE_UPS={fuse}", flush=True)
    _w4(monkeypatch, w4)
    monkeypatch.setenv("SNHIP_RKQ_FUSE_UPS", fuse)
    hm = HipRwkv7(p, weights="int4", block=32, max_batch=64)
    pick = [0, 17, 31, 48, 63]
    orc = oracle.RkOracle(dq, batch=len(pick))
    rng = np.random.default_rng(64)
    for _ in range(4):
        toks = rng.integers(0, cfg.vocab, 64).astype(np.int32)
        a = hm.step_batch(torch.from_numpy(toks).cuda()).cpu().numpy()
        b = orc.step(toks[pick])
        print("B=64 worst |dlogit|", float(np.abs(a[pick] - b).max()), flush=True)
        assert np.array_equal(a[pick], b)


@pytest.mark.parametrize("w4", ["1", "0"])
def test_cfg4_int4_ragged_batch_exact(gpu, cfg4, monkeypatch, w4):
    """B=37: the r/k/v and LoRA-up launches then take the staged-X form
    (four consumers per workgroup, 16 sequences of X rows in LDS), with a last
    sequence tile of 5 rows, and the wide vocabulary head four 16-sequence
    chains per workgroup (three would cover 37, but only 1, 2 and 4 are
    built: B = 33..48 once asked for three and the launch was refused);
    sequences from the first and the partial tile replayed on the oracle,
    three steps, logits identical."""
    p, dq = cfg4
    cfg = RWKV_CFG4
    B = 37
    print(f"rwkv7 cfg4 int4 g32 B={B}, exact, SNHIP_RKQ_W4={w4}", flush=True)
    _w4(monkeypatch, w4)
    hm = HipRwkv7(p, weights="int4", block=32, max_batch=B)
    pick = [0, 15, 32, 36]
    orc = oracle.RkOracle(dq, batch=len(pick))
    rng = np.random.default_rng(37)
    for _ in range(3):
        toks = rng.integers(0, cfg.vocab, B).astype(np.int32)
        a = hm.step_batch(torch.from_numpy(toks).cuda()).cpu().numpy()
        b = orc.step(toks[pick])
        print(f"B={B} worst |dlogit|", float(np.abs(a[pick] - b).max()), flush=True)
        assert np.array_equal(a[pick], b)


@pytest.mark.parametrize("shape", ["1,1", "1,2", "1,4", "2,1", "2,2", "2,4", "4,1", "4,2"])
def test_cfg4_int4_tiled_product_shapes(gpu, cfg4, monkeypatch, shape):
    """Every workgroup shape of the tiled fp32 products (S chains of 4
    sequences per wave, NW waves per workgroup), forced with
    SNHIP_RKQ_W4_SHAPE wherever it fits (the channel-mix value's K = 3072
    takes one chain per wave; a shape over 64 KiB of LDS falls back to the
    chosen one): B = 37, so the last sequence tile is partial and a
    workgroup's last waves may have no tile; sequences of the first and the
    partial tile replayed on the oracle, two steps, logits identical."""
    p, dq = cfg4
    cfg = RWKV_CFG4
    B = 37
    print(f"rwkv7 cfg4 int4 g32 B={B}, tiled products forced to S,NW={shape}", flush=True)
    monkeypatch.setenv("SNHIP_RKQ_W4_SHAPE", shape)
    hm = HipRwkv7(p, weights="int4", block=32, max_batch=B)
    pick = [0, 3, 33, 36]
    orc = oracle.RkOracle(dq, batch=len(pick))
    rng = np.random.default_rng(7)
    for _ in range(2):
        toks = rng.integers(0, cfg.vocab, B).astype(np.int32)
        a = hm.step_batch(torch.from_numpy(toks).cuda()).cpu().numpy()
        b = orc.step(toks[pick])
        assert np.array_equal(a[pick], b), float(np.abs(a[pick] - b).max())


@pytest.mark.parametrize("w4", ["1", "0"])
def test_cfg4_int4_every_batch_size(gpu, cfg4, monkeypatch, w4):
    """Every batch size 1..64 of the 12-layer INT4 model (1..8 on the exact
    one-launch kernel, one grid slice per sequence; from 9 on the per-kernel
    step, whose launch shapes change with B: one or four consumers per
    workgroup, staged or global X, narrow or wide chains and their counts):
    one step from the reset state, the first and the last sequence identical
    to the oracle's."""
    p, dq = cfg4
    cfg = RWKV_CFG4
    print(f"rwkv7 cfg4 int4 g32 B=1..64, one step each, SNHIP_RKQ_W4={w4}", flush=True)
    _w4(monkeypatch, w4)
    hm = HipRwkv7(p, weights="int4", block=32, max_batch=64)
    rng = np.random.default_rng(99)
    orc = oracle.RkOracle(dq, batch=2)
    for B in range(1, 65):
        toks = rng.integers(0, cfg.vocab, B).astype(np.int32)
        hm.reset()
        a = hm.step_batch(torch.from_numpy(toks).cuda()).cpu().numpy()
        orc.reset()
        b = orc.step(toks[[0, B - 1]])
        assert np.array_equal(a[[0, B - 1]], b), B


def test_loader_rejects_truncated_and_malformed_blobs(gpu, tiny, tmp_path):
    """The v3 loader checks every size before it reads (the reference's
    sn_rk_load reads past the end of such files): a file cut anywhere, a wrong
    magic or version, an out-of-range LoRA rank and an unknown tensor tag all
    give NULL with an error text, never a crash, and a good blob still loads."""
    import struct
    w, p32, p4 = tiny
    L = _native.lib()
    for src in (p32, p4):
        blob = src.read_bytes()
        bad = tmp_path / "bad.bin"
        for cut in (0, 20, 44, 60, len(blob) // 3, len(blob) - 4, len(blob) - 1):
            bad.write_bytes(blob[:cut])
            assert not L.snhip_rk_load(str(bad).encode()), cut
            assert _native.last_error()
        for off, val in ((0, 0x12345678), (4, 2), (4, 4)):   # magic, version
            b = bytearray(blob)
            struct.pack_into("<i", b, off, val)
            bad.write_bytes(bytes(b))
            assert not L.snhip_rk_load(str(bad).encode()), (off, val)
        for rank in (0, 300, 6):                               # rank table, layer 0 Rw
            b = bytearray(blob)
            struct.pack_into("<i", b, 44, rank)
            bad.write_bytes(bytes(b))
            assert not L.snhip_rk_load(str(bad).encode()), rank
        b = bytearray(blob)
        first_tag = 44 + 16 * RWKV_TINY.layers
        struct.pack_into("<i", b, first_tag, 7)                # ln1 tag: neither fp32 nor INT4
        bad.write_bytes(bytes(b))
        assert not L.snhip_rk_load(str(bad).encode())
        h = L.snhip_rk_load(str(src).encode())
        assert h
        L.snhip_rk_free(h)


@pytest.mark.parametrize("layer", [0, 1])
def test_dbg_equals_reference_sn_rk_dbg(gpu, tiny, monkeypatch, ref_built, layer):
    """snhip_rk_dbg mirrors sn_rk_dbg (rwkv7.c:366-374): after the same steps
    on both handles, the nine intermediates of the layer (xn, r, k, v, a, g,
    ww, y, x) equal the reference's own dump bit for bit, and both handles
    keep stepping identically afterwards (the dump advanced the same
    layers' state)."""
    w, p32 = tiny[0], tiny[1]
    hm = HipRwkv7(p32, RWKV_TINY.vocab)
    ref = oracle.RefRk(p32, RWKV_TINY.vocab)
    for t in (5, 77, 300):
        assert np.array_equal(np.asarray(hm.step(t), np.float32), ref.step(t))
    print(f"rwkv7 dbg layer {layer}", flush=True)
    a = hm.dbg(41, layer)
    b = ref.dbg(41, layer, RWKV_TINY.dim)
    for i, name in enumerate(("xn", "r", "k", "v", "a", "g", "ww", "y", "x")):
        assert np.array_equal(a[i], b[i]), name
    for t in (9, 200):
        assert np.array_equal(np.asarray(hm.step(t), np.float32), ref.step(t))
    with pytest.raises(RuntimeError):
        hm.dbg(RWKV_TINY.vocab, 0)
    with pytest.raises(RuntimeError):
        hm.dbg(1, RWKV_TINY.layers)
    hm.close()
    ref.close()
