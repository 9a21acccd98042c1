"""The exact one-launch RWKV-7 step (rkexact.hip), the default for one
sequence and for 2..8 sequences on grid slices, against the oracle.

Bar: logits, S and shift EQUAL the oracle's bit for bit (the oracle is
bit-identical to the reference's sn_rk_step on fp32 blobs; INT4 handles are
held to the oracle run on the bit-identically dequantized weights), step
after step and over greedy chains whose every token is checked. The kernel
keeps the reference's rounding order: every product output is one sequential
FMA chain over its inputs, LayerNorm and group-norm sums are sequential, and
expf / tanhf are glibc's algorithms.

Its code paths depend on the grid: with one workgroup per CU (256 on the
MI355X) the head owners take no first-product rows and stage their operands
meanwhile, every phase's weights are issued in one piece before its wait,
and the output and channel-mix value products (3 rows per workgroup) run on
lane-sliced chains; smaller grids (SNHIP_RK_PERSIST_WG, and the slices of
batched steps) give owners rows, stage weights in chunks and run every
product on LDS-fed chains. The tests run each of those shapes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from sunnynet_amd.runtime.rwkv7 import HipRwkv7
from sunnynet_amd.rwkv7 import RWKV_CFG4, RWKV_TINY, init_rwkv7, pack_rwkv7_blob
from tests.test_rwkv7_gpu import dequant_weights

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _exact_default(monkeypatch):
    for k in ("SNHIP_RK_PERSIST", "SNHIP_RK_EXACT", "SNHIP_RK_PERSIST_WG", "SNHIP_RK_PERSIST_MI"):
        monkeypatch.delenv(k, raising=False)


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    w = init_rwkv7(RWKV_TINY, 7)
    d = tmp_path_factory.mktemp("rke")
    p32 = d / "tiny.bin"
    p32.write_bytes(pack_rwkv7_blob(w))
    p4 = d / "tiny_q4.bin"
    p4.write_bytes(pack_rwkv7_blob(w, int4=True))
    return w, p32, p4


@pytest.fixture(scope="module")
def cfg4(tmp_path_factory):
    """12 layers, D=768, 12 heads, F=3072, vocab 65536 (seed 2): the fp32
    blob, and the oracle's blob of its INT4 g32 dequantized weights."""
    print("rwkv7 cfg4 exact: generating weights", flush=True)
    w = init_rwkv7(RWKV_CFG4, 2)
    p = tmp_path_factory.mktemp("rke4") / "cfg4.bin"
    p.write_bytes(pack_rwkv7_blob(w))
    return p, pack_rwkv7_blob(dequant_weights(w, 32))


def _handle(path, monkeypatch, grid=None, **kw):
    if grid:
        monkeypatch.setenv("SNHIP_RK_PERSIST_WG", str(grid))
    h = HipRwkv7(path, **kw)
    monkeypatch.delenv("SNHIP_RK_PERSIST_WG", raising=False)
    assert h.persist_grid > 0 and h.persist_exact, h.persist_grid
    if grid:
        assert h.persist_grid == grid, (h.persist_grid, grid)
    return h


def _same_steps(h, orc, toks):
    for t in toks:
        a = np.asarray(h.step(int(t)), np.float32)
        b = orc.step([t])[0]
        assert np.array_equal(a, b), (int(t), float(np.abs(a - b).max()))


def _same_state(h, orc, B=1):
    S, sh = h.get_state(B)
    So, sho = orc.get_state()
    assert np.array_equal(S.cpu().numpy(), So) and np.array_equal(sh.cpu().numpy(), sho)


def test_default_selection(gpu, tiny, monkeypatch):
    """The handle as loaded runs the exact kernel; SNHIP_RK_PERSIST=1 picks
    the fast one instead, SNHIP_RK_EXACT=0 the per-kernel step."""
    w, p32, _ = tiny
    h = HipRwkv7(p32, max_batch=8)
    assert h.persist_grid > 0 and h.persist_exact and h.persist_grid_for(8) > 0
    monkeypatch.setenv("SNHIP_RK_PERSIST", "1")
    hf = HipRwkv7(p32)
    assert hf.persist_grid > 0 and not hf.persist_exact
    monkeypatch.delenv("SNHIP_RK_PERSIST")
    monkeypatch.setenv("SNHIP_RK_EXACT", "0")
    assert HipRwkv7(p32).persist_grid == 0


@pytest.mark.parametrize("fmt", ["fp32", "int4_blob", "int4_g32"])
@pytest.mark.parametrize("grid", [None, 64, 16])
def test_tiny_steps_exact(gpu, tiny, monkeypatch, fmt, grid):
    """24 steps from the reset state, then a set state: logits and states
    identical to the oracle's, on the default grid and on 64 and 16
    workgroups (owners with rows, chunked weights)."""
    w, p32, p4 = tiny
    print(f"rwkv7 exact tiny {fmt} grid {grid}", flush=True)
    if fmt == "fp32":
        h, ob = _handle(p32, monkeypatch, grid), p32.read_bytes()
    elif fmt == "int4_blob":
        h, ob = _handle(p4, monkeypatch, grid), p4.read_bytes()
    else:
        h = _handle(p32, monkeypatch, grid, weights="int4", block=32)
        ob = pack_rwkv7_blob(dequant_weights(w, 32))
    orc = oracle.RkOracle(ob)
    _same_steps(h, orc, np.random.default_rng(1).integers(0, RWKV_TINY.vocab, 24))
    _same_state(h, orc)
    cfg = RWKV_TINY
    g = torch.Generator().manual_seed(3)
    S = torch.randn(1, cfg.layers, cfg.n_head, 64, 64, generator=g) * 0.1
    sh = torch.randn(1, cfg.layers, 2, cfg.dim, generator=g)
    h.set_state(S.cuda(), sh.cuda())
    orc.set_state(S.numpy(), sh.numpy())
    _same_steps(h, orc, [7, 100, 311])
    _same_state(h, orc)
    h.close()


def test_tiny_greedy_exact(gpu, tiny, monkeypatch):
    """One launch for all of a greedy call's steps: every token the oracle's
    argmax of the oracle's logits, the last logits and the state identical."""
    w, p32, _ = tiny
    h = _handle(p32, monkeypatch)
    orc = oracle.RkOracle(p32.read_bytes())
    for t in (5, 9, 200):
        h.step(t)
        orc.step([t])
    n = 20
    lg = torch.empty(1, RWKV_TINY.vocab, device="cuda")
    out = h.decode_greedy(torch.tensor([17], dtype=torch.int32, device="cuda"), n, logits=lg).cpu().numpy()[:, 0]
    cur = np.array([17], np.int32)
    for i in range(n):
        r = orc.step(cur)
        nxt = r.argmax(1).astype(np.int32)
        assert out[i] == nxt[0], i
        cur = nxt
    assert np.array_equal(lg.cpu().numpy()[0], r[0])
    _same_state(h, orc)
    h.close()


@pytest.mark.parametrize("grid", [None, 128, 32, 16])
def test_cfg4_first_steps_exact(gpu, cfg4, monkeypatch, grid):
    """The 12-layer INT4 g32 model from the reset state: first steps of
    random tokens identical to the oracle's (the fast kernel was up to
    1.26e-4 off on such steps), on the default grid (lane-sliced chains) and
    on 128, 32 and 16 workgroups."""
    p, dq = cfg4
    print(f"rwkv7 exact cfg4 first steps, grid {grid}", flush=True)
    h = _handle(p, monkeypatch, grid, weights="int4", block=32)
    orc = oracle.RkOracle(dq)
    rng = np.random.default_rng(1234)
    for _ in range(4 if grid else 8):
        t = int(rng.integers(0, RWKV_CFG4.vocab))
        h.reset()
        orc.reset()
        a = np.asarray(h.step(t), np.float32)
        b = orc.step([t])[0]
        assert np.array_equal(a, b), (t, float(np.abs(a - b).max()))
    h.close()


def test_cfg4_greedy_chain_exact(gpu, cfg4, monkeypatch):
    """A 32-token prompt by steps, then 24 greedy steps in one launch: every
    token and the last logits identical to the oracle's chain."""
    p, dq = cfg4
    cfg = RWKV_CFG4
    print("rwkv7 exact cfg4 greedy chain", flush=True)
    h = _handle(p, monkeypatch, weights="int4", block=32)
    orc = oracle.RkOracle(dq)
    prompt = np.random.default_rng(8).integers(0, cfg.vocab, 32).astype(np.int32)
    lg = torch.empty(1, cfg.vocab, device="cuda")
    for t in prompt:
        h.step_batch(torch.tensor([t], dtype=torch.int32, device="cuda"), out=lg)
        r = orc.step([t])
    assert np.array_equal(lg.cpu().numpy()[0], r[0])
    cur = r.argmax(1).astype(np.int32)
    n = 24
    out = h.decode_greedy(torch.from_numpy(cur).cuda(), n, logits=lg).cpu().numpy()[:, 0]
    for i in range(n):
        r = orc.step(cur)
        nxt = r.argmax(1).astype(np.int32)
        assert out[i] == nxt[0], i
        cur = nxt
    assert np.array_equal(lg.cpu().numpy()[0], r[0])
    h.close()


@pytest.mark.parametrize("B", [2, 3, 8])
def test_cfg4_slices_exact(gpu, cfg4, B):
    """B sequences on a grid slice each (one launch): single steps from the
    reset state and a greedy call, each sequence identical to the oracle."""
    p, dq = cfg4
    cfg = RWKV_CFG4
    h = HipRwkv7(p, weights="int4", block=32, max_batch=B)
    g = h.persist_grid_for(B)
    assert g > 0 and g % B == 0 and h.persist_exact
    print(f"rwkv7 exact cfg4 B={B}: {g // B} workgroups per sequence", flush=True)
    orc = oracle.RkOracle(dq, batch=B)
    rng = np.random.default_rng(40 + B)
    for _ in range(2):
        t = rng.integers(0, cfg.vocab, B).astype(np.int32)
        a = h.step_batch(torch.from_numpy(t).cuda()).cpu().numpy()
        assert np.array_equal(a, orc.step(t))
    cur = rng.integers(0, cfg.vocab, B).astype(np.int32)
    n = 6
    lg = torch.empty(B, cfg.vocab, device="cuda")
    out = h.decode_greedy(torch.from_numpy(cur).cuda(), n, logits=lg).cpu().numpy()
    for i in range(n):
        r = orc.step(cur)
        nxt = r.argmax(1).astype(np.int32)
        assert np.array_equal(out[i], nxt), i
        cur = nxt
    assert np.array_equal(lg.cpu().numpy(), r)
    h.close()


def test_tiny_slices_every_batch_exact(gpu, tiny):
    """B = 2..8 on the tiny model (slices of 128 down to 32 workgroups): two
    steps each from the reset state, identical to the oracle."""
    w, p32, _ = tiny
    h = HipRwkv7(p32, max_batch=8)
    rng = np.random.default_rng(77)
    for B in range(2, 9):
        assert h.persist_grid_for(B) > 0, B
        h.reset()
        orc = oracle.RkOracle(p32.read_bytes(), batch=B)
        for _ in range(2):
            t = rng.integers(0, RWKV_TINY.vocab, B).astype(np.int32)
            a = h.step_batch(torch.from_numpy(t).cuda()).cpu().numpy()
            assert np.array_equal(a, orc.step(t)), B
    h.close()


def test_timeout_reports_error(gpu, tiny, monkeypatch):
    """Every exchange wait given a target the host raised out of reach (each
    workgroup gives up after its poll limit and leaves the kernel): one
    sequence and three slices, a step and a greedy call, each reported as an
    error; the handle then refuses steps until reset() or set_state(), and
    after that matches the oracle bit for bit again."""
    w, p32, _ = tiny
    cfg = RWKV_TINY
    monkeypatch.setenv("SNHIP_PERSIST_SPIN", "2048")
    h = _handle(p32, monkeypatch, max_batch=3)
    assert h.persist_grid_for(3) > 0
    monkeypatch.setenv("SNHIP_PERSIST_STALL", "1")
    print("rwkv7 exact time-out", flush=True)
    with pytest.raises(RuntimeError, match="timed out"):
        h.step_batch(torch.tensor([3], dtype=torch.int32, device="cuda"))
    with pytest.raises(RuntimeError, match="part-stepped"):
        h.step(3)
    h.reset()
    with pytest.raises(RuntimeError, match="timed out"):
        h.decode_greedy(torch.tensor([3, 40, 500], dtype=torch.int32, device="cuda"), 3)
    monkeypatch.delenv("SNHIP_PERSIST_STALL")
    with pytest.raises(RuntimeError, match="part-stepped"):
        h.step_batch(torch.tensor([3, 40, 500], dtype=torch.int32, device="cuda"))
    h.reset()
    orc = oracle.RkOracle(p32.read_bytes())
    _same_steps(h, orc, [3, 4])
    S = torch.zeros(3, cfg.layers, cfg.n_head, 64, 64, device="cuda")
    sh = torch.zeros(3, cfg.layers, 2, cfg.dim, device="cuda")
    monkeypatch.setenv("SNHIP_PERSIST_STALL", "1")
    with pytest.raises(RuntimeError, match="timed out"):
        h.step_batch(torch.tensor([1, 2, 3], dtype=torch.int32, device="cuda"))
    monkeypatch.delenv("SNHIP_PERSIST_STALL")
    h.set_state(S, sh)
    orc3 = oracle.RkOracle(p32.read_bytes(), batch=3)
    t = np.array([9, 99, 199], np.int32)
    assert np.array_equal(h.step_batch(torch.from_numpy(t).cuda()).cpu().numpy(), orc3.step(t))
    h.close()
