"""The persistent single-sequence decode (one cooperative launch per call,
grid barriers between the phases of every layer) against the oracle and the
per-kernel step path.

Bar as for every decode path: logits within 2e-5 absolute of the C oracle
(bit-identical to the reference's sn_step), the greedy token equal to the
oracle's argmax on every step. INT4 compares with the oracle on the
bit-identically dequantized weights.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from sunnynet_amd.blob import pack_sunny_blob
from sunnynet_amd.config import SMALL, SUNNY_100M, TINY
from sunnynet_amd.runtime.model import HipModel
from sunnynet_amd.weights import gaussian_matmuls, init_sunnynet
from tests.test_decode_gpu import dequant_blob

pytestmark = pytest.mark.gpu
TOL = 2e-5


def _model(path, cfg, **kw):
    return HipModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, **kw)


def _blob(tmp_path_factory, name, buf):
    p = tmp_path_factory.mktemp("pblobs") / name
    p.write_bytes(buf)
    return p


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    w = init_sunnynet(TINY, 0)
    buf = pack_sunny_blob(w)
    return w, buf, _blob(tmp_path_factory, "tiny.bin", buf)


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    w = init_sunnynet(SMALL, 0)
    buf = pack_sunny_blob(w)
    return w, buf, _blob(tmp_path_factory, "small.bin", buf)


@pytest.fixture(scope="module")
def small_int4_path(tmp_path_factory):
    """SunnyNet small with N(0, 0.02) matmuls: the fp32 blob (quantized to
    INT4 g32 at load) and the blob of its dequantized weights (the oracle's)."""
    w = gaussian_matmuls(init_sunnynet(SMALL, 0), seed=3)
    return _blob(tmp_path_factory, "small_g.bin", pack_sunny_blob(w)), dequant_blob(w, 32)


def _greedy_vs_oracle(gpu, hm, orc, start, n):
    """decode_greedy on the device vs the oracle's greedy chain; also the
    last step's logits."""
    lg = torch.empty(hm.vocab, device=gpu)
    out = hm.decode_greedy(torch.tensor([start], dtype=torch.int32, device=gpu), n,
                           logits=lg).cpu().numpy()[:, 0]
    cur = start
    for i in range(n):
        ref = orc.step([cur])[0]
        nxt = int(ref.argmax())
        assert out[i] == nxt, f"step {i}: {out[i]} != {nxt}"
        cur = nxt
    d = float(np.abs(lg.cpu().numpy() - ref).max())
    assert d < TOL, d
    return out


def test_enabled_and_switch(gpu, tiny, monkeypatch):
    w, buf, path = tiny
    hm = _model(path, TINY)
    assert hm.persistent_grid > 0
    monkeypatch.setenv("SNHIP_PERSIST", "0")
    assert _model(path, TINY).persistent_grid == 0


def test_step_matches_per_kernel_path(gpu, small, monkeypatch):
    """The same tokens through both paths of one model: logits within TOL of
    each other and of the oracle, and the same state afterwards."""
    w, buf, path = small
    print("small fp32: persistent vs per-kernel, 40 steps", flush=True)
    hp = _model(path, SMALL)
    monkeypatch.setenv("SNHIP_PERSIST", "0")
    hk = _model(path, SMALL)
    assert hp.persistent_grid > 0 and hk.persistent_grid == 0
    orc = oracle.SnOracle(buf)
    for t in np.random.default_rng(5).integers(0, SMALL.vocab_size, 40):
        a = np.asarray(hp.step(int(t)), np.float32)
        b = np.asarray(hk.step(int(t)), np.float32)
        r = orc.step([t])[0]
        assert np.abs(a - r).max() < TOL and np.abs(a - b).max() < TOL
        assert a.argmax() == r.argmax()
    sp, hpst = hp.get_state(1)
    sk, hkst = hk.get_state(1)
    assert float((sp - sk).abs().max()) < 1e-5 and float((hpst - hkst).abs().max()) < 1e-5


@pytest.mark.parametrize("grid", [1, 3, 8, 64, 512])
def test_grid_sizes(gpu, tiny, monkeypatch, grid):
    """Any grid size gives the same tokens: one workgroup doing every phase,
    grids that are not a multiple of the 8 barrier groups, fewer workgroups
    than channel groups, two workgroups per CU."""
    w, buf, path = tiny
    print(f"tiny fp32 persistent grid={grid}", flush=True)
    monkeypatch.setenv("SNHIP_PERSIST_WG", str(grid))
    hm = _model(path, TINY)
    assert 0 < hm.persistent_grid <= grid
    _greedy_vs_oracle(gpu, hm, oracle.SnOracle(buf), 7, 48)


def test_long_greedy_tiny(gpu, tiny):
    """300 greedy steps in one launch (14 700 grid barriers on TINY)."""
    w, buf, path = tiny
    print("tiny fp32 persistent greedy 300", flush=True)
    _greedy_vs_oracle(gpu, _model(path, TINY), oracle.SnOracle(buf), 11, 300)


def test_prefill_then_persistent_greedy(gpu, small):
    """Chunked prefill (matrix-core path) hands its state to the persistent
    greedy decode; then single steps continue from the greedy state."""
    w, buf, path = small
    print("small fp32: prefill 100 + persistent greedy 32 + 4 steps", flush=True)
    hm = _model(path, SMALL)
    orc = oracle.SnOracle(buf)
    prompt = np.random.default_rng(2).integers(0, SMALL.vocab_size, 100).astype(np.int32)
    lg = hm.prefill_batch(torch.from_numpy(prompt[None]).to(gpu))[0].cpu().numpy()
    for t in prompt:
        ref = orc.step([t])[0]
    assert np.abs(lg - ref).max() < TOL
    out = _greedy_vs_oracle(gpu, hm, orc, int(ref.argmax()), 32)
    cur = int(out[-1])
    for _ in range(4):
        a = np.asarray(hm.step(cur), np.float32)
        r = orc.step([cur])[0]
        assert np.abs(a - r).max() < TOL
        cur = int(r.argmax())


@pytest.mark.parametrize("block", [32, 64])
def test_int4_greedy(gpu, tmp_path_factory, block):
    print(f"small int4 g{block} persistent greedy 40", flush=True)
    w = gaussian_matmuls(init_sunnynet(SMALL, 0), seed=3)
    path = _blob(tmp_path_factory, f"small_g{block}.bin", pack_sunny_blob(w))
    hm = _model(path, SMALL, weights="int4", block=block)
    assert hm.persistent_grid > 0
    _greedy_vs_oracle(gpu, hm, oracle.SnOracle(dequant_blob(w, block)), 3, 40)


def test_100m_fp32_and_int4(gpu, tmp_path_factory):
    """SunnyNet-100M (12 layers, D=1024, V=32000): fp32 seed 1 and INT4 g32 on
    N(0, 0.02) matmuls (seed 3), 16 greedy steps each."""
    cfg = SUNNY_100M
    print("100M fp32 persistent greedy 16", flush=True)
    w = init_sunnynet(cfg, 1)
    buf = pack_sunny_blob(w)
    path = _blob(tmp_path_factory, "m100.bin", buf)
    _greedy_vs_oracle(gpu, _model(path, cfg), oracle.SnOracle(buf), 17, 16)
    print("100M int4 g32 persistent greedy 16", flush=True)
    wq = gaussian_matmuls(w, seed=3)
    pq = _blob(tmp_path_factory, "m100q.bin", pack_sunny_blob(wq))
    _greedy_vs_oracle(gpu, _model(pq, cfg, weights="int4", block=32),
                      oracle.SnOracle(dequant_blob(wq, 32)), 17, 16)


def test_barrier_timeout_reports_error(gpu, tiny, monkeypatch):
    """A barrier target the host raised out of reach: every workgroup gives up
    after its poll limit and leaves the kernel, and the call reports the error
    (device-tensor step, greedy decoding and host step alike). Workgroups stop
    independently and write their channels' state back after their own last
    wait, so a timed-out call may leave sequence 0 part-stepped: the handle
    then refuses every stepping call until a state is set (or reset), after
    which it continues from that state as the oracle does."""
    w, buf, path = tiny
    monkeypatch.setenv("SNHIP_PERSIST_SPIN", "2048")
    hm = _model(path, TINY)
    assert hm.persistent_grid > 0
    orc = oracle.SnOracle(buf)
    t = torch.tensor([3], dtype=torch.int32, device=gpu)
    a = hm.step_batch(t).cpu().numpy()[0]          # a non-zero state to restore later
    assert np.abs(a - orc.step([3])[0]).max() < TOL
    saved = [x.clone() for x in hm.get_state(1)]
    print("persistent time-out: device step, greedy, host step", flush=True)
    calls = [lambda: hm.step_batch(t), lambda: hm.decode_greedy(t, 4),
             lambda: hm.step_batch_host([3]), lambda: hm.step(3)]
    for call in calls:
        monkeypatch.setenv("SNHIP_PERSIST_STALL", "1")
        with pytest.raises(RuntimeError, match="timed out"):
            call()
        monkeypatch.delenv("SNHIP_PERSIST_STALL")
        with pytest.raises(RuntimeError, match="part-stepped"):
            call()
        hm.set_state(*saved)
    monkeypatch.delenv("SNHIP_PERSIST_SPIN")
    a = hm.step_batch(t).cpu().numpy()[0]
    assert np.abs(a - orc.step([3])[0]).max() < TOL
    b = np.asarray(hm.step(5), np.float32)
    assert np.abs(b - orc.step([5])[0]).max() < TOL


@pytest.mark.parametrize("B", [1, 8])
def test_ordinary_launch_equals_cooperative(gpu, small, monkeypatch, B):
    """SNHIP_COOP=0 launches the same co-resident grid without the
    cooperative flag (for tools that do not handle cooperative launches):
    the B=1 persistent kernel and the batched one give the same tokens and
    logits, bit for bit."""
    w, buf, path = small
    print(f"cooperative vs ordinary launch, B={B}", flush=True)
    start = torch.arange(3, 3 + B, dtype=torch.int32, device=gpu)
    res = []
    for coop in ("1", "0"):
        monkeypatch.setenv("SNHIP_COOP", coop)
        hm = _model(path, SMALL, max_batch=B)
        assert (hm.persistent_grid if B == 1 else hm.batch_grid) > 0
        lg = torch.empty(B, SMALL.vocab_size, device=gpu)
        toks = hm.decode_greedy(start, 12, logits=lg)
        res.append((toks.cpu(), lg.cpu()))
        hm.close()
    assert torch.equal(res[0][0], res[1][0])
    assert torch.equal(res[0][1], res[1][1])


@pytest.mark.parametrize("fmt,B", [("int4", 2), ("int4", 5), ("int4", 16), ("fp32", 3)])
def test_sequences_on_grid_slices(gpu, small, small_int4_path, fmt, B):
    """Steps of B sequences run as B copies of the single-sequence kernel in
    one launch, each on its own slice of the grid: after a prefill, every
    sequence's greedy tokens, last logits, state and history equal those of
    its own one-sequence launch bit for bit, and so do single steps (device
    tokens); from the zero state the greedy chains follow the oracle (on the
    dequantized weights for INT4) within 2e-5 with the same argmax."""
    if fmt == "int4":
        path, dq = small_int4_path
        kw = dict(weights="int4", block=32)
    else:
        _, dq, path = small
        kw = {}
    hm = _model(path, SMALL, max_batch=B, **kw)
    h1 = _model(path, SMALL, **kw)
    assert h1.persistent_grid > 0
    g = hm.persistent_grid_for(B)
    assert g > 0 and g % B == 0, g
    print(f"small {fmt} B={B}: {g // B} workgroups per sequence", flush=True)
    rng = np.random.default_rng(100 + B)
    prompts = rng.integers(0, SMALL.vocab_size, (B, 20)).astype(np.int32)
    hm.prefill_batch(torch.from_numpy(prompts).to(gpu))
    s0, k0 = (x.clone() for x in hm.get_state(B))
    start = torch.from_numpy(rng.integers(0, SMALL.vocab_size, B).astype(np.int32)).to(gpu)
    n = 9
    lg = torch.empty(B, SMALL.vocab_size, device=gpu)
    out = hm.decode_greedy(start, n, logits=lg).cpu().numpy()
    s1, k1 = (x.cpu().numpy() for x in hm.get_state(B))
    one = hm.step_batch(torch.from_numpy(out[-1]).to(gpu)).cpu().numpy()
    lg = lg.cpu().numpy()
    for b in range(B):
        h1.set_state(s0[b:b + 1], k0[b:b + 1])
        lb = torch.empty(1, SMALL.vocab_size, device=gpu)
        ob = h1.decode_greedy(start[b:b + 1], n, logits=lb).cpu().numpy()[:, 0]
        assert np.array_equal(ob, out[:, b]), b
        assert np.array_equal(lb.cpu().numpy()[0], lg[b]), b
        sb, kb = (x.cpu().numpy()[0] for x in h1.get_state(1))
        assert np.array_equal(sb, s1[b]) and np.array_equal(kb, k1[b]), b
        step = h1.step_batch(torch.from_numpy(out[-1, b:b + 1]).to(gpu)).cpu().numpy()[0]
        assert np.array_equal(step, one[b]), b
    hm.reset()
    orc = oracle.SnOracle(dq, batch=B)
    cur = rng.integers(0, SMALL.vocab_size, B).astype(np.int32)
    out = hm.decode_greedy(torch.from_numpy(cur).to(gpu), 6).cpu().numpy()
    for i in range(6):
        ref = orc.step(cur)
        nxt = ref.argmax(1).astype(np.int32)
        assert np.array_equal(out[i], nxt), i
        cur = nxt
    a = hm.step_batch(torch.from_numpy(cur).to(gpu)).cpu().numpy()
    assert np.abs(a - orc.step(cur)).max() < TOL
    hm.close()
    h1.close()


def test_sequences_on_grid_slices_timeout(gpu, small_int4_path, monkeypatch):
    """A time-out in a launch of four sequences ends every slice (the error
    word is shared): the call reports it, all four sequences are refused as
    part-stepped, setting the state of three of them is not enough, and after
    all four are set the handle steps them as the oracle does."""
    path, dq = small_int4_path
    B = 4
    monkeypatch.setenv("SNHIP_PERSIST_SPIN", "2048")
    hm = _model(path, SMALL, weights="int4", block=32, max_batch=B)
    assert hm.persistent_grid_for(B) > 0
    orc = oracle.SnOracle(dq, batch=B)
    cur = np.array([7, 9, 11, 13], np.int32)
    t = torch.from_numpy(cur).to(gpu)
    a = hm.step_batch(t).cpu().numpy()
    assert np.abs(a - orc.step(cur)).max() < TOL
    saved = [x.clone() for x in hm.get_state(B)]
    print("four sequences on grid slices: time-out", flush=True)
    monkeypatch.setenv("SNHIP_PERSIST_STALL", "1")
    with pytest.raises(RuntimeError, match="timed out"):
        hm.decode_greedy(t, 2)
    monkeypatch.delenv("SNHIP_PERSIST_STALL")
    with pytest.raises(RuntimeError, match="part-stepped"):
        hm.step_batch(t)
    hm.set_state(saved[0][:3], saved[1][:3])
    with pytest.raises(RuntimeError, match="part-stepped"):
        hm.step_batch(t)
    hm.set_state(*saved)
    monkeypatch.delenv("SNHIP_PERSIST_SPIN")
    a = hm.step_batch(t).cpu().numpy()
    assert np.abs(a - orc.step(cur)).max() < TOL
    hm.close()
