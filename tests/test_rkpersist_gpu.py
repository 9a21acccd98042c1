"""The fast one-launch-per-step RWKV-7 kernel (rkpersist.hip), opt-in with
SNHIP_RK_PERSIST=1 (every test here sets it), against the oracle and against
the per-kernel step.

Bar: logits within PTOL = 2e-4 absolute of the C oracle (bit-identical to the
reference's sn_rk_step on fp32 blobs) with the same argmax on every step,
states within the tolerances of tests/test_rwkv7_gpu.py. This path sums its
products and LayerNorms in parallel rather than in the reference's sequential
order, and RWKV-7 amplifies that rounding, most from the zero state: on the
12-layer INT4 model its logits were up to 1.26e-4 from sn_rk_step over 256
first steps (32 of them past 2e-5) and up to 2.7e-5 over the benchmark's
640-step chain. That is why it is not the default: the default one-launch
kernel (rkexact.hip, tests/test_rkexact_gpu.py) and the per-kernel step are
bit-exact. For comparison, the reference's own
tests hold its C runtime to 1e-3 against its numpy restatement
(tests/test_rwkv7_c.py:29-50). Covers fp32, the INT4 blob as stored (group
64, the 32-input V_2 kept fp32) and INT4 group 32 quantized at load, the
12-layer 65536-vocab configuration, greedy decoding, where one launch runs
every step of the call (each workgroup reducing the argmax keys to the next
token itself), and steps of 2..8 sequences on a grid slice each
(bit-identical to one-sequence launches).
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
PTOL = 2e-4


@pytest.fixture(autouse=True)
def _persist_on(monkeypatch):
    monkeypatch.setenv("SNHIP_RK_PERSIST", "1")


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    w = init_rwkv7(RWKV_TINY, 7)
    d = tmp_path_factory.mktemp("rkp")
    p32 = d / "tiny.bin"
    p32.write_bytes(pack_rwkv7_blob(w))
    p4 = d / "tiny_q4.bin"
    p4.write_bytes(pack_rwkv7_blob(w, int4=True))
    return w, p32, p4


@pytest.fixture(scope="module")
def cfg4(tmp_path_factory):
    """12 layers, D=768, 12 heads, F=3072, vocab 65536 (seed 2): the fp32
    blob, and the oracle's blob of its INT4 g32 dequantized weights."""
    print("rwkv7 cfg4 persistent: generating weights", flush=True)
    w = init_rwkv7(RWKV_CFG4, 2)
    p = tmp_path_factory.mktemp("rkp4") / "cfg4.bin"
    p.write_bytes(pack_rwkv7_blob(w))
    return p, pack_rwkv7_blob(dequant_weights(w, 32))


def _pair(path, monkeypatch, **kw):
    """The fast kernel's handle and a per-kernel one."""
    hp = HipRwkv7(path, **kw)
    monkeypatch.setenv("SNHIP_RK_PERSIST", "0")
    monkeypatch.setenv("SNHIP_RK_EXACT", "0")
    hg = HipRwkv7(path, **kw)
    monkeypatch.setenv("SNHIP_RK_PERSIST", "1")
    monkeypatch.delenv("SNHIP_RK_EXACT")
    assert hp.persist_grid > 0 and not hp.persist_exact and hg.persist_grid == 0
    return hp, hg


@pytest.mark.parametrize("fmt", ["fp32", "int4_blob", "int4_g32"])
def test_persist_matches_oracle_and_per_kernel_step(gpu, tiny, monkeypatch, fmt):
    w, p32, p4 = tiny
    print(f"rwkv7 persistent B=1 tiny {fmt}", flush=True)
    if fmt == "fp32":
        hp, hg = _pair(p32, monkeypatch)
        orc = oracle.RkOracle(p32.read_bytes())
    elif fmt == "int4_blob":
        hp, hg = _pair(p4, monkeypatch)
        orc = oracle.RkOracle(p4.read_bytes())
    else:
        hp, hg = _pair(p32, monkeypatch, weights="int4", block=32)
        orc = oracle.RkOracle(pack_rwkv7_blob(dequant_weights(w, 32)))
    for t in np.random.default_rng(11).integers(0, RWKV_TINY.vocab, 24):
        a = np.asarray(hp.step(int(t)), np.float32)
        g = np.asarray(hg.step(int(t)), np.float32)
        b = orc.step([t])[0]
        assert np.abs(a - b).max() < PTOL and np.abs(a - g).max() < PTOL
        assert a.argmax() == b.argmax() == g.argmax()
    S, sh = hp.get_state(1)
    So, sho = orc.get_state()
    assert np.abs(S.cpu().numpy() - So).max() < 1e-4 and np.abs(sh.cpu().numpy() - sho).max() < 1e-5


def test_persist_greedy_matches_oracle_chain(gpu, tiny):
    w, p32, _ = tiny
    n = 20
    print(f"rwkv7 persistent greedy tiny n={n}", flush=True)
    hm = HipRwkv7(p32)
    assert hm.persist_grid > 0
    orc = oracle.RkOracle(p32.read_bytes())
    lg = torch.empty(1, RWKV_TINY.vocab, device="cuda")
    start = np.array([42], np.int32)
    out = hm.decode_greedy(torch.from_numpy(start).cuda(), n, logits=lg).cpu().numpy()
    cur = start
    for i in range(n):
        ref = orc.step(cur)
        nxt = ref.argmax(1).astype(np.int32)
        assert np.array_equal(out[i], nxt), i
        cur = nxt
    assert np.abs(lg.cpu().numpy() - ref).max() < PTOL
    # A second call continues from the state the first one left.
    out2 = hm.decode_greedy(torch.from_numpy(cur).cuda(), 4).cpu().numpy()
    for i in range(4):
        nxt = orc.step(cur).argmax(1).astype(np.int32)
        assert np.array_equal(out2[i], nxt), i
        cur = nxt


def test_persist_cfg4_int4(gpu, cfg4, monkeypatch):
    """12 layers, D=768, 12 heads, F=3072, vocab 65536, INT4 g32 at load."""
    cfg = RWKV_CFG4
    p, ob = cfg4
    orc = oracle.RkOracle(ob)
    hp, hg = _pair(p, monkeypatch, weights="int4", block=32)
    print("rwkv7 cfg4 persistent: stepping", flush=True)
    for t in np.random.default_rng(5).integers(0, cfg.vocab, 4):
        a = np.asarray(hp.step(int(t)), np.float32)
        g = np.asarray(hg.step(int(t)), np.float32)
        b = orc.step([t])[0]
        print("worst |dlogit| persist", float(np.abs(a - b).max()), "per-kernel", float(np.abs(g - b).max()),
              flush=True)
        assert np.abs(a - b).max() < PTOL and np.abs(a - g).max() < PTOL
        assert a.argmax() == b.argmax() == g.argmax()


def test_persist_cfg4_first_step_deviation(gpu, cfg4):
    """The deviation that keeps this path opt-in, measured: 64 first steps
    from the zero state (8 launches of 8 grid slices, each sequence's result
    that of its own one-sequence launch) of the 12-layer INT4 g32 model
    against the oracle: every logit within PTOL, every argmax equal."""
    p, ob = cfg4
    hm = HipRwkv7(p, weights="int4", block=32, max_batch=8)
    assert hm.persist_grid_for(8) > 0
    orc = oracle.RkOracle(ob, batch=8)
    rng = np.random.default_rng(1234)
    devs = []
    for _ in range(8):
        t = rng.integers(0, RWKV_CFG4.vocab, 8).astype(np.int32)
        hm.reset()
        orc.reset()
        a = hm.step_batch(torch.from_numpy(t).cuda()).cpu().numpy()
        r = orc.step(t)
        devs += list(np.abs(a - r).max(axis=1))
        assert np.array_equal(a.argmax(1), r.argmax(1))
    devs = np.array(devs)
    print(f"rwkv7 cfg4 persistent first steps: max |dlogit| {devs.max():.3g}, "
          f"median {np.median(devs):.3g}, {(devs > 2e-5).sum()} of {devs.size} past 2e-5", flush=True)
    assert devs.max() < PTOL
    hm.close()


def test_persist_cfg4_greedy_chain(gpu, cfg4):
    """The benchmarked workload's form: greedy steps of the 12-layer INT4 g32
    model at one sequence, all in one launch, then a second call continuing
    from the state the first left; every token equal to the oracle chain's."""
    p, ob = cfg4
    hm = HipRwkv7(p, weights="int4", block=32)
    assert hm.persist_grid > 0
    orc = oracle.RkOracle(ob)
    n = 12
    print(f"rwkv7 cfg4 persistent greedy n={n}", flush=True)
    lg = torch.empty(1, RWKV_CFG4.vocab, device="cuda")
    cur = np.array([1234], np.int32)
    out = hm.decode_greedy(torch.from_numpy(cur).cuda(), n, logits=lg).cpu().numpy()
    for i in range(n):
        ref = orc.step(cur)
        nxt = ref.argmax(1).astype(np.int32)
        assert np.array_equal(out[i], nxt), i
        cur = nxt
    print("worst |dlogit| last step", float(np.abs(lg.cpu().numpy() - ref).max()), flush=True)
    assert np.abs(lg.cpu().numpy() - ref).max() < PTOL
    out2 = hm.decode_greedy(torch.from_numpy(cur).cuda(), 3).cpu().numpy()
    for i in range(3):
        nxt = orc.step(cur).argmax(1).astype(np.int32)
        assert np.array_equal(out2[i], nxt), i
        cur = nxt


def test_persist_cfg4_bench_chain(gpu, cfg4, tmp_path, ref_built):
    """The benchmark's B=1 chain at full length: a 512-token random prompt
    stepped one token per call, then 128 greedy steps in one launch, on one
    INT4 g32 handle. The reference's own sn_rk_step (oracle/_ref, built from
    rwkv7.c) runs the same chain on the blob of the dequantized weights: every
    greedy token equal, the prompt's last logits and the chain's last logits
    within PTOL (rwkv7.c:349-360)."""
    p, ob = cfg4
    rp = tmp_path / "cfg4_dq32.bin"
    rp.write_bytes(ob)
    ref = oracle.RefRk(rp, RWKV_CFG4.vocab)
    hm = HipRwkv7(p, weights="int4", block=32)
    assert hm.persist_grid > 0
    prompt = np.random.default_rng(512).integers(0, RWKV_CFG4.vocab, 512).astype(np.int32)
    lg = torch.empty(1, RWKV_CFG4.vocab, device="cuda")
    print("rwkv7 cfg4 B=1: 512-token prompt on the device", flush=True)
    for t in prompt:
        hm.step_batch(torch.tensor([int(t)], dtype=torch.int32, device="cuda"), out=lg)
    lg0 = lg.cpu().numpy()[0]
    print("rwkv7 cfg4 B=1: 512-token prompt on the reference", flush=True)
    for t in prompt:
        r0 = ref.step(int(t))
    d0 = float(np.abs(lg0 - r0).max())
    print(f"rwkv7 cfg4 B=1 prompt: last |dlogit| {d0:.3g}", flush=True)
    assert d0 < PTOL and lg0.argmax() == r0.argmax()
    n = 128
    last = torch.empty(1, RWKV_CFG4.vocab, device="cuda")
    toks = hm.decode_greedy(torch.tensor([int(lg0.argmax())], dtype=torch.int32, device="cuda"),
                            n, logits=last).cpu().numpy()[:, 0]
    tok, rl = int(r0.argmax()), None
    for i in range(n):
        rl = ref.step(tok)
        tok = int(rl.argmax())
        assert toks[i] == tok, f"greedy chain diverges at step {i}"
    d1 = float(np.abs(last.cpu().numpy()[0] - rl).max())
    print(f"rwkv7 cfg4 B=1 {n} greedy steps: tokens equal, last |dlogit| {d1:.3g}", flush=True)
    assert d1 < PTOL
    hm.close()
    ref.close()


@pytest.mark.parametrize("fmt,B", [("fp32", 2), ("int4_g32", 3), ("fp32", 8)])
def test_sequences_on_grid_slices(gpu, tiny, monkeypatch, fmt, B):
    """Steps of B = 2..8 sequences as B copies of the one-sequence kernel in
    one launch, each on its own slice of the grid: from a set state, every
    sequence's greedy tokens,
    last logits, S and shift equal those of a one-sequence launch on the same
    slice size bit for bit, and so does a single step; from the reset state,
    single steps follow the oracle within 2e-5 with the same argmax."""
    w, p32, _ = tiny
    cfg = RWKV_TINY
    kw = dict(weights="int4", block=32) if fmt == "int4_g32" else {}
    dq = pack_rwkv7_blob(dequant_weights(w, 32)) if fmt == "int4_g32" else p32.read_bytes()
    monkeypatch.setenv("SNHIP_RK_PERSIST_MI", "8")
    hm = HipRwkv7(p32, max_batch=B, **kw)
    assert HipRwkv7(p32, max_batch=2, **kw).persist_grid_for(2) > 0
    monkeypatch.setenv("SNHIP_RK_PERSIST_WG", str(hm.persist_grid_for(B) // B))
    h1 = HipRwkv7(p32, **kw)            # one sequence on the same slice size
    monkeypatch.delenv("SNHIP_RK_PERSIST_WG")
    g = hm.persist_grid_for(B)
    assert g > 0 and g % B == 0 and h1.persist_grid == g // B, (g, h1.persist_grid)
    print(f"rwkv7 tiny {fmt} B={B}: {g // B} workgroups per sequence", flush=True)
    rng = np.random.default_rng(30 + B)
    gen = torch.Generator().manual_seed(B)
    S = torch.randn(B, cfg.layers, cfg.n_head, 64, 64, generator=gen) * 0.1
    sh = torch.randn(B, cfg.layers, 2, cfg.dim, generator=gen)
    hm.set_state(S.cuda(), sh.cuda())
    start = torch.from_numpy(rng.integers(0, cfg.vocab, B).astype(np.int32)).cuda()
    n = 7
    lg = torch.empty(B, cfg.vocab, device="cuda")
    out = hm.decode_greedy(start, n, logits=lg).cpu().numpy()
    lg = lg.cpu().numpy()
    S1, sh1 = (x.cpu().numpy() for x in hm.get_state(B))
    one = hm.step_batch(torch.from_numpy(out[-1]).cuda()).cpu().numpy()
    for b in range(B):
        h1.set_state(S[b:b + 1].cuda(), sh[b:b + 1].cuda())
        lb = torch.empty(1, cfg.vocab, device="cuda")
        ob = h1.decode_greedy(start[b:b + 1], n, logits=lb).cpu().numpy()[:, 0]
        assert np.array_equal(ob, out[:, b]), b
        assert np.array_equal(lb.cpu().numpy()[0], lg[b]), b
        Sb, shb = (x.cpu().numpy()[0] for x in h1.get_state(1))
        assert np.array_equal(Sb, S1[b]) and np.array_equal(shb, sh1[b]), b
        step = h1.step_batch(torch.from_numpy(out[-1, b:b + 1]).cuda()).cpu().numpy()[0]
        assert np.array_equal(step, one[b]), b
    hm.reset()
    orc = oracle.RkOracle(dq, batch=B)
    for _ in range(5):
        t = rng.integers(0, cfg.vocab, B).astype(np.int32)
        a = hm.step_batch(torch.from_numpy(t).cuda()).cpu().numpy()
        r = orc.step(t)
        assert np.abs(a - r).max() < PTOL and np.array_equal(a.argmax(1), r.argmax(1))
    hm.close()
    h1.close()


def test_sequences_on_grid_slices_timeout(gpu, tiny, monkeypatch):
    """A time-out in a launch of three slices ends every slice: the call
    reports it, the handle refuses steps until its state is set, and then
    steps the three sequences as the oracle does."""
    w, p32, _ = tiny
    cfg = RWKV_TINY
    B = 3
    monkeypatch.setenv("SNHIP_PERSIST_SPIN", "2048")
    monkeypatch.setenv("SNHIP_RK_PERSIST_MI", "8")
    hm = HipRwkv7(p32, max_batch=B)
    assert hm.persist_grid_for(B) > 0
    tok = torch.tensor([3, 40, 500], dtype=torch.int32, device="cuda")
    monkeypatch.setenv("SNHIP_PERSIST_STALL", "1")
    print("rwkv7 slices time-out", flush=True)
    with pytest.raises(RuntimeError, match="timed out"):
        hm.decode_greedy(tok, 3)
    monkeypatch.delenv("SNHIP_PERSIST_STALL")
    with pytest.raises(RuntimeError, match="part-stepped"):
        hm.step_batch(tok)
    S = torch.zeros(B, cfg.layers, cfg.n_head, 64, 64, device="cuda")
    sh = torch.zeros(B, cfg.layers, 2, cfg.dim, device="cuda")
    hm.set_state(S, sh)
    monkeypatch.delenv("SNHIP_PERSIST_SPIN")
    orc = oracle.RkOracle(p32.read_bytes(), batch=B)
    a = hm.step_batch(tok).cpu().numpy()
    assert np.abs(a - orc.step(tok.cpu().numpy())).max() < PTOL
    hm.close()


def test_persist_barrier_timeout_reports_error(gpu, tiny, monkeypatch):
    """Every exchange wait is given a target the host raised out of reach: each
    workgroup gives up after its poll limit and leaves the kernel and the call
    reports an error (device step and host step alike). The kernel writes S
    and shift in place layer by layer, so the handle then refuses steps until
    reset() or set_state(), after which it matches the oracle again."""
    w, p32, _ = tiny
    monkeypatch.setenv("SNHIP_PERSIST_SPIN", "2048")
    hm = HipRwkv7(p32)
    assert hm.persist_grid > 0
    tok = torch.tensor([3], dtype=torch.int32, device="cuda")
    monkeypatch.setenv("SNHIP_PERSIST_STALL", "1")
    print("rwkv7 persistent time-out", flush=True)
    with pytest.raises(RuntimeError, match="timed out"):
        hm.step_batch(tok)
    monkeypatch.delenv("SNHIP_PERSIST_STALL")
    with pytest.raises(RuntimeError, match="part-stepped"):
        hm.step(3)
    with pytest.raises(RuntimeError, match="part-stepped"):
        hm.prefill([3, 4])
    hm.reset()
    orc = oracle.RkOracle(p32.read_bytes())
    a = np.asarray(hm.step(3), np.float32)
    assert np.abs(a - orc.step([3])[0]).max() < PTOL
    monkeypatch.setenv("SNHIP_PERSIST_STALL", "1")
    with pytest.raises(RuntimeError, match="timed out"):
        hm.step_raw(4)
    monkeypatch.delenv("SNHIP_PERSIST_STALL")
    S = torch.zeros(1, RWKV_TINY.layers, RWKV_TINY.n_head, 64, 64, device="cuda")
    sh = torch.zeros(1, RWKV_TINY.layers, 2, RWKV_TINY.dim, device="cuda")
    hm.set_state(S, sh)
    orc.reset()
    a = np.asarray(hm.step(4), np.float32)
    assert np.abs(a - orc.step([4])[0]).max() < PTOL
    # a greedy call (many steps in one launch) gives up the same way
    monkeypatch.setenv("SNHIP_PERSIST_STALL", "1")
    with pytest.raises(RuntimeError, match="timed out"):
        hm.decode_greedy(tok, 5)
    monkeypatch.delenv("SNHIP_PERSIST_STALL")
    hm.reset()
    orc.reset()
    out = hm.decode_greedy(tok, 3).cpu().numpy()
    cur = np.array([3], np.int32)
    for i in range(3):
        nxt = orc.step(cur).argmax(1).astype(np.int32)
        assert np.array_equal(out[i], nxt), i
        cur = nxt
    monkeypatch.delenv("SNHIP_PERSIST_SPIN")
