"""GPU parity of the whole-model decode step against the oracle.

Bar: logits within 2e-5 absolute of the C oracle (bit-identical to the
reference's sn_step) and of the fp32 torch restatement of forward_step, with
the greedy argmax equal on every token. INT4: the oracle runs the fp32 path
on the dequantized weights (bit-identical dequantization is checked too).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle.torch_ref import TorchSunny
from sunnynet_amd.blob import BlobMatrices, layer_matrices, pack_sunny_blob
from sunnynet_amd.config import SMALL, SUNNY_100M, TINY
from sunnynet_amd.runtime.model import HipModel
from sunnynet_amd.weights import gaussian_matmuls, init_sunnynet

pytestmark = pytest.mark.gpu
TOL = 2e-5


def _write(tmp_path_factory, name, buf):
    p = tmp_path_factory.mktemp("blobs") / name
    p.write_bytes(buf)
    return p


def _model(path, cfg, **kw):
    return HipModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, **kw)


def dequant_blob(w, block):
    """fp32 blob holding the INT4-dequantized matmul and head weights."""
    mats = []
    for l in range(w.cfg.layers):
        M = layer_matrices(w, l)
        dq = {}
        for name in ("V", "U", "W_z", "W_c", "W_s_eff"):
            W = getattr(M, name)
            q, s = oracle.quant_i4(W, block)
            dq[name] = oracle.dequant_i4(q, s, W.shape[1], block)
        mats.append(BlobMatrices(**dq))
    H = w.embed.numpy()
    q, s = oracle.quant_i4(H, block)
    return pack_sunny_blob(w, matrices=mats, head=oracle.dequant_i4(q, s, H.shape[1], block))


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    w = init_sunnynet(TINY, 0)
    buf = pack_sunny_blob(w)
    return w, buf, _write(tmp_path_factory, "tiny.bin", buf)


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    w = init_sunnynet(SMALL, 0)
    buf = pack_sunny_blob(w)
    return w, buf, _write(tmp_path_factory, "small.bin", buf)


def test_tiny_step_matches_oracle_and_torch(gpu, tiny):
    w, buf, path = tiny
    print("tiny fp32 B=1", flush=True)
    hm = _model(path, TINY)
    orc = oracle.SnOracle(buf)
    tr = TorchSunny(w, torch.float32)
    st = tr.init_state(1)
    toks = np.random.default_rng(1).integers(0, TINY.vocab_size, 40)
    for t in toks:
        a = np.asarray(hm.step(int(t)), np.float32)
        b = orc.step([t])[0]
        c, st = tr.forward_step(torch.tensor([int(t)]), st)
        c = c[0].numpy()
        assert np.abs(a - b).max() < TOL and np.abs(a - c).max() < TOL
        assert a.argmax() == b.argmax() == c.argmax()
    s, h = hm.get_state(1)
    so, ho = orc.get_state()
    assert np.abs(s.cpu().numpy() - so).max() < 1e-5
    assert np.abs(h.cpu().numpy() - ho).max() < 1e-5


def test_small_prefill_then_greedy_matches_oracle(gpu, small):
    """SunnyNet small (4 layers, D=256, V=4096), seed 0: 256-token prompt by
    stepping, then 64 greedy tokens, every step checked."""
    w, buf, path = small
    print("small fp32: prompt 256 + greedy 64", flush=True)
    hm = _model(path, SMALL)
    orc = oracle.SnOracle(buf)
    prompt = np.random.default_rng(0).integers(0, SMALL.vocab_size, 256)
    worst = 0.0
    for t in prompt:
        a = np.asarray(hm.step(int(t)), np.float32)
        b = orc.step([t])[0]
        worst = max(worst, float(np.abs(a - b).max()))
        assert a.argmax() == b.argmax()
    nxt = int(b.argmax())
    for _ in range(64):
        a = np.asarray(hm.step(nxt), np.float32)
        b = orc.step([nxt])[0]
        worst = max(worst, float(np.abs(a - b).max()))
        assert a.argmax() == b.argmax()
        nxt = int(b.argmax())
    print("worst |dlogit|", worst)
    assert worst < TOL


def test_reference_surface(gpu, small):
    """prefill == stepping (the chunked prefill, to float rounding); reset
    clears the state (runtime/model.py:110-121)."""
    w, buf, path = small
    hm = _model(path, SMALL)
    toks = list(np.random.default_rng(3).integers(0, SMALL.vocab_size, 12))
    a = np.asarray(hm.prefill(toks))
    hm.reset()
    for t in toks:
        b = np.asarray(hm.step(int(t)))
    assert np.abs(a - b).max() < TOL and a.argmax() == b.argmax()
    hm.reset()
    s, h = hm.get_state(1)
    assert float(s.abs().max()) == 0.0 and float(h.abs().max()) == 0.0
    assert hm.vocab == SMALL.vocab_size


@pytest.mark.parametrize("B", [2, 3, 8, 11, 16, 33])
def test_batched_matches_oracle(gpu, small, monkeypatch, B):
    """fp32 steps of B sequences on the GEMV (B=2) or batched step (the
    per-sequence grid slices turned off by SNHIP_PERSIST_MI=1)."""
    w, buf, path = small
    print(f"small fp32 batched B={B}", flush=True)
    monkeypatch.setenv("SNHIP_PERSIST_MI", "1")
    hm = _model(path, SMALL, max_batch=64)
    assert hm.persistent_grid_for(B) == 0
    orc = oracle.SnOracle(buf, batch=B)
    rng = np.random.default_rng(B)
    for _ in range(12):
        toks = rng.integers(0, SMALL.vocab_size, B).astype(np.int32)
        a = hm.step_batch(torch.from_numpy(toks).to(gpu)).cpu().numpy()
        b = orc.step(toks)
        assert np.abs(a - b).max() < TOL
        assert np.array_equal(a.argmax(1), b.argmax(1))
    s, h = hm.get_state(B)
    so, ho = orc.get_state()
    assert np.abs(s.cpu().numpy() - so).max() < 1e-5 and np.abs(h.cpu().numpy() - ho).max() < 1e-5


def test_state_import_export(gpu, tiny):
    w, buf, path = tiny
    B = 4
    hm = _model(path, TINY, max_batch=B)
    orc = oracle.SnOracle(buf, batch=B)
    g = torch.Generator().manual_seed(0)
    s = torch.randn(B, TINY.layers, TINY.dim, generator=g)
    h = torch.randn(B, TINY.layers, TINY.taps - 1, TINY.dim, generator=g)
    hm.set_state(s.to(gpu), h.to(gpu))
    orc.set_state(s.numpy(), h.numpy())
    toks = np.array([1, 2, 3, 4], np.int32)
    a = hm.step_batch(torch.from_numpy(toks).to(gpu)).cpu().numpy()
    assert np.abs(a - orc.step(toks)).max() < TOL
    s2, h2 = hm.get_state(B)
    so, ho = orc.get_state()
    assert np.abs(s2.cpu().numpy() - so).max() < 1e-5 and np.abs(h2.cpu().numpy() - ho).max() < 1e-5


def test_greedy_decode_on_device(gpu, small):
    w, buf, path = small
    B, n = 3, 20
    hm = _model(path, SMALL, max_batch=B)
    orc = oracle.SnOracle(buf, batch=B)
    start = np.array([5, 900, 4095], np.int32)
    out = hm.decode_greedy(torch.from_numpy(start).to(gpu), n).cpu().numpy()
    cur = start
    for i in range(n):
        nxt = orc.step(cur).argmax(1).astype(np.int32)
        assert np.array_equal(out[i], nxt), i
        cur = nxt


@pytest.mark.parametrize("block,B,path", [(32, 2, "slices"), (64, 2, "slices"), (32, 2, "gemv"),
                                          (64, 2, "gemv"), (32, 4, "slices"), (64, 4, "batched"),
                                          (32, 16, "slices"), (64, 16, "batched")])
def test_int4_matches_dequantized_oracle(gpu, tmp_path_factory, monkeypatch, block, B, path):
    """INT4 group-quantized weights (N(0, 0.02) matmuls): HIP dequantizes in
    registers on every path a step of B sequences can take (the
    single-sequence persistent kernel on a grid slice per sequence, the GEMV
    step for two sequences, and the batched kernel, the last two with the
    slices turned off by SNHIP_PERSIST_MI=1); the oracle runs fp32 on the
    bit-identical dequantized blob."""
    print(f"small int4 block={block} B={B} {path}", flush=True)
    if path != "slices":
        monkeypatch.setenv("SNHIP_PERSIST_MI", "1")
    w = gaussian_matmuls(init_sunnynet(SMALL, 0), seed=3)
    blob = _write(tmp_path_factory, f"small_g{block}.bin", pack_sunny_blob(w))
    hm = _model(blob, SMALL, weights="int4", block=block, max_batch=B)
    assert (hm.persistent_grid_for(B) > 0) == (path == "slices")
    assert path != "batched" or hm.batch_grid > 0
    orc = oracle.SnOracle(dequant_blob(w, block), batch=B)
    rng = np.random.default_rng(block + B)
    for _ in range(24):
        toks = rng.integers(0, SMALL.vocab_size, B).astype(np.int32)
        a = hm.step_batch(torch.from_numpy(toks).to(gpu)).cpu().numpy()
        b = orc.step(toks)
        assert np.abs(a - b).max() < TOL
        assert np.array_equal(a.argmax(1), b.argmax(1))


def test_quant_dequant_kernels_bitexact(gpu):
    from sunnynet_amd import _native
    L = _native.lib()
    rng = np.random.default_rng(7)
    for block in (32, 64, 128):
        x = (rng.standard_normal((96, 1024)) * 0.02).astype(np.float32)
        x[5, :block] = 0.0
        qr, sr = oracle.quant_i4(x, block)
        dx = torch.from_numpy(x).to(gpu)
        q = torch.empty(96, 512, dtype=torch.uint8, device=gpu)
        s = torch.empty(96, 1024 // block, device=gpu)
        _native.check(L.snhip_abi_quant_i4_dev(dx.data_ptr(), q.data_ptr(), s.data_ptr(), 96, 1024,
                                               block, _native.stream_handle()), "quant")
        y = torch.empty_like(dx)
        _native.check(L.snhip_abi_dequant_i4_dev(q.data_ptr(), s.data_ptr(), y.data_ptr(), 96, 1024,
                                                 block, _native.stream_handle()), "dequant")
        torch.cuda.synchronize()
        assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().numpy(), sr)
        assert np.array_equal(y.cpu().numpy(), oracle.dequant_i4(qr, sr, 1024, block))


@pytest.fixture(scope="module")
def m100(tmp_path_factory):
    print("generating SunnyNet-100M weights (seed 1)", flush=True)
    w = init_sunnynet(SUNNY_100M, 1)
    buf = pack_sunny_blob(w)
    return w, buf, _write(tmp_path_factory, "m100.bin", buf)


def test_100m_b1_matches_oracle(gpu, m100):
    w, buf, path = m100
    cfg = SUNNY_100M
    print("100M fp32 B=1: prompt 24 + greedy 8", flush=True)
    hm = _model(path, cfg)
    orc = oracle.SnOracle(buf)
    toks = list(np.random.default_rng(1).integers(0, cfg.vocab_size, 24))
    worst = 0.0
    for t in toks:
        a = np.asarray(hm.step(int(t)), np.float32)
        b = orc.step([t])[0]
        worst = max(worst, float(np.abs(a - b).max()))
        assert a.argmax() == b.argmax()
    nxt = int(b.argmax())
    for _ in range(8):
        a = np.asarray(hm.step(nxt), np.float32)
        b = orc.step([nxt])[0]
        worst = max(worst, float(np.abs(a - b).max()))
        assert a.argmax() == b.argmax()
        nxt = int(b.argmax())
    print("100M worst |dlogit|", worst)
    assert worst < TOL


def test_100m_b64_matches_oracle_on_sampled_sequences(gpu, m100):
    w, buf, path = m100
    cfg = SUNNY_100M
    B = 64
    pick = [0, 17, 63]
    print("100M fp32 B=64: 6 steps, sequences 0/17/63 vs oracle", flush=True)
    hm = _model(path, cfg, max_batch=B)
    orc = oracle.SnOracle(buf, batch=len(pick))
    rng = np.random.default_rng(64)
    for _ in range(6):
        toks = rng.integers(0, cfg.vocab_size, B).astype(np.int32)
        a = hm.step_batch(torch.from_numpy(toks).to(gpu)).cpu().numpy()
        b = orc.step(toks[pick])
        assert np.abs(a[pick] - b).max() < TOL
        assert np.array_equal(a[pick].argmax(1), b.argmax(1))


@pytest.mark.parametrize("B", [4, 16])
def test_graph_replays_match_eager(gpu, small, monkeypatch, B):
    """The step runs as a captured HIP graph; replay it many times with host
    work and synchronization in between and compare every replay with the
    eager (uncaptured) launch sequence, bit for bit (B = 16: the MFMA GEMMs,
    whose split-K tile counters are re-armed by every launch)."""
    w, buf, path = small
    print(f"small graph vs eager B={B}", flush=True)
    monkeypatch.setenv("SNHIP_PERSIST_MI", "1")     # B=4 on the batched step, not grid slices
    rng = np.random.default_rng(11)
    seqs = [rng.integers(0, SMALL.vocab_size, B).astype(np.int32) for _ in range(10)]
    hg = _model(path, SMALL, max_batch=B)
    monkeypatch.setenv("SNHIP_NO_GRAPH", "1")
    he = _model(path, SMALL, max_batch=B)
    for toks in seqs:
        t = torch.from_numpy(toks).to(gpu)
        a = hg.step_batch(t).cpu().numpy()
        torch.cuda.synchronize()
        b = he.step_batch(t).cpu().numpy()
        assert np.array_equal(a, b)
    ga = hg.decode_greedy(torch.from_numpy(seqs[0]).to(gpu), 16).cpu().numpy()
    gb = he.decode_greedy(torch.from_numpy(seqs[0]).to(gpu), 16).cpu().numpy()
    assert np.array_equal(ga, gb)
