"""The persistent batched step (every layer of a step of 3..64 sequences in one
cooperative launch, each tile waiting on the flags of the tiles it reads)
against the oracle and the per-kernel step path.

Bar as for every decode path: logits within 2e-5 absolute of the C oracle
(bit-identical to the reference's sn_step), greedy tokens equal to the
oracle's argmax chain. The per-kernel path (SNHIP_BATCH_PERSIST=0) is a second
witness: both paths must agree with each other to the same bound and pick the
same tokens. INT4 compares with the oracle on the bit-identically dequantized
weights.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from sunnynet_amd.blob import pack_sunny_blob
from sunnynet_amd.config import SMALL
from sunnynet_amd.runtime.model import HipModel
from sunnynet_amd.weights import gaussian_matmuls, init_sunnynet
from tests.test_decode_gpu import dequant_blob

pytestmark = pytest.mark.gpu
TOL = 2e-5


def _model(path, cfg, **kw):
    return HipModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, **kw)


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    w = init_sunnynet(SMALL, 0)
    buf = pack_sunny_blob(w)
    p = tmp_path_factory.mktemp("bblobs") / "small.bin"
    p.write_bytes(buf)
    return w, buf, p


@pytest.mark.parametrize("B", [8, 13, 16, 40, 64])
def test_batched_kernel_matches_oracle_and_per_kernel_path(gpu, small, monkeypatch, B):
    w, buf, path = small
    print(f"small fp32 batched kernel B={B}", flush=True)
    hb = _model(path, SMALL, max_batch=64)
    assert hb.batch_grid > 0
    monkeypatch.setenv("SNHIP_BATCH_PERSIST", "0")
    hk = _model(path, SMALL, max_batch=64)
    assert hk.batch_grid == 0
    orc = oracle.SnOracle(buf, batch=B)
    rng = np.random.default_rng(100 + B)
    for _ in range(10):
        toks = rng.integers(0, SMALL.vocab_size, B).astype(np.int32)
        t = torch.from_numpy(toks).to(gpu)
        a = hb.step_batch(t).cpu().numpy()
        k = hk.step_batch(t).cpu().numpy()
        b = orc.step(toks)
        assert np.abs(a - b).max() < TOL
        assert np.abs(a - k).max() < TOL
        assert np.array_equal(a.argmax(1), b.argmax(1))
    s, h = hb.get_state(B)
    so, ho = orc.get_state()
    assert np.abs(s.cpu().numpy() - so).max() < 1e-5 and np.abs(h.cpu().numpy() - ho).max() < 1e-5


def test_batched_greedy_decode_matches_oracle(gpu, small):
    w, buf, path = small
    B, n = 9, 24
    print(f"small fp32 batched greedy B={B} n={n}", flush=True)
    hm = _model(path, SMALL, max_batch=16)
    assert hm.batch_grid > 0
    orc = oracle.SnOracle(buf, batch=B)
    start = np.arange(B, dtype=np.int32) * 401 % SMALL.vocab_size
    lg = torch.empty(B, SMALL.vocab_size, device=gpu)
    out = hm.decode_greedy(torch.from_numpy(start).to(gpu), n, logits=lg).cpu().numpy()
    cur = start
    for i in range(n):
        ref = orc.step(cur)
        nxt = ref.argmax(1).astype(np.int32)
        assert np.array_equal(out[i], nxt), i
        cur = nxt
    assert np.abs(lg.cpu().numpy() - ref).max() < TOL


@pytest.mark.parametrize("block", [32, 64])
def test_batched_kernel_int4_matches_dequantized_oracle(gpu, tmp_path_factory, block):
    B = 24
    print(f"small int4 block={block} batched kernel B={B}", flush=True)
    w = gaussian_matmuls(init_sunnynet(SMALL, 0), seed=5)
    path = tmp_path_factory.mktemp("bq") / f"small_g{block}.bin"
    path.write_bytes(pack_sunny_blob(w))
    hm = _model(path, SMALL, weights="int4", block=block, max_batch=B)
    assert hm.batch_grid > 0
    orc = oracle.SnOracle(dequant_blob(w, block), batch=B)
    rng = np.random.default_rng(block)
    for _ in range(12):
        toks = rng.integers(0, SMALL.vocab_size, B).astype(np.int32)
        a = hm.step_batch(torch.from_numpy(toks).to(gpu)).cpu().numpy()
        b = orc.step(toks)
        assert np.abs(a - b).max() < TOL
        assert np.array_equal(a.argmax(1), b.argmax(1))


def test_batched_kernel_is_deterministic(gpu, small):
    """Fixed summation orders: two handles stepping the same tokens give
    bit-identical logits, step after step."""
    w, buf, path = small
    B = 32
    ha = _model(path, SMALL, max_batch=B)
    hb = _model(path, SMALL, max_batch=B)
    rng = np.random.default_rng(3)
    for _ in range(6):
        t = torch.from_numpy(rng.integers(0, SMALL.vocab_size, B).astype(np.int32)).to(gpu)
        assert np.array_equal(ha.step_batch(t).cpu().numpy(), hb.step_batch(t).cpu().numpy())


def test_batched_barrier_timeout_reports_error(gpu, small, monkeypatch):
    """Every dataflow wait is given a target the host raised out of reach: each
    workgroup gives up after its poll limit and leaves the kernel, and the
    call itself reports the error, on the device-tensor path as on the host
    one. The state may be part-stepped, so the handle refuses further steps
    until reset(); then it matches the oracle again."""
    w, buf, path = small
    B = 8
    monkeypatch.setenv("SNHIP_PERSIST", "0")
    monkeypatch.setenv("SNHIP_PERSIST_SPIN", "2048")
    hm = _model(path, SMALL, max_batch=B)
    assert hm.batch_grid > 0
    toks = np.arange(B, dtype=np.int32)
    dt = torch.from_numpy(toks).to(gpu)
    monkeypatch.setenv("SNHIP_PERSIST_STALL", "1")
    print("batched time-out: device path", flush=True)
    with pytest.raises(RuntimeError, match="timed out"):
        hm.step_batch(dt)
    monkeypatch.delenv("SNHIP_PERSIST_STALL")
    with pytest.raises(RuntimeError, match="part-stepped"):
        hm.step_batch(dt)
    with pytest.raises(RuntimeError, match="part-stepped"):
        hm.decode_greedy(dt, 2)
    hm.reset()
    orc = oracle.SnOracle(buf, batch=B)
    a = hm.step_batch(dt).cpu().numpy()
    assert np.abs(a - orc.step(toks)).max() < TOL
    print("batched time-out: host path", flush=True)
    monkeypatch.setenv("SNHIP_PERSIST_STALL", "1")
    with pytest.raises(RuntimeError, match="timed out"):
        hm.step_batch_host(toks)
    monkeypatch.delenv("SNHIP_PERSIST_STALL")
    s, h = (torch.zeros(B, SMALL.layers, SMALL.dim, device=gpu),
            torch.zeros(B, SMALL.layers, SMALL.taps - 1, SMALL.dim, device=gpu))
    hm.set_state(s[:1], h[:1])   # sequences 1..B-1 may still be part-stepped
    with pytest.raises(RuntimeError, match="part-stepped"):
        hm.step_batch_host(toks)
    hm.set_state(s, h)     # a valid state over every stepped sequence clears the refusal
    a = hm.step_batch_host(toks)
    assert np.abs(a - oracle.SnOracle(buf, batch=B).step(toks)).max() < TOL
    monkeypatch.delenv("SNHIP_PERSIST_SPIN")
    monkeypatch.delenv("SNHIP_PERSIST")


def test_batched_kernel_out_of_range_token_gives_nan_row(gpu, small):
    """An id outside the vocabulary on the device path gives that sequence a
    NaN embedding row (as the per-kernel path's gather does); sequences are
    independent, so every other row still matches the oracle."""
    w, buf, path = small
    B = 8
    hm = _model(path, SMALL, max_batch=B)
    assert hm.batch_grid > 0
    toks = np.arange(B, dtype=np.int32) * 37
    bad = toks.copy()
    bad[3] = SMALL.vocab_size + 5
    a = hm.step_batch(torch.from_numpy(bad).to(gpu)).cpu().numpy()
    b = oracle.SnOracle(buf, batch=B).step(toks)
    assert np.isnan(a[3]).all()
    keep = [i for i in range(B) if i != 3]
    assert np.abs(a[keep] - b[keep]).max() < TOL
