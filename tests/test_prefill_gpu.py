"""GPU parity of the MFMA linear and the chunked batched prefill.

The prefill runs the prompt through matrix-core GEMMs and the fused
gate + exact sequential scan; its result must equal stepping the oracle
through the same prompt (logits within 2e-5, argmax equal, state within
1e-5), be invariant to the chunk length (the reference's chunk-invariance
property, tests/test_architecture.py:126-160) and continue a segment from a
carried state (tests/test_architecture.py:380-393).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from sunnynet_amd import _native
from sunnynet_amd.blob import pack_sunny_blob
from sunnynet_amd.config import SMALL, SUNNY_100M, TINY
from sunnynet_amd.runtime.model import HipModel
from sunnynet_amd.weights import gaussian_matmuls, init_sunnynet

pytestmark = pytest.mark.gpu
TOL = 2e-5


def _model(path, cfg, **kw):
    return HipModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, **kw)


@pytest.mark.parametrize("M,N,K", [(1, 64, 32), (7, 100, 96), (64, 512, 1024), (130, 70, 64),
                                   (1024, 2048, 512), (3, 32000, 1024)])
def test_linear_matches_fp64(gpu, M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.05
    ref = (x.double() @ w.double().T)
    y = torch.empty(M, N, device=gpu)
    xd, wd = x.to(gpu), w.to(gpu)      # keep the device copies alive until the kernel ran
    L = _native.lib()
    _native.check(L.snhip_abi_linear_dev(xd.data_ptr(), wd.data_ptr(), y.data_ptr(),
                                         M, N, K, _native.stream_handle()), "linear")
    torch.cuda.synchronize()
    err = (y.cpu().double() - ref).abs().max().item()
    scale = ref.abs().max().item()
    assert err <= 2e-6 * max(1.0, scale) * (K / 32) ** 0.5, (err, scale)


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    w = init_sunnynet(SMALL, 0)
    buf = pack_sunny_blob(w)
    p = tmp_path_factory.mktemp("b") / "small.bin"
    p.write_bytes(buf)
    return w, buf, p


def _oracle_prefill(buf, prompts, B):
    orc = oracle.SnOracle(buf, batch=B)
    last = None
    for t in range(prompts.shape[1]):
        last = orc.step(prompts[:, t])
    return orc, last


@pytest.mark.parametrize("B,T", [(1, 300), (1, 1100), (3, 77), (5, 1)])
def test_prefill_matches_stepping(gpu, small, B, T):
    """Small batches take the split gate/scan path (several 512-step scan
    tiles at T = 1100); the 100M B=64 test below takes the fused one."""
    w, buf, path = small
    print(f"prefill small B={B} T={T}", flush=True)
    prompts = np.random.default_rng(B * 1000 + T).integers(0, SMALL.vocab_size, (B, T)).astype(np.int32)
    hm = _model(path, SMALL, max_batch=8)
    lg = hm.prefill_batch(torch.from_numpy(prompts).to(gpu)).cpu().numpy()
    orc, ref = _oracle_prefill(buf, prompts, B)
    assert np.abs(lg - ref).max() < TOL
    assert np.array_equal(lg.argmax(1), ref.argmax(1))
    s, h = hm.get_state(B)
    so, ho = orc.get_state()
    assert np.abs(s.cpu().numpy() - so).max() < 1e-5
    assert np.abs(h.cpu().numpy() - ho).max() < 1e-5
    # decoding continues from the prefilled state
    nxt = ref.argmax(1).astype(np.int32)
    a = hm.step_batch(torch.from_numpy(nxt).to(gpu)).cpu().numpy()
    assert np.abs(a - orc.step(nxt)).max() < TOL


def test_prefill_chunk_invariance_and_continuation(gpu, small, monkeypatch):
    w, buf, path = small
    B, T = 2, 200
    prompts = np.random.default_rng(7).integers(0, SMALL.vocab_size, (B, T)).astype(np.int32)
    dp = torch.from_numpy(prompts).to(gpu)
    hm = _model(path, SMALL, max_batch=B)
    ref = hm.prefill_batch(dp).cpu().numpy()
    s_ref, h_ref = (x.cpu().numpy() for x in hm.get_state(B))
    for chunk in ("1", "37", "64", "200"):
        monkeypatch.setenv("SNHIP_PREFILL_CHUNK", chunk)
        hc = _model(path, SMALL, max_batch=B)
        lg = hc.prefill_batch(dp).cpu().numpy()
        s, h = (x.cpu().numpy() for x in hc.get_state(B))
        assert np.abs(lg - ref).max() < 1e-5, chunk
        assert np.abs(s - s_ref).max() < 1e-5 and np.abs(h - h_ref).max() < 1e-5, chunk
    monkeypatch.delenv("SNHIP_PREFILL_CHUNK")
    for split in (1, 2, 60, 199):
        hs = _model(path, SMALL, max_batch=B)
        hs.prefill_batch(dp[:, :split].contiguous(), logits=False)
        lg = hs.prefill_batch(dp[:, split:].contiguous()).cpu().numpy()
        assert np.abs(lg - ref).max() < 1e-5, split


def test_prefill_int4_matches_dequantized_oracle(gpu, tmp_path_factory):
    from tests.test_decode_gpu import dequant_blob
    w = gaussian_matmuls(init_sunnynet(SMALL, 0), seed=3)
    p = tmp_path_factory.mktemp("b") / "q.bin"
    p.write_bytes(pack_sunny_blob(w))
    B, T = 3, 96
    prompts = np.random.default_rng(3).integers(0, SMALL.vocab_size, (B, T)).astype(np.int32)
    for block in (32, 64):
        hm = _model(p, SMALL, weights="int4", block=block, max_batch=B)
        lg = hm.prefill_batch(torch.from_numpy(prompts).to(gpu)).cpu().numpy()
        _, ref = _oracle_prefill(dequant_blob(w, block), prompts, B)
        assert np.abs(lg - ref).max() < TOL, block
        assert np.array_equal(lg.argmax(1), ref.argmax(1))


def test_prefill_unsupported_shape_falls_back_to_stepping(gpu, tmp_path_factory):
    """TINY (D = 64) uses the chunked path; a D not divisible by 64 uses the
    reference's step loop for snhip_prefill and refuses the batched call."""
    cfg = TINY.with_(dim=72, inner=96, rank=32)
    w = init_sunnynet(cfg, 0)
    buf = pack_sunny_blob(w)
    p = tmp_path_factory.mktemp("b") / "t72.bin"
    p.write_bytes(buf)
    hm = _model(p, cfg)
    toks = list(range(1, 20))
    a = np.asarray(hm.prefill(toks), np.float32)
    orc = oracle.SnOracle(buf)
    for t in toks:
        b = orc.step([t])[0]
    assert np.abs(a - b).max() < TOL
    with pytest.raises(RuntimeError):
        hm.prefill_batch(torch.tensor([[1, 2, 3]], device=gpu))


def test_100m_prefill_b64_sampled(gpu, tmp_path_factory):
    cfg = SUNNY_100M
    print("100M prefill B=64 T=48 (sequences 0/31/63 vs oracle)", flush=True)
    w = init_sunnynet(cfg, 1)
    buf = pack_sunny_blob(w)
    p = tmp_path_factory.mktemp("b") / "m100.bin"
    p.write_bytes(buf)
    B, T = 64, 48
    prompts = np.random.default_rng(64).integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    hm = _model(p, cfg, max_batch=B)
    lg = hm.prefill_batch(torch.from_numpy(prompts).to(gpu)).cpu().numpy()
    pick = [0, 31, 63]
    _, ref = _oracle_prefill(buf, prompts[pick], len(pick))
    assert np.abs(lg[pick] - ref).max() < TOL
    assert np.array_equal(lg[pick].argmax(1), ref.argmax(1))
