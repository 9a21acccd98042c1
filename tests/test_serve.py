"""Serving: the Engine protocol (HipEngine) and continuous batching
(BatchScheduler) on the HIP backend.

Requests must be independent: under continuous batching every request's
greedy tokens equal those of the same request run alone through the oracle
(prompt stepped token by token as sn_prefill does, then greedy), whatever the
admission order, slot moves and batch size of each step (1..max_batch, so the
B=1 persistent kernel, the same kernel on a grid slice per sequence (2..4
sequences) and the batched kernel (5..8) all take part).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from sunnynet_amd.blob import pack_sunny_blob
from sunnynet_amd.config import SMALL
from sunnynet_amd.runtime.serve import sample_logits
from sunnynet_amd.weights import init_sunnynet

TOL = 2e-5


def test_sample_logits_rules():
    rng = np.random.default_rng(0)
    z = rng.standard_normal(100).astype(np.float32)
    assert sample_logits(z, temperature=0) == int(np.argmax(z))
    assert sample_logits(z, temperature=1.0, top_k=1, rng=np.random.default_rng(1)) == int(np.argmax(z))
    assert sample_logits(z, temperature=1.0, top_p=1e-6, rng=np.random.default_rng(1)) == int(np.argmax(z))
    a = [sample_logits(z, 0.8, 0.9, 20, np.random.default_rng(7)) for _ in range(3)]
    assert len(set(a)) == 1                                   # seeded: reproducible
    top = set(np.argsort(-z)[:20].tolist())
    draws = [sample_logits(z, 1.0, 1.0, 20, rng) for _ in range(200)]
    assert set(draws) <= top                                   # never outside the top k


def _oracle_chain(buf, prompt, n):
    o = oracle.SnOracle(buf)
    for t in prompt:
        lg = o.step([int(t)])[0]
    out = []
    for _ in range(n):
        t = int(np.argmax(lg))
        out.append(t)
        lg = o.step([t])[0]
    return out


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    w = init_sunnynet(SMALL, 0)
    buf = pack_sunny_blob(w)
    p = tmp_path_factory.mktemp("serve") / "small.bin"
    p.write_bytes(buf)
    return buf, p


@pytest.mark.gpu
def test_continuous_batching_matches_solo_runs(gpu, small):
    from sunnynet_amd.runtime.model import HipModel
    from sunnynet_amd.runtime.serve import BatchScheduler
    buf, path = small
    cfg = SMALL
    hm = HipModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, max_batch=8)
    sch = BatchScheduler(hm)
    rng = np.random.default_rng(5)
    reqs = []
    for i in range(13):
        prompt = rng.integers(0, cfg.vocab_size, int(rng.integers(1, 30))).tolist()
        reqs.append(sch.submit(prompt, int(rng.integers(1, 16))))
    # a few steps, then more arrivals while others run
    for _ in range(5):
        sch.step()
    for i in range(4):
        prompt = rng.integers(0, cfg.vocab_size, int(rng.integers(1, 12))).tolist()
        reqs.append(sch.submit(prompt, int(rng.integers(2, 10))))
    sch.run()
    print(f"serve: {len(reqs)} requests in {sch.steps} batched steps", flush=True)
    for r in reqs:
        assert r.done and len(r.output) == r.max_tokens
        assert r.output == _oracle_chain(buf, r.prompt, r.max_tokens)


@pytest.mark.gpu
def test_engine_protocol_interleaved_requests(gpu, small):
    from sunnynet_amd.runtime.serve import HipEngine
    buf, path = small
    cfg = SMALL
    eng = HipEngine(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers)
    sa, sb = eng.init_state(), eng.init_state()
    oa, ob = oracle.SnOracle(buf), oracle.SnOracle(buf)
    ta, tb = [5, 77, 1024, 3], [4000, 2, 9]
    for i in range(12):
        if i < len(ta):
            la, sa = eng.step(ta[i], sa)
            assert np.abs(la - oa.step([ta[i]])[0]).max() < TOL
        if i < len(tb):
            lb, sb = eng.step(tb[i], sb)
            assert np.abs(lb - ob.step([tb[i]])[0]).max() < TOL
        if i >= len(ta):
            t = int(np.argmax(la))
            la, sa = eng.step(t, sa)
            assert np.abs(la - oa.step([t])[0]).max() < TOL
        if i >= len(tb):
            t = int(np.argmax(lb))
            lb, sb = eng.step(t, sb)
            assert np.abs(lb - ob.step([t])[0]).max() < TOL
    eng.sync_state(sb)
    so, ho = ob.get_state()
    assert np.abs(sb.s.cpu().numpy() - so).max() < 1e-5


@pytest.mark.gpu
def test_rwkv_engine_interleaved_requests(gpu, tmp_path):
    """Two RWKV-7 requests stepped alternately through one HipRwkvEngine give
    each request's solo logits (oracle, one handle per request)."""
    from sunnynet_amd.runtime.serve import HipRwkvEngine
    from sunnynet_amd.rwkv7 import RWKV_TINY, init_rwkv7, pack_rwkv7_blob
    blob = pack_rwkv7_blob(init_rwkv7(RWKV_TINY, 9))
    path = tmp_path / "rk.bin"
    path.write_bytes(blob)
    eng = HipRwkvEngine(path, RWKV_TINY.vocab)
    oa, ob = oracle.RkOracle(blob), oracle.RkOracle(blob)
    sa, sb = eng.init_state(), eng.init_state()
    rng = np.random.default_rng(10)
    ta = rng.integers(0, RWKV_TINY.vocab, 12)
    tb = rng.integers(0, RWKV_TINY.vocab, 12)
    for i in range(12):
        la, sa = eng.step(int(ta[i]), sa)
        lb, sb = eng.step(int(tb[i]), sb)
        assert np.abs(la - oa.step([ta[i]])[0]).max() < TOL
        assert np.abs(lb - ob.step([tb[i]])[0]).max() < TOL
    eng.sync_state(sb)
    S, sh = ob.get_state()
    assert np.abs(sb.S.cpu().numpy() - S).max() < 1e-4 and np.abs(sb.shift.cpu().numpy() - sh).max() < 1e-5
