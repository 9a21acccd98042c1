"""Every SunnyNet-100M configuration the benchmark times, checked against the
reference C runtime (oracle/_ref, the reference's own sn_load / sn_prefill /
sn_step compiled from its sources), at the benchmark's own kernel
instantiations and chain lengths:

* fp32 B=1: chunked prefill of T=1024 tokens, then 256 greedy steps in one
  persistent launch (the whole chain's tokens and the last logits);
* INT4 g32 B=1: T=2048 prefill, then 256 greedy steps;
* INT4 g32 B=2 and B=8: T=2048 prefill, then 256 greedy steps of the
  single-sequence persistent kernel on a grid slice per sequence (128 and 32
  workgroups each), both / three sampled sequences replayed on the reference;
* INT4 g32 B=32: T=2048 prefill, then 256 greedy steps of the persistent
  batched step (k_decode_batch at the 100M product depths with INT4 g32
  weights), three sampled sequences replayed on the reference;
* fp32 B=64: T=1024 prefill then 256 greedy steps, three sampled sequences;
* every batch size 1..64, INT4 and fp32, one step each (every decode path
  and row-block count the batch size selects).

INT4 references run the reference's fp32 runtime on a blob holding the
bit-identically dequantized weights (W4A32). Bar: logits within 2e-5, argmax
(hence every greedy token) equal.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from sunnynet_amd.blob import pack_sunny_blob
from sunnynet_amd.config import SUNNY_100M
from sunnynet_amd.runtime.model import HipModel
from sunnynet_amd.weights import gaussian_matmuls, init_sunnynet
from tests.test_decode_gpu import dequant_blob

pytestmark = pytest.mark.gpu
TOL = 2e-5
CFG = SUNNY_100M


def _model(path, **kw):
    c = CFG
    return HipModel(path, c.vocab_size, c.dim, c.inner, c.rank, c.taps, c.layers, **kw)


def _ref(path):
    c = CFG
    return oracle.RefSnModel(path, c.vocab_size, c.dim, c.inner, c.rank, c.taps, c.layers)


@pytest.fixture(scope="module")
def blobs(tmp_path_factory, ref_built):
    d = tmp_path_factory.mktemp("cfgs")
    print("generating SunnyNet-100M weights: seed 1 (fp32) and N(0, 0.02) matmuls (INT4)",
          flush=True)
    w = init_sunnynet(CFG, 1)
    p32 = d / "m100.bin"
    p32.write_bytes(pack_sunny_blob(w))
    w4 = gaussian_matmuls(init_sunnynet(CFG, 1), seed=3)
    p4 = d / "m100_gauss.bin"
    p4.write_bytes(pack_sunny_blob(w4))
    pdq = d / "m100_gauss_dq32.bin"
    pdq.write_bytes(dequant_blob(w4, 32))
    return p32, p4, pdq


def _ref_greedy(ref, prompt, n):
    """Reference chain: sn_prefill over the prompt, then n greedy sn_steps.
    Returns (prefill logits, tokens chosen after each step, last logits)."""
    lg0 = ref.prefill(prompt)
    tok, toks, lg = int(lg0.argmax()), [], lg0
    for _ in range(n):
        lg = ref.step(tok)
        tok = int(lg.argmax())
        toks.append(tok)
    return lg0, np.array(toks, np.int32), lg


def _check_b1_chain(gpu, path, ref_path, T, weights, seed):
    prompt = np.random.default_rng(seed).integers(0, CFG.vocab_size, T).astype(np.int32)
    hm = _model(path, weights=weights, block=32)
    assert hm.persistent_grid > 0
    lg0 = hm.prefill_batch(torch.from_numpy(prompt[None]).to(gpu)).cpu().numpy()[0]
    print(f"{weights} B=1: reference prefill T={T}", flush=True)
    ref = _ref(ref_path)
    rl0, rtoks, rlast = _ref_greedy(ref, prompt, 256)
    d0 = float(np.abs(lg0 - rl0).max())
    print(f"{weights} B=1 prefill T={T}: |dlogit| {d0:.3g}", flush=True)
    assert d0 < TOL and lg0.argmax() == rl0.argmax()
    last = torch.empty(1, CFG.vocab_size, device=gpu)
    toks = hm.decode_greedy(torch.tensor([int(lg0.argmax())], dtype=torch.int32, device=gpu),
                            256, logits=last).cpu().numpy()[:, 0]
    first_bad = int(np.argmax(toks != rtoks)) if (toks != rtoks).any() else -1
    assert first_bad < 0, f"greedy chain diverges at step {first_bad}"
    d1 = float(np.abs(last.cpu().numpy()[0] - rlast).max())
    print(f"{weights} B=1 256 greedy steps: tokens equal, last |dlogit| {d1:.3g}", flush=True)
    assert d1 < TOL
    hm.close()
    ref.close()


def test_fp32_b1_prefill_1024_then_256_greedy(gpu, blobs):
    p32, _, _ = blobs
    _check_b1_chain(gpu, p32, p32, 1024, "fp32", 1024)


def test_int4_b1_prefill_2048_then_256_greedy(gpu, blobs):
    _, p4, pdq = blobs
    _check_b1_chain(gpu, p4, pdq, 2048, "int4", 2048)


@pytest.mark.parametrize("weights,B,T,n", [("int4", 2, 2048, 256), ("int4", 8, 2048, 256),
                                            ("int4", 32, 2048, 256), ("fp32", 64, 1024, 256)])
def test_batched_chain_sampled(gpu, blobs, weights, B, T, n):
    """The benchmark's batched chains at full length: all B sequences prefill
    T tokens and decode n greedy steps on the device in one call; three of
    them are replayed on reference handles (sn_prefill, then sn_step), token
    for token, with the last logits within 2e-5."""
    p32, p4, pdq = blobs
    path, ref_path = (p4, pdq) if weights == "int4" else (p32, p32)
    prompts = np.random.default_rng(B * 7 + T).integers(0, CFG.vocab_size, (B, T)).astype(np.int32)
    hm = _model(path, weights=weights, block=32, max_batch=B)
    slices = weights == "int4" and B <= 16
    assert hm.persistent_grid_for(B) > 0 if slices else hm.batch_grid > 0
    lg0 = hm.prefill_batch(torch.from_numpy(prompts).to(gpu)).cpu().numpy()
    start = torch.from_numpy(lg0.argmax(1).astype(np.int32)).to(gpu)
    last = torch.empty(B, CFG.vocab_size, device=gpu)
    toks = hm.decode_greedy(start, n, logits=last).cpu().numpy()
    last = last.cpu().numpy()
    for b in sorted({0, min(B // 2 + 1, B - 1), B - 1}):
        print(f"{weights} B={B}: reference chain of sequence {b}", flush=True)
        ref = _ref(ref_path)
        rl0, rtoks, rlast = _ref_greedy(ref, prompts[b], n)
        ref.close()
        assert np.abs(lg0[b] - rl0).max() < TOL and lg0[b].argmax() == rl0.argmax()
        assert np.array_equal(toks[:, b], rtoks), (b, toks[:, b], rtoks)
        d = float(np.abs(last[b] - rlast).max())
        print(f"{weights} B={B} sequence {b}: {n} tokens equal, last |dlogit| {d:.3g}", flush=True)
        assert d < TOL
    hm.close()


@pytest.mark.parametrize("weights", ["int4", "fp32"])
def test_every_batch_size_one_step(gpu, blobs, weights):
    """Every batch size 1..64 at the 100M shape (B=1 the persistent step,
    2..16 (INT4) or 2..4 (fp32) the persistent step on a grid slice per
    sequence (eight grid sizes), the rest the persistent batched step with
    two to four 16-row blocks and partial ones): one step from the reset
    state, the first and the last sequence against the reference runtime,
    within 2e-5 and with the same argmax."""
    p32, p4, pdq = blobs
    path, ref_path = (p4, pdq) if weights == "int4" else (p32, p32)
    print(f"{weights} B=1..64, one step each", flush=True)
    hm = _model(path, weights=weights, block=32, max_batch=64)
    ref = _ref(ref_path)
    rng = np.random.default_rng(7)
    worst = 0.0
    for B in range(1, 65):
        toks = rng.integers(0, CFG.vocab_size, B).astype(np.int32)
        hm.reset()
        lg = hm.step_batch(torch.from_numpy(toks).to(gpu)).cpu().numpy()
        for b in sorted({0, B - 1}):
            ref.reset()
            r = ref.step(int(toks[b]))
            d = float(np.abs(lg[b] - r).max())
            worst = max(worst, d)
            assert d < TOL and lg[b].argmax() == r.argmax(), (B, b, d)
    print(f"{weights} B=1..64: worst |dlogit| {worst:.3g}", flush=True)
    hm.close()
    ref.close()
