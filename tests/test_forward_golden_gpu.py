"""The HIP handle against the reference's own fp32 ``forward_step`` and
``forward`` (sunnynet/model.py:89-124), recorded by
tests/golden/make_step_fixture.py on the weights ``SunnyNet(cfg)`` draws after
``torch.manual_seed(0)``, and the every-position logits of the chunked prefill
(``snhip_prefill_all_dev``, the reference's ``forward``) against the
reference runtime stepping the same tokens.

Bar: logits within 2e-5 absolute with the same greedy argmax at every
position; states within 1e-5 absolute plus 1e-5 relative.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from sunnynet_amd.blob import pack_sunny_blob
from sunnynet_amd.config import SMALL, SUNNY_100M
from sunnynet_amd.runtime.model import HipModel, HipSunnyNet
from sunnynet_amd.weights import init_sunnynet
from tests.test_forward_step_golden import load_case, state_close

pytestmark = pytest.mark.gpu
TOL = 2e-5


def _model(path, cfg, **kw):
    return HipModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, **kw)


@pytest.mark.parametrize("name", ["tiny", "small"])
def test_forward_step_matches_reference_fixture(gpu, tmp_path, name):
    """forward_step along the recorded greedy chain (tiny B=2: the persistent
    step on a grid slice per sequence; small B=1: the persistent step)."""
    cfg, seed, z = load_case(name)
    tokens, logits = z["tokens"], z["logits"]
    T, B = tokens.shape
    p = tmp_path / f"{name}.bin"
    p.write_bytes(pack_sunny_blob(init_sunnynet(cfg, seed)))
    net = HipSunnyNet(_model(p, cfg, max_batch=B))
    st = net.init_state(B)
    worst = 0.0
    print(f"forward_step fixture {name}: {T} steps x B={B}", flush=True)
    for t in range(T):
        lg, st = net.forward_step(torch.from_numpy(tokens[t]).to(gpu), st)
        lg = lg.cpu().numpy()
        worst = max(worst, float(np.abs(lg - logits[t]).max()))
        assert np.array_equal(lg.argmax(-1), logits[t].argmax(-1)), f"argmax differs at step {t}"
    print(f"forward_step fixture {name}: max |dlogit| {worst:.3g}", flush=True)
    assert worst < TOL
    assert state_close(st.s.cpu().numpy(), z["s"]) and state_close(st.hist.cpu().numpy(), z["hist"])
    net.handle.close()


@pytest.mark.parametrize("name", ["tiny", "small"])
def test_forward_all_positions_matches_reference_fixture(gpu, tmp_path, name):
    """forward(idx, return_state=True): (B, T, V) logits and the state with
    the history oldest first, as the reference's forward returns them."""
    cfg, seed, z = load_case(name)
    p = tmp_path / f"{name}.bin"
    p.write_bytes(pack_sunny_blob(init_sunnynet(cfg, seed)))
    B = z["tokens"].shape[1]
    net = HipSunnyNet(_model(p, cfg, max_batch=B))
    idx = torch.from_numpy(z["tokens"].T.copy()).to(gpu)
    lg, st = net.forward(idx, return_state=True)
    lg = lg.cpu().numpy()
    d = float(np.abs(lg - z["fwd_logits"]).max())
    print(f"forward fixture {name}: (B,T,V)={lg.shape}, max |dlogit| {d:.3g}", flush=True)
    assert d < TOL
    assert np.array_equal(lg.argmax(-1), z["fwd_logits"].argmax(-1))
    assert state_close(st.s.cpu().numpy(), z["fwd_s"])
    assert state_close(st.hist.cpu().numpy(), z["fwd_hist"])
    # forward without return_state gives the same logits; a carried state
    # (oldest-first history) continues the sequence like the torch path
    half = idx.shape[1] // 2
    l1, s1 = net.forward(idx[:, :half], return_state=True)
    l2 = net.forward(idx[:, half:], state=s1)
    both = np.concatenate([l1.cpu().numpy(), l2.cpu().numpy()], axis=1)
    assert np.abs(both - z["fwd_logits"]).max() < TOL
    net.handle.close()


def _ref_positions(ref, prompt):
    ref.reset()
    return np.stack([ref.step(int(t)) for t in prompt])


@pytest.mark.parametrize("chunk", [None, "128"])
def test_prefill_all_positions_small(gpu, tmp_path, ref_built, monkeypatch, chunk):
    """SunnyNet small, B=2, T=300: every position's logits against the
    reference runtime stepping each prompt (sn_step), in one chunk and in
    chunks of 128 (three chunks, the last ragged); the last position equals
    the last-token prefill's logits, and the state the last-token prefill's."""
    cfg = SMALL
    p = tmp_path / "small.bin"
    p.write_bytes(pack_sunny_blob(init_sunnynet(cfg, 0)))
    if chunk:
        monkeypatch.setenv("SNHIP_PREFILL_CHUNK", chunk)
    B, T = 2, 300
    prompts = np.random.default_rng(300).integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    hm = _model(p, cfg, max_batch=B)
    lg = hm.prefill_all(torch.from_numpy(prompts).to(gpu)).cpu().numpy()
    s_all, h_all = (x.cpu().numpy() for x in hm.get_state(B))
    hm.reset()
    last = hm.prefill_batch(torch.from_numpy(prompts).to(gpu)).cpu().numpy()
    s_last, h_last = (x.cpu().numpy() for x in hm.get_state(B))
    assert np.array_equal(s_all, s_last) and np.array_equal(h_all, h_last)
    assert np.abs(lg[:, -1] - last).max() < TOL
    ref = oracle.RefSnModel(p, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers)
    worst = 0.0
    for b in range(B):
        r = _ref_positions(ref, prompts[b])
        worst = max(worst, float(np.abs(lg[b] - r).max()))
        assert np.array_equal(lg[b].argmax(-1), r.argmax(-1)), b
    print(f"small B=2 T=300 chunk {chunk}: every position max |dlogit| {worst:.3g}", flush=True)
    assert worst < TOL
    ref.close()
    hm.close()


def test_prefill_all_positions_100m(gpu, tmp_path, ref_built):
    """SunnyNet-100M (seed 1), B=1, T=64: every position's logits against the
    reference runtime stepping the prompt."""
    cfg = SUNNY_100M
    print("generating SunnyNet-100M weights (seed 1)", flush=True)
    p = tmp_path / "m100.bin"
    p.write_bytes(pack_sunny_blob(init_sunnynet(cfg, 1)))
    T = 64
    prompt = np.random.default_rng(64).integers(0, cfg.vocab_size, (1, T)).astype(np.int32)
    hm = _model(p, cfg)
    lg = hm.prefill_all(torch.from_numpy(prompt).to(gpu)).cpu().numpy()[0]
    ref = oracle.RefSnModel(p, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers)
    r = _ref_positions(ref, prompt[0])
    d = float(np.abs(lg - r).max())
    print(f"100M B=1 T=64: every position max |dlogit| {d:.3g}", flush=True)
    assert d < TOL and np.array_equal(lg.argmax(-1), r.argmax(-1))
    ref.close()
    hm.close()


def test_prefill_all_rejects_bad_arguments(gpu, tmp_path):
    cfg = SMALL
    p = tmp_path / "small.bin"
    p.write_bytes(pack_sunny_blob(init_sunnynet(cfg, 0)))
    hm = _model(p, cfg, max_batch=2)
    with pytest.raises(RuntimeError):
        hm.prefill_all(torch.zeros(3, 4, dtype=torch.int32, device=gpu))   # B > max_batch
    hm.close()
