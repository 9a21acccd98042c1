"""The oracles against the reference's own fp32 ``forward_step`` and
``forward`` (sunnynet/model.py:89-124), recorded by
tests/golden/make_step_fixture.py on the weights ``SunnyNet(cfg)`` draws after
``torch.manual_seed(0)``: the C oracle (the reference C runtime's rounding,
sunnynet.c:212-334) and the torch restatement stay within the north-star bar
(2e-5 absolute, equal greedy argmax) of the real function along a greedy
chain, and the restated prefill matches the reference's every-position
logits."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from oracle.torch_ref import TorchSunny, forward_hist_to_step
from sunnynet_amd.blob import pack_sunny_blob
from sunnynet_amd.config import SunnyConfig
from sunnynet_amd.weights import init_sunnynet

GOLD = Path(__file__).parent / "golden"
TOL = 2e-5


def state_close(a, b):
    """State entries within 1e-5 absolute plus 1e-5 relative: the history
    holds LayerNorm outputs of magnitude up to ~4, where fp32 rounding of the
    residual stream moves them by a few ulps more than the logits."""
    return bool((np.abs(np.asarray(a) - np.asarray(b)) <= 1e-5 + 1e-5 * np.abs(np.asarray(b))).all())


def load_case(name):
    z = np.load(GOLD / f"forward_step_{name}.npz")
    V, D, I, R, K, L, seed = (int(v) for v in z["config"])
    cfg = SunnyConfig(vocab_size=V, dim=D, inner=I, rank=R, taps=K, layers=L)
    return cfg, seed, {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", ["tiny", "small"])
def test_c_oracle_follows_forward_step(name):
    cfg, seed, z = load_case(name)
    tokens, logits = z["tokens"], z["logits"]
    T, B = tokens.shape
    orc = oracle.SnOracle(pack_sunny_blob(init_sunnynet(cfg, seed)), batch=B)
    worst = 0.0
    for t in range(T):
        lg = orc.step(tokens[t])
        worst = max(worst, float(np.abs(lg - logits[t]).max()))
        assert np.array_equal(lg.argmax(-1), logits[t].argmax(-1)), f"argmax differs at step {t}"
    print(f"{name}: C oracle vs forward_step max |diff| {worst:.3e} over {T} steps x B={B}")
    assert worst < TOL
    s, h = orc.get_state()
    assert state_close(s, z["s"]) and state_close(h, z["hist"])


@pytest.mark.parametrize("name", ["tiny", "small"])
def test_torch_restatement_follows_forward_step(name):
    cfg, seed, z = load_case(name)
    tokens, logits = z["tokens"], z["logits"]
    T, B = tokens.shape
    ts = TorchSunny(init_sunnynet(cfg, seed))
    st = ts.init_state(B)
    worst = 0.0
    for t in range(T):
        lg, st = ts.forward_step(torch.from_numpy(tokens[t].astype(np.int64)), st)
        worst = max(worst, float(np.abs(lg.numpy() - logits[t]).max()))
    print(f"{name}: torch restatement vs forward_step max |diff| {worst:.3e}")
    assert worst < TOL


@pytest.mark.parametrize("name", ["tiny", "small"])
def test_fixture_forward_is_forward_step(name):
    """The reference's own prefill and step agree on the recorded tokens: its
    every-position logits are the per-step logits to fp32 rounding, and
    forward's (oldest-first) history is the step's reversed."""
    cfg, seed, z = load_case(name)
    fl = np.transpose(z["fwd_logits"], (1, 0, 2))      # (T, B, V)
    assert np.abs(fl - z["logits"]).max() < TOL
    assert state_close(z["fwd_s"], z["s"])
    assert state_close(forward_hist_to_step(torch.from_numpy(z["fwd_hist"])).numpy(), z["hist"])


@pytest.mark.parametrize("name", ["tiny", "small"])
def test_torch_prefill_matches_reference_forward(name):
    cfg, seed, z = load_case(name)
    ts = TorchSunny(init_sunnynet(cfg, seed))
    idx = torch.from_numpy(z["tokens"].T.astype(np.int64).copy())
    lg, (s, h) = ts.forward(idx)
    assert np.abs(lg.numpy() - z["fwd_logits"]).max() < TOL
    assert state_close(s.numpy(), z["fwd_s"]) and state_close(h.numpy(), z["fwd_hist"])
