"""Pins of the weight inputs.

* Seeded init: ``init_sunnynet(cfg, seed)`` against the reference's own
  ``SunnyNet(cfg)`` after ``torch.manual_seed(seed)`` (sunnynet/model.py:55-72,
  sunnynet/layers.py:88-157, sunnynet/init.py:10-23), through the fingerprints
  that tests/golden/make_init_fixture.py wrote by importing the reference:
  sha256 of every tensor's fp32 bytes, sums, and 64 sampled values.
* The feedback fold (sunnynet/layers.py:33-42, 219-226; the reference's own
  check is tests/test_architecture.py:510-520): W_s(circ(x)) == W_eff x, with
  circ written out from StateCirculant's definition
  y_i = t0 x_{i-1} + t1 x_i + t2 x_{i+1} (indices mod D), on asymmetric taps so
  that a fold with the roll directions swapped fails.
* The forgetting bound (sunnynet/layers.py:137-141 with theta at
  horizon_logit, ops.py:62-65): sigmoid(theta_i) = (i + 0.5) / D, so
  delta_i = 1 / (h_min (h_max / h_min)^((i + 0.5) / D)) = 1 / (2 * 4096^((i + 0.5) / D)).
"""
from __future__ import annotations

import hashlib
import json
from types import SimpleNamespace
from pathlib import Path

import numpy as np
import pytest
import torch

from sunnynet_amd.config import SMALL, SUNNY_100M, TINY
from sunnynet_amd.weights import SunnyWeights, horizon_logit, init_sunnynet

FIXTURE = Path(__file__).parent / "golden" / "init_weights.json"


def _named(w):
    out = {"embed.weight": w.embed, "head.weight": w.embed, "norm_out.gamma": w.no_g,
           "norm_out.center": w.no_c}
    for i, L in enumerate(w.layers):
        b = f"blocks.{i}."
        out.update({b + "a": L.a, b + "b_gain": L.b_gain, b + "theta": L.theta,
                    b + "norm_in.gamma": L.ni_g, b + "norm_in.center": L.ni_c,
                    b + "norm_mix.gamma": L.nm_g, b + "norm_mix.center": L.nm_c,
                    b + "circ.t": L.circ, b + "dw.weight": L.dw, b + "V.weight": L.V,
                    b + "U.weight": L.U, b + "W_z.weight": L.W_z, b + "W_c.weight": L.W_c,
                    b + "W_s.weight": L.W_s})
    return out


@pytest.mark.parametrize("name,cfg,seed", [("tiny", TINY, 0), ("small", SMALL, 0),
                                           ("100m", SUNNY_100M, 1)])
def test_init_equals_reference_weights(name, cfg, seed):
    case = json.loads(FIXTURE.read_text())["cases"][name]
    assert case["seed"] == seed
    for k, v in case["config"].items():
        assert getattr(cfg, k) == v
    ref = case["tensors"]
    mine = _named(init_sunnynet(cfg, seed))
    # every tensor the runtime consumes has a reference fingerprint
    assert set(mine) <= set(ref)
    for k, t in mine.items():
        a = t.detach().float().contiguous().numpy()
        r = ref[k]
        assert list(a.shape) == r["shape"], k
        flat = a.reshape(-1)
        idx = np.linspace(0, flat.size - 1, num=min(64, flat.size)).round().astype(np.int64)
        assert flat[idx].tolist() == r["val"], k
        assert hashlib.sha256(flat.tobytes()).hexdigest() == r["sha256"], k


def _circ(x, t):
    """StateCirculant.forward written out: y_i = t0 x_{i-1} + t1 x_i + t2 x_{i+1}."""
    D = x.shape[-1]
    y = torch.empty_like(x)
    for i in range(D):
        y[..., i] = t[0] * x[..., (i - 1) % D] + t[1] * x[..., i] + t[2] * x[..., (i + 1) % D]
    return y


def test_feedback_fold_identity():
    w = init_sunnynet(TINY, 0)
    D = TINY.dim
    g = torch.Generator().manual_seed(7)
    W = torch.randn(D, D, generator=g, dtype=torch.float64)
    x = torch.randn(5, D, generator=g, dtype=torch.float64)
    for t in (torch.tensor([0.25, 0.5, 0.25], dtype=torch.float64),
              torch.tensor([0.1, 0.5, 0.3], dtype=torch.float64)):
        L = w.layers[0]
        L.W_s, L.circ = W, t
        Weff = w.ws_eff(0)
        ref = _circ(x, t) @ W.T
        assert float((x @ Weff.T - ref).abs().max()) < 1e-12
    # the same check rejects a fold with the roll directions swapped
    t = torch.tensor([0.1, 0.5, 0.3], dtype=torch.float64)
    swapped = t[0] * torch.roll(W, 1, dims=1) + t[1] * W + t[2] * torch.roll(W, -1, dims=1)
    assert float((x @ swapped.T - _circ(x, t) @ W.T).abs().max()) > 1e-3


@pytest.mark.parametrize("cfg", [TINY, SMALL, SUNNY_100M])
def test_delta_closed_form(cfg):
    D = cfg.dim
    # SunnyWeights.delta on the initial theta (the layers' theta at init)
    w = SunnyWeights(cfg=cfg, embed=torch.zeros(1, D))
    w.layers = [SimpleNamespace(theta=horizon_logit(D))]
    i = np.arange(D, dtype=np.float64)
    closed = 1.0 / (cfg.h_min * (cfg.h_max / cfg.h_min) ** ((i + 0.5) / D))
    assert cfg.h_min == 2 and cfg.h_max == 8192
    np.testing.assert_allclose(closed, 1.0 / (2.0 * 4096.0 ** ((i + 0.5) / D)), rtol=1e-15)
    got = w.delta(0).double().numpy()
    np.testing.assert_allclose(got, closed, rtol=2e-6)
    assert got[0] > got[-1] and np.all(np.diff(got) < 0)      # log-spaced, decreasing
