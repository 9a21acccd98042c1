"""The torch backend's step contract on the HIP handle: ``forward_step(idx_t,
SunnyState) -> (logits, SunnyState)`` (sunnynet/model.py:113-124,
sunnynet/layers.py:21-30).

Sequences move between the fp32 torch restatement of ``forward_step`` and the
HIP handle mid-stream (torch -> HIP -> torch), and every step's logits must
equal the all-torch run within 2e-5 with the same argmax; the state the HIP
side hands back must match the torch state within 1e-5.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.torch_ref import TorchSunny
from sunnynet_amd.blob import pack_sunny_blob
from sunnynet_amd.config import SMALL
from sunnynet_amd.runtime.model import HipModel, HipSunnyNet, SunnyState
from sunnynet_amd.weights import init_sunnynet

pytestmark = pytest.mark.gpu
TOL = 2e-5


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    w = init_sunnynet(SMALL, 0)
    p = tmp_path_factory.mktemp("fs") / "small.bin"
    p.write_bytes(pack_sunny_blob(w))
    return w, p


def _torch_step(tr, idx, st: SunnyState):
    lg, (s, h) = tr.forward_step(idx, (st.s, st.hist))
    return lg, SunnyState(s, h)


@pytest.mark.parametrize("B", [1, 3])
def test_sequence_swaps_between_torch_and_hip(gpu, small, B):
    w, path = small
    c = SMALL
    print(f"forward_step swap B={B}: torch 6 -> hip 6 -> torch 6", flush=True)
    tr = TorchSunny(w, torch.float32)
    hm = HipModel(path, c.vocab_size, c.dim, c.inner, c.rank, c.taps, c.layers, max_batch=4)
    net = HipSunnyNet(hm)
    toks = torch.from_numpy(np.random.default_rng(B).integers(0, c.vocab_size, (18, B)))
    ref = SunnyState(*tr.init_state(B))
    ref_logits = []
    for t in range(18):
        lg, ref = _torch_step(tr, toks[t], ref)
        ref_logits.append(lg)
        if t == 11:
            ref_mid = ref
    st = net.init_state(B, device="cpu")
    assert st.s.shape == (B, c.layers, c.dim) and st.hist.shape == (B, c.layers, c.taps - 1, c.dim)
    for t in range(18):
        if 6 <= t < 12:
            lg, st = net.forward_step(toks[t], st)
            assert lg.device.type == "cuda" and st.s.device.type == "cuda"
            lg = lg.cpu()
            st = st.to(device="cpu")
        else:
            lg, st = _torch_step(tr, toks[t], st)
        d = float((lg - ref_logits[t]).abs().max())
        assert d < TOL, (t, d)
        assert torch.equal(lg.argmax(-1), ref_logits[t].argmax(-1)), t
        if t == 11:
            assert float((st.s - ref_mid.s).abs().max()) < 1e-5
            assert float((st.hist - ref_mid.hist).abs().max()) < 1e-5
    hm.close()


def test_forward_step_accepts_other_dtypes_and_checks_batch(gpu, small):
    w, path = small
    c = SMALL
    hm = HipModel(path, c.vocab_size, c.dim, c.inner, c.rank, c.taps, c.layers, max_batch=2)
    net = HipSunnyNet(hm)
    st64 = net.init_state(2, dtype=torch.float64)
    idx = torch.tensor([5, 7])
    lg, st = net.forward_step(idx, st64)
    assert lg.shape == (2, c.vocab_size) and st.s.dtype == torch.float32
    lg32, _ = net.forward_step(idx, net.init_state(2))
    assert torch.equal(lg, lg32)
    with pytest.raises(ValueError):
        net.forward_step(torch.tensor([1, 2, 3]), net.init_state(3))
    with pytest.raises(ValueError):
        net.forward_step(idx, net.init_state(1))
    hm.close()
