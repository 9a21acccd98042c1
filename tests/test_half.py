"""fp16 weights as the reference's sn_load_h (sunnynet.c:455-579) holds them:
V, U, W_z, W_c, W_s_eff and the LM head rounded to fp16 (nearest, ties to
even: _cvtss_sh(x, 0)) at load, multiplied in fp32; the lookup embedding and
the small parameters stay fp32.

The rounding rule is pinned on the CPU: the oracle stepping a blob whose
matrices were rounded through numpy's float16 agrees with the reference's own
sn_load_h handle (different accumulation order, so within 2e-5, not bit for
bit); a plain fp32 handle differs from both by far more, so the check sees the
rounding. On the GPU, the backend's fp16 format matches the same oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from sunnynet_amd.blob import BlobMatrices, layer_matrices, pack_sunny_blob
from sunnynet_amd.config import SMALL, TINY
from sunnynet_amd.weights import init_sunnynet

TOL = 2e-5


def half_blob(w) -> bytes:
    r = lambda M: np.asarray(M, np.float32).astype(np.float16).astype(np.float32)
    mats = []
    for l in range(w.cfg.layers):
        M = layer_matrices(w, l)
        mats.append(BlobMatrices(**{k: r(getattr(M, k)) for k in ("V", "U", "W_z", "W_c", "W_s_eff")}))
    return pack_sunny_blob(w, matrices=mats, head=r(w.head_weight().detach().numpy()))


def test_half_rounding_matches_reference_sn_load_h(tmp_path):
    if not oracle.ref_available():
        pytest.skip("reference build absent")
    cfg = TINY
    w = init_sunnynet(cfg, 0)
    full = tmp_path / "f32.bin"
    full.write_bytes(pack_sunny_blob(w))
    ref_h = oracle.RefSnModel(full, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers,
                              half=True)
    orc_h = oracle.SnOracle(half_blob(w))
    orc_f = oracle.SnOracle(pack_sunny_blob(w))
    worst_h = worst_f = 0.0
    for t in (3, 17, 200, 5, 511, 64, 9, 300):
        a = ref_h.step(t)
        worst_h = max(worst_h, float(np.abs(a - orc_h.step([t])[0]).max()))
        worst_f = max(worst_f, float(np.abs(a - orc_f.step([t])[0]).max()))
    assert worst_h < TOL
    assert worst_f > 10 * TOL          # the fp16 rounding is visible at this scale


@pytest.mark.gpu
@pytest.mark.parametrize("B", [1, 8])
def test_half_weights_match_rounded_oracle(gpu, tmp_path, B):
    import torch
    from sunnynet_amd.runtime.model import HipModel
    cfg = SMALL
    w = init_sunnynet(cfg, 0)
    p = tmp_path / "f32.bin"
    p.write_bytes(pack_sunny_blob(w))
    hm = HipModel(p, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, half=True,
                  max_batch=B)
    orc = oracle.SnOracle(half_blob(w), batch=B)
    rng = np.random.default_rng(B)
    for _ in range(8):
        toks = rng.integers(0, cfg.vocab_size, B).astype(np.int32)
        a = hm.step_batch(torch.from_numpy(toks).to(gpu)).cpu().numpy()
        b = orc.step(toks)
        assert np.abs(a - b).max() < TOL
        assert np.array_equal(a.argmax(1), b.argmax(1))


@pytest.mark.gpu
@pytest.mark.parametrize("cfg_name", ["small", "100m"])
def test_half_storage_step_equals_fp32_step_on_rounded_weights(gpu, tmp_path, cfg_name):
    """The fp16 format stores the matrices as fp16 for the single-sequence
    persistent step (half the bytes streamed) and converts them in registers:
    its greedy chain and logits equal, bit for bit, the fp32 persistent step
    on a blob holding the same fp16-rounded values (same kernel geometry,
    same values multiplied)."""
    import torch
    from sunnynet_amd.config import SUNNY_100M
    from sunnynet_amd.runtime.model import HipModel
    cfg = {"small": SMALL, "100m": SUNNY_100M}[cfg_name]
    w = init_sunnynet(cfg, 0 if cfg is SMALL else 1)
    p32 = tmp_path / "f32.bin"
    p32.write_bytes(pack_sunny_blob(w))
    prd = tmp_path / "rounded.bin"
    prd.write_bytes(half_blob(w))
    dims = (cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers)
    print(f"fp16 storage vs fp32 on rounded weights: {cfg_name}", flush=True)
    hh = HipModel(p32, *dims, half=True)
    hr = HipModel(prd, *dims)
    assert hh.persistent_grid > 0 and hr.persistent_grid > 0
    start = torch.tensor([7], dtype=torch.int32, device=gpu)
    lh = torch.empty(1, cfg.vocab_size, device=gpu)
    lr = torch.empty(1, cfg.vocab_size, device=gpu)
    th = hh.decode_greedy(start, 24, logits=lh)
    tr = hr.decode_greedy(start, 24, logits=lr)
    assert torch.equal(th, tr)
    assert torch.equal(lh, lr)
    # and the one-step surface: host logits of a fresh pair of handles
    hh.reset(); hr.reset()
    for t in (5, 900, 31):
        assert hh.step(t) == hr.step(t)
    hh.close(); hr.close()
