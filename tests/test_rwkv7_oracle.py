"""RWKV-7 oracle pinning (CPU).

* The C restatement (``RkOracle``) against the reference's own rwkv7.c
  (``sn_rk_step``, compiled unmodified into oracle/_ref) on fp32 v3 blobs from
  this package's writer: bit-identical logits, step after step.
* The numpy INT4 quantizer of the blob writer against the oracle's quant.c
  restatement (itself bit-exact vs the reference's ``sn_quant_i4``).
* The blob layout: the reference loader accepts the fp32 and the INT4 blob,
  and its vocabulary matches the header.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from sunnynet_amd.rwkv7 import (RWKV_TINY, RwkvConfig, dequant_i4_np, init_rwkv7,
                                pack_rwkv7_blob, quant_i4_np)


@pytest.mark.parametrize("block", [32, 64])
def test_quant_np_matches_oracle(block):
    rng = np.random.default_rng(block)
    x = (rng.standard_normal((40, 256)) * 0.3).astype(np.float32)
    x[3, :block] = 0.0
    x[7, 5] = 1e-30
    q, s = quant_i4_np(x, block)
    qo, so = oracle.quant_i4(x, block)
    assert np.array_equal(q, qo) and np.array_equal(s, so)
    assert np.array_equal(dequant_i4_np(q, s, 256, block), oracle.dequant_i4(qo, so, 256, block))


def _ref_or_skip():
    if not oracle.ref_available():
        pytest.skip("reference C build (oracle/_ref) not present")


@pytest.mark.parametrize("cfg", [RWKV_TINY, RwkvConfig(layers=3, dim=192, head_size=64, ff=320,
                                                        vocab=300, ranks=(32, 48, 16, 40))],
                         ids=["tiny", "odd"])
def test_oracle_matches_reference_step(tmp_path, cfg):
    _ref_or_skip()
    w = init_rwkv7(cfg, 2)
    blob = pack_rwkv7_blob(w)
    path = tmp_path / "rk.bin"
    path.write_bytes(blob)
    ref = oracle.RefRk(path, cfg.vocab)
    orc = oracle.RkOracle(blob)
    for t in np.random.default_rng(5).integers(0, cfg.vocab, 24):
        a = ref.step(int(t))
        b = orc.step([t])[0]
        assert np.array_equal(a, b)
    assert np.isfinite(a).all() and np.abs(a).max() > 1e-3


def test_reference_loads_int4_blob(tmp_path):
    _ref_or_skip()
    w = init_rwkv7(RWKV_TINY, 3)
    path = tmp_path / "rk4.bin"
    path.write_bytes(pack_rwkv7_blob(w, int4=True))
    ref = oracle.RefRk(path, RWKV_TINY.vocab)
    lg = ref.step(7)
    assert lg.shape == (RWKV_TINY.vocab,) and np.isfinite(lg).all()
    # The oracle dequantizes the same blob at load (W4A32); the reference
    # runs W4A8, so the two agree only to activation-quantization error.
    orc = oracle.RkOracle(path.read_bytes())
    lo = orc.step([7])[0]
    assert np.corrcoef(lg, lo)[0, 1] > 0.99
