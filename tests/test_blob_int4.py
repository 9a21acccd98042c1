"""The INT4 SunnyNet blob (pre-quantized V, U, W_z, W_c, W_s_eff and head):
its writer against quant.c's arithmetic, and its reader.

The codes and scales must be exactly what sn_quant_i4 (quant.c:34-66) gives
for the fp32 blob's matrices: the oracle's restatement of it is pinned
bit-exact against the reference build (tests/test_oracle.py), and here it is
the witness for every matrix of a converted blob.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

import oracle
from sunnynet_amd.blob import (I4_HEADER_BYTES, I4_MAGIC, convert_blob_int4, pack_sunny_blob,
                               parse_blob_int4, parse_sunny_blob)
from sunnynet_amd.config import TINY
from sunnynet_amd.weights import gaussian_matmuls, init_sunnynet


@pytest.fixture(scope="module")
def blob():
    return pack_sunny_blob(gaussian_matmuls(init_sunnynet(TINY, 0), seed=3))


@pytest.mark.parametrize("block", [32])
def test_int4_blob_matches_quant_c(blob, block):
    q = convert_blob_int4(blob, block)
    h = struct.unpack_from("<12i", q, 0)
    cfg = TINY
    assert h[0] == I4_MAGIC and h[1] == 1
    assert h[2:8] == (cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers)
    assert h[11] == block
    f = parse_sunny_blob(blob)
    p = parse_blob_int4(q)
    for lf, lq in zip(f["layers"], p["layers"]):
        for k in ("ni_g", "ni_c", "nm_g", "nm_c", "dw_t", "delta"):
            assert np.array_equal(lf[k], lq[k])
        assert lf["a_tanh"] == lq["a_tanh"] and lf["b_gain"] == lq["b_gain"]
        for k in ("V", "U", "W_z", "W_c", "W_s_eff"):
            qo, so = oracle.quant_i4(lf[k], block)
            assert np.array_equal(lq[k][0], qo) and np.array_equal(lq[k][1], so), k
    assert np.array_equal(f["embed"], p["embed"])
    qo, so = oracle.quant_i4(f["head"], block)
    assert np.array_equal(p["head"][0], qo) and np.array_equal(p["head"][1], so)
    assert f["eps"] == p["eps"] and f["p_floor"] == p["p_floor"]


def test_int4_blob_size_and_errors(blob):
    q = convert_blob_int4(blob, 32)
    cfg = TINY
    D, I, R, K, L, V = cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, cfg.vocab_size
    qb = lambda out, inn: out * inn // 2 + 4 * out * (inn // 32)
    per_layer = 4 * (2 * D + 2 * I + K * D + D + 2) + qb(R, D) + qb(2 * D, R) + qb(I, D) + qb(D, I) + qb(D, D)
    assert len(q) == I4_HEADER_BYTES + L * per_layer + 4 * (2 + 2 * D + V * D) + qb(V, D)
    with pytest.raises(ValueError):
        parse_blob_int4(q + b"\0")
    with pytest.raises(ValueError):
        convert_blob_int4(blob, 48)
    with pytest.raises(ValueError):
        parse_blob_int4(blob)               # an fp32 blob is not an INT4 blob
