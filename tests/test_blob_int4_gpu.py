"""Loading the INT4 blob: a handle built from it holds the same codes and
scales as one that quantizes the fp32 blob at load, so every decode path gives
bit-identical logits (B=1 persistent kernel, the same kernel on a grid slice
per sequence at B=3 and 16, the batched kernel at B=24, chunked prefill); and
the loader refuses the format where it does not apply.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from sunnynet_amd.blob import convert_blob_int4, pack_sunny_blob
from sunnynet_amd.config import SMALL
from sunnynet_amd.runtime.model import HipModel
from sunnynet_amd.weights import gaussian_matmuls, init_sunnynet

pytestmark = pytest.mark.gpu


def _model(path, cfg, **kw):
    return HipModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, **kw)


@pytest.fixture(scope="module")
def blobs(tmp_path_factory):
    buf = pack_sunny_blob(gaussian_matmuls(init_sunnynet(SMALL, 0), seed=3))
    d = tmp_path_factory.mktemp("i4blob")
    (d / "f32.bin").write_bytes(buf)
    for block in (32, 64):
        (d / f"q{block}.bin").write_bytes(convert_blob_int4(buf, block))
    return d


@pytest.mark.parametrize("block", [32, 64])
def test_int4_blob_loads_bit_identical(gpu, blobs, block):
    print(f"INT4 blob block={block}", flush=True)
    rng = np.random.default_rng(block)
    for B in (1, 3, 16, 24):
        ha = _model(blobs / "f32.bin", SMALL, weights="int4", block=block, max_batch=B)
        hb = _model(blobs / f"q{block}.bin", SMALL, weights="int4", block=block, max_batch=B)
        for _ in range(4):
            t = torch.from_numpy(rng.integers(0, SMALL.vocab_size, B).astype(np.int32)).to(gpu)
            assert np.array_equal(ha.step_batch(t).cpu().numpy(), hb.step_batch(t).cpu().numpy()), B
    ha = _model(blobs / "f32.bin", SMALL, weights="int4", block=block, max_batch=2)
    hb = _model(blobs / f"q{block}.bin", SMALL, weights="int4", block=block, max_batch=2)
    ids = torch.from_numpy(rng.integers(0, SMALL.vocab_size, (2, 300)).astype(np.int32)).to(gpu)
    assert np.array_equal(ha.prefill_batch(ids).cpu().numpy(), hb.prefill_batch(ids).cpu().numpy())


def test_int4_blob_refused_where_it_does_not_apply(gpu, blobs):
    with pytest.raises(RuntimeError, match="INT4"):
        _model(blobs / "q32.bin", SMALL)                                     # fp32 handle
    with pytest.raises(RuntimeError, match="group size"):
        _model(blobs / "q32.bin", SMALL, weights="int4", block=64)           # other block
