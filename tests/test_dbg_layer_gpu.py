"""snhip_dbg_layer against the reference's sn_dbg_layer (sunnynet/runtime/
sunnynet.c:336-345, through the C oracle, which equals it bit for bit):
every intermediate of the asked layer (LN_in output, conv output, V at, the
gates, u, the new state, z, LN_I(z), W_eff s_old, the output) within 1e-5
absolute plus 1e-5 relative, on fresh and on stepped states, every layer; and
the state it leaves behind gives the oracle's next step within 2e-5."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from sunnynet_amd.blob import pack_sunny_blob
from sunnynet_amd.config import SMALL, TINY
from sunnynet_amd.runtime.model import HipModel
from sunnynet_amd.weights import init_sunnynet

pytestmark = pytest.mark.gpu


def _close(a, b):
    return bool((np.abs(a - b) <= 1e-5 + 1e-5 * np.abs(b)).all())


@pytest.mark.parametrize("cfg", [TINY, SMALL], ids=["tiny", "small"])
def test_dbg_layer_matches_reference(gpu, tmp_path, cfg):
    buf = pack_sunny_blob(init_sunnynet(cfg, 0))
    p = tmp_path / "m.bin"
    p.write_bytes(buf)
    hm = HipModel(p, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers)
    orc = oracle.SnOracle(buf)
    rng = np.random.default_rng(11)
    for t in rng.integers(0, cfg.vocab_size, 3):        # a stepped state first
        hm.step(int(t))
        orc.step([int(t)])
    print(f"dbg_layer {cfg.layers} layers", flush=True)
    for layer in range(cfg.layers):
        t = int(rng.integers(0, cfg.vocab_size))
        a = hm.dbg_layer(t, layer)
        b = orc.dbg_layer(0, t, layer)
        for k in a:
            assert _close(a[k], b[k]), (layer, k, float(np.abs(a[k] - b[k]).max()))
    t = int(rng.integers(0, cfg.vocab_size))
    lg = np.asarray(hm.step(t), np.float32)
    assert np.abs(lg - orc.step([t])[0]).max() < 2e-5
    with pytest.raises(RuntimeError):
        hm.dbg_layer(0, cfg.layers)
    hm.close()
