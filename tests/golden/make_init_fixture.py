"""Writes tests/golden/init_weights.json: fingerprints of the reference's own
``SunnyNet(cfg)`` weights right after ``torch.manual_seed(seed)``
(sunnynet/model.py:55-72, sunnynet/layers.py:88-157, sunnynet/init.py:10-23),
which only an import of the reference can produce (torch's RNG stream).

Run in a container that has the reference checkout (read-only; nothing is
compiled or written there: the optional C kernels stay off and no bytecode is
written):

    python tests/golden/make_init_fixture.py /root/reference

Per tensor: shape, float64 sum and sum of squares, sha256 of the fp32 bytes,
and the values at 64 evenly spaced flat positions
(``numpy.linspace(0, n - 1, 64).round()``).
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
from pathlib import Path

sys.dont_write_bytecode = True
os.environ["SUNNY_KERNEL"] = "0"

CASES = [  # name, SunnyConfig fields, seed
    ("tiny", dict(vocab_size=512, dim=64, inner=96, rank=32, taps=4, layers=2), 0),
    ("small", dict(vocab_size=4096, dim=256, inner=384, rank=128, taps=4, layers=4), 0),
    ("100m", dict(vocab_size=32000, dim=1024, inner=1536, rank=512, taps=4, layers=12), 1),
]
NSAMP = 64


def fingerprint(t):
    import numpy as np
    a = t.detach().to("cpu").float().contiguous().numpy()
    flat = a.reshape(-1)
    idx = np.linspace(0, flat.size - 1, num=min(NSAMP, flat.size)).round().astype(np.int64)
    return {"shape": list(a.shape), "sum": float(flat.astype(np.float64).sum()),
            "sumsq": float((flat.astype(np.float64) ** 2).sum()),
            "sha256": hashlib.sha256(flat.tobytes()).hexdigest(),
            "val": [float(v) for v in flat[idx]]}


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import torch
    from sunnynet.model import SunnyConfig, SunnyNet
    out = {"torch": torch.__version__, "cases": {}}
    for name, fields, seed in CASES:
        torch.manual_seed(seed)
        m = SunnyNet(SunnyConfig(**fields))
        out["cases"][name] = {"config": fields, "seed": seed,
                              "tensors": {k: fingerprint(v) for k, v in m.state_dict().items()}}
        print(name, len(out["cases"][name]["tensors"]), "tensors", flush=True)
    Path(__file__).with_name("init_weights.json").write_text(json.dumps(out, indent=0))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
