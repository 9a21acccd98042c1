"""Fixed launch sequence for rocprofv3 kernel-trace summaries of the
SunnyNet-100M token loop (seed-1 random init; INT4 g32 on N(0, 0.02)
matmuls): a chunked prefill of 1024 random ids, then 256 greedy decode steps
at B=1, for fp32 and INT4 weights.

    rocprofv3 --kernel-trace --stats -d <dir> -- python3 -m sunnynet_amd.profile_decode
"""
from __future__ import annotations

import os
import sys
import tempfile

import torch

from sunnynet_amd.blob import pack_sunny_blob
from sunnynet_amd.config import SUNNY_100M
from sunnynet_amd.runtime.model import HipModel
from sunnynet_amd.weights import gaussian_matmuls, init_sunnynet


def main() -> int:
    cfg = SUNNY_100M
    dev = torch.device("cuda:0")
    tmp = tempfile.mkdtemp(prefix="snhip_prof_")
    w = init_sunnynet(cfg, 1)
    g = torch.Generator(device="cpu").manual_seed(5)
    for fmt, weights in (("fp32", w), ("int4", gaussian_matmuls(w, seed=3))):
        path = os.path.join(tmp, f"m100_{fmt}.bin")
        with open(path, "wb") as f:
            f.write(pack_sunny_blob(weights))
        hm = HipModel(path, cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers,
                      max_batch=1, weights=fmt, block=32)
        ids = torch.randint(0, cfg.vocab_size, (1, 1024), generator=g, dtype=torch.int32).to(dev)
        lg = hm.prefill_batch(ids)
        tok = lg.argmax(1).int()
        hm.decode_greedy(tok, 256)
        torch.cuda.synchronize()
        hm.close()
        print(f"[profile] {fmt}: prefill 1024 + 256 greedy steps at B=1", file=sys.stderr, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
