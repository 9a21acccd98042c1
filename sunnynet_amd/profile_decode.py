"""Fixed launch sequences for rocprofv3 kernel-trace summaries of the
SunnyNet-100M token loop (seed-1 random init; INT4 g32 on N(0, 0.02)
matmuls).

    rocprofv3 --kernel-trace --stats -d <dir> -- python3 -m sunnynet_amd.profile_decode [b1|batch|rwkv]

b1 (default): a chunked prefill of 1024 random ids, then 256 greedy decode
steps at B=1, for fp32 and INT4 weights. batch: 64 greedy steps at B=64 with
fp32 weights and at B=8 and B=32 with INT4 weights, from random tokens.
rwkv: the RWKV-7 configuration (12 layers, D=768, vocab 65536, seed-2
weights, INT4 g32 at load), 64 greedy steps at B=1 and at B=64 after 8
warm-up steps.
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


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    which = argv[0] if argv else "b1"
    if which == "rwkv":
        return rwkv()
    cfg = SUNNY_100M
    dev = torch.device("cuda:0")
    tmp = tempfile.mkdtemp(prefix="snhip_prof_")
    w = init_sunnynet(cfg, 1)
    g = torch.Generator(device="cpu").manual_seed(5)
    paths = {}
    for fmt, weights in (("fp32", w), ("int4", gaussian_matmuls(w, seed=3))):
        paths[fmt] = os.path.join(tmp, f"m100_{fmt}.bin")
        with open(paths[fmt], "wb") as f:
            f.write(pack_sunny_blob(weights))
    cases = ([("fp32", 1), ("int4", 1)] if which == "b1" else
             [("fp32", 64), ("int4", 8), ("int4", 32)])
    for fmt, B in cases:
        hm = HipModel(paths[fmt], cfg.vocab_size, cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers,
                      max_batch=B, weights=fmt, block=32)
        if B == 1:
            ids = torch.randint(0, cfg.vocab_size, (1, 1024), generator=g, dtype=torch.int32).to(dev)
            tok = hm.prefill_batch(ids).argmax(1).int()
            n = 256
        else:
            tok = torch.randint(0, cfg.vocab_size, (B,), generator=g, dtype=torch.int32).to(dev)
            n = 64
        hm.decode_greedy(tok, n)
        torch.cuda.synchronize()
        hm.close()
        print(f"[profile] {fmt} B={B}: {n} greedy steps", file=sys.stderr, flush=True)
    return 0


def rwkv() -> int:
    from sunnynet_amd.runtime.rwkv7 import HipRwkv7
    from sunnynet_amd.rwkv7 import RWKV_CFG4, init_rwkv7, pack_rwkv7_blob
    cfg = RWKV_CFG4
    tmp = tempfile.mkdtemp(prefix="snhip_prof_rk_")
    path = os.path.join(tmp, "rk.bin")
    with open(path, "wb") as f:
        f.write(pack_rwkv7_blob(init_rwkv7(cfg, 2)))
    g = torch.Generator(device="cpu").manual_seed(7)
    for B in (1, 64):
        hm = HipRwkv7(path, weights="int4", block=32, max_batch=B)
        tok = torch.randint(0, cfg.vocab, (B,), generator=g, dtype=torch.int32).cuda()
        hm.decode_greedy(tok, 8)
        hm.decode_greedy(tok, 64)
        torch.cuda.synchronize()
        print(f"[profile] rwkv7 int4 B={B}: 64 greedy steps (persistent grid {hm.persist_grid})",
              file=sys.stderr, flush=True)
        hm.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
