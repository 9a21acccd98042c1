"""Writes tests/golden/forward_step_{tiny,small}.npz: the reference's own fp32
``SunnyNet.forward_step`` logits and state along a greedy chain, and its
``SunnyNet.forward`` logits at every position over the same tokens
(sunnynet/model.py:89-124, sunnynet/layers.py:256-326), for the weights
``SunnyNet(cfg)`` draws right after ``torch.manual_seed(seed)``.

The north-star parity bar (logits within 2e-5 absolute, equal greedy argmax)
is stated against ``forward_step`` itself; torch's own fp32 rounding of
``layer_norm``, ``linear`` and ``sigmoid`` can only be captured by running it.

Run in a container that has the reference checkout (read-only; nothing is
compiled or written there: the optional C kernels stay off, SUNNY_KERNEL=0,
and no bytecode is written), on one CPU thread:

    python tests/golden/make_step_fixture.py /root/reference

Per case (numpy arrays, no pickled objects):
  config  int64 [vocab, dim, inner, rank, taps, layers, seed]
  tokens  int32 (T, B)       token fed at each step: P prompt ids drawn by
                             numpy PCG64(seed 7), then the greedy argmax
  logits  float32 (T, B, V)  forward_step logits after each step
  s, hist float32            state after the last step: s (B, L, D), hist
                             (B, L, K-1, D) newest first
  fwd_logits float32 (B, T, V)  forward(tokens.T) logits at every position
  fwd_s, fwd_hist            forward's final state (hist oldest first, as
                             forward returns it: layers.py:266)
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

sys.dont_write_bytecode = True
os.environ["SUNNY_KERNEL"] = "0"

CASES = [  # name, SunnyConfig fields, seed, batch, prompt length, total steps
    ("tiny", dict(vocab_size=512, dim=64, inner=96, rank=32, taps=4, layers=2), 0, 2, 8, 32),
    ("small", dict(vocab_size=4096, dim=256, inner=384, rank=128, taps=4, layers=4), 0, 1, 4, 12),
]


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import numpy as np
    import torch
    torch.set_num_threads(1)
    from sunnynet.model import SunnyConfig, SunnyNet
    for name, fields, seed, B, P, T in CASES:
        torch.manual_seed(seed)
        m = SunnyNet(SunnyConfig(**fields)).eval()
        rng = np.random.default_rng(7)
        prompt = rng.integers(0, fields["vocab_size"], (P, B)).astype(np.int64)
        st = m.init_state(B)
        toks, logits = [], []
        nxt = None
        with torch.no_grad():
            for t in range(T):
                cur = prompt[t] if t < P else nxt
                toks.append(cur.astype(np.int32))
                lg, st = m.forward_step(torch.from_numpy(cur), st)
                logits.append(lg.numpy().astype(np.float32))
                nxt = lg.argmax(-1).numpy().astype(np.int64)
            idx = torch.from_numpy(np.stack(toks).T.astype(np.int64).copy())
            flg, fst = m.forward(idx, return_state=True)
        out = Path(__file__).with_name(f"forward_step_{name}.npz")
        cfg = [fields[k] for k in ("vocab_size", "dim", "inner", "rank", "taps", "layers")] + [seed]
        np.savez_compressed(
            out, config=np.asarray(cfg, np.int64), tokens=np.stack(toks),
            logits=np.stack(logits), s=st.s.numpy(), hist=st.hist.numpy(),
            fwd_logits=flg.numpy().astype(np.float32), fwd_s=fst.s.numpy(),
            fwd_hist=fst.hist.numpy(), torch_version=np.frombuffer(
                torch.__version__.encode(), np.uint8))
        print(name, out.stat().st_size, "bytes", flush=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
