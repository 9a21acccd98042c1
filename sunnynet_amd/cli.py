"""Text-generation driver over the HIP decode handle.

The reference CLI's decode loop (``decode_stream``, sunnynet/cli.py:57-106)
with the handle selected by ``--backend hip`` (the reference's switch,
cli.py:299-300, 337-347): the prompt goes through ``runtime.prefill(ids)``,
every generated token through ``runtime.step(token)``, sampling happens on
the host, and the statistics dict has the reference's keys.

    python -m sunnynet_amd.cli --backend hip --blob m.bin --config small \\
        --prompt-ids 1,2,3 --max-new 64 --temperature 0 --json

Prompts are token ids (``--prompt-ids``) or text encoded with the reference
CLI's byte fallback (cli.py:224-225: id 1, then each UTF-8 byte + 2); the
reference's BPE tokenizer file is not part of this package.
"""
from __future__ import annotations

import argparse
import json
import sys
import time

import torch

from .config import PRESETS
from .runtime.model import HipModel, recommended_threads, set_threads

__all__ = ["ByteTokenizer", "decode_stream", "main", "sample"]


class ByteTokenizer:
    """The reference CLI's byte fallback (cli.py:224-225): ``bos_id`` 1, then
    one id per UTF-8 byte (byte + 2). No end token."""

    bos_id = 1
    eos_id = None

    def encode(self, text: str) -> list:
        return [self.bos_id] + [b + 2 for b in text.encode("utf-8")]

    def decode(self, ids) -> str:
        return bytes(i - 2 for i in ids if 2 <= i < 258).decode("utf-8", errors="replace")


def sample(last: torch.Tensor, temperature: float, top_k: int, top_p: float) -> int:
    """Next token from logits (V,): argmax when ``temperature <= 0``;
    otherwise the logits are divided by the temperature, restricted to the
    ``top_k`` largest (k > 0) and then to the most probable tokens up to and
    including the first one at which their cumulative probability exceeds
    ``top_p`` (0 < p < 1), and one token is drawn from the softmax of what
    remains with ``torch.multinomial`` (torch's generator, so
    ``torch.manual_seed`` fixes the draw)."""
    if temperature <= 0:
        return int(last.argmax())
    z = last.to(torch.float32) / temperature
    if top_k > 0 and top_k < z.numel():
        kth = torch.topk(z, top_k).values[-1]
        z = torch.where(z < kth, torch.full_like(z, float("-inf")), z)
    if 0.0 < top_p < 1.0:
        zs, order = torch.sort(z, descending=True)
        cum = torch.softmax(zs, dim=-1).cumsum(-1)
        drop = torch.zeros_like(cum, dtype=torch.bool)
        drop[1:] = cum[:-1] > top_p            # the mass before the token already exceeds top_p
        keep = torch.full_like(z, float("-inf"))
        keep[order] = torch.where(drop, torch.full_like(zs, float("-inf")), zs)
        z = keep
    return int(torch.multinomial(torch.softmax(z, dim=-1), 1))


@torch.no_grad()
def decode_stream(runtime, tk, prompt, max_new: int = 80, temperature: float = 0.8,
                  top_k: int = 40, top_p: float = 0.95, seed: int | None = None,
                  verbose: bool = False):
    """Yields each generated token's text piece (cli.py:57-106 with a runtime
    given). ``prompt`` is text (encoded by ``tk``) or a list of token ids.
    Afterwards ``decode_stream.stats`` holds the reference's statistics
    (backend "hip"), ``decode_stream.ids`` the prompt plus generated ids and
    ``decode_stream.text`` their decoding."""
    if seed is not None:
        torch.manual_seed(seed)
    ids = list(prompt) if isinstance(prompt, (list, tuple)) else (tk.encode(prompt) or [tk.bos_id])
    t0 = time.perf_counter()
    last = torch.tensor(runtime.prefill(ids))
    prefill_s = time.perf_counter() - t0
    out = list(ids)
    step_times = []
    for _ in range(max_new):
        nxt = sample(last, temperature, top_k, top_p)
        out.append(nxt)
        yield tk.decode([nxt])
        if tk.eos_id is not None and nxt == tk.eos_id:
            break
        t0 = time.perf_counter()
        last = torch.tensor(runtime.step(nxt))
        step_times.append(time.perf_counter() - t0)
    decode_stream.stats = {
        "prefill_tokens": len(ids),
        "prefill_ms": prefill_s * 1e3,
        "backend": "hip",
        "gen_tokens": len(step_times),
        "decode_ms_median": (sorted(step_times)[len(step_times) // 2] * 1e3 if step_times else 0.0),
        "decode_ms_per_token": (sum(step_times) / len(step_times) * 1e3 if step_times else 0.0),
    }
    decode_stream.ids = out
    decode_stream.text = tk.decode(out)


def _dims(args):
    if args.dims:
        v = [int(x) for x in args.dims.split(",")]
        if len(v) != 6:
            raise SystemExit("--dims takes vocab,dim,inner,rank,taps,layers")
        return v
    c = PRESETS[args.config]
    return [c.vocab_size, c.dim, c.inner, c.rank, c.taps, c.layers]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m sunnynet_amd.cli",
                                 description="SunnyNet decoding on the HIP backend")
    ap.add_argument("--backend", choices=["hip"], default="hip",
                    help="hip = whole-model step on the GPU (the reference's torch and c "
                         "backends stay in the reference CLI)")
    ap.add_argument("--blob", required=True, help="packed runtime blob (the reference's format)")
    ap.add_argument("--config", choices=sorted(PRESETS), default="small")
    ap.add_argument("--dims", default=None, help="vocab,dim,inner,rank,taps,layers (overrides --config)")
    ap.add_argument("--weights", choices=["fp32", "int4", "fp16"], default="fp32")
    ap.add_argument("--block", type=int, default=32, help="INT4 group size")
    ap.add_argument("--half", action="store_true", help="the reference's flag: --weights fp16")
    ap.add_argument("--prompt", default="", help="text, encoded with the byte fallback")
    ap.add_argument("--prompt-ids", default=None, help="comma-separated token ids")
    ap.add_argument("--max-new", type=int, default=80)
    ap.add_argument("--temperature", type=float, default=0.8)
    ap.add_argument("--top-k", type=int, default=40)
    ap.add_argument("--top-p", type=float, default=0.95)
    ap.add_argument("--seed", type=int, default=None)
    ap.add_argument("--threads", type=int, default=0, help="host threads for loading; 0 = recommended")
    ap.add_argument("--stats", action="store_true", help="print decode timing")
    ap.add_argument("--json", action="store_true", help="print the result as JSON")
    args = ap.parse_args(argv)

    vocab, dim, inner, rank, taps, layers = _dims(args)
    tk = ByteTokenizer()
    if args.prompt_ids:
        prompt = [int(x) for x in args.prompt_ids.split(",") if x.strip()]
    else:
        prompt = tk.encode(args.prompt)
    bad = [t for t in prompt if not 0 <= t < vocab]
    if bad:
        raise SystemExit(f"prompt ids outside the vocabulary of {vocab}: {bad[:5]}")
    set_threads(args.threads if args.threads > 0 else recommended_threads())
    runtime = HipModel(args.blob, vocab, dim, inner, rank, taps, layers, 8, 1,
                       weights="fp16" if args.half else args.weights, block=args.block)
    try:
        pieces = []
        for p in decode_stream(runtime, tk, prompt, args.max_new, args.temperature, args.top_k,
                               args.top_p, args.seed):
            pieces.append(p)
            if not args.json:
                sys.stdout.write(p)
                sys.stdout.flush()
    finally:
        runtime.close()
    st = decode_stream.stats
    if args.json:
        print(json.dumps({"prompt": prompt, "ids": decode_stream.ids, "text": "".join(pieces),
                          "stats": st}, ensure_ascii=False))
    else:
        print()
        if args.stats:
            print(f"[backend hip; prefill {st['prefill_tokens']} tok {st['prefill_ms']:.1f} ms; "
                  f"decode {st['gen_tokens']} tok {st['decode_ms_per_token']:.3f} ms/tok]")
    return 0


if __name__ == "__main__":
    sys.exit(main())
