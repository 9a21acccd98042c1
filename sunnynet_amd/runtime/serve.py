"""Serving on the HIP backend: the reference's engine protocol and continuous
batching over the batched decode step.

``HipEngine`` implements the reference's ``Engine`` protocol
(``sunnynet/serve.py:60-78``: ``encode``, ``decode``, ``init_state``,
``step(token, state) -> (logits, state)``) on a one-sequence handle, so the
reference's ``generate_stream`` (``serve.py:252-``) and HTTP server can drive
it unchanged. Each request's state is a pair of device tensors; the handle
holds one of them at a time and swaps states in and out only when another
request steps, so a single stream costs one step per token.

``HipRwkvEngine`` does the same for RWKV-7 (the reference's C-runtime RWKV-7
engine, ``serve.py:177-207``).

``BatchScheduler`` serves many requests on one ``max_batch`` handle. Every
iteration each active request consumes one input token (the next prompt token
while it is prefilling, as ``sn_prefill`` steps through a prompt,
``sunnynet.c:347-349``, else its last generated token), all active requests
step together as sequences ``[0, n)`` of the batched step, and the logits of
requests past their prompt give their next token (greedy, or the reference's
``sample_logits`` sampling, ``serve.py:29-56``). Requests join in free slots
(their state zeroed) and leave when they reach ``max_tokens`` or an end token;
the last active request then moves into the freed slot, so the active
sequences stay ``[0, n)``. Requests are independent: each one's tokens are the
ones it would produce alone.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .model import HipModel

__all__ = ["HipEngine", "HipState", "HipRwkvEngine", "HipRwkvState", "BatchScheduler", "Request",
           "sample_logits"]


def sample_logits(logits, temperature=1.0, top_p=1.0, top_k=0, rng=None) -> int:
    """Next token from logits (V,): argmax at temperature <= 0, else softmax
    sampling after top-k and top-p (nucleus) filtering (serve.py:29-56)."""
    if temperature is None or temperature <= 0:
        return int(np.argmax(logits))
    z = np.asarray(logits, dtype=np.float64) / float(temperature)
    if top_k and top_k < z.size:
        thr = np.partition(z, -int(top_k))[-int(top_k)]
        z = np.where(z < thr, -np.inf, z)
    if 0.0 < top_p < 1.0:
        order = np.argsort(-z)
        srt = z[order]
        p = np.exp(srt - srt.max())
        p /= p.sum()
        cut = np.cumsum(p) > top_p
        cut[1:] = cut[:-1].copy()
        cut[0] = False
        z = np.full_like(z, -np.inf)
        z[order] = np.where(cut, -np.inf, srt)
    z = z - z.max()
    p = np.exp(z)
    total = p.sum()
    if not np.isfinite(total) or total <= 0:
        return int(np.argmax(logits))
    rng = rng or np.random.default_rng()
    return int(rng.choice(z.size, p=p / total))


class HipState:
    """One request's recurrent state: s (1, L, D) and hist (1, L, K-1, D) on
    the device (the SunnyState layout, newest history first)."""

    def __init__(self, s: torch.Tensor, hist: torch.Tensor):
        self.s, self.hist = s, hist


class HipEngine:
    """The reference's Engine protocol on the HIP backend (one sequence per
    step; requests interleave through their states)."""

    name = "sunnynet-hip"

    def __init__(self, path, vocab, dim, inner, rank, taps, layers, *, tokenizer=None, eos=None,
                 weights="fp32", block=32, half=False, device=None):
        self.model = HipModel(path, vocab, dim, inner, rank, taps, layers, half=half, max_batch=1,
                              weights=weights, block=block, device=device)
        self.vocab = vocab
        self.eos = eos
        self.tk = tokenizer
        self._live = None              # the state the handle currently holds
        self._tok = torch.empty(1, dtype=torch.int32, device=self.model.device)

    def encode(self, text: str) -> list[int]:
        if self.tk is None:
            raise RuntimeError("no tokenizer given")
        return list(self.tk.encode(text))

    def decode(self, ids) -> str:
        if self.tk is None:
            raise RuntimeError("no tokenizer given")
        return self.tk.decode([int(i) for i in ids])

    def init_state(self) -> HipState:
        m = self.model
        return HipState(torch.zeros(1, m.layers, m.dim, device=m.device),
                        torch.zeros(1, m.layers, m.kh, m.dim, device=m.device))

    def _swap_in(self, state: HipState):
        if self._live is state:
            return
        m = self.model
        if self._live is not None:
            s, h = m.get_state(1)
            self._live.s.copy_(s)
            self._live.hist.copy_(h)
        m.set_state(state.s, state.hist)
        self._live = state

    def step(self, token: int, state: HipState):
        """-> (logits (V,) float32 numpy, state): the state object is updated
        (lazily, when another request next steps) and returned, as the
        reference's numpy backends do."""
        self._swap_in(state)
        self._tok.fill_(int(token))
        logits = self.model.step_batch(self._tok)
        return logits[0].float().cpu().numpy(), state

    def sync_state(self, state: HipState):
        """Write the handle's copy of `state` back into its tensors now."""
        if self._live is state:
            s, h = self.model.get_state(1)
            state.s.copy_(s)
            state.hist.copy_(h)


class HipRwkvState:
    """One request's RWKV-7 state on the device: S (1, L, H, 64, 64) and the
    two token-shift vectors (1, L, 2, D)."""

    def __init__(self, S: torch.Tensor, shift: torch.Tensor):
        self.S, self.shift = S, shift


class HipRwkvEngine:
    """The reference's RWKV-7 engine over its C runtime (sunnynet/serve.py:
    177-207, GGUFCEngine: one handle, step(token) then logits) on the HIP
    backend, with each request's state kept on the device and swapped in when
    another request steps, as HipEngine does."""

    name = "rwkv7-hip"

    def __init__(self, blob, vocab=None, *, tokenizer=None, eos=None, weights="stored", block=32,
                 device=None):
        from .rwkv7 import HipRwkv7
        self.model = HipRwkv7(blob, vocab, weights=weights, block=block, device=device)
        self.vocab = self.model.vocab
        self.eos = eos
        self.tk = tokenizer
        self._live = None
        self._tok = torch.empty(1, dtype=torch.int32, device=self.model.device)

    def encode(self, text: str) -> list[int]:
        if self.tk is None:
            raise RuntimeError("no tokenizer given")
        return list(self.tk.encode(text))

    def decode(self, ids) -> str:
        if self.tk is None:
            raise RuntimeError("no tokenizer given")
        return self.tk.decode([int(i) for i in ids])

    def init_state(self) -> HipRwkvState:
        m = self.model
        return HipRwkvState(torch.zeros(1, m.layers, m.n_head, m.head_size, m.head_size, device=m.device),
                            torch.zeros(1, m.layers, 2, m.dim, device=m.device))

    def _swap_in(self, state: HipRwkvState):
        if self._live is state:
            return
        if self._live is not None:
            S, sh = self.model.get_state(1)
            self._live.S.copy_(S)
            self._live.shift.copy_(sh)
        self.model.set_state(state.S, state.shift)
        self._live = state

    def step(self, token: int, state: HipRwkvState):
        """-> (logits (V,) float32 numpy, state), the state updated lazily."""
        self._swap_in(state)
        self._tok.fill_(int(token))
        logits = self.model.step_batch(self._tok)
        return logits[0].float().cpu().numpy(), state

    def sync_state(self, state: HipRwkvState):
        if self._live is state:
            S, sh = self.model.get_state(1)
            state.S.copy_(S)
            state.shift.copy_(sh)


@dataclass
class Request:
    prompt: list
    max_tokens: int
    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    eos: int | None = None
    seed: int | None = None
    output: list = field(default_factory=list)
    done: bool = False
    pos: int = 0                       # prompt tokens consumed
    rng: object = None

    def next_input(self) -> int:
        return int(self.prompt[self.pos]) if self.pos < len(self.prompt) else int(self.output[-1])


class BatchScheduler:
    """Continuous batching of requests over one handle's max_batch slots."""

    def __init__(self, model: HipModel):
        self.model = model
        self.active: list[Request] = []
        self.waiting: list[Request] = []
        self.finished: list[Request] = []
        self.steps = 0

    def submit(self, prompt, max_tokens: int, **kw) -> Request:
        if len(prompt) == 0:
            raise ValueError("a request needs at least one prompt token")
        r = Request(list(prompt), int(max_tokens), **kw)
        r.rng = np.random.default_rng(r.seed)
        if r.max_tokens <= 0:
            r.done = True
            self.finished.append(r)
        else:
            self.waiting.append(r)
        return r

    def _admit(self):
        n = len(self.active)
        free = self.model.max_batch - n
        if free <= 0 or not self.waiting:
            return
        take = self.waiting[:free]
        self.waiting = self.waiting[free:]
        s, h = self.model.get_state(n + len(take))
        s[n:].zero_()
        h[n:].zero_()
        self.model.set_state(s, h)
        self.active += take

    def _retire(self, gone: list[int]):
        """Drop finished slots; later slots move down so the active ones stay
        [0, n) (state rows copied with them)."""
        if not gone:
            return
        n = len(self.active)
        keep = [i for i in range(n) if i not in set(gone)]
        s, h = self.model.get_state(n)
        idx = torch.tensor(keep, dtype=torch.long, device=s.device)
        if keep:
            self.model.set_state(s.index_select(0, idx).contiguous(), h.index_select(0, idx).contiguous())
        for i in gone:
            self.active[i].done = True
            self.finished.append(self.active[i])
        self.active = [self.active[i] for i in keep]

    def step(self) -> int:
        """One iteration over every active request; returns how many stepped."""
        self._admit()
        n = len(self.active)
        if n == 0:
            return 0
        dev = self.model.device
        toks = torch.tensor([r.next_input() for r in self.active], dtype=torch.int32, device=dev)
        logits = self.model.step_batch(toks)
        self.steps += 1
        greedy = all(r.temperature is None or r.temperature <= 0 for r in self.active)
        picks = logits.argmax(1).cpu().numpy() if greedy else None
        host = None if greedy else logits.float().cpu().numpy()
        gone = []
        for i, r in enumerate(self.active):
            if r.pos < len(r.prompt):
                r.pos += 1
                if r.pos < len(r.prompt):
                    continue                   # still prefilling: logits unused
            t = int(picks[i]) if greedy else sample_logits(host[i], r.temperature, r.top_p, r.top_k, r.rng)
            r.output.append(t)
            if len(r.output) >= r.max_tokens or (r.eos is not None and t == r.eos):
                gone.append(i)
        self._retire(gone)
        return n

    def run(self) -> list[Request]:
        """Step until every submitted request is finished."""
        while self.active or self.waiting:
            self.step()
        return self.finished
