"""Whole-model decode handle on the GPU, with the reference's ``SnModel``
interface (sunnynet/runtime/model.py:92-128).

``HipModel(path, vocab, dim, inner, rank, taps, layers, group=8, tied=1)``
loads the reference's packed fp32 runtime blob; ``reset()``, ``step(token)``
and ``prefill(tokens)`` behave like the reference's (one B=1 sequence, host
``list[float]`` logits, ``RuntimeError`` when loading fails).

Extensions: ``max_batch`` independent sequences, ``weights="int4"`` with a
group ``block`` (INT4 quantized at load in the reference's quant.c format),
``step_batch`` / ``decode_greedy`` on torch device tensors without host
round trips, and ``get_state`` / ``set_state`` in the torch ``SunnyState``
layout (s (B,L,D), hist (B,L,K-1,D), newest entry first).

``HipSunnyNet`` puts the torch backend's contract on a handle:
``init_state(B)``, ``forward(idx, state, return_state)`` with every
position's logits and ``forward_step(idx_t, state) -> (logits, SunnyState)``
(sunnynet/model.py:82-124), so a sequence can move between the torch path and
this one mid-stream.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from .. import _native

__all__ = ["HipModel", "SnModel", "HipSunnyNet", "SunnyState", "model_available",
           "set_threads", "get_threads", "recommended_threads"]

WEIGHT_FORMATS = {"fp32": 0, "int4": 1, "fp16": 3}


def model_available() -> bool:
    return _native.available()


def set_threads(n: int) -> int:
    """sunnynet/runtime/model.py:69-73: sets the host thread count (n <= 0
    keeps it) and returns the count in effect. The products run on the GPU;
    the count sizes host-side load preparation."""
    L = _native.lib()
    L.snhip_set_threads(int(n))
    return int(L.snhip_get_threads())


def get_threads() -> int:
    """sunnynet/runtime/model.py:76-77."""
    return int(_native.lib().snhip_get_threads())


def recommended_threads() -> int:
    """sunnynet/runtime/model.py:80-89: physical cores; half the logical
    count when the library cannot tell."""
    n = int(_native.lib().snhip_recommended_threads())
    if n <= 0:
        import os
        n = max(1, (os.cpu_count() or 2) // 2)
    return n


class HipModel:
    """Decode handle (B sequences) backed by libsnhip.so."""

    def __init__(self, path, vocab, dim, inner, rank, taps, layers, group=8, tied=1,
                 half=False, *, max_batch: int = 1, weights: str = "fp32", block: int = 32,
                 device=None):
        if half:
            # sn_load_h (runtime/model.py:100): the matrices rounded to fp16 at load
            weights = "fp16"
        self._lib = _native.lib()
        self.device = torch.device(device or "cuda:0")
        self.vocab, self.dim, self.layers, self.taps = vocab, dim, layers, taps
        self.inner, self.rank = inner, rank
        self.kh = max(0, taps - 1)
        self.max_batch = int(max_batch)
        with torch.cuda.device(self.device):
            self._h = self._lib.snhip_load_ex(str(path).encode(), vocab, dim, inner, rank, taps,
                                              layers, group, int(tied), self.max_batch,
                                              WEIGHT_FORMATS[weights], int(block))
        if not self._h:
            raise RuntimeError(f"snhip_load failed: {path}: {_native.last_error()}")
        if not self._lib.snhip_ready(self._h):
            raise RuntimeError("snhip_load returned a handle that is not ready")
        self._logits = np.empty(vocab, np.float32)
        self._bind_stream()
        _native.track(self)

    def _bind_stream(self):
        _native.check(self._lib.snhip_set_stream(self._h, _native.stream_handle(self.device)),
                      "snhip_set_stream")

    # ---------------------------------------------- reference-shaped surface
    def reset(self):
        self._bind_stream()
        self._lib.snhip_reset(self._h)

    def step(self, token: int) -> list:
        """One step of sequence 0 (sn_step); raises on an invalid token or a
        device failure, which the reference's void call cannot report."""
        t = np.array([int(token)], np.int32)
        self._bind_stream()
        _native.check(self._lib.snhip_step_batch(self._h, t.ctypes.data, 1,
                                                 self._logits.ctypes.data), "snhip_step")
        return self._logits.tolist()

    def prefill(self, tokens) -> list:
        toks = np.ascontiguousarray(np.asarray(list(tokens), np.int32))
        self._bind_stream()
        _native.check(self._lib.snhip_prefill_host(self._h, toks.ctypes.data, toks.size,
                                                   self._logits.ctypes.data), "snhip_prefill")
        return self._logits.tolist()

    # -------------------------------------------------------- device surface
    def step_batch(self, tokens: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """tokens (B,) int32 on the device -> logits (B, vocab) on the device."""
        B = int(tokens.shape[0])
        tokens = tokens.to(device=self.device, dtype=torch.int32).contiguous()
        if out is None:
            out = torch.empty(B, self.vocab, device=self.device, dtype=torch.float32)
        self._bind_stream()
        _native.check(self._lib.snhip_step_batch_dev(self._h, tokens.data_ptr(), B, out.data_ptr()),
                      "snhip_step_batch_dev")
        return out

    def step_batch_host(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(np.asarray(tokens, np.int32))
        out = np.empty((t.size, self.vocab), np.float32)
        self._bind_stream()
        _native.check(self._lib.snhip_step_batch(self._h, t.ctypes.data, t.size, out.ctypes.data),
                      "snhip_step_batch")
        return out

    def prefill_batch(self, tokens: torch.Tensor, logits: bool = True):
        """Chunked prefill of tokens (B, T) (sequences [0, B)) from the current
        state; returns the last token's logits (B, vocab) on the device."""
        B, T = (int(x) for x in tokens.shape)
        tokens = tokens.to(device=self.device, dtype=torch.int32).contiguous()
        out = torch.empty(B, self.vocab, device=self.device) if logits else None
        self._bind_stream()
        _native.check(self._lib.snhip_prefill_batch_dev(self._h, tokens.data_ptr(), B, T,
                                                        out.data_ptr() if logits else None),
                      "snhip_prefill_batch_dev")
        return out

    def prefill_all(self, tokens: torch.Tensor) -> torch.Tensor:
        """Chunked prefill of tokens (B, T) from the current state, returning
        the logits of every position, (B, T, vocab) on the device (the
        reference's ``SunnyNet.forward``, sunnynet/model.py:89-111); the state
        after the last token stays in the handle."""
        B, T = (int(x) for x in tokens.shape)
        tokens = tokens.to(device=self.device, dtype=torch.int32).contiguous()
        out = torch.empty(B, T, self.vocab, device=self.device)
        self._bind_stream()
        _native.check(self._lib.snhip_prefill_all_dev(self._h, tokens.data_ptr(), B, T,
                                                      out.data_ptr()), "snhip_prefill_all_dev")
        return out

    def dbg_layer(self, token: int, layer: int) -> dict:
        """sn_dbg_layer (sunnynet/runtime/sunnynet.c:336-345): steps sequence 0
        from ``token``'s embedding through layers 0..layer (their state
        advances, as in the reference) and returns that layer's
        intermediates by name (host float32 arrays)."""
        D, I, R = self.dim, self.inner, self.rank
        buf = np.empty(7 * D + R + 2 * I, np.float32)
        self._bind_stream()
        _native.check(self._lib.snhip_dbg_layer(self._h, int(token), int(layer), buf.ctypes.data),
                      "snhip_dbg_layer")
        names = (("raw", D), ("at", D), ("v", R), ("gate", D), ("u", D), ("s", D), ("zn", I),
                 ("yn", I), ("sfb", D), ("out", D))
        out, o = {}, 0
        for n, k in names:
            out[n] = buf[o:o + k].copy()
            o += k
        return out

    def decode_greedy(self, tokens: torch.Tensor, n_steps: int, logits: torch.Tensor | None = None):
        """Greedy decoding on the device; returns (n_steps, B) int32 tokens."""
        B = int(tokens.shape[0])
        tokens = tokens.to(device=self.device, dtype=torch.int32).contiguous()
        out = torch.empty(n_steps, B, device=self.device, dtype=torch.int32)
        self._bind_stream()
        _native.check(self._lib.snhip_decode_greedy_dev(
            self._h, tokens.data_ptr(), B, int(n_steps), out.data_ptr(),
            logits.data_ptr() if logits is not None else None), "snhip_decode_greedy_dev")
        return out

    @property
    def batch_grid(self) -> int:
        """Workgroups of the persistent batched step (0: per-kernel steps)."""
        return int(self._lib.snhip_batch_grid(self._h))

    @property
    def persistent_grid(self) -> int:
        """Workgroups of the persistent B=1 decode kernel (0: per-kernel steps)."""
        return int(self._lib.snhip_persistent_grid(self._h))

    def persistent_grid_for(self, B: int) -> int:
        """Workgroups of the persistent decode for steps of B sequences, each on
        its own slice of the grid (0: B takes the batched or per-kernel step)."""
        return int(self._lib.snhip_persistent_grid_batch(self._h, B))

    def get_state(self, B: int | None = None):
        B = self.max_batch if B is None else B
        s = torch.empty(B, self.layers, self.dim, device=self.device)
        h = torch.empty(B, self.layers, self.kh, self.dim, device=self.device)
        self._bind_stream()
        _native.check(self._lib.snhip_get_state_dev(self._h, s.data_ptr(), h.data_ptr(), B),
                      "snhip_get_state_dev")
        return s, h

    def set_state(self, s: torch.Tensor, hist: torch.Tensor):
        B = int(s.shape[0])
        s = s.to(device=self.device, dtype=torch.float32).contiguous()
        hist = hist.to(device=self.device, dtype=torch.float32).contiguous()
        if s.shape != (B, self.layers, self.dim) or hist.shape != (B, self.layers, self.kh, self.dim):
            raise ValueError("state must be s (B,L,D) and hist (B,L,K-1,D)")
        self._bind_stream()
        _native.check(self._lib.snhip_set_state_dev(self._h, s.data_ptr(), hist.data_ptr(), B),
                      "snhip_set_state_dev")

    def close(self):
        if getattr(self, "_h", None):
            self._lib.snhip_free(self._h)
            self._h = None

    def __del__(self):
        # During interpreter teardown the HIP runtime may already be gone
        # (and this module's globals with it); the atexit hook has closed
        # every open handle before that point.
        try:
            if not _native.finalizing():
                self.close()
        except Exception:
            pass


# The reference's name, for drop-in use with the same constructor arguments.
SnModel = HipModel


@dataclass
class SunnyState:
    """The torch backend's recurrent state (sunnynet/layers.py:21-30): per
    layer rolling state ``s`` (B, L, D) and causal-conv history ``hist``
    (B, L, K-1, D), newest entry first."""

    s: torch.Tensor
    hist: torch.Tensor

    def to(self, device=None, dtype=None):
        return SunnyState(self.s.to(device=device, dtype=dtype),
                          self.hist.to(device=device, dtype=dtype))


class HipSunnyNet:
    """``SunnyNet``'s single-step surface over a ``HipModel``.

    ``forward_step(idx_t, state)`` (sunnynet/model.py:113-124) loads ``state``
    into sequences [0, B) of the handle, steps them on ``idx_t`` and returns
    the logits (B, V) with a new ``SunnyState`` (fresh tensors, fp32, on the
    handle's device), as the torch path returns new tensors. Any float dtype
    or device is accepted for ``state``; the handle computes in fp32.
    """

    def __init__(self, handle: HipModel):
        self.handle = handle

    @property
    def device(self):
        return self.handle.device

    def init_state(self, batch: int, device=None, dtype=torch.float32) -> SunnyState:
        """model.py:82-87: zero state for ``batch`` sequences."""
        h = self.handle
        dev = device if device is not None else h.device
        return SunnyState(torch.zeros(batch, h.layers, h.dim, device=dev, dtype=dtype),
                          torch.zeros(batch, h.layers, h.kh, h.dim, device=dev, dtype=dtype))

    @torch.no_grad()
    def forward(self, idx: torch.Tensor, state: SunnyState | None = None,
                return_state: bool = False):
        """model.py:89-111: idx (B, T) -> logits (B, T, V) for every position,
        and with ``return_state`` the state after the last token. As in the
        reference's ``forward``, the history of ``state`` and of the returned
        state is oldest entry first (layers.py:266; ``forward_step`` uses
        newest first). The history carried in follows stepping: for T below
        taps - 1 the older entries of ``state.hist`` stay in the window
        (the reference's ``forward`` restarts it from zeros there,
        layers.py:264-266); both agree from a zero state and for longer
        prompts."""
        h = self.handle
        B = int(idx.shape[0])
        if B > h.max_batch:
            raise ValueError(f"batch {B} exceeds the handle's max_batch {h.max_batch}")
        if state is None:
            state = self.init_state(B)
        elif state.s.shape[0] != B or state.hist.shape[0] != B:
            raise ValueError("state batch does not match idx")
        h.set_state(state.s, torch.flip(state.hist, dims=[-2]))
        logits = h.prefill_all(idx)
        if not return_state:
            return logits
        s, hist = h.get_state(B)
        return logits, SunnyState(s, torch.flip(hist, dims=[-2]).contiguous())

    @torch.no_grad()
    def forward_step(self, idx_t: torch.Tensor, state: SunnyState):
        h = self.handle
        B = int(idx_t.shape[0])
        if B > h.max_batch:
            raise ValueError(f"batch {B} exceeds the handle's max_batch {h.max_batch}")
        if state.s.shape[0] != B or state.hist.shape[0] != B:
            raise ValueError("state batch does not match idx_t")
        h.set_state(state.s, state.hist)
        logits = h.step_batch(idx_t.to(device=h.device, dtype=torch.int32))
        s, hist = h.get_state(B)
        return logits, SunnyState(s, hist)
