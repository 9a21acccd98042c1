"""RWKV-7 decode handle on the GPU (include/snhip_rwkv7.h).

``HipRwkv7(path[, vocab])`` loads the reference's v3 runtime blob and offers
the reference handle's operations (sunnynet/runtime/rwkv7.h:16-28 and the
ctypes class ``SnRWKV7``, sunnynet/runtime/rwkv7_c.py:65-104): ``reset()``,
``step(token) -> list[float]``, ``step_raw(token)``, ``logits()`` and
``prefill(tokens) -> list[float]`` (host logits, one B=1 sequence); a
``vocab`` given positionally must equal the blob's. Extensions: ``max_batch`` sequences, weight format
(``"stored"`` as in the blob, ``"fp32"``, ``"int4"`` with a group ``block``),
``step_batch`` / ``decode_greedy`` on device tensors, and ``get_state`` /
``set_state`` (S (B, L, H, 64, 64), shift (B, L, 2, D)).
"""
from __future__ import annotations

import ctypes
import struct

import numpy as np
import torch

from .. import _native

__all__ = ["HipRwkv7"]

FORMATS = {"fp32": 0, "int4": 1, "stored": 2}


class HipRwkv7:
    def __init__(self, path, vocab: int | None = None, *, max_batch: int = 1,
                 weights: str = "stored", block: int = 32, device=None):
        self._lib = _native.lib()
        self.device = torch.device(device or "cuda:0")
        with open(path, "rb") as f:
            h = struct.unpack("<10i", f.read(40))
        self.layers, self.dim, self.head_size, self.n_head = h[2], h[3], h[4], h[5]
        self.max_batch = int(max_batch)
        with torch.cuda.device(self.device):
            self._h = self._lib.snhip_rk_load_ex(str(path).encode(), self.max_batch,
                                                 FORMATS[weights], int(block))
        if not self._h:
            raise RuntimeError(f"snhip_rk_load failed: {path}: {_native.last_error()}")
        if not self._lib.snhip_rk_ready(self._h):
            raise RuntimeError("snhip_rk_load returned a handle that is not ready")
        self.vocab = int(self._lib.snhip_rk_vocab(self._h))
        if vocab is not None and int(vocab) != self.vocab:
            self.close()
            raise ValueError(f"vocab {vocab} does not match the blob's {self.vocab}")
        self._logits = np.empty(self.vocab, np.float32)
        self._bind_stream()
        _native.track(self)

    @property
    def persist_grid(self) -> int:
        """Workgroups of the one-launch-per-step path for single-sequence steps
        (0 when off)."""
        return int(self._lib.snhip_rk_persist_grid(self._h))

    @property
    def persist_exact(self) -> bool:
        """Whether the one-launch step is the exact-order kernel (bit-identical
        to the reference's sn_rk_step)."""
        return bool(self._lib.snhip_rk_persist_exact(self._h))

    def persist_grid_for(self, B: int) -> int:
        """Workgroups of the persistent launch for steps of B sequences, each
        on its own slice of the grid (0: B takes the per-kernel path)."""
        return int(self._lib.snhip_rk_persist_grid_batch(self._h, B))

    def _bind_stream(self):
        _native.check(self._lib.snhip_rk_set_stream(self._h, _native.stream_handle(self.device)),
                      "snhip_rk_set_stream")

    # ---------------------------------------------- reference-shaped surface
    def reset(self):
        self._bind_stream()
        self._lib.snhip_rk_reset(self._h)

    def step(self, token: int) -> list:
        self.step_raw(token)
        return self._logits.tolist()

    def step_raw(self, token: int) -> None:
        """Advance the state; the logits stay in the handle's buffer. Raises
        on an invalid token or a device failure (a timed-out step leaves the
        handle refusing steps until reset() or set_state())."""
        self._bind_stream()
        _native.check(self._lib.snhip_abi_rwkv7_step(self._h, int(token), self._logits.ctypes.data),
                      "snhip_rk_step")

    def logits(self) -> list:
        return self._logits.tolist()

    def dbg(self, token: int, layer: int) -> np.ndarray:
        """rwkv7_c.py:98-101 / sn_rk_dbg: steps sequence 0 through layers
        0..layer and returns that layer's intermediates (9, dim): xn, r, k, v,
        a, g, ww, y and the layer's output x."""
        out = np.empty(9 * self.dim, np.float32)
        self._bind_stream()
        _native.check(self._lib.snhip_rk_dbg(self._h, int(token), int(layer), out.ctypes.data),
                      "snhip_rk_dbg")
        return out.reshape(9, self.dim)

    def prefill(self, tokens) -> list:
        toks = np.ascontiguousarray(np.asarray([int(t) for t in tokens], np.int32))
        self._bind_stream()
        _native.check(self._lib.snhip_abi_rwkv7_prefill(self._h, toks.ctypes.data, toks.size,
                                                        self._logits.ctypes.data),
                      "snhip_rk_prefill")
        return self._logits.tolist()

    # -------------------------------------------------------- device surface
    def step_batch(self, tokens: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        B = int(tokens.shape[0])
        tokens = tokens.to(device=self.device, dtype=torch.int32).contiguous()
        if out is None:
            out = torch.empty(B, self.vocab, device=self.device, dtype=torch.float32)
        self._bind_stream()
        _native.check(self._lib.snhip_rk_step_batch_dev(self._h, tokens.data_ptr(), B,
                                                        out.data_ptr()), "snhip_rk_step_batch_dev")
        return out

    def decode_greedy(self, tokens: torch.Tensor, n_steps: int, logits: torch.Tensor | None = None):
        B = int(tokens.shape[0])
        tokens = tokens.to(device=self.device, dtype=torch.int32).contiguous()
        out = torch.empty(n_steps, B, device=self.device, dtype=torch.int32)
        self._bind_stream()
        _native.check(self._lib.snhip_rk_decode_greedy_dev(
            self._h, tokens.data_ptr(), B, int(n_steps), out.data_ptr(),
            logits.data_ptr() if logits is not None else None), "snhip_rk_decode_greedy_dev")
        return out

    def get_state(self, B: int | None = None):
        B = self.max_batch if B is None else B
        S = torch.empty(B, self.layers, self.n_head, self.head_size, self.head_size,
                        device=self.device)
        sh = torch.empty(B, self.layers, 2, self.dim, device=self.device)
        self._bind_stream()
        _native.check(self._lib.snhip_rk_get_state_dev(self._h, S.data_ptr(), sh.data_ptr(), B),
                      "snhip_rk_get_state_dev")
        return S, sh

    def set_state(self, S: torch.Tensor, shift: torch.Tensor):
        B = int(S.shape[0])
        S = S.to(device=self.device, dtype=torch.float32).contiguous()
        shift = shift.to(device=self.device, dtype=torch.float32).contiguous()
        if S.shape != (B, self.layers, self.n_head, self.head_size, self.head_size) or \
                shift.shape != (B, self.layers, 2, self.dim):
            raise ValueError("state must be S (B,L,H,64,64) and shift (B,L,2,D)")
        self._bind_stream()
        _native.check(self._lib.snhip_rk_set_state_dev(self._h, S.data_ptr(), shift.data_ptr(), B),
                      "snhip_rk_set_state_dev")

    def close(self):
        if getattr(self, "_h", None):
            self._lib.snhip_rk_free(self._h)
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
