"""First-order recurrence on the GPU, with the reference runtime's interface.

Mirrors ``sunnynet/runtime/__init__.py:147-178``: ``scan(a, b, s0, gated)``
returns ``(out, send)`` and ``step(a, b, s, gated)`` updates ``s`` in place,
with ``s_t = a_t * s_{t-1} + b_t`` (``FMA``) or ``b_t = (1 - a_t) * u_t``
(``GATED``). Results are bit-identical to the reference C runtime.

Device (``cuda``) tensors run on torch's current stream without a host
synchronization. CPU tensors go through the host-pointer ABI (the library
copies to the GPU and back), which is the reference's calling convention.
"""
from __future__ import annotations

import torch

from .. import _native

__all__ = ["FMA", "GATED", "load_runtime", "runtime_available", "scan", "step"]

FMA = 0
GATED = 1


def runtime_available() -> bool:
    return _native.available()


def load_runtime():
    return _native.lib()


def _check_f32(*ts):
    for t in ts:
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("expected contiguous float32 tensors")


def scan(a: torch.Tensor, b: torch.Tensor, s0: torch.Tensor, gated: bool = False):
    """a, b: (B,T,N); s0: (B,N) -> (out (B,T,N), send (B,N))."""
    _check_f32(a, b, s0)
    B, T, N = a.shape
    if b.shape != a.shape or s0.shape != (B, N):
        raise ValueError("shape mismatch: a, b (B,T,N); s0 (B,N)")
    if len({a.device, b.device, s0.device}) != 1:
        raise ValueError("a, b and s0 must live on one device")
    L = _native.lib()
    out = torch.empty_like(a)
    send = torch.empty_like(s0)
    g = GATED if gated else FMA
    if a.is_cuda:
        rc = L.snhip_abi_recur_scan_dev(a.data_ptr(), b.data_ptr(), s0.data_ptr(),
                                        out.data_ptr(), send.data_ptr(), B, T, N, g,
                                        _native.stream_handle(a.device))
    else:
        rc = L.snhip_abi_recur_scan(a.data_ptr(), b.data_ptr(), s0.data_ptr(),
                                    out.data_ptr(), send.data_ptr(), B, T, N, g)
    _native.check(rc, "snhip_abi_recur_scan")
    return out, send


def step(a: torch.Tensor, b: torch.Tensor, s: torch.Tensor, gated: bool = False):
    """a, b, s: (B,N); s updated in place and returned."""
    _check_f32(a, b, s)
    B, N = a.shape
    if b.shape != a.shape or s.shape != a.shape:
        raise ValueError("shape mismatch: a, b, s (B,N)")
    L = _native.lib()
    g = GATED if gated else FMA
    if a.is_cuda:
        rc = L.snhip_abi_recur_step_dev(a.data_ptr(), b.data_ptr(), s.data_ptr(), B, N, g,
                                        _native.stream_handle(a.device))
    else:
        rc = L.snhip_abi_recur_step(a.data_ptr(), b.data_ptr(), s.data_ptr(), B, N, g)
    _native.check(rc, "snhip_abi_recur_step")
    return s
