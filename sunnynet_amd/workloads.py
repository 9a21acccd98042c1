"""Seeded synthetic inputs for the measured workloads.

Gated scan (prefill) workload: B=16, D=2048 channels, T=4096, fp32.
``u, g ~ N(0,1)``; ``p = 1 - delta * sigmoid(g)`` with ``delta_i = 1/H_i`` and
``H = multiscale_decay(D, 2, 8192)`` (sunnynet/ops.py:50-59); ``s0 = 0``.
FMA form: ``a ~ U(0.9, 1)``, ``b ~ N(0, 1)``. numpy PCG64 seeds: 0 for u / a,
1 for g / b. ``p`` is computed here on the host and handed to both the GPU
kernel and the oracle.
"""
from __future__ import annotations

import math

import numpy as np
import torch

SCAN_B, SCAN_T, SCAN_D = 16, 4096, 2048


def multiscale_decay(n: int, h_min: float = 2.0, h_max: float = 8192.0) -> torch.Tensor:
    """ops.py:50-59 (fp32)."""
    if n == 1:
        h = torch.tensor([h_max], dtype=torch.float32)
    else:
        lo, hi = math.log(h_min), math.log(h_max)
        t = torch.arange(n, dtype=torch.float32) / (n - 1.0)
        h = torch.exp(lo + (hi - lo) * t)
    return 1.0 / h


def scan_inputs(B: int = SCAN_B, T: int = SCAN_T, D: int = SCAN_D, gated: bool = True,
                seed: int = 0):
    """(a, b, s0) numpy fp32 arrays: a = p, b = u for the gated form."""
    r0 = np.random.default_rng(seed)
    r1 = np.random.default_rng(seed + 1)
    if gated:
        u = r0.standard_normal((B, T, D), dtype=np.float32)
        g = r1.standard_normal((B, T, D), dtype=np.float32)
        delta = multiscale_decay(D).numpy()
        sig = np.float32(1.0) / (np.float32(1.0) + np.exp(-g))
        del g
        p = np.float32(1.0) - delta[None, None, :] * sig
        del sig
        a, b = p.astype(np.float32, copy=False), u
    else:
        a = r0.uniform(0.9, 1.0, size=(B, T, D)).astype(np.float32)
        b = r1.standard_normal((B, T, D), dtype=np.float32)
    s0 = np.zeros((B, D), np.float32)
    return a, b, s0


def scan_bytes(B: int, T: int, D: int) -> int:
    """Algorithmic HBM bytes of one scan: read a and b, write out (+ s0, send)."""
    return 3 * B * T * D * 4 + 2 * B * D * 4
