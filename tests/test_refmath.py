"""The step's expf / tanhf (sunnynet_amd/csrc/refmath.h) against the host C
library's, bit for bit (the reference runtime's transcendentals are libm's).

CPU: the library's host build of the restatement over every 61st float
pattern of the whole 32-bit range (about 70 million inputs, every exponent)
and the special values. GPU: the device build over a sample of the same.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from sunnynet_amd import _native

SPECIAL = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 88.72, 88.73, -103.9,
                    -104.0, 9.0, -9.0, 22.0, -22.0, 2.0 ** -26, 0.3465, 0.3466, 1.0397, 1.0398],
                   np.float32)


def _patterns(step: int, offset: int = 0, chunk: int = 1 << 24):
    total = 1 << 32
    start = offset
    while start < total:
        n = min(chunk, (total - start + step - 1) // step)
        idx = start + step * np.arange(n, dtype=np.uint64)
        yield idx.astype(np.uint32).view(np.float32)
        start += step * n


def _same(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_host_restatement_matches_libm():
    L = _native.lib()
    for x in [SPECIAL] + list(_patterns(61, 7)):
        e, t = np.empty_like(x), np.empty_like(x)
        _native.check(L.snhip_refmath_host(x.ctypes.data, e.ctypes.data, t.ctypes.data, x.size),
                      "refmath_host")
        re, rt = oracle.libm(x)
        assert _same(e, re), x[(e.view(np.uint32) != re.view(np.uint32))][:5]
        assert _same(t, rt), x[(t.view(np.uint32) != rt.view(np.uint32))][:5]


@pytest.mark.gpu
def test_device_restatement_matches_libm(gpu):
    import torch
    L = _native.lib()
    xs = [SPECIAL] + list(_patterns(257, 3))
    for x in xs:
        dx = torch.from_numpy(x).to(gpu)
        e, t = torch.empty_like(dx), torch.empty_like(dx)
        _native.check(L.snhip_refmath_dev(dx.data_ptr(), e.data_ptr(), t.data_ptr(), x.size,
                                          _native.stream_handle(gpu)), "refmath_dev")
        re, rt = oracle.libm(x)
        assert _same(e.cpu().numpy(), re)
        assert _same(t.cpu().numpy(), rt)
