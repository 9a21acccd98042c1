"""The allocation-free core backward (snhip_abi_core_bwd_dev_noalloc) against
the allocating one (snhip_abi_core_bwd_dev), through the C-ABI: identical
dq, ddelta (accumulated into, as the reference's `ddelta[d] += ...`) and ds0,
bit for bit, on two calls in a row, the second smaller than the first (the
scratch keeps the first call's partials, and every element the second call
reads is one it wrote). Both the ring kernels (D % 128 == 0, T a multiple of
the tile) and the one-lane-per-channel kernels run. A call whose (B, D)
partials exceed the scratch is refused on the host with an error text.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from sunnynet_amd import _native, runtime

pytestmark = pytest.mark.gpu


def _inputs(B, T, D, seed):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((B, T, 2 * D)) * 0.6).astype(np.float32)
    delta = (0.01 + 0.4 * rng.random(D)).astype(np.float32)
    s0 = (rng.standard_normal((B, D)) * 0.1).astype(np.float32)
    dstate = rng.standard_normal((B, T, D)).astype(np.float32)
    du_in = rng.standard_normal((B, T, D)).astype(np.float32)
    return [torch.from_numpy(x).cuda() for x in (q, delta, s0, dstate, du_in)]


def _bwd(fn, q, delta, s0, fwd, dstate, du_in, B, T, D):
    dq = torch.empty_like(q)
    ddelta = torch.full((D,), 0.25, device=q.device)
    ds0 = torch.empty_like(s0)
    ptrs = [t.data_ptr() for t in (q, delta, s0, *fwd, dstate, du_in, dq, ddelta, ds0)]
    rc = fn(*ptrs, B, T, D, _native.stream_handle(q.device))
    return rc, dq, ddelta, ds0


@pytest.mark.parametrize("shapes", [[(8, 256, 512), (3, 128, 256)], [(4, 100, 200), (2, 37, 40)]])
def test_noalloc_core_bwd_equals_allocating_call(gpu, shapes):
    L = _native.lib()
    for i, (B, T, D) in enumerate(shapes):
        print(f"core bwd without allocation, call {i}: B={B} T={T} D={D}", flush=True)
        q, delta, s0, dstate, du_in = _inputs(B, T, D, 100 * i + D)
        fwd = runtime.core_fwd(q, delta, s0)
        ra, *a = _bwd(L.snhip_abi_core_bwd_dev, q, delta, s0, fwd, dstate, du_in, B, T, D)
        rb, *b = _bwd(L.snhip_abi_core_bwd_dev_noalloc, q, delta, s0, fwd, dstate, du_in, B, T, D)
        _native.check(ra, "snhip_abi_core_bwd_dev")
        _native.check(rb, "snhip_abi_core_bwd_dev_noalloc")
        torch.cuda.synchronize()
        for name, x, y in zip(("dq", "ddelta", "ds0"), a, b):
            assert torch.equal(x, y), name


def test_noalloc_core_bwd_refuses_partials_beyond_the_scratch(gpu):
    L = _native.lib()
    B, T, D = 1025, 1, 1024          # B * D = 1049600 > 2^20
    q, delta, s0, dstate, du_in = _inputs(1, 1, 8, 0)   # never touched: refused before any launch
    ptrs = [t.data_ptr() for t in (q, delta, s0, q, q, q, dstate, du_in, q, delta, s0)]
    rc = L.snhip_abi_core_bwd_dev_noalloc(*ptrs, B, T, D, _native.stream_handle(q.device))
    assert rc == -1
    assert "exceeds the scratch" in _native.last_error()
