"""C-ABI contract checks that need no GPU (mirrors the reference's
tests/test_abi.py:28-95): the library loads, exports every declared symbol,
reports version / caps / backend, and rejects bad arguments before touching
the device."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from sunnynet_amd import _native
from sunnynet_amd.runtime import abi


def test_library_exports_every_declared_symbol():
    L = _native.lib()
    declared = _native.declared_symbols()
    assert len(declared) >= 14
    missing = [n for n in declared if not hasattr(L, n)]
    assert not missing, missing


def test_version_matches_header():
    assert abi.version() == abi.ABI_VERSION == 0x10100
    assert abi.version_string() == "1.1.0"
    assert abi.backend_string() == "hip"


def test_caps_include_core():
    names = abi.cap_names()
    for want in ("recur_scan", "recur_step", "rwkv7", "threads", "device_ptr", "sunny_model",
                 "int4", "batch", "prefill"):
        assert want in names
    assert "quant_i8" not in names


def test_check_compat_and_incompat():
    assert abi.check(abi.ABI_MAJOR) == abi.STATUS_OK
    assert abi.check(abi.ABI_MAJOR + 1) == -5


def test_status_messages_are_defined():
    for code in (0, -1, -2, -3, -4, -5, -6):
        assert abi.status_str(code)


def test_invalid_args_return_einval():
    """tests/test_abi.py:86-95: NULL pointers, non-positive dims, zero threads."""
    L = _native.lib()
    a = np.zeros((2, 8), np.float32)
    pa = a.ctypes.data
    assert L.snhip_abi_recur_step(None, pa, pa, 2, 8, 0) == -1
    assert L.snhip_abi_recur_step(pa, pa, pa, 2, -8, 0) == -1
    assert L.snhip_abi_recur_scan(pa, pa, pa, pa, pa, 2, 0, 8, 1) == -1
    assert L.snhip_abi_recur_scan(pa, None, pa, pa, pa, 2, 1, 8, 1) == -1
    assert L.snhip_abi_recur_scan_dev(pa, pa, pa, pa, pa, 0, 1, 8, 1, None) == -1
    assert L.snhip_abi_recur_step_dev(pa, pa, None, 2, 8, 1, None) == -1
    assert L.snhip_abi_quant_i4_dev(pa, pa, pa, 2, 8, 3, None) == -1      # odd block
    assert L.snhip_abi_quant_i4_dev(pa, pa, pa, 2, 48, 32, None) == -1    # N % block
    assert L.snhip_abi_dequant_i4_dev(None, pa, pa, 2, 64, 32, None) == -1
    assert L.snhip_abi_set_threads(0) == -1
    assert L.snhip_abi_set_threads(4) == 0 and L.snhip_abi_get_threads() == 4


def test_string_buffer_protocol():
    L = _native.lib()
    n = L.snhip_abi_backend_string(None, 0)
    assert n == 4
    small = ctypes.create_string_buffer(2)
    assert L.snhip_abi_backend_string(small, 2) == 4 and small.value == b""


def test_model_load_rejects_bad_blobs(tmp_path):
    """sn_load semantics (sunnynet.c:358-413): NULL on missing file, wrong
    magic, dimension mismatch or truncation — all detected before any device
    work, so this runs without a GPU."""
    from sunnynet_amd.blob import pack_sunny_blob
    from sunnynet_amd.config import TINY
    from sunnynet_amd.weights import init_sunnynet
    L = _native.lib()
    c = TINY
    buf = pack_sunny_blob(init_sunnynet(c, 0))
    good = tmp_path / "good.bin"
    good.write_bytes(buf)
    args = (c.vocab_size, c.dim, c.inner, c.rank, c.taps, c.layers, 8, 1)
    assert not L.snhip_load(str(tmp_path / "missing.bin").encode(), *args)
    bad = tmp_path / "magic.bin"
    bad.write_bytes(b"\0\0\0\0" + buf[4:])
    assert not L.snhip_load(str(bad).encode(), *args)
    assert not L.snhip_load(str(good).encode(), c.vocab_size, c.dim + 8, *args[2:])
    trunc = tmp_path / "trunc.bin"
    trunc.write_bytes(buf[:-4])
    assert not L.snhip_load(str(trunc).encode(), *args)
    assert "truncated" in _native.last_error()
    # group other than 8 is refused up front
    assert not L.snhip_load(str(good).encode(), *args[:6], 4, 1)
    # NULL handles are tolerated by the void entry points
    L.snhip_free(None)
    L.snhip_reset(None)
    assert L.snhip_vocab(None) == 0 and L.snhip_ready(None) == 0
    assert L.snhip_step_batch(None, None, 1, None) == -1


def test_thread_controls_mirror_sunnynet_h():
    """sunnynet.h:42-47 / runtime/model.py:69-89: set_threads(n <= 0) keeps the
    setting, a positive n takes effect and is what get_threads reports (the
    same setting as the stable ABI's); recommended_threads is the number of
    distinct (physical id, core id) pairs in /proc/cpuinfo."""
    from sunnynet_amd.runtime import model as rt
    L = _native.lib()
    before = rt.get_threads()
    assert before >= 1
    assert rt.set_threads(0) == before
    assert rt.set_threads(-3) == before
    assert rt.set_threads(3) == 3 and L.snhip_abi_get_threads() == 3
    assert L.snhip_abi_set_threads(5) == 0 and rt.get_threads() == 5
    rt.set_threads(before)
    pairs, phys, core = set(), -1, -1
    with open("/proc/cpuinfo") as f:
        for line in list(f) + ["\n"]:
            k, _, v = line.partition(":")
            if k.strip() == "physical id":
                phys = int(v)
            elif k.strip() == "core id":
                core = int(v)
            elif line == "\n":
                if core >= 0:
                    pairs.add((phys, core))
                phys = core = -1
    want = len(pairs) if pairs else __import__("os").cpu_count()
    assert L.snhip_recommended_threads() == want
    assert rt.recommended_threads() == want
