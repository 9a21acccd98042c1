"""ctypes view of the stable C ABI, mirroring ``sunnynet/runtime/abi.py``.

Same helpers (``load_abi``, ``version``, ``caps``, ``cap_names``, ``check``,
``version_string``, ``backend_string``, ``status_str``) over
``include/snhip_abi.h``; the backend string is ``"hip"``.
"""
from __future__ import annotations

import ctypes

from .. import _native

__all__ = ["abi_available", "load_abi", "ABI_VERSION", "CAPS", "STATUS_OK"]

ABI_MAJOR, ABI_MINOR, ABI_PATCH = 1, 1, 0
ABI_VERSION = (ABI_MAJOR << 16) | (ABI_MINOR << 8) | ABI_PATCH

# Bit positions as in include/snhip_abi.h; bits 0..4 keep the reference's names.
CAPS = {0: "recur_scan", 1: "recur_step", 2: "quant_i8", 3: "rwkv7", 4: "threads",
        8: "device_ptr", 9: "sunny_model", 10: "int4", 11: "batch", 12: "prefill"}
STATUS_OK = 0


def abi_available() -> bool:
    return _native.available()


def load_abi():
    return _native.lib()


def status_str(code: int) -> str:
    return _native.STATUS.get(int(code), f"unknown status {code}")


def version() -> int:
    return int(load_abi().snhip_abi_version())


def caps() -> int:
    return int(load_abi().snhip_abi_caps())


def cap_names() -> list:
    m = caps()
    return [n for bit, n in sorted(CAPS.items()) if m & (1 << bit)]


def check(caller_major: int = ABI_MAJOR) -> int:
    return int(load_abi().snhip_abi_check(int(caller_major)))


def _string(fn) -> str:
    n = fn(None, 0)
    buf = ctypes.create_string_buffer(n)
    fn(buf, n)
    return buf.value.decode()


def version_string() -> str:
    return _string(load_abi().snhip_abi_version_string)


def backend_string() -> str:
    return _string(load_abi().snhip_abi_backend_string)
