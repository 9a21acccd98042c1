"""Loader for the in-tree HIP library ``libsnhip.so``.

The library is the product's only compute path: nothing here falls back to a
CPU implementation. If the library is missing, every entry point raises.

``torch`` is imported first on purpose: torch ships its own
``libamdhip64.so.7``, and loading it before ``libsnhip.so`` makes the two
share one HIP runtime (same SONAME), so device pointers and streams from
torch are valid in the library.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libsnhip.so"
INCLUDE = PKG.parent / "include"

STATUS = {
    0: "OK",
    -1: "E_INVAL (NULL pointer or non-positive dimension)",
    -2: "E_NOMEM (allocation failed)",
    -3: "E_IO (open or read failed)",
    -4: "E_FORMAT (magic / version / size mismatch)",
    -5: "E_UNSUPPORTED (not supported by this build)",
    -6: "E_DEVICE (HIP runtime error)",
}


class SnHipError(RuntimeError):
    def __init__(self, what: str, code: int):
        detail = last_error() if code == -6 else ""
        super().__init__(f"{what}: {STATUS.get(code, code)}" + (f": {detail}" if detail else ""))
        self.code = code


_lib = None

V = ctypes.c_void_p
I32 = ctypes.c_int32
U32 = ctypes.c_uint32
CP = ctypes.c_char_p
INT = ctypes.c_int

# name -> (restype, argtypes)
_SIGS = {
    "snhip_abi_version": (I32, []),
    "snhip_abi_caps": (U32, []),
    "snhip_abi_check": (I32, [I32]),
    "snhip_abi_version_string": (I32, [V, I32]),
    "snhip_abi_backend_string": (I32, [V, I32]),
    "snhip_abi_last_error": (I32, [V, I32]),
    "snhip_abi_set_threads": (I32, [I32]),
    "snhip_abi_get_threads": (I32, []),
    "snhip_abi_recur_step": (I32, [V, V, V, I32, I32, I32]),
    "snhip_abi_recur_scan": (I32, [V, V, V, V, V, I32, I32, I32, I32]),
    "snhip_abi_recur_step_dev": (I32, [V, V, V, I32, I32, I32, V]),
    "snhip_abi_recur_scan_dev": (I32, [V, V, V, V, V, I32, I32, I32, I32, V]),
    "snhip_abi_scan_bwd_dev": (I32, [V, V, V, V, V, V, V, V, I32, I32, I32, V]),
    "snhip_abi_core_fwd_dev": (I32, [V, V, V, V, V, V, I32, I32, I32, V]),
    "snhip_abi_core_bwd_dev": (I32, [V, V, V, V, V, V, V, V, V, V, V, I32, I32, I32, V]),
    "snhip_abi_core_bwd_dev_noalloc": (I32, [V, V, V, V, V, V, V, V, V, V, V, I32, I32, I32, V]),
    "snhip_abi_quant_i4_dev": (I32, [V, V, V, I32, I32, I32, V]),
    "snhip_abi_dequant_i4_dev": (I32, [V, V, V, I32, I32, I32, V]),
    "snhip_abi_linear_dev": (I32, [V, V, V, I32, I32, I32, V]),
    "snhip_abi_hbm_probe_dev": (I32, [I32, V, V, V, ctypes.c_int64, I32, V]),
    # include/snhip.h
    "snhip_load": (V, [CP, INT, INT, INT, INT, INT, INT, INT, INT]),
    "snhip_load_ex": (V, [CP, INT, INT, INT, INT, INT, INT, INT, INT, I32, I32, I32]),
    "snhip_load_h": (V, [CP, INT, INT, INT, INT, INT, INT, INT, INT]),
    "snhip_free": (None, [V]),
    "snhip_reset": (None, [V]),
    "snhip_step": (None, [V, INT, V]),
    "snhip_prefill": (None, [V, V, INT, V]),
    "snhip_prefill_host": (I32, [V, V, I32, V]),
    "snhip_vocab": (INT, [V]),
    "snhip_ready": (INT, [V]),
    "snhip_set_threads": (None, [INT]),
    "snhip_get_threads": (INT, []),
    "snhip_recommended_threads": (INT, []),
    "snhip_set_stream": (I32, [V, V]),
    "snhip_max_batch": (I32, [V]),
    "snhip_persistent_grid": (I32, [V]),
    "snhip_persistent_grid_batch": (I32, [V, I32]),
    "snhip_batch_grid": (I32, [V]),
    "snhip_step_batch_dev": (I32, [V, V, I32, V]),
    "snhip_step_batch": (I32, [V, V, I32, V]),
    "snhip_decode_greedy_dev": (I32, [V, V, I32, I32, V, V]),
    "snhip_prefill_batch_dev": (I32, [V, V, I32, I32, V]),
    "snhip_prefill_all_dev": (I32, [V, V, I32, I32, V]),
    "snhip_dbg_layer": (I32, [V, I32, I32, V]),
    "snhip_get_state_dev": (I32, [V, V, V, I32]),
    "snhip_set_state_dev": (I32, [V, V, V, I32]),
    # include/snhip_rwkv7.h
    "snhip_rk_load": (V, [CP]),
    "snhip_rk_load_ex": (V, [CP, I32, I32, I32]),
    "snhip_rk_free": (None, [V]),
    "snhip_rk_reset": (None, [V]),
    "snhip_rk_step": (None, [V, INT, V]),
    "snhip_rk_prefill": (None, [V, V, INT, V]),
    "snhip_rk_vocab": (INT, [V]),
    "snhip_rk_dbg": (I32, [V, INT, INT, V]),
    "snhip_rk_ready": (INT, [V]),
    "snhip_rk_set_stream": (I32, [V, V]),
    "snhip_rk_max_batch": (I32, [V]),
    "snhip_rk_persist_grid": (I32, [V]),
    "snhip_rk_persist_grid_batch": (I32, [V, I32]),
    "snhip_rk_persist_exact": (I32, [V]),
    "snhip_rk_step_batch_dev": (I32, [V, V, I32, V]),
    "snhip_rk_decode_greedy_dev": (I32, [V, V, I32, I32, V, V]),
    "snhip_rk_get_state_dev": (I32, [V, V, V, I32]),
    "snhip_rk_set_state_dev": (I32, [V, V, V, I32]),
    "snhip_abi_rwkv7_load": (V, [CP]),
    "snhip_abi_rwkv7_step": (I32, [V, I32, V]),
    "snhip_abi_rwkv7_prefill": (I32, [V, V, I32, V]),
    "snhip_abi_rwkv7_reset": (I32, [V]),
    "snhip_abi_rwkv7_free": (None, [V]),
    "snhip_abi_rwkv7_vocab": (I32, [V]),
    "snhip_refmath_host": (I32, [V, V, V, I32]),
    "snhip_refmath_dev": (I32, [V, V, V, I32, V]),
}


def available() -> bool:
    return LIB_PATH.exists()


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built; run `python -m sunnynet_amd.build` "
                           "(the HIP backend has no CPU fallback)")
    L = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGS.items():
        if hasattr(L, name):
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
    _lib = L
    return L


def register(sigs: dict) -> None:
    """Declare more signatures (used by the model bindings)."""
    _SIGS.update(sigs)
    if _lib is not None:
        for name, (res, args) in sigs.items():
            if hasattr(_lib, name):
                f = getattr(_lib, name)
                f.restype = res
                f.argtypes = args


def last_error() -> str:
    L = lib()
    n = L.snhip_abi_last_error(None, 0)
    buf = ctypes.create_string_buffer(max(1, n))
    L.snhip_abi_last_error(buf, n)
    return buf.value.decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise SnHipError(what, int(rc))


def stream_handle(device=None) -> int:
    """The raw hipStream_t of torch's current stream."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int:
    return t.data_ptr()


# Handles still open when the interpreter exits are closed by an atexit hook,
# which runs before module teardown (torch and its HIP runtime are still up);
# a handle's __del__ during finalization then finds nothing left to free.
_open_handles = None


def track(handle_owner) -> None:
    """Register an object with a close() method to be closed at exit."""
    global _open_handles
    if _open_handles is None:
        import atexit
        import weakref
        _open_handles = weakref.WeakSet()

        def _close_all():
            for h in list(_open_handles):
                try:
                    h.close()
                except Exception:
                    pass
        atexit.register(_close_all)
    _open_handles.add(handle_owner)


def finalizing() -> bool:
    import sys
    return sys.is_finalizing()


def declared_symbols() -> list:
    """Every snhip_* function declared in include/*.h."""
    names = set()
    for h in sorted(INCLUDE.glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"\b(snhip_\w+)\s*\(", text))
    return sorted(names)
