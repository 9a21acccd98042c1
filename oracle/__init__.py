"""CPU oracle for the SunnyNet token loop — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this package, and only as the checker. The product
(``sunnynet_amd``) never imports, links or falls back to anything here.

Two layers:

* ``liboracle.so`` (``sn_oracle.c``, ``rwkv7_oracle.c``): a scalar ISO-C
  restatement of the reference's C runtime with its exact operation order.
  Each function cites the reference ``file:line`` it follows.
* ``_ref/*.so``: the reference's own C sources compiled unmodified from the
  reference tree by ``oracle/Makefile``. They pin the restatement (bit-exact)
  and serve as the timed CPU baseline. They exist only where the reference
  tree was present at build time.

Parity status of each oracle function (what pins it):

* ``recur_scan`` / ``recur_step``: bit-exact vs ``_ref`` ``sn_recur_scan`` /
  ``sn_recur_step``, vs ``sn_abi_recur_*``, and vs an fp64 loop (closed form).
* ``quant_i4`` / ``dequant_i4``: bit-exact vs ``_ref`` ``sn_quant_i4`` /
  ``sn_dequant_i4``; the packing is checked against the explicit nibble formula
  of the reference's ``tests/test_quant_i4.py:32-70``.
* ``SnOracle`` (decode step): bit-exact vs ``_ref`` ``sn_step`` on the same
  blob, per-layer intermediates vs ``sn_dbg_layer``; fp64 torch restatement of
  ``forward_step`` within 1e-5 (see ``torch_ref``).
* ``RkOracle`` (RWKV-7 step): bit-exact vs ``_ref`` ``sn_rk_step`` on fp32 v3
  blobs.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_DIR = HERE / "_ref"
REFERENCE_ROOT = Path(os.environ.get("SUNNY_REFERENCE", "/root/reference/sunnynet"))

_lib = None
_ref = {}


def build(ref: bool = True) -> None:
    """Compile liboracle.so (and oracle/_ref from the reference tree if present)."""
    target = "all" if ref else "oracle"
    r = subprocess.run(["make", "-C", str(HERE), target, f"REF={REFERENCE_ROOT}"],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout[-2000:]}\n{r.stderr[-2000:]}")


def _f(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB.exists():
        build(ref=False)
    lib = ctypes.CDLL(str(LIB))
    V, I, L = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    lib.orc_recur_scan.argtypes = [V, V, V, V, V, I, I, I, I]
    lib.orc_recur_step.argtypes = [V, V, V, I, I, I]
    lib.orc_scan_bwd.argtypes = [V, V, V, V, V, V, V, V, I, I, I]
    lib.orc_core_fwd.argtypes = [V, V, V, V, V, V, I, I, I]
    lib.orc_core_bwd.argtypes = [V, V, V, V, V, V, V, V, V, V, V, I, I, I]
    lib.orc_quant_i4.argtypes = [V, V, V, I, I, I]
    lib.orc_dequant_i4.argtypes = [V, V, V, I, I, I]
    lib.orc_sn_new.restype = V
    lib.orc_sn_new.argtypes = [V, L, I]
    for n in ("orc_sn_free", "orc_sn_reset"):
        getattr(lib, n).argtypes = [V]
    lib.orc_sn_dims.argtypes = [V, V]
    lib.orc_sn_step.argtypes = [V, V, V]
    lib.orc_sn_step_one.argtypes = [V, I, ctypes.c_int32, V]
    lib.orc_sn_get_state.argtypes = [V, V, V]
    lib.orc_sn_set_state.argtypes = [V, V, V]
    lib.orc_sn_dbg_layer.argtypes = [V, I, ctypes.c_int32, I, V]
    lib.orc_libm.argtypes = [V, V, V, L]
    lib.orc_rk_new.restype = V
    lib.orc_rk_new.argtypes = [V, L, I, I]
    for n in ("orc_rk_free", "orc_rk_reset"):
        getattr(lib, n).argtypes = [V]
    lib.orc_rk_dims.argtypes = [V, V]
    lib.orc_rk_step.argtypes = [V, V, V]
    lib.orc_rk_step_one.argtypes = [V, I, ctypes.c_int32, V]
    lib.orc_rk_get_state.argtypes = [V, V, V]
    lib.orc_rk_set_state.argtypes = [V, V, V]
    _lib = lib
    return lib


# ---------------------------------------------------------------- recurrence
def recur_scan(a, b, s0, gated: bool):
    """recur.c:13-48. a, b (B,T,N) fp32; s0 (B,N) -> (out (B,T,N), send (B,N))."""
    lib = load()
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    s0 = np.ascontiguousarray(s0, np.float32)
    B, T, N = a.shape
    out = np.empty_like(a)
    send = np.empty_like(s0)
    lib.orc_recur_scan(_f(a), _f(b), _f(s0), _f(out), _f(send), B, T, N, int(bool(gated)))
    return out, send


def scan_bwd(p, nu, s0, out, dout):
    """scan_avx2.c:50-99: gradients of the gated scan s_t = p s + (1-p) nu.
    p, nu, out (forward states), dout (B,T,N); s0 (B,N) -> (dp, dnu, ds0)."""
    lib = load()
    p, nu, out, dout = (np.ascontiguousarray(x, np.float32) for x in (p, nu, out, dout))
    s0 = np.ascontiguousarray(s0, np.float32)
    B, T, N = p.shape
    dp, dnu = np.empty_like(p), np.empty_like(p)
    ds0 = np.empty_like(s0)
    lib.orc_scan_bwd(_f(p), _f(nu), _f(s0), _f(out), _f(dout), _f(dp), _f(dnu), _f(ds0), B, T, N)
    return dp, dnu, ds0


def core_fwd(q, delta, s0):
    """core_avx2.c:34-73: q (B,T,2D) [u_raw | gate], delta (D), s0 (B,D) ->
    (states, u, p), each (B,T,D)."""
    lib = load()
    q = np.ascontiguousarray(q, np.float32)
    delta = np.ascontiguousarray(delta, np.float32)
    s0 = np.ascontiguousarray(s0, np.float32)
    B, T, D2 = q.shape
    D = D2 // 2
    st, u, p = (np.empty((B, T, D), np.float32) for _ in range(3))
    lib.orc_core_fwd(_f(q), _f(delta), _f(s0), _f(st), _f(u), _f(p), B, T, D)
    return st, u, p


def core_bwd(q, delta, s0, states, u, p, dstate, du_in):
    """core_avx2.c:78-149 -> (dq (B,T,2D), ddelta (D), ds0 (B,D)); ddelta sums
    the rows in order."""
    lib = load()
    arrs = [np.ascontiguousarray(x, np.float32) for x in (q, delta, s0, states, u, p, dstate, du_in)]
    q = arrs[0]
    B, T, D2 = q.shape
    D = D2 // 2
    dq = np.empty_like(q)
    dd = np.zeros(D, np.float32)
    ds0 = np.empty((B, D), np.float32)
    lib.orc_core_bwd(*[_f(a) for a in arrs], _f(dq), _f(dd), _f(ds0), B, T, D)
    return dq, dd, ds0


def recur_step(a, b, s, gated: bool):
    """recur.c:109-131. Returns the updated copy of s (B,N)."""
    lib = load()
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    s = np.array(s, np.float32, copy=True, order="C")
    B, N = a.shape
    lib.orc_recur_step(_f(a), _f(b), _f(s), B, N, int(bool(gated)))
    return s


# ---------------------------------------------------------------------- INT4
def quant_i4(x, block: int):
    """quant.c:34-65. x (rows,N) -> q (rows,N/2) u8, scale (rows,N/block) f32."""
    lib = load()
    x = np.ascontiguousarray(x, np.float32)
    rows, N = x.shape
    q = np.empty((rows, N // 2), np.uint8)
    sc = np.empty((rows, N // block), np.float32)
    lib.orc_quant_i4(_f(x), _f(q), _f(sc), rows, N, block)
    return q, sc


def dequant_i4(q, scale, N: int, block: int):
    """quant.c:67-87."""
    lib = load()
    q = np.ascontiguousarray(q, np.uint8)
    scale = np.ascontiguousarray(scale, np.float32)
    x = np.empty((q.shape[0], N), np.float32)
    lib.orc_dequant_i4(_f(q), _f(scale), _f(x), q.shape[0], N, block)
    return x


# --------------------------------------------------------------- decode step
class SnOracle:
    """sunnynet.c decode step over `batch` independent sequences of one blob."""

    def __init__(self, blob: bytes | np.ndarray, batch: int = 1):
        self._lib = load()
        self._blob = np.frombuffer(bytes(blob), np.uint8) if not isinstance(blob, np.ndarray) else blob
        self._h = self._lib.orc_sn_new(_f(self._blob), self._blob.nbytes, int(batch))
        if not self._h:
            raise RuntimeError("oracle: blob rejected (magic/size)")
        hdr = np.zeros(10, np.int32)
        self._lib.orc_sn_dims(self._h, _f(hdr))
        (self.vocab, self.D, self.I, self.R, self.K, self.L, self.group,
         self.tied, self.clamp, self.batch) = (int(v) for v in hdr)
        self.kh = max(0, self.K - 1)

    def reset(self):
        self._lib.orc_sn_reset(self._h)

    def step(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(np.asarray(tokens, np.int32).reshape(self.batch))
        out = np.empty((self.batch, self.vocab), np.float32)
        self._lib.orc_sn_step(self._h, _f(t), _f(out))
        return out

    def step_one(self, b: int, token: int) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        self._lib.orc_sn_step_one(self._h, int(b), int(token), _f(out))
        return out

    def get_state(self):
        s = np.empty((self.batch, self.L, self.D), np.float32)
        h = np.empty((self.batch, self.L, self.kh, self.D), np.float32)
        self._lib.orc_sn_get_state(self._h, _f(s), _f(h))
        return s, h

    def set_state(self, s, hist):
        s = np.ascontiguousarray(s, np.float32)
        hist = np.ascontiguousarray(hist, np.float32)
        assert s.shape == (self.batch, self.L, self.D)
        assert hist.shape == (self.batch, self.L, self.kh, self.D)
        self._lib.orc_sn_set_state(self._h, _f(s), _f(hist))

    def dbg_layer(self, b: int, token: int, layer: int) -> dict:
        D, I, R = self.D, self.I, self.R
        buf = np.empty(8 * D + R + 2 * I, np.float32)
        self._lib.orc_sn_dbg_layer(self._h, int(b), int(token), int(layer), _f(buf))
        names = [("raw", D), ("at", D), ("v", R), ("gate", D), ("u", D), ("s", D),
                 ("zn", I), ("yn", I), ("sfb", D), ("out", D)]
        out, o = {}, 0
        for n, k in names:
            out[n] = buf[o:o + k].copy()
            o += k
        return out

    def close(self):
        if getattr(self, "_h", None):
            self._lib.orc_sn_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class RkOracle:
    """rwkv7.c decode step (fp32 path; INT4 tags dequantized at load)."""

    def __init__(self, blob: bytes | np.ndarray, batch: int = 1, block: int = 64):
        self._lib = load()
        self._blob = np.frombuffer(bytes(blob), np.uint8) if not isinstance(blob, np.ndarray) else blob
        self._h = self._lib.orc_rk_new(_f(self._blob), self._blob.nbytes, int(batch), int(block))
        if not self._h:
            raise RuntimeError("oracle: RWKV-7 blob rejected")
        hdr = np.zeros(8, np.int32)
        self._lib.orc_rk_dims(self._h, _f(hdr))
        (self.L, self.D, self.HS, self.NH, self.F, self.vocab, self.q4,
         self.batch) = (int(v) for v in hdr)

    def reset(self):
        self._lib.orc_rk_reset(self._h)

    def step(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(np.asarray(tokens, np.int32).reshape(self.batch))
        out = np.empty((self.batch, self.vocab), np.float32)
        self._lib.orc_rk_step(self._h, _f(t), _f(out))
        return out

    def step_one(self, b: int, token: int) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        self._lib.orc_rk_step_one(self._h, int(b), int(token), _f(out))
        return out

    def get_state(self):
        S = np.empty((self.batch, self.L, self.NH, self.HS, self.HS), np.float32)
        sh = np.empty((self.batch, self.L, 2, self.D), np.float32)
        self._lib.orc_rk_get_state(self._h, _f(S), _f(sh))
        return S, sh

    def set_state(self, S, shift):
        S = np.ascontiguousarray(S, np.float32)
        shift = np.ascontiguousarray(shift, np.float32)
        self._lib.orc_rk_set_state(self._h, _f(S), _f(shift))

    def close(self):
        if getattr(self, "_h", None):
            self._lib.orc_rk_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------- the reference's own C
def libm(x):
    """(expf(x), tanhf(x)) from the host C library, elementwise."""
    x = np.ascontiguousarray(x, np.float32)
    e = np.empty_like(x)
    t = np.empty_like(x)
    load().orc_libm(_f(x), _f(e), _f(t), x.size)
    return e, t


def ref_available() -> bool:
    return (REF_DIR / "libref_model.so").exists()


def ref_lib(name: str):
    """Load oracle/_ref/libref_<name>.so (the reference's unmodified C)."""
    if name in _ref:
        return _ref[name]
    path = REF_DIR / f"libref_{name}.so"
    if not path.exists():
        raise FileNotFoundError(f"{path} not built (reference tree absent at build time)")
    lib = ctypes.CDLL(str(path))
    V, I, P = ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p
    if name == "model":
        lib.sn_load.restype = V
        lib.sn_load.argtypes = [P, I, I, I, I, I, I, I, I]
        lib.sn_load_h.restype = V
        lib.sn_load_h.argtypes = [P, I, I, I, I, I, I, I, I]
        lib.sn_free.argtypes = [V]
        lib.sn_reset.argtypes = [V]
        lib.sn_step.argtypes = [V, I, V]
        lib.sn_prefill.argtypes = [V, V, I, V]
        lib.sn_vocab.argtypes = [V]
        lib.sn_vocab.restype = I
        lib.sn_ready.argtypes = [V]
        lib.sn_ready.restype = I
        lib.sn_set_threads.argtypes = [I]
        lib.sn_get_threads.restype = I
        lib.sn_recommended_threads.restype = I
        lib.sn_dbg_layer.argtypes = [V, I, I, V]
    elif name == "recur":
        lib.sn_recur_scan.argtypes = [V, V, V, V, V, I, I, I, I]
        lib.sn_recur_step.argtypes = [V, V, V, I, I, I]
        lib.sn_set_threads.argtypes = [I]
        lib.sn_threads.restype = I
    elif name == "quant":
        lib.sn_quant_i4.argtypes = [V, V, V, I, I, I]
        lib.sn_dequant_i4.argtypes = [V, V, V, I, I, I]
        lib.sn_gemv_i4.argtypes = [V, V, V, V, I, I, I]
        lib.sn_gemv_f32.argtypes = [V, V, V, I, I]
    elif name == "rwkv7":
        lib.sn_rk_load.restype = V
        lib.sn_rk_load.argtypes = [P]
        lib.sn_rk_free.argtypes = [V]
        lib.sn_rk_reset.argtypes = [V]
        lib.sn_rk_step.argtypes = [V, I, V]
        lib.sn_rk_prefill.argtypes = [V, V, I, V]
        lib.sn_rk_vocab.argtypes = [V]
        lib.sn_rk_vocab.restype = I
        lib.sn_rk_dbg.argtypes = [V, I, I, V]
    elif name == "scan":
        lib.scan_f32.argtypes = [V, V, V, V, V, I, I, I]
        lib.scan_bwd_f32.argtypes = [V, V, V, V, V, V, V, V, I, I, I]
    elif name == "core":
        lib.core_fwd_f32.argtypes = [V, V, V, V, V, V, I, I, I]
        lib.core_bwd_f32.argtypes = [V, V, V, V, V, V, V, V, V, V, V, I, I, I]
        lib.sn_set_threads.argtypes = [I]
    elif name == "abi":
        I32 = ctypes.c_int32
        lib.sn_abi_recur_scan.argtypes = [V, V, V, V, V, I32, I32, I32, I32]
        lib.sn_abi_recur_scan.restype = I32
        lib.sn_abi_recur_step.argtypes = [V, V, V, I32, I32, I32]
        lib.sn_abi_recur_step.restype = I32
        lib.sn_abi_version.restype = I32
        lib.sn_abi_caps.restype = ctypes.c_uint32
    _ref[name] = lib
    return lib


class RefSnModel:
    """The reference's sn_load/sn_step handle (B=1), for pinning and timing."""

    def __init__(self, path, vocab, dim, inner, rank, taps, layers, group=8, tied=1, half=False):
        self._lib = ref_lib("model")
        self.vocab = vocab
        load = self._lib.sn_load_h if half else self._lib.sn_load
        self._h = load(str(path).encode(), vocab, dim, inner, rank, taps, layers, group, tied)
        if not self._h:
            raise RuntimeError(f"reference sn_load rejected {path}")
        self._logits = np.empty(vocab, np.float32)

    def reset(self):
        self._lib.sn_reset(self._h)

    def step(self, token: int) -> np.ndarray:
        self._lib.sn_step(self._h, int(token), _f(self._logits))
        return self._logits.copy()

    def prefill(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(np.asarray(tokens, np.int32))
        self._lib.sn_prefill(self._h, _f(t), len(t), _f(self._logits))
        return self._logits.copy()

    def dbg_layer(self, token: int, layer: int, D, I, R) -> np.ndarray:
        buf = np.empty(8 * D + R + 2 * I, np.float32)
        self._lib.sn_dbg_layer(self._h, int(token), int(layer), _f(buf))
        return buf

    def close(self):
        if getattr(self, "_h", None):
            self._lib.sn_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class RefRk:
    """The reference's sn_rk_load/sn_rk_step handle (B=1)."""

    def __init__(self, path, vocab: int):
        self._lib = ref_lib("rwkv7")
        self._h = self._lib.sn_rk_load(str(path).encode())
        if not self._h:
            raise RuntimeError(f"reference sn_rk_load rejected {path}")
        self.vocab = vocab
        self._logits = np.empty(vocab, np.float32)

    def reset(self):
        self._lib.sn_rk_reset(self._h)

    def step(self, token: int) -> np.ndarray:
        self._lib.sn_rk_step(self._h, int(token), _f(self._logits))
        return self._logits.copy()

    def dbg(self, token: int, layer: int, dim: int) -> np.ndarray:
        out = np.empty(9 * dim, np.float32)
        self._lib.sn_rk_dbg(self._h, int(token), int(layer), _f(out))
        return out.reshape(9, dim)

    def close(self):
        if getattr(self, "_h", None):
            self._lib.sn_rk_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
