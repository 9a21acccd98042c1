"""GGUF files: a reader, a writer, and RWKV-7 ingestion into the v3 runtime blob.

The reference reads GGUF through the third-party ``gguf`` package
(sunnynet/runtime/gguf.py:15-19, used by experiments/_export_rwkv7.py), which
is not part of this build; this module reads and writes the container itself,
following the published GGUF layout (ggml's GGUF specification, version 3):

* header: ``b"GGUF"``, uint32 version, uint64 tensor count, uint64 metadata
  count; all little-endian;
* metadata: key (uint64 length + UTF-8 bytes), uint32 value type, value.
  Types 0..12: uint8, int8, uint16, int16, uint32, int32, float32, bool,
  string, array (uint32 element type, uint64 count, elements), uint64, int64,
  float64;
* tensor infos: name, uint32 n_dims, uint64 ne[n_dims] (ne[0] the innermost,
  contiguous dimension), uint32 ggml type, uint64 offset into the data section;
* the data section starts at the first multiple of ``general.alignment``
  (default 32) after the infos; every tensor offset is a multiple of it.

Tensor types read here: F32 (0), F16 (1), Q4_0 (2), Q4_1 (3), Q8_0 (8), BF16
(30). Blocks of 32 elements: Q4_0 = fp16 d + 16 bytes, element j = d
((qs[j] & 15) - 8) and element j + 16 = d ((qs[j] >> 4) - 8); Q4_1 = fp16 d,
fp16 m + 16 bytes, element = d q + m with the same nibble order; Q8_0 = fp16 d
+ 32 int8, element = d q. BF16 is the upper half of an fp32. A tensor's
logical (row-major) shape is ``ne`` reversed (sunnynet/runtime/gguf.py:44-46).

``gguf_to_rwkv7_blob`` turns an RWKV-7 GGUF (llama.cpp's tensor names and
metadata keys) into the v3 blob the runtimes load, with the rules of
experiments/_export_rwkv7.py:43-148: shape and vocabulary from the metadata,
every matrix ``M`` (logical ``(out, in)`` in the file) stored as ``M^T`` or
INT4 group 64 where its input length allows, ``time_mix_lerp_fused`` as
``(6, D)``, vectors and the embedding table fp32, the head from
``output.weight`` or, when absent, the tied embedding.
"""
from __future__ import annotations

import codecs
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .rwkv7 import RwkvConfig, RwkvWeights, pack_rwkv7_blob

__all__ = ["GGUFFile", "GGMLType", "read_gguf", "write_gguf", "gguf_to_rwkv7_blob",
           "rwkv7_to_gguf_tensors", "main"]

GGUF_MAGIC = b"GGUF"
GGUF_VERSION = 3
DEFAULT_ALIGNMENT = 32


class GGMLType:
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q8_0 = 8
    BF16 = 30


# (elements per block, bytes per block) of each readable type.
_BLOCK = {GGMLType.F32: (1, 4), GGMLType.F16: (1, 2), GGMLType.BF16: (1, 2),
          GGMLType.Q4_0: (32, 18), GGMLType.Q4_1: (32, 20), GGMLType.Q8_0: (32, 34)}

# Metadata value types.
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALAR = {_U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f",
           _BOOL: "<?", _U64: "<Q", _I64: "<q", _F64: "<d"}


@dataclass
class TensorInfo:
    name: str
    ne: tuple          # ne[0] innermost
    ggml_type: int
    offset: int        # absolute file offset of the data

    @property
    def shape(self) -> tuple:
        """Logical row-major shape (ne reversed)."""
        return tuple(reversed(self.ne))

    @property
    def n_elements(self) -> int:
        return int(np.prod(self.ne, dtype=np.int64)) if self.ne else 1

    @property
    def n_bytes(self) -> int:
        per, nb = _BLOCK[self.ggml_type]
        return self.n_elements // per * nb


class _Reader:
    def __init__(self, mm):
        self.mm, self.pos = mm, 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.mm, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def string(self) -> str:
        n = self.take("<Q")
        b = bytes(self.mm[self.pos:self.pos + n])
        self.pos += n
        return b.decode("utf-8", errors="surrogateescape")

    def value(self, t):
        if t in _SCALAR:
            return self.take(_SCALAR[t])
        if t == _STR:
            return self.string()
        if t == _ARR:
            et = self.take("<I")
            n = self.take("<Q")
            if et in _SCALAR and et != _BOOL:
                dt = np.dtype(_SCALAR[et])
                a = np.frombuffer(self.mm, dtype=dt, count=n, offset=self.pos)
                self.pos += n * dt.itemsize
                return a.tolist()
            return [self.value(et) for _ in range(n)]
        raise ValueError(f"unknown GGUF metadata type {t}")


class GGUFFile:
    """A GGUF file opened read-only (memory-mapped); tensors decoded on demand
    to float32 in their logical shape."""

    def __init__(self, path):
        self.path = str(path)
        self._mm = np.memmap(self.path, dtype=np.uint8, mode="r")
        r = _Reader(self._mm)
        if bytes(self._mm[:4]) != GGUF_MAGIC:
            raise ValueError(f"{self.path}: not a GGUF file")
        r.pos = 4
        self.version = r.take("<I")
        if self.version not in (2, 3):
            raise ValueError(f"{self.path}: GGUF version {self.version} not supported")
        n_tensors = r.take("<Q")
        n_kv = r.take("<Q")
        self.meta: dict = {}
        for _ in range(n_kv):
            key = r.string()
            self.meta[key] = r.value(r.take("<I"))
        infos = []
        for _ in range(n_tensors):
            name = r.string()
            nd = r.take("<I")
            ne = tuple(r.take("<Q") for _ in range(nd))
            t = r.take("<I")
            off = r.take("<Q")
            infos.append((name, ne, t, off))
        self.alignment = int(self.meta.get("general.alignment", DEFAULT_ALIGNMENT))
        data = (r.pos + self.alignment - 1) // self.alignment * self.alignment
        self.tensors: dict[str, TensorInfo] = {}
        for name, ne, t, off in infos:
            if off % self.alignment:
                raise ValueError(f"{self.path}: tensor {name} offset {off} not aligned")
            self.tensors[name] = TensorInfo(name, ne, t, data + off)
        for ti in self.tensors.values():
            if ti.ggml_type in _BLOCK and ti.offset + ti.n_bytes > self._mm.size:
                raise ValueError(f"{self.path}: tensor {ti.name} runs past the end of the file")

    def names(self) -> list:
        return list(self.tensors)

    def has(self, name: str) -> bool:
        return name in self.tensors

    def get_int(self, key: str, default: int = 0) -> int:
        v = self.meta.get(key, default)
        return int(v) if v is not None else default

    def get_float(self, key: str, default: float = 0.0) -> float:
        v = self.meta.get(key, default)
        return float(v) if v is not None else default

    def tokens(self) -> list:
        """Vocabulary as bytes: strings carry ``\\xNN`` escapes, undone as the
        reference does (sunnynet/runtime/gguf.py:90-103)."""
        out = []
        for t in self.meta.get("tokenizer.ggml.tokens", []):
            if not isinstance(t, str):
                out.append(bytes(t))
                continue
            try:
                out.append(codecs.escape_decode(t.encode("latin-1"))[0])
            except (UnicodeEncodeError, ValueError):
                out.append(t.encode("utf-8"))
        return out

    def tensor(self, name: str) -> np.ndarray:
        """float32 copy of a tensor in its logical shape (name or name + ".weight")."""
        if name not in self.tensors and name + ".weight" in self.tensors:
            name += ".weight"
        ti = self.tensors[name]
        if ti.ggml_type not in _BLOCK:
            raise NotImplementedError(f"{name}: GGML type {ti.ggml_type} is not decoded here "
                                      "(F32, F16, BF16, Q4_0, Q4_1 and Q8_0 are)")
        raw = np.asarray(self._mm[ti.offset:ti.offset + ti.n_bytes])
        return _decode(raw, ti.ggml_type, ti.n_elements).reshape(ti.shape)


def read_gguf(path) -> GGUFFile:
    return GGUFFile(path)


def _decode(raw: np.ndarray, t: int, n: int) -> np.ndarray:
    if t == GGMLType.F32:
        return raw.view(np.float32).copy()
    if t == GGMLType.F16:
        return raw.view(np.float16).astype(np.float32)
    if t == GGMLType.BF16:
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    nb = n // 32
    if t == GGMLType.Q8_0:
        blk = raw.reshape(nb, 34)
        d = blk[:, :2].copy().view(np.float16).astype(np.float32)
        q = blk[:, 2:].view(np.int8).astype(np.float32)
        return (d * q).reshape(-1)
    if t in (GGMLType.Q4_0, GGMLType.Q4_1):
        hb = 2 if t == GGMLType.Q4_0 else 4
        blk = raw.reshape(nb, 16 + hb)
        d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)
        qs = blk[:, hb:]
        q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.float32)
        if t == GGMLType.Q4_0:
            return (d * (q - 8.0)).reshape(-1)
        m = blk[:, 2:4].copy().view(np.float16).astype(np.float32)
        return (d * q + m).reshape(-1)
    raise NotImplementedError(t)


# ------------------------------------------------------------------- writer
def _pack_value(v, t=None) -> bytes:
    if t is None:
        if isinstance(v, bool):
            t = _BOOL
        elif isinstance(v, int):
            t = _I64 if v < -2**31 or v >= 2**31 else (_U32 if v >= 0 else _I32)
        elif isinstance(v, float):
            t = _F32
        elif isinstance(v, str):
            t = _STR
        elif isinstance(v, (list, tuple)):
            t = _ARR
        else:
            raise TypeError(f"no GGUF type for {type(v)}")
    body = struct.pack("<I", t)
    if t in _SCALAR:
        return body + struct.pack(_SCALAR[t], v)
    if t == _STR:
        b = v.encode("utf-8", errors="surrogateescape")
        return body + struct.pack("<Q", len(b)) + b
    et = _pack_value(v[0])[:4] if v else struct.pack("<I", _U32)
    elem_t = struct.unpack("<I", et)[0]
    out = body + et + struct.pack("<Q", len(v))
    for x in v:
        out += _pack_value(x, elem_t)[4:]
    return out


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, meta: dict, tensors: dict, alignment: int = DEFAULT_ALIGNMENT) -> None:
    """Write a GGUF v3 file. `tensors`: name -> (ggml_type, ne tuple, raw
    bytes) or a float32 array (stored F32, ne = shape reversed). `meta` values
    are Python scalars, strings or lists, or (type code, value) pairs."""
    meta = dict(meta)
    if alignment != DEFAULT_ALIGNMENT:
        meta["general.alignment"] = (_U32, alignment)
    kv = b""
    for k, v in meta.items():
        kv += _str(k) + (_pack_value(v[1], v[0]) if isinstance(v, tuple) and len(v) == 2
                         and isinstance(v[0], int) and not isinstance(v[0], bool) else _pack_value(v))
    entries = []
    for name, spec in tensors.items():
        if isinstance(spec, np.ndarray):
            a = np.ascontiguousarray(spec, np.float32)
            spec = (GGMLType.F32, tuple(reversed(a.shape)), a.tobytes())
        entries.append((name, *spec))
    infos, blobs, off = b"", [], 0
    for name, t, ne, raw in entries:
        per, nb = _BLOCK[t]
        n = int(np.prod(ne, dtype=np.int64))
        if n % per or len(raw) != n // per * nb:
            raise ValueError(f"{name}: {len(raw)} bytes do not hold {n} elements of type {t}")
        infos += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", x) for x in ne)
        infos += struct.pack("<IQ", t, off)
        pad = (-len(raw)) % alignment
        blobs.append(raw + b"\0" * pad)
        off += len(raw) + pad
    head = GGUF_MAGIC + struct.pack("<IQQ", GGUF_VERSION, len(entries), len(meta)) + kv + infos
    head += b"\0" * ((-len(head)) % alignment)
    with open(path, "wb") as f:
        f.write(head)
        for b in blobs:
            f.write(b)


# ------------------------------------------------------------- RWKV-7 mapping
# llama.cpp's RWKV-7 tensor names for the blob's per-layer fields
# (experiments/_export_rwkv7.py:101-135).
_LAYER_VEC = [("ln1_w", "attn_norm.weight"), ("ln1_b", "attn_norm.bias"),
              ("ln2_w", "attn_norm_2.weight"), ("ln2_b", "attn_norm_2.bias")]
_LAYER_MAT = [("r", "time_mix_receptance"), ("k", "time_mix_key"), ("v", "time_mix_value"),
              ("o", "time_mix_output"), ("w1", "time_mix_w1"), ("w2", "time_mix_w2"),
              ("a1", "time_mix_a1"), ("a2", "time_mix_a2"), ("v1", "time_mix_v1"),
              ("v2", "time_mix_v2"), ("g1", "time_mix_g1"), ("g2", "time_mix_g2"),
              ("cmk", "channel_mix_key"), ("cmv", "channel_mix_value")]
_LAYER_VEC2 = [("w0", "time_mix_w0"), ("a0", "time_mix_a0"), ("v0", "time_mix_v0"),
               ("kk", "time_mix_k_k"), ("ka", "time_mix_k_a"), ("rk", "time_mix_r_k"),
               ("lnx_w", "time_mix_ln.weight"), ("lnx_b", "time_mix_ln.bias"),
               ("cmk_lerp", "channel_mix_lerp_k")]


def _w(name: str) -> str:
    return name if name.endswith((".weight", ".bias")) else name + ".weight"


def gguf_to_rwkv7_blob(path, int4: bool = True) -> bytes:
    """v3 runtime blob (INT4 group 64 where allowed, else fp32) of an RWKV-7
    GGUF file (experiments/_export_rwkv7.py:43-148)."""
    g = GGUFFile(path)
    L = g.get_int("rwkv7.block_count", 12)
    D = g.get_int("rwkv7.embedding_length", 768)
    HS = g.get_int("rwkv7.wkv.head_size", 64)
    F = g.get_int("rwkv7.feed_forward_length", 3072)
    vocab = len(g.tokens())
    eps = g.get_float("rwkv7.attention.layer_norm_epsilon", 1e-5)

    def vec(name):
        return np.ascontiguousarray(g.tensor(name), np.float32).reshape(-1)

    layers, ranks = [], []
    for i in range(L):
        p = f"blk.{i}."
        Ld = {k: vec(p + n) for k, n in _LAYER_VEC}
        Ld["lerp"] = g.tensor(p + "time_mix_lerp_fused.weight").reshape(6, D)
        for k, n in _LAYER_MAT:
            M = g.tensor(p + n + ".weight")
            if M.ndim != 2:
                raise ValueError(f"{p + n}: expected a matrix, got shape {M.shape}")
            Ld[k] = np.ascontiguousarray(M, np.float32)
        for k, n in _LAYER_VEC2:
            Ld[k] = vec(p + _w(n))
        ranks.append((Ld["w1"].shape[0], Ld["a1"].shape[0], Ld["v1"].shape[0], Ld["g1"].shape[0]))
        layers.append(Ld)
    embed = np.ascontiguousarray(g.tensor("token_embd.weight"), np.float32)
    head = g.tensor("output.weight") if g.has("output.weight") else embed
    if embed.shape != (vocab, D):
        raise ValueError(f"token_embd.weight is {embed.shape}, expected ({vocab}, {D})")
    cfg = RwkvConfig(layers=L, dim=D, head_size=HS, ff=F, vocab=vocab, ranks=ranks[0] if ranks else (0,) * 4,
                     eps=eps)
    w = RwkvWeights(cfg=cfg, layers=layers, en_w=vec("token_embd_norm.weight"),
                    en_b=vec("token_embd_norm.bias"), on_w=vec("output_norm.weight"),
                    on_b=vec("output_norm.bias"), embed=embed,
                    head=np.ascontiguousarray(head, np.float32))
    return pack_rwkv7_blob(w, int4=int4, ranks=ranks)


def rwkv7_to_gguf_tensors(w: RwkvWeights, ggml_type: int = GGMLType.F32, tied: bool = False) -> dict:
    """The tensors of `w` under llama.cpp's RWKV-7 names and shapes (every
    matrix logical (out, in); the mix vector (6, 1, 1, D) as in the files),
    as write_gguf specs of type F32, F16 or BF16."""
    D = w.cfg.dim

    def spec(a, shape=None):
        a = np.ascontiguousarray(a, np.float32)
        shape = a.shape if shape is None else shape
        ne = tuple(reversed(shape))
        if ggml_type == GGMLType.F32:
            return (GGMLType.F32, ne, a.tobytes())
        if ggml_type == GGMLType.F16:
            return (GGMLType.F16, ne, a.astype(np.float16).tobytes())
        if ggml_type == GGMLType.BF16:
            u = a.view(np.uint32)
            r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)   # nearest even
            return (GGMLType.BF16, ne, r.tobytes())
        raise ValueError(ggml_type)

    out = {"token_embd.weight": spec(w.embed), "token_embd_norm.weight": spec(w.en_w),
           "token_embd_norm.bias": spec(w.en_b), "output_norm.weight": spec(w.on_w),
           "output_norm.bias": spec(w.on_b)}
    if not tied:
        out["output.weight"] = spec(w.head)
    for i, Ld in enumerate(w.layers):
        p = f"blk.{i}."
        for k, n in _LAYER_VEC:
            out[p + n] = spec(Ld[k])
        out[p + "time_mix_lerp_fused.weight"] = spec(Ld["lerp"], (6, 1, 1, D))
        for k, n in _LAYER_MAT:
            out[p + n + ".weight"] = spec(Ld[k])
        for k, n in _LAYER_VEC2:
            out[p + _w(n)] = spec(Ld[k], (1, 1, D) if k in ("w0", "a0", "v0", "kk", "ka") else None)
    return out


def main(argv=None) -> int:
    """python -m sunnynet_amd.gguf IN.gguf OUT.bin [--f32]"""
    import sys
    argv = sys.argv[1:] if argv is None else argv
    if len(argv) < 2:
        print(main.__doc__)
        return 2
    buf = gguf_to_rwkv7_blob(argv[0], int4="--f32" not in argv)
    Path(argv[1]).write_bytes(buf)
    print(f"{argv[1]}: {len(buf)} bytes")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
