"""SunnyNet runtime blob: the packed fp32 weight file the reference C runtime
loads (writer: experiments/_export_runtime.py:43-100; reader:
sunnynet/runtime/sunnynet.c:358-454).

Layout (little-endian): 10 x int32 header
``magic=0x4E4E5355, vocab, dim, inner, rank, taps, layers, group=8, tied, clamp``
then fp32 payload, per layer
``norm_in.gamma (D), norm_in.center (D), norm_mix.gamma (I), norm_mix.center (I),
dw^T (K,D), V^T (D,R), U^T (R,2D), W_z^T (D,I), W_c^T (I,D), W_s_eff^T (D,D),
delta (D), tanh(a), b_gain``
then ``eps, p_floor, norm_out.gamma (D), norm_out.center (D), embed (V,D),
head^T (D,V)``.

The format is the reference's (it is the drop-in artefact), so the field order
is identical by necessity.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np
import torch

from .config import SunnyConfig
from .weights import SunnyWeights

MAGIC = 0x4E4E5355
HEADER_BYTES = 40


def _np(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        t = t.detach().float().contiguous().cpu().numpy()
    return np.ascontiguousarray(t, dtype=np.float32)


def norm_eps(s_min: float = 0.02, eps: float = 1e-5) -> float:
    """CenteredScaleNorm's effective epsilon s_min^2 + eps (ops.py:45-47);
    the exporter stores the max over blocks (_export_runtime.py:58-62)."""
    return s_min * s_min + eps


@dataclass
class BlobMatrices:
    """The (out,in) fp32 matrices a decode step multiplies, per layer."""
    V: np.ndarray
    U: np.ndarray
    W_z: np.ndarray
    W_c: np.ndarray
    W_s_eff: np.ndarray


def layer_matrices(w: SunnyWeights, l: int) -> BlobMatrices:
    L = w.layers[l]
    return BlobMatrices(V=_np(L.V), U=_np(L.U), W_z=_np(L.W_z), W_c=_np(L.W_c),
                        W_s_eff=_np(w.ws_eff(l)))


def pack_sunny_blob(w: SunnyWeights, matrices: list | None = None,
                    head: np.ndarray | None = None) -> bytes:
    """Serialize weights into the runtime blob.

    `matrices` (one BlobMatrices per layer) and `head` ((V,D) row-major)
    override the matrices taken from `w` — used to store dequantized INT4
    weights for the fp32 reference path. The lookup embedding always comes
    from ``w.embed``.
    """
    cfg = w.cfg
    D, I, R, K, L, V = cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, cfg.vocab_size
    if not cfg.tie_embeddings:
        raise ValueError("the runtime blob requires tied embeddings (_export_runtime.py:53-54)")
    parts = [struct.pack("<10i", MAGIC, V, D, I, R, K, L, 8, 1, int(cfg.need_clamp))]
    for l in range(L):
        Lw = w.layers[l]
        M = matrices[l] if matrices is not None else layer_matrices(w, l)
        parts += [_np(Lw.ni_g).tobytes(), _np(Lw.ni_c).tobytes(),
                  _np(Lw.nm_g).tobytes(), _np(Lw.nm_c).tobytes(),
                  np.ascontiguousarray(_np(Lw.dw).reshape(D, K).T).tobytes(),
                  np.ascontiguousarray(M.V.T).tobytes(),
                  np.ascontiguousarray(M.U.T).tobytes(),
                  np.ascontiguousarray(M.W_z.T).tobytes(),
                  np.ascontiguousarray(M.W_c.T).tobytes(),
                  np.ascontiguousarray(M.W_s_eff.T).tobytes(),
                  _np(w.delta(l)).tobytes(),
                  struct.pack("<2f", float(torch.tanh(Lw.a)), float(Lw.b_gain))]
    parts.append(struct.pack("<2f", norm_eps(), 1.0 / cfg.h_max))
    parts += [_np(w.no_g).tobytes(), _np(w.no_c).tobytes(), _np(w.embed).tobytes()]
    hd = _np(w.head_weight()) if head is None else np.ascontiguousarray(head, np.float32)
    parts.append(np.ascontiguousarray(hd.T).tobytes())
    return b"".join(parts)


def write_sunny_blob(path, w: SunnyWeights, **kw) -> int:
    buf = pack_sunny_blob(w, **kw)
    with open(path, "wb") as f:
        f.write(buf)
    return len(buf)


def blob_floats(cfg: SunnyConfig) -> int:
    D, I, R, K, L, V = cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, cfg.vocab_size
    per_layer = 2 * D + 2 * I + K * D + D * R + R * 2 * D + D * I + I * D + D * D + D + 2
    return L * per_layer + 2 + 2 * D + V * D + D * V


def parse_sunny_blob(buf) -> dict:
    """Header and (out,in) matrices of a runtime blob, as numpy views/copies."""
    raw = np.frombuffer(bytes(buf) if not isinstance(buf, (bytes, bytearray, memoryview)) else buf,
                        dtype=np.uint8)
    h = np.frombuffer(raw[:HEADER_BYTES].tobytes(), np.int32)
    if int(h[0]) != MAGIC:
        raise ValueError("bad magic")
    V, D, I, R, K, L, G, tied, clamp = (int(x) for x in h[1:10])
    cfg = SunnyConfig(vocab_size=V, dim=D, inner=I, rank=R, taps=K, layers=L)
    f = np.frombuffer(raw[HEADER_BYTES:].tobytes(), np.float32)
    if f.size != blob_floats(cfg):
        raise ValueError(f"blob payload has {f.size} floats, expected {blob_floats(cfg)}")
    o = 0

    def take(n, shape=None):
        nonlocal o
        a = f[o:o + n]
        o += n
        return a.reshape(shape) if shape else a

    layers = []
    for _ in range(L):
        d = {}
        d["ni_g"], d["ni_c"] = take(D), take(D)
        d["nm_g"], d["nm_c"] = take(I), take(I)
        d["dw_t"] = take(K * D, (K, D))
        d["V"] = take(D * R, (D, R)).T.copy()
        d["U"] = take(R * 2 * D, (R, 2 * D)).T.copy()
        d["W_z"] = take(D * I, (D, I)).T.copy()
        d["W_c"] = take(I * D, (I, D)).T.copy()
        d["W_s_eff"] = take(D * D, (D, D)).T.copy()
        d["delta"] = take(D)
        d["a_tanh"], d["b_gain"] = (float(x) for x in take(2))
        layers.append(d)
    eps, p_floor = (float(x) for x in take(2))
    out = dict(cfg=cfg, group=G, tied=tied, clamp=clamp, layers=layers, eps=eps,
               p_floor=p_floor, no_g=take(D), no_c=take(D), embed=take(V * D, (V, D)))
    out["head"] = take(D * V, (D, V)).T.copy()
    return out


# ---------------------------------------------------------------------------
# INT4 blob: the same model with every matrix a decode step multiplies (V, U,
# W_z, W_c, W_s_eff and the head) stored pre-quantized, so an INT4 handle loads
# it without quantizing. The reference has no quantized SunnyNet file; its
# INT4 arithmetic (quant.c:34-87, group size 32 or 64) is what is stored.
#
# Layout (little-endian): 12 x int32 header
# ``magic=0x34514E53 ('SNQ4'), version=1, vocab, dim, inner, rank, taps,
# layers, group=8, tied, clamp, block``
# then, per layer, ``norm_in.gamma (D), norm_in.center (D), norm_mix.gamma (I),
# norm_mix.center (I), dw^T (K,D)`` (fp32), the five matrices V (R,D), U (2D,R),
# W_z (I,D), W_c (D,I), W_s_eff (D,D) (row-major (out, in); U's rows in the
# model's order, values then gates), each as ``codes (out, in/2) uint8`` then
# ``scales (out, in/block) float32``, then ``delta (D), tanh(a), b_gain``;
# then ``eps, p_floor, norm_out.gamma (D), norm_out.center (D), embed (V,D)``
# (fp32, the lookup table) and the head (V,D) as codes then scales.
# Codes pack the quant.c way: byte k of a group holds q[k] | q[k + block/2] << 4.

I4_MAGIC = 0x34514E53
I4_VERSION = 1
I4_HEADER_BYTES = 48


def convert_blob_int4(buf, block: int = 32) -> bytes:
    """The INT4 blob of an fp32 runtime blob (quantized as quant.c does)."""
    from .rwkv7 import quant_i4_np
    if block not in (32, 64):
        raise ValueError("block must be 32 or 64")
    b = parse_sunny_blob(buf)
    cfg = b["cfg"]
    D, I, R, K, L, V = cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.layers, cfg.vocab_size
    for n in (D, I, R):
        if n % block:
            raise ValueError("block must divide dim, inner and rank")
    parts = [struct.pack("<12i", I4_MAGIC, I4_VERSION, V, D, I, R, K, L, b["group"], b["tied"],
                         b["clamp"], block)]

    def mat(M):
        q, s = quant_i4_np(np.ascontiguousarray(M, np.float32), block)
        return [q.tobytes(), s.tobytes()]

    for d in b["layers"]:
        parts += [d[k].astype(np.float32).tobytes() for k in ("ni_g", "ni_c", "nm_g", "nm_c")]
        parts.append(np.ascontiguousarray(d["dw_t"], np.float32).tobytes())
        for k in ("V", "U", "W_z", "W_c", "W_s_eff"):
            parts += mat(d[k])
        parts += [d["delta"].astype(np.float32).tobytes(),
                  struct.pack("<2f", d["a_tanh"], d["b_gain"])]
    parts.append(struct.pack("<2f", b["eps"], b["p_floor"]))
    parts += [b["no_g"].astype(np.float32).tobytes(), b["no_c"].astype(np.float32).tobytes(),
              np.ascontiguousarray(b["embed"], np.float32).tobytes()]
    parts += mat(b["head"])
    return b"".join(parts)


def parse_blob_int4(buf) -> dict:
    """Header, small parameters and (codes, scales) pairs of an INT4 blob."""
    raw = bytes(buf)
    h = struct.unpack_from("<12i", raw, 0)
    if h[0] != I4_MAGIC or h[1] != I4_VERSION:
        raise ValueError("not an INT4 SunnyNet blob (magic or version)")
    V, D, I, R, K, L, G, tied, clamp, block = h[2:]
    o = I4_HEADER_BYTES

    def f32(n):
        nonlocal o
        a = np.frombuffer(raw, np.float32, n, o)
        o += 4 * n
        return a

    def mat(out, inn):
        nonlocal o
        q = np.frombuffer(raw, np.uint8, out * inn // 2, o).reshape(out, inn // 2)
        o += out * inn // 2
        s = np.frombuffer(raw, np.float32, out * inn // block, o).reshape(out, inn // block)
        o += 4 * out * inn // block
        return q, s

    layers = []
    for _ in range(L):
        d = dict(ni_g=f32(D), ni_c=f32(D), nm_g=f32(I), nm_c=f32(I), dw_t=f32(K * D).reshape(K, D))
        for k, (out, inn) in (("V", (R, D)), ("U", (2 * D, R)), ("W_z", (I, D)),
                              ("W_c", (D, I)), ("W_s_eff", (D, D))):
            d[k] = mat(out, inn)
        d["delta"] = f32(D)
        d["a_tanh"], d["b_gain"] = (float(x) for x in f32(2))
        layers.append(d)
    eps, p_floor = (float(x) for x in f32(2))
    out = dict(cfg=SunnyConfig(vocab_size=V, dim=D, inner=I, rank=R, taps=K, layers=L), group=G,
               tied=tied, clamp=clamp, block=block, layers=layers, eps=eps, p_floor=p_floor,
               no_g=f32(D), no_c=f32(D), embed=f32(V * D).reshape(V, D))
    out["head"] = mat(V, D)
    if o != len(raw):
        raise ValueError(f"INT4 blob has {len(raw) - o} trailing bytes")
    return out


def main(argv=None) -> int:
    """python -m sunnynet_amd.blob --int4 IN.bin OUT.bin [--block 32|64]:
    write the INT4 blob of an fp32 runtime blob."""
    import argparse
    ap = argparse.ArgumentParser(prog="python -m sunnynet_amd.blob")
    ap.add_argument("--int4", nargs=2, metavar=("IN", "OUT"), required=True)
    ap.add_argument("--block", type=int, default=32, choices=(32, 64))
    a = ap.parse_args(argv)
    with open(a.int4[0], "rb") as f:
        buf = f.read()
    out = convert_blob_int4(buf, a.block)
    with open(a.int4[1], "wb") as f:
        f.write(out)
    print(f"{a.int4[1]}: {len(out)} bytes (fp32 blob {len(buf)}), INT4 group {a.block}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
