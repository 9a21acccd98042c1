"""RWKV-7 configurations, seeded weights and the v3 runtime blob.

The blob is the format the reference's C runtime reads (``sn_rk_load``,
sunnynet/runtime/rwkv7.c:376-508), written the way
experiments/_export_rwkv7.py:3-19,43-148 writes it from a GGUF file:

* header: 10 int32 ``magic 0x4B57524B, version 3, layers, dim, head_size,
  n_head, ff, max g-rank, vocab, int4 flag``; then ``eps`` (float32) and the
  rank table ``layers x (Rw, Ra, Rv, Rg)`` (int32);
* a stream of tensors, each preceded by an int32 tag: 0 = fp32, stored as the
  transpose ``M^T`` (``(len(x), len(y))`` row-major for ``y = M x``); 1 =
  INT4, ``M`` quantized along its input (quant.c format, group 64: codes
  ``(out, in/2)`` bytes, then scales ``(out, in/64)`` float32). A matrix is
  INT4 only when its input length is a multiple of 64 (_export_rwkv7.py:85-88);
  vectors and the embedding table stay fp32;
* per layer ``ln1 ln1.b ln2 ln2.b lerp(6, D)``, ``r k v o`` (D, D),
  ``w1 w2 a1 a2 v1 v2 g1 g2`` (LoRA pairs D->R->D), ``w0 a0 v0 kk ka rk lnx_w
  lnx_b`` (D each), ``cmk`` (D->F), ``cmv`` (F->D), ``cmk_lerp`` (D); then
  ``en en.b on on.b`` (D), ``embed`` (vocab, D), ``head`` (D->vocab).

No reference initialisation exists for RWKV-7 (weights come from a GGUF
file), so ``init_rwkv7`` draws documented synthetic weights of the model's
shape from a seeded generator.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

__all__ = ["RwkvConfig", "RwkvWeights", "RWKV_TINY", "RWKV_CFG4", "init_rwkv7",
           "quant_i4_np", "dequant_i4_np", "pack_rwkv7_blob", "RK_MAGIC", "RK_VERSION",
           "RK_BLOCK"]

RK_MAGIC = 0x4B57524B
RK_VERSION = 3
RK_BLOCK = 64          # INT4 group of the v3 format (rwkv7.c: SN_Q4_BLOCK)


@dataclass(frozen=True)
class RwkvConfig:
    layers: int
    dim: int
    head_size: int
    ff: int
    vocab: int
    ranks: tuple = (64, 64, 32, 128)   # (Rw, Ra, Rv, Rg)
    eps: float = 1e-5

    @property
    def n_head(self) -> int:
        return self.dim // self.head_size

    def matmul_params(self) -> int:
        D, F, V = self.dim, self.ff, self.vocab
        Rw, Ra, Rv, Rg = self.ranks
        per = 4 * D * D + 2 * D * (Rw + Ra + Rv + Rg) + 2 * D * F
        return self.layers * per + D * V


# A small model for parity tests, and the 12-layer 768-wide configuration
# the decode benchmark runs (12 heads of 64, ff 3072, vocab 65536).
RWKV_TINY = RwkvConfig(layers=2, dim=128, head_size=64, ff=256, vocab=512, ranks=(64, 64, 32, 64))
RWKV_CFG4 = RwkvConfig(layers=12, dim=768, head_size=64, ff=3072, vocab=65536,
                       ranks=(64, 64, 32, 128))


@dataclass
class RwkvWeights:
    """Logical matrices M (out, in) with y = M x; vectors (n,)."""
    cfg: RwkvConfig
    layers: list            # dicts of the per-layer tensors
    en_w: np.ndarray
    en_b: np.ndarray
    on_w: np.ndarray
    on_b: np.ndarray
    embed: np.ndarray       # (vocab, D)
    head: np.ndarray        # (vocab, D)


def init_rwkv7(cfg: RwkvConfig, seed: int) -> RwkvWeights:
    """Synthetic weights (numpy PCG64, seed): matrices N(0, 1/in) scaled
    so activations stay O(1); LayerNorm gains 1 + N(0, 0.1), biases
    N(0, 0.05); token-shift mixes U(0, 1); decay bias w0 ~ U(-3, 1)."""
    rng = np.random.default_rng(seed)
    D, F, V = cfg.dim, cfg.ff, cfg.vocab
    Rw, Ra, Rv, Rg = cfg.ranks
    f32 = np.float32

    def mat(out, inp, gain=1.0):
        return (rng.standard_normal((out, inp)) * (gain / np.sqrt(inp))).astype(f32)

    def vec(n, mean=0.0, std=1.0):
        return (mean + std * rng.standard_normal(n)).astype(f32)

    layers = []
    for _ in range(cfg.layers):
        L = {
            "ln1_w": vec(D, 1.0, 0.1), "ln1_b": vec(D, 0.0, 0.05),
            "ln2_w": vec(D, 1.0, 0.1), "ln2_b": vec(D, 0.0, 0.05),
            "lerp": rng.random((6, D)).astype(f32),
            "r": mat(D, D), "k": mat(D, D), "v": mat(D, D), "o": mat(D, D, 0.5),
            "w1": mat(Rw, D), "w2": mat(D, Rw, 0.5),
            "a1": mat(Ra, D), "a2": mat(D, Ra, 0.5),
            "v1": mat(Rv, D), "v2": mat(D, Rv, 0.5),
            "g1": mat(Rg, D), "g2": mat(D, Rg, 0.5),
            "w0": rng.uniform(-3.0, 1.0, D).astype(f32),
            "a0": vec(D, 0.0, 0.5), "v0": vec(D, 0.0, 0.5),
            "kk": rng.uniform(0.5, 1.5, D).astype(f32), "ka": rng.random(D).astype(f32),
            "rk": vec(D, 0.0, 0.1),
            "lnx_w": vec(D, 1.0, 0.1), "lnx_b": vec(D, 0.0, 0.05),
            "cmk": mat(F, D), "cmv": mat(D, F, 0.5),
            "cmk_lerp": rng.random(D).astype(f32),
        }
        layers.append(L)
    return RwkvWeights(cfg=cfg, layers=layers,
                       en_w=vec(D, 1.0, 0.1), en_b=vec(D, 0.0, 0.05),
                       on_w=vec(D, 1.0, 0.1), on_b=vec(D, 0.0, 0.05),
                       embed=rng.standard_normal((V, D)).astype(f32),
                       head=mat(V, D))


def quant_i4_np(x: np.ndarray, block: int):
    """sunnynet/runtime/quant.c:34-66 in float32 numpy: per group of `block`
    along each row, scale = amax / 7 (1 when amax is 0), q = clamp(rint(w *
    (1 / scale)), -8, 7) + 8; byte k of a group = q[k] | q[k + block/2] << 4.
    Returns (codes (rows, N/2) uint8, scales (rows, N/block) float32)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, N = x.shape
    if N % block or block % 2:
        raise ValueError("row length must be a multiple of an even block")
    g = x.reshape(rows, N // block, block)
    amax = np.abs(g).max(axis=2)
    scale = (amax / np.float32(7.0)).astype(np.float32)
    scale[amax == 0] = np.float32(1.0)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    q = np.rint((g * inv[:, :, None]).astype(np.float32))
    q = (np.clip(q, -8, 7) + 8).astype(np.uint8)
    half = block // 2
    codes = (q[:, :, :half] | (q[:, :, half:] << 4)).astype(np.uint8)
    return codes.reshape(rows, N // 2), scale


def dequant_i4_np(codes: np.ndarray, scale: np.ndarray, N: int, block: int) -> np.ndarray:
    rows = codes.shape[0]
    half = block // 2
    c = codes.reshape(rows, N // block, half)
    lo = (c & 0x0F).astype(np.int32) - 8
    hi = (c >> 4).astype(np.int32) - 8
    q = np.concatenate([lo, hi], axis=2).astype(np.float32)
    return (q * scale[:, :, None]).reshape(rows, N).astype(np.float32)


def pack_rwkv7_blob(w: RwkvWeights, int4: bool = False, ranks=None) -> bytes:
    """The v3 blob of `w` (fp32, or INT4 group 64 where allowed). `ranks`:
    per-layer (Rw, Ra, Rv, Rg), default cfg.ranks for every layer; the header
    holds the largest Rg (_export_rwkv7.py:73-79)."""
    cfg = w.cfg
    L, D, HS, NH, F, V = cfg.layers, cfg.dim, cfg.head_size, cfg.n_head, cfg.ff, cfg.vocab
    ranks = [tuple(cfg.ranks)] * L if ranks is None else [tuple(r) for r in ranks]
    parts = [struct.pack("<10i", RK_MAGIC, RK_VERSION, L, D, HS, NH, F, max(r[3] for r in ranks), V,
                         1 if int4 else 0),
             struct.pack("<f", cfg.eps)]
    for r in ranks:
        parts.append(struct.pack("<4i", *r))

    def vecs(a):
        parts.append(struct.pack("<i", 0))
        parts.append(np.ascontiguousarray(a, np.float32).tobytes())

    def mat(M):   # M (out, in): y = M x
        out, inp = M.shape
        if int4 and inp % RK_BLOCK == 0:
            q, s = quant_i4_np(M, RK_BLOCK)
            parts.append(struct.pack("<i", 1))
            parts.append(q.tobytes() + s.astype(np.float32).tobytes())
        else:
            parts.append(struct.pack("<i", 0))
            parts.append(np.ascontiguousarray(M.T, np.float32).tobytes())

    for Ld in w.layers:
        for k in ("ln1_w", "ln1_b", "ln2_w", "ln2_b", "lerp"):
            vecs(Ld[k])
        for k in ("r", "k", "v", "o", "w1", "w2", "a1", "a2", "v1", "v2", "g1", "g2"):
            mat(Ld[k])
        for k in ("w0", "a0", "v0", "kk", "ka", "rk", "lnx_w", "lnx_b"):
            vecs(Ld[k])
        mat(Ld["cmk"])
        mat(Ld["cmv"])
        vecs(Ld["cmk_lerp"])
    for a in (w.en_w, w.en_b, w.on_w, w.on_b, w.embed):
        vecs(a)
    mat(w.head)
    return b"".join(parts)
