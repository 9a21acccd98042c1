"""Model configuration, mirroring the reference's ``SunnyConfig``.

Field names, defaults and meaning follow ``sunnynet/model.py:23-52``. The
named workloads below are the shapes this backend is measured on.
"""
from __future__ import annotations

from dataclasses import dataclass, field, replace


@dataclass
class SunnyConfig:
    """sunnynet/model.py:23-37."""

    vocab_size: int = 12000
    dim: int = 256
    inner: int = 384
    rank: int = 128
    taps: int = 4
    layers: int = 6
    scan_chunk: int = 64
    rho0: float = 1.0
    decay_beta: float = 0.0
    h_min: float = 2.0
    h_max: float = 8192.0
    tie_embeddings: bool = True
    ablation: dict = field(default_factory=dict)

    @staticmethod
    def small(vocab_size: int) -> "SunnyConfig":
        """sunnynet/model.py:39-42."""
        return SunnyConfig(vocab_size=vocab_size, dim=128, inner=192, rank=64,
                           layers=4, h_max=2048.0)

    @property
    def group(self) -> int:
        """SunnyBlock._pick_group(dim, 8) (sunnynet/layers.py:74-82)."""
        for g in (8, 4, 3):
            if g >= 3 and self.dim % g == 0:
                return g
        for g in range(3, self.dim + 1):
            if self.dim % g == 0:
                return g
        return self.dim

    @property
    def need_clamp(self) -> bool:
        """SunnyBlock._need_clamp (sunnynet/layers.py:126-129)."""
        return (1.0 - 1.0 / self.h_min) < (1.0 / self.h_max)

    def with_(self, **kw) -> "SunnyConfig":
        return replace(self, **kw)


# SunnyNet "small": SunnyConfig(vocab_size=4096, dim=256, layers=4) defaults.
SMALL = SunnyConfig(vocab_size=4096, dim=256, inner=384, rank=128, taps=4, layers=4)

# SunnyNet-100M: L=12, D=1024, V=32000 with the default ratios
# inner = 1.5 D, rank = D / 2 (102.1M parameters).
SUNNY_100M = SunnyConfig(vocab_size=32000, dim=1024, inner=1536, rank=512, taps=4,
                         layers=12)

# A tiny shape for fast CPU tests.
TINY = SunnyConfig(vocab_size=512, dim=64, inner=96, rank=32, taps=4, layers=2)

PRESETS = {"tiny": TINY, "small": SMALL, "100m": SUNNY_100M}


def param_count(cfg: SunnyConfig) -> int:
    """Parameters of SunnyNet(cfg) counted like ``num_params`` (tied head once)."""
    D, I, R, K, V = cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.vocab_size
    per_layer = (2 * D + 2 * I + (D * K if K > 1 else 0) + D * R + R * 2 * D
                 + D * I + I * D + D * D + 3 + 2 + D)
    return cfg.layers * per_layer + V * D + 2 * D


def matmul_params(cfg: SunnyConfig) -> int:
    """Weights read by one decode step's GEMVs: V, U, W_z, W_c, W_s_eff, head."""
    D, I, R, V = cfg.dim, cfg.inner, cfg.rank, cfg.vocab_size
    return cfg.layers * (D * R + R * 2 * D + D * I + I * D + D * D) + V * D
