"""Seeded SunnyNet weights ("random-init (seed s) per sunnynet/model.py").

Restates the reference's construction order so that the global torch RNG is
consumed exactly as ``SunnyNet(cfg)`` consumes it after
``torch.manual_seed(seed)``:

* ``nn.Embedding(V, D)`` default init                    (model.py:60)
* per block, in ``SunnyBlock.__init__`` order             (layers.py:88-135)
  ``DepthwiseCausal`` weight ``randn(D,1,K) * 0.1``       (layers.py:54)
  five ``nn.Linear`` default inits: V, U, W_z, W_c, W_s  (layers.py:112-116)
  ``_init_spectral``: ``orthogonal_spectrum_`` on V, U, W_z, W_c with rho and
  on W_s with rho/2                                        (layers.py:150-157,
                                                            init.py:10-23)
* ``nn.Linear(D, V)`` head default init, then tying       (model.py:69-71)
* ``normal_(embed, 0, 0.02)``                             (model.py:72)

Norm gains are 1, centres 0, circulant taps (0.25, 0.5, 0.25), a = b_gain =
0.5, theta = horizon_logit(D) (ops.py:62-65).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from .config import SunnyConfig


@dataclass
class SunnyLayerWeights:
    ni_g: torch.Tensor
    ni_c: torch.Tensor
    nm_g: torch.Tensor
    nm_c: torch.Tensor
    dw: torch.Tensor        # (D, 1, K)
    V: torch.Tensor         # (R, D)   nn.Linear layout (out, in)
    U: torch.Tensor         # (2D, R)
    W_z: torch.Tensor       # (I, D)
    W_c: torch.Tensor       # (D, I)
    W_s: torch.Tensor       # (D, D)
    circ: torch.Tensor      # (3,)
    theta: torch.Tensor     # (D,)
    a: torch.Tensor         # ()
    b_gain: torch.Tensor    # ()


@dataclass
class SunnyWeights:
    cfg: SunnyConfig
    embed: torch.Tensor     # (V, D); the tied head is embed itself
    layers: list = field(default_factory=list)
    no_g: torch.Tensor = None
    no_c: torch.Tensor = None
    head: torch.Tensor = None  # (V, D) when it differs from embed (quantized head)

    def delta(self, l: int) -> torch.Tensor:
        """SunnyBlock.delta (layers.py:137-141), fp32."""
        cfg = self.cfg
        span = math.log(cfg.h_max / cfg.h_min)
        H = cfg.h_min * torch.exp(span * torch.sigmoid(self.layers[l].theta))
        return 1.0 / H

    def ws_eff(self, l: int) -> torch.Tensor:
        """SunnyBlock._Ws_eff (layers.py:219-226): circ folded into W_s."""
        L = self.layers[l]
        W = L.W_s
        t0, t1, t2 = L.circ[0], L.circ[1], L.circ[2]
        return t0 * torch.roll(W, -1, dims=1) + t1 * W + t2 * torch.roll(W, 1, dims=1)

    def head_weight(self) -> torch.Tensor:
        return self.embed if self.head is None else self.head


def horizon_logit(n: int) -> torch.Tensor:
    """ops.py:62-65."""
    s = (torch.arange(n, dtype=torch.float32) + 0.5) / n
    return torch.log(s) - torch.log1p(-s)


def orthogonal_spectrum_(weight: torch.Tensor, rho: float) -> torch.Tensor:
    """init.py:10-23 with the global generator."""
    out_f, in_f = weight.shape
    n = max(out_f, in_f)
    a = torch.randn(n, n, dtype=weight.dtype, device=weight.device)
    q, r = torch.linalg.qr(a)
    sign = torch.sign(torch.diagonal(r))
    sign = torch.where(sign == 0, torch.ones_like(sign), sign)
    q = q * sign.unsqueeze(0)
    base = q[:out_f, :in_f] if out_f <= in_f else q[:, :in_f]
    with torch.no_grad():
        weight.copy_(base.mul(rho))
    return weight


@torch.no_grad()
def init_sunnynet(cfg: SunnyConfig, seed: int) -> SunnyWeights:
    """Weights of ``SunnyNet(cfg)`` right after ``torch.manual_seed(seed)``."""
    if cfg.ablation:
        raise ValueError("only the default (non-ablated) path is supported")
    nn = torch.nn
    D, I, R, K, V = cfg.dim, cfg.inner, cfg.rank, cfg.taps, cfg.vocab_size
    torch.manual_seed(seed)
    embed = nn.Embedding(V, D).weight
    layers = []
    for i in range(cfg.layers):
        dw = torch.randn(D, 1, K) * 0.1 if K > 1 else torch.ones(D, 1, 1)
        lin = [nn.Linear(D, R, bias=False), nn.Linear(R, 2 * D, bias=False),
               nn.Linear(D, I, bias=False), nn.Linear(I, D, bias=False),
               nn.Linear(D, D, bias=False)]
        theta = horizon_logit(D).clone()
        rho = cfg.rho0 * (float(i + 1) ** -cfg.decay_beta)
        for m in lin[:4]:
            orthogonal_spectrum_(m.weight, rho)
        orthogonal_spectrum_(lin[4].weight, rho * 0.5)
        layers.append(SunnyLayerWeights(
            ni_g=torch.ones(D), ni_c=torch.zeros(D), nm_g=torch.ones(I), nm_c=torch.zeros(I),
            dw=dw, V=lin[0].weight.detach().clone(), U=lin[1].weight.detach().clone(),
            W_z=lin[2].weight.detach().clone(), W_c=lin[3].weight.detach().clone(),
            W_s=lin[4].weight.detach().clone(), circ=torch.tensor([0.25, 0.5, 0.25]),
            theta=theta, a=torch.tensor(0.5), b_gain=torch.tensor(0.5)))
    nn.Linear(D, V, bias=False)          # head default init, then tied
    nn.init.normal_(embed, mean=0.0, std=0.02)
    return SunnyWeights(cfg=cfg, embed=embed.detach().clone(), layers=layers,
                        no_g=torch.ones(D), no_c=torch.zeros(D))


@torch.no_grad()
def gaussian_matmuls(w: SunnyWeights, seed: int, std: float = 0.02) -> SunnyWeights:
    """Replace every matmul weight (V, U, W_z, W_c, W_s) by N(0, std^2) draws
    from a generator seeded with `seed`; the embedding (= tied head) is already
    N(0, 0.02^2). Used for the INT4 workload."""
    g = torch.Generator().manual_seed(seed)
    for L in w.layers:
        for name in ("V", "U", "W_z", "W_c", "W_s"):
            t = getattr(L, name)
            setattr(L, name, torch.randn(t.shape, generator=g) * std)
    return w
