"""Torch restatement of the reference's torch path — TEST INFRASTRUCTURE ONLY.

Restates ``SunnyNet.forward_step`` / ``SunnyBlock.step`` (sunnynet/model.py:113-124,
sunnynet/layers.py:287-326) and the prefill ``SunnyNet.forward`` /
``SunnyBlock.forward`` with the chunked log-space ``gated_scan``
(model.py:89-111, layers.py:256-285, ops.py:68-126) on a ``SunnyWeights``
object, in any float dtype. Used as the fp32 ``forward_step`` semantics that the
decode logits are held to (2e-5), and in fp64 as a closed-form check of the C
oracle and of step/forward equivalence.

State layout is the reference's ``SunnyState``: s (B,L,D), hist (B,L,K-1,D).
``forward_step`` treats hist[:, :, 0] as the newest entry (layers.py:64,304);
``forward`` returns hist oldest-first (layers.py:266), exactly like the
reference, and ``forward_hist_to_step`` converts between the two.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

S_MIN, EPS = 0.02, 1e-5


def _ln(x, g, c):
    """CenteredScaleNorm.forward (ops.py:45-47)."""
    return F.layer_norm(x, (x.shape[-1],), g.to(x.dtype), c.to(x.dtype), S_MIN * S_MIN + EPS)


class _Layer:
    def __init__(self, w, l, dtype):
        L = w.layers[l]
        cv = lambda t: t.detach().to(dtype)
        self.ni_g, self.ni_c, self.nm_g, self.nm_c = cv(L.ni_g), cv(L.ni_c), cv(L.nm_g), cv(L.nm_c)
        self.dw = cv(L.dw)                       # (D,1,K)
        self.V, self.U, self.W_z, self.W_c = cv(L.V), cv(L.U), cv(L.W_z), cv(L.W_c)
        W = cv(L.W_s)
        t = cv(L.circ)
        self.W_eff = t[0] * torch.roll(W, -1, dims=1) + t[1] * W + t[2] * torch.roll(W, 1, dims=1)
        self.a = cv(L.a)
        self.b_gain = cv(L.b_gain)
        cfg = w.cfg
        span = math.log(cfg.h_max / cfg.h_min)
        H = cfg.h_min * torch.exp(span * torch.sigmoid(cv(L.theta)))
        self.delta = 1.0 / H
        self.K = cfg.taps
        self.G = cfg.group
        self.D = cfg.dim


class TorchSunny:
    def __init__(self, w, dtype=torch.float32):
        self.w = w
        self.cfg = w.cfg
        self.dtype = dtype
        self.layers = [_Layer(w, l, dtype) for l in range(self.cfg.layers)]
        self.embed = w.embed.detach().to(dtype)
        self.head = w.head_weight().detach().to(dtype)
        self.no_g = w.no_g.detach().to(dtype)
        self.no_c = w.no_c.detach().to(dtype)

    def init_state(self, B: int):
        k = max(0, self.cfg.taps - 1)
        return (torch.zeros(B, self.cfg.layers, self.cfg.dim, dtype=self.dtype),
                torch.zeros(B, self.cfg.layers, k, self.cfg.dim, dtype=self.dtype))

    # ---------------------------------------------------------------- pieces
    def _compete(self, L, gate):
        """layers.py:176-182."""
        shp = gate.shape
        gg = gate.reshape(*shp[:-1], shp[-1] // L.G, L.G)
        wgt = torch.sigmoid(gg - torch.roll(gg, -1, dims=-1)) * \
            torch.sigmoid(gg - torch.roll(gg, -2, dims=-1))
        return wgt.reshape(shp)

    def _core(self, L, a):
        """layers.py:194-206 (clamp unreachable for h_min = 2)."""
        q = F.linear(F.linear(a, L.V), L.U)
        u_raw, gate = q.split(L.D, dim=-1)
        u = u_raw * self._compete(L, gate)
        p = 1.0 - L.delta * (1.0 - torch.sigmoid(gate))
        return u, gate, p

    def _readout(self, L, u):
        """layers.py:228-241: norm_mix(wedge(W_z u))."""
        z = F.linear(u, L.W_z)
        at = torch.tanh(L.a)
        return _ln(z * (1.0 + 0.5 * at / (1.0 + z.abs())), L.nm_g, L.nm_c)

    # ------------------------------------------------------------ decode step
    def block_step(self, L, x_t, s, hist):
        """layers.py:287-326 (torch path, newest-first hist)."""
        raw = _ln(x_t, L.ni_g, L.ni_c)
        k = max(0, L.K - 1)
        if k:
            acc = raw * L.dw[:, 0, L.K - 1].view(1, -1)
            for j in range(k):
                acc = acc + hist[:, j] * L.dw[:, 0, L.K - 2 - j].view(1, -1)
            a_t = raw + acc
            hist_new = torch.cat([raw[:, None, :], hist[:, :k - 1]], dim=1)
        else:
            a_t, hist_new = raw, hist
        u_t, gate, p_t = self._core(L, a_t)
        s_new = p_t * s + (1.0 - p_t) * u_t
        y = self._readout(L, u_t)
        sfb = F.linear(s, L.W_eff)
        out = F.linear(y, L.W_c) + L.b_gain * s_new + sfb + x_t
        return out, s_new, hist_new

    @torch.no_grad()
    def forward_step(self, idx_t, state):
        """model.py:113-124: idx_t (B,) -> logits (B,V), new (s, hist)."""
        s, hist = state
        x = self.embed[idx_t]
        ns, nh = torch.empty_like(s), torch.empty_like(hist)
        for i, L in enumerate(self.layers):
            x, s_i, h_i = self.block_step(L, x, s[:, i], hist[:, i])
            ns[:, i] = s_i
            nh[:, i] = h_i
        logits = F.linear(_ln(x, self.no_g, self.no_c), self.head)
        return logits, (ns, nh)

    # ------------------------------------------------------- prefill forward
    @staticmethod
    def gated_scan(p, g, s0, chunk=64, p_min_hint=None):
        """ops.py:68-102 with _safe_chunk (ops.py:115-126)."""
        T = p.shape[-2]
        p_min = float(p.min()) if p_min_hint is None else p_min_hint
        if not math.isfinite(p_min) or p_min <= 0 or p_min >= 1:
            chunk = min(chunk, 64)
        else:
            per_bit = -math.log(p_min)
            if per_bit > 0:
                chunk = max(1, min(chunk, int(64 * math.log(2.0) / per_bit)))
        nblk = (T + chunk - 1) // chunk
        pad = nblk * chunk - T
        lead, N = p.shape[:-2], p.shape[-1]
        if pad:
            p = torch.cat([p, p.new_ones(*lead, pad, N)], dim=-2)
            g = torch.cat([g, g.new_zeros(*lead, pad, N)], dim=-2)
        lp = torch.log(p).reshape(*lead, nblk, chunk, N)
        gg = g.reshape(*lead, nblk, chunk, N)
        P = torch.cumsum(lp, dim=-2)
        E = torch.exp(P)
        A = torch.cumsum(gg * torch.exp(-P), dim=-2)
        s = s0
        s_in = []
        for c in range(nblk):
            s_in.append(s)
            s = E[..., c, -1, :] * (s + A[..., c, -1, :])
        sin = torch.stack(s_in, dim=-2)
        S = (E * (sin.unsqueeze(-2) + A)).reshape(*lead, nblk * chunk, N)
        return S[..., :T, :], s

    def block_forward(self, L, x, s, hist_old_first, chunk):
        """layers.py:256-285; hist is oldest-first like the reference."""
        B, T, D = x.shape
        raw = _ln(x, L.ni_g, L.ni_c)
        k = max(0, L.K - 1)
        if k:
            rf = torch.cat([hist_old_first, raw], dim=1)
            xt = F.pad(rf.transpose(1, 2), (k, 0))                  # layers.py:56-61
            conv = F.conv1d(xt, L.dw, groups=D).transpose(1, 2)
            a = (rf + conv)[:, k:]                                   # layers.py:189-191
            hist_new = raw[:, T - k:T] if T >= k else \
                torch.cat([raw.new_zeros(B, k - T, D), raw], dim=1)
        else:
            a, hist_new = raw, hist_old_first
        c = min(chunk, T)
        u, gate, p = self._core(L, a)
        states, _ = self.gated_scan(p, (1.0 - p) * u, s, chunk=c,
                                    p_min_hint=1.0 - 1.0 / self.cfg.h_min)
        y = self._readout(L, u)
        prev = torch.cat([s[:, None, :], states[:, :-1]], dim=1)
        out = F.linear(y, L.W_c) + L.b_gain * states + F.linear(prev, L.W_eff) + x
        return out, states[:, -1], hist_new

    @torch.no_grad()
    def forward(self, idx, state=None, chunk=None):
        """model.py:89-111 with return_state=True; hist oldest-first."""
        B, T = idx.shape
        x = self.embed[idx]
        s, hist = self.init_state(B) if state is None else state
        ns, nh = torch.empty_like(s), torch.empty_like(hist)
        for i, L in enumerate(self.layers):
            x, s_i, h_i = self.block_forward(L, x, s[:, i], hist[:, i],
                                             chunk or self.cfg.scan_chunk)
            ns[:, i] = s_i
            nh[:, i] = h_i
        logits = F.linear(_ln(x, self.no_g, self.no_c), self.head)
        return logits, (ns, nh)


def forward_hist_to_step(hist):
    """Oldest-first (forward) -> newest-first (step) conv history."""
    return torch.flip(hist, dims=[-2])
