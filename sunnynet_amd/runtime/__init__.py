"""First-order recurrence on the GPU, with the reference runtime's interface.

Mirrors ``sunnynet/runtime/__init__.py:147-178``: ``scan(a, b, s0, gated)``
returns ``(out, send)`` and ``step(a, b, s, gated)`` updates ``s`` in place,
with ``s_t = a_t * s_{t-1} + b_t`` (``FMA``) or ``b_t = (1 - a_t) * u_t``
(``GATED``). Results are bit-identical to the reference C runtime.

Device (``cuda``) tensors run on torch's current stream without a host
synchronization. CPU tensors go through the host-pointer ABI (the library
copies to the GPU and back), which is the reference's calling convention.
"""
from __future__ import annotations

import torch

from .. import _native

__all__ = ["FMA", "GATED", "CoreFused", "GatedScan", "core_bwd", "core_forward", "core_fwd", "gated_scan",
           "load_runtime", "runtime_available", "scan", "scan_bwd", "step"]

FMA = 0
GATED = 1


def runtime_available() -> bool:
    return _native.available()


def load_runtime():
    return _native.lib()


def _check_f32(*ts):
    for t in ts:
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("expected contiguous float32 tensors")


def scan(a: torch.Tensor, b: torch.Tensor, s0: torch.Tensor, gated: bool = False):
    """a, b: (B,T,N); s0: (B,N) -> (out (B,T,N), send (B,N))."""
    _check_f32(a, b, s0)
    B, T, N = a.shape
    if b.shape != a.shape or s0.shape != (B, N):
        raise ValueError("shape mismatch: a, b (B,T,N); s0 (B,N)")
    if len({a.device, b.device, s0.device}) != 1:
        raise ValueError("a, b and s0 must live on one device")
    L = _native.lib()
    out = torch.empty_like(a)
    send = torch.empty_like(s0)
    g = GATED if gated else FMA
    if a.is_cuda:
        rc = L.snhip_abi_recur_scan_dev(a.data_ptr(), b.data_ptr(), s0.data_ptr(),
                                        out.data_ptr(), send.data_ptr(), B, T, N, g,
                                        _native.stream_handle(a.device))
    else:
        rc = L.snhip_abi_recur_scan(a.data_ptr(), b.data_ptr(), s0.data_ptr(),
                                    out.data_ptr(), send.data_ptr(), B, T, N, g)
    _native.check(rc, "snhip_abi_recur_scan")
    return out, send


def scan_bwd(p: torch.Tensor, nu: torch.Tensor, s0: torch.Tensor, out: torch.Tensor,
             dout: torch.Tensor):
    """Gradients of the gated scan s_t = p_t s_{t-1} + (1 - p_t) nu_t
    (sunnynet/kernels/scan_avx2.c:50-99) on the device: p, nu, out (the
    forward states), dout (B,T,N); s0 (B,N) -> (dp, dnu, ds0)."""
    _check_f32(p, nu, s0, out, dout)
    B, T, N = p.shape
    if any(t.shape != p.shape for t in (nu, out, dout)) or s0.shape != (B, N):
        raise ValueError("shape mismatch: p, nu, out, dout (B,T,N); s0 (B,N)")
    if not all(t.is_cuda for t in (p, nu, s0, out, dout)):
        raise ValueError("scan_bwd takes device tensors")
    dp, dnu, ds0 = torch.empty_like(p), torch.empty_like(p), torch.empty_like(s0)
    rc = _native.lib().snhip_abi_scan_bwd_dev(p.data_ptr(), nu.data_ptr(), s0.data_ptr(),
                                              out.data_ptr(), dout.data_ptr(), dp.data_ptr(),
                                              dnu.data_ptr(), ds0.data_ptr(), B, T, N,
                                              _native.stream_handle(p.device))
    _native.check(rc, "snhip_abi_scan_bwd_dev")
    return dp, dnu, ds0


def core_fwd(q: torch.Tensor, delta: torch.Tensor, s0: torch.Tensor):
    """The fused compete gate + decay gate + gated scan of a block
    (sunnynet/kernels/core_avx2.c:34-73) on the device: q (B,T,2D) =
    [u_raw | gate], delta (D), s0 (B,D) -> (states, u, p), each (B,T,D)."""
    _check_f32(q, delta, s0)
    if q.dim() != 3 or q.shape[2] % 2:
        raise ValueError("q must be (B,T,2D)")
    B, T, D2 = q.shape
    D = D2 // 2
    if delta.shape != (D,) or s0.shape != (B, D):
        raise ValueError("shape mismatch: q (B,T,2D), delta (D), s0 (B,D)")
    if D % 8:
        raise ValueError("the compete gate works on groups of 8 channels: D % 8 must be 0")
    if not all(t.is_cuda for t in (q, delta, s0)):
        raise ValueError("core_fwd takes device tensors")
    st, u, p = (torch.empty(B, T, D, device=q.device) for _ in range(3))
    rc = _native.lib().snhip_abi_core_fwd_dev(q.data_ptr(), delta.data_ptr(), s0.data_ptr(), st.data_ptr(),
                                              u.data_ptr(), p.data_ptr(), B, T, D,
                                              _native.stream_handle(q.device))
    _native.check(rc, "snhip_abi_core_fwd_dev")
    return st, u, p


def core_bwd(q, delta, s0, states, u, p, dstate, du_in):
    """Backward of core_fwd (sunnynet/kernels/core_avx2.c:78-149) on the
    device -> (dq (B,T,2D), ddelta (D), ds0 (B,D))."""
    _check_f32(q, delta, s0, states, u, p, dstate, du_in)
    B, T, D2 = q.shape
    D = D2 // 2
    if any(t.shape != (B, T, D) for t in (states, u, p, dstate, du_in)) or delta.shape != (D,) \
            or s0.shape != (B, D) or D % 8:
        raise ValueError("shape mismatch: q (B,T,2D); states, u, p, dstate, du_in (B,T,D); delta (D); s0 (B,D)")
    if not all(t.is_cuda for t in (q, delta, s0, states, u, p, dstate, du_in)):
        raise ValueError("core_bwd takes device tensors")
    dq = torch.empty_like(q)
    ddelta = torch.zeros(D, device=q.device)
    ds0 = torch.empty_like(s0)
    rc = _native.lib().snhip_abi_core_bwd_dev(q.data_ptr(), delta.data_ptr(), s0.data_ptr(), states.data_ptr(),
                                              u.data_ptr(), p.data_ptr(), dstate.data_ptr(), du_in.data_ptr(),
                                              dq.data_ptr(), ddelta.data_ptr(), ds0.data_ptr(), B, T, D,
                                              _native.stream_handle(q.device))
    _native.check(rc, "snhip_abi_core_bwd_dev")
    return dq, ddelta, ds0


class CoreFused(torch.autograd.Function):
    """The reference's CoreAVX2 seam (sunnynet/kernels/core_auto.py:43-74) on
    the HIP kernels: (q (B,T,2D), delta (D), s0 (B,D)) -> (u, states)."""

    @staticmethod
    def forward(ctx, q, delta, s0):
        q, delta, s0 = q.contiguous().float(), delta.contiguous().float(), s0.contiguous().float()
        st, u, p = core_fwd(q, delta, s0)
        ctx.save_for_backward(q, delta, s0, st, u, p)
        return u, st

    @staticmethod
    def backward(ctx, du, dstate):
        q, delta, s0, st, u, p = ctx.saved_tensors
        du = torch.zeros_like(u) if du is None else du.contiguous().float()
        dstate = torch.zeros_like(st) if dstate is None else dstate.contiguous().float()
        return core_bwd(q, delta, s0, st, u, p, dstate, du)


def core_forward(q: torch.Tensor, delta: torch.Tensor, s0: torch.Tensor):
    """(u, states) of the fused block core under autograd (core_auto.py:77-79)."""
    return CoreFused.apply(q, delta, s0)


class GatedScan(torch.autograd.Function):
    """The gated scan under autograd: forward is the HIP scan, backward the
    HIP scan_bwd (the seam the reference's kernels serve, core_auto.py:43-74).
    Returns (out (B,T,N), send (B,N)); send is out's last step, so its
    gradient joins dout there."""

    @staticmethod
    def forward(ctx, p, nu, s0):
        p, nu, s0 = p.contiguous(), nu.contiguous(), s0.contiguous()
        out, send = scan(p, nu, s0, gated=True)
        ctx.save_for_backward(p, nu, s0, out)
        return out, send

    @staticmethod
    def backward(ctx, dout, dsend):
        p, nu, s0, out = ctx.saved_tensors
        dout = torch.zeros_like(out) if dout is None else dout.contiguous().clone()
        if dsend is not None:
            dout[:, -1] += dsend
        return scan_bwd(p, nu, s0, out, dout)


def gated_scan(p: torch.Tensor, nu: torch.Tensor, s0: torch.Tensor):
    """Differentiable gated scan (see GatedScan)."""
    return GatedScan.apply(p, nu, s0)


def step(a: torch.Tensor, b: torch.Tensor, s: torch.Tensor, gated: bool = False):
    """a, b, s: (B,N); s updated in place and returned."""
    _check_f32(a, b, s)
    B, N = a.shape
    if b.shape != a.shape or s.shape != a.shape:
        raise ValueError("shape mismatch: a, b, s (B,N)")
    L = _native.lib()
    g = GATED if gated else FMA
    if a.is_cuda:
        rc = L.snhip_abi_recur_step_dev(a.data_ptr(), b.data_ptr(), s.data_ptr(), B, N, g,
                                        _native.stream_handle(a.device))
    else:
        rc = L.snhip_abi_recur_step(a.data_ptr(), b.data_ptr(), s.data_ptr(), B, N, g)
    _native.check(rc, "snhip_abi_recur_step")
    return s
