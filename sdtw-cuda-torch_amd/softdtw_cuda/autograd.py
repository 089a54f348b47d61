from __future__ import annotations

import torch
from torch.autograd import Function

from . import _engine
from ._device import compute_device, engine_dtype, to_engine
from .utils.checks import check_D


def _normalize_bandwidth(bandwidth) -> float:
    """None or <= 0 disables the band: -1.0 (reference autograd.py:19-23)."""
    if bandwidth is None:
        return -1.0
    bw = float(bandwidth)
    return -1.0 if bw <= 0 else bw


class SoftDTWAutograd(Function):
    """Soft-DTW over a materialised cost D (B,N,M) -> (B,).

    Forward: sdtw_fwd_f32 (fp64 recursion, R stored fp32 once).  Backward:
    sdtw_bwd_f32 returns grad_D = g * E directly (reference autograd.py:11-48).  A float64 D
    takes sdtw_fwd_f64 / sdtw_bwd_f64 (double throughout, as the reference's CPU path
    computes float64 inputs)."""

    @staticmethod
    def forward(ctx, D: torch.Tensor, gamma: float, bandwidth: float | None):
        check_D(D)
        gamma_f = float(gamma)
        if gamma_f <= 0:
            raise ValueError(f"gamma must be > 0, got {gamma_f}")
        bandwidth_f = _normalize_bandwidth(bandwidth)
        dev = compute_device(D)
        dt = engine_dtype(D)
        Dg = to_engine(D.detach(), dev, dt)
        fwd = _engine.dtw_fwd64 if dt == torch.float64 else _engine.dtw_fwd
        out, R = fwd(Dg, gamma_f, bandwidth_f)
        ctx.save_for_backward(Dg, R)
        ctx.gamma = gamma_f
        ctx.bandwidth = bandwidth_f
        ctx.orig = (D.device, D.dtype)
        return out.to(device=D.device, dtype=D.dtype)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        Dg, R = ctx.saved_tensors
        g = grad_output.reshape(-1).to(device=Dg.device, dtype=Dg.dtype).contiguous()
        bwd = _engine.dtw_bwd64 if Dg.dtype == torch.float64 else _engine.dtw_bwd
        G = bwd(Dg, R, ctx.gamma, ctx.bandwidth, gout=g)
        dev, dt = ctx.orig
        return G.to(device=dev, dtype=dt), None, None


class SoftDTWSqEuclidAutograd(Function):
    """Unfused mode over float32 (x, y) with both forwards in one launch: the (B,N,M) cost D
    (the bits sdtw_sqeuclid_fwd_f32 writes, from the fused forward's matrix-core producer
    waves) and the recursion over it (sdtw_fused_fwd_d_f32).  The backward is the unfused
    chain: G = g * E over D (sdtw_bwd_f32), then the distance's chain rule with the clamp
    mask (sdtw_sqeuclid_bwd_f32), which skips D for the pairs the forward recorded as free of
    clamped costs and takes the row norms the forward formed.  Same results as pairwise_distance followed by SoftDTWAutograd (reference
    distances.py:6-28, autograd.py:11-48)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, y: torch.Tensor, gamma: float, bandwidth: float | None):
        gamma_f = float(gamma)
        if gamma_f <= 0:
            raise ValueError(f"gamma must be > 0, got {gamma_f}")
        bandwidth_f = _normalize_bandwidth(bandwidth)
        out, R, D, record = _engine.fused_fwd_d(x, y, gamma_f, bandwidth_f)
        ctx.save_for_backward(x, y, D, R, record)
        ctx.gamma = gamma_f
        ctx.bandwidth = bandwidth_f
        return out

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        x, y, D, R, record = ctx.saved_tensors
        g = grad_output.reshape(-1).to(device=D.device, dtype=torch.float32).contiguous()
        G = _engine.dtw_bwd(D, R, ctx.gamma, ctx.bandwidth, gout=g)
        gx, gy = _engine.sqeuclid_bwd(x, y, D, G, mask=True, need=ctx.needs_input_grad[:2],
                                      record=record)
        return gx, gy, None, None
