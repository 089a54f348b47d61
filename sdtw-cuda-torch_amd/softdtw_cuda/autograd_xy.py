from __future__ import annotations

import torch
from torch.autograd import Function

from . import _engine
from ._device import engine_dtype, to_engine
from .autograd import _normalize_bandwidth


class SoftDTWXYAutograd(Function):
    """Fused Soft-DTW over (X, Y) with the squared-Euclidean cost recomputed per cell; no
    (B,N,M) cost tensor is formed (reference autograd_xy.py:12-51).

    Forward: sdtw_fused_fwd_f32.  Backward: sdtw_fused_bwd_f32 returns
    grad_X = 2 (X * sum_j gE - gE Y), grad_Y = 2 (Y * sum_i gE - gE^T X), gE = g * E.
    float64 X, Y take the float64 kernels: the cost is formed (sdtw_sqeuclid_fwd_f64), the
    recursions run on it (sdtw_fwd_f64 / sdtw_bwd_f64), and the same chain rule without a
    clamp mask gives the gradients (sdtw_sqeuclid_bwd_f64, mask 0)."""

    @staticmethod
    def forward(ctx, X: torch.Tensor, Y: torch.Tensor, gamma: float, bandwidth: float | None):
        if not (X.is_cuda and Y.is_cuda):
            raise ValueError("Expected CUDA tensors X and Y")
        if X.dim() != 3 or Y.dim() != 3:
            raise ValueError(f"Expected X,Y as (B,N,D)/(B,M,D). Got {tuple(X.shape)} and {tuple(Y.shape)}")
        if X.shape[0] != Y.shape[0] or X.shape[2] != Y.shape[2]:
            raise ValueError(f"Batch/features mismatch: {tuple(X.shape)} vs {tuple(Y.shape)}")
        gamma_f = float(gamma)
        if not gamma_f > 0:
            raise ValueError(f"gamma must be > 0, got {gamma_f}")
        dt = engine_dtype(X, Y)
        Xg = to_engine(X.detach(), X.device, dt)
        Yg = to_engine(Y.detach(), X.device, dt)
        # forward takes the band as given (-1 for None), the backward normalised
        # (reference autograd_xy.py:16, :22-27); both disable it for values <= 0.
        bw_fwd = -1.0 if bandwidth is None else float(bandwidth)
        if dt == torch.float64:
            D = _engine.sqeuclid_fwd64(Xg, Yg)
            out, R = _engine.dtw_fwd64(D, gamma_f, bw_fwd)
            ctx.save_for_backward(Xg, Yg, R, D)
        else:
            out, R = _engine.fused_fwd(Xg, Yg, gamma_f, bw_fwd)
            ctx.save_for_backward(Xg, Yg, R)
        ctx.gamma = gamma_f
        ctx.bandwidth = _normalize_bandwidth(bandwidth)
        ctx.dtypes = (X.dtype, Y.dtype)
        return out.to(dtype=X.dtype)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        Xg, Yg, R = ctx.saved_tensors[:3]
        g = grad_output.reshape(-1).to(device=Xg.device, dtype=Xg.dtype).contiguous()
        need = ctx.needs_input_grad[:2]
        if Xg.dtype == torch.float64:
            D = ctx.saved_tensors[3]
            G = _engine.dtw_bwd64(D, R, ctx.gamma, ctx.bandwidth, gout=g)
            gx, gy = _engine.sqeuclid_bwd64(Xg, Yg, None, G, mask=False)
        else:
            # only the gradients autograd asks for (a barycenter's sequences need none)
            gx, gy = _engine.fused_bwd(Xg, Yg, R, ctx.gamma, ctx.bandwidth, gout=g, need=need)
        dx, dy = ctx.dtypes
        return (gx.to(dtype=dx) if need[0] else None, gy.to(dtype=dy) if need[1] else None,
                None, None)


class SoftDTWNormalizedXYAutograd(Function):
    """Fused normalised Soft-DTW, sdtw(X,Y) - (sdtw(X,X) + sdtw(Y,Y)) / 2, as one autograd
    node: the reference's concatenation trick (module.py:101-111: the 3B pairs [X,X,Y] vs
    [Y,X,Y] in one fused call) with the three-way split, the combination and, in the backward,
    the per-pair upstream gradients (g, -g/2, -g/2) and the sums of each input's three
    appearances formed here instead of by separate graph nodes.  The values are the same
    operations as the reference's expression: out_xy - 0.5 * (out_xx + out_yy) forward, and
    0.5 * (-g) for the self terms backward."""

    @staticmethod
    def forward(ctx, X: torch.Tensor, Y: torch.Tensor, gamma: float, bandwidth: float | None):
        if not (X.is_cuda and Y.is_cuda):
            raise ValueError("Expected CUDA tensors X and Y")
        if X.dim() != 3 or Y.dim() != 3 or X.shape != Y.shape:
            raise ValueError(f"Expected X,Y as (B,N,D) of one shape. Got {tuple(X.shape)} and {tuple(Y.shape)}")
        gamma_f = float(gamma)
        if not gamma_f > 0:
            raise ValueError(f"gamma must be > 0, got {gamma_f}")
        B = X.shape[0]
        dt = engine_dtype(X, Y)
        Xg = to_engine(X.detach(), X.device, dt)
        Yg = to_engine(Y.detach(), X.device, dt)
        Xc = torch.cat((Xg, Xg, Yg), dim=0)
        Yc = torch.cat((Yg, Xg, Yg), dim=0)
        bw_fwd = -1.0 if bandwidth is None else float(bandwidth)
        if dt == torch.float64:
            D = _engine.sqeuclid_fwd64(Xc, Yc)
            out, R = _engine.dtw_fwd64(D, gamma_f, bw_fwd)
            ctx.save_for_backward(Xc, Yc, R, D)
        else:
            out, R = _engine.fused_fwd(Xc, Yc, gamma_f, bw_fwd)
            ctx.save_for_backward(Xc, Yc, R)
        ctx.gamma = gamma_f
        ctx.bandwidth = _normalize_bandwidth(bandwidth)
        ctx.dtypes = (X.dtype, Y.dtype)
        ctx.B = B
        o = out.view(3, B)
        res = o[0] - 0.5 * (o[1] + o[2])
        return res.to(dtype=X.dtype)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        Xc, Yc, R = ctx.saved_tensors[:3]
        B = ctx.B
        g = grad_output.reshape(-1).to(device=Xc.device, dtype=Xc.dtype)
        h = 0.5 * (-g)
        gout = torch.cat((g, h, h)).contiguous()
        need = ctx.needs_input_grad[:2]
        if Xc.dtype == torch.float64:
            D = ctx.saved_tensors[3]
            G = _engine.dtw_bwd64(D, R, ctx.gamma, ctx.bandwidth, gout=gout)
            gx, gy = _engine.sqeuclid_bwd64(Xc, Yc, None, G, mask=False)
        else:
            gx, gy = _engine.fused_bwd(Xc, Yc, R, ctx.gamma, ctx.bandwidth, gout=gout,
                                       need=(True, True))
        gx = gx.view(3, B, *gx.shape[1:])
        gy = gy.view(3, B, *gy.shape[1:])
        dx, dy = ctx.dtypes
        # X appears as pairs 0 and 1 of the first argument and pair 1 of the second, Y as
        # pair 0 of the second and pair 2 of both
        gX = (gx[0] + gx[1] + gy[1]).to(dtype=dx) if need[0] else None
        gY = (gy[0] + gx[2] + gy[2]).to(dtype=dy) if need[1] else None
        return gX, gY, None, None
