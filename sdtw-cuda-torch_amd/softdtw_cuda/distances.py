from __future__ import annotations

import torch
from torch.autograd import Function

from . import _engine
from ._device import compute_device, engine_dtype, to_engine


class _SqEuclideanHIP(Function):
    """D = clamp_min(|x|^2 + |y|^2 - 2 x.y^T, 0) on the GPU with the reference's fp32 bits
    (sdtw_sqeuclid_fwd_f32, exact mode); backward = the chain rule torch autograd applies to
    the reference's op sequence, clamp mask included (sdtw_sqeuclid_bwd_f32)."""

    @staticmethod
    def forward(ctx, x, y):
        D = _engine.sqeuclid_fwd(x, y, _engine.DIST_EXACT)
        ctx.save_for_backward(x, y, D)
        return D

    @staticmethod
    def backward(ctx, G):
        x, y, D = ctx.saved_tensors
        gx, gy = _engine.sqeuclid_bwd(x, y, D, G.contiguous().to(torch.float32), mask=True,
                                      need=ctx.needs_input_grad[:2])
        return gx, gy


class _SqEuclideanHIP64(Function):
    """The same distance and chain rule in double (sdtw_sqeuclid_fwd_f64 / _bwd_f64) for
    float64 inputs, which the reference computes in float64 (distances.py:20-25)."""

    @staticmethod
    def forward(ctx, x, y):
        D = _engine.sqeuclid_fwd64(x, y)
        ctx.save_for_backward(x, y, D)
        return D

    @staticmethod
    def backward(ctx, G):
        x, y, D = ctx.saved_tensors
        gx, gy = _engine.sqeuclid_bwd64(x, y, D, G.contiguous().to(torch.float64), mask=True)
        return (gx if ctx.needs_input_grad[0] else None,
                gy if ctx.needs_input_grad[1] else None)


def sqeuclidean(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """
    Squared Euclidean distance D[b,i,j] = ||x[b,i]-y[b,j]||^2, computed on the GPU as
    ||x||^2 + ||y||^2 - 2 x.y^T clamped at 0 (reference distances.py:6-28).

    x: (B,N,D), y: (B,M,D) -> (B,N,M)
    """
    if x.dim() != 3 or y.dim() != 3:
        raise ValueError(f"Expected x,y as (B,N,D)/(B,M,D). Got {tuple(x.shape)} and {tuple(y.shape)}")
    if x.shape[0] != y.shape[0] or x.shape[2] != y.shape[2]:
        raise ValueError(f"Batch/features mismatch: {tuple(x.shape)} vs {tuple(y.shape)}")
    dev = compute_device(x)
    dt = engine_dtype(x, y)
    fn = _SqEuclideanHIP64 if dt == torch.float64 else _SqEuclideanHIP
    D = fn.apply(to_engine(x, dev, dt), to_engine(y, dev, dt))
    return D.to(device=x.device, dtype=torch.promote_types(x.dtype, y.dtype))


def pairwise_distance(x: torch.Tensor, y: torch.Tensor, *, dist: str) -> torch.Tensor:
    """Reference distances.py:31-35: only the squared Euclidean cost is supported."""
    dist = dist.lower()
    if dist in ("sqeuclidean", "sq_euclidean", "squared_euclidean"):
        return sqeuclidean(x, y)
    raise ValueError(f"Unknown dist='{dist}'. Supported: 'sqeuclidean'")
