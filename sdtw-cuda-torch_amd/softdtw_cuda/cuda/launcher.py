"""Operator-level functions with the names of the reference's launcher
(softdtw_cuda/cuda/launcher.py), computed by the HIP engine.

Each keeps the reference's contract:
  * torch tensors in and out; inputs are detached and made contiguous inside;
  * R is (B, N+2, M+2) in the input's dtype: R[:, 0, 0] = 0, the cells in R[:, 1:N+1, 1:M+1],
    +inf everywhere else (launcher.py:53-56, :176-178);
  * the backward functions take that R and read only its cells (the reference overwrites the
    last row and column of its working copy, launcher.py:241-245, :336-338), and return
    E = d out / d D, (B, N, M) in the input's dtype.

float64 inputs run the float64 kernels, whose R is this table already.  float32, float16 and
bfloat16 run the float32 engine; its band-skewed R table is unpacked into the dense layout
(and packed back for the backward), and results come back in the input's dtype.

The *_cpu names have the reference's CPU semantics (launcher.py:356-368) but this engine has
only the GPU implementation: CPU tensors are staged through the GPU and the results are
returned on the input's device.
"""
from __future__ import annotations

import math

import torch

from .. import _engine
from .._device import compute_device, to_engine


def _bw(bandwidth) -> float:
    bw = float(bandwidth)
    return -1.0 if bw <= 0 else bw


def _edtype(t: torch.Tensor) -> torch.dtype:
    return torch.float64 if t.dtype == torch.float64 else torch.float32


def _dense_R(out, R_engine, B, N, M, dtype):
    """(out, R) of an engine forward -> the reference's (out (B,), R (B, N+2, M+2))."""
    if R_engine.dtype == torch.float64:
        R = R_engine
    else:
        R = torch.full((B, N + 2, M + 2), math.inf, dtype=torch.float32, device=R_engine.device)
        R[:, 0, 0] = 0.0
        R[:, 1:N + 1, 1:M + 1] = _engine.table_unpack(R_engine, B, N, M)
    return out.to(dtype), R.to(dtype)


def _engine_R(R: torch.Tensor, B, N, M, dtype, device):
    """The reference's R (B, N+2, M+2) -> what the engine's backward reads."""
    if tuple(R.shape) != (B, N + 2, M + 2):
        raise ValueError(f"Expected R shape {(B, N + 2, M + 2)}, got {tuple(R.shape)}")
    if dtype == torch.float64:
        return to_engine(R.detach(), device, torch.float64)
    cells = to_engine(R.detach()[:, 1:N + 1, 1:M + 1], device, torch.float32)
    return _engine.table_pack(cells)


def _forward(D: torch.Tensor, gamma: float, bandwidth: float, dev):
    dt = _edtype(D)
    B, N, M = D.shape
    Dg = to_engine(D.detach(), dev, dt)
    fwd = _engine.dtw_fwd64 if dt == torch.float64 else _engine.dtw_fwd
    out, R = fwd(Dg, float(gamma), _bw(bandwidth))
    out, R = _dense_R(out, R, B, N, M, D.dtype)
    return out.to(D.device), R.to(D.device)


def _backward(D: torch.Tensor, R: torch.Tensor, gamma: float, bandwidth: float, dev):
    dt = _edtype(D)
    B, N, M = D.shape
    Dg = to_engine(D.detach(), dev, dt)
    Rg = _engine_R(R, B, N, M, dt, dev)
    bwd = _engine.dtw_bwd64 if dt == torch.float64 else _engine.dtw_bwd
    E = bwd(Dg, Rg, float(gamma), _bw(bandwidth))
    return E.to(device=D.device, dtype=D.dtype)


def _check_xy(X: torch.Tensor, Y: torch.Tensor):
    if X.dim() != 3 or Y.dim() != 3:
        raise ValueError(f"Expected X,Y as (B,N,D)/(B,M,D). Got {tuple(X.shape)} and {tuple(Y.shape)}")
    if X.shape[0] != Y.shape[0] or X.shape[2] != Y.shape[2]:
        raise ValueError(f"Batch/features mismatch: {tuple(X.shape)} vs {tuple(Y.shape)}")


def softdtw_forward_cuda(D: torch.Tensor, gamma: float, bandwidth: float):
    """launcher.py:167-223 -> (out (B,), R (B, N+2, M+2)), in D's dtype."""
    if not D.is_cuda:
        raise ValueError("Expected CUDA tensor D")
    if gamma <= 0:
        raise ValueError(f"gamma must be > 0, got {gamma}")
    return _forward(D, gamma, bandwidth, D.device)


def softdtw_backward_cuda_log(D: torch.Tensor, R: torch.Tensor, gamma: float, bandwidth: float):
    """launcher.py:226-300 -> E (B, N, M) = d out / d D, in D's dtype."""
    if not D.is_cuda:
        raise ValueError("Expected CUDA tensor D")
    if gamma <= 0:
        raise ValueError(f"gamma must be > 0, got {gamma}")
    return _backward(D, R, gamma, bandwidth, D.device)


def softdtw_forward_cuda_fused_sqeuclid(X: torch.Tensor, Y: torch.Tensor, gamma: float, bandwidth: float):
    """launcher.py:33-87 -> (out (B,), R (B, N+2, M+2)) in X's dtype; no (B,N,M) cost tensor
    for float32 (float64 forms the cost and runs the float64 recursion)."""
    if not (X.is_cuda and Y.is_cuda):
        raise ValueError("Expected CUDA tensors X and Y")
    _check_xy(X, Y)
    B, N, _ = X.shape
    M = Y.shape[1]
    dt = torch.float64 if torch.float64 in (X.dtype, Y.dtype) else torch.float32
    Xg = to_engine(X.detach(), X.device, dt)
    Yg = to_engine(Y.detach(), X.device, dt)
    if dt == torch.float64:
        out, R = _engine.dtw_fwd64(_engine.sqeuclid_fwd64(Xg, Yg), float(gamma), float(bandwidth))
    else:
        out, R = _engine.fused_fwd(Xg, Yg, float(gamma), float(bandwidth))
    return _dense_R(out, R, B, N, M, X.dtype)


def softdtw_backward_cuda_fused_sqeuclid(X: torch.Tensor, Y: torch.Tensor, R: torch.Tensor,
                                         gamma: float, bandwidth: float):
    """launcher.py:90-162 -> E (B, N, M) in X's dtype (costs recomputed from X, Y for
    float32)."""
    if not (X.is_cuda and Y.is_cuda and R.is_cuda):
        raise ValueError("Expected CUDA tensors X, Y, R")
    _check_xy(X, Y)
    B, N, _ = X.shape
    M = Y.shape[1]
    dt = torch.float64 if torch.float64 in (X.dtype, Y.dtype) else torch.float32
    Xg = to_engine(X.detach(), X.device, dt)
    Yg = to_engine(Y.detach(), X.device, dt)
    Rg = _engine_R(R, B, N, M, dt, X.device)
    if dt == torch.float64:
        E = _engine.dtw_bwd64(_engine.sqeuclid_fwd64(Xg, Yg), Rg, float(gamma), _bw(bandwidth))
    else:
        E = _engine.fused_bwd_e(Xg, Yg, Rg, float(gamma), _bw(bandwidth))
    return E.to(X.dtype)


def softdtw_forward_cpu(D: torch.Tensor, gamma: float, bandwidth: float):
    """launcher.py:356-361 semantics -> (out (B,), R (B, N+2, M+2)) on D's device, in D's
    dtype (computed by the GPU engine)."""
    return _forward(D, gamma, bandwidth, compute_device(D))


def softdtw_backward_cpu(D: torch.Tensor, R: torch.Tensor, gamma: float, bandwidth: float):
    """launcher.py:364-368 semantics -> E (B, N, M) on D's device, in D's dtype (computed by
    the GPU engine).  R is not modified (the reference works on a copy, :366)."""
    return _backward(D, R, gamma, bandwidth, compute_device(D))
