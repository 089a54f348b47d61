"""Operator-level functions with the names of the reference's launcher
(softdtw_cuda/cuda/launcher.py), implemented by the HIP engine.

Differences from the reference, by design:
  * R is the engine's table (fp32, band-skewed, see include/sdtw.h); its cells are the
    reference's R[b,i+1,j+1] (launcher.py:177), rounded once from an fp64 recursion.
    _engine.table_unpack(R, B, N, M) gives the dense (B, N, M) view.
  * The *_cpu functions do not run on the CPU: this engine has only the GPU
    implementation, so they stage D through the GPU and return tensors on D's device.
"""
from __future__ import annotations

import torch

from .. import _engine
from .._device import compute_device, to_engine


def _bw(bandwidth) -> float:
    bw = float(bandwidth)
    return -1.0 if bw <= 0 else bw


def softdtw_forward_cuda(D: torch.Tensor, gamma: float, bandwidth: float):
    """launcher.py:167-223 -> (out (B,), R)."""
    if not D.is_cuda:
        raise ValueError("Expected CUDA tensor D")
    if gamma <= 0:
        raise ValueError(f"gamma must be > 0, got {gamma}")
    return _engine.dtw_fwd(to_engine(D.detach(), D.device), float(gamma), _bw(bandwidth))


def softdtw_backward_cuda_log(D: torch.Tensor, R: torch.Tensor, gamma: float, bandwidth: float):
    """launcher.py:226-300 -> E (B,N,M) = d out / d D."""
    if not D.is_cuda:
        raise ValueError("Expected CUDA tensor D")
    if gamma <= 0:
        raise ValueError(f"gamma must be > 0, got {gamma}")
    return _engine.dtw_bwd(to_engine(D.detach(), D.device), R.contiguous(), float(gamma), _bw(bandwidth))


def softdtw_forward_cuda_fused_sqeuclid(X: torch.Tensor, Y: torch.Tensor, gamma: float, bandwidth: float):
    """launcher.py:33-87 -> (out (B,), R); no (B,N,M) cost tensor."""
    if not (X.is_cuda and Y.is_cuda):
        raise ValueError("Expected CUDA tensors X and Y")
    if X.dim() != 3 or Y.dim() != 3:
        raise ValueError(f"Expected X,Y as (B,N,D)/(B,M,D). Got {tuple(X.shape)} and {tuple(Y.shape)}")
    if X.shape[0] != Y.shape[0] or X.shape[2] != Y.shape[2]:
        raise ValueError(f"Batch/features mismatch: {tuple(X.shape)} vs {tuple(Y.shape)}")
    return _engine.fused_fwd(to_engine(X.detach(), X.device), to_engine(Y.detach(), X.device),
                             float(gamma), float(bandwidth))


def softdtw_backward_cuda_fused_sqeuclid(X: torch.Tensor, Y: torch.Tensor, R: torch.Tensor,
                                         gamma: float, bandwidth: float):
    """launcher.py:90-162 -> E (B,N,M)."""
    if not (X.is_cuda and Y.is_cuda and R.is_cuda):
        raise ValueError("Expected CUDA tensors X, Y, R")
    if X.dim() != 3 or Y.dim() != 3:
        raise ValueError(f"Expected X,Y as (B,N,D)/(B,M,D). Got {tuple(X.shape)} and {tuple(Y.shape)}")
    if X.shape[0] != Y.shape[0] or X.shape[2] != Y.shape[2]:
        raise ValueError(f"Batch/features mismatch: {tuple(X.shape)} vs {tuple(Y.shape)}")
    return _engine.fused_bwd_e(to_engine(X.detach(), X.device), to_engine(Y.detach(), X.device),
                               R.contiguous(), float(gamma), _bw(bandwidth))


def softdtw_forward_cpu(D: torch.Tensor, gamma: float, bandwidth: float):
    """launcher.py:356-361 semantics, computed by the GPU engine; returns on D's device."""
    dev = compute_device(D)
    out, R = _engine.dtw_fwd(to_engine(D.detach(), dev), float(gamma), _bw(bandwidth))
    return out.to(D.device, D.dtype), R


def softdtw_backward_cpu(D: torch.Tensor, R: torch.Tensor, gamma: float, bandwidth: float):
    """launcher.py:364-368 semantics, computed by the GPU engine; returns on D's device."""
    dev = compute_device(D)
    E = _engine.dtw_bwd(to_engine(D.detach(), dev), R, float(gamma), _bw(bandwidth))
    return E.to(D.device, D.dtype)
