from __future__ import annotations

import math

import torch
from torch import nn

from . import _engine
from ._device import compute_device
from .autograd import SoftDTWAutograd, SoftDTWSqEuclidAutograd
from .autograd_xy import SoftDTWNormalizedXYAutograd, SoftDTWXYAutograd
from .distances import pairwise_distance

_SQEUCLID_NAMES = ("sqeuclidean", "sq_euclidean", "squared_euclidean")


class SoftDTW(nn.Module):
    """
    Soft-DTW loss module (drop-in for the reference's softdtw_cuda.SoftDTW, module.py:12-118).

    - gamma: soft-min temperature (> 0, finite)
    - bandwidth: Sakoe-Chiba band; None or <= 0 disables it
    - normalize: SoftDTW(x,y) - 0.5*(SoftDTW(x,x)+SoftDTW(y,y)), requires N == M
    - dist: "sqeuclidean" (aliases "sq_euclidean", "squared_euclidean")
    - fused:
        None  -> fused (no (B,N,M) cost tensor) when x, y are GPU tensors on one device
        True  -> require fused (ValueError otherwise)
        False -> materialise D and differentiate through it

    Inputs (B,N,D) and (B,M,D), or unbatched (N,D)/(M,D); returns (B,).
    """

    def __init__(
        self,
        *,
        gamma: float = 1.0,
        bandwidth: float | None = None,
        normalize: bool = False,
        dist: str = "sqeuclidean",
        fused: bool | None = None,
    ):
        super().__init__()
        self.gamma = float(gamma)
        if self.gamma <= 0:
            raise ValueError(f"gamma must be > 0, got {self.gamma}")
        if not math.isfinite(self.gamma):
            raise ValueError(f"gamma must be finite, got {self.gamma}")
        if bandwidth is None:
            self.bandwidth = None
        else:
            bw = float(bandwidth)
            self.bandwidth = None if bw <= 0 else bw
        self.normalize = bool(normalize)
        self.dist = str(dist)
        self.fused = fused

    def _use_fused(self, x: torch.Tensor, y: torch.Tensor) -> bool:
        fused_ok = (
            self.dist.lower() in _SQEUCLID_NAMES
            and x.is_cuda
            and y.is_cuda
            and x.device == y.device
        )
        if self.fused is True and not fused_ok:
            raise ValueError("fused=True requires CUDA tensors and dist='sqeuclidean'.")
        if self.fused is False:
            return False
        return fused_ok

    def forward(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        if x.dim() == 2:
            x = x.unsqueeze(0)
        if y.dim() == 2:
            y = y.unsqueeze(0)
        if x.dim() != 3 or y.dim() != 3:
            raise ValueError(
                f"Expected x,y to have shape (B,N,D) and (B,M,D) (or unbatched (N,D)). "
                f"Got x={tuple(x.shape)}, y={tuple(y.shape)}"
            )
        if self.normalize and x.shape[1] != y.shape[1]:
            raise ValueError(
                f"normalize=True currently requires equal sequence lengths (N==M) because it uses the "
                f"concatenation trick. Got N={x.shape[1]}, M={y.shape[1]}."
            )
        bx, _, dx = x.shape
        by, _, dy = y.shape
        if dx != dy:
            raise ValueError(f"Feature dims must match. Got x.shape[-1]={dx}, y.shape[-1]={dy}")
        if bx != by:
            raise ValueError(f"Batch sizes must match. Got x.shape[0]={bx}, y.shape[0]={by}")
        if x.shape[1] == 0 or y.shape[1] == 0:
            raise ValueError(f"Sequence lengths must be > 0. Got N={x.shape[1]}, M={y.shape[1]}.")

        use_fused = self._use_fused(x, y)

        # CPU inputs: the unfused route runs on the GPU; results come back to x's device.
        home = x.device
        if not x.is_cuda or not y.is_cuda:
            dev = compute_device(x if x.is_cuda else y)
            x = x.to(dev)
            y = y.to(dev)

        if self.normalize and use_fused:
            # the concatenation trick below, as one autograd node (fewer host-side graph
            # nodes and launches per step; the same values)
            res = SoftDTWNormalizedXYAutograd.apply(x, y, self.gamma, self.bandwidth)
        elif self.normalize:
            x_cat = torch.cat([x, x, y], dim=0)
            y_cat = torch.cat([y, x, y], dim=0)
            out = _unfused(x_cat, y_cat, self.gamma, self.bandwidth, self.dist)
            out_xy, out_xx, out_yy = out.split(bx, dim=0)
            res = out_xy - 0.5 * (out_xx + out_yy)
        elif use_fused:
            res = SoftDTWXYAutograd.apply(x, y, self.gamma, self.bandwidth)
        else:
            res = _unfused(x, y, self.gamma, self.bandwidth, self.dist)
        return res.to(home)


def _unfused(x, y, gamma, bandwidth, dist):
    """pairwise_distance, then SoftDTWAutograd over the cost.  For float32 GPU inputs of the
    shapes where it is quicker (_engine.one_launch_unfused_forward), both forwards run in one
    launch (SoftDTWSqEuclidAutograd), with the same results."""
    if (x.dtype == torch.float32 and y.dtype == torch.float32 and x.is_cuda and y.is_cuda
            and x.device == y.device
            and dist.lower() in _SQEUCLID_NAMES
            and _engine.one_launch_unfused_forward(x.shape[0], x.shape[1], y.shape[1],
                                                   x.shape[2], x.device)):
        return SoftDTWSqEuclidAutograd.apply(x.contiguous(), y.contiguous(), gamma, bandwidth)
    D = pairwise_distance(x, y, dist=dist)
    return SoftDTWAutograd.apply(D, gamma, bandwidth)
