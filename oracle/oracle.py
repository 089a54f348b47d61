"""CPU restatement of the reference's CPU Soft-DTW path -- TEST INFRASTRUCTURE ONLY.

The reference (BGU-CS-VIL/sdtw-cuda-torch) runs its CPU path as
    distances.py:6-28      D = clamp_min(x2 + y2 - 2*bmm(x, y^T), 0) with torch CPU ops
    autograd.py:11-48      SoftDTWAutograd: bandwidth normalisation, grad_D = g * E
    launcher.py:356-368    softdtw_forward_cpu / softdtw_backward_cpu (numba loops)
    launcher.py:307-353    the numba loops themselves -> restated in C in sdtw_oracle.c
    module.py:71-123       validation, 2-D promotion, normalize concat trick
    barycenters.py:17-229  Adam + cosine schedule + clipping barycenter loop

This module rebuilds that path on CPU tensors: the distance uses the same torch CPU ops
(so its bits equal the reference's on the same host), the DP is the C restatement, and the
gradient through the distance comes from torch autograd exactly as in the reference.

Parity status of each function (what pins it) is listed in tests/test_oracle.py and in the
repository's design notes; nothing here is shipped.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libsdtw_oracle.so")
_lib = None
_lock = threading.Lock()


def load_library(rebuild: bool = False):
    """Load (building with make if needed) the C oracle library."""
    global _lib
    with _lock:
        if _lib is not None and not rebuild:
            return _lib
        if rebuild or not os.path.exists(_LIB_PATH):
            subprocess.run(["make", "-s", "-C", _HERE], check=True)
        lib = ctypes.CDLL(_LIB_PATH)
        i64, dbl, vp, cint = ctypes.c_int64, ctypes.c_double, ctypes.c_void_p, ctypes.c_int
        for name in ("sdtw_oracle_forward_f32", "sdtw_oracle_forward_f64"):
            fn = getattr(lib, name)
            fn.argtypes = [vp, vp, i64, i64, i64, dbl, dbl, cint]
            fn.restype = cint
        for name in ("sdtw_oracle_backward_f32", "sdtw_oracle_backward_f64"):
            fn = getattr(lib, name)
            fn.argtypes = [vp, vp, vp, i64, i64, i64, dbl, dbl, cint]
            fn.restype = cint
        _lib = lib
        return lib


def _nthreads(nthreads):
    if nthreads is not None and nthreads > 0:
        return int(nthreads)
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def sqeuclidean(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Squared-Euclidean cost on CPU with the reference's torch op sequence
    (distances.py:20-28): row norms by sum of squares, batched x.y^T, broadcast
    x2 + y2 - 2*xy, clamped at zero.  Same ops => same bits on the same host."""
    xn = (x * x).sum(dim=-1)
    yn = (y * y).sum(dim=-1)
    cross = torch.bmm(x, y.transpose(1, 2))
    return (xn.unsqueeze(2) + yn.unsqueeze(1) - 2.0 * cross).clamp_min(0.0)


def _bw(bandwidth) -> float:
    """autograd.py:19-23: None or <= 0 disables the band (-1.0)."""
    if bandwidth is None:
        return -1.0
    bw = float(bandwidth)
    return -1.0 if bw <= 0 else bw


def forward(D: torch.Tensor, gamma: float, bandwidth, nthreads=None, return_r64=False):
    """launcher.py:356-361 -> (out (B,), R (B,N+2,M+2) in D's dtype[, R64])."""
    lib = load_library()
    D_ = D.detach().cpu().contiguous()
    if D_.dtype == torch.float32:
        fn = lib.sdtw_oracle_forward_f32
    elif D_.dtype == torch.float64:
        fn = lib.sdtw_oracle_forward_f64
    else:
        raise TypeError(f"oracle supports float32/float64 D, got {D_.dtype}")
    B, N, M = D_.shape
    R64 = torch.empty((B, N + 2, M + 2), dtype=torch.float64)
    rc = fn(D_.data_ptr(), R64.data_ptr(), B, N, M, float(gamma), _bw(bandwidth), _nthreads(nthreads))
    if rc != 0:
        raise RuntimeError(f"oracle forward failed rc={rc}")
    R = R64.to(D_.dtype)  # launcher.py:359 `.type_as(D)`: one rounding of the fp64 table
    out = R[:, -2, -2].contiguous()
    if return_r64:
        return out, R, R64
    return out, R


def backward(D: torch.Tensor, R: torch.Tensor, gamma: float, bandwidth, nthreads=None):
    """launcher.py:364-368 -> E (B,N,M) in D's dtype.  R is copied first (launcher.py:366)."""
    lib = load_library()
    D_ = D.detach().cpu().contiguous()
    R_ = R.detach().cpu().to(D_.dtype).contiguous().clone()
    if D_.dtype == torch.float32:
        fn = lib.sdtw_oracle_backward_f32
    elif D_.dtype == torch.float64:
        fn = lib.sdtw_oracle_backward_f64
    else:
        raise TypeError(f"oracle supports float32/float64 D, got {D_.dtype}")
    B, N, M = D_.shape
    if tuple(R_.shape) != (B, N + 2, M + 2):
        raise ValueError(f"Expected R shape {(B, N + 2, M + 2)}, got {tuple(R_.shape)}")
    E = torch.empty((B, N, M), dtype=D_.dtype)
    rc = fn(D_.data_ptr(), R_.data_ptr(), E.data_ptr(), B, N, M, float(gamma), _bw(bandwidth),
            _nthreads(nthreads))
    if rc != 0:
        raise RuntimeError(f"oracle backward failed rc={rc}")
    return E


class OracleSoftDTWFunction(torch.autograd.Function):
    """autograd.py:11-48 on CPU: saves D and R, backward returns g * E."""

    @staticmethod
    def forward(ctx, D, gamma, bandwidth, nthreads=None):
        out, R = forward(D, gamma, bandwidth, nthreads)
        ctx.save_for_backward(D, R)
        ctx.gamma = float(gamma)
        ctx.bandwidth = bandwidth
        ctx.nthreads = nthreads
        return out

    @staticmethod
    def backward(ctx, grad_output):
        D, R = ctx.saved_tensors
        E = backward(D, R, ctx.gamma, ctx.bandwidth, ctx.nthreads)
        g = grad_output.reshape(-1).to(dtype=E.dtype).view(-1, 1, 1)
        return g * E, None, None, None


def softdtw(x, y, gamma=1.0, bandwidth=None, normalize=False, nthreads=None):
    """module.py:71-123 on CPU (the reference's unfused CPU route)."""
    if x.dim() == 2:
        x = x.unsqueeze(0)
    if y.dim() == 2:
        y = y.unsqueeze(0)
    bw = None
    if bandwidth is not None and float(bandwidth) > 0:
        bw = float(bandwidth)
    if normalize:
        bx = x.shape[0]
        xc = torch.cat([x, x, y], dim=0)
        yc = torch.cat([y, x, y], dim=0)
        out = OracleSoftDTWFunction.apply(sqeuclidean(xc, yc), float(gamma), bw, nthreads)
        oxy, oxx, oyy = out.split(bx, dim=0)
        return oxy - 0.5 * (oxx + oyy)
    return OracleSoftDTWFunction.apply(sqeuclidean(x, y), float(gamma), bw, nthreads)


def barycenter(X, gamma=1.0, weights=None, max_iter=100, lr=0.1, init=None,
               early_stopping=True, patience=10, tol=1e-5, nthreads=None, history=None):
    """barycenters.py:17-180 on CPU with the oracle loss.  ``history`` (a list) receives
    (loss, barycenter-after-step) per iteration for step-wise parity checks."""
    X = X.detach().cpu()
    B, N, D = X.shape
    if weights is None:
        w = torch.ones(B) / B
    else:
        w = weights.detach().cpu()
        w = w / w.sum()
    if init is None:
        bary = (X * w.view(B, 1, 1)).sum(dim=0).clone()
    else:
        bary = init.detach().cpu().clone()
    bary.requires_grad_(True)
    opt = torch.optim.Adam([bary], lr=lr)
    sched = torch.optim.lr_scheduler.CosineAnnealingLR(opt, T_max=max_iter, eta_min=lr * 0.1)
    best = float("inf")
    wait = 0
    for it in range(max_iter):
        opt.zero_grad()
        d = softdtw(bary.unsqueeze(0).expand(B, -1, -1), X, gamma=gamma, nthreads=nthreads)
        loss = (w * d).sum()
        loss.backward()
        torch.nn.utils.clip_grad_norm_([bary], max_norm=1.0)
        opt.step()
        sched.step()
        lv = loss.item()
        if history is not None:
            history.append((lv, bary.detach().clone()))
        if early_stopping:
            if best - lv > tol:
                best = lv
                wait = 0
            else:
                wait += 1
            if wait >= patience and it > max_iter // 2:
                break
    return bary.detach()


def _selftest():  # pragma: no cover - manual use
    torch.manual_seed(0)
    x = torch.randn(2, 5, 3)
    y = torch.randn(2, 4, 3)
    print(softdtw(x, y))


if __name__ == "__main__":  # pragma: no cover
    _selftest()
