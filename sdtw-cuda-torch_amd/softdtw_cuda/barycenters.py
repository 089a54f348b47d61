"""
Soft-DTW barycenter averaging (Cuturi & Blondel, ICML 2017) on top of the engine.

Same algorithm and arguments as the reference (barycenters.py:17-229): weighted-mean
initialisation, Adam with a cosine-annealed learning rate, gradient-norm clipping at 1.0
and optional early stopping on absolute loss improvement.  Each iteration is one batched
Soft-DTW forward+backward over the B sequences.
"""
from __future__ import annotations

import time

import torch

from . import _engine
from .module import SoftDTW


def _cosine_lrs(lr: float, max_iter: int) -> list[float]:
    """The learning rate of each iteration: Adam(lr) under CosineAnnealingLR(T_max=max_iter,
    eta_min=0.1 lr), read off torch's own scheduler (barycenters.py:101-106)."""
    p = torch.zeros(1, requires_grad=True)
    opt = torch.optim.Adam([p], lr=lr)
    sched = torch.optim.lr_scheduler.CosineAnnealingLR(opt, T_max=max_iter, eta_min=lr * 0.1)
    out = []
    for _ in range(max_iter):
        out.append(float(opt.param_groups[0]["lr"]))
        opt.step()  # no gradient: nothing changes, but the scheduler sees a step first
        sched.step()
    return out


def _device_loop_applies(X, barycenter, weights, fused, verbose) -> bool:
    """The device loop (sdtw_barycenter_f32) runs the reference's GPU default: float32 CUDA
    tensors, the fused Soft-DTW, no progress printing."""
    return (X.is_cuda and X.dtype == torch.float32 and barycenter.dtype == torch.float32
            and weights.dtype == torch.float32 and fused in (None, True) and not verbose
            and X.dim() == 3 and X.shape[0] > 0)


def softdtw_barycenter(
    X: torch.Tensor,
    *,
    gamma: float = 1.0,
    weights: torch.Tensor | None = None,
    max_iter: int = 100,
    lr: float = 0.1,
    init: torch.Tensor | None = None,
    device: str | torch.device | None = None,
    verbose: bool = False,
    fused: bool | None = None,
    early_stopping: bool = True,
    patience: int = 10,
    tol: float = 1e-5,
) -> torch.Tensor:
    """
    Barycenter of X (B, N, D) minimising sum_b w_b * SoftDTW(barycenter, X_b).

    Returns the barycenter (N, D).  `weights` (B,) default uniform; `init` (N, D) default
    the weighted mean; `device` default X's device; `fused` as in SoftDTW; early stopping
    after `patience` iterations without an absolute improvement > `tol`, only in the
    second half of the iterations.
    """
    device = device or X.device
    X = X.to(device)
    B, N, D = X.shape

    if weights is None:
        weights = torch.ones(B, device=device) / B
    else:
        weights = weights.to(device)
        weights = weights / weights.sum()

    if init is None:
        barycenter = (X * weights.view(B, 1, 1)).sum(dim=0).clone()
    else:
        barycenter = init.clone().to(device)

    if _device_loop_applies(X, barycenter, weights, fused, verbose):
        # the whole loop on the device: the recursions on the fused kernels, the gradient sum,
        # clipping and Adam step in one kernel per iteration, the learning rates from torch's
        # own scheduler
        bary, _ = _engine.barycenter(X.contiguous(), weights.contiguous(), barycenter.contiguous(),
                                     gamma, _cosine_lrs(lr, max_iter), early_stopping, patience,
                                     tol)
        return bary

    barycenter = barycenter.requires_grad_(True)

    loss_fn = SoftDTW(gamma=gamma, normalize=False, fused=fused)
    optimizer = torch.optim.Adam([barycenter], lr=lr)
    scheduler = torch.optim.lr_scheduler.CosineAnnealingLR(optimizer, T_max=max_iter, eta_min=lr * 0.1)

    t0 = time.time()
    best_loss = float("inf")
    patience_counter = 0
    need_value = early_stopping or verbose

    for iteration in range(max_iter):
        optimizer.zero_grad()
        distances = loss_fn(barycenter.unsqueeze(0).expand(B, -1, -1), X)
        loss = (weights * distances).sum()
        loss.backward()
        torch.nn.utils.clip_grad_norm_([barycenter], max_norm=1.0)
        optimizer.step()
        scheduler.step()

        if not need_value:
            continue  # no host sync needed: nothing reads the loss
        loss_val = loss.item()
        improvement = float("nan")
        if early_stopping:
            improvement = best_loss - loss_val
            if improvement > tol:
                best_loss = loss_val
                patience_counter = 0
            else:
                patience_counter += 1
            if patience_counter >= patience and iteration > max_iter // 2:
                if verbose:
                    print(f"Early stopping at iteration {iteration + 1} "
                          f"(no improvement for {patience} iterations)")
                break
        if verbose and (iteration + 1) % 20 == 0:
            lr_val = optimizer.param_groups[0]["lr"]
            imp = f"{improvement:9.6f}" if early_stopping else "     N/A "
            print(f"Iteration {iteration + 1:3d}/{max_iter} | Loss: {loss_val:9.6f} | "
                  f"Improvement: {imp} | LR: {lr_val:.2e} | {time.time() - t0:.2f}s")

    return barycenter.detach()


def softdtw_barycenter_cpu(
    X: torch.Tensor,
    *,
    gamma: float = 1.0,
    weights: torch.Tensor | None = None,
    max_iter: int = 100,
    lr: float = 0.1,
    init: torch.Tensor | None = None,
    verbose: bool = False,
    fused: bool | None = None,
    early_stopping: bool = True,
    patience: int = 10,
    tol: float = 1e-5,
) -> torch.Tensor:
    """Barycenter with the optimisation state on the CPU (reference barycenters.py:183-229).
    The Soft-DTW evaluations themselves are staged through the GPU engine."""
    return softdtw_barycenter(
        X, gamma=gamma, weights=weights, max_iter=max_iter, lr=lr, init=init, device="cpu",
        verbose=verbose, fused=fused, early_stopping=early_stopping, patience=patience, tol=tol,
    )
