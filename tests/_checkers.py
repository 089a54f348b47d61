"""Independent checkers for the Soft-DTW oracle (test infrastructure).

None of these reuse the oracle's recursion:
  * brute_force(): enumerates every monotone alignment path (steps (1,0), (0,1), (1,1))
    and evaluates  -gamma * log sum_paths exp(-cost(path)/gamma)  and the path marginals
    E_ij = P(path visits (i,j)) in float64 -- the definition of Soft-DTW and of its gradient
    dR/dD (Cuturi & Blondel 2017), not a recursion;
  * torch_dp64(): an autograd-differentiable float64 recursion written with torch.logsumexp
    (a different formula and evaluation order from the reference's max-shifted exp/log);
  * hard_dtw(): textbook DTW with min (the gamma -> 0 limit).
"""
from __future__ import annotations

import math

import numpy as np
import torch


def _in_band(bw, i, j):
    return bw is None or bw <= 0 or abs(i - j) <= bw


def enumerate_paths(N, M):
    out = []

    def rec(i, j, acc):
        acc.append((i, j))
        if i == N - 1 and j == M - 1:
            out.append(list(acc))
        else:
            if i + 1 < N:
                rec(i + 1, j, acc)
            if j + 1 < M:
                rec(i, j + 1, acc)
            if i + 1 < N and j + 1 < M:
                rec(i + 1, j + 1, acc)
        acc.pop()

    rec(0, 0, [])
    return out


def brute_force(D, gamma, bandwidth=None):
    """Soft-DTW value and path marginals of one (N, M) cost matrix, float64."""
    D = np.asarray(D, dtype=np.float64)
    N, M = D.shape
    paths = [p for p in enumerate_paths(N, M) if all(_in_band(bandwidth, i, j) for i, j in p)]
    if not paths:
        return math.inf, np.zeros((N, M))
    costs = np.array([math.fsum(D[i, j] for i, j in p) for p in paths])
    z = -costs / gamma
    zmax = z.max()
    w = np.exp(z - zmax)
    val = -gamma * (math.log(w.sum()) + zmax)
    w /= w.sum()
    E = np.zeros((N, M))
    for wk, p in zip(w, paths):
        for i, j in p:
            E[i, j] += wk
    return val, E


def torch_dp64(D, gamma, bandwidth=None):
    """Differentiable float64 Soft-DTW of one (N, M) cost tensor via torch.logsumexp."""
    N, M = D.shape
    inf = torch.tensor(math.inf, dtype=torch.float64)
    zero = torch.tensor(0.0, dtype=torch.float64)
    R = [[inf] * (M + 1) for _ in range(N + 1)]
    R[0][0] = zero
    for i in range(1, N + 1):
        for j in range(1, M + 1):
            if not _in_band(bandwidth, i, j):
                continue
            prev = torch.stack([R[i - 1][j - 1], R[i - 1][j], R[i][j - 1]])
            R[i][j] = D[i - 1, j - 1] - gamma * torch.logsumexp(-prev / gamma, dim=0)
    return R[N][M], R


def hard_dtw(D):
    D = np.asarray(D, dtype=np.float64)
    N, M = D.shape
    R = np.full((N + 1, M + 1), np.inf)
    R[0, 0] = 0.0
    for i in range(1, N + 1):
        for j in range(1, M + 1):
            R[i, j] = D[i - 1, j - 1] + min(R[i - 1, j - 1], R[i - 1, j], R[i, j - 1])
    return R[N, M]
