"""numpy statement of the 'exact' distance contract (test infrastructure).

The GPU distance kernel promises torch-CPU's fp32 bits for
clamp_min(x2 + y2 - 2*bmm(x, y^T), 0).  This module states that promise as arithmetic
(ATen's 8-lane cascade order for the row norms; a sequential FMA chain for the dot, or
multiply-then-add when K*N*M < 400), so a CPU test can check the promise against torch
itself on whatever host runs the tests.  The kernel (csrc/sdtw_device.hpp) implements the
same order; the GPU tests compare the kernel's D with torch-CPU's D bit for bit.
"""
from __future__ import annotations

import numpy as np

f32 = np.float32


def _row_sum(vals):
    """ATen row_sum<ilp=4> with the 16-row cascade, on a list of float32 (scalars or
    equal-length float32 vectors)."""
    size = len(vals)
    size_ilp = size // 4
    zero = vals[0] * f32(0)
    acc = [[zero.copy() if isinstance(zero, np.ndarray) else f32(0) for _ in range(4)] for _ in range(4)]
    i = 0
    step, mask = 16, 15
    add = lambda a, b: (a + b).astype(f32) if isinstance(a, np.ndarray) else f32(a + b)  # noqa: E731
    while i + step <= size_ilp:
        for _ in range(step):
            for k in range(4):
                acc[0][k] = add(acc[0][k], vals[i * 4 + k])
            i += 1
        for j in range(1, 4):
            for k in range(4):
                acc[j][k] = add(acc[j][k], acc[j - 1][k])
                acc[j - 1][k] = acc[j - 1][k] * f32(0)
            if i & (mask << (j * 4)):
                break
    while i < size_ilp:
        for k in range(4):
            acc[0][k] = add(acc[0][k], vals[i * 4 + k])
        i += 1
    for j in range(1, 4):
        for k in range(4):
            acc[0][k] = add(acc[0][k], acc[j][k])
    p = acc[0]
    for e in range(size_ilp * 4, size):
        p[0] = add(p[0], vals[e])
    for k in range(1, 4):
        p[0] = add(p[0], p[k])
    return p[0]


def aten_sumsq(v):
    sq = (v.astype(f32) * v.astype(f32)).astype(f32)
    K = len(sq)
    if K >= 8:
        nv = K // 8
        lanes = _row_sum([sq[c * 8:(c + 1) * 8] for c in range(nv)])
        fa = f32(0)
        for t in sq[nv * 8:]:
            fa = f32(fa + t)
        for t in lanes:
            fa = f32(fa + t)
        return fa
    return f32(f32(0) + _row_sum([f32(t) for t in sq]))


def exact_dot_matrix(a, b, muladd):
    """(N,K) x (M,K) -> (N,M): sequential chain over k from 0."""
    N, K = a.shape
    acc = np.zeros((N, b.shape[0]), dtype=f32)
    for k in range(K):
        if muladd:
            acc = (acc + (a[:, k:k + 1] * b[None, :, k]).astype(f32)).astype(f32)
        else:  # exact fma: the fp64 product of two fp32 is exact, one rounding at the end
            acc = (a[:, k:k + 1].astype(np.float64) * b[None, :, k].astype(np.float64)
                   + acc.astype(np.float64)).astype(f32)
    return acc


def exact_sqeuclid(x, y):
    """x (B,N,K), y (B,M,K) float32 numpy -> D (B,N,M) float32."""
    B, N, K = x.shape
    M = y.shape[1]
    muladd = K * N * M < 400
    out = np.empty((B, N, M), dtype=f32)
    for b in range(B):
        x2 = np.array([aten_sumsq(x[b, i]) for i in range(N)], dtype=f32)
        y2 = np.array([aten_sumsq(y[b, j]) for j in range(M)], dtype=f32)
        dot = exact_dot_matrix(x[b], y[b], muladd)
        pre = ((x2[:, None] + y2[None, :]).astype(f32) - (f32(2) * dot).astype(f32)).astype(f32)
        out[b] = np.where(pre < 0, f32(0), pre)
    return out
