"""Helpers shared by the GPU parity tests (test infrastructure)."""
from __future__ import annotations

import math
import sys

import torch

# forward rtol 1e-5; gradients rtol 1e-4 / atol 1e-5
FWD_RTOL = 1e-5
GRAD_RTOL = 1e-4
GRAD_ATOL = 1e-5


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def randn_pair(B, N, M, K, seed=0):
    """Seeded CPU inputs (x drawn before y), as in the reference benchmark."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, N, K, generator=g)
    y = torch.randn(B, M, K, generator=g)
    return x, y


def sinusoid_pair(B, N, K, seed=0):
    """Config-4 inputs: a*sin(f t + phi) + 0.1*noise, f~U[0.5,3], phi~U[0,2pi], a~U[0.5,2]."""
    g = torch.Generator().manual_seed(seed)
    t = torch.linspace(0, 2 * math.pi, N)

    def draw():
        f = 0.5 + 2.5 * torch.rand(B, 1, K, generator=g)
        ph = 2 * math.pi * torch.rand(B, 1, K, generator=g)
        a = 0.5 + 1.5 * torch.rand(B, 1, K, generator=g)
        return a * torch.sin(f * t.view(1, N, 1) + ph) + 0.1 * torch.randn(B, N, K, generator=g)

    return draw(), draw()


def random_walks(Kseq, N, D, seed=0):
    """Config-5 inputs: cumsum of N(0, 0.1) plus a shared sinusoid template."""
    g = torch.Generator().manual_seed(seed)
    n = torch.arange(N, dtype=torch.float32).view(N, 1)
    d = torch.arange(D, dtype=torch.float32).view(1, D)
    template = torch.sin(2 * math.pi * n / N * (d + 1) * 0.5)
    return torch.cumsum(0.1 * torch.randn(Kseq, N, D, generator=g), dim=1) + template


def grad_violation(got, ref, rtol=GRAD_RTOL, atol=GRAD_ATOL):
    """max |got - ref| / (atol + rtol |ref|): <= 1 passes."""
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float(((got - ref).abs() / (atol + rtol * ref.abs())).max())


def engine_R_from_oracle(R_pad):
    """Oracle R (B,N+2,M+2) -> engine layout (B,N,M)."""
    return R_pad[:, 1:-1, 1:-1].contiguous()
