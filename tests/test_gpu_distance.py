"""GPU distance kernels vs the reference's torch-CPU distance (exact mode: bit-equal)."""
import pytest
import torch

import oracle
from _gpu_util import randn_pair, say
from softdtw_cuda import _engine

pytestmark = pytest.mark.gpu

SHAPES = [
    (4, 64, 64, 8),      # config 1
    (32, 512, 512, 64),  # config 2 (headline)
    (2, 4096, 3072, 4),  # config 3 shape, 2 of its 16 pairs
    (8, 256, 256, 16),   # config 4 feature count
    (2, 12, 9, 3),       # small: ATen naive kernel (multiply-add)
    (1, 5, 4, 2),
    (3, 33, 47, 12),
    (2, 100, 70, 130),   # K > 128 spans several LDS slices
]


@pytest.mark.parametrize("B,N,M,K", SHAPES)
def test_distance_bits_equal_torch_cpu(B, N, M, K):
    say(f"[dist exact] B={B} N={N} M={M} K={K}")
    x, y = randn_pair(B, N, M, K, seed=N + M + K)
    ref = oracle.sqeuclidean(x, y)
    D = _engine.sqeuclid_fwd(x.cuda(), y.cuda()).cpu()
    eq = (D == ref).double().mean().item()
    assert eq == 1.0, f"bit-equal fraction {eq}"


def test_distance_clamp_and_self():
    x, _ = randn_pair(2, 40, 40, 7, seed=3)
    D = _engine.sqeuclid_fwd(x.cuda(), x.cuda()).cpu()
    ref = oracle.sqeuclidean(x, x)
    assert torch.equal(D, ref)
    assert torch.all(D >= 0)


@pytest.mark.parametrize("B,N,M,K,selfpair", [(2, 30, 20, 5, False), (3, 64, 64, 8, True),
                                              (2, 128, 96, 64, False),
                                              # split reduction (several pieces per tile),
                                              # padded and multi-tile feature widths
                                              (4, 300, 500, 33, False), (2, 70, 90, 100, False),
                                              (1, 1000, 40, 1, False)])
def test_distance_backward_matches_torch_autograd(B, N, M, K, selfpair):
    say(f"[dist bwd] B={B} N={N} M={M} K={K} self={selfpair}")
    x, y = randn_pair(B, N, M, K, seed=11)
    if selfpair:
        y = x.clone()
    G = torch.rand(B, N, M, generator=torch.Generator().manual_seed(2))
    xr = x.clone().requires_grad_(True)
    yr = y.clone().requires_grad_(True)
    oracle.sqeuclidean(xr, yr).backward(G)
    xg, yg = x.cuda(), y.cuda()
    D = _engine.sqeuclid_fwd(xg, yg)
    gx, gy = _engine.sqeuclid_bwd(xg, yg, D, G.cuda(), mask=True)
    torch.testing.assert_close(gx.cpu(), xr.grad, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(gy.cpu(), yr.grad, rtol=1e-4, atol=1e-4)
