"""The 'exact' distance contract holds on this host's torch CPU.

The GPU distance kernel reproduces a specific arithmetic order (see _exact_model.py).  This
test checks that order against torch-CPU's own D -- the reference's distance on the same
host -- so a host whose torch dispatches differently is detected before any GPU run.
"""
import numpy as np
import pytest
import torch

import oracle
from _exact_model import aten_sumsq, exact_sqeuclid


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 31, 32, 64, 100, 128, 129, 600])
def test_row_norm_order_matches_aten(K):
    g = torch.Generator().manual_seed(K)
    x = torch.randn(64, K, generator=g)
    ref = (x * x).sum(-1).numpy()
    ours = np.array([aten_sumsq(r) for r in x.numpy()], dtype=np.float32)
    assert np.array_equal(ours, ref)


@pytest.mark.parametrize("B,N,M,K", [
    (4, 64, 64, 8),      # config 1
    (2, 128, 96, 64),    # headline feature count
    (1, 200, 150, 4),    # long-config feature count
    (2, 64, 64, 16),     # normalize-config feature count
    (2, 12, 9, 3),       # K*N*M < 400: ATen's naive multiply-add kernel
    (1, 5, 4, 2),
    (2, 33, 47, 12),
])
def test_distance_order_matches_torch_cpu(B, N, M, K):
    g = torch.Generator().manual_seed(B * 1000 + N + M + K)
    x = torch.randn(B, N, K, generator=g)
    y = torch.randn(B, M, K, generator=g)
    ref = oracle.sqeuclidean(x, y).numpy()
    ours = exact_sqeuclid(x.numpy(), y.numpy())
    assert np.array_equal(ours, ref), (ours != ref).mean()
