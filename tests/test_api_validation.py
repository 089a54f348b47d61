"""Input validation of the public API: the reference's softdtw_cuda/tests/test_validation.py
error messages, which are raised before any device work (so these run on the CPU)."""
import math

import pytest
import torch

from softdtw_cuda import SoftDTW, softdtw
from softdtw_cuda.distances import pairwise_distance, sqeuclidean
from softdtw_cuda.utils.checks import check_D


def test_gamma_zero_raises():
    with pytest.raises(ValueError, match="gamma must be > 0"):
        SoftDTW(gamma=0.0)


def test_gamma_negative_raises():
    with pytest.raises(ValueError, match="gamma must be > 0"):
        SoftDTW(gamma=-1.0)


def test_gamma_inf_raises():
    with pytest.raises(ValueError, match="gamma must be finite"):
        SoftDTW(gamma=math.inf)


def test_gamma_nan_raises():
    with pytest.raises(ValueError, match="gamma must be finite"):
        SoftDTW(gamma=math.nan)


def test_fused_true_on_cpu_raises():
    sdtw = SoftDTW(gamma=1.0, fused=True)
    with pytest.raises(ValueError, match="fused=True requires CUDA"):
        sdtw(torch.randn(2, 5, 3), torch.randn(2, 5, 3))


def test_normalize_unequal_lengths_raises():
    with pytest.raises(ValueError, match="normalize=True"):
        SoftDTW(gamma=1.0, normalize=True)(torch.randn(2, 5, 3), torch.randn(2, 7, 3))


@pytest.mark.parametrize("nx,ny", [(0, 5), (5, 0)])
def test_empty_sequence_raises(nx, ny):
    with pytest.raises(ValueError, match="Sequence lengths must be > 0"):
        SoftDTW(gamma=1.0)(torch.randn(2, nx, 3), torch.randn(2, ny, 3))


def test_batch_size_mismatch_raises():
    with pytest.raises(ValueError, match="Batch sizes must match"):
        SoftDTW(gamma=1.0)(torch.randn(2, 5, 3), torch.randn(3, 5, 3))


def test_feature_dim_mismatch_raises():
    with pytest.raises(ValueError, match="Feature dims must match"):
        SoftDTW(gamma=1.0)(torch.randn(2, 5, 3), torch.randn(2, 5, 4))


def test_bad_rank_raises():
    with pytest.raises(ValueError, match="Expected x,y to have shape"):
        SoftDTW()(torch.randn(5), torch.randn(5))


def test_unknown_dist_raises():
    with pytest.raises(ValueError, match="Unknown dist"):
        pairwise_distance(torch.randn(1, 2, 2), torch.randn(1, 2, 2), dist="cosine")


def test_sqeuclidean_shape_errors():
    with pytest.raises(ValueError, match="Expected x,y as"):
        sqeuclidean(torch.randn(2, 2), torch.randn(1, 2, 2))
    with pytest.raises(ValueError, match="Batch/features mismatch"):
        sqeuclidean(torch.randn(1, 2, 2), torch.randn(1, 2, 3))


def test_check_D():
    with pytest.raises(TypeError, match="must be a torch.Tensor"):
        check_D([1.0])
    with pytest.raises(ValueError, match=r"D must have shape \(B,N,M\)"):
        check_D(torch.zeros(2, 2))
    with pytest.raises(TypeError, match="Unsupported dtype"):
        check_D(torch.zeros(1, 2, 2, dtype=torch.int32))


def test_bandwidth_normalisation():
    assert SoftDTW(bandwidth=-3).bandwidth is None
    assert SoftDTW(bandwidth=0).bandwidth is None
    assert SoftDTW(bandwidth=2).bandwidth == 2.0


def test_use_fused_selection_on_cpu():
    m = SoftDTW()
    assert m._use_fused(torch.zeros(1, 2, 2), torch.zeros(1, 2, 2)) is False
    assert SoftDTW(fused=False)._use_fused(torch.zeros(1, 2, 2), torch.zeros(1, 2, 2)) is False


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
def test_cpu_tensors_without_gpu_fail_loudly():
    with pytest.raises(RuntimeError, match="no GPU is visible"):
        softdtw(torch.randn(2, 5, 3), torch.randn(2, 5, 3), fused=None)
