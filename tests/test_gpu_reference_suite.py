"""The reference's own GPU tests (softdtw_cuda/tests/*.py), run against this engine, plus
CPU-tensor staging and dtype handling."""
import pytest
import torch

from softdtw_cuda import SoftDTW, softdtw

pytestmark = pytest.mark.gpu


def test_softdtw_cpu_tensors_run():
    # reference test_softdtw_small.py:4-13 (CPU tensors; here staged through the GPU)
    torch.manual_seed(0)
    x = torch.randn(2, 10, 4, requires_grad=True)
    y = torch.randn(2, 11, 4)
    out = SoftDTW(gamma=1.0, dist="sqeuclidean")(x, y)
    out.sum().backward()
    assert out.device.type == "cpu" and torch.isfinite(out).all()
    assert torch.isfinite(x.grad).all()


def test_softdtw_cuda_matches_cpu_small():
    # reference test_softdtw_small.py:15-27
    torch.manual_seed(0)
    x = torch.randn(2, 12, 3, requires_grad=True)
    y = torch.randn(2, 9, 3)
    sdtw = SoftDTW(gamma=1.0, dist="sqeuclidean")
    out_cpu = sdtw(x, y).detach().cpu()
    out_gpu = sdtw(x.cuda(), y.cuda()).detach().cpu()
    assert torch.allclose(out_cpu, out_gpu, atol=1e-4, rtol=1e-4)


def test_gradcheck_tiny_fp64():
    # reference test_softdtw_small.py:29-37
    torch.manual_seed(0)
    x = torch.randn(1, 6, 2, dtype=torch.float64, requires_grad=True)
    y = torch.randn(1, 5, 2, dtype=torch.float64)
    out = SoftDTW(gamma=1.0, dist="sqeuclidean")(x, y)
    out.sum().backward()
    assert out.dtype == torch.float64 and torch.isfinite(x.grad).all()


def test_softdtw_cuda_runs_longer_than_1024():
    # reference test_softdtw_long.py
    torch.manual_seed(0)
    x = torch.randn(1, 5000, 2, device="cuda", requires_grad=True)
    y = torch.randn(1, 5000, 2, device="cuda")
    out = SoftDTW(gamma=1.0, dist="sqeuclidean", fused=True)(x, y)
    assert torch.isfinite(out).all()
    out.sum().backward()
    assert torch.isfinite(x.grad).all()
    assert x.grad.abs().mean() > 0


def test_log_backward_stability_long_small_gamma():
    # reference test_softdtw_log_backward.py
    torch.manual_seed(0)
    x = torch.randn(2, 128, 3, device="cuda", requires_grad=True)
    y = torch.randn(2, 128, 3, device="cuda")
    out = SoftDTW(gamma=0.01, dist="sqeuclidean")(x, y)
    assert torch.isfinite(out).all()
    out.sum().backward()
    assert torch.isfinite(x.grad).all()
    assert x.grad.abs().mean() > 1e-6


def test_fused_forward_matches_unfused_small():
    # reference test_fused_sqeuclid.py:12-28
    torch.manual_seed(0)
    x = torch.randn(2, 12, 3, device="cuda", requires_grad=True)
    y = torch.randn(2, 9, 3, device="cuda", requires_grad=True)
    a = SoftDTW(gamma=1.0, fused=True)(x, y)
    b = SoftDTW(gamma=1.0, fused=False)(x, y)
    assert torch.allclose(a, b, atol=1e-4, rtol=1e-4)


def test_fused_backward_matches_unfused_tiny():
    # reference test_fused_sqeuclid.py:31-62
    torch.manual_seed(0)
    x1 = torch.randn(1, 5, 2, device="cuda", requires_grad=True)
    y1 = torch.randn(1, 4, 2, device="cuda", requires_grad=True)
    x2 = x1.detach().clone().requires_grad_(True)
    y2 = y1.detach().clone().requires_grad_(True)
    SoftDTW(gamma=1.0, fused=True)(x1, y1).sum().backward()
    SoftDTW(gamma=1.0, fused=False)(x2, y2).sum().backward()
    assert torch.allclose(x1.grad, x2.grad, atol=5e-3, rtol=5e-3)
    assert torch.allclose(y1.grad, y2.grad, atol=5e-3, rtol=5e-3)


def test_fused_normalize_runs_and_matches_unfused_small():
    # reference test_fused_sqeuclid.py:65-80
    torch.manual_seed(0)
    x = torch.randn(2, 10, 3, device="cuda", requires_grad=True)
    y = torch.randn(2, 10, 3, device="cuda", requires_grad=True)
    a = SoftDTW(gamma=1.0, fused=True, normalize=True)(x, y)
    b = SoftDTW(gamma=1.0, fused=False, normalize=True)(x, y)
    assert torch.allclose(a, b, atol=1e-4, rtol=1e-4)


def test_functional_fused_true_on_cuda():
    # reference test_validation.py:116-127
    torch.manual_seed(0)
    x = torch.randn(2, 8, 3, device="cuda", requires_grad=True)
    y = torch.randn(2, 8, 3, device="cuda")
    out = softdtw(x, y, fused=True)
    assert out.shape == (2,) and torch.isfinite(out).all()
    out.sum().backward()
    assert torch.isfinite(x.grad).all()


def test_functional_fused_none_cpu_runs():
    # reference test_validation.py:106-113
    torch.manual_seed(0)
    out = softdtw(torch.randn(2, 5, 3), torch.randn(2, 5, 3), fused=None)
    assert out.shape == (2,) and torch.isfinite(out).all()


def test_unbatched_inputs_and_dtypes():
    torch.manual_seed(0)
    x = torch.randn(7, 3, device="cuda")
    y = torch.randn(9, 3, device="cuda")
    out = softdtw(x, y)
    assert out.shape == (1,)
    for dt in (torch.float16, torch.bfloat16, torch.float64):
        o = softdtw(x.to(dt), y.to(dt), fused=False)
        assert o.dtype == dt and torch.isfinite(o).all()


def test_self_normalized_is_zero_and_symmetric():
    torch.manual_seed(1)
    x = torch.randn(3, 20, 4, device="cuda")
    y = torch.randn(3, 20, 4, device="cuda")
    for fused in (False, True):
        z = softdtw(x, x.clone(), normalize=True, fused=fused)
        assert torch.all(z == 0)
        a = softdtw(x, y, fused=fused)
        b = softdtw(y, x, fused=fused)
        torch.testing.assert_close(a, b, rtol=1e-6, atol=0)
