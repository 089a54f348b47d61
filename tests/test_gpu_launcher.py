"""The six reference launcher names (softdtw_cuda/cuda/launcher.py) against the oracle.

Each keeps the reference's contract: R (B, N+2, M+2) in the input's dtype with R[0,0] = 0 and
+inf outside the cells, E (B, N, M); the backward functions take that R.  float32 runs the
engine's default (mixed) arithmetic, whose forward is bit-identical to the CPU path.
"""
import numpy as np
import pytest
import torch

import oracle
from _gpu_util import FWD_RTOL, grad_violation, randn_pair, say
from softdtw_cuda.cuda import launcher

pytestmark = pytest.mark.gpu


def _same_bits_rate(a, b):
    """Share of R entries with identical bits (the survey's R protocol: >= 99.9%), after
    checking that every differing entry is one fp32 ulp away.  The engine's fp64 exp / log
    are not the C library's, and in cells with one finite predecessor it forms m where the
    reference forms -gamma * (-m / gamma); either can move a rare fp32 rounding by one ulp."""
    same = (a == b) | (torch.isinf(a) & torch.isinf(b) & (torch.sign(a) == torch.sign(b)))
    if not same.all():
        da, db = a[~same].double(), b[~same].double()
        ulp = torch.from_numpy(np.spacing(b[~same].float().abs().numpy())).double()
        assert torch.all((da - db).abs() <= ulp), (da, db)
    return same.double().mean().item()


def _check_R_layout(R, N, M):
    assert R.shape[1:] == (N + 2, M + 2)
    assert torch.all(R[:, 0, 0] == 0)
    pad = torch.ones_like(R, dtype=torch.bool)
    pad[:, 0, 0] = False
    pad[:, 1:N + 1, 1:M + 1] = False
    assert torch.all(torch.isposinf(R[pad]))


@pytest.mark.parametrize("B,N,M,K,gamma,bw", [(3, 70, 45, 4, 1.0, None), (2, 130, 150, 8, 0.3, 20.0)])
def test_unfused_launcher_vs_oracle(B, N, M, K, gamma, bw):
    say(f"[launcher] unfused B={B} N={N} M={M} gamma={gamma} bw={bw}")
    x, y = randn_pair(B, N, M, K, seed=N + M)
    D = oracle.sqeuclidean(x, y)
    bwv = -1.0 if bw is None else bw
    out_o, R_o = oracle.forward(D, gamma, bw)
    E_o = oracle.backward(D, R_o, gamma, bw)
    out, R = launcher.softdtw_forward_cuda(D.cuda(), gamma, bwv)
    assert out.dtype == torch.float32 and R.dtype == torch.float32 and R.is_cuda
    _check_R_layout(R.cpu(), N, M)
    torch.testing.assert_close(out.cpu(), out_o, rtol=FWD_RTOL, atol=0)
    assert _same_bits_rate(R.cpu(), R_o) >= 0.999
    # backward from the reference's own R, and from the launcher's
    for Rin in (R_o.cuda(), R):
        E = launcher.softdtw_backward_cuda_log(D.cuda(), Rin, gamma, bwv)
        assert E.shape == (B, N, M) and E.dtype == torch.float32
        assert grad_violation(E, E_o, rtol=1e-5, atol=1e-7) <= 1.0
    with pytest.raises(ValueError, match="Expected R shape"):
        launcher.softdtw_backward_cuda_log(D.cuda(), R[:, :-1], gamma, bwv)


def test_fused_launcher_vs_oracle():
    B, N, M, K, gamma = 3, 90, 77, 6, 0.7
    say(f"[launcher] fused B={B} N={N} M={M}")
    x, y = randn_pair(B, N, M, K, seed=5)
    D = oracle.sqeuclidean(x, y)
    out_o, R_o = oracle.forward(D, gamma, None)
    E_o = oracle.backward(D, R_o, gamma, None)
    out, R = launcher.softdtw_forward_cuda_fused_sqeuclid(x.cuda(), y.cuda(), gamma, -1.0)
    _check_R_layout(R.cpu(), N, M)
    torch.testing.assert_close(out.cpu(), out_o, rtol=FWD_RTOL, atol=0)
    assert _same_bits_rate(R.cpu(), R_o) >= 0.999
    E = launcher.softdtw_backward_cuda_fused_sqeuclid(x.cuda(), y.cuda(), R, gamma, -1.0)
    assert E.shape == (B, N, M)
    assert grad_violation(E, E_o, rtol=1e-5, atol=1e-7) <= 1.0


def test_float64_launcher_keeps_dtype():
    B, N, M, K, gamma = 2, 40, 33, 3, 1.0
    x, y = randn_pair(B, N, M, K, seed=9)
    D = oracle.sqeuclidean(x.double(), y.double())
    out_o, R_o = oracle.forward(D, gamma, None)
    E_o = oracle.backward(D, R_o, gamma, None)
    out, R = launcher.softdtw_forward_cuda(D.cuda(), gamma, -1.0)
    assert out.dtype == torch.float64 and R.dtype == torch.float64
    _check_R_layout(R.cpu(), N, M)
    torch.testing.assert_close(out.cpu(), out_o, rtol=1e-12, atol=0)
    torch.testing.assert_close(R.cpu(), R_o, rtol=1e-12, atol=0)
    E = launcher.softdtw_backward_cuda_log(D.cuda(), R, gamma, -1.0)
    assert E.dtype == torch.float64
    torch.testing.assert_close(E.cpu(), E_o, rtol=1e-10, atol=1e-12)
    # the fused names on float64 inputs
    out_f, R_f = launcher.softdtw_forward_cuda_fused_sqeuclid(x.double().cuda(), y.double().cuda(), gamma, -1.0)
    assert out_f.dtype == torch.float64
    torch.testing.assert_close(out_f.cpu(), out_o, rtol=1e-12, atol=0)
    E_f = launcher.softdtw_backward_cuda_fused_sqeuclid(x.double().cuda(), y.double().cuda(), R_f, gamma, -1.0)
    torch.testing.assert_close(E_f.cpu(), E_o, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_cpu_names_return_on_cpu(dtype):
    B, N, M, K, gamma = 2, 30, 25, 3, 1.0
    x, y = randn_pair(B, N, M, K, seed=13)
    D = oracle.sqeuclidean(x.to(dtype), y.to(dtype))
    out_o, R_o = oracle.forward(D, gamma, None)
    E_o = oracle.backward(D, R_o, gamma, None)
    out, R = launcher.softdtw_forward_cpu(D, gamma, -1.0)
    assert out.device.type == "cpu" and R.device.type == "cpu"
    assert out.dtype == dtype and R.dtype == dtype
    _check_R_layout(R, N, M)
    torch.testing.assert_close(out, out_o, rtol=FWD_RTOL if dtype == torch.float32 else 1e-12, atol=0)
    Rsave = R.clone()
    E = launcher.softdtw_backward_cpu(D, R, gamma, -1.0)
    assert torch.equal(R, Rsave)  # not modified in place
    assert E.device.type == "cpu" and E.dtype == dtype
    if dtype == torch.float32:
        assert grad_violation(E, E_o, rtol=1e-5, atol=1e-7) <= 1.0
    else:
        torch.testing.assert_close(E, E_o, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_half_launcher_is_float32_engine_rounded(dtype):
    # half inputs run the float32 engine on the same values: the results equal the oracle on
    # the values upcast to float32, rounded once to the input's dtype
    B, N, M, K, gamma = 2, 48, 40, 4, 1.0
    x, y = randn_pair(B, N, M, K, seed=17)
    D = oracle.sqeuclidean(x, y).to(dtype)
    out_o, R_o = oracle.forward(D.float(), gamma, None)
    out, R = launcher.softdtw_forward_cuda(D.cuda(), gamma, -1.0)
    assert out.dtype == dtype and R.dtype == dtype
    assert torch.equal(out.cpu(), out_o.to(dtype))
    fin = torch.isfinite(R_o)
    assert torch.equal(R.cpu()[fin], R_o.to(dtype)[fin])
    # the backward on half D and half R equals the oracle on the same values upcast, rounded
    # once to the input's dtype (one ulp of the dtype for the rounding of a ~1e-6 difference)
    Rh = R_o.to(dtype)
    E = launcher.softdtw_backward_cuda_log(D.cuda(), Rh.cuda(), gamma, -1.0)
    assert E.dtype == dtype
    E_oh = oracle.backward(D.float(), Rh.float(), gamma, None)
    rt = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    torch.testing.assert_close(E.cpu().float(), E_oh.to(dtype).float(), rtol=rt, atol=1e-6)
