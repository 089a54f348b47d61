"""End to end: SoftDTW (unfused and fused) on the GPU vs the reference CPU path (oracle).

mixed (the default) and exact arithmetic: loss within rtol 1e-5, dL/dx and dL/dy within
rtol 1e-4 / atol 1e-5 of the CPU path.  fast arithmetic: the same loss tolerance; gradients
within that tolerance or no farther from an fp64 evaluation of the algorithm than the CPU
path itself (_gpu_util.no_less_accurate)."""
import pytest
import torch

import oracle
from _gpu_util import (FWD_RTOL, grad_violation, no_less_accurate, numerics, randn_pair, say,
                       sinusoid_pair)
from softdtw_cuda import SoftDTW

pytestmark = pytest.mark.gpu


def _run_gpu(x, y, fused, gamma, bw=None, normalize=False, reduce="mean"):
    xg = x.clone().cuda().requires_grad_(True)
    yg = y.clone().cuda().requires_grad_(True)
    out = SoftDTW(gamma=gamma, bandwidth=bw, normalize=normalize, fused=fused)(xg, yg)
    (out.mean() if reduce == "mean" else out.sum()).backward()
    return out.detach().cpu(), xg.grad.cpu(), yg.grad.cpu()


def _run_oracle(x, y, gamma, bw=None, normalize=False, reduce="mean", dtype=torch.float32):
    xo = x.clone().to(dtype).requires_grad_(True)
    yo = y.clone().to(dtype).requires_grad_(True)
    out = oracle.softdtw(xo, yo, gamma=gamma, bandwidth=bw, normalize=normalize)
    (out.mean() if reduce == "mean" else out.sum()).backward()
    return out.detach(), xo.grad, yo.grad


def _compare(tag, x, y, gamma, bw=None, normalize=False, reduce="mean", modes=(False, True),
             arith=("mixed", "exact", "fast")):
    ref = _run_oracle(x, y, gamma, bw, normalize, reduce)
    ref64 = _run_oracle(x, y, gamma, bw, normalize, reduce, torch.float64) if "fast" in arith else None
    for mode in arith:
        for fused in modes:
            with numerics(mode):
                got = _run_gpu(x, y, fused, gamma, bw, normalize, reduce)
            lossrel = ((got[0] - ref[0]).abs() / ref[0].abs().clamp_min(1e-30)).max().item()
            torch.testing.assert_close(got[0], ref[0], rtol=FWD_RTOL, atol=1e-6)
            if mode != "fast":
                vx = grad_violation(got[1], ref[1])
                vy = grad_violation(got[2], ref[2])
                say(f"[e2e {tag}] {mode} fused={fused} loss maxrel={lossrel:.3e} "
                    f"grad violation x={vx:.4f} y={vy:.4f}")
                assert vx <= 1.0 and vy <= 1.0
            else:
                okx, vx, vx64, rx = no_less_accurate(got[1], ref[1], ref64[1])
                oky, vy, vy64, ry = no_less_accurate(got[2], ref[2], ref64[2])
                say(f"[e2e {tag}] fast fused={fused} loss maxrel={lossrel:.3e} grad violation "
                    f"vs CPU path x={vx:.3f} y={vy:.3f}; vs fp64 x={vx64:.3f} y={vy64:.3f} "
                    f"(CPU path vs fp64: x={rx:.3f} y={ry:.3f})")
                assert okx and oky


def test_config1_plumbing():
    x, y = randn_pair(4, 64, 64, 8, seed=0)
    _compare("C1", x, y, 1.0)


def test_small_shapes():
    for (B, N, M, K) in [(2, 12, 9, 3), (1, 5, 4, 2), (2, 10, 11, 4), (3, 31, 17, 6)]:
        x, y = randn_pair(B, N, M, K, seed=N * M)
        _compare(f"small{B}x{N}x{M}x{K}", x, y, 1.0, reduce="sum")


def test_bandwidth_and_gamma():
    x, y = randn_pair(2, 60, 70, 3, seed=9)
    _compare("band", x, y, 0.5, bw=12.0)
    _compare("sharp", x, y, 0.05)


def test_config2_headline():
    x, y = randn_pair(32, 512, 512, 64, seed=0)
    _compare("C2", x, y, 1.0, reduce="sum")


def test_config4_normalize():
    x, y = sinusoid_pair(64, 256, 16, seed=0)
    _compare("C4", x, y, 1.0, normalize=True, modes=(True, False))


@pytest.mark.slow
def test_config3_long_subset():
    # 2 of the 16 pairs at the full config-3 length; the oracle takes seconds per pair
    x, y = randn_pair(2, 4096, 3072, 4, seed=0)
    _compare("C3", x, y, 0.1, reduce="sum", arith=("mixed", "exact"))
