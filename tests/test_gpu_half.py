"""float16 and bfloat16 inputs: the stated contract, checked against the oracle.

The engine has no half-precision arithmetic.  Half inputs are upcast to float32 on entry,
computed by the float32 engine, and every tensor the reference's op sequence would hold in
the input dtype is rounded to it at the same point:
  * unfused (fused=False): the distance D is formed in float32 and returned in the input dtype
    (the reference's pairwise_distance gives D in the input dtype, distances.py:20-28); the
    recursion runs on that D upcast; the loss, dL/dD and the gradients come back in the
    input dtype;
  * fused (the default on GPU): the costs are formed in float32 from the upcast inputs and
    never rounded (no D tensor exists); the loss and gradients come back in the input dtype.
The oracle runs the same sequence on the CPU with float32 arithmetic and the same roundings,
so the engine's half results equal the oracle's up to one unit in the last place of the
half dtype (a float32 value within ~1e-6 of the oracle's can round to either neighbour).
"""
import pytest
import torch

import oracle
from _gpu_util import randn_pair, say
from softdtw_cuda import SoftDTW

pytestmark = pytest.mark.gpu

ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def _oracle_half(x, y, dtype, gamma, fused):
    """The contract's op sequence on the CPU: float32 arithmetic, roundings to `dtype` where
    the engine rounds."""
    xo = x.to(dtype).float().requires_grad_(True)
    yo = y.to(dtype).float().requires_grad_(True)
    D = oracle.sqeuclidean(xo, yo)
    if not fused:
        D = D.to(dtype).float()  # the unfused route materialises D in the input dtype
    out = oracle.OracleSoftDTWFunction.apply(D, gamma, None)
    out_h = out.to(dtype)
    out_h.float().sum().backward()
    return out_h.detach(), xo.grad.to(dtype), yo.grad.to(dtype)


def _close_in_ulps(got, ref, dtype, what):
    got = got.detach().cpu().float()
    ref = ref.float()
    tol = ULP[dtype] * ref.abs() + 1e-6
    bad = (got - ref).abs() > tol
    say(f"    {what}: {int(bad.sum())} values beyond one {dtype} ulp, max |diff| "
        f"{float((got - ref).abs().max()):.3g}")
    assert not bad.any()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("fused", [False, True])
def test_half_inputs_follow_the_float32_engine(dtype, fused):
    B, N, M, K, gamma = 3, 96, 80, 6, 1.0
    x, y = randn_pair(B, N, M, K, seed=21)
    say(f"[half] {dtype} fused={fused}")
    xg = x.to(dtype).cuda().requires_grad_(True)
    yg = y.to(dtype).cuda().requires_grad_(True)
    out = SoftDTW(gamma=gamma, fused=fused)(xg, yg)
    assert out.dtype == dtype
    out.float().sum().backward()
    assert xg.grad.dtype == dtype and yg.grad.dtype == dtype
    ref = _oracle_half(x, y, dtype, gamma, fused)
    _close_in_ulps(out, ref[0], dtype, "loss")
    _close_in_ulps(xg.grad, ref[1], dtype, "dL/dx")
    _close_in_ulps(yg.grad, ref[2], dtype, "dL/dy")
