"""The fused backward's gradient mode (sdtw_fused_bwd_f32 forming dL/dx and dL/dy inside the
recursion kernel, with no (B, N, M) buffer) against the same gradients formed from E.

E comes from sdtw_fused_bwd_e_f32, the same recursion writing g*E (which the end-to-end
tests pin against the oracle); the reference chain rule (autograd_xy.py:41-49) is then
applied to it in float64 on the host.  Both sides hold the same E values, so they differ
only in the order the fp32 sums are taken: compared at the gradient tolerance.  dL/dx is
formed in a fixed order (the same bits on every run); dL/dy adds the bands' shares with
atomics in arrival order, so a second run agrees to float32 rounding, and under
torch.use_deterministic_algorithms the E path gives identical bits.
"""
import pytest
import torch

from _gpu_util import grad_violation, randn_pair, say
from softdtw_cuda import _engine

pytestmark = pytest.mark.gpu

# (B, N, M, K, gamma, bandwidth): every matrix-core width, ragged bands and tiles, a single
# band, several workgroups per pair, 4-band workgroups (a batch whose 2-band workgroups do
# not all fit on the GPU, K <= 16), 2-band workgroups (a batch whose one-band workgroups do
# not all fit: 80 pairs x 4 bands on a 256-CU GPU), a Sakoe-Chiba band, the headline shape
# (one-band workgroups)
CASES = [
    (3, 200, 150, 4, 1.0, -1.0),
    (2, 130, 300, 8, 0.5, -1.0),
    (4, 256, 256, 16, 1.0, -1.0),
    (2, 100, 90, 32, 1.0, -1.0),
    (3, 300, 260, 64, 1.0, -1.0),
    (2, 40, 70, 16, 1.0, -1.0),
    (1, 700, 180, 8, 0.3, -1.0),
    (160, 256, 64, 16, 1.0, -1.0),
    (80, 256, 200, 64, 1.0, -1.0),
    (2, 300, 280, 16, 1.0, 40.0),
    (32, 512, 512, 64, 1.0, -1.0),
]


def _from_e(x, y, E):
    x, y, E = x.double().cpu(), y.double().cpu(), E.double().cpu()
    gx = 2.0 * (x * E.sum(dim=2, keepdim=True) - torch.bmm(E, y))
    gy = 2.0 * (y * E.sum(dim=1).unsqueeze(2) - torch.bmm(E.transpose(1, 2).contiguous(), x))
    return gx, gy


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}-N{c[1]}-M{c[2]}-K{c[3]}-bw{c[5]:g}" for c in CASES])
def test_gradient_mode_matches_chain_rule_on_e(case):
    B, N, M, K, gamma, bw = case
    say(f"[fused grad] B={B} N={N} M={M} K={K} gamma={gamma} bw={bw} "
        f"(bands per workgroup {_engine.fused_bands_per_workgroup(B, N, M, K, torch.device('cuda'))})")
    x, y = randn_pair(B, N, M, K, seed=7)
    x, y = x.cuda(), y.cuda()
    gout = (torch.rand(B, generator=torch.Generator().manual_seed(8)) + 0.5).cuda()
    _, R = _engine.fused_fwd(x, y, gamma, bw)
    gx, gy = _engine.fused_bwd(x, y, R, gamma, bw, gout=gout)
    E = _engine.fused_bwd_e(x, y, R, gamma, bw, gout=gout)
    torch.cuda.synchronize()
    gx_ref, gy_ref = _from_e(x, y, E)
    vx, vy = grad_violation(gx, gx_ref), grad_violation(gy, gy_ref)
    say(f"    violation dL/dx {vx:.4f}, dL/dy {vy:.4f}")
    assert vx <= 1.0 and vy <= 1.0
    # a second run: dL/dx has the same bits; dL/dy's band shares may meet in another order
    gx2, gy2 = _engine.fused_bwd(x, y, R, gamma, bw, gout=gout)
    assert torch.equal(gx2, gx)
    torch.testing.assert_close(gy2, gy, rtol=1e-5, atol=1e-6 * float(gy.abs().max()))
    # one gradient alone: the same values as with both
    gxo, none_y = _engine.fused_bwd(x, y, R, gamma, bw, gout=gout, need=(True, False))
    none_x, gyo = _engine.fused_bwd(x, y, R, gamma, bw, gout=gout, need=(False, True))
    assert none_y is None and none_x is None
    assert torch.equal(gxo, gx)
    torch.testing.assert_close(gyo, gy, rtol=1e-5, atol=1e-6 * float(gy.abs().max()))


@pytest.fixture
def deterministic():
    was = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        yield
    finally:
        torch.use_deterministic_algorithms(was)
        _engine.sync_deterministic()


@pytest.mark.parametrize("case", [CASES[4], CASES[-1]], ids=["B3-N300-K64", "headline"])
def test_deterministic_algorithms_give_identical_bits(case, deterministic):
    """Under torch.use_deterministic_algorithms(True) the fused backward takes its E path:
    two runs give the same bits, within the gradient tolerance of the gradient mode's."""
    B, N, M, K, gamma, bw = case
    x, y = randn_pair(B, N, M, K, seed=9)
    x, y = x.cuda(), y.cuda()
    _, R = _engine.fused_fwd(x, y, gamma, bw)
    assert _engine.sync_deterministic()
    a = _engine.fused_bwd(x, y, R, gamma, bw)
    b = _engine.fused_bwd(x, y, R, gamma, bw)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    torch.use_deterministic_algorithms(False)
    assert not _engine.sync_deterministic()
    c = _engine.fused_bwd(x, y, R, gamma, bw)
    vx, vy = grad_violation(c[0], a[0].double()), grad_violation(c[1], a[1].double())
    say(f"[fused grad] gradient mode vs deterministic E path: violation {vx:.4f} / {vy:.4f}")
    assert vx <= 1.0 and vy <= 1.0

