"""The production launch sequence, the full long-sequence geometry, and the give-up path.

The other GPU tests synchronise after every wavefront launch (SDTW_DEBUG_SYNC=1, set in
conftest) so that a kernel's bounded-wait flag is checked each time.  These tests turn that
off and run what a user runs: the prep launch, the recursions and the distance kernels back to
back on one stream, then compare with the oracle.  A wave that gave up would show as NaN in
the results (the kernels mark the pair's results when a wait expires), which the comparisons
reject.
"""
import pytest
import torch

import oracle
from _gpu_util import FWD_RTOL, grad_violation, randn_pair, say
from softdtw_cuda import SoftDTW, _engine

pytestmark = pytest.mark.gpu


@pytest.fixture
def production(monkeypatch):
    monkeypatch.setattr(_engine, "_DEBUG_SYNC", False)


def _gpu(x, y, fused, gamma, reps=1):
    for _ in range(reps):
        xg = x.clone().cuda().requires_grad_(True)
        yg = y.clone().cuda().requires_grad_(True)
        out = SoftDTW(gamma=gamma, fused=fused)(xg, yg)
        out.sum().backward()
    torch.cuda.synchronize()
    return out.detach().cpu(), xg.grad.cpu(), yg.grad.cpu()


def _oracle(x, y, gamma):
    xo = x.clone().requires_grad_(True)
    yo = y.clone().requires_grad_(True)
    out = oracle.softdtw(xo, yo, gamma=gamma)
    out.sum().backward()
    return out.detach(), xo.grad, yo.grad


def _check(tag, got, ref):
    torch.testing.assert_close(got[0], ref[0], rtol=FWD_RTOL, atol=1e-6)
    vx = grad_violation(got[1], ref[1])
    vy = grad_violation(got[2], ref[2])
    say(f"[{tag}] grad violation x={vx:.4f} y={vy:.4f}")
    assert vx <= 1.0 and vy <= 1.0


def test_headline_production_sequence(production):
    # three steps back to back per mode (the workspace of one step is reused memory for the
    # next), no synchronisation between launches
    x, y = randn_pair(32, 512, 512, 64, seed=0)
    ref = _oracle(x, y, 1.0)
    for fused in (False, True):
        say(f"[production] C2 fused={fused}")
        _check(f"C2 production fused={fused}", _gpu(x, y, fused, 1.0, reps=3), ref)


@pytest.mark.slow
def test_config3_full_batch_geometry(production):
    """B = 16 at 4096 x 3072: 16 * 32 two-band workgroups exceed the CU count, so the fused
    recursions take 4 bands per workgroup (producers sharing their compute waves' SIMDs) and
    the unfused forward takes two launches.  The gradients of a summed loss are per pair, so
    pairs 0 and 15 are checked against the oracle run on those two pairs."""
    B, N, M, K, gamma = 16, 4096, 3072, 4, 0.1
    assert _engine.fused_bands_per_workgroup(B, N, M, K, "cuda") == 4
    assert not _engine.one_launch_unfused_forward(B, N, M, K, "cuda")
    x, y = randn_pair(B, N, M, K, seed=0)
    pick = torch.tensor([0, B - 1])
    ref = _oracle(x[pick], y[pick], gamma)
    for fused in (False, True):
        say(f"[production] C3 B={B} fused={fused}")
        got = _gpu(x, y, fused, gamma)
        _check(f"C3 full fused={fused}", (got[0][pick], got[1][pick], got[2][pick]), ref)
        assert torch.isfinite(got[0]).all()


def test_giveup_marks_results_nan(production):
    """With the poll limit at 0 every wait that would have to poll gives up at once (each
    kernel still runs to its end).  Band 1 of each pair must wait for band 0's first entries,
    so every pair's forward gives up: out is NaN.  In the backward the band above the bottom
    band gives up, and its rows of G (fused: of dL/dx through E) come back NaN.  With the limit
    restored, the same calls give the normal results."""
    B, N, M, K, gamma = 2, 512, 384, 8, 1.0
    x, y = randn_pair(B, N, M, K, seed=3)
    D = oracle.sqeuclidean(x, y).cuda()
    xg, yg = x.cuda(), y.cuda()
    out_ok, R_ok = _engine.dtw_fwd(D, gamma, -1.0)
    G_ok = _engine.dtw_bwd(D, R_ok, gamma, -1.0)
    outf_ok, Rf_ok = _engine.fused_fwd(xg, yg, gamma, -1.0)
    gx_ok, gy_ok = _engine.fused_bwd(xg, yg, Rf_ok, gamma, -1.0)
    torch.cuda.synchronize()
    prev = _engine.set_wait_limit(0)
    try:
        out, _ = _engine.dtw_fwd(D, gamma, -1.0)
        G = _engine.dtw_bwd(D, R_ok, gamma, -1.0)
        outf, _ = _engine.fused_fwd(xg, yg, gamma, -1.0)
        gx, gy = _engine.fused_bwd(xg, yg, Rf_ok, gamma, -1.0)
        torch.cuda.synchronize()
    finally:
        _engine.set_wait_limit(prev)
    say(f"[give-up] out {out.tolist()} fused {outf.tolist()}; NaN rows of G per pair "
        f"{torch.isnan(G).any(-1).sum(-1).tolist()}; NaN rows of gx {torch.isnan(gx).any(-1).sum(-1).tolist()}")
    assert torch.isnan(out).all() and torch.isnan(outf).all()
    # band 6 (rows 384..447) waits for the bottom band at its first group
    assert torch.isnan(G[:, 384:448]).all(-1).all()
    assert torch.isnan(gx).any(-1).sum().item() >= B * 64
    # the kernels ended normally: the same calls now give the normal results
    out2, R2 = _engine.dtw_fwd(D, gamma, -1.0)
    G2 = _engine.dtw_bwd(D, R2, gamma, -1.0)
    outf2, Rf2 = _engine.fused_fwd(xg, yg, gamma, -1.0)
    gx2, gy2 = _engine.fused_bwd(xg, yg, Rf2, gamma, -1.0)
    torch.cuda.synchronize()
    assert torch.equal(out2, out_ok) and torch.equal(G2, G_ok)
    assert torch.equal(outf2, outf_ok) and torch.equal(gx2, gx_ok) and torch.equal(gy2, gy_ok)
