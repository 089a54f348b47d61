"""softdtw_barycenter on the engine vs the same loop on the CPU oracle (config 5 shape).

Adam's first steps move every coordinate by ~lr*sign(grad), so trajectories of any two
implementations separate after a few iterations (a one-ulp change of the oracle's own
initial barycenter moves its final objective by ~1e-4 relative).  Parity is therefore
gated on (a) the first iteration's loss and gradient, (b) one optimiser step, and (c) the
final objective of the full 100-iteration run against the oracle's own one-ulp spread."""
import pytest
import torch

import oracle
from _gpu_util import FWD_RTOL, grad_violation, no_less_accurate, numerics, random_walks, say
from softdtw_cuda import SoftDTW, softdtw_barycenter, softdtw_barycenter_cpu

pytestmark = pytest.mark.gpu

KSEQ, N, D = 64, 256, 8


def _objective(bary, X, gamma=1.0):
    d = oracle.softdtw(bary.cpu().unsqueeze(0).expand(X.shape[0], -1, -1), X.cpu(), gamma=gamma)
    return float(d.mean())


@pytest.mark.parametrize("mode", ["mixed", "exact", "fast"])
def test_first_iteration_loss_and_gradient(mode):
    X = random_walks(KSEQ, N, D, seed=0)
    init = X.mean(dim=0)

    def oracle_iter0(dtype):
        w = torch.ones(KSEQ, dtype=dtype) / KSEQ
        b = init.clone().to(dtype).requires_grad_(True)
        loss = (w * oracle.softdtw(b.unsqueeze(0).expand(KSEQ, -1, -1), X.to(dtype), gamma=1.0)).sum()
        loss.backward()
        return loss.detach(), b.grad

    lo, go = oracle_iter0(torch.float32)
    w = torch.ones(KSEQ) / KSEQ
    for fused in (True, False):
        bg = init.clone().cuda().requires_grad_(True)
        with numerics(mode):
            lg = (w.cuda() * SoftDTW(gamma=1.0, fused=fused)(bg.unsqueeze(0).expand(KSEQ, -1, -1), X.cuda())).sum()
            lg.backward()
        torch.testing.assert_close(lg.detach().cpu(), lo, rtol=FWD_RTOL, atol=0)
        if mode != "fast":
            v = grad_violation(bg.grad, go)
            say(f"[bary iter0] {mode} fused={fused} loss {lg.item():.6f} vs {lo.item():.6f} grad violation {v:.4f}")
            assert v <= 1.0
        else:
            _, g64 = oracle_iter0(torch.float64)
            ok, v32, v64, vref = no_less_accurate(bg.grad, go, g64)
            say(f"[bary iter0] fast fused={fused} grad violation vs CPU path {v32:.3f}, vs fp64 "
                f"{v64:.3f} (CPU path vs fp64 {vref:.3f})")
            assert ok


def test_one_step():
    X = random_walks(KSEQ, N, D, seed=0)
    one_gpu = softdtw_barycenter(X.cuda(), gamma=1.0, lr=0.1, max_iter=1, early_stopping=False).cpu()
    one_cpu = oracle.barycenter(X, gamma=1.0, lr=0.1, max_iter=1, early_stopping=False)
    v = grad_violation(one_gpu, one_cpu)
    say(f"[bary step1] violation {v:.4f}")
    assert v <= 1.0


def test_final_objective_within_oracle_noise_floor():
    # The oracle's own sensitivity: the same 100 iterations from an init perturbed by one
    # ulp (one element, then every element).  The engine's final objective must sit within
    # twice that spread of the oracle's (plus 1e-5 relative).
    X = random_walks(KSEQ, N, D, seed=0)
    init = (X * (torch.ones(KSEQ) / KSEQ).view(KSEQ, 1, 1)).sum(dim=0)
    kw = dict(gamma=1.0, lr=0.1, max_iter=100, early_stopping=False)
    base = oracle.barycenter(X, init=init, **kw)
    one = init.clone()
    one[0, 0] = torch.nextafter(one[0, 0], torch.tensor(-1e9))
    every = torch.nextafter(init, torch.full_like(init, 1e9))
    f_base = _objective(base, X)
    spread = max(abs(_objective(oracle.barycenter(X, init=i, **kw), X) - f_base) for i in (one, every))
    full_gpu = softdtw_barycenter(X.cuda(), **kw).cpu()
    f_gpu = _objective(full_gpu, X)
    init_obj = _objective(init, X)
    say(f"[bary final] objective gpu {f_gpu:.7f} oracle {f_base:.7f} (init {init_obj:.4f}); "
        f"oracle 1-ulp spread {spread:.4f}; max |bary diff| {(full_gpu - base).abs().max().item():.3e}")
    assert f_gpu < init_obj
    assert abs(f_gpu - f_base) <= 2.0 * spread + 1e-5 * abs(f_base)


def test_barycenter_cpu_wrapper_and_weights():
    X = random_walks(8, 32, 2, seed=1)
    w = torch.rand(8)
    b1 = softdtw_barycenter_cpu(X, weights=w, max_iter=5)
    assert b1.device.type == "cpu" and b1.shape == (32, 2)
    b2 = softdtw_barycenter(X.cuda(), weights=w.cuda(), max_iter=5, fused=False)
    assert b2.shape == (32, 2) and torch.isfinite(b2).all()


def test_device_loop_matches_python_loop(monkeypatch):
    """The device loop (sdtw_barycenter_f32) and the engine's Python loop (autograd, torch's
    Adam, clip_grad_norm_ and scheduler) agree step by step, with non-uniform weights: both
    compute the same gradients; the device loop sums them over pairs and forms the norm in
    its own order, so the iterates agree to float32 rounding."""
    from softdtw_cuda import barycenters
    X = random_walks(16, 96, 4, seed=2).cuda()
    w = (torch.rand(16, generator=torch.Generator().manual_seed(3)) + 0.5).cuda()
    kw = dict(gamma=0.7, weights=w, lr=0.1, early_stopping=False)
    for iters in (1, 3):
        dev = softdtw_barycenter(X, max_iter=iters, **kw)
        with monkeypatch.context() as mp:
            mp.setattr(barycenters, "_device_loop_applies", lambda *a: False)
            py = softdtw_barycenter(X, max_iter=iters, **kw)
        err = (dev - py).abs().max().item()
        say(f"[bary device vs python] {iters} iterations: max |diff| {err:.3e}")
        assert err <= 1e-5 * (1 + iters)


def test_device_loop_one_weighted_step_vs_oracle():
    """One step with non-uniform weights against the oracle's gradient.  Adam's first step is
    -lr g / (|g| + 1e-8) on the clipped gradient g = c G (c = 1 / |G| here): a gradient G
    within the gradient tolerance of the oracle's (rtol 1e-4, atol 1e-5) may still differ by
    up to 1e-5 absolutely, which after the clip moves the step of an element with a small G by
    lr 1e-8 c 1e-5 / (c G)^2, beyond rtol 1e-4 of the step.  The step is therefore compared at
    rtol 1e-4 where |G| >= 1e-2 (the atol term is then at most 1e-3 of G) and bounded by
    2 lr elsewhere."""
    X = random_walks(KSEQ, N, D, seed=4)
    w = torch.rand(KSEQ, generator=torch.Generator().manual_seed(5)) + 0.2
    wn = w / w.sum()
    init = (X * wn.view(KSEQ, 1, 1)).sum(dim=0)
    lr = 0.1
    one_gpu = softdtw_barycenter(X.cuda(), weights=w.cuda(), gamma=1.0, lr=lr, max_iter=1,
                                 early_stopping=False).cpu()
    b = init.clone().requires_grad_(True)
    (wn * oracle.softdtw(b.unsqueeze(0).expand(KSEQ, -1, -1), X, gamma=1.0)).sum().backward()
    G = b.grad.double()
    g = G * min(1.0, 1.0 / (G.norm().item() + 1e-6))
    step_o = -lr * g / (g.abs() + 1e-8)
    step = (one_gpu - init).double()
    ok = G.abs() >= 1e-2
    v = grad_violation(step[ok], step_o[ok])
    say(f"[bary weighted step1] violation {v:.4f} over {int(ok.sum())} of {ok.numel()} elements "
        f"(the rest: max |diff| {float((step - step_o)[~ok].abs().max()) if (~ok).any() else 0:.3g})")
    assert ok.float().mean() > 0.8
    assert v <= 1.0
    assert float((step - step_o).abs().max()) <= 2 * lr + 1e-6


def test_device_loop_early_stopping_rule():
    """The device loop stops where the reference's rule (barycenters.py:149-165), applied to
    the losses it reports, says it must."""
    from softdtw_cuda import _engine
    from softdtw_cuda.barycenters import _cosine_lrs
    X = random_walks(8, 64, 2, seed=6).cuda()
    w = torch.full((8,), 1 / 8, device="cuda")
    init = (X * w.view(8, 1, 1)).sum(0)
    max_iter, patience, tol = 60, 4, 5e-3
    _, losses = _engine.barycenter(X, w, init.clone(), 1.0, _cosine_lrs(0.1, max_iter), True,
                                   patience, tol)
    losses = losses.cpu().tolist()
    best, wait, stop = float("inf"), 0, max_iter
    for it, lv in enumerate(losses):
        if best - lv > tol:
            best, wait = lv, 0
        else:
            wait += 1
        if wait >= patience and it > max_iter // 2:
            stop = it + 1
            break
    say(f"[bary early stop] ran {len(losses)} of {max_iter}; rule says {stop}")
    assert len(losses) == stop and stop < max_iter
    # without early stopping every iteration runs, with the same losses up to the stop
    _, all_losses = _engine.barycenter(X, w, init.clone(), 1.0, _cosine_lrs(0.1, max_iter), False,
                                       patience, tol)
    assert all_losses.numel() == max_iter
    torch.testing.assert_close(all_losses[:stop].cpu(), torch.tensor(losses), rtol=0, atol=0)
