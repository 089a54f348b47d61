"""softdtw_barycenter on the engine vs the same loop on the CPU oracle (config 5 shape).

Adam's first steps move every coordinate by ~lr*sign(grad), so trajectories of any two
implementations separate after a few iterations; parity is therefore judged on (a) the
first iteration's loss and gradient, (b) one optimiser step, and (c) the final objective
after the full 100-iteration run."""
import pytest
import torch

import oracle
from _gpu_util import FWD_RTOL, grad_violation, random_walks, say
from softdtw_cuda import SoftDTW, softdtw_barycenter, softdtw_barycenter_cpu

pytestmark = pytest.mark.gpu

KSEQ, N, D = 64, 256, 8


def _objective(bary, X, gamma=1.0):
    d = oracle.softdtw(bary.cpu().unsqueeze(0).expand(X.shape[0], -1, -1), X.cpu(), gamma=gamma)
    return float(d.mean())


def test_first_iteration_loss_and_gradient():
    X = random_walks(KSEQ, N, D, seed=0)
    init = X.mean(dim=0)
    w = torch.ones(KSEQ) / KSEQ
    bo = init.clone().requires_grad_(True)
    lo = (w * oracle.softdtw(bo.unsqueeze(0).expand(KSEQ, -1, -1), X, gamma=1.0)).sum()
    lo.backward()
    for fused in (True, False):
        bg = init.clone().cuda().requires_grad_(True)
        lg = (w.cuda() * SoftDTW(gamma=1.0, fused=fused)(bg.unsqueeze(0).expand(KSEQ, -1, -1), X.cuda())).sum()
        lg.backward()
        v = grad_violation(bg.grad, bo.grad)
        say(f"[bary iter0] fused={fused} loss {lg.item():.6f} vs {lo.item():.6f} grad violation {v:.4f}")
        torch.testing.assert_close(lg.detach().cpu(), lo.detach(), rtol=FWD_RTOL, atol=0)
        assert v <= 1.0


def test_one_step_and_final_objective():
    X = random_walks(KSEQ, N, D, seed=0)
    one_gpu = softdtw_barycenter(X.cuda(), gamma=1.0, lr=0.1, max_iter=1, early_stopping=False).cpu()
    one_cpu = oracle.barycenter(X, gamma=1.0, lr=0.1, max_iter=1, early_stopping=False)
    v = grad_violation(one_gpu, one_cpu)
    say(f"[bary step1] violation {v:.4f}")
    assert v <= 1.0
    full_gpu = softdtw_barycenter(X.cuda(), gamma=1.0, lr=0.1, max_iter=100, early_stopping=False).cpu()
    full_cpu = oracle.barycenter(X, gamma=1.0, lr=0.1, max_iter=100, early_stopping=False)
    f_gpu = _objective(full_gpu, X)
    f_cpu = _objective(full_cpu, X)
    init_obj = _objective(X.mean(dim=0), X)
    say(f"[bary final] objective gpu {f_gpu:.7f} oracle {f_cpu:.7f} (init {init_obj:.4f}); "
        f"max |bary diff| {(full_gpu - full_cpu).abs().max().item():.3e}")
    assert f_gpu < init_obj
    assert abs(f_gpu - f_cpu) <= 1e-5 * abs(f_cpu)


def test_barycenter_cpu_wrapper_and_weights():
    X = random_walks(8, 32, 2, seed=1)
    w = torch.rand(8)
    b1 = softdtw_barycenter_cpu(X, weights=w, max_iter=5)
    assert b1.device.type == "cpu" and b1.shape == (32, 2)
    b2 = softdtw_barycenter(X.cuda(), weights=w.cuda(), max_iter=5, fused=False)
    assert b2.shape == (32, 2) and torch.isfinite(b2).all()
