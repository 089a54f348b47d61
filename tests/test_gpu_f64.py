"""The float64 path (sdtw_*_f64) against float64 references.

The reference computes float64 inputs in float64 end to end (distances.py:20-25 on float64
tensors; launcher.py:307-368 on float64 arrays), so here every comparison is at float64
accuracy, far inside the north-star tolerances:
  - the brute-force golden vectors (value and path marginals of tiny cost matrices);
  - the C oracle's float64 forward / backward (oracle/sdtw_oracle.c, fwd_f64 / bwd_f64,
    the same loops as launcher.py:307-353) on the same D: R and out within 1e-12 relative
    with the same infinite cells, E within 1e-9 relative / 1e-12 absolute;
  - the distance against torch's CPU float64 ops (the reference's own op sequence);
  - the module end to end against a differentiable float64 recursion (torch.logsumexp);
  - torch.autograd.gradcheck through the public SoftDTW, fused and unfused, which needs
    float64 arithmetic throughout (what the reference's test_softdtw_small.py:29-37 runs in
    float64 for).
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from _checkers import torch_dp64
from _gpu_util import randn_pair, say
from softdtw_cuda import SoftDTW, _engine

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bruteforce.json")
F64 = torch.float64


def _golden():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _golden(), ids=lambda c: f"N{c['N']}M{c['M']}g{c['gamma']}bw{c['bandwidth']}")
def test_f64_dp_matches_bruteforce_golden(case):
    D = torch.tensor(case["D"], dtype=F64).unsqueeze(0).cuda()
    bw = -1.0 if case["bandwidth"] is None else case["bandwidth"]
    out, R = _engine.dtw_fwd64(D, case["gamma"], bw)
    E = _engine.dtw_bwd64(D, R, case["gamma"], bw).cpu()[0].numpy()
    np.testing.assert_allclose(out.item(), case["value"], rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(E, np.array(case["E"]), rtol=1e-11, atol=1e-11)


CASES = [
    # B, N, M, K, gamma, bandwidth
    (4, 64, 64, 8, 1.0, None),
    (2, 12, 9, 3, 1.0, None),
    (3, 37, 53, 4, 0.5, None),
    (2, 100, 80, 6, 0.1, 10.0),       # band, non-square
    (2, 64, 64, 3, 0.01, None),       # sharp soft-min
    (2, 1300, 700, 3, 1.0, None),     # more rows than threads in a workgroup
    (2, 700, 1300, 3, 0.3, 50.0),
    (1, 1, 1, 2, 1.0, None),
    (2, 1, 7, 2, 1.0, None),
    (2, 7, 1, 2, 0.5, None),
    (1, 3000, 40, 2, 0.5, 100.0),     # backward diagonals beyond LDS: global-memory sweep
    (1, 7000, 20, 2, 1.0, None),      # forward diagonals beyond LDS too
]


@pytest.mark.parametrize("B,N,M,K,gamma,bw", CASES)
def test_f64_dp_matches_oracle(B, N, M, K, gamma, bw):
    say(f"[f64 dp] B={B} N={N} M={M} gamma={gamma} bw={bw}")
    x, y = randn_pair(B, N, M, K, seed=N + 7 * M)
    D = oracle.sqeuclidean(x.double(), y.double())
    bwn = -1.0 if bw is None else bw
    out, R = _engine.dtw_fwd64(D.cuda(), gamma, bwn)
    out_o, R_o = oracle.forward(D, gamma, bw)
    R = R.cpu()
    assert torch.equal(torch.isinf(R), torch.isinf(R_o))
    fin = torch.isfinite(R_o)
    rel = ((R[fin] - R_o[fin]).abs() / R_o[fin].abs().clamp_min(1e-300)).max().item()
    assert rel <= 1e-12, rel
    np.testing.assert_allclose(out.cpu().numpy(), out_o.numpy(), rtol=1e-12)
    g = torch.linspace(0.5, 1.5, B, dtype=F64)
    G = _engine.dtw_bwd64(D.cuda(), R.cuda(), gamma, bwn, gout=g.cuda()).cpu()
    E_o = oracle.backward(D, R_o, gamma, bw)
    np.testing.assert_allclose(G.numpy(), (g.view(-1, 1, 1) * E_o).numpy(), rtol=1e-9, atol=1e-12)
    E = _engine.dtw_bwd64(D.cuda(), R.cuda(), gamma, bwn).cpu()
    np.testing.assert_allclose(E.numpy(), E_o.numpy(), rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize("B,N,M,K", [(2, 37, 53, 4), (3, 64, 64, 64), (1, 5, 300, 130)])
def test_f64_distance_matches_torch_ops(B, N, M, K):
    x, y = randn_pair(B, N, M, K, seed=K)
    x, y = x.double(), y.double()
    D = _engine.sqeuclid_fwd64(x.cuda(), y.cuda()).cpu()
    D_ref = oracle.sqeuclidean(x, y)
    scale = float(((x * x).sum(-1).max() + (y * y).sum(-1).max()))
    assert float((D - D_ref).abs().max()) <= 1e-13 * scale
    # the chain rule (clamp mask included; x == y rows make clamped cells with pre == 0)
    x2 = x.clone()
    x2[:, 0] = y[:, 0]
    xr = x2.clone().requires_grad_(True)
    yr = y.clone().requires_grad_(True)
    Dr = oracle.sqeuclidean(xr, yr)
    G = torch.randn(Dr.shape, dtype=F64, generator=torch.Generator().manual_seed(1))
    Dr.backward(G)
    D2 = _engine.sqeuclid_fwd64(x2.cuda(), y.cuda())
    gx, gy = _engine.sqeuclid_bwd64(x2.cuda(), y.cuda(), D2, G.cuda(), mask=True)
    np.testing.assert_allclose(gx.cpu().numpy(), xr.grad.numpy(), rtol=1e-10, atol=1e-10 * scale)
    np.testing.assert_allclose(gy.cpu().numpy(), yr.grad.numpy(), rtol=1e-10, atol=1e-10 * scale)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("bandwidth", [None, 3.0])
def test_f64_module_matches_torch_dp64(fused, bandwidth):
    say(f"[f64 module] fused={fused} bandwidth={bandwidth}")
    x, y = randn_pair(2, 13, 11, 3, seed=5)
    x, y = x.double(), y.double()
    xr = x.cuda().requires_grad_(True)
    yr = y.cuda().requires_grad_(True)
    out = SoftDTW(gamma=0.7, bandwidth=bandwidth, fused=fused)(xr, yr)
    assert out.dtype == F64
    out.sum().backward()
    for b in range(2):
        xc = x[b].clone().requires_grad_(True)
        yc = y[b].clone().requires_grad_(True)
        Dc = oracle.sqeuclidean(xc.unsqueeze(0), yc.unsqueeze(0))[0]
        val, _ = torch_dp64(Dc, 0.7, bandwidth)
        val.backward()
        np.testing.assert_allclose(out[b].item(), val.item(), rtol=1e-12)
        np.testing.assert_allclose(xr.grad[b].cpu().numpy(), xc.grad.numpy(), rtol=1e-9, atol=1e-11)
        np.testing.assert_allclose(yr.grad[b].cpu().numpy(), yc.grad.numpy(), rtol=1e-9, atol=1e-11)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("bandwidth", [None, 2.0])
def test_f64_gradcheck(fused, bandwidth):
    say(f"[f64 gradcheck] fused={fused} bandwidth={bandwidth}")
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 6, 2, dtype=F64, generator=g).cuda().requires_grad_(True)
    y = torch.randn(1, 5, 2, dtype=F64, generator=g).cuda().requires_grad_(True)
    sdtw = SoftDTW(gamma=1.0, dist="sqeuclidean", bandwidth=bandwidth, fused=fused)
    assert torch.autograd.gradcheck(lambda a, b: sdtw(a, b), (x, y))


def test_f64_cpu_inputs_return_f64_on_cpu():
    x, y = randn_pair(2, 10, 11, 4, seed=3)
    x = x.double().requires_grad_(True)
    y = y.double()
    out = SoftDTW(gamma=1.0)(x, y)
    out.sum().backward()
    assert out.dtype == F64 and out.device.type == "cpu" and x.grad.dtype == F64
    D = oracle.sqeuclidean(x.detach(), y)
    out_o, _ = oracle.forward(D, 1.0, None)
    np.testing.assert_allclose(out.detach().numpy(), out_o.numpy(), rtol=1e-12)
