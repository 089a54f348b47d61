"""The CPU oracle (oracle/) pinned against independent checks.

What pins what:
  forward value  : brute-force path enumeration (golden fixtures), closed forms for N=1 /
                   M=1 / N=M=1, the gamma->0 DTW limit, symmetry under transposition;
  fp64 state     : the oracle's fp32 R equals an independent float64 recursion rounded once
                   (an fp32-state recursion would not);
  backward E     : brute-force path marginals (golden), autograd of an independent fp64
                   recursion, E endpoints = 1, 0 <= E <= 1;
  band           : brute force restricted to the band (golden);
  distance       : the reference's own test (naive broadcast, atol 1e-6) and x = y => 0.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import oracle
from _checkers import brute_force, hard_dtw, torch_dp64

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bruteforce.json")


def _cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"N{c['N']}M{c['M']}g{c['gamma']}bw{c['bandwidth']}")
def test_oracle_matches_bruteforce_golden(case):
    D = torch.tensor(case["D"], dtype=torch.float32).unsqueeze(0)
    out, R = oracle.forward(D, case["gamma"], case["bandwidth"])
    assert out.dtype == torch.float32 and R.shape == (1, case["N"] + 2, case["M"] + 2)
    np.testing.assert_allclose(out.item(), case["value"], rtol=2e-6, atol=1e-6)
    E = oracle.backward(D, R, case["gamma"], case["bandwidth"])
    # E reads fp32 differences of R (launcher.py:347-349): its accuracy is ~ulp(R)/gamma
    rmax = float(R[torch.isfinite(R)].abs().max())
    tol = max(1e-5, 8 * 2.0 ** -24 * rmax / case["gamma"])
    np.testing.assert_allclose(E[0].numpy(), np.array(case["E"]), rtol=tol, atol=tol)


def test_golden_fixture_is_self_consistent():
    # regenerate one case from scratch: the fixture file is what the generator writes
    c = _cases()[4]
    val, E = brute_force(np.array(c["D"], dtype=np.float64), c["gamma"], c["bandwidth"])
    assert val == pytest.approx(c["value"], rel=1e-14)
    np.testing.assert_allclose(E, np.array(c["E"]), rtol=1e-12)


def test_closed_forms_single_row_and_column():
    g = torch.Generator().manual_seed(3)
    D = torch.rand(1, 1, 9, generator=g) * 5
    out, _ = oracle.forward(D, 1.0, None)
    assert out.item() == pytest.approx(math.fsum(D[0, 0].double().tolist()), rel=1e-7)
    Dt = D.transpose(1, 2).contiguous()
    out_t, _ = oracle.forward(Dt, 0.37, None)
    assert out_t.item() == pytest.approx(math.fsum(D[0, 0].double().tolist()), rel=1e-7)
    one = torch.tensor([[[2.5]]])
    assert oracle.forward(one, 0.1, None)[0].item() == 2.5
    E = oracle.backward(D, oracle.forward(D, 1.0, None)[1], 1.0, None)
    # one path: every marginal is 1, up to the fp32 differences of R (ulp(R)/gamma)
    torch.testing.assert_close(E, torch.ones_like(E), rtol=0, atol=1e-5)


def test_symmetry_under_transpose():
    g = torch.Generator().manual_seed(4)
    D = torch.rand(3, 17, 23, generator=g) * 4
    a, _ = oracle.forward(D, 0.7, None)
    b, _ = oracle.forward(D.transpose(1, 2).contiguous(), 0.7, None)
    torch.testing.assert_close(a, b, rtol=1e-6, atol=0)


def test_gamma_to_zero_is_dtw():
    g = torch.Generator().manual_seed(5)
    D = torch.rand(2, 12, 15, generator=g) * 3
    out, _ = oracle.forward(D, 1e-3, None)
    for b in range(2):
        dtw = hard_dtw(D[b].double().numpy())
        assert out[b].item() <= dtw + 1e-5
        assert out[b].item() >= dtw - 1e-3 * math.log(3) * (12 + 15) - 1e-5


def test_forward_state_is_fp64_rounded_once():
    # An independent float64 recursion rounded once to fp32 reproduces the oracle's R table;
    # an fp32 running state (the reference GPU model) does not.
    g = torch.Generator().manual_seed(6)
    D = (torch.rand(1, 40, 40, generator=g) * 50).float()
    _, R32 = oracle.forward(D, 1.0, None)
    _, Rt = torch_dp64(D[0].double(), 1.0)
    ref = np.array([[float(Rt[i][j]) for j in range(1, 41)] for i in range(1, 41)], dtype=np.float64)
    ours = R32[0, 1:41, 1:41].double().numpy()
    match = (ours == ref.astype(np.float32).astype(np.float64)).mean()
    assert match > 0.995, match
    # fp32-state model for contrast
    Rf = np.full((41, 41), np.inf, dtype=np.float32)
    Rf[0, 0] = 0
    Dn = D[0].numpy()
    for i in range(1, 41):
        for j in range(1, 41):
            r = np.array([Rf[i - 1, j - 1], Rf[i - 1, j], Rf[i, j - 1]], dtype=np.float64)
            m = r.min()
            Rf[i, j] = np.float32(Dn[i - 1, j - 1]) + np.float32(m - math.log(np.exp(-(r - m)).sum()))
    match32 = (ours == Rf[1:, 1:].astype(np.float64)).mean()
    assert match32 < match - 0.05, (match32, match)


@pytest.mark.parametrize("gamma,bw", [(1.0, None), (0.1, None), (0.5, 3.0)])
def test_backward_matches_fp64_autograd(gamma, bw):
    g = torch.Generator().manual_seed(7)
    N, M = 9, 11
    D = (torch.rand(1, N, M, generator=g) * 4).float()
    out, R = oracle.forward(D, gamma, bw)
    E = oracle.backward(D, R, gamma, bw)[0].double()
    D64 = D[0].double().clone().requires_grad_(True)
    val, _ = torch_dp64(D64, gamma, bw)
    val.backward()
    assert out.item() == pytest.approx(val.item(), rel=1e-6)
    torch.testing.assert_close(E, D64.grad, rtol=1e-4, atol=1e-5)


def test_independent_fp64_recursion_passes_gradcheck():
    g = torch.Generator().manual_seed(8)
    D = (torch.rand(5, 6, generator=g, dtype=torch.float64) * 2).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda d: torch_dp64(d, 0.8)[0], (D,))


def test_backward_probability_properties():
    g = torch.Generator().manual_seed(9)
    D = (torch.rand(4, 30, 25, generator=g) * 6).float()
    _, R = oracle.forward(D, 1.0, None)
    E = oracle.backward(D, R, 1.0, None)
    slack = 16 * 2.0 ** -24 * float(R[torch.isfinite(R)].abs().max())  # ulp(R)/gamma
    assert torch.all(E >= 0) and torch.all(E <= 1 + slack)
    torch.testing.assert_close(E[:, -1, -1], torch.ones(4))
    torch.testing.assert_close(E[:, 0, 0], torch.ones(4), rtol=0, atol=1e-5)


def test_oracle_distance_matches_naive():
    # the reference's own test_sqeuclidean.py: naive broadcast, atol 1e-6
    torch.manual_seed(0)
    x = torch.randn(2, 5, 3)
    y = torch.randn(2, 7, 3)
    D = oracle.sqeuclidean(x, y)
    naive = ((x[:, :, None, :] - y[:, None, :, :]) ** 2).sum(-1)
    torch.testing.assert_close(D, naive, atol=1e-6, rtol=1e-5)  # torch.allclose defaults
    assert torch.all(oracle.sqeuclidean(x, x).diagonal(dim1=1, dim2=2) <= 1e-5)


def test_oracle_end_to_end_autograd_runs():
    # the reference's test_softdtw_cpu_runs, on the oracle
    torch.manual_seed(0)
    x = torch.randn(2, 10, 4, requires_grad=True)
    y = torch.randn(2, 11, 4)
    out = oracle.softdtw(x, y, gamma=1.0)
    out.sum().backward()
    assert torch.isfinite(out).all() and torch.isfinite(x.grad).all()


def test_oracle_fp64_path():
    torch.manual_seed(0)
    x = torch.randn(1, 6, 2, dtype=torch.float64, requires_grad=True)
    y = torch.randn(1, 5, 2, dtype=torch.float64)
    out = oracle.softdtw(x, y, gamma=1.0)
    out.sum().backward()
    assert out.dtype == torch.float64 and torch.isfinite(x.grad).all()
    # fp64 D: value equals the brute force on the same D
    D = oracle.sqeuclidean(x.detach(), y)
    val, _ = brute_force(D[0].numpy(), 1.0)
    assert out.item() == pytest.approx(val, rel=1e-12)


def test_oracle_normalize_self_is_zero():
    torch.manual_seed(1)
    x = torch.randn(3, 8, 2)
    out = oracle.softdtw(x, x.clone(), gamma=1.0, normalize=True)
    assert torch.all(out == 0)
