"""Independent pins of the oracle's normalize and barycenter loops (CPU only).

oracle.softdtw (the forward/backward restatement) is pinned elsewhere by brute force; these
tests pin what the oracle builds on top of it:

  normalize (reference module.py:99-111): sdtw(x, y) - 0.5 * (sdtw(x, x) + sdtw(y, y)), each
      term checked against brute-force path enumeration of the float64 cost, for x != y;
  barycenter (reference barycenters.py:17-180):
      * initialisation = the weighted mean with weights normalised to sum 1 (:80-90);
      * the first two optimiser steps recomputed by hand in float64 from the published Adam
        update (Kingma & Ba 2015, with torch's defaults beta = (0.9, 0.999), eps = 1e-8),
        the cosine-annealed learning rate eta_min + (lr - eta_min)(1 + cos(pi t / T)) / 2
        with eta_min = 0.1 lr and T = max_iter (:101-106), and gradient-norm clipping to 1
        (scale max_norm / (norm + 1e-6) when the norm exceeds 1, :134) applied before the
        step.  Gradients come from the pinned oracle.softdtw, one pair at a time.

Each check is also shown to reject the plausible wrong variants (a formula with the wrong
terms or split order, unnormalised weights, no clipping, eta_min = 0): the wrong variant's
value lies far outside the tolerance the check applies.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from _checkers import brute_force


# ---------------------------------------------------------------------------------------
# normalize
# ---------------------------------------------------------------------------------------
def _cost64(a, b):
    """Squared-Euclidean cost of two (N, K) sequences in float64 (closed form)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return ((a[:, None, :] - b[None, :, :]) ** 2).sum(-1)


def _brute_terms(x, y, gamma):
    """(xy, xx, yy) brute-force Soft-DTW values per pair."""
    out = []
    for b in range(x.shape[0]):
        xy, _ = brute_force(_cost64(x[b], y[b]), gamma)
        xx, _ = brute_force(_cost64(x[b], x[b]), gamma)
        yy, _ = brute_force(_cost64(y[b], y[b]), gamma)
        out.append((xy, xx, yy))
    return np.array(out)


@pytest.mark.parametrize("N,K,gamma", [(5, 2, 1.0), (6, 3, 0.5), (4, 1, 2.0)])
def test_oracle_normalize_matches_bruteforce(N, K, gamma):
    g = torch.Generator().manual_seed(11 + N)
    B = 3
    x = torch.randn(B, N, K, generator=g)
    y = torch.randn(B, N, K, generator=g) * 1.5 + 0.3
    got = oracle.softdtw(x, y, gamma=gamma, normalize=True).double().numpy()
    t = _brute_terms(x.numpy(), y.numpy(), gamma)
    want = t[:, 0] - 0.5 * (t[:, 1] + t[:, 2])
    # the fp32 cost and the fp32 rounding of each R: a few ulp of the largest term
    tol = 4e-6 * np.abs(t).max(axis=1) + 1e-6
    assert np.all(np.abs(got - want) <= tol), (got, want)
    # plausible wrong formulas are far outside that tolerance
    wrong = {
        "xy - xx": t[:, 0] - t[:, 1],
        "xy - yy": t[:, 0] - t[:, 2],
        "split (xx, xy, yy)": t[:, 1] - 0.5 * (t[:, 0] + t[:, 2]),
        "xy - (xx + yy)": t[:, 0] - (t[:, 1] + t[:, 2]),
    }
    for name, w in wrong.items():
        assert np.any(np.abs(w - want) > 100 * tol), name


def test_oracle_normalize_self_terms_not_zero_for_distinct_inputs():
    # x != y: the self terms are negative (several near-zero-cost paths), so normalize differs
    # from the plain value by a known amount
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 5, 2, generator=g)
    y = torch.randn(2, 5, 2, generator=g)
    plain = oracle.softdtw(x, y, gamma=1.0).double().numpy()
    norm = oracle.softdtw(x, y, gamma=1.0, normalize=True).double().numpy()
    t = _brute_terms(x.numpy(), y.numpy(), 1.0)
    np.testing.assert_allclose(plain - norm, 0.5 * (t[:, 1] + t[:, 2]), rtol=1e-5, atol=1e-5)
    assert np.all(t[:, 1] < 0) and np.all(t[:, 2] < 0)


# ---------------------------------------------------------------------------------------
# barycenter
# ---------------------------------------------------------------------------------------
BETA1, BETA2, EPS = 0.9, 0.999, 1e-8


def _walks(Kseq, N, D, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return scale * torch.cumsum(torch.randn(Kseq, N, D, generator=g), dim=1)


def _grad64(bary, X, w, gamma):
    """d/d bary of sum_b w_b sdtw(bary, X_b), from the pinned oracle, pair by pair."""
    g = np.zeros(bary.shape, dtype=np.float64)
    loss = 0.0
    for b in range(X.shape[0]):
        z = bary.clone().float().unsqueeze(0).requires_grad_(True)
        d = oracle.softdtw(z, X[b:b + 1], gamma=gamma)
        d.sum().backward()
        g += float(w[b]) * z.grad[0].double().numpy()
        loss += float(w[b]) * float(d.item())
    return g, loss


def _clip(g):
    n = math.sqrt(float((g * g).sum()))
    return g * (1.0 / (n + 1e-6)) if n > 1.0 else g, n


def _cosine_lr(lr, t, T):
    eta_min = 0.1 * lr
    return eta_min + (lr - eta_min) * (1 + math.cos(math.pi * t / T)) / 2


def _two_steps_by_hand(X, w, lr, gamma, T, clip=True, eta_min_frac=0.1):
    """Barycenter after one and after two iterations, computed here in float64."""
    w = np.asarray(w, dtype=np.float64)
    w = w / w.sum()
    bary = (X.double().numpy() * w[:, None, None]).sum(0)
    m = np.zeros_like(bary)
    v = np.zeros_like(bary)
    out = []
    norms = []
    for t in range(2):
        g, _ = _grad64(torch.from_numpy(bary), X, w, gamma)
        if clip:
            g, n = _clip(g)
        else:
            n = math.sqrt(float((g * g).sum()))
        norms.append(n)
        m = BETA1 * m + (1 - BETA1) * g
        v = BETA2 * v + (1 - BETA2) * g * g
        mh = m / (1 - BETA1 ** (t + 1))
        vh = v / (1 - BETA2 ** (t + 1))
        eta_min = eta_min_frac * lr
        lr_t = eta_min + (lr - eta_min) * (1 + math.cos(math.pi * t / T)) / 2
        bary = bary - lr_t * mh / (np.sqrt(vh) + EPS)
        out.append(bary.copy())
    return out, norms


def test_oracle_barycenter_init_is_normalised_weighted_mean():
    X = _walks(4, 6, 2, seed=21)
    w = torch.tensor([1.0, 2.0, 3.0, 4.0])  # deliberately not summing to 1
    # lr = 0: Adam does not move, so the result is the initialisation
    got = oracle.barycenter(X, weights=w, max_iter=1, lr=0.0, early_stopping=False)
    wn = w.double().numpy() / w.double().sum().item()
    want = np.zeros((6, 2))
    for b in range(4):
        want += wn[b] * X[b].double().numpy()
    np.testing.assert_allclose(got.double().numpy(), want, rtol=1e-6, atol=1e-6)
    # plausible wrong initialisations
    unnorm = sum(float(w[b]) * X[b].double().numpy() for b in range(4))
    plain_mean = X.double().mean(0).numpy()
    assert np.abs(unnorm - want).max() > 1e-2
    assert np.abs(plain_mean - want).max() > 1e-2


def test_oracle_barycenter_two_steps_match_hand_computed_adam():
    X = _walks(5, 6, 2, seed=22, scale=2.0)
    w = [0.5, 1.0, 1.5, 2.0, 1.0]
    lr, gamma, T = 0.1, 1.0, 2
    hist = []
    oracle.barycenter(X, weights=torch.tensor(w), max_iter=T, lr=lr, gamma=gamma,
                      early_stopping=False, history=hist)
    (b1, b2), norms = _two_steps_by_hand(X, w, lr, gamma, T)
    # both gradients exceed the clip norm, with different norms: clipping changes the
    # relative weight of the two gradients in Adam's second step
    assert norms[0] > 1.5 and norms[1] > 1.5 and abs(norms[0] - norms[1]) > 0.1
    tol = 2e-5
    np.testing.assert_allclose(hist[0][1].double().numpy(), b1, rtol=0, atol=tol)
    np.testing.assert_allclose(hist[1][1].double().numpy(), b2, rtol=0, atol=tol)
    # the loss history is the weighted objective before each step
    wn = np.asarray(w) / np.sum(w)
    _, loss0 = _grad64(torch.from_numpy((X.double().numpy() * wn[:, None, None]).sum(0)), X, wn, gamma)
    assert hist[0][0] == pytest.approx(loss0, rel=1e-6)
    # the wrong variants move the second step far beyond that tolerance
    (_, b2_noclip), _ = _two_steps_by_hand(X, w, lr, gamma, T, clip=False)
    (_, b2_eta0), _ = _two_steps_by_hand(X, w, lr, gamma, T, eta_min_frac=0.0)
    assert np.abs(b2_noclip - b2).max() > 50 * tol
    assert np.abs(b2_eta0 - b2).max() > 50 * tol


def test_oracle_barycenter_rejects_planted_schedule_and_clip_mistakes(monkeypatch):
    """The two-step check fails when a mistake is planted in the oracle's loop (here by
    swapping the library pieces it calls for wrong ones)."""
    X = _walks(5, 6, 2, seed=22, scale=2.0)
    w = [0.5, 1.0, 1.5, 2.0, 1.0]
    lr, gamma, T = 0.1, 1.0, 2
    (_, b2), _ = _two_steps_by_hand(X, w, lr, gamma, T)

    def second_step():
        hist = []
        oracle.barycenter(X, weights=torch.tensor(w), max_iter=T, lr=lr, gamma=gamma,
                          early_stopping=False, history=hist)
        return np.abs(hist[1][1].double().numpy() - b2).max()

    real_sched = torch.optim.lr_scheduler.CosineAnnealingLR
    with monkeypatch.context() as mp:
        mp.setattr(torch.optim.lr_scheduler, "CosineAnnealingLR",
                   lambda opt, T_max, eta_min: real_sched(opt, T_max=T_max, eta_min=0.0))
        assert second_step() > 1e-3
    with monkeypatch.context() as mp:
        mp.setattr(torch.nn.utils, "clip_grad_norm_", lambda params, max_norm: None)
        assert second_step() > 1e-3
    assert second_step() < 2e-5


def test_oracle_barycenter_early_stopping_rule():
    # early stopping only in the second half, after `patience` non-improving iterations
    # (barycenters.py:149-165): with tol huge every iteration counts as non-improving
    X = _walks(3, 5, 2, seed=23)
    hist = []
    oracle.barycenter(X, max_iter=20, lr=0.1, early_stopping=True, patience=3, tol=1e9,
                      history=hist)
    # stops at the first iteration it > max_iter // 2 = 10 with wait >= 3: it = 11
    assert len(hist) == 12
