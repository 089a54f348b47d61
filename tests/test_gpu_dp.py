"""GPU Soft-DTW recursion kernels vs the CPU oracle, given identical costs.

Every cell arithmetic is checked.  exact and mixed (exact forward): R bit-identical to the
oracle's.  fast: R within 1e-6 relative (the north-star forward tolerance is 1e-5) with the
same infinite cells.  All: out within rtol 1e-5, E (= G with g = 1) within rtol 1e-4 /
atol 1e-5 given the same D and R (exact: to the last bit but for rare cells; mixed: within
rtol 1e-5 / atol 1e-7), and the brute-force golden vectors.
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from _gpu_util import (FWD_RTOL, GRAD_ATOL, GRAD_RTOL, engine_R_from_oracle, grad_violation,
                       max_rel_err, no_less_accurate, numerics, randn_pair, say)
from softdtw_cuda import _engine

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bruteforce.json")


def _golden():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


MODES = ["exact", "mixed", "fast"]


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("case", _golden(), ids=lambda c: f"N{c['N']}M{c['M']}g{c['gamma']}bw{c['bandwidth']}")
def test_dp_matches_bruteforce_golden(case, mode):
    D = torch.tensor(case["D"], dtype=torch.float32).unsqueeze(0).cuda()
    bw = -1.0 if case["bandwidth"] is None else case["bandwidth"]
    with numerics(mode):
        out, R = _engine.dtw_fwd(D, case["gamma"], bw)
        E = _engine.dtw_bwd(D, R, case["gamma"], bw).cpu()[0].numpy()
    np.testing.assert_allclose(out.item(), case["value"], rtol=2e-6, atol=1e-6)
    rmax = float(R[torch.isfinite(R)].abs().max())
    tol = max(1e-5, 8 * 2.0 ** -24 * rmax / case["gamma"])
    np.testing.assert_allclose(E, np.array(case["E"]), rtol=tol, atol=tol)


CASES = [
    # B, N, M, K, gamma, bandwidth
    (4, 64, 64, 8, 1.0, None),        # config 1
    (2, 12, 9, 3, 1.0, None),
    (3, 37, 53, 4, 0.5, None),
    (2, 100, 80, 6, 0.1, 10.0),       # band, non-square
    (2, 64, 64, 3, 0.01, None),       # sharp soft-min
    (32, 512, 512, 64, 1.0, None),    # config 2 (headline)
    (2, 1300, 700, 3, 1.0, None),     # N > 1024: several row blocks
    (2, 700, 1300, 3, 0.3, 50.0),
    (2, 192, 160, 5, 0.5, None),      # full last band with interior groups
    (2, 64, 300, 4, 1.0, None),       # one full band, interior groups
]


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("B,N,M,K,gamma,bw", CASES)
def test_dp_forward_backward_vs_oracle_same_D(B, N, M, K, gamma, bw, mode):
    say(f"[dp] {mode} B={B} N={N} M={M} gamma={gamma} bw={bw}")
    x, y = randn_pair(B, N, M, K, seed=B + N + M)
    D = oracle.sqeuclidean(x, y)
    out_o, R_o = oracle.forward(D, gamma, bw)
    bwv = -1.0 if bw is None else bw
    Dg = D.cuda()
    Rref = engine_R_from_oracle(R_o)
    E_o = oracle.backward(D, R_o, gamma, bw)
    with numerics(mode):
        out, R = _engine.dtw_fwd(Dg, gamma, bwv)
        E = _engine.dtw_bwd(Dg, _engine.table_pack(Rref.cuda()), gamma, bwv).cpu()
        E2 = _engine.dtw_bwd(Dg, R, gamma, bwv).cpu()
    Rc = _engine.table_unpack(R, B, N, M).cpu()
    if mode in ("exact", "mixed"):
        same = (Rc == Rref) | (torch.isinf(Rc) & torch.isinf(Rref))
        rate = same.double().mean().item()
        say(f"    R bit-equal rate {rate:.6f}")
        assert rate == 1.0
    else:
        err = max_rel_err(Rc, Rref)
        say(f"    R max relative error {err:.3e}")
        assert err <= 1e-6
    torch.testing.assert_close(out.cpu(), out_o, rtol=FWD_RTOL, atol=0)
    # backward from identical D and R
    v = grad_violation(E, E_o)
    say(f"    E violation {v:.4f} (<= 1 passes)")
    assert v <= 1.0
    if mode == "exact":
        # fp64-accurate (not correctly rounded) exp: rare last-bit differences of E
        erate = (E == E_o).double().mean().item()
        say(f"    E bit-equal rate {erate:.6f}")
        assert erate >= 0.999
    if mode == "mixed":
        # fp32 hardware exp2 of the CPU path's own fp32 differences: ~1e-6 relative
        vt = grad_violation(E, E_o, rtol=1e-5, atol=1e-7)
        say(f"    mixed E violation at rtol 1e-5 / atol 1e-7: {vt:.4f}")
        assert vt <= 1.0
    # and from the engine's own R
    v2 = grad_violation(E2, E_o)
    say(f"    E (own R) violation {v2:.4f}")
    if mode == "fast":
        # E takes differences of R: one-ulp differences of R move E by ~ulp(R)/gamma, the
        # noise the CPU path itself carries against an fp64 evaluation
        D64 = D.double()
        _, R64p = oracle.forward(D64, gamma, bw)
        E64 = oracle.backward(D64, R64p, gamma, bw)
        ok, v32, v64, vref = no_less_accurate(E2, E_o, E64)
        say(f"    fast E (own R): vs CPU path {v32:.3f}, vs fp64 {v64:.3f} (CPU path vs fp64 {vref:.3f})")
        assert ok
        return
    if not v2 <= 1.0:
        bad = ~torch.isclose(E2, E_o, rtol=1e-4, atol=1e-5)
        idx = bad.nonzero()
        say(f"    {bad.sum().item()} bad cells; rows by band: "
            f"{sorted(set((idx[:, 1] // 64).tolist()))[:20]}; cols {idx[:, 2].min().item()}..{idx[:, 2].max().item()}; "
            f"pairs {sorted(set(idx[:, 0].tolist()))}; E1 vs E2 equal: {torch.equal(E, E2)}")
    assert v2 <= 1.0


def test_numerics_switch():
    prev = _engine.set_numerics("exact")
    try:
        assert _engine.get_numerics() == "exact"
        assert _engine.set_numerics("fast") == "exact"
        assert _engine.get_numerics() == "fast"
        assert _engine.set_numerics("mixed") == "fast"
        assert _engine.load().sdtw_get_numerics() == 2
        assert _engine.set_numerics("fast") == "mixed"
        with pytest.raises(ValueError):
            _engine.set_numerics("bf16")
        assert _engine.load().sdtw_set_numerics(7) == -1
        assert _engine.get_numerics() == "fast"
    finally:
        _engine.set_numerics(prev)


def test_backward_scales_by_grad_output():
    x, y = randn_pair(3, 20, 30, 4, seed=5)
    D = oracle.sqeuclidean(x, y).cuda()
    out, R = _engine.dtw_fwd(D, 1.0, -1.0)
    g = torch.tensor([0.5, -2.0, 3.0]).cuda()
    G = _engine.dtw_bwd(D, R, 1.0, -1.0, gout=g)
    E = _engine.dtw_bwd(D, R, 1.0, -1.0)
    torch.testing.assert_close(G, g.view(-1, 1, 1) * E, rtol=0, atol=0)


@pytest.mark.parametrize("K", [1, 33, 100])
def test_fused_feature_widths_match_unfused(K):
    # K = 1: matrix-core tiles padded from 1 to 4 features; K = 33: padded to 64; K = 100:
    # the scalar tile fallback beyond the register-resident width
    B, N, M = 2, 150, 90
    x, y = randn_pair(B, N, M, K, seed=K)
    xg, yg = x.cuda(), y.cuda()
    D = _engine.sqeuclid_fwd(xg, yg)
    assert torch.equal(D.cpu(), oracle.sqeuclidean(x, y))
    o1, R1 = _engine.dtw_fwd(D, 0.5, -1.0)
    o2, R2 = _engine.fused_fwd(xg, yg, 0.5, -1.0)
    assert torch.equal(o1, o2) and torch.equal(R1, R2)
    E1 = _engine.dtw_bwd(D, R1, 0.5, -1.0)
    E2 = _engine.fused_bwd_e(xg, yg, R2, 0.5, -1.0)
    assert torch.equal(E1, E2)


def _linear_domain(B, N, M, K, bw):
    """Whether the fused forward of this call takes the scaled linear-domain recursion:
    mixed arithmetic, no band, matrix-core costs, 1 or 2 bands per workgroup."""
    return (_engine.get_numerics() == "mixed" and not bw > 0
            and _engine.fused_costs_on_matrix_cores(N, M, K)
            and _engine.fused_bands_per_workgroup(B, N, M, K, "cuda") <= 2)


def _oracle_R_check(R, D, gamma, bw, B, N, M):
    """Against the CPU path on the same D: the share of the engine R table's cells with its
    fp32 bits (both +inf counts as equal), the largest distance in fp32 ulps of the finite
    ones (the same infinities required), and the CPU path's out."""
    out_o, R_o = oracle.forward(D.cpu(), gamma, None if bw <= 0 else bw)
    Rref = engine_R_from_oracle(R_o)
    Rc = _engine.table_unpack(R, B, N, M).cpu()
    same = (Rc == Rref) | (torch.isinf(Rc) & torch.isinf(Rref))
    assert torch.equal(torch.isfinite(Rc), torch.isfinite(Rref))
    fin = torch.isfinite(Rref)
    ulps = (Rc[fin].view(torch.int32).long() - Rref[fin].view(torch.int32).long()).abs()
    return same.double().mean().item(), int(ulps.max().item()) if ulps.numel() else 0, out_o


# The scaled linear-domain forward evaluates the recursion more accurately than the CPU
# path's log-domain form (a few gamma 2^-53 per cell against ulp(R)), so where the CPU path's
# own fp64 rounding puts a cell next to an fp32 rounding boundary the two can round to
# neighbouring floats: R within one fp32 ulp everywhere, with a few cells in 10^4 differing
# on some inputs (none of the 8.4M at the headline shape).  The log-domain D-reading forward
# shows such cells too, on other inputs.
LIN_RATE = 0.999


@pytest.mark.parametrize("mode", MODES)
def test_fused_matches_unfused_kernels(mode):
    # fused recomputes the same cost bits.  Under exact and fast arithmetic, and with a band,
    # both run the same recursion: identical out / R / E.  Under mixed arithmetic the fused
    # forward of an unbanded call is the scaled linear-domain recursion and the D-reading one
    # the log-domain form: each gives R within one fp32 ulp of the CPU path's, and the fused
    # backward equals the D-reading one on the same R.  The shapes with 300 and 70
    # pairs need more 2-band workgroups than the GPU has CUs, so the fused launch takes 4
    # bands per workgroup (the log-domain recursion, producers sharing their compute waves'
    # SIMDs), one of them with cross-workgroup boundaries and a partial last workgroup.
    for (B, N, M, K, bw) in [(3, 50, 40, 5, -1.0), (2, 12, 9, 3, -1.0), (2, 1100, 300, 4, -1.0),
                             (300, 200, 150, 16, -1.0), (70, 600, 100, 8, -1.0),
                             (70, 600, 100, 8, 40.0), (2, 1, 7, 3, -1.0), (2, 7, 1, 3, -1.0),
                             (1, 65, 1, 2, -1.0)]:
        say(f"[fused vs unfused] mode={mode} B={B} N={N} M={M} K={K} bw={bw}")
        x, y = randn_pair(B, N, M, K, seed=N)
        xg, yg = x.cuda(), y.cuda()
        with numerics(mode):
            D = _engine.sqeuclid_fwd(xg, yg)
            o1, R1 = _engine.dtw_fwd(D, 0.7, bw)
            o2, R2 = _engine.fused_fwd(xg, yg, 0.7, bw)
            E2 = _engine.fused_bwd_e(xg, yg, R2, 0.7, bw)
            E2d = _engine.dtw_bwd(D, R2, 0.7, bw)
            lin = _linear_domain(B, N, M, K, bw)
        assert torch.equal(E2, E2d)
        if not lin:
            assert torch.equal(o1, o2) and torch.equal(R1, R2)
        else:
            r1, u1, out_o = _oracle_R_check(R1, D, 0.7, bw, B, N, M)
            r2, u2, _ = _oracle_R_check(R2, D, 0.7, bw, B, N, M)
            say(f"    R vs CPU path: D-reading rate {r1:.8f} (max {u1} ulp), fused rate {r2:.8f} "
                f"(max {u2} ulp)")
            assert u1 <= 1 and r1 >= LIN_RATE and u2 <= 1 and r2 >= LIN_RATE
            torch.testing.assert_close(o2.cpu(), out_o, rtol=FWD_RTOL, atol=0)


@pytest.mark.parametrize("mode", ["mixed", "fast", "exact"])
@pytest.mark.parametrize("B,N,M,gamma,bw", [
    (4, 512, 512, 1.0, -1.0),    # full bands, the row below read from the next band's R and D
    (3, 150, 120, 0.7, 30.0),    # Sakoe-Chiba band, a partial last band
    (2, 100, 77, 0.1, -1.0),     # sharp soft-min, the corner inside a partial band
    (3, 70, 10, 1.0, -1.0),      # fewer columns than a group
])
def test_weight_wave_backward_matches_classic(mode, B, N, M, gamma, bw):
    # The D-reading backward takes one band per workgroup with weight waves where the
    # batch's one-band workgroups all fit on the GPU, else the classic geometry (4 bands per
    # workgroup, the weights in the compute wave).  Pairs are
    # independent, so the same pairs inside a batch too large for one-band workgroups give
    # the classic result: G must be identical to the bit, with an upstream gradient too.
    nb = (N + 63) // 64
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    Bbig = cus // nb + 1
    assert B * nb <= cus < Bbig * nb
    say(f"[weight wave] mode={mode} B={B} (classic batch {Bbig}) N={N} M={M} gamma={gamma} bw={bw}")
    x, y = randn_pair(Bbig, N, M, 6, seed=N + M)
    with numerics(mode):
        D = _engine.sqeuclid_fwd(x.cuda(), y.cuda())
        _, R = _engine.dtw_fwd(D, gamma, bw)
        g = torch.linspace(0.5, 2.0, Bbig, device=D.device)
        Gbig = _engine.dtw_bwd(D, R, gamma, bw, gout=g)
        Ds = D[:B].contiguous()
        S = (M + 63 + 15) // 16 * 16  # steps per band of the R table (pairs are contiguous)
        Rs = R[:B * nb * S * 64].contiguous()
        Gs = _engine.dtw_bwd(Ds, Rs, gamma, bw, gout=g[:B].contiguous())
    assert torch.isfinite(Gs).all()
    assert torch.equal(Gs, Gbig[:B])


@pytest.mark.parametrize("mode", ["mixed", "exact"])
def test_weight_wave_backward_nonfinite_costs(mode):
    # +inf costs (pair 0, two of them on the rows either side of a band boundary; +inf R
    # maps to -inf, so some cells' weights are exp(+inf) and their E is NaN, as in the
    # reference's kernels) and a NaN cost (pair 1; the reference's kernels take any D): the
    # weight-wave geometry gives the classic geometry's G to the bit where it is a number,
    # and NaN in the same cells (the sign of a NaN result is not specified, and the
    # compilers' forms of a - b differ in it).
    B, N, M = 2, 130, 90
    nb = (N + 63) // 64
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    Bbig = cus // nb + 1
    say(f"[weight wave, non-finite D] mode={mode} B={B} (classic batch {Bbig}) N={N} M={M}")
    g = torch.Generator().manual_seed(7)
    D = torch.rand((Bbig, N, M), generator=g) * 3.0
    D[0, 5, 7] = float("inf")
    D[0, 64, 40] = float("inf")       # the first row of a band below
    D[0, 63, 41] = float("inf")       # the last row of a band above
    D[1, 100, 3] = float("nan")
    D = D.cuda()
    with numerics(mode):
        _, R = _engine.dtw_fwd(D, 0.8, -1.0)
        Gbig = _engine.dtw_bwd(D, R, 0.8, -1.0)
        S = (M + 63 + 15) // 16 * 16
        Gs = _engine.dtw_bwd(D[:B].contiguous(), R[:B * nb * S * 64].contiguous(), 0.8, -1.0)
    Gc = Gbig[:B]
    nan_s, nan_c = torch.isnan(Gs), torch.isnan(Gc)
    assert nan_s[1].any() and (~nan_s[0]).any()
    assert torch.equal(nan_s, nan_c)
    assert torch.equal(Gs[~nan_s].view(torch.int32), Gc[~nan_c].view(torch.int32))


@pytest.mark.parametrize("B,N,M,K,gamma,scale", [
    (32, 512, 512, 64, 1.0, None),   # the headline shape: one band per workgroup
    (64, 512, 128, 16, 0.5, None),   # 512 bands: two per workgroup (LDS and global handover)
    (2, 150, 200, 8, 1.0, None),     # a partial last band
    (2, 200, 180, 8, 0.05, None),    # sharp soft-min
    (3, 70, 10, 4, 1.0, None),       # fewer columns than a group (no interior group)
    (3, 200, 150, 8, 0.01, 300.0),   # pair 1 past the linear domain's bound: log domain
    (3, 200, 150, 8, 1.0, "nan"),    # pair 2 with a NaN feature: log domain, NaN results
])
def test_linear_domain_forward_vs_oracle(B, N, M, K, gamma, scale):
    # the fused forward's scaled linear-domain recursion (mixed arithmetic, no band),
    # against the CPU path's recursion on the same cost bits (the one-launch forward's D):
    # R within one fp32 ulp, out to its tolerance; pairs whose norms fall outside the linear
    # domain run the log-domain recursion in the same launch.  fused_fwd, which keeps no D,
    # gives the same out and R.
    say(f"[linear domain] B={B} N={N} M={M} K={K} gamma={gamma} scale={scale} "
        f"bands/workgroup {_engine.fused_bands_per_workgroup(B, N, M, K, 'cuda')}")
    x, y = randn_pair(B, N, M, K, seed=B + N + M)
    if scale == "nan":
        x[2, 5, 1] = float("nan")
    elif scale is not None:
        x[1] *= scale
        y[1] *= scale
    assert _linear_domain(B, N, M, K, -1.0)
    out, R, Dg, _ = _engine.fused_fwd_d(x.cuda(), y.cuda(), gamma, -1.0)
    out2, R2 = _engine.fused_fwd(x.cuda(), y.cuda(), gamma, -1.0)
    torch.testing.assert_close(out2, out, rtol=0, atol=0, equal_nan=True)
    torch.testing.assert_close(R2, R, rtol=0, atol=0, equal_nan=True)
    out_o, R_o = oracle.forward(Dg.cpu(), gamma, None)
    Rc = _engine.table_unpack(R, B, N, M).cpu()
    Rref = engine_R_from_oracle(R_o)
    nan = torch.isnan(Rref)
    assert torch.equal(torch.isnan(Rc), nan)
    same = (Rc == Rref) | (torch.isinf(Rc) & torch.isinf(Rref)) | nan
    fin = torch.isfinite(Rref)
    assert torch.equal(torch.isfinite(Rc), fin)
    ulps = (Rc[fin].view(torch.int32).long() - Rref[fin].view(torch.int32).long()).abs()
    rate = same.double().mean().item()
    say(f"    R bit-equal rate {rate:.8f}, max {int(ulps.max())} ulp")
    assert int(ulps.max()) <= 1 and rate >= LIN_RATE
    torch.testing.assert_close(out.cpu(), out_o, rtol=FWD_RTOL, atol=0, equal_nan=True)


@pytest.mark.parametrize("B,N,M,K,bw", [(3, 100, 80, 16, -1.0), (2, 130, 70, 64, 20.0),
                                        (300, 200, 150, 16, -1.0), (70, 600, 100, 8, 40.0)])
def test_unfused_one_launch_forward_matches_two_calls(B, N, M, K, bw):
    # D from the fused forward's producers has the distance kernel's bits, and R / out are the
    # recursion over it (2-band and 4-band fused geometries, with and without a band)
    say(f"[one-launch unfused forward] B={B} N={N} M={M} K={K} bw={bw}")
    x, y = randn_pair(B, N, M, K, seed=N)
    xg, yg = x.cuda(), y.cuda()
    D1 = _engine.sqeuclid_fwd(xg, yg)
    o1, R1 = _engine.dtw_fwd(D1, 0.7, bw)
    o2, R2, D2, rec = _engine.fused_fwd_d(xg, yg, 0.7, bw)
    assert torch.equal(D1, D2)
    if not _linear_domain(B, N, M, K, bw):
        assert torch.equal(R1, R2) and torch.equal(o1, o2)
    else:
        # the linear-domain recursion (unbanded, exact or mixed arithmetic)
        r2, u2, out_o = _oracle_R_check(R2, D1, 0.7, bw, B, N, M)
        say(f"    fused R vs CPU path: rate {r2:.8f}, max {u2} ulp")
        assert u2 <= 1 and r2 >= LIN_RATE
        torch.testing.assert_close(o2.cpu(), out_o, rtol=FWD_RTOL, atol=0)
    # the distance record: per pair 1 exactly where it holds a cost that is not positive,
    # then the row norms (256-byte aligned parts) with the norms kernel's bits
    cl = rec[:4 * B].view(torch.int32)
    want = (~(D1 > 0)).flatten(1).any(dim=1).to(torch.int32)
    assert torch.equal(cl, want)
    up = lambda n: (n + 255) // 256 * 256
    x2 = rec[up(4 * B):up(4 * B) + 4 * B * N].view(torch.float32)
    y2 = rec[up(4 * B) + up(4 * B * N):up(4 * B) + up(4 * B * N) + 4 * B * M].view(torch.float32)
    # the row norms of the reference's op sequence (oracle.sqeuclidean: (x * x).sum(-1))
    assert torch.equal(x2.cpu(), (x * x).sum(dim=-1).flatten())
    assert torch.equal(y2.cpu(), (y * y).sum(dim=-1).flatten())


@pytest.mark.parametrize("bandwidth", [None, 15.0])
def test_unfused_module_matches_two_node_graph(bandwidth):
    # SoftDTW(fused=False) takes the one-launch forward; its loss and gradients equal those of
    # pairwise_distance followed by SoftDTWAutograd (the reference's unfused graph)
    from softdtw_cuda import SoftDTW
    from softdtw_cuda.autograd import SoftDTWAutograd
    from softdtw_cuda.distances import pairwise_distance

    x, y = randn_pair(4, 90, 70, 8, seed=3)
    xa, ya = x.cuda().requires_grad_(True), y.cuda().requires_grad_(True)
    out_a = SoftDTW(gamma=0.5, bandwidth=bandwidth, fused=False)(xa, ya)
    out_a.sum().backward()
    xb, yb = x.cuda().requires_grad_(True), y.cuda().requires_grad_(True)
    out_b = SoftDTWAutograd.apply(pairwise_distance(xb, yb, dist="sqeuclidean"), 0.5, bandwidth)
    out_b.sum().backward()
    assert torch.equal(out_a, out_b)
    assert torch.equal(xa.grad, xb.grad) and torch.equal(ya.grad, yb.grad)


def test_unfused_normalize_matches_two_node_graph():
    # normalize=True, fused=False: x-y minus half of x-x and y-y, each term through the
    # one-launch forward; equal to pairwise_distance + SoftDTWAutograd term by term
    from softdtw_cuda import SoftDTW
    from softdtw_cuda.autograd import SoftDTWAutograd
    from softdtw_cuda.distances import pairwise_distance

    x, y = randn_pair(3, 80, 80, 8, seed=11)
    xa, ya = x.cuda().requires_grad_(True), y.cuda().requires_grad_(True)
    out_a = SoftDTW(gamma=0.5, normalize=True, fused=False)(xa, ya)
    out_a.sum().backward()
    xb, yb = x.cuda().requires_grad_(True), y.cuda().requires_grad_(True)

    def term(a, b):
        return SoftDTWAutograd.apply(pairwise_distance(a, b, dist="sqeuclidean"), 0.5, None)

    out_b = term(xb, yb) - 0.5 * (term(xb, xb) + term(yb, yb))
    out_b.sum().backward()
    torch.testing.assert_close(out_a, out_b, rtol=1e-6, atol=1e-5)
    torch.testing.assert_close(xa.grad, xb.grad, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(ya.grad, yb.grad, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_fused_normalize_node_matches_concatenation_graph(dtype):
    # normalize=True, fused=True runs one autograd node (SoftDTWNormalizedXYAutograd); the
    # reference's concatenation trick as separate graph nodes gives the same loss bits and the
    # same gradients up to the order the three appearances of each input are summed in
    from softdtw_cuda import SoftDTW
    from softdtw_cuda.autograd_xy import SoftDTWXYAutograd

    x, y = randn_pair(4, 96, 96, 16, seed=12)
    x, y = x.to(dtype), y.to(dtype)
    xa, ya = x.cuda().requires_grad_(True), y.cuda().requires_grad_(True)
    out_a = SoftDTW(gamma=0.7, normalize=True, fused=True)(xa, ya)
    (out_a * torch.arange(1, 5, device="cuda", dtype=dtype)).sum().backward()
    xb, yb = x.cuda().requires_grad_(True), y.cuda().requires_grad_(True)
    out = SoftDTWXYAutograd.apply(torch.cat([xb, xb, yb]), torch.cat([yb, xb, yb]), 0.7, None)
    o_xy, o_xx, o_yy = out.split(4, dim=0)
    out_b = o_xy - 0.5 * (o_xx + o_yy)
    (out_b * torch.arange(1, 5, device="cuda", dtype=dtype)).sum().backward()
    assert torch.equal(out_a, out_b)
    tol = dict(rtol=1e-6, atol=1e-6) if dtype == torch.float32 else dict(rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(xa.grad, xb.grad, **tol)
    torch.testing.assert_close(ya.grad, yb.grad, **tol)


def _same_R(Rc, Ro):
    """R tables equal as the CPU path leaves them: NaN where it has NaN, the same infinities,
    and every finite value with the same bits."""
    assert torch.equal(torch.isnan(Rc), torch.isnan(Ro)), "NaN pattern differs"
    fin = ~torch.isnan(Ro)
    assert torch.equal(Rc[fin], Ro[fin]), "values differ"


@pytest.mark.parametrize("mode", ["exact", "mixed"])
@pytest.mark.parametrize("N,M", [(200, 150), (700, 180)])
def test_dp_forward_nonfinite_costs_vs_oracle(N, M, mode):
    """Costs with NaN and +inf entries in chosen bands.  The forward runs a band with the
    finite-input cell only while its inputs are finite, and switches to the general cell
    (NaN restored, all-+inf predecessors give NaN as in the reference) from the group that
    first sees a non-finite cost or a non-finite entry of the band above; at 700 rows the
    entries also cross workgroups through the helper wave."""
    say(f"[dp nonfinite] {mode} N={N} M={M}")
    B = 4
    x, y = randn_pair(B, N, M, 3, seed=N + 7)
    D = oracle.sqeuclidean(x, y)
    D[0, N // 2, M // 3] = float("nan")          # a NaN in a middle band
    D[1, 5, 5] = float("inf")                    # +inf in band 0
    D[1, N - 40, 2] = float("inf")               # and in the last band, near the left edge
    D[2, 63, 10] = float("inf")                  # the last row of band 0: crosses to band 1
    D[2, 0, M - 1] = float("nan")                # top-right corner: reaches only column M - 1
    # pair 3 stays finite
    out_o, R_o = oracle.forward(D, 1.0, None)
    with numerics(mode):
        out, R = _engine.dtw_fwd(D.cuda(), 1.0, -1.0)
    Rc = _engine.table_unpack(R, B, N, M).cpu()
    _same_R(Rc, engine_R_from_oracle(R_o))
    _same_R(out.cpu(), out_o)
    # the NaN spreads to every cell after it; an infinite cost leaves only its own cell
    # infinite (its neighbours keep a finite predecessor)
    assert torch.isnan(Rc[0]).any() and torch.isposinf(Rc[1]).any() and torch.isfinite(Rc[3]).all()


def test_fused_forward_nonfinite_inputs_vs_oracle():
    """x with a NaN feature and an infinite one: the producer waves' cost tiles carry them,
    and the recursion switches to the general cell as in the unfused forward."""
    B, N, M, K = 3, 300, 260, 8
    x, y = randn_pair(B, N, M, K, seed=11)
    x[0, 150, 2] = float("nan")
    x[1, 70, 0] = float("inf")
    D = oracle.sqeuclidean(x, y)
    out_o, R_o = oracle.forward(D, 0.5, None)
    out, R = _engine.fused_fwd(x.cuda(), y.cuda(), 0.5, -1.0)
    Rc = _engine.table_unpack(R, B, N, M).cpu()
    _same_R(Rc, engine_R_from_oracle(R_o))
    _same_R(out.cpu(), out_o)
