"""sdtw_fwd_f32_noalloc (the forward without a workspace or any allocation) against
sdtw_fwd_f32, through the C ABI.

Both run the same kernels, so out and the R table must be identical bit for bit.  Two calls
of the no-allocation entry point run back to back, the second on a smaller input: the static
scratch still holds the first call's ticket, flag and cross-workgroup rows, which the second
call must reset rather than read.
"""
import pytest
import torch

from _gpu_util import randn_pair, say
from softdtw_cuda import _engine

pytestmark = pytest.mark.gpu


def _cost(B, N, M, K, seed):
    x, y = randn_pair(B, N, M, K, seed=seed)
    return _engine.sqeuclid_fwd(x.cuda(), y.cuda())


def test_noalloc_forward_matches_workspace_forward():
    cases = [
        # B, N, M, K, gamma, bandwidth: several workgroups per pair, then a smaller one
        (8, 700, 500, 6, 1.0, -1.0),
        (3, 130, 120, 4, 0.5, 20.0),  # the band (|i - j| <= 20) covers the corner
    ]
    Ds = [_cost(B, N, M, K, seed=N + M) for (B, N, M, K, _, _) in cases]
    got = []
    for D, (B, N, M, K, g, bw) in zip(Ds, cases):
        say(f"[noalloc] B={B} N={N} M={M} gamma={g} bw={bw}")
        # preallocated outputs: the call itself allocates nothing
        R = torch.empty((_engine.table_elems(B, N, M),), dtype=torch.float32, device="cuda")
        out = torch.empty((B,), dtype=torch.float32, device="cuda")
        got.append(_engine.dtw_fwd_noalloc(D, g, bw, R=R, out=out))
    torch.cuda.synchronize()
    for D, (B, N, M, K, g, bw), (out, R) in zip(Ds, cases, got):
        out_ref, R_ref = _engine.dtw_fwd(D, g, bw)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert torch.equal(out, out_ref)
        assert torch.equal(R, R_ref)
    # and once more at the first shape, after the smaller call
    B, N, M, K, g, bw = cases[0]
    out2, R2 = _engine.dtw_fwd_noalloc(Ds[0], g, bw)
    torch.cuda.synchronize()
    assert torch.equal(out2, got[0][0]) and torch.equal(R2, got[0][1])


def test_noalloc_rejects_shapes_beyond_its_scratch():
    lib = _engine.load()
    limit = lib.sdtw_fwd_f32_noalloc_scratch_limit()
    assert limit == 16 << 20
    # B * ceil(ceil(N/64)/4) * (M + 128) * 16 bytes of rows: B = 64, N = 4096, M = 8192 needs
    # 64 * 16 * 8320 * 16 = 136 MB
    B, N, M = 64, 4096, 8192
    assert lib.sdtw_workspace_bytes(_engine.OP_FWD, B, N, M, 0) > limit
    D = torch.empty((1,), device="cuda")  # never read: the size check comes first
    rc = lib.sdtw_fwd_f32_noalloc(_engine._ptr(D), _engine._ptr(D), _engine._ptr(D), B, N, M,
                                  1.0, -1.0, _engine._stream(D.device))
    assert rc == 6
    assert "no-allocation" in _engine.strerror(rc)
