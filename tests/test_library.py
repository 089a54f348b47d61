"""The C-ABI library: it exists, loads, and exports every entry point include/sdtw.h
declares; argument validation answers without touching a device."""
import ctypes
import os
import re

import pytest

from softdtw_cuda import _engine

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sdtw.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sdtw_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    for must in ("sdtw_fwd_f32", "sdtw_bwd_f32", "sdtw_fused_fwd_f32", "sdtw_fused_bwd_f32",
                 "sdtw_sqeuclid_fwd_f32", "sdtw_sqeuclid_bwd_f32", "sdtw_workspace_bytes",
                 "sdtw_strerror"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _engine.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_engine.exported_symbols()) == set(_declared())


def test_status_strings_and_version():
    lib = _engine.load()
    assert lib.sdtw_version() >= 1
    assert _engine.strerror(0) == "success"
    assert "workspace" in _engine.strerror(2)


def test_invalid_arguments_rejected_before_launch():
    lib = _engine.load()
    null = ctypes.c_void_p(0)
    # N = 0, gamma <= 0, gamma = inf: rejected by validation, no HIP call is made
    assert lib.sdtw_fwd_f32(null, null, null, 1, 0, 4, 1.0, -1.0, null, 0, null) == 1
    assert lib.sdtw_fwd_f32(null, null, null, 1, 4, 4, 0.0, -1.0, null, 0, null) == 1
    assert lib.sdtw_bwd_f32(null, null, null, null, 1, 4, 4, float("inf"), -1.0, null, 0, null) == 1
    assert lib.sdtw_fused_fwd_f32(null, null, null, null, 1, 4, 4, 0, 1.0, -1.0, null, 0, null) == 1
    # empty batch is a no-op success
    assert lib.sdtw_fwd_f32(null, null, null, 0, 4, 4, 1.0, -1.0, null, 0, null) == 0


def test_workspace_sizes():
    lib = _engine.load()
    B, N, M, K = 32, 512, 512, 64
    assert lib.sdtw_workspace_bytes(_engine.OP_FWD, B, N, M, K) >= 8 * B * M
    # the fused backward forms the gradients in the recursion kernel with matrix-core costs:
    # its workspace holds nothing of (B, N, M) size (norms, row scratch, one flag per tile)
    assert lib.sdtw_workspace_bytes(_engine.OP_FUSED_BWD, B, N, M, K) < B * N * M * 4 // 8
    # wider features take the scalar cost tiles, whose backward reduces g*E from the workspace
    assert lib.sdtw_workspace_bytes(_engine.OP_FUSED_BWD, B, N, M, 96) >= 4 * B * N * M
    # so does every fused backward forming dL/dy under the deterministic setting
    prev = lib.sdtw_set_deterministic(1)
    try:
        assert lib.sdtw_workspace_bytes(_engine.OP_FUSED_BWD, B, N, M, K) >= 4 * B * N * M
    finally:
        lib.sdtw_set_deterministic(prev)
    assert lib.sdtw_workspace_bytes(99, B, N, M, K) == 0


def test_fused_geometry_query():
    # the library's own choice of bands per workgroup (without a visible GPU it assumes 256
    # CUs, the MI355X count): 1 while the batch's one-band workgroups all fit at once under
    # mixed arithmetic (the linear-domain forward), else 2 while the 2-band ones fit
    q = _engine.load().sdtw_fused_bands_per_workgroup
    prev = _engine.set_numerics("mixed")
    try:
        for mode in ("mixed", "exact", "fast"):
            _engine.set_numerics(mode)
            one = 1 if mode == "mixed" else 2
            assert q(32, 512, 512, 64) == one    # 32 * 8 = 256 one-band workgroups
            assert q(32, 1024, 1024, 64) == 2    # 32 * 16 = 512; 32 * 8 = 256 2-band ones
            assert q(32, 2048, 2048, 64) == 4    # 32 * 16 = 512 2-band ones
            assert q(16, 4096, 3072, 4) == 4     # the long configuration: 16 * 32 = 512
            assert q(256, 64, 64, 8) == one      # one band per pair
            assert q(257, 64, 64, 8) == 4
            assert q(4, 512, 512, 65) == 4       # K > 64: scalar cost tiles
            assert q(1, 5, 5, 3) == 4            # K*N*M < 400: scalar cost tiles
            assert q(1, 0, 5, 3) == 0            # invalid shape
    finally:
        _engine.set_numerics(prev)


def test_one_launch_unfused_forward_choice(monkeypatch):
    # the unfused module takes the one-launch forward only with matrix-core costs, in the
    # library's 2-band geometry and outside "fast" arithmetic
    lib = _engine.load()
    monkeypatch.setattr(_engine, "fused_bands_per_workgroup",
                        lambda B, N, M, K, device: lib.sdtw_fused_bands_per_workgroup(B, N, M, K))
    prev = _engine.set_numerics("mixed")
    try:
        pick = _engine.one_launch_unfused_forward
        assert pick(32, 512, 512, 64, "cuda:0")
        assert pick(32, 1024, 1024, 64, "cuda:0")
        assert not pick(32, 2048, 2048, 64, "cuda:0")
        assert pick(256, 64, 64, 8, "cuda:0")
        assert not pick(257, 64, 64, 8, "cuda:0")
        assert pick(16, 2048, 2048, 1, "cuda:0")
        assert not pick(4, 512, 512, 65, "cuda:0")
        assert not pick(1, 5, 5, 3, "cuda:0")
        assert _engine.set_numerics("exact") == "mixed"
        assert pick(32, 512, 512, 64, "cuda:0")
        _engine.set_numerics("fast")
        assert not pick(32, 512, 512, 64, "cuda:0")
    finally:
        _engine.set_numerics(prev)


def test_wait_limit_setter():
    assert _engine.set_wait_limit(1000) == 1 << 22
    assert _engine.set_wait_limit(1 << 22) == 1000


def test_noalloc_forward_limit_checked_before_any_device_call():
    # the size check returns before the runtime is touched, so it answers without a GPU
    lib = _engine.load()
    assert lib.sdtw_fwd_f32_noalloc_scratch_limit() == 16 << 20
    fake = ctypes.c_void_p(256)  # never dereferenced
    assert lib.sdtw_fwd_f32_noalloc(fake, fake, fake, 64, 4096, 8192, 1.0, -1.0, None) == 6
    assert lib.sdtw_fwd_f32_noalloc(fake, fake, fake, 1, 0, 8, 1.0, -1.0, None) == 1
    assert lib.sdtw_fwd_f32_noalloc(fake, fake, fake, 0, 8, 8, 1.0, -1.0, None) == 0
    # the largest batch of the long configuration's shape that fits: 16 * 16 * 3200 * 16 B
    assert lib.sdtw_workspace_bytes(_engine.OP_FWD, 16, 4096, 3072, 0) <= 16 << 20
