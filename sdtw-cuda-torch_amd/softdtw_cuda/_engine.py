"""ctypes binding of the gfx950 Soft-DTW engine (libsdtw_hip.so, C ABI in include/sdtw.h).

Every function here takes CUDA (ROCm) fp32 contiguous tensors, allocates outputs and the
workspace through torch's caching allocator, and enqueues the engine's kernels on torch's
current stream.  There is no CPU implementation behind these functions: if the library is
missing or no GPU is present, they raise.
"""
from __future__ import annotations

import ctypes
import functools
import os
import threading

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libsdtw_hip.so")
# SDTW_DEBUG_SYNC=1: synchronise after every wavefront launch and raise if a kernel's bounded
# inter-band wait expired (diagnostics and tests; off by default, it costs a device sync).
_DEBUG_SYNC = os.environ.get("SDTW_DEBUG_SYNC", "0") == "1"
_lib = None
_lock = threading.Lock()

# include/sdtw.h enums
OP_SQEUCLID_FWD, OP_SQEUCLID_BWD, OP_FWD, OP_BWD, OP_FUSED_FWD, OP_FUSED_BWD = range(6)
DIST_EXACT = 0
NUMERICS = {"fast": 0, "exact": 1, "mixed": 2}

_SIGS = {
    "sdtw_strerror": ([ctypes.c_int], ctypes.c_char_p),
    "sdtw_version": ([], ctypes.c_int),
    "sdtw_set_numerics": ([ctypes.c_int], ctypes.c_int),
    "sdtw_get_numerics": ([], ctypes.c_int),
    "sdtw_set_wait_limit": ([ctypes.c_uint], ctypes.c_uint),
    "sdtw_set_deterministic": ([ctypes.c_int], ctypes.c_int),
    "sdtw_dist_record_bytes": ([ctypes.c_int64] * 3, ctypes.c_size_t),
    "sdtw_fused_bands_per_workgroup": ([ctypes.c_int64] * 4, ctypes.c_int),
    "sdtw_workspace_bytes": ([ctypes.c_int] + [ctypes.c_int64] * 4, ctypes.c_size_t),
    "sdtw_table_elems": ([ctypes.c_int64] * 3, ctypes.c_int64),
    "sdtw_debug_status": ([ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t] + [ctypes.c_int64] * 4, ctypes.c_int),
    "sdtw_table_unpack_f32": ([ctypes.c_void_p] * 2 + [ctypes.c_int64] * 3 + [ctypes.c_void_p], ctypes.c_int),
    "sdtw_table_pack_f32": ([ctypes.c_void_p] * 2 + [ctypes.c_int64] * 3 + [ctypes.c_void_p], ctypes.c_int),
    "sdtw_sqeuclid_fwd_f32": ([ctypes.c_void_p] * 3 + [ctypes.c_int64] * 4
                              + [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
                              ctypes.c_int),
    "sdtw_sqeuclid_bwd_f32": ([ctypes.c_void_p] * 7 + [ctypes.c_int64] * 4
                              + [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
                              ctypes.c_int),
    "sdtw_fwd_f32": ([ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3
                     + [ctypes.c_double] * 2 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
                     ctypes.c_int),
    "sdtw_fwd_f32_noalloc": ([ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3
                             + [ctypes.c_double] * 2 + [ctypes.c_void_p], ctypes.c_int),
    "sdtw_fwd_f32_noalloc_scratch_limit": ([], ctypes.c_size_t),
    "sdtw_bwd_f32": ([ctypes.c_void_p] * 4 + [ctypes.c_int64] * 3
                     + [ctypes.c_double] * 2 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
                     ctypes.c_int),
    "sdtw_fused_fwd_f32": ([ctypes.c_void_p] * 4 + [ctypes.c_int64] * 4
                           + [ctypes.c_double] * 2 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
                           ctypes.c_int),
    "sdtw_fused_fwd_d_f32": ([ctypes.c_void_p] * 6 + [ctypes.c_int64] * 4
                             + [ctypes.c_double] * 2 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
                             ctypes.c_int),
    "sdtw_fused_bwd_f32": ([ctypes.c_void_p] * 6 + [ctypes.c_int64] * 4
                           + [ctypes.c_double] * 2 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
                           ctypes.c_int),
    "sdtw_fused_bwd_e_f32": ([ctypes.c_void_p] * 5 + [ctypes.c_int64] * 4
                             + [ctypes.c_double] * 2 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
                             ctypes.c_int),
    "sdtw_barycenter_workspace_bytes": ([ctypes.c_int64] * 3 + [ctypes.c_int], ctypes.c_size_t),
    "sdtw_barycenter_f32": ([ctypes.c_void_p] * 4 + [ctypes.c_int64] * 3
                            + [ctypes.c_double, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                               ctypes.c_int, ctypes.c_double, ctypes.c_void_p, ctypes.c_void_p,
                               ctypes.c_size_t, ctypes.c_void_p], ctypes.c_int),
    "sdtw_table_elems_f64": ([ctypes.c_int64] * 3, ctypes.c_int64),
    "sdtw_sqeuclid_fwd_f64": ([ctypes.c_void_p] * 3 + [ctypes.c_int64] * 4 + [ctypes.c_void_p],
                              ctypes.c_int),
    "sdtw_sqeuclid_bwd_f64": ([ctypes.c_void_p] * 6 + [ctypes.c_int64] * 4
                              + [ctypes.c_int, ctypes.c_void_p], ctypes.c_int),
    "sdtw_fwd_f64": ([ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [ctypes.c_double] * 2
                     + [ctypes.c_void_p], ctypes.c_int),
    "sdtw_bwd_f64": ([ctypes.c_void_p] * 4 + [ctypes.c_int64] * 3 + [ctypes.c_double] * 2
                     + [ctypes.c_void_p], ctypes.c_int),
}


def library_path() -> str:
    return _LIB_PATH


def load():
    """Load libsdtw_hip.so (once).  Raises RuntimeError if it has not been built."""
    global _lib
    lib = _lib
    if lib is not None:  # loaded: no lock needed to read it
        return lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"softdtw_cuda: HIP engine library not found at {_LIB_PATH}. "
                "Build it with `python sdtw-cuda-torch_amd/build.py` (hipcc, gfx950)."
            )
        lib = ctypes.CDLL(_LIB_PATH)
        for name, (args, res) in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
        return lib


def exported_symbols():
    return list(_SIGS)


def set_numerics(mode: str) -> str:
    """Select the recursions' cell arithmetic for this process; returns the previous mode.

    "mixed" (default): the forward is the reference CPU arithmetic with fp64-accurate
    exp/log, so R matches the CPU path bit for bit; the backward takes the CPU path's own
    fp32 differences of R and D and evaluates their transition weights with the hardware
    fp32 exp2: E within ~1e-6 relative, gradients within rtol 1e-4 / atol 1e-5.
    "exact": fp64-accurate exp/log in both recursions; E to the last bit but for rare
    differences.
    "fast": hardware fp32 exp2/log2 in both recursions (fp64 state); forward within ~1 fp32
    ulp, gradients as accurate (against an fp64 evaluation) as the reference's own fp32
    path, but not within rtol 1e-4 of it where differences of R cancel."""
    if mode not in NUMERICS:
        raise ValueError(f"softdtw_cuda: numerics must be one of {sorted(NUMERICS)}, got {mode!r}")
    prev = load().sdtw_set_numerics(NUMERICS[mode])
    return {v: k for k, v in NUMERICS.items()}[prev]


def get_numerics() -> str:
    return {v: k for k, v in NUMERICS.items()}[load().sdtw_get_numerics()]


def set_wait_limit(polls: int) -> int:
    """Polls a wavefront kernel's bounded wait makes before giving up (process-wide); returns
    the previous limit.  A test hook: a wave that gives up marks its pair's results NaN."""
    return int(load().sdtw_set_wait_limit(int(polls)))


_deterministic = None  # the library's setting as last set from here


def sync_deterministic() -> bool:
    """Make the library's fused-backward choice follow torch.use_deterministic_algorithms():
    under it, sdtw_fused_bwd_f32 takes its E path (run-to-run identical bits) instead of
    forming dL/dy with atomics in the recursion kernel.  Returns the setting."""
    global _deterministic
    want = bool(torch.are_deterministic_algorithms_enabled())
    if want != _deterministic:
        load().sdtw_set_deterministic(int(want))
        _deterministic = want
    return want


def strerror(rc: int) -> str:
    return load().sdtw_strerror(int(rc)).decode()


def _check(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"softdtw_cuda: {what} failed: {strerror(rc)} (status {rc})")


def require_gpu(t: torch.Tensor, what: str, dtype=torch.float32):
    if not t.is_cuda:
        raise RuntimeError(f"softdtw_cuda: {what} expects a ROCm/CUDA tensor, got {t.device}")
    if t.dtype != dtype or not t.is_contiguous():
        raise RuntimeError(f"softdtw_cuda: {what} expects contiguous {dtype}, got {t.dtype}")


@functools.lru_cache(maxsize=256)
def table_elems(B, N, M) -> int:
    """Floats in the engine's R table for B pairs of N x M cells."""
    return int(load().sdtw_table_elems(B, N, M))


def table_unpack(Rt: torch.Tensor, B: int, N: int, M: int) -> torch.Tensor:
    """Engine R table -> dense (B, N, M)."""
    require_gpu(Rt, "table")
    if Rt.numel() != table_elems(B, N, M):
        raise ValueError("softdtw_cuda: R table size does not match (B, N, M)")
    R = torch.empty((B, N, M), dtype=torch.float32, device=Rt.device)
    with torch.cuda.device(Rt.device):
        rc = load().sdtw_table_unpack_f32(_ptr(Rt), _ptr(R), B, N, M, _stream(Rt.device))
    _check(rc, "table unpack")
    return R


def table_pack(R: torch.Tensor) -> torch.Tensor:
    """Dense (B, N, M) -> engine R table."""
    require_gpu(R, "dense R")
    B, N, M = R.shape
    Rt = torch.full((table_elems(B, N, M),), float("inf"), dtype=torch.float32, device=R.device)
    with torch.cuda.device(R.device):
        rc = load().sdtw_table_pack_f32(_ptr(R), _ptr(Rt), B, N, M, _stream(R.device))
    _check(rc, "table pack")
    return Rt


def _check_table(R, B, N, M):
    if R.dim() != 1 or R.numel() != table_elems(B, N, M):
        raise ValueError(f"softdtw_cuda: R must be the engine table of {table_elems(B, N, M)} "
                         f"floats for (B,N,M)={(B, N, M)}, got shape {tuple(R.shape)}")


def _check_shapes(x=None, y=None, D=None, R=None, gout=None):
    """Validate every operand's shape against the others before any launch: the kernels
    trust B, N, M, K."""
    B = N = M = K = None
    if x is not None:
        if x.dim() != 3:
            raise ValueError(f"softdtw_cuda: x must be (B,N,K), got {tuple(x.shape)}")
        B, N, K = x.shape
    if y is not None:
        if y.dim() != 3 or (B is not None and (y.shape[0] != B or y.shape[2] != K)):
            raise ValueError(f"softdtw_cuda: y must be (B,M,K) matching x, got {tuple(y.shape)}")
        B, M, K = y.shape
    for name, t in (("D", D),):
        if t is None:
            continue
        if t.dim() != 3:
            raise ValueError(f"softdtw_cuda: {name} must be (B,N,M), got {tuple(t.shape)}")
        if B is None:
            B, N, M = t.shape
        elif tuple(t.shape) != (B, N, M):
            raise ValueError(f"softdtw_cuda: {name} shape {tuple(t.shape)} != {(B, N, M)}")
    if R is not None:
        _check_table(R, B, N, M)
    if gout is not None and gout.numel() != B:
        raise ValueError(f"softdtw_cuda: grad_output has {gout.numel()} elements, expected {B}")
    if N is not None and (N == 0 or M == 0):
        raise ValueError("softdtw_cuda: sequence lengths must be > 0")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _debug_check(op, ws, nws, B, N, M, K, what):
    if _DEBUG_SYNC and ws is not None:
        _check(load().sdtw_debug_status(op, _ptr(ws), nws, B, N, M, K), what + " (debug status)")


_ws_sizes = {}


def _device_index(device) -> int:
    d = torch.device(device)
    return d.index if d.index is not None else torch.cuda.current_device()


def _workspace(op, B, N, M, K, device):
    """The workspace of one engine call.  Its size depends on the shape, the device (the
    recursions' workgroup geometry follows its CU count: queried with that device current),
    the arithmetic and the deterministic setting, and is cached under all of them; the buffer
    is allocated per call."""
    idx = _device_index(device)
    key = (op, B, N, M, K, idx, int(load().sdtw_get_numerics()), _deterministic)
    n = _ws_sizes.get(key)
    if n is None:
        with torch.cuda.device(idx):
            n = int(load().sdtw_workspace_bytes(op, B, N, M, K))
        _ws_sizes[key] = n
    if n == 0:
        return None, 0
    return torch.empty(n, dtype=torch.uint8, device=torch.device("cuda", idx)), n


def sqeuclid_fwd(x: torch.Tensor, y: torch.Tensor, mode: int = DIST_EXACT) -> torch.Tensor:
    require_gpu(x, "sqeuclid x")
    require_gpu(y, "sqeuclid y")
    _check_shapes(x=x, y=y)
    B, N, K = x.shape
    M = y.shape[1]
    D = torch.empty((B, N, M), dtype=torch.float32, device=x.device)
    ws, nws = _workspace(OP_SQEUCLID_FWD, B, N, M, K, x.device)
    with torch.cuda.device(x.device):
        rc = load().sdtw_sqeuclid_fwd_f32(_ptr(x), _ptr(y), _ptr(D), B, N, M, K, int(mode),
                                          _ptr(ws), nws, _stream(x.device))
    _check(rc, "sqeuclid forward")
    return D


def sqeuclid_bwd(x, y, D, G, mask: bool = True, need=(True, True), record=None):
    """(gx, gy) of the distance given G = dL/dD; an entry of `need` that is False skips that
    gradient (returned as None).  record: the distance record fused_fwd_d wrote with D (per
    pair clamp flags and row norms: pairs without a clamped cost skip reading D, and no norms
    launch is needed), or None."""
    for t, n in ((x, "x"), (y, "y"), (G, "G")):
        require_gpu(t, f"sqeuclid backward {n}")
    if mask:
        require_gpu(D, "sqeuclid backward D")
    _check_shapes(x=x, y=y, D=G)
    if mask:
        _check_shapes(x=x, y=y, D=D)
    B, N, K = x.shape
    M = y.shape[1]
    gx = torch.empty_like(x) if need[0] else None
    gy = torch.empty_like(y) if need[1] else None
    ws, nws = _workspace(OP_SQEUCLID_BWD, B, N, M, K, x.device)
    with torch.cuda.device(x.device):
        rc = load().sdtw_sqeuclid_bwd_f32(_ptr(x), _ptr(y), _ptr(D if mask else None),
                                          _ptr(record if mask else None), _ptr(G), _ptr(gx),
                                          _ptr(gy), B, N, M, K, 1 if mask else 0, _ptr(ws), nws,
                                          _stream(x.device))
    _check(rc, "sqeuclid backward")
    return gx, gy


def dtw_fwd(D: torch.Tensor, gamma: float, bandwidth: float):
    require_gpu(D, "softdtw forward D")
    _check_shapes(D=D)
    B, N, M = D.shape
    R = torch.empty((table_elems(B, N, M),), dtype=torch.float32, device=D.device)
    out = torch.empty((B,), dtype=torch.float32, device=D.device)
    ws, nws = _workspace(OP_FWD, B, N, M, 0, D.device)
    with torch.cuda.device(D.device):
        rc = load().sdtw_fwd_f32(_ptr(D), _ptr(R), _ptr(out), B, N, M, float(gamma),
                                 float(bandwidth), _ptr(ws), nws, _stream(D.device))
    _check(rc, "softdtw forward")
    _debug_check(OP_FWD, ws, nws, B, N, M, 0, "softdtw forward")
    return out, R


def dtw_fwd_noalloc(D: torch.Tensor, gamma: float, bandwidth: float, R=None, out=None):
    """sdtw_fwd_f32_noalloc: the forward of dtw_fwd with the library's static scratch instead
    of a workspace.  R and out may be passed in (preallocated); they are returned."""
    require_gpu(D, "softdtw forward D")
    _check_shapes(D=D)
    B, N, M = D.shape
    if R is None:
        R = torch.empty((table_elems(B, N, M),), dtype=torch.float32, device=D.device)
    if out is None:
        out = torch.empty((B,), dtype=torch.float32, device=D.device)
    require_gpu(R, "softdtw forward R")
    require_gpu(out, "softdtw forward out")
    if R.numel() != table_elems(B, N, M) or out.numel() != B:
        raise ValueError("softdtw_cuda: R / out sizes do not match (B, N, M)")
    with torch.cuda.device(D.device):
        rc = load().sdtw_fwd_f32_noalloc(_ptr(D), _ptr(R), _ptr(out), B, N, M, float(gamma),
                                         float(bandwidth), _stream(D.device))
    _check(rc, "softdtw forward (no allocation)")
    return out, R


def dtw_bwd(D, R, gamma: float, bandwidth: float, gout=None):
    require_gpu(D, "softdtw backward D")
    require_gpu(R, "softdtw backward R")
    if gout is not None:
        require_gpu(gout, "softdtw backward grad_output")
    _check_shapes(D=D, R=R, gout=gout)
    B, N, M = D.shape
    G = torch.empty((B, N, M), dtype=torch.float32, device=D.device)
    ws, nws = _workspace(OP_BWD, B, N, M, 0, D.device)
    with torch.cuda.device(D.device):
        rc = load().sdtw_bwd_f32(_ptr(D), _ptr(R), _ptr(gout), _ptr(G), B, N, M, float(gamma),
                                 float(bandwidth), _ptr(ws), nws, _stream(D.device))
    _check(rc, "softdtw backward")
    _debug_check(OP_BWD, ws, nws, B, N, M, 0, "softdtw backward")
    return G


def fused_fwd(x, y, gamma: float, bandwidth: float):
    require_gpu(x, "fused forward x")
    require_gpu(y, "fused forward y")
    _check_shapes(x=x, y=y)
    B, N, K = x.shape
    M = y.shape[1]
    R = torch.empty((table_elems(B, N, M),), dtype=torch.float32, device=x.device)
    out = torch.empty((B,), dtype=torch.float32, device=x.device)
    ws, nws = _workspace(OP_FUSED_FWD, B, N, M, K, x.device)
    with torch.cuda.device(x.device):
        rc = load().sdtw_fused_fwd_f32(_ptr(x), _ptr(y), _ptr(R), _ptr(out), B, N, M, K,
                                       float(gamma), float(bandwidth), _ptr(ws), nws,
                                       _stream(x.device))
    _check(rc, "fused forward")
    _debug_check(OP_FUSED_FWD, ws, nws, B, N, M, K, "fused forward")
    return out, R


def fused_costs_on_matrix_cores(N: int, M: int, K: int) -> bool:
    """Whether the fused recursions take their cost tiles from matrix-core producer waves
    (K <= 64 and K*N*M >= 400: the shapes whose reference dot is a fused multiply-add
    chain), which sdtw_fused_fwd_d_f32 needs."""
    return K <= 64 and K * N * M >= 400


_bands_cache = {}


def fused_bands_per_workgroup(B: int, N: int, M: int, K: int, device) -> int:
    """The fused forward recursions' bands per workgroup for an unbanded call at this shape
    on `device` under the current arithmetic (the library's own choice,
    sdtw_fused_bands_per_workgroup): 1, 2 or 4.  Cached per shape, device and arithmetic."""
    idx = _device_index(device)
    key = (B, N, M, K, idx, int(load().sdtw_get_numerics()))
    w = _bands_cache.get(key)
    if w is None:
        with torch.cuda.device(idx):
            w = int(load().sdtw_fused_bands_per_workgroup(B, N, M, K))
        _bands_cache[key] = w
    return w


def one_launch_unfused_forward(B: int, N: int, M: int, K: int, device) -> bool:
    """Whether sdtw_fused_fwd_d_f32 beats the distance launch plus the D-reading recursion.
    It needs matrix-core costs, and the library must take its 1- or 2-band geometry (the
    batch's workgroups all fit on the GPU at once): the producer waves then have SIMDs of
    their own, whereas sharing their compute waves' SIMDs, the D stores slow the recursion
    (B=32 N=M=2048 D=64: 2.78 against 2.70 ms per step).  Not under "fast" arithmetic,
    whose short recursion step makes the storing producers the limit."""
    if not fused_costs_on_matrix_cores(N, M, K) or get_numerics() == "fast":
        return False
    return fused_bands_per_workgroup(B, N, M, K, device) <= 2


@functools.lru_cache(maxsize=256)
def _dist_record_bytes(B, N, M) -> int:
    return int(load().sdtw_dist_record_bytes(B, N, M))


def fused_fwd_d(x, y, gamma: float, bandwidth: float):
    """Unfused mode's forward in one launch: (out, R, D, record) with D the (B,N,M) cost
    tensor and record its distance record for sqeuclid_bwd (uint8 device buffer: per-pair
    int32 flags, 1 where a cost is not positive, then the row norms of x and y)."""
    require_gpu(x, "fused forward x")
    require_gpu(y, "fused forward y")
    _check_shapes(x=x, y=y)
    B, N, K = x.shape
    M = y.shape[1]
    D = torch.empty((B, N, M), dtype=torch.float32, device=x.device)
    R = torch.empty((table_elems(B, N, M),), dtype=torch.float32, device=x.device)
    out = torch.empty((B,), dtype=torch.float32, device=x.device)
    record = torch.empty((_dist_record_bytes(B, N, M),), dtype=torch.uint8, device=x.device)
    ws, nws = _workspace(OP_FUSED_FWD, B, N, M, K, x.device)
    with torch.cuda.device(x.device):
        rc = load().sdtw_fused_fwd_d_f32(_ptr(x), _ptr(y), _ptr(D), _ptr(record), _ptr(R),
                                         _ptr(out), B, N, M, K, float(gamma), float(bandwidth),
                                         _ptr(ws), nws, _stream(x.device))
    _check(rc, "fused forward (with D)")
    _debug_check(OP_FUSED_FWD, ws, nws, B, N, M, K, "fused forward (with D)")
    return out, R, D, record


def fused_bwd(x, y, R, gamma: float, bandwidth: float, gout=None, need=(True, True)):
    """(gx, gy) of the fused Soft-DTW; an entry of `need` that is False skips that gradient
    (returned as None)."""
    require_gpu(x, "fused backward x")
    require_gpu(y, "fused backward y")
    require_gpu(R, "fused backward R")
    if gout is not None:
        require_gpu(gout, "fused backward grad_output")
    _check_shapes(x=x, y=y, R=R, gout=gout)
    B, N, K = x.shape
    M = y.shape[1]
    gx = torch.empty_like(x) if need[0] else None
    gy = torch.empty_like(y) if need[1] else None
    sync_deterministic()
    ws, nws = _workspace(OP_FUSED_BWD, B, N, M, K, x.device)
    with torch.cuda.device(x.device):
        rc = load().sdtw_fused_bwd_f32(_ptr(x), _ptr(y), _ptr(R), _ptr(gout), _ptr(gx), _ptr(gy),
                                       B, N, M, K, float(gamma), float(bandwidth), _ptr(ws), nws,
                                       _stream(x.device))
    _check(rc, "fused backward")
    _debug_check(OP_FUSED_BWD, ws, nws, B, N, M, K, "fused backward")
    return gx, gy


def fused_bwd_e(x, y, R, gamma: float, bandwidth: float, gout=None):
    require_gpu(x, "fused backward x")
    require_gpu(y, "fused backward y")
    require_gpu(R, "fused backward R")
    if gout is not None:
        require_gpu(gout, "fused backward grad_output")
    _check_shapes(x=x, y=y, R=R, gout=gout)
    B, N, K = x.shape
    M = y.shape[1]
    E = torch.empty((B, N, M), dtype=torch.float32, device=x.device)
    ws, nws = _workspace(OP_FUSED_BWD, B, N, M, K, x.device)
    with torch.cuda.device(x.device):
        rc = load().sdtw_fused_bwd_e_f32(_ptr(x), _ptr(y), _ptr(R), _ptr(gout), _ptr(E), B, N, M,
                                         K, float(gamma), float(bandwidth), _ptr(ws), nws,
                                         _stream(x.device))
    _check(rc, "fused backward (E)")
    _debug_check(OP_FUSED_BWD, ws, nws, B, N, M, K, "fused backward (E)")
    return E


def barycenter(X, w, bary, gamma: float, lrs, early_stopping: bool, patience: int, tol: float):
    """sdtw_barycenter_f32: the barycenter loop on the device.  X (B, N, K) sequences, w (B,)
    normalised weights, bary (N, K) the initial barycenter, updated in place; lrs the
    learning rate of each iteration.  Returns (bary, losses of the iterations run)."""
    for t, n in ((X, "X"), (w, "weights"), (bary, "barycenter")):
        require_gpu(t, f"barycenter {n}")
    if X.dim() != 3 or tuple(bary.shape) != tuple(X.shape[1:]) or w.numel() != X.shape[0]:
        raise ValueError("softdtw_cuda: barycenter expects X (B,N,K), weights (B,), init (N,K)")
    B, N, K = X.shape
    max_iter = len(lrs)
    n = int(load().sdtw_barycenter_workspace_bytes(B, N, K, max_iter))
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=X.device)
    losses = torch.empty(max(max_iter, 1), dtype=torch.float32, device=X.device)
    lr_arr = (ctypes.c_double * max(max_iter, 1))(*lrs)
    iters = ctypes.c_int(0)
    with torch.cuda.device(X.device):
        rc = load().sdtw_barycenter_f32(_ptr(X), _ptr(w), _ptr(bary), _ptr(losses), B, N, K,
                                        float(gamma), max_iter, lr_arr, 1 if early_stopping else 0,
                                        int(patience), float(tol), ctypes.byref(iters), _ptr(ws), n,
                                        _stream(X.device))
    _check(rc, "barycenter")
    return bary, losses[:iters.value]


# ---- float64 path (sdtw_*_f64): double throughout, R the dense (B, N+2, M+2) table -------
F64 = torch.float64


def sqeuclid_fwd64(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    require_gpu(x, "sqeuclid x", F64)
    require_gpu(y, "sqeuclid y", F64)
    _check_shapes(x=x, y=y)
    B, N, K = x.shape
    M = y.shape[1]
    D = torch.empty((B, N, M), dtype=F64, device=x.device)
    with torch.cuda.device(x.device):
        rc = load().sdtw_sqeuclid_fwd_f64(_ptr(x), _ptr(y), _ptr(D), B, N, M, K, _stream(x.device))
    _check(rc, "sqeuclid forward (float64)")
    return D


def sqeuclid_bwd64(x, y, D, G, mask: bool = True):
    for t, n in ((x, "x"), (y, "y"), (G, "G")):
        require_gpu(t, f"sqeuclid backward {n}", F64)
    if mask:
        require_gpu(D, "sqeuclid backward D", F64)
    _check_shapes(x=x, y=y, D=G)
    if mask:
        _check_shapes(x=x, y=y, D=D)
    B, N, K = x.shape
    M = y.shape[1]
    gx = torch.empty_like(x)
    gy = torch.empty_like(y)
    with torch.cuda.device(x.device):
        rc = load().sdtw_sqeuclid_bwd_f64(_ptr(x), _ptr(y), _ptr(D if mask else None), _ptr(G),
                                          _ptr(gx), _ptr(gy), B, N, M, K, 1 if mask else 0,
                                          _stream(x.device))
    _check(rc, "sqeuclid backward (float64)")
    return gx, gy


def _check_table64(R, B, N, M):
    if tuple(R.shape) != (B, N + 2, M + 2):
        raise ValueError(f"softdtw_cuda: float64 R must be (B,N+2,M+2)={(B, N + 2, M + 2)}, "
                         f"got {tuple(R.shape)}")


def dtw_fwd64(D: torch.Tensor, gamma: float, bandwidth: float):
    """(out (B,), R (B, N+2, M+2)), both float64."""
    require_gpu(D, "softdtw forward D", F64)
    _check_shapes(D=D)
    B, N, M = D.shape
    R = torch.empty((B, N + 2, M + 2), dtype=F64, device=D.device)
    out = torch.empty((B,), dtype=F64, device=D.device)
    with torch.cuda.device(D.device):
        rc = load().sdtw_fwd_f64(_ptr(D), _ptr(R), _ptr(out), B, N, M, float(gamma),
                                 float(bandwidth), _stream(D.device))
    _check(rc, "softdtw forward (float64)")
    return out, R


def dtw_bwd64(D, R, gamma: float, bandwidth: float, gout=None):
    """G = gout * E (B, N, M) float64; gout None gives E."""
    require_gpu(D, "softdtw backward D", F64)
    require_gpu(R, "softdtw backward R", F64)
    if gout is not None:
        require_gpu(gout, "softdtw backward grad_output", F64)
    _check_shapes(D=D, gout=gout)
    B, N, M = D.shape
    _check_table64(R, B, N, M)
    G = torch.empty((B, N, M), dtype=F64, device=D.device)
    with torch.cuda.device(D.device):
        rc = load().sdtw_bwd_f64(_ptr(D), _ptr(R), _ptr(gout), _ptr(G), B, N, M, float(gamma),
                                 float(bandwidth), _stream(D.device))
    _check(rc, "softdtw backward (float64)")
    return G
