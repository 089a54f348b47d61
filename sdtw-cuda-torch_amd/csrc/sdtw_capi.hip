// sdtw_capi.hip -- the extern "C" boundary declared in include/sdtw.h.
//
// Responsibilities: argument validation, carving the caller's workspace, choosing kernel
// variants and enqueueing them on the caller's stream.  No allocation, no synchronisation.
#include <math.h>

#include <atomic>
#include <mutex>

#include "../../include/sdtw.h"
#include "sdtw_internal.hpp"

using namespace sdtw;

// Scratch of the no-allocation forward (sdtw_fwd_f32_noalloc): a file-scope device array,
// one copy per GPU, held until the process ends.  In host code `scratch` names a host-side
// stand-in, not device memory: its device address is taken once per device with
// hipGetSymbolAddress (with that device current) and only that address is used.
static constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Sub-buffer carving of a caller workspace.
struct Carver {
    char* base;
    size_t cap;
    size_t off = 0;
    bool ok = true;
    template <class T>
    T* take(size_t count) {
        const size_t bytes = align_up(count * sizeof(T));
        if (base == nullptr || off + bytes > cap) {
            ok = false;
            off += bytes;
            return nullptr;
        }
        T* p = reinterpret_cast<T*>(base + off);
        off += bytes;
        return p;
    }
};

bool shape_ok(int64_t B, int64_t N, int64_t M, int64_t K, bool need_k) {
    if (B < 0 || N <= 0 || M <= 0) return false;
    if (need_k && K <= 0) return false;
    // kernels index with int; keep every dimension and per-pair table within range
    if (B > INT32_MAX || N > INT32_MAX || M > INT32_MAX || K > INT32_MAX) return false;
    if (N * M > (int64_t)INT32_MAX * 16) return false;
    return true;
}

// distance kernels put B on grid.z and row tiles on grid.y (<= 65535 each)
bool dist_grid_ok(int64_t B, int64_t N, int64_t M) {
    return B <= 65535 && (N + 63) / 64 <= 65535 && (M + 63) / 64 <= 65535 &&
           (N + 255) / 256 <= 65535 && (M + 255) / 256 <= 65535;
}

bool gamma_ok(double gamma) { return gamma > 0.0 && isfinite(gamma); }

// ATen's naive bmm kernel (multiply, then add) runs when K*N*M < 400.
bool small_bmm(int64_t N, int64_t M, int64_t K) { return K * N * M < 400; }

// Compute units of the current device (cached per device).
int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// Bands per workgroup of the fused recursions.  With matrix-core cost tiles a producer wave
// per band computes them; it runs on a SIMD of its own (the fp32 matrix instructions take
// the cycles of the SIMD they run on) when a workgroup holds 2 bands.  A 2-band workgroup
// needs about 85 KiB of LDS, so one fits per CU: when the batch needs more 2-band
// workgroups than there are CUs, the later pairs would wait for the earlier ones to finish,
// and 4 bands per workgroup (producers sharing their compute waves' SIMDs, every
// workgroup resident) finish sooner.  Scalar cost tiles always take 4.
bool mfma_costs(int64_t N, int64_t M, int64_t K) { return !small_bmm(N, M, K) && K <= 64; }
int fused_wmax(int64_t B, int64_t N, int64_t M, int64_t K) {
    if (!mfma_costs(N, M, K)) return 4;
    return B * dp_geom(N, 2).G <= cu_count() ? 2 : 4;
}
// The fused backward: one band per workgroup when the batch's one-band workgroups all fit
// on the GPU at once.  Its producer wave (matrix-core cost tiles) and, in gradient mode, its
// dL/dx and dL/dy waves (matrix-core products with the E tiles) then each have a SIMD and its
// matrix core to themselves; at two bands per workgroup two of these waves share one.
int fused_bwd_wmax(int64_t B, int64_t N, int64_t M, int64_t K) {
    if (mfma_costs(N, M, K) && B * dp_geom(N, 1).G <= cu_count()) return 1;
    return fused_wmax(B, N, M, K);
}
// Workspace sizing: the geometry with the most cross-workgroup rows a launch can take: the
// 1-band one where either direction takes it on this device (a launch on a device with fewer
// CUs then reports SDTW_ERR_WORKSPACE), else the 2-band one.
int fused_ws_wmax(int64_t B, int64_t N, int64_t M, int64_t K, bool bwd) {
    (void)bwd;
    if (!mfma_costs(N, M, K)) return 4;
    return fused_bwd_wmax(B, N, M, K) == 1 ? 1 : 2;
}
// Process-wide: whether the fused backward must give run-to-run identical bits
// (sdtw_set_deterministic).
std::atomic<int> g_deterministic{0};
// The fused backward forms dL/dx and dL/dy inside the recursion kernel (gradient mode,
// no (B,N,M) buffer) with matrix-core cost tiles in a geometry whose waves fit: workgroups
// of up to 2 bands, or up to 4 for K <= 16.  Its dL/dy sums the bands' shares in arrival
// order, so under the deterministic setting a call that forms dL/dy, like every other call,
// writes g*E and reduces it with the distance backward (dL/dx alone is formed in a fixed
// order either way).  Workspace queries assume dL/dy is formed: the E path's workspace
// holds the gradient mode's.
bool fused_grad_mode(int64_t B, int64_t N, int64_t M, int64_t K, bool forms_gy = true) {
    if (forms_gy && g_deterministic.load(std::memory_order_relaxed)) return false;
    if (!mfma_costs(N, M, K)) return false;
    return fused_bwd_wmax(B, N, M, K) <= 2 || K <= 16;
}

// distance-backward split-reduction scratch: partials, then counters
size_t ws_dist_bwd(int64_t B, int64_t N, int64_t M, int64_t K) {
    return align_up(sizeof(float) * dist_bwd_split_floats(B, N, M, K)) +
           align_up(sizeof(int) * dist_bwd_counters(B, N, M, K)) +
           align_up(sizeof(int) * dist_bwd_flags(B, N, M, K));
}

// Distance record (sdtw_fused_fwd_d_f32 -> sdtw_sqeuclid_bwd_f32): [per-pair clamp flags,
// B ints][row norms of x, B*N floats][row norms of y, B*M floats], each part 256-byte aligned.
struct DistRecord {
    int* clamped;
    float* x2;
    float* y2;
};
size_t dist_record_bytes(int64_t B, int64_t N, int64_t M) {
    return align_up(sizeof(int) * B) + align_up(sizeof(float) * B * N) + align_up(sizeof(float) * B * M);
}
DistRecord dist_record(void* rec, int64_t B, int64_t N, int64_t M) {
    (void)M;
    char* c = static_cast<char*>(rec);
    DistRecord r{};
    if (!c) return r;
    r.clamped = reinterpret_cast<int*>(c);
    r.x2 = reinterpret_cast<float*>(c + align_up(sizeof(int) * B));
    r.y2 = reinterpret_cast<float*>(c + align_up(sizeof(int) * B) + align_up(sizeof(float) * B * N));
    return r;
}

size_t ws_norms(int64_t B, int64_t N, int64_t M) {
    return align_up(sizeof(float) * B * N) + align_up(sizeof(float) * B * M);
}

// Wavefront-kernel scratch: [ticket, error flag][per-boundary rows].  The rows hold fp64
// values (forward) or (E, R, D, tag) float4 (backward): 16 bytes per column.
size_t ws_dp(int64_t B, int64_t N, int64_t M, int wmax = 4) {
    const DPGeom g = dp_geom(N, wmax);
    return 256 + align_up((size_t)16 * B * g.G * dp_row_entries(M));
}

struct DPScratch {
    int* ticket;
    int* err;
    void* gring;
};

DPScratch carve_dp(Carver& c, int64_t B, int64_t N, int64_t M, int wmax = 4) {
    const DPGeom g = dp_geom(N, wmax);
    DPScratch d{};
    int* hdr = c.take<int>(64);
    d.gring = c.take<unsigned char>((size_t)16 * B * g.G * dp_row_entries(M));
    if (hdr) {
        d.ticket = hdr;
        d.err = hdr + 1;
    }
    return d;
}

// Process-wide poll limit of the wavefront kernels' bounded waits (sdtw_set_wait_limit).
std::atomic<unsigned> g_spin_limit{kDefaultSpinLimit};

void fill_dp(DPParams& p, const DPScratch& d, int64_t B, int64_t N, int64_t M, int64_t K,
             double gamma, double bandwidth, int wmax = 4) {
    const DPGeom g = dp_geom(N, wmax);
    p.ticket = d.ticket;
    p.err = d.err;
    p.gring = static_cast<double*>(d.gring);
    p.gring4 = static_cast<float4*>(d.gring);
    p.B = (int)B;
    p.N = (int)N;
    p.M = (int)M;
    p.K = (int)K;
    p.nb = g.nb;
    p.W = g.W;
    p.G = g.G;
    p.S = dp_band_steps(M);
    p.RW = (int)dp_row_entries(M);
    p.gamma = gamma;
    p.inv_gamma = 1.0 / gamma;
    p.bw = bandwidth;
    p.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
}

int status_of(hipError_t e) { return e == hipSuccess ? SDTW_OK : SDTW_ERR_LAUNCH; }

// Process-wide cell arithmetic of the wavefront kernels (sdtw_set_numerics).
std::atomic<int> g_numerics{SDTW_NUMERICS_MIXED};
// forward: fp64-accurate exp / log unless FAST; backward: only in EXACT
bool exact_forward() { return g_numerics.load(std::memory_order_relaxed) != SDTW_NUMERICS_FAST; }
bool exact_backward() { return g_numerics.load(std::memory_order_relaxed) == SDTW_NUMERICS_EXACT; }
// The D-reading backward takes one band per workgroup, with weight waves per band, where the
// batch's one-band workgroups all fit at once.  Its workspace is sized for that geometry.
bool bwd_one_band(int64_t B, int64_t N) { return B * ((N + 63) / 64) <= cu_count(); }
int bwd_wmax(int64_t B, int64_t N) { return bwd_one_band(B, N) ? 1 : 4; }
// the fused forwards' scaled linear-domain recursion: mixed arithmetic only (exact keeps the
// log-domain form, whose R carries the CPU path's fp32 bits)
bool lin_forward() { return g_numerics.load(std::memory_order_relaxed) == SDTW_NUMERICS_MIXED; }

// The fused forward: one band per workgroup where the batch's one-band workgroups all fit
// and the call takes the scaled linear-domain recursion (mixed arithmetic, matrix-core
// costs, no band): its compute, producer, helper and converter waves then have a SIMD each.
// Otherwise fused_wmax.
int fused_fwd_wmax(int64_t B, int64_t N, int64_t M, int64_t K, double bandwidth) {
    if (lin_forward() && !(bandwidth > 0.0) && fused_bwd_wmax(B, N, M, K) == 1) return 1;
    return fused_wmax(B, N, M, K);
}

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's `scratch`, or nullptr on a runtime error.
void* device_scratch() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (ptr) return ptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (ptr) return ptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    return ptr;
}

}  // namespace

extern "C" {

const char* sdtw_strerror(int status) {
    switch (status) {
        case SDTW_OK: return "success";
        case SDTW_ERR_INVALID_VALUE: return "invalid argument (shape, gamma or pointer)";
        case SDTW_ERR_WORKSPACE: return "workspace too small (see sdtw_workspace_bytes)";
        case SDTW_ERR_LAUNCH: return "HIP kernel launch failed";
        case SDTW_ERR_UNSUPPORTED: return "unsupported configuration";
        case SDTW_ERR_TIMEOUT: return "a wavefront kernel gave up waiting on a neighbour band";
        case SDTW_ERR_SCRATCH_LIMIT:
            return "shape needs more scratch than the no-allocation entry point holds "
                   "(sdtw_fwd_f32_noalloc_scratch_limit); use sdtw_fwd_f32 with a workspace";
        default: return "unknown sdtw status";
    }
}

int sdtw_version(void) { return 6; }

int sdtw_set_numerics(int mode) {
    if (mode != SDTW_NUMERICS_FAST && mode != SDTW_NUMERICS_EXACT && mode != SDTW_NUMERICS_MIXED)
        return -1;
    return g_numerics.exchange(mode);
}

int sdtw_get_numerics(void) { return g_numerics.load(); }

unsigned sdtw_set_wait_limit(unsigned polls) { return g_spin_limit.exchange(polls); }

int sdtw_set_deterministic(int on) { return g_deterministic.exchange(on ? 1 : 0); }

size_t sdtw_dist_record_bytes(int64_t B, int64_t N, int64_t M) {
    if (B < 0 || N < 0 || M < 0) return 0;
    return dist_record_bytes(B, N, M);
}

int sdtw_fused_bands_per_workgroup(int64_t B, int64_t N, int64_t M, int64_t K) {
    if (!shape_ok(B, N, M, K, true)) return 0;
    return fused_fwd_wmax(B, N, M, K, -1.0);
}

int sdtw_debug_status(int op, const void* ws, size_t ws_bytes, int64_t B, int64_t N, int64_t M,
                      int64_t K) {
    (void)K;
    if (!ws || B <= 0 || N <= 0 || M <= 0) return SDTW_ERR_INVALID_VALUE;
    Carver c{static_cast<char*>(const_cast<void*>(ws)), ws_bytes};
    if (op == SDTW_OP_FUSED_FWD || op == SDTW_OP_FUSED_BWD) {
        c.take<float>(B * N);
        c.take<float>(B * M);
    } else if (op != SDTW_OP_FWD && op != SDTW_OP_BWD) {
        return SDTW_OK;
    }
    // only the scratch header [ticket, error flag] is read; its place does not depend on
    // the band geometry the launch chose
    const int* hdr = c.take<int>(64);
    if (!c.ok || !hdr) return SDTW_ERR_WORKSPACE;
    int flag = 0;
    if (hipDeviceSynchronize() != hipSuccess) return SDTW_ERR_LAUNCH;
    if (hipMemcpy(&flag, hdr + 1, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
        return SDTW_ERR_LAUNCH;
    return flag ? SDTW_ERR_TIMEOUT : SDTW_OK;
}

int64_t sdtw_table_elems(int64_t B, int64_t N, int64_t M) {
    if (B < 0 || N <= 0 || M <= 0) return 0;
    return dp_table_elems(B, N, M);
}

int sdtw_table_unpack_f32(const float* Rt, float* R, int64_t B, int64_t N, int64_t M,
                          void* stream) {
    if (!shape_ok(B, N, M, 1, false)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!Rt || !R) return SDTW_ERR_INVALID_VALUE;
    return status_of(launch_table_unpack(Rt, R, (int)B, (int)N, (int)M, (hipStream_t)stream));
}

int sdtw_table_pack_f32(const float* R, float* Rt, int64_t B, int64_t N, int64_t M,
                        void* stream) {
    if (!shape_ok(B, N, M, 1, false)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!Rt || !R) return SDTW_ERR_INVALID_VALUE;
    return status_of(launch_table_pack(R, Rt, (int)B, (int)N, (int)M, (hipStream_t)stream));
}

size_t sdtw_workspace_bytes(int op, int64_t B, int64_t N, int64_t M, int64_t K) {
    (void)K;
    if (B < 0 || N < 0 || M < 0) return 0;
    switch (op) {
        case SDTW_OP_SQEUCLID_FWD:
        case SDTW_OP_SQEUCLID_BWD:
            return ws_norms(B, N, M) + ws_dist_bwd(B, N, M, K);
        case SDTW_OP_FWD:
            return ws_dp(B, N, M);
        case SDTW_OP_BWD:
            return ws_dp(B, N, M, bwd_wmax(B, N));
        case SDTW_OP_FUSED_FWD:
            return ws_norms(B, N, M) + ws_dp(B, N, M, fused_ws_wmax(B, N, M, K, false));
        case SDTW_OP_FUSED_BWD:
            if (fused_grad_mode(B, N, M, K))
                return ws_norms(B, N, M) + ws_dp(B, N, M, fused_ws_wmax(B, N, M, K, true));
            return ws_norms(B, N, M) + ws_dp(B, N, M, fused_ws_wmax(B, N, M, K, true)) + align_up(sizeof(float) * B * N * M) +
                   ws_dist_bwd(B, N, M, K);
        default:
            return 0;
    }
}

int sdtw_sqeuclid_fwd_f32(const float* x, const float* y, float* D, int64_t B, int64_t N,
                          int64_t M, int64_t K, int mode, void* ws, size_t ws_bytes,
                          void* stream) {
    if (!shape_ok(B, N, M, K, true)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!x || !y || !D) return SDTW_ERR_INVALID_VALUE;
    if (mode != SDTW_DIST_EXACT) return SDTW_ERR_UNSUPPORTED;
    if (!dist_grid_ok(B, N, M)) return SDTW_ERR_UNSUPPORTED;
    (void)ws;
    (void)ws_bytes;
    DistParams p{};
    p.x = x;
    p.y = y;
    p.D = D;
    p.B = (int)B;
    p.N = (int)N;
    p.M = (int)M;
    p.K = (int)K;
    return status_of(launch_dist(p, small_bmm(N, M, K), false, (hipStream_t)stream));
}

int sdtw_sqeuclid_bwd_f32(const float* x, const float* y, const float* D, const void* record,
                          const float* G, float* gx, float* gy, int64_t B, int64_t N, int64_t M,
                          int64_t K, int mask, void* ws, size_t ws_bytes, void* stream) {
    if (!shape_ok(B, N, M, K, true)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0 || (!gx && !gy)) return SDTW_OK;
    if (!x || !y || !G || (mask && !D)) return SDTW_ERR_INVALID_VALUE;
    if (!dist_grid_ok(B, N, M)) return SDTW_ERR_UNSUPPORTED;
    hipStream_t st = (hipStream_t)stream;
    DistBwdParams p{};
    p.x = x;
    p.y = y;
    p.D = mask ? D : nullptr;
    p.G = G;
    p.gx = gx;
    p.gy = gy;
    p.B = (int)B;
    p.N = (int)N;
    p.M = (int)M;
    p.K = (int)K;
    p.mask = mask ? 1 : 0;
    const DistRecord rec = dist_record(const_cast<void*>(record), B, N, M);
    p.clamped = (mask && record) ? rec.clamped : nullptr;
    p.muladd = small_bmm(N, M, K) ? 1 : 0;
    Carver c{static_cast<char*>(ws), ws_bytes};
    float* x2 = c.take<float>(B * N);
    float* y2 = c.take<float>(B * M);
    p.part = c.take<float>(dist_bwd_split_floats(B, N, M, K));
    p.cnt = c.take<int>(dist_bwd_counters(B, N, M, K));
    p.flags = c.take<int>(dist_bwd_flags(B, N, M, K));
    if (!c.ok) return SDTW_ERR_WORKSPACE;
    if (mask && record) {  // the forward formed the norms (the exact clamp check's inputs)
        p.x2 = rec.x2;
        p.y2 = rec.y2;
    } else if (mask) {
        if (launch_norms(x, x2, B * N, y, y2, B * M, (int)K, st) != hipSuccess)
            return SDTW_ERR_LAUNCH;
        p.x2 = x2;
        p.y2 = y2;
    }
    return status_of(launch_dist_bwd(p, st));
}

int sdtw_fwd_f32(const float* D, float* R, float* out, int64_t B, int64_t N, int64_t M,
                 double gamma, double bandwidth, void* ws, size_t ws_bytes, void* stream) {
    if (!shape_ok(B, N, M, 1, false) || !gamma_ok(gamma)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!D || !R || !out) return SDTW_ERR_INVALID_VALUE;
    Carver c{static_cast<char*>(ws), ws_bytes};
    const DPScratch d = carve_dp(c, B, N, M);
    if (!c.ok) return SDTW_ERR_WORKSPACE;
    DPParams p{};
    fill_dp(p, d, B, N, M, 0, gamma, bandwidth);
    p.D = D;
    p.R = R;
    p.out = out;
    return status_of(launch_fwd(p, false, false, exact_forward(), (hipStream_t)stream));
}

size_t sdtw_fwd_f32_noalloc_scratch_limit(void) { return kNoAllocScratchBytes; }

int sdtw_fwd_f32_noalloc(const float* D, float* R, float* out, int64_t B, int64_t N, int64_t M,
                         double gamma, double bandwidth, void* stream) {
    if (!shape_ok(B, N, M, 1, false) || !gamma_ok(gamma)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!D || !R || !out) return SDTW_ERR_INVALID_VALUE;
    // the size check comes before any runtime call (in 128 bits: no shape wraps it round)
    const DPGeom g = dp_geom(N);
    const unsigned __int128 need =
        256 + (unsigned __int128)16 * (unsigned __int128)B * g.G * dp_row_entries(M);
    if (need > kNoAllocScratchBytes) return SDTW_ERR_SCRATCH_LIMIT;
    void* ws = device_scratch();
    if (!ws) return SDTW_ERR_LAUNCH;
    // the prep launch that precedes the recursion resets the ticket and the error flag and
    // empties the cross-workgroup rows, so nothing of an earlier call's contents is read
    return sdtw_fwd_f32(D, R, out, B, N, M, gamma, bandwidth, ws, kNoAllocScratchBytes, stream);
}

int sdtw_bwd_f32(const float* D, const float* R, const float* gout, float* G, int64_t B,
                 int64_t N, int64_t M, double gamma, double bandwidth, void* ws,
                 size_t ws_bytes, void* stream) {
    if (!shape_ok(B, N, M, 1, false) || !gamma_ok(gamma)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!D || !R || !G) return SDTW_ERR_INVALID_VALUE;
    Carver c{static_cast<char*>(ws), ws_bytes};
    const bool ww = bwd_one_band(B, N);
    const int wmax = ww ? 1 : 4;
    const DPScratch d = carve_dp(c, B, N, M, wmax);
    if (!c.ok) return SDTW_ERR_WORKSPACE;
    DPParams p{};
    fill_dp(p, d, B, N, M, 0, gamma, bandwidth, wmax);
    p.ww = ww;
    p.D = D;
    p.R = const_cast<float*>(R);
    p.gout = gout;
    p.G_out = G;
    return status_of(launch_bwd(p, false, false, exact_backward(), (hipStream_t)stream));
}

// Fused forward; with D non-null the matrix-core producer waves also store each cost tile
// into D (B,N,M).
static int fused_fwd_common(const float* x, const float* y, float* D, void* record, float* R,
                            float* out, int64_t B, int64_t N, int64_t M, int64_t K, double gamma,
                            double bandwidth, void* ws, size_t ws_bytes, void* stream) {
    if (!shape_ok(B, N, M, K, true) || !gamma_ok(gamma)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!x || !y || !R || !out) return SDTW_ERR_INVALID_VALUE;
    hipStream_t st = (hipStream_t)stream;
    Carver c{static_cast<char*>(ws), ws_bytes};
    float* x2 = c.take<float>(B * N);
    float* y2 = c.take<float>(B * M);
    const int wmax = fused_fwd_wmax(B, N, M, K, bandwidth);
    const DPScratch d = carve_dp(c, B, N, M, wmax);
    if (!c.ok) return SDTW_ERR_WORKSPACE;
    DPParams p{};
    fill_dp(p, d, B, N, M, K, gamma, bandwidth, wmax);
    p.x = x;
    p.y = y;
    p.x2 = x2;
    p.y2 = y2;
    p.x2_fill = x2;  // the norms are formed by the prep launch
    p.y2_fill = y2;
    p.R = R;
    p.out = out;
    p.D_out = D;
    // pairs whose norms allow it take the scaled linear-domain recursion (mixed arithmetic,
    // matrix-core costs, no band, up to 2 bands per workgroup)
    p.lin = lin_forward() && !(p.bw > 0.0) && mfma_costs(N, M, K) && p.W <= 2 ? 1 : 0;
    if (D && record) {  // the distance record: clamp flags, and the norms formed here
        const DistRecord rec = dist_record(record, B, N, M);
        p.clamped = rec.clamped;
        p.x2 = p.x2_fill = rec.x2;
        p.y2 = p.y2_fill = rec.y2;
    }
    return status_of(launch_fwd(p, true, small_bmm(N, M, K), exact_forward(), st));
}

int sdtw_fused_fwd_f32(const float* x, const float* y, float* R, float* out, int64_t B,
                       int64_t N, int64_t M, int64_t K, double gamma, double bandwidth,
                       void* ws, size_t ws_bytes, void* stream) {
    return fused_fwd_common(x, y, nullptr, nullptr, R, out, B, N, M, K, gamma, bandwidth, ws,
                            ws_bytes, stream);
}

int sdtw_fused_fwd_d_f32(const float* x, const float* y, float* D, void* record, float* R,
                         float* out, int64_t B, int64_t N, int64_t M, int64_t K, double gamma,
                         double bandwidth, void* ws, size_t ws_bytes, void* stream) {
    if (!shape_ok(B, N, M, K, true)) return SDTW_ERR_INVALID_VALUE;
    if (!mfma_costs(N, M, K)) return SDTW_ERR_UNSUPPORTED;  // scalar cost tiles: no producer
    if (B > 0 && !D) return SDTW_ERR_INVALID_VALUE;
    return fused_fwd_common(x, y, D, record, R, out, B, N, M, K, gamma, bandwidth, ws, ws_bytes,
                            stream);
}

// Fused backward core: norms (formed by the prep launch), then the reverse wavefront writing
// gout * E into `E`.
static int fused_bwd_common(const float* x, const float* y, const float* R, const float* gout,
                            float* E, float* x2, float* y2, const DPScratch& d, int64_t B,
                            int64_t N, int64_t M, int64_t K, double gamma, double bandwidth,
                            hipStream_t st) {
    DPParams p{};
    fill_dp(p, d, B, N, M, K, gamma, bandwidth, fused_bwd_wmax(B, N, M, K));
    p.x = x;
    p.y = y;
    p.x2 = x2;
    p.y2 = y2;
    p.x2_fill = x2;
    p.y2_fill = y2;
    p.R = const_cast<float*>(R);
    p.gout = gout;
    p.G_out = E;
    return status_of(launch_bwd(p, true, small_bmm(N, M, K), exact_backward(), st));
}

int sdtw_fused_bwd_f32(const float* x, const float* y, const float* R, const float* gout,
                       float* gx, float* gy, int64_t B, int64_t N, int64_t M, int64_t K,
                       double gamma, double bandwidth, void* ws, size_t ws_bytes,
                       void* stream) {
    if (!shape_ok(B, N, M, K, true) || !gamma_ok(gamma)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0 || (!gx && !gy)) return SDTW_OK;
    if (!x || !y || !R) return SDTW_ERR_INVALID_VALUE;
    hipStream_t st = (hipStream_t)stream;
    Carver c{static_cast<char*>(ws), ws_bytes};
    float* x2 = c.take<float>(B * N);
    float* y2 = c.take<float>(B * M);
    const DPScratch d = carve_dp(c, B, N, M, fused_bwd_wmax(B, N, M, K));
    if (fused_grad_mode(B, N, M, K, gy != nullptr)) {
        // the gradients inside the recursion kernel: dL/dy is zeroed by the prep launch and
        // accumulated band by band, dL/dx written per band
        if (!c.ok) return SDTW_ERR_WORKSPACE;
        DPParams p{};
        fill_dp(p, d, B, N, M, K, gamma, bandwidth, fused_bwd_wmax(B, N, M, K));
        p.x = x;
        p.y = y;
        p.x2 = x2;
        p.y2 = y2;
        p.x2_fill = x2;
        p.y2_fill = y2;
        p.R = const_cast<float*>(R);
        p.gout = gout;
        p.gx_out = gx;
        p.gy_out = gy;
        return status_of(launch_bwd(p, true, false, exact_backward(), st));
    }
    if (!dist_grid_ok(B, N, M)) return SDTW_ERR_UNSUPPORTED;
    float* Ebuf = c.take<float>(B * N * M);
    float* part = c.take<float>(dist_bwd_split_floats(B, N, M, K));
    int* cnt = c.take<int>(dist_bwd_counters(B, N, M, K));
    if (!c.ok) return SDTW_ERR_WORKSPACE;
    int rc = fused_bwd_common(x, y, R, gout, Ebuf, x2, y2, d, B, N, M, K, gamma, bandwidth, st);
    if (rc != SDTW_OK) return rc;
    DistBwdParams q{};
    q.x = x;
    q.y = y;
    q.D = nullptr;
    q.G = Ebuf;
    q.gx = gx;
    q.gy = gy;
    q.B = (int)B;
    q.N = (int)N;
    q.M = (int)M;
    q.K = (int)K;
    q.mask = 0;
    q.muladd = small_bmm(N, M, K) ? 1 : 0;
    q.part = part;
    q.cnt = cnt;
    return status_of(launch_dist_bwd(q, st));
}

int sdtw_fused_bwd_e_f32(const float* x, const float* y, const float* R, const float* gout,
                         float* E, int64_t B, int64_t N, int64_t M, int64_t K, double gamma,
                         double bandwidth, void* ws, size_t ws_bytes, void* stream) {
    if (!shape_ok(B, N, M, K, true) || !gamma_ok(gamma)) return SDTW_ERR_INVALID_VALUE;
    if (B == 0) return SDTW_OK;
    if (!x || !y || !R || !E) return SDTW_ERR_INVALID_VALUE;
    Carver c{static_cast<char*>(ws), ws_bytes};
    float* x2 = c.take<float>(B * N);
    float* y2 = c.take<float>(B * M);
    const DPScratch d = carve_dp(c, B, N, M, fused_bwd_wmax(B, N, M, K));
    if (!c.ok) return SDTW_ERR_WORKSPACE;
    return fused_bwd_common(x, y, R, gout, E, x2, y2, d, B, N, M, K, gamma, bandwidth,
                            (hipStream_t)stream);
}

// Barycenter loop: [xb (B,N,K)][out (B)][gx (B,N,K)][m, v, grad (N,K) each][norm partials]
// [losses][R][recursion workspace, the larger of the fused forward's and backward's]
static size_t bary_rec_bytes(int64_t B, int64_t N, int64_t K) {
    const size_t f = sdtw_workspace_bytes(SDTW_OP_FUSED_FWD, B, N, N, K);
    const size_t g = sdtw_workspace_bytes(SDTW_OP_FUSED_BWD, B, N, N, K);
    return f > g ? f : g;
}

size_t sdtw_barycenter_workspace_bytes(int64_t B, int64_t N, int64_t K, int max_iter) {
    if (!shape_ok(B, N, N, K, true) || B == 0 || max_iter < 0) return 0;
    const int64_t nk = N * K;
    return 2 * align_up(sizeof(float) * B * nk) + align_up(sizeof(float) * B) +
           3 * align_up(sizeof(float) * nk) + align_up(sizeof(float) * bary_parts(nk)) +
           align_up(sizeof(float) * (max_iter > 0 ? max_iter : 1)) +
           align_up(sizeof(float) * dp_table_elems(B, N, N)) + bary_rec_bytes(B, N, K);
}

int sdtw_barycenter_f32(const float* X, const float* w, float* bary, float* losses,
                        int64_t B, int64_t N, int64_t K, double gamma, int max_iter,
                        const double* lrs, int early_stopping, int patience, double tol,
                        int* iters_run, void* ws, size_t ws_bytes, void* stream) {
    if (!shape_ok(B, N, N, K, true) || B == 0 || !gamma_ok(gamma) || max_iter < 0)
        return SDTW_ERR_INVALID_VALUE;
    if (!X || !w || !bary || (max_iter > 0 && !lrs)) return SDTW_ERR_INVALID_VALUE;
    if (!dist_grid_ok(B, N, N)) return SDTW_ERR_UNSUPPORTED;
    hipStream_t st = (hipStream_t)stream;
    const int64_t nk = N * K;
    Carver c{static_cast<char*>(ws), ws_bytes};
    float* xb = c.take<float>(B * nk);
    float* out = c.take<float>(B);
    float* gx = c.take<float>(B * nk);
    float* m = c.take<float>(nk);
    float* v = c.take<float>(nk);
    float* gbuf = c.take<float>(nk);
    float* part = c.take<float>(bary_parts(nk));
    float* loss = c.take<float>(max_iter > 0 ? max_iter : 1);
    float* R = c.take<float>(dp_table_elems(B, N, N));
    const size_t rec_bytes = bary_rec_bytes(B, N, K);
    void* rec = c.take<unsigned char>(rec_bytes);
    if (!c.ok) return SDTW_ERR_WORKSPACE;
    if (launch_fill_zero(m, nk, st) != hipSuccess || launch_fill_zero(v, nk, st) != hipSuccess ||
        launch_bary_broadcast(bary, xb, B, nk, st) != hipSuccess)
        return SDTW_ERR_LAUNCH;
    double best = INFINITY;
    int wait = 0, it = 0;
    for (; it < max_iter; ++it) {
        // losses of the barycenter (xb: its copy per pair) against every sequence, and
        // d loss / d barycenter per pair (the backward's upstream gradient is the weights;
        // dL/dX is not formed)
        int rc = fused_fwd_common(xb, X, nullptr, nullptr, R, out, B, N, N, K, gamma, -1.0, rec,
                                  rec_bytes, stream);
        if (rc != SDTW_OK) return rc;
        rc = sdtw_fused_bwd_f32(xb, X, R, w, gx, nullptr, B, N, N, K, gamma, -1.0, rec, rec_bytes,
                                stream);
        if (rc != SDTW_OK) return rc;
        // Adam step t = it + 1 with the scalars torch's Adam forms in double
        const double t = (double)(it + 1);
        const double bc1 = 1.0 - pow(0.9, t), bc2 = 1.0 - pow(0.999, t);
        BaryStep s;
        s.one_m_b1 = (float)(1.0 - 0.9);
        s.b2 = (float)0.999;
        s.one_m_b2 = (float)(1.0 - 0.999);
        s.bc2_sqrt = (float)pow(bc2, 0.5);
        s.eps = (float)1e-8;
        s.neg_step = (float)(lrs[it] / bc1 * -1.0);
        s.max_norm = 1.0f;
        if (launch_bary_update(gx, out, w, bary, xb, m, v, gbuf, part, loss + it, (int)B, (int)nk,
                               s, st) != hipSuccess)
            return SDTW_ERR_LAUNCH;
        if (early_stopping) {  // the reference's rule (barycenters.py:149-165) needs the loss
            float lv = 0.0f;
            if (hipMemcpyAsync(&lv, loss + it, sizeof(float), hipMemcpyDeviceToHost, st) != hipSuccess ||
                hipStreamSynchronize(st) != hipSuccess)
                return SDTW_ERR_LAUNCH;
            const double improvement = best - (double)lv;
            if (improvement > tol) {
                best = lv;
                wait = 0;
            } else {
                ++wait;
            }
            if (wait >= patience && it > max_iter / 2) {
                ++it;
                break;
            }
        }
    }
    if (iters_run) *iters_run = it;
    if (losses && it > 0 &&
        hipMemcpyAsync(losses, loss, sizeof(float) * it, hipMemcpyDeviceToDevice, st) != hipSuccess)
        return SDTW_ERR_LAUNCH;
    return SDTW_OK;
}

}  // extern "C"
