#!/usr/bin/env python
"""Headline benchmark of the MI355X Soft-DTW engine (one JSON line on stdout).

Workload: x, y ~ N(0,1) fp32, B=32, N=M=512, D=64, gamma=1,
sqeuclidean; one step = SoftDTW(...)(x, y).sum().backward() with fresh leaf clones of the
resident inputs, as in the reference's bench/bench_memory.py:51-58.  Both modes are timed:
unfused (materialised (B,N,M) cost) and fused (cost recomputed per cell).

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--mode both|unfused|fused]
                    [--no-cpu-baseline] [--kernel NAME --launches L] [--grid] [--configs]

`value` is unfused DP cells/s = B*N*M / (fwd+bwd seconds); the fused figures ride along in
the same line.  `roofline` covers the dominant kernel (largest share of a step), timed with
HIP events on the stream the engine launches on.  `cpu_baseline` times the CPU restatement
of the reference's CPU path (oracle/) on the host cores.
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sdtw-cuda-torch_amd"))
sys.path.insert(0, ROOT)

METRIC = "fwd+bwd ms & DP cells/s at B=32 N=M=512 D=64 (unfused, fused); peak MB"
HBM_PEAK_GBS = 8000.0
# reference CSV artefact, bench/softdtw_memory_benchmark.csv:13 (unfused 20.102 ms)
REF_UNFUSED_MS = 20.102
REF_FUSED_MS = 141.358


# The reference's benchmark grid and its own timings (bench/bench_memory.py:163-167 for the
# configurations, bench/softdtw_memory_benchmark.csv:2-17 for the figures: columns
# ours_unfused_ms and ours_fused_ms, its engine on an unstated NVIDIA GPU): B, N = M, D,
# unfused ms, fused ms.
REF_GRID = [
    (16, 128, 1, 2.1553, 36.7759), (16, 128, 64, 2.1559, 35.9518),
    (16, 512, 1, 21.1427, 139.8459), (16, 512, 64, 19.3399, 141.8058),
    (16, 1024, 1, 71.2458, 281.7823), (16, 1024, 64, 71.7209, 278.0873),
    (16, 2048, 1, 489.8424, 557.3357), (16, 2048, 64, 484.7632, 592.2209),
    (32, 128, 1, 1.8979, 35.7862), (32, 128, 64, 1.9554, 35.9961),
    (32, 512, 1, 19.6090, 140.4723), (32, 512, 64, 20.1023, 141.3577),
    (32, 1024, 1, 73.6546, 281.0321), (32, 1024, 64, 75.2204, 288.9885),
    (32, 2048, 1, 489.4542, 567.0535), (32, 2048, 64, 491.6920, 1838.2080),
]


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_inputs(B, N, M, K, seed=0):
    import torch

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, N, K, generator=g)
    y = torch.randn(B, M, K, generator=g)
    return x, y


def algorithmic_bytes(kernel, B, N, M, K):
    """Minimal HBM bytes one launch of `kernel` must move (fp32)."""
    cells = B * N * M
    xy = B * (N + M) * K
    return {
        "dist_fwd": 4 * (cells + xy),          # read x, y; write D
        "dp_fwd": 4 * (2 * cells),             # read D; write R
        "dp_bwd": 4 * (3 * cells),             # read D, R; write G
        "dist_bwd": 4 * (cells + 2 * xy),      # read G, x, y; write gx, gy
        "fused_fwd": 4 * (cells + xy),         # read x, y; write R
        "fused_fwd_d": 4 * (2 * cells + xy),   # read x, y; write D, R
        "fused_bwd_e": 4 * (2 * cells + xy),   # read R, x, y; write g*E
        "fused_bwd": 4 * (cells + 2 * xy),     # read R, x, y; write gx, gy (no E)
    }[kernel]


COPY_BYTES = 256 * 2 ** 20  # calibration copy: 256 MiB read + 256 MiB written


def kernel_launcher(name, xg, yg, gamma):
    """Closure launching exactly one engine kernel family on torch's current stream
    ("copy": a plain device copy of known size, the counter calibration)."""
    import torch

    from softdtw_cuda import _engine

    if name == "copy":
        src = torch.ones(COPY_BYTES // 4, device=xg.device)
        dst = torch.empty_like(src)
        return lambda: dst.copy_(src)

    D = _engine.sqeuclid_fwd(xg, yg)
    out, R = _engine.dtw_fwd(D, gamma, -1.0)
    G = _engine.dtw_bwd(D, R, gamma, -1.0)
    # the distance backward as the unfused module runs it: with the one-launch forward's
    # distance record where that forward is taken
    B_, N_, K_ = xg.shape
    M_ = yg.shape[1]
    record = (_engine.fused_fwd_d(xg, yg, gamma, -1.0)[3]
               if _engine.one_launch_unfused_forward(B_, N_, M_, K_, xg.device) else None)
    fn = {
        "dist_fwd": lambda: _engine.sqeuclid_fwd(xg, yg),
        "dp_fwd": lambda: _engine.dtw_fwd(D, gamma, -1.0),
        "dp_bwd": lambda: _engine.dtw_bwd(D, R, gamma, -1.0),
        "dist_bwd": lambda: _engine.sqeuclid_bwd(xg, yg, D, G, mask=True, record=record),
        "fused_fwd": lambda: _engine.fused_fwd(xg, yg, gamma, -1.0),
        "fused_fwd_d": lambda: _engine.fused_fwd_d(xg, yg, gamma, -1.0),
        "fused_bwd_e": lambda: _engine.fused_bwd_e(xg, yg, R, gamma, -1.0),
        "fused_bwd": lambda: _engine.fused_bwd(xg, yg, R, gamma, -1.0),
    }[name]
    return fn


class _no_gc:
    """Collect garbage before a timed region and keep the collector off inside it, as
    timeit does: a full collection of the interpreter's objects (tens of ms with torch
    loaded) otherwise lands, at an allocation-count-determined point, inside a host-bound
    step of a few hundred microseconds."""

    def __enter__(self):
        self.was = gc.isenabled()
        gc.collect()
        gc.disable()

    def __exit__(self, *exc):
        if self.was:
            gc.enable()


def time_kernel(fn, launches, warmup=2):
    """ms per engine launch: one pair of HIP events around `launches` back-to-back launches
    on the engine's stream (an event pair around every launch would add its own marker
    packets, about 10 us each, between the kernels)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    with _no_gc():
        a.record(st)
        for _ in range(launches):
            fn()
        b.record(st)
        torch.cuda.synchronize()
    return a.elapsed_time(b) / launches


def time_steps(step, steps, warmup):
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    st = torch.cuda.current_stream()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    with _no_gc():
        torch.cuda.synchronize()
        a.record(st)
        for _ in range(steps):
            step()
        b.record(st)
        torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    peak = torch.cuda.max_memory_allocated() / 2 ** 20
    return ms, peak


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` at the headline shape from the committed rocprofv3
    counter summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), or
    None if no summary is committed."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_B32_N512_D64_traffic.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    return None


def cpu_baseline(x, y, gamma, budget_s=15.0):
    """The oracle (reference CPU path restated: torch-CPU distance + C DP + autograd),
    fwd+bwd over the same headline batch, on this host's cores."""
    import torch

    import oracle

    cores = len(os.sched_getaffinity(0))
    cores = min(cores, 16)  # the GPU box grants one GPU's share of host cores
    torch.set_num_threads(cores)
    oracle.load_library()

    def run():
        xo = x.clone().requires_grad_(True)
        yo = y.clone().requires_grad_(True)
        oracle.softdtw(xo, yo, gamma=gamma, nthreads=cores).sum().backward()

    run()  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    B, N, K = x.shape
    M = y.shape[1]
    return {
        "value": B * N * M / med,
        "unit": "cells/s",
        "cores": cores,
        "kind": "port",
        "ms_per_step": med * 1e3,
        "sample": f"full headline batch B={B} N={N} M={M} D={K}, unfused CPU route "
                  f"(torch-CPU distance + C/OpenMP DP over pairs), median of {len(times)} "
                  f"fwd+bwd runs after 1 warm-up",
    }


def run_grid(numerics):
    """The reference's grid, timed as its bench_memory.py:24-58 does (fresh leaf clones,
    fwd + sum + bwd per step; one warm-up, then the mean of 5 between events)."""
    import torch

    from softdtw_cuda import SoftDTW

    rows = []
    for B, N, K, ref_u, ref_f in REF_GRID:
        x, y = make_inputs(B, N, N, K, seed=0)
        X, Y = x.cuda(), y.cuda()
        row = {"B": B, "N": N, "M": N, "D": K}
        for mode, ref in (("unfused", ref_u), ("fused", ref_f)):
            sdtw = SoftDTW(gamma=1.0, fused=(mode == "fused"))

            def step():
                xs = X.detach().clone().requires_grad_(True)
                ys = Y.detach().clone().requires_grad_(True)
                sdtw(xs, ys).sum().backward()

            torch.cuda.empty_cache()
            ms, peak = time_steps(step, 5, 1)
            row[mode] = {"ms": round(ms, 4), "peak_mib": round(peak, 2), "reference_ms": ref,
                         "speedup": round(ref / ms, 2)}
            log(f"[grid] B={B} N=M={N} D={K} {mode}: {ms:.3f} ms (reference {ref} ms, "
                f"{ref / ms:.1f}x), peak {peak:.1f} MiB")
        rows.append(row)
        del X, Y
    line = {
        "metric": "fwd+bwd ms per step over the reference's benchmark grid",
        "unit": "ms", "higher_is_better": False, "n_gpus": 1, "numerics": numerics,
        "dtype": "f32 (fp64 DP state)", "data": "synthetic (randn seed 0, y drawn after x)",
        "reference_source": "bench/softdtw_memory_benchmark.csv:2-17 (unstated NVIDIA GPU)",
        "grid": rows,
    }
    print(json.dumps(line), flush=True)
    return 0


def sinusoids(B, N, K, g):
    """Normalize-config inputs: a sin(f t + phi) + N(0, 0.1), f ~ U[0.5, 3], phi ~ U[0, 2 pi],
    a ~ U[0.5, 2] per (batch, feature)."""
    import math

    import torch

    t = torch.linspace(0, 2 * math.pi, N).view(1, N, 1)
    f = 0.5 + 2.5 * torch.rand(B, 1, K, generator=g)
    ph = 2 * math.pi * torch.rand(B, 1, K, generator=g)
    a = 0.5 + 1.5 * torch.rand(B, 1, K, generator=g)
    return a * torch.sin(f * t + ph) + 0.1 * torch.randn(B, N, K, generator=g)


def random_walks(Kseq, N, D, g):
    """Barycenter-config inputs: cumsum of N(0, 0.1) steps plus a shared sinusoid template
    sin(2 pi n / N (d + 1) / 2)."""
    import math

    import torch

    n = torch.arange(N, dtype=torch.float32).view(N, 1)
    d = torch.arange(D, dtype=torch.float32).view(1, D)
    template = torch.sin(2 * math.pi * n / N * (d + 1) * 0.5)
    return torch.cumsum(0.1 * torch.randn(Kseq, N, D, generator=g), dim=1) + template


def run_configs(numerics):
    """BASELINE.json configs 0, 2, 3, 4 on the GPU (config 1 is the default run): fwd+bwd
    ms per step with fresh leaf clones (plumbing: loss .mean(); the others .sum()), the median
    of three timed runs after a warm-up, and the barycenter's 100 iterations end to end."""
    import torch

    def median_of_runs(step, steps, warmup, runs=3):
        res = [time_steps(step, steps, warmup if r == 0 else 1) for r in range(runs)]
        return statistics.median(r[0] for r in res), max(r[1] for r in res)

    from softdtw_cuda import SoftDTW, softdtw_barycenter

    out = {}

    def step_of(sdtw, X, Y, reduce):
        def step():
            xs = X.detach().clone().requires_grad_(True)
            ys = Y.detach().clone().requires_grad_(True)
            loss = sdtw(xs, ys)
            (loss.mean() if reduce == "mean" else loss.sum()).backward()
        return step

    x, y = make_inputs(4, 64, 64, 8, seed=0)
    ms, peak = median_of_runs(step_of(SoftDTW(gamma=1.0, fused=False), x.cuda(), y.cuda(), "mean"), 20, 10)
    out["plumbing B=4 N=M=64 D=8 unfused"] = {"ms": round(ms, 4), "peak_mib": round(peak, 2)}
    log(f"[configs] plumbing: {ms:.3f} ms")

    x, y = make_inputs(16, 4096, 3072, 4, seed=0)
    X, Y = x.cuda(), y.cuda()
    for fused in (False, True):
        ms, peak = median_of_runs(step_of(SoftDTW(gamma=0.1, fused=fused), X, Y, "sum"), 5, 1)
        key = f"long B=16 N=4096 M=3072 D=4 gamma=0.1 {'fused' if fused else 'unfused'}"
        out[key] = {"ms": round(ms, 3), "peak_mib": round(peak, 1),
                    "cells_per_s": 16 * 4096 * 3072 / (ms * 1e-3)}
        log(f"[configs] {key}: {ms:.3f} ms")
    del X, Y
    torch.cuda.empty_cache()

    g = torch.Generator().manual_seed(0)
    x = sinusoids(64, 256, 16, g)
    y = sinusoids(64, 256, 16, g)
    ms, peak = median_of_runs(step_of(SoftDTW(gamma=1.0, normalize=True, fused=True), x.cuda(),
                                      y.cuda(), "sum"), 20, 10)
    out["normalize B=64 N=M=256 D=16 fused"] = {"ms": round(ms, 4), "peak_mib": round(peak, 2)}
    log(f"[configs] normalize: {ms:.3f} ms")

    g = torch.Generator().manual_seed(0)
    Xb = random_walks(64, 256, 8, g).cuda()
    softdtw_barycenter(Xb, gamma=1.0, max_iter=2, lr=0.1, early_stopping=False)  # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    softdtw_barycenter(Xb, gamma=1.0, max_iter=100, lr=0.1, early_stopping=False)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3
    out["barycenter K=64 N=256 D=8, 100 Adam iterations"] = {"ms": round(ms, 2),
                                                              "ms_per_iteration": round(ms / 100, 4)}
    log(f"[configs] barycenter: {ms:.1f} ms")

    print(json.dumps({"metric": "fwd+bwd ms per step at the other BASELINE.json configs",
                      "unit": "ms", "higher_is_better": False, "n_gpus": 1,
                      "numerics": numerics, "dtype": "f32 (fp64 DP state)",
                      "data": "synthetic (seed 0)", "configs": out}), flush=True)
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--mode", choices=["both", "unfused", "fused"], default="both")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel", default=None,
                    help="only launch one kernel family repeatedly (for rocprofv3 runs): "
                         "dist_fwd, dp_fwd, dp_bwd, dist_bwd, fused_fwd, fused_fwd_d, fused_bwd, "
                         "fused_bwd_e, copy")
    ap.add_argument("--launches", type=int, default=20)
    ap.add_argument("--shape", default=None,
                    help="B,N,M,D for --kernel runs (default: the headline 32,512,512,64)")
    ap.add_argument("--grid", action="store_true",
                    help="time the reference's benchmark grid (16 configurations, unfused and "
                         "fused, its protocol: one warm-up step, then the mean of 5) and print "
                         "one JSON line with the reference's figures beside ours")
    ap.add_argument("--configs", action="store_true",
                    help="time the other BASELINE.json configurations (plumbing, long "
                         "sequences, normalize, barycenter) and print one JSON line")
    ap.add_argument("--numerics", choices=["mixed", "exact", "fast"], default="mixed",
                    help="cell arithmetic of the recursions (mixed, the default: forward "
                         "bit-identical to the reference CPU path, backward weights in fp32; "
                         "exact: both recursions fp64-accurate)")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this engine is measured on one GPU only (pairs are independent, so "
              "a batch shards across GPUs by pairs with no exchange). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    import torch

    from softdtw_cuda import SoftDTW, set_numerics

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    set_numerics(args.numerics)

    if args.grid:
        return run_grid(args.numerics)
    if args.configs:
        return run_configs(args.numerics)

    B, N, M, K, gamma = 32, 512, 512, 64, 1.0
    cells = B * N * M
    x, y = make_inputs(B, N, M, K, seed=0)
    X = x.cuda()
    Y = y.cuda()

    if args.kernel:
        if args.shape:
            B, N, M, K = (int(v) for v in args.shape.split(","))
            xk, yk = make_inputs(B, N, M, K, seed=0)
            X, Y = xk.cuda(), yk.cuda()
        fn = kernel_launcher(args.kernel, X, Y, gamma)
        ms = time_kernel(fn, args.launches)
        log(f"kernel {args.kernel}: {ms:.4f} ms/launch over {args.launches} launches")
        return 0

    modes = ["unfused", "fused"] if args.mode == "both" else [args.mode]
    res = {}
    others = {a: {} for a in ("mixed", "exact", "fast") if a != args.numerics}  # reported beside
    for arith, table in [(args.numerics, res)] + list(others.items()):
        set_numerics(arith)
        for mode in modes:
            sdtw = SoftDTW(gamma=gamma, fused=(mode == "fused"))

            def step():
                xs = X.detach().clone().requires_grad_(True)
                ys = Y.detach().clone().requires_grad_(True)
                sdtw(xs, ys).sum().backward()

            log(f"[bench] numerics={arith} mode={mode} warmup={args.warmup} steps={args.steps}")
            ms, peak = time_steps(step, args.steps, args.warmup)
            table[mode] = {"ms_per_step": ms, "cells_per_s": cells / (ms * 1e-3), "peak_mib": peak}
            log(f"[bench] numerics={arith} mode={mode} {ms:.3f} ms/step  "
                f"{cells / (ms * 1e-3):.3e} cells/s  peak {peak:.1f} MiB")
    set_numerics(args.numerics)

    # per-kernel timing (HIP events on the engine's stream) -> dominant kernel roofline
    kernels = []
    # unfused mode's forward: one launch forming D and R (fused_fwd_d) where the module takes
    # it (not under "fast" arithmetic), else the distance and the recursion apart
    from softdtw_cuda import _engine
    unfused_kernels = (["fused_fwd_d", "dp_bwd", "dist_bwd"]
                       if _engine.one_launch_unfused_forward(B, N, M, K, X.device)
                       else ["dist_fwd", "dp_fwd", "dp_bwd", "dist_bwd"])
    if "unfused" in res:
        kernels += unfused_kernels
    if "fused" in res:
        kernels += ["fused_fwd", "fused_bwd"]
    per = {}
    for kname in kernels:
        fn = kernel_launcher(kname, X, Y, gamma)
        per[kname] = time_kernel(fn, max(5, min(args.steps, 20)))
        log(f"[bench] kernel {kname}: {per[kname]:.4f} ms/launch")
    head_mode = "unfused" if "unfused" in res else "fused"
    head_kernels = {"unfused": unfused_kernels, "fused": ["fused_fwd", "fused_bwd"]}[head_mode]
    dom = max(head_kernels, key=per.get)  # dominant kernel of the step `value` measures
    abytes = algorithmic_bytes(dom, B, N, M, K)
    achieved = abytes / (per[dom] * 1e-3) / 1e9
    roofline = {
        "bound": "hbm",
        "kernel": dom,
        "achieved": round(achieved, 3),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 6),
        "traffic": measured_traffic(dom),
        "algorithmic_bytes_per_launch": abytes,
        "avg_launch_ms": round(per[dom], 5),
        "diagonal_steps_per_launch": N + M - 1,
        "ns_per_diagonal_step": round(per[dom] * 1e6 / (N + M - 1), 2),
        "kernel_ms": {k: round(v, 5) for k, v in per.items()},
    }

    head = res.get("unfused") or res["fused"]
    line = {
        "metric": METRIC,
        "value": head["cells_per_s"],
        "unit": "cells/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (head["cells_per_s"] / (cells / (REF_UNFUSED_MS * 1e-3)))
        if "unfused" in res else None,
        "dtype": "f32 (fp64 DP state)",
        "data": "synthetic",
        "config": {
            "workload": "headline (BASELINE.json configs[1]): SoftDTW fwd+bwd, "
                        "B=32 N=M=512 D=64 gamma=1 sqeuclidean, randn seed 0",
            "B": B, "N": N, "M": M, "D": K, "gamma": gamma,
            "value_mode": "unfused" if "unfused" in res else "fused",
        },
        "numerics": args.numerics,
        "modes": {k: {kk: (round(vv, 4) if kk != "cells_per_s" else vv) for kk, vv in v.items()}
                  for k, v in res.items()},
        **{f"modes_{alt}_numerics": {k: {kk: (round(vv, 4) if kk != "cells_per_s" else vv)
                                         for kk, vv in v.items()} for k, v in other.items()}
           for alt, other in others.items()},
        "reference_ms": {"unfused": REF_UNFUSED_MS, "fused": REF_FUSED_MS,
                         "source": "bench/softdtw_memory_benchmark.csv:13 (unstated NVIDIA GPU)"},
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline (oracle on host cores)")
        line["cpu_baseline"] = cpu_baseline(x, y, gamma)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
