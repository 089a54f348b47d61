"""Build the gfx950 Soft-DTW engine: csrc/*.hip -> softdtw_cuda/_lib/libsdtw_hip.so.

Plain hipcc, no torch headers: the library exposes only the C ABI of include/sdtw.h and is
loaded with ctypes after `import torch` (so it binds to the HIP runtime torch has loaded).

    python sdtw-cuda-torch_amd/build.py [--jobs N] [--verbose]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "softdtw_cuda", "_lib")
OBJDIR = os.path.join(HERE, "_build")
LIB = os.path.join(LIBDIR, "libsdtw_hip.so")
ARCH = os.environ.get("SDTW_OFFLOAD_ARCH", "gfx950")

# every translation unit in csrc/ (the wavefront kernels are split per variant so they
# compile in parallel)
SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))

# -ffp-contract=off: the exact-distance and DP arithmetic is order-sensitive (fmas are
# written explicitly where wanted).  The packed-fp32 feature is switched off for all device
# code (v_pk_* fp32 forms are not trusted on this pool).
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines()
                    if "unknown target feature" not in l and "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build(jobs: int | None = None, verbose: bool = False) -> str:
    hipcc = _hipcc()
    os.makedirs(OBJDIR, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    objs = []
    cmds = []
    for stale in os.listdir(OBJDIR):  # objects of removed sources must not be linked
        if stale.endswith(".o") and stale.replace(".o", ".hip") not in SOURCES:
            os.remove(os.path.join(OBJDIR, stale))
    for src in SOURCES:
        obj = os.path.join(OBJDIR, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([hipcc, *COMMON, "-c", os.path.join(CSRC, src), "-o", obj])
    jobs = jobs or min(len(cmds), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args(argv)
    path = build(a.jobs, a.verbose)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
