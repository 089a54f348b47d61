"""Accuracy of the table-driven fp64 exp / log of the exact recursions (sdtw_math.hpp).

The header is compiled for the host with g++ (the same source the kernels include) and
checked against long double (x87, 64-bit mantissa) libm on random arguments over the ranges
the recursions use, plus the special values the kernels rely on.  CPU only.
"""
import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "sdtw-cuda-torch_amd", "csrc")

HARNESS = r"""
#include <cmath>
#include <cstdio>
#include <random>
#include "sdtw_math.hpp"
using namespace sdtw::fm;
int main() {
    double Tf[kExpTabN];  // the forward's table for exp_tab_abs
    for (int j = 0; j < kExpTabN; ++j) Tf[j] = exp2tab_folded(j);
    std::mt19937_64 g(12345);
    std::uniform_real_distribution<double> u01(0.0, 1.0);
    double emax = 0.0, amax = 0.0, lmax = 0.0;
    for (int i = 0; i < 400000; ++i) {
        // exp arguments: -2^e * U[0,1), e in [0, 11]: the recursions pass (m - R) / gamma <= 0
        const double x = -std::ldexp(u01(g), (int)(g() % 12));
        const long double ref = expl((long double)x);
        if (ref > 1e-300L) {
            const double err = (double)fabsl(((long double)exp_tab(x, kExp2Tab) - ref) / ref);
            if (err > emax) emax = err;
        }
        // the forward's variant: absolute accuracy (its result is added to 1)
        const double aerr = (double)fabsl((long double)exp_tab_abs(x, Tf) - ref);
        if (aerr > amax) amax = aerr;
        // log arguments: a soft-min's sum of exponentials, in [1, 3]
        const double s = 1.0 + 2.0 * u01(g);
        const double le = (double)fabsl((long double)log_tab_1to3(s, kLogTab) - logl((long double)s));
        if (le > lmax) lmax = le;
    }
    std::printf("%.6e %.6e %.6e\n", emax, lmax, amax);
    std::printf("%a %a %a %a\n", exp_tab(0.0, kExp2Tab), exp_tab(-INFINITY, kExp2Tab),
                log_tab_1to3(1.0, kLogTab), log_tab_1to3(3.0, kLogTab));
    std::printf("%d %d\n", (int)std::isnan(log_tab_1to3(NAN, kLogTab)),
                (int)(exp_tab(-1e300, kExp2Tab) == 0.0));
    // below the clamp: exp(-708), normal, and nothing next to 1
    const double lo = exp_tab_abs(-708.0, Tf);
    std::printf("%a %d %d\n", exp_tab_abs(0.0, Tf),
                (int)(exp_tab_abs(-INFINITY, Tf) == lo && exp_tab_abs(-1e300, Tf) == lo &&
                      exp_tab_abs(-750.0, Tf) == lo),
                (int)(lo > 0x1p-1022 && lo < 0x1p-1020 && 1.0 + lo == 1.0 && 0.25 + lo == 0.25));
    return 0;
}
"""


@pytest.fixture(scope="module")
def harness_output():
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "t.cpp")
        exe = os.path.join(d, "t")
        with open(src, "w") as f:
            f.write(HARNESS)
        subprocess.run([gxx, "-O2", "-std=c++17", "-ffp-contract=off", "-I", CSRC, src, "-o", exe],
                       check=True, capture_output=True)
        return subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split("\n")


def test_exp_and_log_accuracy(harness_output):
    emax, lmax, amax = (float(v) for v in harness_output[0].split())
    assert emax < 4e-16, emax  # relative
    assert amax < 4e-16, amax  # absolute (exp_tab_abs, the forward's)
    assert lmax < 4e-16, lmax  # absolute, |log s| <= 1.1


def test_special_values(harness_output):
    e0, einf, l1, l3 = (float.fromhex(v) for v in harness_output[1].split())
    assert e0 == 1.0          # the soft-min's minimum term is exactly 1
    assert einf == 0.0        # +inf predecessors contribute nothing
    assert l1 == 0.0          # log(1) = 0 exactly, as the reference's libm gives
    assert abs(l3 - 1.0986122886681098) < 4e-16
    nan_ok, tiny_ok = (int(v) for v in harness_output[2].split())
    assert nan_ok == 1 and tiny_ok == 1
    # the forward's exp_tab_abs: exactly 1 at 0; every argument below -708 (and -inf, for
    # +inf predecessors) gives exp(-708), a normal number that vanishes next to 1 and to any
    # other term of the soft-min's sum, as 0 would
    a0, aclamp, avanish = harness_output[3].split()
    assert float.fromhex(a0) == 1.0 and int(aclamp) == 1 and int(avanish) == 1


def test_tables_are_generated_from_the_committed_generator():
    # the committed tables are what gen_tables.py writes
    import sys

    sys.path.insert(0, CSRC)
    try:
        import gen_tables  # noqa: F401
    finally:
        sys.path.pop(0)
    with tempfile.TemporaryDirectory() as d:
        here = os.path.join(d, "csrc")
        os.makedirs(here)
        shutil.copy(os.path.join(CSRC, "gen_tables.py"), here)
        subprocess.run(["python3", os.path.join(here, "gen_tables.py")], check=True)
        with open(os.path.join(here, "sdtw_tables.hpp")) as a, open(os.path.join(CSRC, "sdtw_tables.hpp")) as b:
            assert a.read() == b.read()
