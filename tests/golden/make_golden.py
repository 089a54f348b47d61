"""Write tests/golden/bruteforce.json: Soft-DTW values and gradients by path enumeration.

Each case holds a float32-representable cost matrix D (seeded), gamma, bandwidth, and the
float64 brute-force value and path marginals E = d value / d D.  These vectors come from
the definition (sum over alignment paths), not from any recursion, so they pin both the
CPU oracle and the GPU engine.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from _checkers import brute_force  # noqa: E402

CASES = [
    # N, M, gamma, bandwidth, seed, scale
    (1, 1, 1.0, None, 1, 3.0),
    (1, 6, 1.0, None, 2, 3.0),
    (5, 1, 0.5, None, 3, 3.0),
    (3, 4, 1.0, None, 4, 3.0),
    (5, 5, 1.0, None, 5, 3.0),
    (6, 4, 0.1, None, 6, 3.0),
    (4, 6, 2.0, None, 7, 3.0),
    (6, 6, 0.3, 2.0, 8, 3.0),
    (5, 6, 1.0, 1.0, 9, 3.0),
    (6, 5, 0.01, None, 10, 3.0),
    (4, 4, 1.0, 0.5, 11, 3.0),
    (6, 6, 1.0, None, 12, 40.0),
]


def main():
    out = []
    for N, M, gamma, bw, seed, scale in CASES:
        rng = np.random.default_rng(seed)
        D = (rng.random((N, M)) * scale).astype(np.float32)
        val, E = brute_force(D.astype(np.float64), gamma, bw)
        out.append({
            "N": N, "M": M, "gamma": gamma, "bandwidth": bw, "seed": seed,
            "D": [[float(v) for v in row] for row in D],
            "value": val,
            "E": [[float(v) for v in row] for row in E],
        })
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "bruteforce.json")
    with open(path, "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py", "cases": out}, f, indent=1)
    print(path, len(out))


if __name__ == "__main__":
    main()
