"""Write the golden subsets of the five benchmark configurations.

For each configuration the full-size synthetic data comes from
mlrs_amd.synthetic (seeded); the CPU oracle (oracle/, the restatement of the
mlrs cpu-backend arithmetic) answers a fixed subset of the queries against the
FULL index, and the answers are stored here as small .npz fixtures.  The GPU
parity tests regenerate the same data on the GPU box, run the engine over the
whole query set and compare the subset bit for bit.

Run from the repository root:  python tests/golden/gen_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from mlrs_amd import synthetic  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

SUBSETS = {
    "c1": np.arange(1000),
    "c2": np.arange(0, 10_000, 39)[:256],
    "c3": np.arange(0, 5_000, 79)[:64],
    "c4": np.arange(0, 500_000, 244)[:2048],
    "c5": np.arange(0, 5_000_000, 305)[:16384],
}


def fingerprint(a):
    """Order-sensitive float64 checksum of a few slices (detects generator drift)."""
    a = np.asarray(a)
    n = a.shape[0]
    parts = [a[:64], a[n // 2:n // 2 + 64], a[-64:]]
    w = np.arange(1, 64 * a.shape[1] + 1, dtype=np.float64)
    return np.array([float(np.dot(p.astype(np.float64).ravel(), w[:p.size])) for p in parts])


def main():
    for name, sub in SUBSETS.items():
        cfg = synthetic.CONFIGS[name]
        a, b = synthetic.generate(name)
        if name == "c5":
            labels, sq = oracle.kmeans_assign(a[sub], b)
            np.savez(os.path.join(OUT, "%s_golden.npz" % name), subset=sub, labels=labels, sqdist=sq,
                     fp_points=fingerprint(a), fp_centroids=fingerprint(b))
        else:
            dist, idx = oracle.knn_topk(a[sub], b, cfg["k"], cfg["metric"])
            np.savez(os.path.join(OUT, "%s_golden.npz" % name), subset=sub, dist=dist, idx=idx,
                     fp_query=fingerprint(a), fp_index=fingerprint(b))
        print(name, "written", sub.size, "rows")


if __name__ == "__main__":
    main()
