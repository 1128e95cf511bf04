import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


def load_golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


def tol(want):
    """The reference's oracle band: 1e-5 relative to max(|v|, 1)
    (crates/mlrs-backend/tests/knn_metric_kernel_test.rs:161-163)."""
    return 1e-5 * np.maximum(np.abs(want), 1.0)


def assert_topk_matches(got_d, got_i, want_d, want_i, ref_dist_fn, atol_rel=1e-5):
    """Distances positionally within the band; an index may differ from the
    reference only where the picked neighbour's reference distance is within the
    band of the reference's pick (knn_metric_kernel_test.rs:166-222)."""
    got_d = np.asarray(got_d, dtype=np.float64)
    want_d = np.asarray(want_d, dtype=np.float64)
    band = atol_rel * np.maximum(np.abs(want_d), 1.0)
    assert np.all(np.abs(got_d - want_d) <= band), np.max(np.abs(got_d - want_d) - band)
    rows, k = want_d.shape
    for r in range(rows):
        for c in range(k):
            if int(got_i[r, c]) != int(want_i[r, c]):
                picked = ref_dist_fn(r, int(got_i[r, c]))
                assert abs(picked - want_d[r, c]) <= band[r, c], (r, c, got_i[r, c], want_i[r, c])
