"""Parity at the benchmark configurations' full sizes (GPU).

Each configuration's full synthetic data is regenerated (mlrs_amd.synthetic,
seeded) and checked against the generator fingerprints stored with the golden
subsets; the engine then answers the WHOLE query set and

* every row must equal the CPU oracle's answer, computed here on the host's
  cores over the whole query set (about 20 s of CPU for c1-c5 together on 16
  threads), bit for bit;
* the golden subset (CPU-oracle answers against the full index, written by
  tests/golden/gen_golden.py when the fixtures were made) must match too --
  it guards against the generator or the oracle drifting between hosts;
* every row must satisfy the size-independent properties of the reference's
  output contract: ascending values (index order on equal cosine values),
  indices in range and distinct per row, finite values; self-kNN rows start
  at distance 0; k-means labels in range with the label's squared distance
  the row minimum over a sampled recomputation.
"""
import os
import sys
import time

import numpy as np
import pytest

from conftest import load_golden

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _fingerprint_ok(z, key, arr):
    # a drift detector for the generator: the float64 dot products behind the
    # fingerprint may sum in another order on another host's BLAS
    from gen_golden import fingerprint
    np.testing.assert_allclose(fingerprint(arr), z[key], rtol=1e-12, atol=0)


def _row_properties(dist, idx, n_index, ordered_by_output):
    assert np.all(np.isfinite(dist))
    assert np.all((idx >= 0) & (idx < n_index))
    dv = np.diff(dist, axis=1)
    assert np.all(dv >= 0)
    if ordered_by_output:
        # cosine emits the selected values themselves: equal values are in index
        # order.  (Euclidean rows are ordered by the squared values; two of those
        # can share one rounded root, so there the root ties carry no order.)
        ties = dv == 0
        assert np.all(np.diff(idx, axis=1)[ties] > 0)
    # distinct neighbours per row
    s = np.sort(idx, axis=1)
    assert np.all(np.diff(s, axis=1) != 0)


@pytest.mark.parametrize("cfg", ["c1", "c2", "c3", "c4"])
def test_config_knn_full_size(cfg):
    from mlrs_amd import prims, synthetic
    print("config", cfg, flush=True)
    c = synthetic.CONFIGS[cfg]
    z = load_golden("%s_golden" % cfg)
    a, b = synthetic.generate(cfg)
    _fingerprint_ok(z, "fp_query", a)
    _fingerprint_ok(z, "fp_index", b)
    dev = torch.device("cuda:0")
    dist, idx = prims.knn_topk(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), c["k"], c["metric"])
    torch.cuda.synchronize()
    dist = dist.cpu().numpy()
    idx = idx.cpu().numpy()
    sub = z["subset"]
    np.testing.assert_array_equal(idx[sub], z["idx"].astype(np.int64))
    np.testing.assert_array_equal(dist[sub], z["dist"])
    _row_properties(dist, idx, b.shape[0], c["metric"] == "cosine")
    import oracle
    t0 = time.time()
    wd, wi = oracle.knn_topk(a, b, c["k"], c["metric"])
    print("%s: oracle answered all %d rows in %.1f s" % (cfg, a.shape[0], time.time() - t0), flush=True)
    bad = np.argwhere(idx != wi.astype(np.int64))
    assert bad.size == 0, "%s: %d index mismatches, first %s" % (cfg, len(bad), bad[:3].tolist())
    bad = np.argwhere(dist != wd)
    assert bad.size == 0, "%s: %d distance mismatches, first %s" % (cfg, len(bad), bad[:3].tolist())
    if cfg == "c4":  # self-kNN: every point finds itself (or an exact duplicate) at distance 0
        assert np.all(dist[:, 0] == 0)


def test_config_kmeans_full_size():
    from mlrs_amd import prims, synthetic
    print("config c5", flush=True)
    z = load_golden("c5_golden")
    a, b = synthetic.generate("c5")
    _fingerprint_ok(z, "fp_points", a)
    _fingerprint_ok(z, "fp_centroids", b)
    dev = torch.device("cuda:0")
    labels, sq = prims.kmeans_assign(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev))
    torch.cuda.synchronize()
    labels = labels.cpu().numpy()
    sq = sq.cpu().numpy()
    sub = z["subset"]
    np.testing.assert_array_equal(labels[sub], z["labels"].astype(np.int64))
    np.testing.assert_array_equal(sq[sub], z["sqdist"])
    assert np.all((labels >= 0) & (labels < b.shape[0]))
    assert np.all(np.isfinite(sq)) and np.all(sq >= 0)
    import oracle
    t0 = time.time()
    wl, ws = oracle.kmeans_assign(a, b)
    print("c5: oracle answered all %d rows in %.1f s" % (a.shape[0], time.time() - t0), flush=True)
    bad = np.argwhere(labels != wl.astype(np.int64))
    assert bad.size == 0, "c5: %d label mismatches, first %s" % (len(bad), bad[:3].tolist())
    bad = np.argwhere(sq != ws)
    assert bad.size == 0, "c5: %d distance mismatches, first %s" % (len(bad), bad[:3].tolist())
    # a sampled recomputation in float64: no centroid is clearly closer than the label's
    rng = np.random.default_rng(7)
    rows = rng.choice(a.shape[0], 4096, replace=False)
    d64 = ((a[rows, None, :].astype(np.float64) - b[None, :, :].astype(np.float64)) ** 2).sum(-1)
    best = d64.min(1)
    assert np.all(d64[np.arange(rows.size), labels[rows]] <= best * (1 + 1e-5) + 1e-6)
