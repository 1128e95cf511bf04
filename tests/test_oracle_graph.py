"""Pins the CPU oracle's X-vs-X scans (oracle/graph_cpu.c) -- CPU only.

* knn_graph against the reference's knn_graph fixtures knn_{metric}_{f32,f64}_
  seed42 (sklearn X-vs-X neighbours, k+1 with self) to the reference test's bar:
  per-row index sets equal and sorted distances within 1e-5 + 1e-5|want|
  (crates/mlrs-backend/tests/knn_graph_test.rs:106-190), the duplicate-point
  self-drop by identity (:312-377) and self at column 0 with include_self
  (:385-447).
* knn_graph against the self-dropped neighbour lists the umap_fuzzy_{metric}_
  f64 fixtures hold (UMAP's include_self = false graph).
* An f64 brute force that sorts every row's distances, for the graph and for
  the HDBSCAN core distances (column k-1 of the self-inclusive lists), on
  inputs with ties, duplicate rows and a NaN row.
* The ranking by the final distance (KNearest::push of `(ops.fin)(a)`,
  crates/mlrs-algos/src/manifold/umap_host_knn.rs:171-198, 494): on rows
  whose aggregates differ by one ulp but root to the same double
  (tests/rooted_ties.py), the oracle's lists are the (root, index) order of
  a numpy brute force and differ from the (aggregate, index) order.
"""
import numpy as np
import pytest

import oracle
import rooted_ties
from conftest import load_golden

METRICS = ["euclidean", "manhattan", "chebyshev", "minkowski", "cosine"]


def _brute(x, metric, p):
    """Every pairwise distance in f64, written independently of the oracle."""
    a = x.astype(np.float64)
    if metric == "cosine":
        nrm = np.sqrt((a * a).sum(1))
        a = a * np.where(nrm > 0, 1.0 / np.where(nrm > 0, nrm, 1.0), 0.0)[:, None]
    diff = a[:, None, :] - a[None, :, :]
    if metric == "euclidean":
        return np.sqrt((diff ** 2).sum(-1))
    if metric == "cosine":
        return 0.5 * (diff ** 2).sum(-1)
    if metric == "manhattan":
        return np.abs(diff).sum(-1)
    if metric == "chebyshev":
        return np.abs(diff).max(-1)
    return (np.abs(diff) ** p).sum(-1) ** (1.0 / p)


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("metric", METRICS)
def test_graph_fixture(s, metric):
    z = load_golden("knn_%s_%s_seed42" % (metric, s))
    X, k = z["X"], int(z["k"][0])
    p = float(z["p"][0]) if metric == "minkowski" else 2.0
    idx, dist = oracle.knn_graph(X, k, metric, p=p)
    ri, rd = z["indices"].astype(np.int64), z["distances"]
    for r in range(X.shape[0]):
        keep = ri[r] != r
        want_i, want_d = ri[r][keep][:k], np.sort(rd[r][keep][:k])
        assert set(idx[r].tolist()) == set(want_i.tolist())
        got = np.sort(dist[r])
        assert np.all(np.abs(got - want_d) <= 1e-5 + 1e-5 * np.abs(want_d))
        assert r not in idx[r].tolist()


def test_graph_duplicate_point_and_self_column():
    z = load_golden("knn_euclidean_f64_seed42")
    X, k = z["X"], int(z["k"][0])
    a, b = int(z["dup_row_a"][0]), int(z["dup_row_b"][0])
    idx, dist = oracle.knn_graph(X, k, "euclidean")
    assert idx[a, 0] == b and idx[b, 0] == a and dist[a, 0] == 0.0 and dist[b, 0] == 0.0
    idx, dist = oracle.knn_graph(X, k, "euclidean", include_self=True)
    for r in range(X.shape[0]):
        want = min(a, b) if r in (a, b) else r
        assert idx[r, 0] == want and dist[r, 0] == 0.0


@pytest.mark.parametrize("metric", ["euclidean", "manhattan", "chebyshev", "minkowski"])
def test_graph_umap_fixture_lists(metric):
    z = load_golden("umap_fuzzy_%s_f64" % metric)
    X = z["X"]
    k = int(z["n_neighbors"][0])
    p = 3.0 if metric == "minkowski" else 2.0
    ref_d = z["knn_dist"]
    # the fixture's Minkowski exponent is not stored; check it is p = 3
    if metric == "minkowski":
        d_all = _brute(X, metric, p)
        assert np.allclose(np.sort(d_all, 1)[:, 1:k + 1], np.sort(ref_d, 1), rtol=1e-5, atol=1e-5)
    idx, dist = oracle.knn_graph(X, k, metric, p=p)
    ref_i = z["knn_idx"].astype(np.int64)
    for r in range(X.shape[0]):
        assert set(idx[r].tolist()) == set(ref_i[r].tolist())
        assert np.allclose(np.sort(dist[r]), np.sort(ref_d[r]), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("metric", METRICS)
@pytest.mark.parametrize("include_self", [False, True])
def test_graph_against_brute_force(metric, include_self):
    rng = np.random.default_rng(4)
    x = rng.integers(-3, 4, size=(120, 5)).astype(np.float64)  # many exact ties
    x[7] = x[50]
    x[8] = x[50]
    p = 3.0
    k = 9
    idx, dist = oracle.knn_graph(x, k, metric, p=p, include_self=include_self)
    full = _brute(x, metric, p)
    for r in range(x.shape[0]):
        cand = [j for j in range(x.shape[0]) if include_self or j != r]
        order = sorted(cand, key=lambda j: (full[r, j], j))[:k]
        want_d = full[r, order]
        np.testing.assert_allclose(dist[r], want_d, rtol=1e-12, atol=1e-12)
        # indices agree wherever the distance is not tied within rounding
        for c in range(k):
            same = np.abs(full[r, cand] - want_d[c]) <= 1e-9 * max(1.0, abs(want_d[c]))
            if same.sum() == 1:
                assert idx[r, c] == order[c]


@pytest.mark.parametrize("metric", ["euclidean", "manhattan", "chebyshev", "minkowski"])
@pytest.mark.parametrize("min_samples", [1, 5, 200])
def test_core_distances_brute_and_graph_column(metric, min_samples):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((150, 4))
    x[3] = x[9]
    core = oracle.core_distances(x, min_samples, metric, p=3.0)
    k = min(max(min_samples, 1), x.shape[0])
    full = _brute(x, metric, 3.0)
    np.testing.assert_allclose(core, np.sort(full, 1)[:, k - 1], rtol=1e-12, atol=1e-15)
    _, dist = oracle.knn_graph(x, k, metric, p=3.0, include_self=True)
    np.testing.assert_array_equal(core, dist[:, k - 1])


def test_nan_row_and_errors():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((40, 3))
    x[5, 1] = np.nan
    idx, dist = oracle.knn_graph(x, 4, "euclidean")
    assert dist[5].tolist() == [0.0] * 4 and idx[5].tolist() == [0] * 4   # nothing finite to offer
    assert 5 not in idx[np.arange(40) != 5].ravel().tolist()
    core = oracle.core_distances(x, 3, "euclidean")
    assert core[5] == np.inf and np.isfinite(np.delete(core, 5)).all()
    with pytest.raises(ValueError):
        oracle.knn_graph(x, 40, "euclidean")      # k > n - 1
    with pytest.raises(ValueError):
        oracle.core_distances(x, 3, "cosine")


@pytest.mark.parametrize("metric", ["euclidean", "minkowski"])
@pytest.mark.parametrize("k", [6, 10, 20, 32])
@pytest.mark.parametrize("include_self", [False, True])
def test_graph_ranks_by_root(metric, k, include_self):
    x, p = rooted_ties.build(metric, k)
    want_i, want_d = rooted_ties.brute_graph(x, k, metric, p, by_root=True, include_self=include_self)
    agg_i, _ = rooted_ties.brute_graph(x, k, metric, p, by_root=False, include_self=include_self)
    assert not np.array_equal(want_i, agg_i)   # the data separates the two orders
    got_i, got_d = oracle.knn_graph(x, k, metric, p=p, include_self=include_self)
    np.testing.assert_array_equal(got_i, want_i)
    # the groups' query rows: every value an exact root
    cen = [i for i in range(x.shape[0]) if x[i, 0] % 100.0 == 0.0]
    np.testing.assert_array_equal(got_d[cen], want_d[cen])
    np.testing.assert_allclose(got_d, want_d, rtol=4 * np.finfo(np.float64).eps, atol=0)
