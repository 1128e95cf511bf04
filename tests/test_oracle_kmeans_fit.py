"""Pins the CPU oracle's k-means fit (oracle/kmeans_cpu.c) -- CPU only.

* The generator: SplitMix64's published outputs (seed 0 and seed 1234567).
* The reference's fixtures kmeans_{f32,f64}_seed42 (sklearn from the same
  injected init): centres, labels, inertia.
* scikit-learn's Lloyd KMeans (an independent implementation of the same
  algorithm, installed here) from the same injected centres on multi-iteration
  data, including a run that empties a cluster (sklearn's
  _relocate_empty_clusters_dense, which the reference follows): labels
  exactly, n_iter up to sklearn's extra leading assignment, centres and
  inertia to rounding.
* feature_mean_var against numpy's variance; the random init against a
  partial Fisher-Yates shuffle on the same stream; k-means++ against what its
  D^2 weighting forces on well-separated clusters; the restart rule against
  the runs made one at a time.
"""
import numpy as np
import pytest

import oracle
from conftest import load_golden


def test_splitmix64_published_values():
    assert [hex(v) for v in oracle.splitmix64(0, 3)] == ["0xe220a8397b1dcdaf", "0x6e789e6aa1b965f4",
                                                          "0x6c45d188009454f"]
    assert int(oracle.splitmix64(1234567, 1)[0]) == 6457827717110365317


@pytest.mark.parametrize("s", ["f32", "f64"])
def test_fixture(s):
    z = load_golden("kmeans_%s_seed42" % s)
    X, init = z["X"], z["init"]
    c, l, inertia, _ = oracle.kmeans_fit(X, init.shape[0], "array", init)
    np.testing.assert_array_equal(l, z["labels"].astype(np.uint32))
    np.testing.assert_allclose(c, z["centers"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(inertia, float(z["inertia"][0]), rtol=1e-5)


def _blobs(seed, n, d, k, spread=1.0, dtype=np.float64):
    rng = np.random.default_rng(seed)
    centres = rng.uniform(-6, 6, size=(k, d))
    lab = rng.integers(0, k, n)
    return (centres[lab] + spread * rng.standard_normal((n, d))).astype(dtype)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("case", [(1, 2000, 3, 6), (2, 1500, 8, 12), (3, 900, 2, 4)])
def test_lloyd_against_sklearn(dtype, case):
    from sklearn.cluster import KMeans as SK
    seed, n, d, k = case
    X = _blobs(seed, n, d, k, spread=2.5, dtype=dtype)
    init = X[np.random.default_rng(seed + 9).choice(n, k, replace=False)]
    c, l, inertia, it = oracle.kmeans_fit(X, k, "array", init, max_iter=300, tol=1e-4)
    sk = SK(n_clusters=k, init=init, n_init=1, max_iter=300, tol=1e-4, algorithm="lloyd").fit(X)
    assert it > 2                      # a real multi-iteration loop
    np.testing.assert_array_equal(l, sk.labels_.astype(np.uint32))
    # sklearn counts the assignment that precedes the first update as an
    # iteration; the reference's loop (update, then assign) does not, so a
    # strict-convergence stop reads one less here (single_run :965-1127)
    assert it in (sk.n_iter_, sk.n_iter_ - 1)
    tol = 1e-10 if dtype == np.float64 else 1e-4
    np.testing.assert_allclose(c, sk.cluster_centers_, rtol=tol, atol=tol)
    np.testing.assert_allclose(inertia, sk.inertia_, rtol=tol)


def test_empty_cluster_relocation_against_sklearn():
    from sklearn.cluster import KMeans as SK
    X = _blobs(5, 800, 3, 3, spread=0.8)
    init = np.array([X[0], X[1], [500.0, 500.0, 500.0], [-400.0, 0.0, 0.0]])   # two centres nobody picks
    c, l, inertia, it = oracle.kmeans_fit(X, 4, "array", init)
    sk = SK(n_clusters=4, init=init, n_init=1, algorithm="lloyd").fit(X)
    np.testing.assert_array_equal(l, sk.labels_.astype(np.uint32))
    np.testing.assert_allclose(c, sk.cluster_centers_, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(inertia, sk.inertia_, rtol=1e-10)
    assert len(set(l.tolist())) == 4


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_feature_mean_var(dtype):
    X = _blobs(7, 3000, 5, 3, dtype=dtype)
    want = X.astype(np.float64).var(axis=0).mean()
    np.testing.assert_allclose(oracle.feature_mean_var(X), want, rtol=1e-12 if dtype == np.float64 else 1e-6)


def _below(stream, bound):
    zone = (2 ** 64 - 1) - ((2 ** 64 - 1) % bound)
    for v in stream:
        if v < zone:
            return v % bound
    raise AssertionError("stream exhausted")


def test_random_init_is_a_partial_fisher_yates():
    X = _blobs(8, 500, 2, 3)
    for seed in (0, 3, 99):
        got = oracle.kmeans_init(X, 7, "random", seed=seed)
        stream = iter(int(v) for v in oracle.splitmix64(seed, 64))
        ids = list(range(500))
        for i in range(7):
            j = i + _below(stream, 500 - i)
            ids[i], ids[j] = ids[j], ids[i]
        assert got.tolist() == ids[:7]


def test_kmeanspp_first_pick_and_d2_weighting():
    # eight tight, far-apart clusters: D^2 weighting puts every later pick in
    # a cluster not yet chosen
    rng = np.random.default_rng(11)
    centres = rng.uniform(-50, 50, size=(8, 4))
    lab = rng.integers(0, 8, 4000)
    X = centres[lab] + 0.01 * rng.standard_normal((4000, 4))
    for seed in (0, 1, 2, 7):
        got = oracle.kmeans_init(X, 8, "k-means++", seed=seed)
        assert got[0] == _below(iter(int(v) for v in oracle.splitmix64(seed, 8)), 4000)
        assert len(set(lab[got].tolist())) == 8


def test_restarts_keep_the_lowest_inertia():
    X = _blobs(12, 1200, 2, 6, spread=1.5)
    runs = [oracle.kmeans_fit(X, 6, "random", seed=100 + r, n_init=1) for r in range(5)]
    c, l, inertia, it = oracle.kmeans_fit(X, 6, "random", seed=100, n_init=5)
    best = min(r[2] for r in runs)
    assert inertia == best
    winner = [r for r in runs if r[2] == best][0]
    np.testing.assert_array_equal(c, winner[0])


def test_relocation_ranks_a_nan_distance_first():
    """A NaN row (distance NaN to its centre) during the empty-cluster
    relocation: the ranking is a total order with NaN above every number, so
    the NaN row moves first (its new centre is NaN) and the farthest finite
    row next (its new centre is that row)."""
    X = _blobs(7, 600, 3, 3, spread=0.8)
    X[37] = np.nan
    init = np.array([X[0], X[1], [500.0, 500.0, 500.0], [-400.0, 0.0, 0.0]])
    first = oracle.kmeans_fit(X, 4, "array", init, max_iter=1)
    again = oracle.kmeans_fit(X, 4, "array", init, max_iter=1)
    np.testing.assert_array_equal(first[0], again[0])
    np.testing.assert_array_equal(first[1], again[1])
    c = first[0]
    assert np.isnan(c[2]).all()
    _, dist = oracle.kmeans_assign(X, init)
    far = int(np.nanargmax(np.where(np.isnan(dist), -np.inf, dist)))
    np.testing.assert_array_equal(c[3], X[far])
