"""GPU parity of the device k-means fit (mlrs_kmeans_fit_*) against the CPU
oracle's restatement of the reference's KMeans::fit, bit for bit: centres,
labels, inertia and iteration count, for explicit, k-means++ and random
initialisation, restarts, empty-cluster relocation, both assignment kernel
families, both centroid-sum bucket paths (labels below and above the LDS
histogram) and both algorithms ('lloyd', and 'elkan': the bound-pruned
assignment, which must return the same bits; it serves k <= 4096 with finite
rows); and the estimator against the reference's fixtures.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import load_golden
from mlrs_amd import _lib, prims
from mlrs_amd.cluster import KMeans

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _blobs(seed, n, d, k, spread=1.0, dtype=np.float64):
    rng = np.random.default_rng(seed)
    centres = rng.uniform(-6, 6, size=(k, d))
    lab = rng.integers(0, k, n)
    return (centres[lab] + spread * rng.standard_normal((n, d))).astype(dtype)


def _same(got, want):
    gc, gl, gi, gn = got
    wc, wl, wi, wn = want
    np.testing.assert_array_equal(gl.cpu().numpy(), wl.astype(np.int64))
    np.testing.assert_array_equal(gc.cpu().numpy(), wc)
    assert gi == wi
    assert gn == wn


@pytest.fixture(params=["auto", "generic"])
def family(request):
    prims.force_path(request.param)
    yield request.param
    prims.force_path("auto")


@pytest.fixture(params=["lloyd", "elkan"])
def algorithm(request):
    return request.param


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("init", ["array", "k-means++", "random"])
@pytest.mark.parametrize("case", [(1, 3000, 5, 7, 1), (2, 20000, 16, 40, 2), (3, 5000, 3, 300, 1)])
def test_fit_matches_oracle(family, algorithm, dtype, init, case):
    seed, n, d, k, n_init = case
    X = _blobs(seed, n, d, max(2, k // 3), spread=2.0, dtype=dtype)
    ini = X[np.random.default_rng(seed).choice(n, k, replace=False)] if init == "array" else None
    want = oracle.kmeans_fit(X, k, init, ini, seed=seed, n_init=n_init, max_iter=60, tol=1e-4)
    got = prims.kmeans_fit(_t(X), k, init, _t(ini) if ini is not None else None, seed=seed, n_init=n_init,
                           max_iter=60, tol=1e-4, algorithm=algorithm)
    _same(got, want)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_fit_many_labels_global_buckets(algorithm, dtype):
    """k above the LDS label histogram: the global-memory bucket path."""
    X = _blobs(4, 40000, 2, 50, spread=3.0, dtype=dtype)
    ini = X[np.random.default_rng(4).choice(40000, 9000, replace=False)]
    want = oracle.kmeans_fit(X, 9000, "array", ini, max_iter=4, tol=0.0)
    got = prims.kmeans_fit(_t(X), 9000, "array", _t(ini), max_iter=4, tol=0.0, algorithm=algorithm)
    _same(got, want)


def test_fit_relocates_empty_clusters(algorithm):
    X = _blobs(5, 2000, 3, 3, spread=0.8)
    ini = np.array([X[0], X[1], [500.0, 500.0, 500.0], [-400.0, 0.0, 0.0]])
    want = oracle.kmeans_fit(X, 4, "array", ini)
    got = prims.kmeans_fit(_t(X), 4, "array", _t(ini), algorithm=algorithm)
    _same(got, want)
    assert len(set(got[1].cpu().tolist())) == 4


def test_fit_relocation_walks_past_the_selected_prefix(algorithm):
    """The farthest rows all sit alone in their clusters (100 outliers, each
    50 from its own centre), so the relocation walk skips every row of the
    selected top 8 * empties + 64 and ranks the rest before it finds donors."""
    X = _blobs(6, 2000, 3, 3, spread=0.8)
    outliers = np.zeros((100, 3))
    outliers[:, 0] = 1000.0 * np.arange(1, 101)
    X = np.concatenate([X, outliers])
    far = outliers.copy()
    far[:, 0] += 50.0
    ini = np.concatenate([X[[0, 1, 2]], far, [[-5000.0, 0.0, 0.0], [0.0, -5000.0, 0.0]]])
    want = oracle.kmeans_fit(X, ini.shape[0], "array", ini, max_iter=3, tol=0.0)
    got = prims.kmeans_fit(_t(X), ini.shape[0], "array", _t(ini), max_iter=3, tol=0.0, algorithm=algorithm)
    _same(got, want)
    assert len(set(got[1].cpu().tolist())) == ini.shape[0]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_fit_relocation_ranked_in_chunks_with_ties(algorithm, dtype):
    """60,000 rows on an integer grid (many equal distances, spread over the
    device ranking's chunks of 8,192 keys) and 40 empty clusters: the top
    8 * 40 + 64 rows by (distance desc, index asc) come from the two-stage
    device selection, and the fit matches the oracle's bits."""
    rng = np.random.default_rng(9)
    X = rng.integers(0, 10, size=(60000, 3)).astype(dtype)
    far = np.zeros((40, 3), dtype=dtype)
    far[:, 0] = 1000.0 + 10.0 * np.arange(40)
    ini = np.concatenate([X[:6], far])
    want = oracle.kmeans_fit(X, ini.shape[0], "array", ini, max_iter=2, tol=0.0)
    got = prims.kmeans_fit(_t(X), ini.shape[0], "array", _t(ini), max_iter=2, tol=0.0, algorithm=algorithm)
    _same(got, want)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_fit_relocation_with_a_nan_distance(algorithm, dtype):
    """A NaN row reaches the relocation ranking (the C ABI does not check
    finiteness, as the reference's Rust fit does not): the ranking is a total
    order, NaN first, and the fit matches the oracle's bits."""
    X = _blobs(7, 600, 3, 3, spread=0.8, dtype=dtype)
    X[37] = np.nan
    ini = np.array([X[0], X[1], [500.0, 500.0, 500.0], [-400.0, 0.0, 0.0]], dtype=dtype)
    wc, wl, wi, wn = oracle.kmeans_fit(X, 4, "array", ini, max_iter=1)
    gc, gl, gi, gn = prims.kmeans_fit(_t(X), 4, "array", _t(ini), max_iter=1, algorithm=algorithm)
    np.testing.assert_array_equal(gl.cpu().numpy(), wl.astype(np.int64))
    np.testing.assert_array_equal(gc.cpu().numpy(), wc)
    assert (gi == wi) or (np.isnan(gi) and np.isnan(wi))
    assert gn == wn
    assert np.isnan(gc.cpu().numpy()[2]).all()


@pytest.mark.parametrize("s", ["f32", "f64"])
def test_estimator_fixture(s):
    z = load_golden("kmeans_%s_seed42" % s)
    km = KMeans(n_clusters=z["init"].shape[0], init=z["init"], n_init=1).fit(z["X"])
    np.testing.assert_array_equal(km.labels_, z["labels"].astype(np.int32))
    np.testing.assert_allclose(km.cluster_centers_, z["centers"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(km.inertia_, z["inertia"][0], rtol=1e-5)
    np.testing.assert_array_equal(km.predict(z["X"]), km.labels_)


def test_estimator_defaults_and_errors():
    X = _blobs(6, 4000, 4, 5, spread=1.0, dtype=np.float32)
    km = KMeans(n_clusters=5, random_state=3).fit(X)
    c, l, inertia, it = oracle.kmeans_fit(X, 5, "k-means++", seed=3, n_init=1)
    np.testing.assert_array_equal(km.labels_, l.astype(np.int32))
    np.testing.assert_array_equal(km.cluster_centers_, c)
    assert km.n_iter_ == it and km._n_init == 1
    assert KMeans(n_clusters=5, init="random").fit(X)._n_init == 10
    with pytest.raises(_lib.InvalidParam):
        KMeans(n_clusters=5000).fit(X[:100])


def _split_blobs(seed, n, d, comps, dtype):
    """Well separated blobs (centres 40 apart on average), so that most rows
    are settled by the bounds once the centres stop moving much."""
    rng = np.random.default_rng(seed)
    centres = rng.normal(0.0, 5.0, size=(comps, d))
    lab = rng.integers(0, comps, n)
    return (centres[lab] + rng.standard_normal((n, d))).astype(dtype)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", [(120000, 16, 200, 160), (60000, 64, 512, 400), (30000, 5, 64, 20)])
def test_elkan_equals_lloyd_and_oracle(family, dtype, shape):
    """Random init draws some blobs twice and leaves others empty, so rows are
    settled by the half-distance test, by their own tightened distance, by a
    short candidate list, or by the fused search of the rows left; both
    algorithms must give the oracle's bits after 25 iterations."""
    n, d, k, comps = shape
    X = _split_blobs(n + d, n, d, comps, dtype)
    want = oracle.kmeans_fit(X, k, "random", seed=5, max_iter=25, tol=0.0)
    for algo in ("lloyd", "elkan"):
        got = prims.kmeans_fit(_t(X), k, "random", seed=5, max_iter=25, tol=0.0, algorithm=algo)
        _same(got, want)


def test_elkan_estimator_and_tie_breaks():
    """Duplicate rows and centres on an integer grid (exact ties between
    centre distances): the lowest centre index wins under both algorithms."""
    rng = np.random.default_rng(12)
    X = rng.integers(-3, 4, size=(20000, 4)).astype(np.float32)
    ini = np.concatenate([X[:40], X[:8]])   # eight centres twice
    want = oracle.kmeans_fit(X, ini.shape[0], "array", ini, max_iter=12, tol=0.0)
    got = prims.kmeans_fit(_t(X), ini.shape[0], "array", _t(ini), max_iter=12, tol=0.0, algorithm="elkan")
    _same(got, want)
    km = KMeans(n_clusters=8, random_state=2, algorithm="elkan").fit(X)
    ref = KMeans(n_clusters=8, random_state=2, algorithm="lloyd").fit(X)
    np.testing.assert_array_equal(km.labels_, ref.labels_)
    np.testing.assert_array_equal(km.cluster_centers_, ref.cluster_centers_)
    assert km.inertia_ == ref.inertia_ and km.n_iter_ == ref.n_iter_ and km._algorithm == "elkan"
