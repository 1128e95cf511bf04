"""GPU parity of radius_neighbors (mlrs_radius_neighbors_*) against the CPU
oracle's radius scan, and the estimator surface against the reference's
sklearn fixtures.

Counts and indices are compared exactly.  Values are compared bit for bit
except where a pow is involved (the Minkowski pow lane loop and every
Minkowski root), whose last bit the device's and the host's C library may
round differently: those are held to 4 ulp, and their radii sit at the
midpoint of a gap in the oracle's values so membership does not hinge on
that bit.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from conftest import load_golden
from mlrs_amd import _lib, prims
from mlrs_amd.neighbors import NearestNeighbors

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _radius(vals, frac, rel=None):
    """The `frac` quantile of the values; with `rel`, the midpoint of the first
    gap of relative width > rel at or after it (a radius no value sits near)."""
    v = np.sort(vals[np.isfinite(vals)].astype(np.float64).ravel())
    start = min(int(v.size * frac), v.size - 2)
    if rel is None:
        return float(v[start])
    for i in range(start, v.size - 1):
        if v[i + 1] > v[i] * (1.0 + rel):
            return 0.5 * (v[i] + v[i + 1])
    return v[-1] * 1.5


def _compare(xq, xt, radius, metric, p=2.0):
    wd, wi, wc = oracle.radius_neighbors(xq, xt, radius, metric, p=p)
    gd, gi, gc = prims.radius_neighbors(_t(xq), _t(xt), radius, metric, p=p)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(gc.cpu().numpy(), wc.astype(np.int64))
    np.testing.assert_array_equal(gi.cpu().numpy(), wi)
    gd = gd.cpu().numpy()
    if metric == "minkowski":
        np.testing.assert_allclose(gd, wd, rtol=4 * np.finfo(xq.dtype).eps, atol=0)
    else:
        np.testing.assert_array_equal(gd, wd)
    return wc


CASES = [("euclidean", 2.0), ("cosine", 2.0), ("manhattan", 2.0), ("chebyshev", 2.0), ("minkowski", 3.0),
         ("minkowski", 2.5)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("metric,p", CASES)
@pytest.mark.parametrize("shape", [(70, 3000, 8), (33, 5000, 7), (5, 900, 6), (130, 2500, 65)])
def test_radius_matches_oracle(dtype, metric, p, shape):
    nq, nt, d = shape
    rng = np.random.default_rng(nq * 7 + d)
    xt = rng.standard_normal((nt, d)).astype(dtype)
    xq = rng.standard_normal((nq, d)).astype(dtype)
    xt[17] = xt[3]
    xq[0] = xt[3]
    # radii from the value distribution: sparse and half; exact quantiles (a
    # pair sits on the threshold) where the values are bitwise, a gap
    # midpoint where a pow may move the last bit
    dist_all = oracle.pairwise(xq, xt, metric, sqrt=True, p=p)
    rel = (1e-5 if dtype == np.float32 else 1e-11) if metric == "minkowski" else None
    for frac in (0.02, 0.5):
        wc = _compare(xq, xt, _radius(dist_all, frac, rel), metric, p)
        assert wc.sum() > 0
    if metric != "minkowski":
        _compare(xq, xt, 0.0, metric, p)
        _compare(xq, xt, float(np.inf), metric, p)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_radius_many_strips_and_partial_groups(dtype):
    """Enough index rows for many strips per query group, a query count that
    leaves the last group partial, and an unaligned feature count."""
    rng = np.random.default_rng(11)
    xt = rng.standard_normal((60000, 5)).astype(dtype)
    xq = rng.standard_normal((45, 5)).astype(dtype)
    radius = _radius(oracle.pairwise(xq[:5], xt[:4000], "euclidean", sqrt=True), 0.05)
    wc = _compare(xq, xt, radius, "euclidean")
    assert wc.min() > 10


def test_radius_nan_rows_and_coincident_points():
    rng = np.random.default_rng(3)
    xt = rng.standard_normal((3000, 4)).astype(np.float32)
    xq = rng.standard_normal((40, 4)).astype(np.float32)
    xt[7] = xq[2]
    xt[2900] = xq[2]
    xt[11, 1] = np.nan
    xq[5, 0] = np.nan
    for metric in ("euclidean", "manhattan", "chebyshev", "cosine"):
        wc = _compare(xq, xt, 0.0, metric)
        if metric != "cosine":
            assert wc[2] == 2
        _compare(xq, xt, 1.0 if metric != "cosine" else 0.3, metric)
        _compare(xq, xt, float(np.inf), metric)


@pytest.fixture
def matrix_core_path():
    """Route f32 Euclidean / cosine radius scans to the matrix-core screen
    (knn_radius_gram.hip) whatever their size."""
    prims.force_path("fused")
    yield
    prims.force_path("auto")


@pytest.mark.parametrize("metric", ["euclidean", "cosine"])
@pytest.mark.parametrize("shape", [(70, 3000, 8), (130, 2500, 65), (300, 5000, 128), (129, 4000, 33),
                                   (5, 900, 6), (257, 20000, 100), (1, 40, 17)])
def test_radius_matrix_core_screen(matrix_core_path, metric, shape):
    nq, nt, d = shape
    rng = np.random.default_rng(nq * 5 + d)
    xt = rng.standard_normal((nt, d)).astype(np.float32)
    xq = rng.standard_normal((nq, d)).astype(np.float32)
    xt[17 % nt] = xt[3 % nt]
    xq[0] = xt[3 % nt]
    dist_all = oracle.pairwise(xq, xt, metric, sqrt=True)
    for frac in (0.001, 0.02, 0.5):
        _compare(xq, xt, _radius(dist_all, frac), metric)
    _compare(xq, xt, 0.0, metric)
    _compare(xq, xt, float(np.inf), metric)


def test_radius_matrix_core_dense_matches_and_specials(matrix_core_path):
    """Clustered rows (hundreds of matches per query, so queues flush many
    times per strip), NaN and zero rows, duplicates of the queries, and a
    query set whose norms overflow the screen (every pair evaluated)."""
    rng = np.random.default_rng(21)
    centres = rng.uniform(-4, 4, size=(6, 48)).astype(np.float32)
    xt = (centres[rng.integers(0, 6, 30000)] + 0.5 * rng.standard_normal((30000, 48))).astype(np.float32)
    xq = (centres[rng.integers(0, 6, 200)] + 0.5 * rng.standard_normal((200, 48))).astype(np.float32)
    xt[[5, 70, 29999]] = np.nan
    xt[[6, 71]] = 0.0
    xt[1000:1040] = xq[3]
    xq[9] = np.nan
    xq[10] = 0.0
    for metric in ("euclidean", "cosine"):
        dist_all = oracle.pairwise(xq[:20], xt, metric, sqrt=True)
        for frac in (0.05, 0.2):
            wc = _compare(xq, xt, _radius(dist_all, frac), metric)
            assert wc.max() > 500
    big = xq * np.float32(1e19)
    _compare(big, xt * np.float32(1e19), 1e20, "euclidean")


def test_radius_empty_index_and_no_matches():
    xq = np.ones((10, 3), np.float32)
    d, i, c = prims.radius_neighbors(_t(xq), _t(np.zeros((0, 3), np.float32)), 1.0)
    assert c.cpu().tolist() == [0] * 10 and i.numel() == 0 and d.numel() == 0
    d, i, c = prims.radius_neighbors(_t(xq), _t(np.full((50, 3), 9.0, np.float32)), 1.0)
    assert c.sum().item() == 0 and i.numel() == 0


def _raw_call(xq, xt, radius, counts, out_d, out_i, cap):
    total = ctypes.c_int64(-1)
    f = _lib.load().mlrs_radius_neighbors_f32
    rc = f(xq.data_ptr(), xq.numel(), xq.shape[0], xq.shape[1], xt.data_ptr(), xt.numel(), xt.shape[0],
           xt.shape[1], 0, 2.0, float(radius), counts.data_ptr(), counts.numel(),
           out_d.data_ptr() if out_d is not None else None, out_i.data_ptr() if out_i is not None else None,
           cap, ctypes.byref(total), torch.cuda.current_stream().cuda_stream)
    return rc, total.value


@pytest.mark.parametrize("path", ["auto", "fused"])
def test_radius_capacity_and_changed_data_between_calls(path):
    """A short buffer is refused with the needed size; a fill call after the
    data changed under the same pointers counts again and stays exact."""
    prims.force_path(path)
    try:
        _capacity_and_changed_data()
    finally:
        prims.force_path("auto")


def _capacity_and_changed_data():
    rng = np.random.default_rng(5)
    xt_np = rng.standard_normal((4000, 6)).astype(np.float32)
    xq_np = rng.standard_normal((50, 6)).astype(np.float32)
    xq, xt = _t(xq_np), _t(xt_np)
    counts = torch.empty(50, dtype=torch.int32, device=DEV)
    rc, total = _raw_call(xq, xt, 1.5, counts, None, None, 0)
    assert rc == 0 and total > 0
    small_d = torch.empty(total - 1, dtype=torch.float32, device=DEV)
    small_i = torch.empty(total - 1, dtype=torch.int32, device=DEV)
    rc, total2 = _raw_call(xq, xt, 1.5, counts, small_d, small_i, total - 1)
    assert rc == _lib.MLRS_ERR_SHAPE_MISMATCH and total2 == total
    e = _lib.ErrorInfo()
    _lib.load().mlrs_last_error(ctypes.byref(e))
    assert e.operand == b"out" and e.rows == total and e.len == total - 1
    # change the index rows in place: the kept counts no longer hold
    xt_np2 = xt_np * np.float32(0.9)
    xt.copy_(_t(xt_np2))
    wd, wi, wc = oracle.radius_neighbors(xq_np, xt_np2, 1.5)
    out_d = torch.empty(max(total, wi.size) + 5, dtype=torch.float32, device=DEV)
    out_i = torch.empty_like(out_d, dtype=torch.int32)
    rc, total3 = _raw_call(xq, xt, 1.5, counts, out_d, out_i, out_d.numel())
    assert rc == 0 and total3 == wi.size
    np.testing.assert_array_equal(counts.cpu().numpy(), wc.astype(np.int32))
    np.testing.assert_array_equal(out_i[:total3].cpu().numpy(), wi)
    np.testing.assert_array_equal(out_d[:total3].cpu().numpy(), wd)


def test_radius_prim_errors():
    xq = _t(np.zeros((4, 3), np.float32))
    with pytest.raises(_lib.InvalidParam):
        prims.radius_neighbors(xq, xq, -1.0)
    with pytest.raises(_lib.DimMismatch):
        prims.radius_neighbors(xq, _t(np.zeros((4, 2), np.float32)), 1.0)


# ---- estimator surface against the sklearn fixtures ------------------------

@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("metric", ["euclidean", "manhattan", "chebyshev", "minkowski", "cosine"])
def test_estimator_radius_fixture(s, metric):
    z = load_golden("nn_radius_%s_seed42" % s)
    nn = NearestNeighbors(metric=metric, p=3.0 if metric == "minkowski" else 2).fit(z["X"])
    dist, ind = nn.radius_neighbors(z["Xq"], radius=float(z["radius_" + metric][0]))
    counts = np.array([len(a) for a in ind])
    np.testing.assert_array_equal(counts, z["radius_counts_" + metric].astype(np.int64))
    np.testing.assert_array_equal(np.concatenate(ind), z["radius_indices_" + metric].astype(np.int32))
    np.testing.assert_allclose(np.concatenate(dist), z["radius_distances_" + metric], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("alias", ["l2", "l1", "cityblock", "infinity", "minkowski"])
def test_estimator_radius_alias_fixture(s, alias):
    z = load_golden("nn_radius_%s_seed42" % s)
    nn = NearestNeighbors(metric=alias).fit(z["X"])
    dist, ind = nn.radius_neighbors(z["Xq"], radius=float(z["radius_alias_r_" + alias][0]))
    np.testing.assert_array_equal(np.concatenate(ind), z["radius_alias_indices_" + alias].astype(np.int32))
    np.testing.assert_allclose(np.concatenate(dist), z["radius_alias_distances_" + alias], rtol=1e-5, atol=1e-5)


def test_estimator_radius_graph_self_drop_and_sorting():
    rng = np.random.default_rng(9)
    X = rng.standard_normal((300, 5)).astype(np.float32)
    X[10] = X[20]                                    # a duplicate: stays after the self drop
    nn = NearestNeighbors(radius=1.2).fit(X)
    dist, ind = nn.radius_neighbors()                # X=None: the training set, own index dropped
    wd, wi, wc = oracle.radius_neighbors(X, X, 1.2)
    off = np.concatenate([[0], np.cumsum(wc.astype(np.int64))])
    for r in range(300):
        keep = wi[off[r]:off[r + 1]] != r
        np.testing.assert_array_equal(ind[r], wi[off[r]:off[r + 1]][keep])
        np.testing.assert_array_equal(dist[r], wd[off[r]:off[r + 1]][keep])
    assert 20 in ind[10].tolist() and 10 not in ind[10].tolist()
    sd, si = nn.radius_neighbors(X[:7], sort_results=True)
    for r in range(7):
        assert np.all(np.diff(sd[r]) >= 0)
        assert sorted(si[r].tolist()) == sorted(nn.radius_neighbors(X[:7])[1][r].tolist())
    g = nn.radius_neighbors_graph(X[:9], mode="distance")
    assert g.shape == (9, 300)
    d9, i9 = nn.radius_neighbors(X[:9])
    for r in range(9):
        row = g.getrow(r)
        np.testing.assert_array_equal(row.indices, i9[r])
        np.testing.assert_allclose(row.data, d9[r].astype(np.float64))
    kg = nn.kneighbors_graph(X[:4], n_neighbors=3, mode="connectivity")
    _, ki = nn.kneighbors(X[:4], 3)
    assert kg.nnz == 12 and all(sorted(kg.getrow(r).indices) == sorted(ki[r]) for r in range(4))
    with pytest.raises(ValueError, match="return_distance must be True"):
        nn.radius_neighbors(X[:2], return_distance=False, sort_results=True)
    with pytest.raises(ValueError, match="radius must be non-negative"):
        nn.radius_neighbors(X[:2], radius=-1)


def _one_call(xq_np, xt_np, radius, cap, metric_id=0):
    """One call with output buffers of `cap` entries (no counting call before
    it): the matrix-core path counts and stages the matches in one pass."""
    xq, xt = _t(xq_np), _t(xt_np)
    counts = torch.empty(xq_np.shape[0], dtype=torch.int32, device=DEV)
    out_d = torch.empty(max(cap, 1), dtype=torch.float32, device=DEV)
    out_i = torch.empty(max(cap, 1), dtype=torch.int32, device=DEV)
    total = ctypes.c_int64(-1)
    f = _lib.load().mlrs_radius_neighbors_f32
    rc = f(xq.data_ptr(), xq.numel(), xq.shape[0], xq.shape[1], xt.data_ptr(), xt.numel(), xt.shape[0],
           xt.shape[1], metric_id, 2.0, float(radius), counts.data_ptr(), counts.numel(), out_d.data_ptr(),
           out_i.data_ptr(), cap, ctypes.byref(total), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    n = max(total.value, 0)
    return rc, total.value, counts.cpu().numpy(), out_d[:n].cpu().numpy(), out_i[:n].cpu().numpy()


@pytest.mark.parametrize("metric,mid", [("euclidean", 0), ("cosine", 1)])
def test_radius_staged_single_call(matrix_core_path, metric, mid):
    """A call that brings large enough buffers is served by the staged count
    pass alone (matches kept per strip, then copied into place), and a strip
    holding more matches than the staging keeps (1,024 per strip and row;
    here 3,000 rows near query 0 over strips of 1,600 rows) falls back to the
    fill pass: both exact."""
    rng = np.random.default_rng(77)
    xt = rng.standard_normal((50000, 20)).astype(np.float32)
    xq = rng.standard_normal((8192, 20)).astype(np.float32)
    dist_all = oracle.pairwise(xq[:40], xt, metric, sqrt=True)
    r = _radius(dist_all, 0.002, rel=1e-4)
    wd, wi, wc = oracle.radius_neighbors(xq, xt, r, metric)
    rc, n, c, d, i = _one_call(xq, xt, r, wi.size + 100, mid)
    assert rc == 0 and n == wi.size
    np.testing.assert_array_equal(c, wc.astype(np.int32))
    np.testing.assert_array_equal(i, wi)
    np.testing.assert_array_equal(d, wd)
    # overflowing staging: a dense cluster around query 0
    xt2 = xt.copy()
    xt2[:3000] = xq[0] + np.float32(1e-3) * rng.standard_normal((3000, 20)).astype(np.float32)
    r2 = 0.2 if metric == "euclidean" else 1e-4
    wd, wi, wc = oracle.radius_neighbors(xq, xt2, r2, metric)
    assert wc[0] >= 2900
    rc, n, c, d, i = _one_call(xq, xt2, r2, wi.size, mid)
    assert rc == 0 and n == wi.size
    np.testing.assert_array_equal(c, wc.astype(np.int32))
    np.testing.assert_array_equal(i, wi)
    np.testing.assert_array_equal(d, wd)
    # buffers too small: the total comes back, nothing is written
    rc, n, c, d, i = _one_call(xq, xt2, r2, wi.size - 1, mid)
    assert rc == _lib.MLRS_ERR_SHAPE_MISMATCH and n == wi.size
    # NaN and zero rows on both sides, duplicates of a query, through staging
    xt3 = xt.copy()
    xq3 = xq.copy()
    xt3[[11, 4000, 49999]] = np.nan
    xt3[[12, 4001]] = 0.0
    xt3[100:140] = xq3[5]
    xq3[7] = np.nan
    xq3[8] = 0.0
    wd, wi, wc = oracle.radius_neighbors(xq3, xt3, r, metric)
    rc, n, c, d, i = _one_call(xq3, xt3, r, wi.size + 7, mid)
    assert rc == 0 and n == wi.size
    np.testing.assert_array_equal(c, wc.astype(np.int32))
    np.testing.assert_array_equal(i, wi)
    np.testing.assert_array_equal(d, wd)


def test_radius_repeated_search_uses_size_hint(matrix_core_path):
    """The Python wrapper sizes a repeated search's buffers from the previous
    total: the second search of a shape takes the one-call path, and a later
    search of the same shape with more matches than the hint allows still
    comes back exact (the call reports the total, then counts are reused)."""
    rng = np.random.default_rng(78)
    xt = rng.standard_normal((20000, 40)).astype(np.float32)
    xq = rng.standard_normal((300, 40)).astype(np.float32)
    r = _radius(oracle.pairwise(xq[:20], xt, "euclidean", sqrt=True), 0.01, rel=1e-4)
    for _ in range(2):
        _compare(xq, xt, r, "euclidean")
    xt_dense = xt.copy()
    xt_dense[:15000] = xq[rng.integers(0, 300, 15000)] + np.float32(0.01)
    wc = _compare(xq, xt_dense, r, "euclidean")
    assert wc.sum() > 15000
    _compare(xq, xt, r, "euclidean")
