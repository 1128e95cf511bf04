"""Pins the CPU oracle (oracle/ref_cpu.c) -- CPU only.

How each oracle function is pinned:

* knn_topk     -- the reference's sklearn fixtures (knn_*_seed42, nn_params_*,
                  knn_{euclidean,cosine}_*), an independent exact-arithmetic
                  model of every arm (below) compared BIT FOR BIT, the
                  known-answer invariants of the reference tests
                  (all-duplicates -> 0..k, ascending order, NaN rows, ties),
                  and sklearn brute force on random data.
* kmeans_assign-- kmeans_* fixture labels/inertia, the exact model, a planted
                  tie, sklearn KMeans.predict.
* pairwise     -- dist_sq_* / dist_sqrt_f64 fixtures, the exact model.
* row_sqnorms  -- the exact model.

The exact model uses numpy scalar float32/float64 arithmetic for +, -, *, /
and sqrt (each an IEEE correctly rounded operation) and rational arithmetic
for the fused multiply-add (one rounding of the exact a*b+c), so it is an
independent restatement of the reference's operation order, not a copy of
the C code.
"""
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle
from conftest import ROOT, assert_topk_matches, load_golden


# ---------------------------------------------------------------------------
# exact arithmetic model
# ---------------------------------------------------------------------------
def _rne(q, dt):
    """Round the rational q to the nearest dt value, ties to even."""
    if dt == np.float64:
        return np.float64(float(q))  # float(Fraction) is correctly rounded
    c = np.float32(float(q))
    cands = [np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))]
    best = None
    for v in cands:
        err = abs(Fraction(float(v)) - q)
        even = (np.array(v, dtype=np.float32).view(np.uint32) & 1) == 0
        key = (err, 0 if even else 1)
        if best is None or key < best[0]:
            best = (key, v)
    return np.float32(best[1])


def _fma(a, b, c):
    dt = type(a)
    return _rne(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)), dt)


def _sumsq(row):
    T = row.dtype.type
    acc = T(0)
    for v in row:
        acc = T(acc + T(v * v))
    return acc


def _inv(s):
    T = type(s)
    return T(T(1) / np.sqrt(s)) if s > 0 else T(0)


def _clamp02(v):
    T = type(v)
    v = T(0) if v < 0 else v
    v = T(2) if v > 2 else v
    return v


def model_pair(q, y, arm, qa=None, ya=None):
    T = q.dtype.type
    if arm in ("euclid_fma", "euclid_muladd"):
        acc = T(0)
        for a, b in zip(q, y):
            diff = T(a - b)
            acc = _fma(diff, diff, acc) if arm == "euclid_fma" else T(acc + T(diff * diff))
        return acc
    if arm == "cos_fold":
        dot = T(0)
        for a, b in zip(q, y):
            dot = _fma(a, b, dot)
        denom = np.sqrt(T(qa * ya))
        sim = T(dot / denom) if denom > 0 else T(0)
        return _clamp02(T(T(1) - sim))
    if arm == "cos_host":
        dot = T(0)
        for a, b in zip(q, y):
            dot = T(dot + T(a * b))
        return _clamp02(T(T(1) - T(T(dot * qa) * ya)))
    raise ValueError(arm)


def model_arm(d, k, metric):
    metric_family = 1 <= d <= 128 and 1 <= k <= 128
    if metric == "euclidean":
        return "euclid_fma" if metric_family else "euclid_muladd"
    return "cos_fold" if metric_family else "cos_host"


def model_knn(xq, xt, k, metric):
    T = xq.dtype.type
    arm = model_arm(xq.shape[1], k, metric)
    if arm == "cos_fold":
        qa = [_sumsq(r) for r in xq]
        ya = [_sumsq(r) for r in xt]
    elif arm == "cos_host":
        qa = [_inv(_sumsq(r)) for r in xq]
        ya = [_inv(_sumsq(r)) for r in xt]
    else:
        qa = [None] * len(xq)
        ya = [None] * len(xt)
    dist = np.empty((len(xq), k), dtype=xq.dtype)
    idx = np.empty((len(xq), k), dtype=np.uint32)
    for i, q in enumerate(xq):
        vals = [(model_pair(q, y, arm, qa[i], ya[t]), t) for t, y in enumerate(xt)]
        vals = [(v, t) for v, t in vals if not np.isnan(v)]
        vals.sort(key=lambda p: (float(p[0]), p[1]))
        vals = vals[:k] + [(T(np.inf), 0)] * max(0, k - len(vals))
        for j, (v, t) in enumerate(vals):
            dist[i, j] = np.sqrt(v) if metric == "euclidean" else v
            idx[i, j] = t
    return dist, idx


def model_kmeans(x, c):
    labels = np.empty(len(x), dtype=np.uint32)
    best_d = np.empty(len(x), dtype=x.dtype)
    for i, r in enumerate(x):
        best, bc = None, 0
        for j, cr in enumerate(c):
            v = model_pair(r, cr, "euclid_muladd")
            if j == 0:
                best = v
            elif v < best:
                best, bc = v, j
        labels[i], best_d[i] = bc, best
    return labels, best_d


def _data(seed, nq, nt, d, dtype, scale=1.0):
    rng = np.random.default_rng(seed)
    return ((rng.standard_normal((nq, d)) * scale).astype(dtype),
            (rng.standard_normal((nt, d)) * scale).astype(dtype))


# ---------------------------------------------------------------------------
# exact model vs the C oracle, every arm of the dispatch
# ---------------------------------------------------------------------------
ARM_CASES = [
    # (nq, nt, d, k, metric)      arm reached
    (5, 40, 3, 4, "euclidean"),    # direct (d<=32, k<=16): fma
    (4, 30, 37, 20, "euclidean"),  # metric family: fma
    (3, 12, 130, 4, "euclidean"),  # host arm (d > 128): mul+add
    (2, 140, 6, 130, "euclidean"),  # host arm (k > 128): mul+add
    (4, 30, 9, 5, "cosine"),       # metric family: fma dot, cosine_fold
    (3, 12, 131, 3, "cosine"),     # host arm: reciprocal norms
]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("case", ARM_CASES)
def test_oracle_matches_exact_model_bitwise(case, dtype):
    nq, nt, d, k, metric = case
    xq, xt = _data(11 + d, nq, nt, d, dtype)
    got_d, got_i = oracle.knn_topk(xq, xt, k, metric)
    want_d, want_i = model_knn(xq, xt, k, metric)
    assert np.array_equal(got_i, want_i)
    assert np.array_equal(got_d.view(np.uint8), want_d.view(np.uint8))


def test_exact_model_separates_fma_from_muladd():
    """The bitwise comparison above has teeth: on these inputs a fused and an
    unfused accumulation give different bits, so an oracle that used the wrong
    one for an arm would fail."""
    xq, xt = _data(3, 4, 30, 37, np.float32)
    diffs = sum(model_pair(q, y, "euclid_fma") != model_pair(q, y, "euclid_muladd") for q in xq for y in xt)
    assert diffs > 0


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_oracle_kmeans_matches_exact_model(dtype):
    x, c = _data(5, 60, 7, 6, dtype)
    got_l, got_d = oracle.kmeans_assign(x, c)
    want_l, want_d = model_kmeans(x, c)
    assert np.array_equal(got_l, want_l)
    assert np.array_equal(got_d, want_d)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("metric", ["euclidean", "cosine"])
def test_oracle_pairwise_and_norms_match_exact_model(dtype, metric):
    x, y = _data(9, 6, 5, 11, dtype)
    got = oracle.pairwise(x, y, metric)
    for i in range(len(x)):
        for j in range(len(y)):
            if metric == "euclidean":
                want = model_pair(x[i], y[j], "euclid_muladd")
            else:
                # cosine_dist: mul+add dot, sqrt(xn*yn), divide, clamp
                T = x.dtype.type
                dot = T(0)
                for a, b in zip(x[i], y[j]):
                    dot = T(dot + T(a * b))
                denom = np.sqrt(T(_sumsq(x[i]) * _sumsq(y[j])))
                want = _clamp02(T(T(1) - (T(dot / denom) if denom > 0 else T(0))))
            assert got[i, j] == want
    norms = oracle.row_sqnorms(x)
    assert all(norms[i] == _sumsq(x[i]) for i in range(len(x)))


def test_arm_dispatch_table():
    # nearest.rs:910-947 with the cpu caps
    assert oracle.knn_arm(32, 16, "euclidean") == oracle.ARM_DIRECT
    assert oracle.knn_arm(33, 16, "euclidean") == oracle.ARM_METRIC
    assert oracle.knn_arm(32, 17, "euclidean") == oracle.ARM_METRIC
    assert oracle.knn_arm(128, 128, "euclidean") == oracle.ARM_METRIC
    assert oracle.knn_arm(129, 5, "euclidean") == oracle.ARM_HOST
    assert oracle.knn_arm(64, 129, "euclidean") == oracle.ARM_HOST
    assert oracle.knn_arm(3, 3, "cosine") == oracle.ARM_METRIC
    assert oracle.knn_arm(256, 16, "cosine") == oracle.ARM_HOST


# ---------------------------------------------------------------------------
# the reference's sklearn fixtures
# ---------------------------------------------------------------------------
def _brute(xq, xt, metric, p=2.0):
    q = xq.astype(np.float64)
    t = xt.astype(np.float64)
    if metric == "euclidean":
        return lambda r, j: float(np.sqrt(np.sum((q[r] - t[j]) ** 2)))
    if metric == "manhattan":
        return lambda r, j: float(np.sum(np.abs(q[r] - t[j])))
    if metric == "chebyshev":
        return lambda r, j: float(np.max(np.abs(q[r] - t[j])))
    if metric == "minkowski":
        return lambda r, j: float(np.sum(np.abs(q[r] - t[j]) ** p) ** (1.0 / p))
    return lambda r, j: float(1.0 - np.dot(q[r], t[j]) / (np.linalg.norm(q[r]) * np.linalg.norm(t[j])))


@pytest.mark.parametrize("s", ["f32", "f64"])
def test_fixture_knn_seed42(s):
    z = load_golden("knn_%s_seed42" % s)
    k = int(z["k"][0])
    d, i = oracle.knn_topk(z["Xq"], z["X"], k)
    assert np.all(np.abs(d - z["distances"]) <= 1e-5 * np.maximum(np.abs(z["distances"]), 1.0))
    assert np.array_equal(i, z["indices"].astype(np.uint32))


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("metric,keys", [
    ("euclidean", ["euclidean", "alias_{}_euclidean", "alias_{}_l2", "alias_{}_minkowski", "alg_{}_auto",
                   "alg_{}_brute"]),
    ("cosine", ["cosine", "alias_{}_cosine"]),
    ("manhattan", ["manhattan", "alias_{}_manhattan", "alias_{}_l1", "alias_{}_cityblock"]),
    ("chebyshev", ["chebyshev", "alias_{}_chebyshev", "alias_{}_infinity"]),
    ("minkowski", ["minkowski"]),
])
def test_fixture_nn_params(s, metric, keys):
    z = load_golden("nn_params_%s_seed42" % s)
    k = int(z["k"][0])
    p = float(z["p"][0])
    d, i = oracle.knn_topk(z["Xq"], z["X"], k, metric, p=p)
    for key in keys:
        dk = ("distances_" + key) if "{}" not in key else key.format("distances")
        ik = ("indices_" + key) if "{}" not in key else key.format("indices")
        assert_topk_matches(d, i, z[dk], z[ik].astype(np.int64), _brute(z["Xq"], z["X"], metric, p))


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("metric", ["euclidean", "cosine", "manhattan", "chebyshev", "minkowski"])
def test_fixture_knn_metric_graph(s, metric):
    """X-vs-X with k+1 (self included) and a planted duplicate pair."""
    z = load_golden("knn_%s_%s_seed42" % (metric, s))
    k = int(z["k"][0]) + 1
    p = float(z["p"][0]) if "p" in z.files else 2.0
    d, i = oracle.knn_topk(z["X"], z["X"], k, metric, p=p)
    assert_topk_matches(d, i, z["distances"], z["indices"].astype(np.int64), _brute(z["X"], z["X"], metric, p))
    a, b = int(z["dup_row_a"][0]), int(z["dup_row_b"][0])
    # identical rows score exactly 0 against each other; lowest index first
    assert d[a, 0] == 0 and d[a, 1] == 0 and list(i[a, :2]) == sorted([a, b])
    assert d[b, 0] == 0 and d[b, 1] == 0 and list(i[b, :2]) == sorted([a, b])


@pytest.mark.parametrize("name", ["dist_sq_f32_seed42", "dist_sq_f64_seed42", "dist_sqrt_f64_seed42"])
def test_fixture_pairwise(name):
    z = load_golden(name)
    got = oracle.pairwise(z["X"], z["Y"], "euclidean", sqrt="sqrt" in name)
    assert np.all(np.abs(got - z["D"]) <= 1e-5 * np.maximum(np.abs(z["D"]), 1.0))


@pytest.mark.parametrize("s", ["f32", "f64"])
def test_fixture_kmeans_labels_and_inertia(s):
    z = load_golden("kmeans_%s_seed42" % s)
    labels, sq = oracle.kmeans_assign(z["X"], z["centers"])
    assert np.array_equal(labels, z["labels"].astype(np.uint32))
    inertia = float(np.sum(sq.astype(np.float64)))
    assert abs(inertia - float(z["inertia"][0])) <= 1e-5 * max(abs(float(z["inertia"][0])), 1.0)


def test_fixture_argmin_tie_rule():
    """argmin_tie_i32: planted row ties resolve to the lowest column.  Rebuilt as
    a 1-D assignment: point 0 against centres at sqrt of each row's values is not
    exact, so instead the values are used as squared distances of centres placed
    on orthogonal axes from the origin (||0 - c||^2 = c^2 exactly for integers)."""
    z = load_golden("argmin_tie_i32_seed42")
    X = z["X"]
    for r in range(X.shape[0]):
        vals = X[r]
        d = len(vals)
        # centre j sits on axis j at distance sqrt(vals[j]); use integer coordinates
        # by encoding vals[j] as a sum of unit squares along private axes
        width = int(vals.max())
        cen = np.zeros((d, d * width), dtype=np.float64)
        for j, v in enumerate(vals):
            cen[j, j * width:j * width + int(v)] = 1.0
        lab, sq = oracle.kmeans_assign(np.zeros((d, d * width)), cen)
        assert lab[0] == int(z["argmin_rows"][r])
        assert sq[0] == vals.min()


# ---------------------------------------------------------------------------
# known-answer invariants of the reference tests
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("metric", ["euclidean", "cosine"])
def test_all_duplicates_give_first_k_indices(metric):
    # knn_metric_kernel_test.rs:269-289
    row = np.array([[0.5, -1.25, 2.0, 3.0]], dtype=np.float32)
    xt = np.repeat(row, 40, axis=0)
    d, i = oracle.knn_topk(row, xt, 7, metric)
    assert list(i[0]) == list(range(7))
    assert np.all(d == 0)


@pytest.mark.parametrize("metric", ["euclidean", "cosine"])
def test_rows_ascending(metric):
    xq, xt = _data(21, 50, 300, 12, np.float32)
    d, i = oracle.knn_topk(xq, xt, 9, metric)
    assert np.all(np.diff(d, axis=1) >= 0)
    for r in range(len(d)):
        for c in range(8):
            if d[r, c] == d[r, c + 1]:
                assert i[r, c] < i[r, c + 1]


def test_nan_rows_never_admitted_and_sentinels_clamp():
    # knn_test.rs:1075-1158 / emit_lists (knn.rs:2931-2961)
    xq, xt = _data(2, 6, 20, 4, np.float32)
    xt[3, 1] = np.nan
    xt[7, 0] = np.nan
    xq[2, 3] = np.nan
    d, i = oracle.knn_topk(xq, xt, 19)
    for r in (0, 1, 3, 4, 5):
        assert 3 not in i[r, :18] and 7 not in i[r, :18]
        assert np.isinf(d[r, 18]) and i[r, 18] == 0   # 18 finite rows, one sentinel slot
    assert np.all(np.isinf(d[2])) and np.all(i[2] == 0)


def test_constructed_tie_lowest_index_first():
    # topk_test.rs:204: equidistant candidates resolve by index
    xq = np.zeros((1, 2), dtype=np.float32)
    xt = np.array([[3, 4], [0, 5], [5, 0], [-4, 3], [1, 1]], dtype=np.float32)
    d, i = oracle.knn_topk(xq, xt, 4)
    assert list(i[0]) == [4, 0, 1, 2]
    assert np.allclose(d[0], [np.sqrt(2), 5, 5, 5])


def test_k_equals_n_train_and_bad_k():
    xq, xt = _data(4, 3, 9, 5, np.float64)
    d, i = oracle.knn_topk(xq, xt, 9)
    assert sorted(i[0].tolist()) == list(range(9))
    with pytest.raises(ValueError):
        oracle.knn_topk(xq, xt, 10)


def test_kmeans_tie_and_nan_rules():
    x = np.array([[0.0, 0.0], [np.nan, 1.0], [1.0, 1.0]], dtype=np.float32)
    c = np.array([[1.0, 0.0], [0.0, 1.0], [-1.0, 0.0]], dtype=np.float32)
    lab, sq = oracle.kmeans_assign(x, c)
    assert lab[0] == 0 and sq[0] == 1.0       # three-way tie -> lowest index
    assert lab[1] == 0 and np.isnan(sq[1])    # NaN distance to centre 0 wins (seeded best)
    assert lab[2] in (0, 1) and lab[2] == 0   # tie between 0 and 1 -> 0


# ---------------------------------------------------------------------------
# independent cross-check: sklearn brute force (tolerance)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("metric", ["euclidean", "cosine"])
def test_oracle_vs_sklearn(dtype, metric):
    from sklearn.neighbors import NearestNeighbors
    xq, xt = _data(31, 40, 500, 24, dtype)
    k = 12
    d, i = oracle.knn_topk(xq, xt, k, metric)
    nn = NearestNeighbors(n_neighbors=k, algorithm="brute", metric=metric).fit(xt.astype(np.float64))
    wd, wi = nn.kneighbors(xq.astype(np.float64))
    assert_topk_matches(d, i, wd, wi, _brute(xq, xt, metric), atol_rel=1e-5 if dtype == np.float32 else 1e-12)


@pytest.mark.parametrize("d", [129, 256])
@pytest.mark.parametrize("metric", ["cosine", "euclidean"])
def test_host_arm_f64_against_numpy_brute_force(d, metric):
    """The knn_host arm (d > 128: reciprocal-norm cosine clamped to [0, 2],
    crates/mlrs-backend/src/prims/knn_host.rs:382-397 and :749-760; mul+add
    Euclidean) in f64 against an independent numpy f64 brute force (BLAS
    products, another summation order) at the north star's 1e-12 relative
    bar; indices equal except where the two picks' values tie within it.
    Inputs as config c3: iid U[0,1), rows not normalised."""
    assert oracle.knn_arm(d, 16, metric) == oracle.ARM_HOST
    rng = np.random.default_rng(d)
    xq, xt = rng.random((60, d)), rng.random((4000, d))
    k = 16
    got_d, got_i = oracle.knn_topk(xq, xt, k, metric)
    if metric == "cosine":
        nq_, nt_ = np.linalg.norm(xq, axis=1), np.linalg.norm(xt, axis=1)
        full = np.clip(1.0 - (xq @ xt.T) / np.outer(nq_, nt_), 0.0, 2.0)
    else:
        full = np.sqrt(np.maximum(((xq[:, None, :] - xt[None, :, :]) ** 2).sum(-1), 0.0))
    order = np.lexsort((np.broadcast_to(np.arange(xt.shape[0]), full.shape), full), axis=1)[:, :k]
    want_d = np.take_along_axis(full, order, axis=1)
    rel = np.abs(got_d - want_d) / np.abs(want_d)
    assert rel.max() <= 1e-12, rel.max()
    for r, c in np.argwhere(got_i != order):
        picked = full[r, got_i[r, c]]
        assert abs(picked - want_d[r, c]) <= 1e-12 * abs(want_d[r, c]), (r, c)


def test_oracle_kmeans_vs_sklearn():
    from sklearn.cluster import KMeans
    rng = np.random.default_rng(8)
    x = rng.standard_normal((400, 8)).astype(np.float32)
    c = rng.standard_normal((6, 8)).astype(np.float32)
    km = KMeans(n_clusters=6, init=c.astype(np.float64), n_init=1, max_iter=1).fit(c.astype(np.float64))
    km.cluster_centers_ = c.astype(np.float64)
    lab, _ = oracle.kmeans_assign(x, c)
    assert np.array_equal(lab, km.predict(x.astype(np.float64)).astype(np.uint32))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("metric,p", [("manhattan", 2.0), ("chebyshev", 2.0), ("minkowski", 3.0),
                                      ("minkowski", 5.0), ("minkowski", 2.5)])
def test_metric_family_matches_exact_model(dtype, metric, p):
    """The oracle's manhattan / chebyshev / minkowski arithmetic against a
    scalar restatement in the same dtype (numpy scalars round each operation):
    running sum of |x-y|, running max by select, |x-y|^p by a multiply chain
    for integer p in 3..8 and pow otherwise, then the 1/p root.  Bit for bit
    except where a pow is involved: numpy's power and the C library's may
    differ in the last place, so those values are held to 4 ulp."""
    T = np.dtype(dtype).type
    rng = np.random.default_rng(9)
    X = rng.standard_normal((40, 5)).astype(dtype)
    Q = rng.standard_normal((6, 5)).astype(dtype)
    k = 7
    d, i = oracle.knn_topk(Q, X, k, metric, p=p)
    pi = int(p) if (p == int(p) and 3 <= int(p) <= 8) else 0
    for r in range(Q.shape[0]):
        vals = []
        for t in range(X.shape[0]):
            acc = T(0)
            for c in range(X.shape[1]):
                ad = T(abs(T(Q[r, c] - X[t, c])))
                if metric == "manhattan":
                    acc = T(acc + ad)
                elif metric == "chebyshev":
                    acc = ad if ad > acc else acc
                else:
                    if pi:
                        rr = ad
                        for _ in range(1, pi):
                            rr = T(rr * ad)
                    else:
                        rr = T(np.power(ad, T(p)))
                    acc = T(acc + rr)
            vals.append((acc, t))
        vals.sort()
        want_i = [t for _, t in vals[:k]]
        want_v = [v for v, _ in vals[:k]]
        if metric == "minkowski":
            want_v = [T(np.power(v, T(1.0 / p))) for v in want_v]
        assert list(i[r]) == want_i
        if metric == "minkowski":
            np.testing.assert_allclose(d[r], np.array(want_v, dtype=dtype), rtol=4 * np.finfo(dtype).eps, atol=0)
        else:
            assert np.array_equal(d[r], np.array(want_v, dtype=dtype))


_ISA_SCRIPT = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[2])
import oracle
assert oracle.host_isa() == sys.argv[3]
rng = np.random.default_rng(0)
out = {}
for d, dt, metric in [(3, np.float32, "euclidean"), (64, np.float32, "euclidean"), (64, np.float32, "cosine"),
                      (131, np.float64, "cosine"), (40, np.float64, "manhattan")]:
    xq = rng.standard_normal((50, d)).astype(dt)
    xt = rng.standard_normal((3000, d)).astype(dt)
    dd, ii = oracle.knn_topk(xq, xt, 9, metric)
    out["d_%d_%s" % (d, metric)], out["i_%d_%s" % (d, metric)] = dd, ii
x = rng.standard_normal((5000, 16)).astype(np.float32)
c = rng.standard_normal((33, 16)).astype(np.float32)
out["lab"], out["sq"] = oracle.kmeans_assign(x, c)
out["pw"] = oracle.pairwise(x[:100], c, "euclidean", sqrt=True)
gi, gd = oracle.knn_graph(x[:800].astype(np.float64), 7, "cosine")
out["gi"], out["gd"] = gi, gd
fit = oracle.kmeans_fit(x, 8, "k-means++", seed=3, max_iter=5)
out["fc"], out["fl"] = fit[0], fit[1]
np.savez(sys.argv[1], **out)
"""


def test_isa_builds_return_the_same_bits(tmp_path):
    """The x86-64-v3 and x86-64-v4 builds of the oracle (the box loads the
    widest its CPU runs) agree bit for bit: -ffp-contract=off and no
    reassociation leave vectorisation nothing to change."""
    import subprocess
    import sys
    if oracle.host_isa() != "x86-64-v4":
        pytest.skip("this host cannot run the AVX-512 build")
    res = {}
    for isa in ("x86-64-v3", "x86-64-v4"):
        f = str(tmp_path / (isa + ".npz"))
        env = dict(os.environ, MLRS_ORACLE_ISA=isa)
        subprocess.run([sys.executable, "-c", _ISA_SCRIPT, f, ROOT, isa], check=True, env=env)
        res[isa] = np.load(f)
    a, b = res["x86-64-v3"], res["x86-64-v4"]
    for key in a.files:
        assert np.array_equal(a[key], b[key], equal_nan=True), key
