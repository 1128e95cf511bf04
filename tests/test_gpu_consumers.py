"""GPU parity of the kNN consumers: the device regressor gathers and
classifier vote against the CPU oracle, bit for bit, on neighbour sets from
the oracle's own search; the index-error paths; and the estimators against
the reference's sklearn fixtures.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import load_golden
from mlrs_amd import _lib, prims
from mlrs_amd.neighbors import KNeighborsClassifier, KNeighborsRegressor

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _search(seed, nq, nt, d, k, dtype, dup=False):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((nt, d)).astype(dtype)
    Xq = rng.standard_normal((nq, d)).astype(dtype)
    if dup:  # coincident queries -> zero distances -> the indicator weighting
        Xq[::7] = X[3]
        X[10] = X[3]
    dist, idx = oracle.knn_topk(Xq, X, k)
    return dist, idx


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("k,n_out,weighted", [(1, 1, False), (5, 1, False), (32, 1, False), (5, 1, True),
                                              (17, 3, False), (17, 3, True), (8, 1, True)])
def test_regress_bitwise(dtype, k, n_out, weighted):
    dist, idx = _search(20 + k, 300, 2000, 8, k, dtype, dup=True)
    rng = np.random.default_rng(k)
    y = (rng.standard_normal((2000, n_out)) * 1e4).astype(dtype)
    y[::5] *= -1e-3
    y = y if n_out > 1 else y.ravel()
    want, oob = oracle.knn_regress(y, idx, dist, weighted=weighted)
    assert not oob.any()
    got = prims.knn_regress(_t(y), _t(idx.astype(np.int64)), _t(dist), weighted=weighted)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("n_classes,k,weighted", [(2, 5, False), (7, 16, True), (300, 9, False), (3, 4, True)])
def test_classify_bitwise(dtype, n_classes, k, weighted):
    dist, idx = _search(40 + k, 500, 3000, 6, k, dtype, dup=True)
    rng = np.random.default_rng(n_classes)
    codes = rng.integers(0, n_classes, 3000)
    want_p, want_l = oracle.knn_classify(codes, n_classes, idx, dist, weighted=weighted, dtype=dtype)
    p, l = prims.knn_classify(_t(codes.astype(np.int32)), n_classes, _t(idx.astype(np.int64)), _t(dist),
                              weighted=weighted, dtype=torch.float32 if dtype == np.float32 else torch.float64)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(p.cpu().numpy(), want_p)
    np.testing.assert_array_equal(l.cpu().numpy(), want_l.astype(np.int64))


def test_regress_bad_index_raises_for_first_row():
    y = np.arange(10, dtype=np.float32)
    idx = np.array([[0, 1], [2, 3], [10, 1], [99, 0]], dtype=np.int64)
    with pytest.raises(_lib.ShapeMismatch) as e:
        prims.knn_regress(_t(y), _t(idx))
    assert e.value.operand == "knn.train_idx" and e.value.rows == 2 and e.value.len == 10


def test_classify_errors_first_in_row_order():
    codes = np.array([0, 1, 2, 9], dtype=np.int32)
    idx = np.array([[0, 1], [1, 3], [7, 0]], dtype=np.int64)
    with pytest.raises(_lib.ShapeMismatch) as e:
        prims.knn_classify(_t(codes), 3, _t(idx), None)
    assert e.value.operand == "knn.class_id" and e.value.rows == 9 and e.value.len == 3
    with pytest.raises(_lib.ShapeMismatch) as e:
        prims.knn_classify(_t(codes), 3, _t(np.array([[0, 1], [5, 0]], np.int64)), None)
    assert e.value.operand == "knn.train_idx" and e.value.rows == 5 and e.value.len == 4


@pytest.mark.parametrize("s", ["f32", "f64"])
def test_estimators_match_fixture(s):
    z = load_golden("knn_%s_seed42" % s)
    k = int(z["k"][0])
    reg = KNeighborsRegressor(n_neighbors=k).fit(z["X"], z["y_reg"])
    np.testing.assert_allclose(reg.predict(z["Xq"]), z["predict_reg"], rtol=1e-5, atol=1e-5)
    clf = KNeighborsClassifier(n_neighbors=k).fit(z["X"], z["y_class"])
    np.testing.assert_array_equal(clf.predict(z["Xq"]), z["predict_class"])
    np.testing.assert_allclose(clf.predict_proba(z["Xq"]), z["predict_proba"], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("metric", ["euclidean", "cosine"])
@pytest.mark.parametrize("weights", ["uniform", "distance"])
def test_estimator_params_fixtures(s, metric, weights):
    zr = load_golden("knn_reg_params_%s_seed42" % s)
    k = int(zr["k"][0])
    reg = KNeighborsRegressor(n_neighbors=k, weights=weights, metric=metric).fit(zr["X"], zr["y"])
    np.testing.assert_allclose(reg.predict(zr["Xq"]), zr["predict_%s_%s" % (metric, weights)], rtol=1e-5,
                               atol=1e-5)
    if metric == "euclidean":
        regm = KNeighborsRegressor(n_neighbors=k, weights=weights, metric=metric).fit(zr["X"], zr["y_multi"])
        np.testing.assert_allclose(regm.predict(zr["Xq"]), zr["predict_multi_%s" % weights], rtol=1e-5, atol=1e-5)
    zc = load_golden("knn_clf_params_%s_seed42" % s)
    clf = KNeighborsClassifier(n_neighbors=k, weights=weights, metric=metric).fit(zc["X"], zc["y"])
    np.testing.assert_array_equal(clf.predict(zc["Xq"]), zc["predict_%s_%s" % (metric, weights)])
    np.testing.assert_allclose(clf.predict_proba(zc["Xq"]), zc["proba_%s_%s" % (metric, weights)], rtol=1e-5,
                               atol=1e-5)
    if metric == "euclidean":  # multi-output target: the host vote over the same neighbour set
        clfm = KNeighborsClassifier(n_neighbors=k, weights=weights).fit(zc["X"], zc["y_multi"])
        np.testing.assert_array_equal(clfm.predict(zc["Xq"]), zc["predict_multi_%s" % weights])


def test_estimators_bitwise_against_oracle():
    """The device predict equals the oracle's consumer applied to the oracle's
    neighbour set, bit for bit (the engine's search is itself bitwise)."""
    rng = np.random.default_rng(5)
    X = rng.standard_normal((4000, 24)).astype(np.float32)
    Xq = rng.standard_normal((700, 24)).astype(np.float32)
    y = rng.standard_normal(4000).astype(np.float32) * 100
    yc = rng.integers(0, 5, 4000) * 3 + 1  # non-contiguous labels
    d, i = oracle.knn_topk(Xq, X, 7)
    for w in ("uniform", "distance"):
        want, _ = oracle.knn_regress(y, i, d, weighted=w == "distance")
        got = KNeighborsRegressor(n_neighbors=7, weights=w).fit(X, y).predict(Xq)
        np.testing.assert_array_equal(got, want)
        classes, codes = np.unique(yc, return_inverse=True)
        wp, wl = oracle.knn_classify(codes, classes.size, i, d, weighted=w == "distance")
        clf = KNeighborsClassifier(n_neighbors=7, weights=w).fit(X, yc)
        np.testing.assert_array_equal(clf.predict(Xq), classes[wl])
        np.testing.assert_array_equal(clf.predict_proba(Xq), wp)
