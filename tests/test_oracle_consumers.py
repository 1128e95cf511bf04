"""Pins the CPU oracle's kNN consumers (oracle/consumers_cpu.c) -- CPU only.

* knn_regress (knn_regress_mean / knn_regress_gather): the reference's sklearn
  fixtures (knn_{f32,f64}_seed42 ``predict_reg``; knn_reg_params_* uniform /
  distance / multi-output) to the reference's 1e-5 band -- sklearn sums with
  numpy, the kernels with Neumaier compensation, so agreement is to tolerance
  -- plus known answers the compensation and the weighting rules fix exactly.
* knn_classify (the classifier vote): the fixtures' ``predict_class`` /
  ``predict_proba`` (knn_{f32,f64}_seed42, knn_clf_params_*), the tie rule and
  the index-error rule.
"""
import numpy as np
import pytest

import oracle
from conftest import load_golden


def _neigh(X, Xq, k, metric="euclidean", p=2.0):
    d, i = oracle.knn_topk(Xq, X, k, metric, p=p)
    return d, i


METRICS = ["euclidean", "cosine", "manhattan", "chebyshev", "minkowski"]


@pytest.mark.parametrize("s", ["f32", "f64"])
def test_regress_and_classify_fixture(s):
    z = load_golden("knn_%s_seed42" % s)
    X, Xq, k = z["X"], z["Xq"], int(z["k"][0])
    d, i = _neigh(X, Xq, k)
    pred, oob = oracle.knn_regress(z["y_reg"], i)
    assert not oob.any()
    np.testing.assert_allclose(pred, z["predict_reg"], rtol=1e-5, atol=1e-5)
    classes, codes = np.unique(z["y_class"], return_inverse=True)
    proba, lab = oracle.knn_classify(codes, classes.size, i, d, dtype=X.dtype)
    np.testing.assert_array_equal(classes[lab], z["predict_class"])
    np.testing.assert_allclose(proba, z["predict_proba"], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("metric", METRICS)
@pytest.mark.parametrize("weights", ["uniform", "distance"])
def test_regress_params_fixture(s, metric, weights):
    z = load_golden("knn_reg_params_%s_seed42" % s)
    X, Xq, k = z["X"], z["Xq"], int(z["k"][0])
    d, i = _neigh(X, Xq, k, metric, float(z["p"][0]))
    pred, _ = oracle.knn_regress(z["y"], i, d, weighted=weights == "distance")
    np.testing.assert_allclose(pred, z["predict_%s_%s" % (metric, weights)], rtol=1e-5, atol=1e-5)
    if metric == "euclidean":
        pm, _ = oracle.knn_regress(np.ascontiguousarray(z["y_multi"]), i, d, weighted=weights == "distance")
        np.testing.assert_allclose(pm, z["predict_multi_%s" % weights], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("metric", METRICS)
@pytest.mark.parametrize("weights", ["uniform", "distance"])
def test_classify_params_fixture(s, metric, weights):
    z = load_golden("knn_clf_params_%s_seed42" % s)
    X, Xq, k = z["X"], z["Xq"], int(z["k"][0])
    d, i = _neigh(X, Xq, k, metric, float(z["p"][0]))
    classes, codes = np.unique(z["y"], return_inverse=True)
    np.testing.assert_array_equal(classes, z["classes"])
    proba, lab = oracle.knn_classify(codes, classes.size, i, d, weighted=weights == "distance", dtype=X.dtype)
    np.testing.assert_array_equal(classes[lab], z["predict_%s_%s" % (metric, weights)])
    # the reference tests' mixed bar: |err| <= 1e-5 + 1e-5|want| (knn_classifier_params_test.rs:68-115)
    np.testing.assert_allclose(proba, z["proba_%s_%s" % (metric, weights)], rtol=1e-5, atol=1e-5)


def test_neumaier_compensation_known_answer():
    """[1e8, 1, -1e8] sums to exactly 1 only with the compensation: a plain f32
    running sum gives 0, so the mean 1/3 distinguishes the two."""
    y = np.array([1e8, 1.0, -1e8], dtype=np.float32)
    idx = np.array([[0, 1, 2]], dtype=np.uint32)
    pred, _ = oracle.knn_regress(y, idx)
    assert pred[0] == np.float32(1.0) / np.float32(3.0)
    # the general gather uses the same compensation, for w*y and for w
    pw, _ = oracle.knn_regress(y, idx, np.ones((1, 3), np.float32), weighted=True)
    assert pw[0] == np.float32(1.0) / np.float32(3.0)


def test_distance_weights_indicator_rule():
    """A row with a zero distance weighs its zero-distance neighbours 1 and the
    rest 0 (knn.rs:161-171, sklearn _get_weights); otherwise 1/d."""
    y = np.array([2.0, 10.0, 4.0, 7.0], dtype=np.float64)
    idx = np.array([[0, 1, 2], [1, 3, 0]], dtype=np.uint32)
    dist = np.array([[0.0, 0.5, 0.0], [1.0, 2.0, 4.0]], dtype=np.float64)
    pred, _ = oracle.knn_regress(y, idx, dist, weighted=True)
    assert pred[0] == 3.0
    assert pred[1] == pytest.approx((10.0 + 7.0 / 2 + 2.0 / 4) / (1 + 0.5 + 0.25), rel=1e-15)
    proba, lab = oracle.knn_classify(np.array([0, 1, 1, 0]), 2, idx, dist, weighted=True, dtype=np.float64)
    assert proba[0].tolist() == [0.5, 0.5] and lab[0] == 0  # tie -> lowest class
    np.testing.assert_allclose(proba[1], [(0.5 + 0.25) / 1.75, 1.0 / 1.75])


def test_index_errors():
    y = np.arange(4, dtype=np.float32)
    idx = np.array([[0, 1], [4, 2], [9, 9]], dtype=np.uint32)
    pred, oob = oracle.knn_regress(y, idx)
    assert oob.tolist() == [0, 1, 1]
    assert pred[1] == np.float32(2.0) / np.float32(2.0)  # the bad index contributes nothing, / k stays
    with pytest.raises(IndexError) as e:
        oracle.knn_classify(np.array([0, 1, 0, 1]), 2, idx, None)
    assert e.value.args[0] == ("train_idx", 4, 1, 0)
    with pytest.raises(IndexError) as e:
        oracle.knn_classify(np.array([0, 5, 0, 1]), 2, np.array([[0, 1]], np.uint32), None)
    assert e.value.args[0] == ("class_id", 5, 0, 1)
