"""GPU parity of the X-vs-X graphs (mlrs_knn_graph_*, mlrs_hdbscan_core_
distances_*) against the CPU oracle's restatement of the reference's host
scans, bit for bit -- except Minkowski, whose pow the device and host C
libraries may round differently in the last place (values held to 4 ulp,
indices exact on these seeded inputs) -- and against the reference's
knn_graph fixtures through the prims.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import load_golden
from mlrs_amd import _lib, prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
METRICS = [("euclidean", 2.0), ("cosine", 2.0), ("manhattan", 2.0), ("chebyshev", 2.0), ("minkowski", 3.0),
           ("minkowski", 2.5)]


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.fixture(params=["auto", "generic"])
def family(request):
    prims.force_path(request.param)
    yield request.param
    prims.force_path("auto")


def _check(got_i, got_d, want_i, want_d, metric):
    np.testing.assert_array_equal(got_i, want_i.astype(np.int64))
    if metric == "minkowski":
        np.testing.assert_allclose(got_d, want_d, rtol=4 * np.finfo(np.float64).eps, atol=0)
    else:
        np.testing.assert_array_equal(got_d, want_d)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("metric,p", METRICS)
@pytest.mark.parametrize("shape", [(1500, 8, 15), (700, 40, 5), (400, 300, 33), (3000, 24, 100)])
@pytest.mark.parametrize("include_self", [False, True])
def test_graph_matches_oracle(family, dtype, metric, p, shape, include_self):
    n, d, k = shape
    rng = np.random.default_rng(n + d + k)
    x = rng.standard_normal((n, d)).astype(dtype)
    x[11] = x[4]
    x[12] = x[4]
    wi, wd = oracle.knn_graph(x, k, metric, p=p, include_self=include_self)
    gi, gd = prims.knn_graph(_t(x), k, metric, p=p, include_self=include_self)
    torch.cuda.synchronize()
    _check(gi.cpu().numpy(), gd.cpu().numpy(), wi, wd, metric)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("metric,p", [m for m in METRICS if m[0] != "cosine"])
@pytest.mark.parametrize("min_samples", [1, 5, 40])
def test_core_distances_match_oracle(family, dtype, metric, p, min_samples):
    rng = np.random.default_rng(min_samples)
    x = rng.standard_normal((2500, 6)).astype(dtype)
    x[100] = x[7]
    want = oracle.core_distances(x, min_samples, metric, p=p)
    got = prims.core_distances(_t(x), min_samples, metric, p=p).cpu().numpy()
    if metric == "minkowski":
        np.testing.assert_allclose(got, want, rtol=4 * np.finfo(np.float64).eps, atol=0)
    else:
        np.testing.assert_array_equal(got, want)


def test_graph_nan_row_and_ties():
    rng = np.random.default_rng(2)
    x = rng.integers(-2, 3, size=(600, 3)).astype(np.float64)   # heavy exact ties
    x[9, 0] = np.nan
    for metric, p in METRICS[:5]:
        wi, wd = oracle.knn_graph(x, 12, metric, p=p)
        gi, gd = prims.knn_graph(_t(x), 12, metric, p=p)
        _check(gi.cpu().numpy(), gd.cpu().numpy(), wi, wd, metric)
    want = oracle.core_distances(x, 7, "manhattan")
    got = prims.core_distances(_t(x), 7, "manhattan").cpu().numpy()
    np.testing.assert_array_equal(got, want)
    assert got[9] == np.inf


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("metric", ["euclidean", "manhattan", "chebyshev", "minkowski", "cosine"])
def test_graph_fixture(s, metric):
    z = load_golden("knn_%s_%s_seed42" % (metric, s))
    X, k = z["X"], int(z["k"][0])
    p = float(z["p"][0]) if metric == "minkowski" else 2.0
    gi, gd = prims.knn_graph(_t(X), k, metric, p=p)
    gi, gd = gi.cpu().numpy(), gd.cpu().numpy()
    ri, rd = z["indices"].astype(np.int64), z["distances"]
    for r in range(X.shape[0]):
        keep = ri[r] != r
        assert set(gi[r].tolist()) == set(ri[r][keep][:k].tolist())
        want = np.sort(rd[r][keep][:k])
        assert np.all(np.abs(np.sort(gd[r]) - want) <= 1e-5 + 1e-5 * np.abs(want))


def test_graph_errors():
    x = _t(np.zeros((10, 3), np.float32))
    with pytest.raises(_lib.ShapeMismatch) as e:
        prims.knn_graph(x, 10, "euclidean")
    assert e.value.operand == "k" and e.value.len == 9
    with pytest.raises(_lib.ShapeMismatch) as e:
        prims.knn_graph(x, 3, "minkowski", p=0.5)
    assert e.value.operand == "p"
    with pytest.raises(_lib.UnsupportedError):
        prims.core_distances(x, 3, "cosine")
