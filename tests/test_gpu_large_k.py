"""GPU parity for k above the LDS selection's 256: every 1 <= k <= n_train is
answered, as the reference's knn_host_possible (crates/mlrs-backend/src/prims/
knn_host.rs:182-184) and top_k (crates/mlrs-backend/src/prims/topk.rs:208-212)
answer it, bit for bit against the CPU oracle.

k <= 8192 (f32) / 4096 (f64) sorts each row's kept pairs in one LDS chunk;
larger k sorts chunks and merges them in global memory -- the n_train = 20k
and 9k cases below take that path.  Ties (duplicated rows) and NaN rows (never
admitted, so k = n_train leaves (+inf, 0) slots) are planted in every case.
"""
import numpy as np
import pytest
import torch

import oracle
from mlrs_amd import prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _data(seed, nq, nt, d, dtype, metric):
    rng = np.random.default_rng(seed)
    if metric == "cosine":
        xq, xt = rng.random((nq, d)), rng.random((nt, d))
    else:
        xq, xt = rng.standard_normal((nq, d)), rng.standard_normal((nt, d))
    xq, xt = xq.astype(dtype), xt.astype(dtype)
    xt[17] = xt[3]          # exact ties
    xt[nt - 1] = xt[3]
    xt[40, 1] = np.nan      # never admitted
    xq[2] = xt[3]           # a query on a tied point
    return xq, xt


def _assert_same(gd, gi, wd, wi, label):
    bad = np.argwhere(gi != wi.astype(np.int64))
    assert bad.size == 0, "%s: %d index mismatches, first %s" % (label, len(bad), bad[:3].tolist())
    same = (gd == wd) | (np.isnan(gd) & np.isnan(wd))
    assert same.all(), "%s: distance bits differ at %s" % (label, np.argwhere(~same)[:3].tolist())


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("metric", ["euclidean", "cosine"])
@pytest.mark.parametrize("k", [257, 1000, 5003])
@pytest.mark.parametrize("d", [24, 131])
def test_large_k_matches_oracle(dtype, metric, k, d):
    nt, nq = 5003, 29
    xq, xt = _data(k + d, nq, nt, d, dtype, metric)
    wd, wi = oracle.knn_topk(xq, xt, k, metric)
    gd, gi = prims.knn_topk(_t(xq), _t(xt), k, metric)
    torch.cuda.synchronize()
    gd, gi = gd.cpu().numpy(), gi.cpu().numpy()
    _assert_same(gd, gi, wd, wi, "%s %s k=%d d=%d" % (np.dtype(dtype).name, metric, k, d))
    if k == nt:
        # the NaN row fills nothing: the last slot is the sentinel
        assert np.all(gd[:, -1] == np.inf) and np.all(gi[:, -1] == 0)


@pytest.mark.parametrize("dtype,nt,k", [(np.float32, 20011, 20011), (np.float32, 20011, 12000),
                                        (np.float64, 9001, 9001), (np.float64, 9001, 5000)])
def test_k_above_one_lds_chunk(dtype, nt, k):
    xq, xt = _data(nt + k, 6, nt, 16, dtype, "euclidean")
    wd, wi = oracle.knn_topk(xq, xt, k)
    gd, gi = prims.knn_topk(_t(xq), _t(xt), k)
    torch.cuda.synchronize()
    _assert_same(gd.cpu().numpy(), gi.cpu().numpy(), wd, wi, "merge path k=%d" % k)


def test_large_k_heavy_ties():
    # integer grid: thousands of exactly equal distances per row, ranked by index
    rng = np.random.default_rng(5)
    xt = rng.integers(-2, 3, size=(6000, 3)).astype(np.float32)
    xq = rng.integers(-2, 3, size=(9, 3)).astype(np.float32)
    for k in (300, 4000, 6000):
        wd, wi = oracle.knn_topk(xq, xt, k)
        gd, gi = prims.knn_topk(_t(xq), _t(xt), k)
        _assert_same(gd.cpu().numpy(), gi.cpu().numpy(), wd, wi, "ties k=%d" % k)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("metric,p", [("euclidean", 2.0), ("cosine", 2.0), ("manhattan", 2.0)])
@pytest.mark.parametrize("k,include_self", [(300, False), (999, True)])
def test_graph_large_k(dtype, metric, p, k, include_self):
    rng = np.random.default_rng(k)
    x = rng.standard_normal((1200, 7)).astype(dtype)
    x[5] = x[9]
    wi, wd = oracle.knn_graph(x, k, metric, p=p, include_self=include_self)
    gi, gd = prims.knn_graph(_t(x), k, metric, p=p, include_self=include_self)
    np.testing.assert_array_equal(gi.cpu().numpy(), wi.astype(np.int64))
    np.testing.assert_array_equal(gd.cpu().numpy(), wd)


@pytest.mark.parametrize("min_samples", [257, 1500, 2500])
def test_core_distances_large_min_samples(min_samples):
    rng = np.random.default_rng(min_samples)
    x = rng.standard_normal((2500, 5)).astype(np.float32)
    x[100] = x[7]
    want = oracle.core_distances(x, min_samples, "euclidean")
    got = prims.core_distances(_t(x), min_samples, "euclidean").cpu().numpy()
    np.testing.assert_array_equal(got, want)
