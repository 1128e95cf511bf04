"""GPU parity of the Gram kernels' seeded screen on a large index: for k > 1
the seed launch bounds each query's k-th value over an evenly spaced sample
of the index (row s * n / m) and starts every query's screen there.  Two
seeds exist: the exact one (the k-th exact value; m = 64 k, at most 2048 and
n / 512, at least 512) and, for Euclidean f32 at d <= 128, the matrix-core
one (the k-th smallest screen value plus its error bound; m = 64 k, at most
8192 and n / 128, at least 512).  The bound only prunes, so the answer must
stay the reference's own top-k, bit for bit against the CPU oracle --
checked with exact ties between a sampled row of either sample and
unsampled copies of it (the seed's k-th value can then equal the final one),
queries on those points, and a NaN row, for both register shapes (d <= 128
and 128 < d <= 256) and the Euclidean and cosine arms."""
import numpy as np
import pytest
import torch

import oracle
from mlrs_amd import prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
NT = 140_000


def _nsamp(k):
    """The exact seed's sample size (gram_seed_rows in knn_kernels.hpp)."""
    return min(NT, max(512, min(2048, NT // 512, 64 * k)))


def _nsamp_screen(k):
    """The matrix-core seed's sample size (seed_screen_rows in knn_gram_f32.hip)."""
    return min(NT, max(512, min(8192, NT // 128, 64 * k)))


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _data(seed, nq, d, metric, k):
    rng = np.random.default_rng(seed)
    if metric == "cosine":
        xq, xt = rng.random((nq, d), dtype=np.float32), rng.random((NT, d), dtype=np.float32)
    else:
        xq, xt = rng.standard_normal((nq, d), dtype=np.float32), rng.standard_normal((NT, d), dtype=np.float32)
    s1 = 1 * NT // _nsamp(k)               # a row of the exact seed's sample
    s2 = 3 * NT // _nsamp_screen(k)        # a row of the matrix-core seed's sample
    for r in (5, 6, 7, NT - 2):            # unsampled exact copies of them
        xt[r] = xt[s1]
    for r in (11, 12, NT - 5):
        xt[r] = xt[s2]
    xt[9, 0] = np.nan                      # never admitted
    xq[0] = xt[s1]                         # queries on the tied points
    xq[1] = xt[s1] * 1.0000001             # and next to them
    xq[2] = xt[s2]
    xq[3] = xt[s2] * 1.0000001
    return xq, xt


@pytest.mark.parametrize("metric,d,k", [
    ("euclidean", 64, 2), ("euclidean", 64, 16), ("euclidean", 64, 64), ("euclidean", 64, 100),
    ("euclidean", 128, 128), ("euclidean", 200, 32), ("cosine", 64, 16), ("cosine", 128, 128),
    ("cosine", 200, 16),
])
def test_seeded_screen_matches_oracle(metric, d, k):
    nq = 256
    xq, xt = _data(k * 1000 + d, nq, d, metric, k)
    wd, wi = oracle.knn_topk(xq, xt, k, metric)
    prims.force_path("fused")
    try:
        gd, gi = prims.knn_topk(_t(xq), _t(xt), k, metric)
        torch.cuda.synchronize()
    finally:
        prims.force_path("auto")
    gd, gi = gd.cpu().numpy(), gi.cpu().numpy()
    bad = np.argwhere(gi != wi.astype(np.int64))
    assert bad.size == 0, "%s d=%d k=%d: %d index mismatches, first %s" % (metric, d, k, len(bad), bad[:3].tolist())
    assert np.array_equal(gd, wd), "%s d=%d k=%d: distance bits differ" % (metric, d, k)


def _fused(xq, xt, k, metric):
    prims.force_path("fused")
    try:
        gd, gi = prims.knn_topk(_t(xq), _t(xt), k, metric)
        torch.cuda.synchronize()
    finally:
        prims.force_path("auto")
    return gd.cpu().numpy(), gi.cpu().numpy()


def _same(gd, gi, wd, wi, label):
    bad = np.argwhere(gi != wi.astype(np.int64))
    assert bad.size == 0, "%s: %d index mismatches, first %s" % (label, len(bad), bad[:3].tolist())
    same = (gd == wd) | (np.isnan(gd) & np.isnan(wd))
    assert same.all(), "%s: distance bits differ at %s" % (label, np.argwhere(~same)[:3].tolist())


def test_seed_large_norms_unseeded():
    # squared norms past 2^124: screen values may overflow, so the matrix-core
    # seed must leave such queries unbounded (their screen is not trusted)
    rng = np.random.default_rng(3)
    scale = np.float32(2.0 ** 59)
    xt = (rng.standard_normal((NT, 64)) * scale).astype(np.float32)
    xq = (rng.standard_normal((64, 64)) * scale).astype(np.float32)
    assert float(np.max(np.sum(xt.astype(np.float64) ** 2, axis=1))) > 2.0 ** 124
    xt[100] = xt[NT // 2]
    xq[0] = xt[NT // 2]
    wd, wi = oracle.knn_topk(xq, xt, 16, "euclidean")
    gd, gi = _fused(xq, xt, 16, "euclidean")
    _same(gd, gi, wd, wi, "large norms")


def test_seed_cosine_zero_query_and_rows():
    # a zero query ties every row at distance 1 (lowest indices win) and is
    # never seeded; zero rows score 1 against every query
    rng = np.random.default_rng(4)
    xt = rng.random((NT, 64), dtype=np.float32)
    xq = rng.random((64, 64), dtype=np.float32)
    xq[0] = 0.0
    xt[7] = 0.0
    xt[NT - 3] = 0.0
    wd, wi = oracle.knn_topk(xq, xt, 16, "cosine")
    gd, gi = _fused(xq, xt, 16, "cosine")
    _same(gd, gi, wd, wi, "cosine zeros")


@pytest.mark.parametrize("metric,d", [("euclidean", 256), ("cosine", 256), ("euclidean", 40), ("cosine", 130)])
def test_seed_f64_matches_oracle(metric, d):
    # the f64 kernel's matrix-core seed, with ties to a sampled row and NaN rows
    nt = 60_000
    rng = np.random.default_rng(d + (7 if metric == "cosine" else 0))
    if metric == "cosine":
        xq, xt = rng.random((96, d)), rng.random((nt, d))
    else:
        xq, xt = rng.standard_normal((96, d)), rng.standard_normal((nt, d))
    m = min(nt, max(512, min(2048, nt // 512, 64 * 16)))
    s1 = 2 * nt // m
    for r in (3, 4, nt - 1):
        xt[r] = xt[s1]
    xt[11, 5] = np.nan
    xq[0] = xt[s1]
    xq[1] = xt[s1] * (1.0 + 1e-15)
    wd, wi = oracle.knn_topk(xq, xt, 16, metric)
    gd, gi = _fused(xq, xt, 16, metric)
    _same(gd, gi, wd, wi, "f64 %s d=%d" % (metric, d))
