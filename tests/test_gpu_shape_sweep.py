"""GPU parity over a seeded sweep of shapes on the fused (Gram) path: f32 and
f64, Euclidean and cosine, d from 2 to 256 (16-byte rows and not, so both
the matrix-core and the exact seed run), k from 1 to 128, index and query
counts that leave partial tiles and several segments, with duplicated rows
(exact ties, lowest index first) and NaN rows planted in every case.  Each
case is bit for bit against the CPU oracle (the reference's brute-force
kNN, crates/mlrs-backend/src/prims/knn_host.rs and
crates/mlrs-kernels/src/knn.rs)."""
import numpy as np
import pytest
import torch

import oracle
from mlrs_amd import prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _case(i):
    rng = np.random.default_rng(1000 + i)
    dtype = np.float32 if i % 3 else np.float64
    metric = "cosine" if i % 4 == 1 else "euclidean"
    d = int(rng.choice([2, 3, 5, 8, 17, 24, 33, 64, 70, 100, 128, 129, 160, 200, 255, 256]))
    k = int(rng.choice([1, 2, 5, 16, 32, 33, 64, 65, 100, 128]))
    nt = int(rng.integers(max(k, 2000), 80000))
    nq = int(rng.integers(1, 200))
    return i, dtype, metric, d, k, nt, nq


CASES = [_case(i) for i in range(48)]


@pytest.mark.parametrize("case", CASES, ids=["%d-%s-%s-d%d-k%d" % (c[0], np.dtype(c[1]).name, c[2], c[3], c[4])
                                              for c in CASES])
def test_fused_shape_sweep(case):
    i, dtype, metric, d, k, nt, nq = case
    rng = np.random.default_rng(7 * i + 1)
    if metric == "cosine":
        xt, xq = rng.random((nt, d)), rng.random((nq, d))
    else:
        xt, xq = rng.standard_normal((nt, d)), rng.standard_normal((nq, d))
    xt, xq = xt.astype(dtype), xq.astype(dtype)
    xt[nt // 3] = xt[nt - 1]          # exact ties
    xt[nt // 2] = xt[nt - 1]
    xt[5 % nt, 0] = np.nan            # never admitted
    xq[0] = xt[nt - 1]                # a query on the tied point
    wd, wi = oracle.knn_topk(xq, xt, k, metric)
    prims.force_path("fused")
    try:
        gd, gi = prims.knn_topk(torch.from_numpy(xq).to(DEV), torch.from_numpy(xt).to(DEV), k, metric)
        torch.cuda.synchronize()
    finally:
        prims.force_path("auto")
    gd, gi = gd.cpu().numpy(), gi.cpu().numpy()
    bad = np.argwhere(gi != wi.astype(np.int64))
    assert bad.size == 0, "case %s: %d index mismatches, first %s" % (case, len(bad), bad[:3].tolist())
    same = (gd == wd) | (np.isnan(gd) & np.isnan(wd))
    assert same.all(), "case %s: distance bits differ at %s" % (case, np.argwhere(~same)[:3].tolist())
