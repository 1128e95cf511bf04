"""GPU parity of the k = 1 Gram kernel's candidate queue, bit for bit against
the CPU oracle (the reference's brute-force kNN with k = 1,
crates/mlrs-backend/src/prims/knn_host.rs; lowest index wins a tie).

With k = 1 the screen tightens on every index tile to the tile's smallest
screen value plus twice the error bound, and a queue whose rows all screen
above the tightened threshold is dropped before the tile's rows join it.
The cases below make that happen on nearly every tile (rows ordered by
falling distance to every query) and plant what must survive it: an exact
copy of the nearest row at a lower index on an earlier tile (the tie goes to
it), rows a rounding step away from the nearest on other tiles, NaN rows,
and norms large enough that screen values may overflow (no queue is dropped
then).  Both register shapes (d <= 128, 128 < d <= 256) and a row length
without 16-byte alignment are covered."""
import numpy as np
import pytest
import torch

import oracle
from mlrs_amd import prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _falling(seed, nq, nt, d, scale=1.0):
    """Index rows at falling distance from the origin along one direction,
    queries near the origin: the running nearest row improves on every tile."""
    rng = np.random.default_rng(seed)
    u = rng.standard_normal(d)
    u /= np.linalg.norm(u)
    t = np.linspace(40.0, 1.0, nt)[:, None]
    xt = (t * u[None, :] + 0.05 * rng.standard_normal((nt, d))) * scale
    xq = 0.05 * rng.standard_normal((nq, d)) * scale
    return xq.astype(np.float32), xt.astype(np.float32)


def _run(xq, xt, label):
    wd, wi = oracle.knn_topk(xq, xt, 1, "euclidean")
    prims.force_path("fused")
    try:
        gd, gi = prims.knn_topk(_t(xq), _t(xt), 1, "euclidean")
        torch.cuda.synchronize()
    finally:
        prims.force_path("auto")
    gd, gi = gd.cpu().numpy(), gi.cpu().numpy()
    bad = np.argwhere(gi != wi.astype(np.int64))
    assert bad.size == 0, "%s: %d index mismatches, first %s" % (label, len(bad), bad[:3].tolist())
    same = (gd == wd) | (np.isnan(gd) & np.isnan(wd))
    assert same.all(), "%s: distance bits differ at %s" % (label, np.argwhere(~same)[:3].tolist())
    return gi


@pytest.mark.parametrize("d", [24, 30, 64, 128, 200])
def test_k1_new_nearest_on_every_tile(d):
    xq, xt = _falling(d, 300, 20000, d)
    _run(xq, xt, "falling d=%d" % d)


@pytest.mark.parametrize("d", [64, 200])
def test_k1_tie_on_an_earlier_tile_wins(d):
    nq, nt = 260, 20000
    xq, xt = _falling(d + 1, nq, nt, d)
    best = nt - 1
    xt[5] = xt[best]              # same row, lower index, first tile
    xt[70] = xt[best]             # and on a later tile of the same segment
    xt[40, 3] = np.nan            # NaN rows on early tiles
    xt[best - 40, 0] = np.nan
    # rows a rounding step from the nearest, before and after it
    xt[100] = np.nextafter(xt[best], np.float32(np.inf))
    xt[best - 33] = xt[best] * np.float32(1.0000001)
    xq[0] = xt[best]              # queries on the nearest row itself
    xq[1] = xt[best] * np.float32(0.9999999)
    gi = _run(xq, xt, "ties d=%d" % d)
    assert gi[0, 0] == 5


def test_k1_large_norms_keep_queue():
    # squared norms past 2^124: screen values may overflow, so no query is in
    # screen-value mode and queues are only emptied by exact evaluation
    xq, xt = _falling(7, 200, 12000, 64, scale=np.float32(2.0 ** 57))
    assert float(np.max(np.sum(xt.astype(np.float64) ** 2, axis=1))) > 2.0 ** 124
    xt[3] = xt[11999]
    xq[0] = xt[11999]
    gi = _run(xq, xt, "large norms")
    assert gi[0, 0] == 3


def test_k1_queries_of_all_distances():
    # random data: records, flushes and ties as they come, several segments
    rng = np.random.default_rng(11)
    xt = rng.standard_normal((30011, 64)).astype(np.float32)
    xq = rng.standard_normal((1000, 64)).astype(np.float32)
    xt[29000] = xt[17]
    xq[:8] = xt[17]
    _run(xq, xt, "random")
