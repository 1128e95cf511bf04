"""GPU: the X-vs-X graph ranks by the final distance, as the host scans'
KNearest does (crates/mlrs-algos/src/manifold/umap_host_knn.rs:171-198, 494).

tests/rooted_ties.py builds rows whose aggregates differ by one ulp but root
to the same double, the larger aggregate at the lower index: at the k-th
boundary, inside the list, and in a tie group larger than a list keeps (which
sends the Gram kernel's flagged queries through the root fill).  The device
graph must equal the oracle's lists: indices everywhere, values bit for bit
for Euclidean; Minkowski values within 4 ulp (the device pow rounds some
exact fourth roots, e.g. 0.09375, one ulp away from the host C library).
Both kernel families: the f64 Gram kernel (forced; Minkowski always takes the
exact tiles) and the exact tiles.
"""
import numpy as np
import pytest
import torch

import oracle
import rooted_ties
from mlrs_amd import prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(params=["fused", "generic"])
def family(request):
    prims.force_path(request.param)
    yield request.param
    prims.force_path("auto")


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("metric", ["euclidean", "minkowski"])
@pytest.mark.parametrize("k", [6, 10, 20, 32])
@pytest.mark.parametrize("include_self", [False, True])
def test_graph_rooted_ties(family, dtype, metric, k, include_self):
    x, p = rooted_ties.build(metric, k)
    want_i, want_d = oracle.knn_graph(x, k, metric, p=p, include_self=include_self)
    agg_i, _ = rooted_ties.brute_graph(x, k, metric, p, by_root=False, include_self=include_self)
    assert not np.array_equal(want_i, agg_i)
    xt = torch.from_numpy(np.ascontiguousarray(x.astype(dtype))).to(DEV)
    gi, gd = prims.knn_graph(xt, k, metric, p=p, include_self=include_self)
    torch.cuda.synchronize()
    gi, gd = gi.cpu().numpy(), gd.cpu().numpy()
    np.testing.assert_array_equal(gi, want_i.astype(np.int64))
    if metric == "euclidean":
        np.testing.assert_array_equal(gd, want_d)
    else:
        np.testing.assert_allclose(gd, want_d, rtol=4 * np.finfo(np.float64).eps, atol=0)


@pytest.mark.parametrize("k", [6, 20])
def test_core_distances_rooted_ties(family, k):
    """Core distances are column k-1 of the self-inclusive lists: the k-th
    smallest root, the same value under either ranking."""
    x, _ = rooted_ties.build("euclidean", k)
    want = oracle.core_distances(x, k, "euclidean")
    got = prims.core_distances(torch.from_numpy(x).to(DEV), k, "euclidean").cpu().numpy()
    np.testing.assert_array_equal(got, want)
