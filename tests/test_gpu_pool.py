"""The fit-time device copy (mlrs_device_copy_*) and the buffer counters
(mlrs_pool_stats_*): the search, assignment, pairwise and graph paths read
nothing back to the host (the reference's memory gate asserts read_backs == 0
across device-resident prims, e.g. crates/mlrs-backend/tests/laplacian_test.rs:
266-276), the radius search reads back its total, and cached buffers are
reused rather than reallocated across calls of one shape.  Growing a cached
buffer waits for nothing outside the call's own stream order: a search that
grows the workspace returns while an unrelated stream is still busy, and its
results are the oracle's."""
import numpy as np
import pytest
import torch

from mlrs_amd import _lib, prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("n,offset", [(1, 0), (3, 0), (1000003, 0), (1000003, 1), (777, 3), (4096, 2)])
def test_device_copy(dtype, n, offset):
    g = torch.Generator(device="cpu").manual_seed(n + offset)
    base = torch.randn(n + offset + 5, generator=g, dtype=dtype).to(DEV)
    src = base[offset:offset + n]
    dst_base = torch.full((n + 7,), -7.0, dtype=dtype, device=DEV)
    dst = dst_base[2:2 + n] if offset else dst_base[:n]
    prims.device_copy(src, out=dst)
    torch.cuda.synchronize()
    assert torch.equal(dst, src)
    # nothing past the destination is touched
    rest = torch.cat([dst_base[:2], dst_base[2 + n:]]) if offset else dst_base[n:]
    assert torch.all(rest == -7.0)
    c = prims.device_copy(src)
    assert torch.equal(c, src) and c.data_ptr() != src.data_ptr()


def test_search_paths_read_nothing_back():
    g = torch.Generator(device="cpu").manual_seed(1)
    xt = torch.randn((20000, 64), generator=g).to(DEV)
    xq = torch.randn((500, 64), generator=g).to(DEV)
    c = torch.randn((40, 64), generator=g).to(DEV)
    prims.knn_topk(xq, xt, 16)                    # grows the buffers once
    torch.cuda.synchronize()
    prims.pool_stats_reset()
    before = prims.pool_stats()
    for _ in range(3):
        prims.knn_topk(xq, xt, 16)
    prims.kmeans_assign(xt, c)
    prims.pairwise_distance(xq, c, "cosine")
    prims.knn_graph(xq.double(), 5)
    torch.cuda.synchronize()
    after = prims.pool_stats()
    assert after["read_backs"] == before["read_backs"] == 0
    assert after["reuses"] >= 3
    assert after["live_bytes"] > 0 and after["peak_bytes"] >= after["live_bytes"]
    prims.radius_neighbors(xq, xt, 9.0)
    assert prims.pool_stats()["read_backs"] > 0


def test_estimator_fit_owns_its_rows():
    # Fit::fit copies the training rows (prims/knn.rs:358-386): writing into
    # the caller's tensor afterwards changes nothing the estimator answers
    import oracle
    from mlrs_amd.neighbors import NearestNeighbors
    rng = np.random.default_rng(5)
    xt = rng.standard_normal((3000, 24)).astype(np.float32)
    xq = rng.standard_normal((200, 24)).astype(np.float32)
    dt = torch.from_numpy(xt).to(DEV)
    nn = NearestNeighbors(n_neighbors=7).fit(dt)
    assert nn._fit_X_dev.data_ptr() != dt.data_ptr()
    dt.fill_(0.0)
    dist, idx = nn.kneighbors(xq)
    wd, wi = oracle.knn_topk(xq, xt, 7)
    np.testing.assert_array_equal(np.asarray(idx), wi.astype(np.int32))
    np.testing.assert_array_equal(np.asarray(dist), wd)


def test_growth_does_not_wait_for_other_streams():
    """The workspace grows in stream order (the old buffer returned and the
    new one taken on the calling stream) while another stream runs ~0.3 s of
    unrelated matrix products: the call returns with that stream still busy."""
    import oracle
    _lib.check(_lib.load().mlrs_release_workspace())
    rng = np.random.default_rng(11)
    xt = rng.standard_normal((60000, 32)).astype(np.float32)
    xq = rng.standard_normal((2000, 32)).astype(np.float32)
    xt[9] = xt[4]  # a tie
    work = torch.cuda.Stream()
    mine = torch.cuda.Stream()
    with torch.cuda.stream(mine):
        dq, dt = torch.from_numpy(xq).to(DEV), torch.from_numpy(xt).to(DEV)
        small_d = torch.empty((100, 5), dtype=torch.float32, device=DEV)
        small_i = torch.empty((100, 5), dtype=torch.int32, device=DEV)
        out_d = torch.empty((2000, 10), dtype=torch.float32, device=DEV)
        out_i = torch.empty((2000, 10), dtype=torch.int32, device=DEV)
        prims.force_path("generic")
        try:
            prims.knn_topk(dq[:100], dt[:3000], 5, out=(small_d, small_i))  # a small workspace
            torch.cuda.synchronize()
            a = torch.randn((4096, 4096), device=DEV)
            torch.cuda.synchronize()
            with torch.cuda.stream(work):
                for _ in range(200):
                    a = torch.mm(a, a) * 1e-3
            before = prims.pool_stats()["allocations"]
            # an exact tile of 2000 x 60000 values (capped at 256 MB) grows it
            prims.knn_topk(dq, dt, 10, out=(out_d, out_i))
            busy = not work.query()
            grew = prims.pool_stats()["allocations"] > before
        finally:
            prims.force_path("auto")
    torch.cuda.synchronize()
    assert grew, "the search did not grow the workspace"
    assert busy, "the call waited for the other stream"
    wd, wi = oracle.knn_topk(xq, xt, 10)
    np.testing.assert_array_equal(out_i.cpu().numpy().astype(np.int64), wi.astype(np.int64))
    np.testing.assert_array_equal(out_d.cpu().numpy(), wd)
