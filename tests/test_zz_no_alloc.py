"""The allocation-free kNN entry point (mlrs_knn_topk_f32_noalloc) against
the allocating one (mlrs_knn_topk_f32), bit for bit, through the C ABI.

Each case makes two calls in a row, the second with a smaller input, so the
static scratch is reused with the first call's contents still in it.  The
three kernel families (fused Gram, low-d, exact tiles) are each reached, and
the library's buffer counters (allocations, reuses, live bytes) must not move
across an allocation-free call: the cached buffers are never touched.  A
search whose scratch would exceed MLRS_NOALLOC_SCRATCH_BYTES is rejected
before any launch.  Calls captured into a HIP graph (torch.cuda.CUDAGraph,
after a first call with n_query = 0 outside the capture) replay with new data
in place, each replay bit-equal to the allocating entry point.
"""
import ctypes

import numpy as np
import pytest
import torch

from mlrs_amd import _lib, prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _call(name, xq, xt, k, metric=0):
    nq, d = xq.shape
    nt = xt.shape[0]
    dist = torch.full((nq, k), -1.0, dtype=torch.float32, device=DEV)
    idx = torch.full((nq, k), -1, dtype=torch.int32, device=DEV)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    rc = getattr(_lib.load(), name)(xq.data_ptr(), xq.numel(), nq, d, xt.data_ptr(), xt.numel(), nt, k, metric, 2.0,
                                   dist.data_ptr(), idx.data_ptr(), dist.numel(), stream)
    return rc, dist, idx


def _counters():
    st = prims.pool_stats()
    return st["allocations"], st["reuses"], st["live_bytes"]


def _both(xq, xt, k, metric=0):
    rc, d0, i0 = _call("mlrs_knn_topk_f32", xq, xt, k, metric)
    _lib.check(rc)
    before = _counters()
    rc, d1, i1 = _call("mlrs_knn_topk_f32_noalloc", xq, xt, k, metric)
    _lib.check(rc)
    assert _counters() == before, "the allocation-free call touched the cached buffers"
    torch.cuda.synchronize()
    assert torch.equal(i0, i1), "indices differ"
    assert torch.equal(d0.view(torch.int32), d1.view(torch.int32)), "distance bits differ"


def _rand(seed, n, d):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn((n, d), generator=g, dtype=torch.float32).to(DEV)


# (family forced, first call (nq, nt, d, k, metric), second smaller call)
CASES = [
    ("fused", (3000, 200000, 128, 32, 0), (700, 50000, 96, 10, 0)),
    ("fused", (2048, 120000, 64, 1, 0), (100, 9000, 64, 1, 0)),
    ("fused", (5000, 3000, 64, 1, 0), (700, 1000, 32, 1, 0)),  # k = 1 with the index resident in LDS
    ("fused", (1500, 80000, 100, 20, 1), (300, 20000, 100, 5, 1)),
    ("lowd", (20000, 200000, 3, 8, 0), (5000, 40000, 3, 8, 0)),
    ("generic", (1000, 10000, 64, 10, 0), (200, 3000, 64, 10, 0)),
    ("generic", (400, 30000, 200, 300, 0), (50, 9000, 200, 257, 1)),
]


@pytest.mark.parametrize("family,first,second", CASES)
def test_noalloc_matches_allocating_entry_point(family, first, second):
    prims.force_path(family)
    try:
        for j, (nq, nt, d, k, metric) in enumerate((first, second)):
            seed = 100 * j + nq + d
            xq, xt = _rand(seed, nq, d), _rand(seed + 1, nt, d)
            xt[5] = xt[2]  # a tie
            _both(xq, xt, k, metric)
    finally:
        prims.force_path("auto")


def test_noalloc_rejects_scratch_beyond_its_size():
    # 150k queries against a 1M-row index on the Gram path need ~176 MiB of
    # norms, per-segment lists and queued screen values: rejected before any
    # launch (the inputs are never read).
    xq = torch.empty((150000, 128), dtype=torch.float32, device=DEV)
    xt = torch.empty((1000000, 128), dtype=torch.float32, device=DEV)
    prims.force_path("fused")
    try:
        rc, _, _ = _call("mlrs_knn_topk_f32_noalloc", xq, xt, 32)
    finally:
        prims.force_path("auto")
    assert rc == _lib.MLRS_ERR_UNSUPPORTED
    info = _lib.ErrorInfo()
    _lib.load().mlrs_last_error(ctypes.byref(info))
    assert info.operand == b"scratch" and info.len == _lib.NOALLOC_SCRATCH_BYTES and info.rows > info.len
    # the device is untouched and usable afterwards
    xq2, xt2 = _rand(1, 300, 128), _rand(2, 30000, 128)
    _both(xq2, xt2, 32)


@pytest.mark.parametrize("family,shape", [("fused", (1200, 60000, 128, 32)), ("fused", (1000, 40000, 64, 1)),
                                          ("fused", (4000, 1500, 64, 1)),
                                          ("lowd", (4000, 50000, 3, 8)), ("generic", (300, 5000, 64, 10))])
def test_noalloc_graph_capture_replays(family, shape):
    nq, nt, d, k = shape
    prims.force_path(family)
    try:
        xq, xt = _rand(nq + d, nq, d), _rand(nt + d, nt, d)
        dist = torch.full((nq, k), -1.0, dtype=torch.float32, device=DEV)
        idx = torch.full((nq, k), -1, dtype=torch.int32, device=DEV)
        lib = _lib.load()

        def call():
            s = torch.cuda.current_stream(DEV).cuda_stream
            return lib.mlrs_knn_topk_f32_noalloc(xq.data_ptr(), xq.numel(), nq, d, xt.data_ptr(), xt.numel(), nt,
                                                 k, 0, 2.0, dist.data_ptr(), idx.data_ptr(), dist.numel(), s)

        # set-up outside the capture: a call with no queries
        _lib.check(lib.mlrs_knn_topk_f32_noalloc(xq.data_ptr(), 0, 0, d, xt.data_ptr(), xt.numel(), nt, k, 0, 2.0,
                                                  dist.data_ptr(), idx.data_ptr(), 0,
                                                  torch.cuda.current_stream(DEV).cuda_stream))
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        rcs = []
        with torch.cuda.graph(g):
            rcs.append(call())
        assert rcs == [0]
        for rep in range(3):
            # new data in the captured buffers, written by eager work
            xq.copy_(_rand(1000 + rep, nq, d))
            xt.copy_(_rand(2000 + rep, nt, d))
            xt[7] = xt[3]  # a tie
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            rc, d0, i0 = _call("mlrs_knn_topk_f32", xq, xt, k)
            _lib.check(rc)
            torch.cuda.synchronize()
            assert torch.equal(i0, idx), "indices differ on replay %d" % rep
            assert torch.equal(d0.view(torch.int32), dist.view(torch.int32)), "distance bits differ on replay %d" % rep
        del g
    finally:
        prims.force_path("auto")
