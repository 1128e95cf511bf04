"""Calls on different streams, back to back with no host synchronization in
between: each call's stream waits for the previous call's work, because all
calls on a device share the library's cached buffers (the reference runs one
stream, crates/mlrs-backend/src/stream_cap.rs:69).  Every result is compared
with the CPU oracle bit for bit.
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


def _same(got, want):
    got = got.cpu().numpy()
    want = np.asarray(want)
    if want.dtype == np.uint32:
        want = want.astype(np.int64)
    assert np.array_equal(got, want), np.argwhere(got != want)[:3].tolist()


def test_two_streams_knn_then_knn():
    rng = np.random.default_rng(11)
    # A: a fused search long enough to still run when B is enqueued; B: another
    # shape whose norms and lists land on the same workspace offsets
    xa_q = rng.standard_normal((2048, 64)).astype(np.float32)
    xa_t = rng.standard_normal((120000, 64)).astype(np.float32)
    xb_q = rng.standard_normal((700, 128)).astype(np.float32)
    xb_t = rng.standard_normal((40000, 128)).astype(np.float32)
    da_q, da_t, db_q, db_t = _t(xa_q), _t(xa_t), _t(xb_q), _t(xb_t)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s1):
        ra = prims.knn_topk(da_q, da_t, 32)
    with torch.cuda.stream(s2):
        rb = prims.knn_topk(db_q, db_t, 16)
    torch.cuda.synchronize()
    wa = oracle.knn_topk(xa_q, xa_t, 32)
    wb = oracle.knn_topk(xb_q, xb_t, 16)
    _same(ra[0], wa[0])
    _same(ra[1], wa[1])
    _same(rb[0], wb[0])
    _same(rb[1], wb[1])


def test_two_streams_mixed_entry_points():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((60000, 32)).astype(np.float32)
    c = rng.standard_normal((300, 32)).astype(np.float32)
    g = rng.standard_normal((3000, 9)).astype(np.float64)
    q = rng.standard_normal((900, 32)).astype(np.float32)
    dx, dc, dg, dq = _t(x), _t(c), _t(g), _t(q)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s1):
        gi, gd = prims.knn_graph(dg, 12, "euclidean")          # auxiliary + main buffers
    with torch.cuda.stream(s2):
        lab, sq = prims.kmeans_assign(dx, dc)                   # main buffers, another shape
    with torch.cuda.stream(s1):
        kd, ki = prims.knn_topk(dq, dx, 8, "cosine")
    with torch.cuda.stream(s2):
        pw = prims.pairwise_distance(dq, dc, "cosine")
    torch.cuda.synchronize()
    wi, wd = oracle.knn_graph(g, 12, "euclidean")
    _same(gi, wi)
    _same(gd, wd)
    wl, ws = oracle.kmeans_assign(x, c)
    _same(lab, wl)
    _same(sq, ws)
    wkd, wki = oracle.knn_topk(q, x, 8, "cosine")
    _same(kd, wkd)
    _same(ki, wki)
    _same(pw, oracle.pairwise(q, c, "cosine"))
