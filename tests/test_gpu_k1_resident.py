"""GPU parity of the k = 1 search with the index resident in LDS
(knn_k1_resident.hip), bit for bit against the CPU oracle: the k-means
assignment (argmin_dist_rows, crates/mlrs-kernels/src/kmeans.rs:284-310:
squared distance by mul + add, lowest index on a tie, a NaN distance to
centre 0 wins) and the k = 1 nearest neighbour (crates/mlrs-backend/src/
prims/knn_host.rs, lowest index on a tie).

The index is cut into chunks of at most 512 rows at d <= 64 (992 at d <= 32),
one per workgroup, and each query's best over the chunks is merged by
(value, index).  The cases put the chunk boundaries at 511/512/513 rows and at
eight full chunks (the most the path takes; nine go to the fused kernel),
exact ties between rows of different chunks (the lower index must win the
merge), NaN rows in a later chunk, NaN queries, padded feature columns
(d = 4, 36, 60), query counts that leave a partial block of 32, and norms
large enough that screen sums may overflow (those waves screen by compare and
never drop a queue).  Each case also checks, through the library's timing
hook, which kernel served it."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from mlrs_amd import _lib, prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _served_by(fn):
    """Run fn with the timing hook on; return the kernel it timed."""
    lib = _lib.load()
    _lib.check(lib.mlrs_timing_enable(1))
    try:
        out = fn()
        torch.cuda.synchronize()
        tot, n = ctypes.c_double(), ctypes.c_int64()
        name = ctypes.create_string_buffer(64)
        _lib.check(lib.mlrs_timing_read(ctypes.byref(tot), ctypes.byref(n), name, 64))
    finally:
        _lib.check(lib.mlrs_timing_enable(0))
    return out, name.value.decode()


def _assign(x, c):
    (lab, sq), kern = _served_by(lambda: prims.kmeans_assign(_t(x), _t(c)))
    wl, ws = oracle.kmeans_assign(x, c)
    np.testing.assert_array_equal(lab.cpu().numpy(), wl.astype(np.int64))
    np.testing.assert_array_equal(sq.cpu().numpy(), ws)
    return lab.cpu().numpy(), sq.cpu().numpy(), kern


def _blobs(seed, n, kc, d, spread=3.0):
    rng = np.random.default_rng(seed)
    c = (rng.standard_normal((kc, d)) * spread).astype(np.float32)
    x = (c[rng.integers(0, kc, n)] + rng.standard_normal((n, d))).astype(np.float32)
    return x, c


@pytest.mark.parametrize("kc", [1, 31, 511, 512, 513, 1024, 1500, 4096])
def test_assign_chunk_boundaries(kc):
    x, c = _blobs(kc, max(3000, kc + 1000), kc, 64)
    _, _, kern = _assign(x, c)
    assert kern == "knn_k1_resident_f32_kernel"


def test_assign_past_eight_chunks_takes_the_fused_kernel():
    x, c = _blobs(5, 5000, 4097, 64)
    _, _, kern = _assign(x, c)
    assert kern == "knn_gram_f32_kernel"


@pytest.mark.parametrize("d", [4, 8, 32, 36, 60, 64])
@pytest.mark.parametrize("n", [1000, 4133])
def test_assign_widths_and_partial_blocks(d, n):
    x, c = _blobs(d + n, n, 700, d)
    _, _, kern = _assign(x, c)
    assert kern == "knn_k1_resident_f32_kernel"


def test_assign_ties_across_chunks_and_nan():
    x, c = _blobs(11, 4000, 1100, 64)
    c[700] = c[100]          # chunk 1 copies a row of chunk 0: index 100 must win
    c[1090] = c[600]         # chunk 2 copies a row of chunk 1: index 600 must win
    c[900] = np.nan          # a NaN centre in chunk 1 is never nearest
    x[:50] = c[100]
    x[50:100] = c[600]
    x[100:110] = np.nan      # NaN points: the centre-0 rule
    lab, sq, kern = _assign(x, c)
    assert kern == "knn_k1_resident_f32_kernel"
    assert (lab[:50] == 100).all() and (lab[50:100] == 600).all()
    assert (lab[100:110] == 0).all() and np.isnan(sq[100:110]).all()


def test_assign_many_equal_centres_across_chunks():
    """600 identical centres over two chunks: every row of those tiles passes
    the screen, the queues flush inside the tile loop, the lowest index wins."""
    rng = np.random.default_rng(21)
    c = rng.standard_normal((1000, 48)).astype(np.float32)
    c[300:900] = c[7]
    x = rng.standard_normal((2500, 48)).astype(np.float32)
    x[::3] = c[7]
    m = len(x[1::3])
    x[1::3] = c[7] + np.float32(1e-3) * rng.standard_normal((m, 48)).astype(np.float32)
    lab, _, kern = _assign(x, c)
    assert kern == "knn_k1_resident_f32_kernel"
    assert (lab[::3] == 7).all()


def test_assign_overflowing_norms():
    x, c = _blobs(13, 2000, 800, 64)
    x[:40] *= np.float32(3e18)
    c[600:610] *= np.float32(3e18)
    _, _, kern = _assign(x, c)
    assert kern == "knn_k1_resident_f32_kernel"


@pytest.mark.parametrize("d", [16, 32, 64])
def test_knn_k1(d):
    """The k = 1 nearest neighbour (the search's own arm for the shape),
    with the fused family forced as small searches would take the exact
    tiles."""
    rng = np.random.default_rng(40 + d)
    xt = rng.standard_normal((1300, d)).astype(np.float32)
    xq = rng.standard_normal((999, d)).astype(np.float32)
    xt[1200] = xt[50]
    xq[:5] = xt[50]
    xt[800] = np.nan
    prims.force_path("fused")
    try:
        (gd, gi), kern = _served_by(lambda: prims.knn_topk(_t(xq), _t(xt), 1, "euclidean"))
    finally:
        prims.force_path("auto")
    assert kern == "knn_k1_resident_f32_kernel"
    wd, wi = oracle.knn_topk(xq, xt, 1, "euclidean")
    np.testing.assert_array_equal(gi.cpu().numpy(), wi.astype(np.int64))
    np.testing.assert_array_equal(gd.cpu().numpy(), wd)
    assert (gi.cpu().numpy()[:5, 0] == 50).all()
