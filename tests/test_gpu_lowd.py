"""GPU parity of the low-d ALU kNN path (knn_lowd.hip) in f32 and f64, bit for
bit against the CPU oracle (euclidean_topk_rows_cpu_direct,
crates/mlrs-kernels/src/knn.rs:2968-3227: the exact value fma(q-x, q-x, acc)
over ascending columns, lists ranked by (value, index) with insert_lane's
rule, knn.rs:2655-2706, NaN never admitted; cosine by the metric arm's
fold: fma dot product, sqrt(||q||^2 ||x||^2), divide, clamp to [0, 2]).

Every d from 1 to 16 and every list capacity (k = 1, 4, 8, 16, 32 and values
between) is reached; index sizes that split the rows into several strips
exercise the strip merge and the shared per-query bound; the edge cases are
exact duplicates around the k-th slot (the lower index wins), NaN rows and
queries, infinite coordinates, values whose squared norms overflow (the screen
bound becomes infinite and every row is evaluated exactly), subnormal
coordinates, zero rows and k = n_train.  The family is forced (the automatic
choice sends some f32 shapes to the Gram kernel, which is faster there), and
each case checks, through the library's timing hook, that the low-d kernel
served it."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from mlrs_amd import _lib, prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
DTYPES = [np.float32, np.float64]


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _knn_served(xq, xt, k, metric):
    """The engine's (distances, indices) and the name of the kernel it timed."""
    lib = _lib.load()
    _lib.check(lib.mlrs_timing_enable(1))
    prims.force_path("lowd")
    try:
        gd, gi = prims.knn_topk(_t(xq), _t(xt), k, metric)
        torch.cuda.synchronize()
        tot, n = ctypes.c_double(), ctypes.c_int64()
        name = ctypes.create_string_buffer(64)
        _lib.check(lib.mlrs_timing_read(ctypes.byref(tot), ctypes.byref(n), name, 64))
    finally:
        prims.force_path("auto")
        _lib.check(lib.mlrs_timing_enable(0))
    return gd.cpu().numpy(), gi.cpu().numpy(), name.value.decode()


def check_lowd(xq, xt, k, label="", metric="euclidean"):
    gd, gi, kern = _knn_served(xq, xt, k, metric)
    assert kern == "knn_lowd_kernel", "%s: served by %s" % (label, kern)
    wd, wi = oracle.knn_topk(xq, xt, k, metric)
    bad = np.argwhere(gi != wi.astype(np.int64))
    assert bad.size == 0, "%s: %d index mismatches, first %s" % (label, len(bad), bad[:3].tolist())
    same = (gd == wd) | (np.isnan(gd) & np.isnan(wd))
    assert same.all(), "%s: distance bits differ at %s" % (label, np.argwhere(~same)[:3].tolist())
    return gd, gi


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", list(range(1, 17)))
def test_every_width(dtype, d):
    rng = np.random.default_rng(500 + d)
    xt = rng.standard_normal((3000, d)).astype(dtype)
    xq = rng.standard_normal((700, d)).astype(dtype)
    check_lowd(xq, xt, 8, "d=%d %s" % (d, np.dtype(dtype).name))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("k", [1, 2, 4, 5, 8, 9, 16, 17, 31, 32])
@pytest.mark.parametrize("d", [2, 7, 16])
def test_list_capacities(dtype, k, d):
    rng = np.random.default_rng(600 + k + d)
    xt = rng.random((2500, d)).astype(dtype)
    xq = rng.random((513, d)).astype(dtype)
    check_lowd(xq, xt, k, "k=%d d=%d" % (k, d))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", [(300, 200000, 3, 8), (1000, 120000, 2, 32), (64, 90000, 16, 16),
                                  (2000, 60000, 5, 1)])
def test_strip_merge(dtype, case):
    """Few query blocks over a long index: the rows split into strips, each
    with its own list, merged at the end; later strips start from the bound
    the earlier ones published."""
    nq, nt, d, k = case
    rng = np.random.default_rng(nq + nt)
    xt = rng.standard_normal((nt, d)).astype(dtype)
    xq = rng.standard_normal((nq, d)).astype(dtype)
    check_lowd(xq, xt, k, str(case))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("k", [4, 32])
def test_duplicates_at_the_kth_slot(dtype, k):
    """Forty copies of one row straddle the k-th slot, in several strips:
    membership and order are decided by index alone."""
    rng = np.random.default_rng(7)
    xt = rng.standard_normal((100000, 3)).astype(dtype)
    dup = np.array([11, 20000, 20001, 45000, 70000, 99999] + list(range(300, 334)))
    xt[dup] = xt[11]
    xq = np.concatenate([xt[11:12], rng.standard_normal((300, 3)).astype(dtype)])
    gd, gi = check_lowd(xq, xt, k, "dups k=%d" % k)
    assert gi[0].tolist() == sorted(dup.tolist())[:k]
    assert np.all(gd[0] == 0)


@pytest.mark.parametrize("dtype", DTYPES)
def test_nan_and_inf(dtype):
    rng = np.random.default_rng(9)
    xt = rng.standard_normal((5000, 4)).astype(dtype)
    xq = rng.standard_normal((400, 4)).astype(dtype)
    xt[[3, 2500, 4999]] = np.nan          # NaN rows are never admitted
    xt[[10, 11]] = np.inf                 # +inf coordinates: infinite or NaN exact values
    xt[12, 1] = -np.inf
    xq[5] = np.nan                        # a NaN query admits nothing: sentinel rows
    xq[6, 2] = np.inf
    check_lowd(xq, xt, 8, "nan/inf")


@pytest.mark.parametrize("dtype,scale", [(np.float32, 1e18), (np.float64, 1e155)])
def test_overflowing_norms(dtype, scale):
    """Squared norms overflow the element type: the screen bound becomes
    infinite and every row is evaluated exactly, still the reference's bits."""
    rng = np.random.default_rng(13)
    xt = (rng.standard_normal((3000, 5)) * scale).astype(dtype)
    xq = (rng.standard_normal((200, 5)) * scale).astype(dtype)
    xt[:10] *= dtype(100)
    check_lowd(xq, xt, 6, "huge")


@pytest.mark.parametrize("dtype,scale", [(np.float32, 1e-20), (np.float64, 1e-160)])
def test_subnormal_distances(dtype, scale):
    """Squared distances in the subnormal range: the screen's absolute term
    keeps every candidate."""
    rng = np.random.default_rng(17)
    xt = (rng.standard_normal((4000, 3)) * scale).astype(dtype)
    xq = (rng.standard_normal((300, 3)) * scale).astype(dtype)
    check_lowd(xq, xt, 8, "tiny")


@pytest.mark.parametrize("dtype", DTYPES)
def test_zero_rows_and_k_equals_n_train(dtype):
    rng = np.random.default_rng(19)
    xt = rng.integers(-2, 3, size=(32, 6)).astype(dtype)
    xt[[0, 5]] = 0
    xq = rng.integers(-2, 3, size=(100, 6)).astype(dtype)
    xq[:3] = 0
    check_lowd(xq, xt, 32, "k = n_train")
    check_lowd(xq, xt, 1, "k = 1 on quantised rows")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [1, 2, 3, 5, 8, 11, 16])
@pytest.mark.parametrize("k", [1, 8, 16, 32])
def test_cosine(dtype, d, k):
    rng = np.random.default_rng(700 + d + k)
    xt = (rng.standard_normal((3000, d)) + 0.3).astype(dtype)
    xq = (rng.standard_normal((600, d)) + 0.3).astype(dtype)
    check_lowd(xq, xt, k, "cosine d=%d k=%d" % (d, k), "cosine")


@pytest.mark.parametrize("dtype", DTYPES)
def test_cosine_strips_ties_zero_and_nan(dtype):
    """Rows that are positive multiples of one direction lead the list of a
    query along it (the ties among them go by index, across strips); zero rows
    score exactly 1; a zero query scores 1 against every row (its norm
    product is 0 or NaN, so the arm's similarity is 0) and is never screened;
    NaN and inf rows are otherwise never admitted; a NaN query admits
    nothing."""
    rng = np.random.default_rng(23)
    xt = rng.standard_normal((80000, 3)).astype(dtype)
    base = xt[17].copy()
    same = np.array([17, 300, 301, 40000, 79999])
    xt[same] = base * np.array([1, 2, 3, 0.5, 7], dtype=dtype)[:, None]
    xt[[5, 60000]] = 0
    xt[[6, 70000]] = np.nan
    xt[7, 1] = np.inf
    xq = rng.standard_normal((300, 3)).astype(dtype)
    xq[0] = base
    xq[1] = 0
    xq[2] = np.nan
    gd, gi = check_lowd(xq, xt, 8, "cosine ties", "cosine")
    assert set(same.tolist()) <= set(gi[0].tolist())
    assert (gd[1] == 1).all()  # the zero query scores 1 against every row


@pytest.mark.parametrize("dtype,scale", [(np.float32, 1e20), (np.float64, 1e160), (np.float32, 1e-20),
                                         (np.float64, 1e-160)])
def test_cosine_extreme_norms(dtype, scale):
    """Norm sums that overflow (the query is evaluated exactly against every
    row) or underflow."""
    rng = np.random.default_rng(29)
    xt = (rng.standard_normal((3000, 4)) * scale).astype(dtype)
    xq = (rng.standard_normal((200, 4)) * scale).astype(dtype)
    check_lowd(xq, xt, 8, "cosine scale %g" % scale, "cosine")
