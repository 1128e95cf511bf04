"""GPU parity: the HIP engine against the CPU oracle, bit for bit.

Every case compares the C-ABI results (through mlrs_amd.prims) with
oracle/ (the restatement of the mlrs cpu-backend arithmetic) on the same
seeded inputs.  The bar is exact equality of distances and indices: the engine
evaluates every kept pair in the reference arm's own operation order, so no
tolerance is needed.  Every test runs twice: with the automatic kernel choice
(small searches take the exact-tile path, d <= 16 the low-d ALU kernel) and
with the fused Gram-MFMA kernels forced wherever they serve the shape, so the
edge cases below reach the fused kernels too.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import assert_topk_matches, load_golden
from mlrs_amd import prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(autouse=True, params=["auto", "fused"])
def kernel_family(request):
    prims.force_path(request.param)
    yield request.param
    prims.force_path("auto")


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def gpu_knn(xq, xt, k, metric="euclidean"):
    d, i = prims.knn_topk(_t(xq), _t(xt), k, metric)
    torch.cuda.synchronize()
    return d.cpu().numpy(), i.cpu().numpy()


def assert_same(got_d, got_i, want_d, want_i, label=""):
    bad = np.argwhere(got_i != want_i.astype(np.int64))
    assert bad.size == 0, "%s: %d index mismatches, first %s got %s want %s" % (
        label, len(bad), bad[:3].tolist(), got_i[tuple(bad[0])], want_i[tuple(bad[0])])
    same = (got_d == want_d) | (np.isnan(got_d) & np.isnan(want_d))
    assert same.all(), "%s: distance bits differ at %s" % (label, np.argwhere(~same)[:3].tolist())


def check_knn(xq, xt, k, metric="euclidean", label=""):
    gd, gi = gpu_knn(xq, xt, k, metric)
    wd, wi = oracle.knn_topk(xq, xt, k, metric)
    assert_same(gd, gi, wd, wi, label)
    return gd, gi


def _data(seed, nq, nt, d, dtype=np.float32, scale=1.0):
    rng = np.random.default_rng(seed)
    return ((rng.standard_normal((nq, d)) * scale).astype(dtype),
            (rng.standard_normal((nt, d)) * scale).astype(dtype))


# (nq, nt, d, k): low-d ALU path (d <= 16, k <= 32)
LOWD = [(300, 2000, 3, 8), (257, 1000, 1, 1), (100, 3000, 16, 32), (1000, 5000, 7, 16), (64, 20, 2, 20)]
# Gram-MFMA path (f32, 16 < d <= 128, k <= 64)
GRAM = [(300, 3000, 64, 10), (129, 1000, 17, 5), (500, 4000, 128, 32), (77, 600, 100, 64),
        (1000, 70000, 128, 32), (5, 100, 33, 1), (200, 2048, 24, 20), (1, 31, 40, 31), (130, 5000, 96, 7)]
# Gram-MFMA path, wide shape (f32, 128 < d <= 256: 16 queries per wave on
# 16x16x4 MFMAs; d not a multiple of 4 takes the element-wise loads)
GRAM_WIDE = [(300, 3000, 256, 10), (129, 1000, 129, 5), (500, 4000, 192, 32), (77, 600, 200, 64),
             (1000, 30000, 256, 32), (5, 100, 160, 1), (200, 2048, 255, 20), (1, 31, 136, 31),
             (130, 5000, 250, 7), (65, 3000, 256, 1), (70, 9000, 176, 16)]
# Gram-MFMA path with 64 < k <= 128 (lists of k + 32 entries in three
# 64-entry blocks), both shapes; large enough that the automatic choice takes
# the fused kernel too
GRAM_K128 = [(300, 20000, 64, 100), (500, 40000, 128, 128), (77, 9000, 100, 65), (130, 9000, 96, 96),
             (64, 5000, 200, 128), (200, 20000, 256, 80), (1, 300, 40, 128), (129, 1000, 17, 127),
             (40, 129, 33, 128)]
# generic exact path (k > 128, d > 256)
GENERIC = [(50, 500, 64, 100), (20, 300, 64, 200), (30, 400, 300, 10)]


@pytest.mark.parametrize("case", LOWD + GRAM + GRAM_WIDE + GRAM_K128 + GENERIC)
def test_f32_euclidean_bitwise(case):
    nq, nt, d, k = case
    xq, xt = _data(100 + d, nq, nt, d)
    check_knn(xq, xt, k, "euclidean", str(case))


@pytest.mark.parametrize("case", [(300, 3000, 64, 10), (100, 2000, 5, 7), (50, 500, 130, 8), (40, 400, 64, 80),
                                  (600, 20000, 128, 32), (300, 5000, 256, 16), (50, 2000, 150, 32),
                                  (129, 3000, 200, 1), (64, 1000, 193, 64), (300, 20000, 128, 100),
                                  (64, 5000, 193, 128), (100, 8000, 48, 65)])
def test_f32_cosine_bitwise(case):
    nq, nt, d, k = case
    xq, xt = _data(200 + d, nq, nt, d)
    xq += 0.3  # keep similarities away from the all-zero-mean regime
    check_knn(xq, xt, k, "cosine", str(case))


# f64: Gram-MFMA path for d <= 256, k <= 128 (direct, metric and knn_host arms;
# 64 < k <= 128 with lists in three 64-entry blocks), generic exact path beyond
F64 = [((100, 2000, 64, 10), "euclidean"), ((50, 1000, 3, 8), "euclidean"), ((64, 2000, 256, 16), "cosine"),
       ((40, 700, 20, 5), "cosine"), ((300, 30000, 256, 16), "cosine"), ((200, 5000, 200, 12), "euclidean"),
       ((77, 3000, 129, 64), "euclidean"), ((65, 2500, 33, 1), "cosine"), ((129, 4000, 128, 40), "cosine"),
       ((10, 400, 300, 7), "euclidean"), ((33, 900, 255, 3), "cosine"), ((1, 17, 17, 17), "euclidean"),
       ((100, 5000, 64, 100), "euclidean"), ((64, 4000, 256, 128), "cosine"), ((50, 3000, 200, 65), "euclidean"),
       ((30, 2000, 129, 127), "cosine"), ((300, 30000, 256, 96), "cosine"), ((40, 6000, 24, 128), "cosine")]


@pytest.mark.parametrize("case,metric", F64)
def test_f64_bitwise(case, metric):
    nq, nt, d, k = case
    rng = np.random.default_rng(300 + d)
    xq = rng.random((nq, d))
    xt = rng.random((nt, d))
    check_knn(xq, xt, k, metric, str(case))


@pytest.mark.parametrize("d", [3, 64, 128, 256])
@pytest.mark.parametrize("k", [32, 100])
def test_duplicates_and_boundary_ties(d, k):
    """100 identical rows around the k-th slot: membership and order are
    decided by index alone (knn_metric_kernel_test.rs:269-289)."""
    rng = np.random.default_rng(5)
    xt = rng.standard_normal((3000, d)).astype(np.float32)
    xt[500:600] = xt[7]            # 101 copies of row 7
    xq = np.concatenate([xt[7:8], xt[:50], rng.standard_normal((20, d)).astype(np.float32)])
    gd, gi = check_knn(xq, xt, k, "euclidean", "dups d=%d k=%d" % (d, k))
    assert gi[0].tolist() == [7] + list(range(500, 500 + k - 1))
    assert np.all(gd[0] == 0)


@pytest.mark.parametrize("d,k", [(3, 8), (48, 24), (208, 24), (48, 100), (208, 128)])
def test_quantized_data_many_ties(d, k):
    rng = np.random.default_rng(6)
    xt = rng.integers(-3, 4, size=(4000, d)).astype(np.float32)
    xq = rng.integers(-3, 4, size=(300, d)).astype(np.float32)
    check_knn(xq, xt, k, "euclidean", "quantized")
    check_knn(xq, xt, k, "cosine", "quantized cosine")


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("k", [1, 100])
def test_nan_rows_sign_screen(d, k):
    """The k = 1 and three-block-list kernels screen by the sign of
    (threshold - value) in waves whose queries all have finite screen sums:
    NaN index rows give NaN screen values, which that screen drops (their exact
    values are NaN, never kept), and the waves holding a NaN query keep the
    compare screen.  Both must give the reference's lists."""
    xq, xt = _data(15, 150, 3000, d)
    xt[[5, 1200, 2999]] = np.nan
    xt[40, 3] = np.nan
    xq[[1, 90]] = np.nan
    check_knn(xq, xt, k, "euclidean", "nan sign screen k=%d" % k)


@pytest.mark.parametrize("d", [4, 64, 200])
def test_nan_rows(d):
    xq, xt = _data(8, 200, 1500, d)
    xt[[3, 700, 1499]] = np.nan
    xt[10, 1] = np.nan
    xq[[0, 57]] = np.nan
    check_knn(xq, xt, 12, "euclidean", "nan")
    # fewer admissible rows than k -> sentinel (+inf, 0) slots
    small = xt[:8].copy()
    small[2] = np.nan
    check_knn(xq[:20], small, 8, "euclidean", "nan sentinel")


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("perturb", [0.0, 1e-4])
@pytest.mark.parametrize("k", [32, 120])
def test_near_ties_across_segments(perturb, d, k):
    """Copies of each query (exact, or perturbed far inside the screen's error
    window) spread through a large index, so they fall in different segments
    of the fused split: each segment's list and the final merge must resolve
    them by exact value, then index."""
    rng = np.random.default_rng(31)
    xt = rng.standard_normal((80000, d)).astype(np.float32)
    xq = rng.standard_normal((12, d)).astype(np.float32)
    for j in range(12):
        rows = np.arange(40) * 1999 + 17 * j + 5
        xt[rows] = xq[j] + perturb * rng.standard_normal((40, d)).astype(np.float32)
    check_knn(xq, xt, k, "euclidean", "near ties %g" % perturb)
    check_knn(xq, xt, k, "cosine", "near ties cosine %g" % perturb)


def test_cosine_nan_rows():
    """A NaN index row scores exactly 1 under the fold arm (its squared norm is
    NaN, so the similarity falls back to 0): it competes as a real row."""
    rng = np.random.default_rng(32)
    xt = rng.standard_normal((3000, 40)).astype(np.float32)
    xq = rng.standard_normal((64, 40)).astype(np.float32)
    xt = np.abs(xt)
    xt[[2, 1500, 2999]] = np.nan
    xq[:32] = -np.abs(xq[:32])             # every real row is farther than 1 from these
    gd, gi = check_knn(xq, xt, 16, "cosine", "cosine nan")
    assert gi[0, :3].tolist() == [2, 1500, 2999] and np.all(gd[0, :3] == 1.0)


@pytest.mark.parametrize("d", [40, 200])
def test_cosine_zero_rows(d):
    xq, xt = _data(9, 100, 1000, d)
    xt[[0, 5, 999]] = 0.0
    xq[3] = 0.0
    check_knn(xq, xt, 10, "cosine", "zero rows")


def test_cosine_host_arm_nan_rows():
    """Above d = 128 cosine is the knn_host arm: a NaN row's value is NaN and
    never admitted (the fold arm scores it 1 instead)."""
    rng = np.random.default_rng(33)
    xt = rng.standard_normal((3000, 144)).astype(np.float32)
    xq = rng.standard_normal((64, 144)).astype(np.float32)
    xt[[2, 1500, 2999]] = np.nan
    xq[7] = np.nan
    gd, gi = check_knn(xq, xt, 16, "cosine", "host cosine nan")
    assert not np.isin(gi[np.arange(64) != 7], [2, 1500, 2999]).any()


@pytest.mark.parametrize("d", [5, 200])
@pytest.mark.parametrize("k", [24, 110])
def test_f64_nan_zero_rows_and_ties(d, k):
    rng = np.random.default_rng(15 + d)
    xt = rng.integers(-2, 3, size=(3000, d)).astype(np.float64)
    xq = rng.integers(-2, 3, size=(150, d)).astype(np.float64)
    xt[[4, 1500]] = np.nan
    xt[[9, 2999]] = 0.0
    xq[[1, 77]] = 0.0
    xq[5] = np.nan
    xt[100:140] = xt[3]                   # duplicates around the k-th slot
    xq[10] = xt[3]
    check_knn(xq, xt, k, "euclidean", "f64 ties/nan")
    check_knn(xq, xt, k, "cosine", "f64 cosine ties/nan/zero")


def test_f64_nonaligned_pointer():
    rng = np.random.default_rng(16)
    xq, xt = rng.random((60, 64)), rng.random((800, 64))
    flat = np.concatenate([np.zeros(1), xq.ravel()])
    tq = _t(flat)[1:].view(60, 64)  # 8-byte offset: not 16-byte aligned
    assert tq.data_ptr() % 16 == 8
    d_, i_ = prims.knn_topk(tq, _t(xt), 9, "cosine")
    torch.cuda.synchronize()
    wd, wi = oracle.knn_topk(xq, xt, 9, "cosine")
    assert_same(d_.cpu().numpy(), i_.cpu().numpy(), wd, wi, "f64 offset")


@pytest.mark.parametrize("d", [64, 240])
@pytest.mark.parametrize("k", [1, 6, 100])
def test_huge_values_overflow_norms(d, k):
    """Squared norms overflow f32: the screen bound becomes infinite and every
    row is evaluated exactly; results still match the reference arithmetic."""
    xq, xt = _data(10, 40, 500, d, scale=1e18)
    xt[:5] *= 1e2
    check_knn(xq, xt, k, "euclidean", "huge")


def test_k_equals_n_train_and_tiny_index():
    xq, xt = _data(11, 33, 40, 50)
    check_knn(xq, xt, 40, "euclidean", "k=n")
    check_knn(xq, xt[:1], 1, "euclidean", "n_train=1")


@pytest.mark.parametrize("d", [37, 137])
def test_nonaligned_pointer_and_odd_d(d):
    xq, xt = _data(12, 70, 900, d)
    tq = _t(np.concatenate([np.zeros((1, d), np.float32), xq]))[1:]  # 4*d-byte offset -> not 16-aligned
    tq = tq.contiguous()
    d_, i_ = prims.knn_topk(tq, _t(xt), 9)
    torch.cuda.synchronize()
    wd, wi = oracle.knn_topk(xq, xt, 9)
    assert_same(d_.cpu().numpy(), i_.cpu().numpy(), wd, wi, "offset")


def test_side_stream():
    xq, xt = _data(13, 256, 4096, 64)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        tq, tt = _t(xq), _t(xt)
        d_, i_ = prims.knn_topk(tq, tt, 16)
    s.synchronize()
    wd, wi = oracle.knn_topk(xq, xt, 16)
    assert_same(d_.cpu().numpy(), i_.cpu().numpy(), wd, wi, "side stream")


# ---------------------------------------------------------------------------
# k-means assignment, pairwise distance, row norms
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,kc,d,dtype", [(5000, 100, 64, np.float32), (3000, 7, 3, np.float32),
                                         (2000, 50, 200, np.float32), (1500, 40, 32, np.float64),
                                         (20000, 1024, 64, np.float32), (4000, 300, 200, np.float64),
                                         (3000, 20, 7, np.float64)])
def test_kmeans_assign_bitwise(n, kc, d, dtype):
    rng = np.random.default_rng(kc + d)
    c = rng.standard_normal((kc, d)).astype(dtype) * 3
    x = (c[rng.integers(0, kc, n)] + rng.standard_normal((n, d))).astype(dtype)
    lab, sq = prims.kmeans_assign(_t(x), _t(c))
    torch.cuda.synchronize()
    wl, ws = oracle.kmeans_assign(x, c)
    assert np.array_equal(lab.cpu().numpy(), wl.astype(np.int64))
    assert np.array_equal(sq.cpu().numpy(), ws)


@pytest.mark.parametrize("d", [4, 64])
def test_kmeans_ties_and_nan(d):
    rng = np.random.default_rng(14)
    c = rng.standard_normal((10, d)).astype(np.float32)
    c[6] = c[2]                       # exact duplicate centre: ties go to 2
    x = rng.standard_normal((500, d)).astype(np.float32)
    x[:20] = c[2]
    x[30] = np.nan                    # NaN distance to centre 0 wins with label 0
    lab, sq = prims.kmeans_assign(_t(x), _t(c))
    torch.cuda.synchronize()
    wl, ws = oracle.kmeans_assign(x, c)
    assert np.array_equal(lab.cpu().numpy(), wl.astype(np.int64))
    assert np.array_equal(sq.cpu().numpy(), ws, equal_nan=True)
    assert lab[30].item() == 0 and np.isnan(sq[30].item())


@pytest.mark.parametrize("d", [8, 33, 64, 100, 200])
def test_kmeans_queue_overflow_ties(d):
    """500 identical centres: every row of a tile passes the k = 1 screen, so
    the candidate queues overflow and flush inside the tile loop many times;
    the lowest index still wins and the squared distances are the oracle's."""
    rng = np.random.default_rng(21 + d)
    c = rng.standard_normal((700, d)).astype(np.float32)
    c[100:600] = c[3]
    x = rng.standard_normal((3000, d)).astype(np.float32)
    x[::3] = c[3]
    x[1::3] = c[3] + np.float32(1e-3) * rng.standard_normal((1000, d)).astype(np.float32)
    lab, sq = prims.kmeans_assign(_t(x), _t(c))
    torch.cuda.synchronize()
    wl, ws = oracle.kmeans_assign(x, c)
    assert np.array_equal(lab.cpu().numpy(), wl.astype(np.int64))
    assert np.array_equal(sq.cpu().numpy(), ws)
    assert lab[0].item() == 3 and sq[0].item() == 0.0


@pytest.mark.parametrize("d", [24, 64, 160])
def test_k1_search_all_duplicates(d):
    """k = 1 search over an index of mostly identical rows (every query's queue
    overflows on every tile): the lowest index of the tied rows wins."""
    rng = np.random.default_rng(40 + d)
    xt = rng.standard_normal((5000, d)).astype(np.float32)
    xt[1000:4500] = xt[999]
    xq = np.concatenate([xt[999:1000], xt[2000:2001] + np.float32(1e-4),
                         rng.standard_normal((200, d)).astype(np.float32)])
    gd, gi = check_knn(xq, xt, 1, "euclidean", "k1 dups d=%d" % d)
    assert gi[0, 0] == 999 and gd[0, 0] == 0


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("metric,sqrt", [("euclidean", False), ("euclidean", True), ("cosine", False)])
def test_pairwise_bitwise(dtype, metric, sqrt):
    x, y = _data(15, 65, 130, 7, dtype)
    got = prims.pairwise_distance(_t(x), _t(y), metric, sqrt)
    torch.cuda.synchronize()
    want = oracle.pairwise(x, y, metric, sqrt)
    assert np.array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_row_sqnorms_bitwise(dtype):
    x, _ = _data(16, 1000, 1, 77, dtype)
    got = prims.row_sqnorms(_t(x))
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle.row_sqnorms(x))


def test_prim_error_on_device():
    with pytest.raises(Exception) as ei:
        prims.knn_topk(_t(np.zeros((4, 3), np.float32)), _t(np.zeros((5, 3), np.float32)), 6)
    assert getattr(ei.value, "operand", None) == "k"


# ---------------------------------------------------------------------------
# estimator replays of the reference fixtures
# ---------------------------------------------------------------------------
def _brute(xq, xt, metric):
    q, t = xq.astype(np.float64), xt.astype(np.float64)
    if metric == "euclidean":
        return lambda r, j: float(np.sqrt(np.sum((q[r] - t[j]) ** 2)))
    return lambda r, j: float(1.0 - np.dot(q[r], t[j]) / (np.linalg.norm(q[r]) * np.linalg.norm(t[j])))


@pytest.mark.parametrize("s", ["f32", "f64"])
def test_estimator_knn_fixture(s):
    from mlrs_amd.neighbors import NearestNeighbors
    z = load_golden("knn_%s_seed42" % s)
    k = int(z["k"][0])
    nn = NearestNeighbors(n_neighbors=k).fit(z["X"])
    d, i = nn.kneighbors(z["Xq"])
    assert i.dtype == np.int32
    assert np.all(np.abs(d - z["distances"]) <= 1e-5 * np.maximum(np.abs(z["distances"]), 1.0))
    assert np.array_equal(i, z["indices"].astype(np.int32))


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("metric", ["euclidean", "l2", "minkowski", "cosine"])
def test_estimator_nn_params_fixture(s, metric):
    from mlrs_amd.neighbors import NearestNeighbors
    z = load_golden("nn_params_%s_seed42" % s)
    k = int(z["k"][0])
    nn = NearestNeighbors(n_neighbors=k, metric=metric, p=2).fit(z["X"])
    d, i = nn.kneighbors(z["Xq"])
    base = "cosine" if metric == "cosine" else "euclidean"
    assert_topk_matches(d, i, z["distances_" + base], z["indices_" + base].astype(np.int64),
                        _brute(z["Xq"], z["X"], base))


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("metric", ["euclidean", "cosine"])
def test_estimator_self_query_drops_self_by_identity(s, metric):
    from mlrs_amd.neighbors import NearestNeighbors
    z = load_golden("knn_%s_%s_seed42" % (metric, s))
    k = int(z["k"][0])
    nn = NearestNeighbors(n_neighbors=k, metric=metric).fit(z["X"])
    d, i = nn.kneighbors()                    # X=None: k+1 search, self dropped
    want_d, want_i = z["distances"], z["indices"].astype(np.int64)
    rows = np.arange(len(want_i))
    keep = want_i != rows[:, None]
    # reference self-drop of the sklearn k+1 result
    wd = np.stack([want_d[r][keep[r]][:k] for r in rows])
    wi = np.stack([want_i[r][keep[r]][:k] for r in rows])
    assert_topk_matches(d, i, wd, wi, _brute(z["X"], z["X"], metric))
    a, b = int(z["dup_row_a"][0]), int(z["dup_row_b"][0])
    assert i[a, 0] == b and i[b, 0] == a and d[a, 0] == 0 and d[b, 0] == 0


def test_kmeans_estimator_fixture():
    from mlrs_amd.cluster import KMeans
    for s in ("f32", "f64"):
        z = load_golden("kmeans_%s_seed42" % s)
        km = KMeans(cluster_centers=z["centers"])
        assert np.array_equal(km.predict(z["X"]), z["labels"].astype(np.int32))
        inertia = float(np.sum(km.transform_min_sqdist(z["X"]).astype(np.float64)))
        assert abs(inertia - float(z["inertia"][0])) <= 1e-5 * max(1.0, abs(float(z["inertia"][0])))
