"""Pins the CPU oracle's radius scan (oracle/ref_cpu.c orc_radius_scan_*) -- CPU only.

* The reference's sklearn fixtures nn_radius_{f32,f64}_seed42 (five metrics,
  their aliases, and the algorithm-name copies): counts and indices exact, the
  distances to the reference test's mixed bar |err| <= 1e-5 + 1e-5|want|
  (nearest_neighbors_params_test.rs:85-100, 304-366).
* The reference's own radius-scan test design (crates/mlrs-backend/tests/
  radius_scan_test.rs:43-298): splitmix64 data, an independent f64 distance
  per pair, radii at gap midpoints of the distance distribution plus 0 and
  1.5x the largest distance, Minkowski on both lane loops (p = 3 and 2.5).
* The lane arithmetic is the k-nearest host arm's: at d > 128 the oracle's
  knn_topk runs that arm, so each match's value must equal, bit for bit, the
  kNN value of the same (query, index) pair.
* Structure the reference states: ascending indices within a row, counts that
  sum to the length, NaN never matches, radius 0 keeps exactly the coincident
  points, an infinite radius keeps every non-NaN point.
"""
import numpy as np
import pytest

import oracle
from conftest import load_golden

P_FIXTURE = 3.0  # the fixtures' Minkowski exponent (nearest_neighbors_params_test.rs:44-45)


def _split(dist, idx, counts):
    off = np.concatenate([[0], np.cumsum(counts.astype(np.int64))])
    return [(dist[off[r]:off[r + 1]], idx[off[r]:off[r + 1]]) for r in range(counts.size)]


def _check_fixture(got, want_d, want_i, want_c):
    d, i, c = got
    np.testing.assert_array_equal(c, want_c.astype(np.uint32))
    np.testing.assert_array_equal(i, want_i.astype(np.int32))
    np.testing.assert_allclose(d, want_d, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("metric", ["euclidean", "manhattan", "chebyshev", "minkowski", "cosine"])
def test_radius_fixture(s, metric):
    z = load_golden("nn_radius_%s_seed42" % s)
    got = oracle.radius_neighbors(z["Xq"], z["X"], float(z["radius_" + metric][0]), metric, p=P_FIXTURE)
    _check_fixture(got, z["radius_distances_" + metric], z["radius_indices_" + metric],
                   z["radius_counts_" + metric])


ALIASES = [("euclidean", "euclidean"), ("l2", "euclidean"), ("manhattan", "manhattan"), ("l1", "manhattan"),
           ("cityblock", "manhattan"), ("chebyshev", "chebyshev"), ("infinity", "chebyshev"),
           ("cosine", "cosine"), ("minkowski", "euclidean")]  # the alias_minkowski case runs p = 2


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("alias,metric", ALIASES)
def test_radius_alias_fixture(s, alias, metric):
    z = load_golden("nn_radius_%s_seed42" % s)
    got = oracle.radius_neighbors(z["Xq"], z["X"], float(z["radius_alias_r_" + alias][0]), metric)
    _check_fixture(got, z["radius_alias_distances_" + alias], z["radius_alias_indices_" + alias],
                   z["radius_alias_counts_" + alias])


@pytest.mark.parametrize("s", ["f32", "f64"])
@pytest.mark.parametrize("alg", ["auto", "brute", "kd_tree", "ball_tree"])
def test_radius_algorithm_fixture(s, alg):
    z = load_golden("nn_radius_%s_seed42" % s)
    got = oracle.radius_neighbors(z["Xq"], z["X"], float(z["radius_euclidean"][0]), "euclidean")
    _check_fixture(got, z["radius_alg_distances_" + alg], z["radius_alg_indices_" + alg],
                   z["radius_alg_counts_" + alg])


# ---- the reference's radius_scan_test design -------------------------------

_M64 = (1 << 64) - 1


def _splitmix_design(rows, cols, seed):
    """radius_scan_test.rs:43-61: splitmix64 words -> f32 in [3, 7)."""
    out = np.empty(rows * cols, dtype=np.float32)
    st = seed
    for n in range(rows * cols):
        st = (st + 0x9E3779B97F4A7C15) & _M64
        z = st
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
        z ^= z >> 31
        out[n] = np.float32((z >> 11) / float(1 << 53)) * np.float32(4.0) + np.float32(3.0)
    return out.reshape(rows, cols)


def _true_distances(xq, xt, metric, p):
    """radius_scan_test.rs:77-110: one pair's true distance in f64."""
    a = xq.astype(np.float64)[:, None, :]
    b = xt.astype(np.float64)[None, :, :]
    if metric == "euclidean":
        return np.sqrt(((a - b) ** 2).sum(-1))
    if metric == "manhattan":
        return np.abs(a - b).sum(-1)
    if metric == "chebyshev":
        return np.abs(a - b).max(-1)
    if metric == "minkowski":
        return (np.abs(a - b) ** p).sum(-1) ** (1.0 / p)
    dot = (a * b).sum(-1)
    nx = (a * a).sum(-1)
    ny = (b * b).sum(-1)
    return np.clip(1.0 - dot / np.sqrt(nx * ny), 0.0, 2.0)


def _radius_at(all_sorted, frac):
    """radius_scan_test.rs:170-178: midpoint of the first >=0.1% gap at or after
    the `frac` quantile, so no pair sits on the threshold."""
    start = min(int(all_sorted.size * frac), all_sorted.size - 2)
    for i in range(start, all_sorted.size - 1):
        if all_sorted[i + 1] > all_sorted[i] * 1.001 + 1e-9:
            return 0.5 * (all_sorted[i] + all_sorted[i + 1])
    return all_sorted[-1] * 1.5


METRIC_CASES = [("euclidean", 2.0), ("manhattan", 2.0), ("chebyshev", 2.0), ("cosine", 2.0), ("minkowski", 3.0),
                ("minkowski", 2.5)]


@pytest.mark.parametrize("metric,p", METRIC_CASES)
def test_radius_against_independent_f64(metric, p):
    xq = _splitmix_design(37, 9, 11)
    xt = _splitmix_design(200, 9, 23)
    true = _true_distances(xq, xt, metric, p)
    srt = np.sort(true.ravel())
    for radius in (0.0, _radius_at(srt, 0.1), _radius_at(srt, 0.5), srt[-1] * 1.5):
        d, i, c = oracle.radius_neighbors(xq, xt, radius, metric, p=p)
        mask = true <= radius
        np.testing.assert_array_equal(c, mask.sum(1).astype(np.uint32))
        want_i = np.concatenate([np.nonzero(mask[r])[0] for r in range(mask.shape[0])]).astype(np.int32)
        np.testing.assert_array_equal(i, want_i)
        want_d = true[mask]
        assert np.all(np.abs(d.astype(np.float64) - want_d) <= 1e-4 * np.maximum(np.abs(want_d), 1.0))


@pytest.mark.parametrize("metric,p", METRIC_CASES)
def test_radius_ascending_and_counts(metric, p):
    """radius_scan_test.rs:301-345: many matches per row, ascending, counts sum."""
    xq = _splitmix_design(5, 6, 41)
    xt = _splitmix_design(900, 6, 43)
    srt = np.sort(_true_distances(xq, xt, metric, p).ravel())
    d, i, c = oracle.radius_neighbors(xq, xt, _radius_at(srt, 0.3), metric, p=p)
    assert int(c.sum()) == i.size == d.size
    assert (c > 1).any()
    for _, ri in _split(d, i, c):
        assert np.all(np.diff(ri) > 0)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("metric,p", [("euclidean", 2.0), ("cosine", 2.0), ("minkowski", 3.0),
                                      ("minkowski", 1.5), ("manhattan", 2.0), ("chebyshev", 2.0)])
def test_radius_values_are_the_knn_host_arm(dtype, metric, p):
    """At d > 128 the k-nearest oracle runs the host arm; every radius match
    must carry exactly that arm's value for its (query, index) pair."""
    rng = np.random.default_rng(7)
    d_ = 140
    xt = rng.standard_normal((300, d_)).astype(dtype)
    xq = rng.standard_normal((9, d_)).astype(dtype)
    assert oracle.knn_arm(d_, 300, metric) == oracle.ARM_HOST
    kd, ki = oracle.knn_topk(xq, xt, 300, metric, p=p)
    full = np.empty((9, 300), dtype=dtype)
    for r in range(9):
        full[r, ki[r]] = kd[r]
    radius = float(np.median(full.astype(np.float64)))
    d, i, c = oracle.radius_neighbors(xq, xt, radius, metric, p=p)
    for r, (rd, ri) in enumerate(_split(d, i, c)):
        np.testing.assert_array_equal(rd, full[r, ri])
        # membership agrees with the kNN values except within a rounding of the radius
        inside = np.nonzero(full[r].astype(np.float64) <= radius)[0]
        sym = set(inside.tolist()) ^ set(ri.tolist())
        for j in sym:
            assert abs(float(full[r, j]) - radius) <= 1e-5 * max(1.0, radius)


def test_radius_edge_cases():
    rng = np.random.default_rng(3)
    xt = rng.standard_normal((50, 4)).astype(np.float32)
    xq = rng.standard_normal((6, 4)).astype(np.float32)
    xt[7] = xq[2]
    xt[30] = xq[2]                       # two coincident points of query 2
    xt[11, 1] = np.nan                   # NaN distance: never matches
    for metric in ("euclidean", "manhattan", "chebyshev"):
        d, i, c = oracle.radius_neighbors(xq, xt, 0.0, metric)
        assert c.tolist() == [0, 0, 2, 0, 0, 0]
        assert i.tolist() == [7, 30] and d.tolist() == [0.0, 0.0]
        d, i, c = oracle.radius_neighbors(xq, xt, np.inf, metric)
        if metric == "chebyshev":
            # the running max is a select that a NaN never replaces
            # (knn_host.rs:719-726): row 11 keeps a finite distance
            assert c.tolist() == [50] * 6
        else:
            assert c.tolist() == [49] * 6 and 11 not in i.tolist()
    d, i, c = oracle.radius_neighbors(xq, xt[:0], 1.0)
    assert c.tolist() == [0] * 6 and i.size == 0
    with pytest.raises(ValueError):
        oracle.radius_neighbors(xq, xt, -1.0)
    with pytest.raises(ValueError):
        oracle.radius_neighbors(xq, xt, float("nan"))
