"""The C-ABI library loads, exports every declared symbol, and rejects bad
geometry before touching the GPU -- CPU only (no compute calls)."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT
from mlrs_amd import _lib

HEADER = os.path.join(ROOT, "include", "mlrs_hip_knn.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int32_t|const char \*)\s*\*?\s*(mlrs_\w+)\s*\(", text, re.M)))


def test_header_declares_the_entry_points():
    syms = declared_symbols()
    for s in ("mlrs_knn_topk_f32", "mlrs_knn_topk_f64", "mlrs_kmeans_assign_f32", "mlrs_kmeans_assign_f64",
              "mlrs_pairwise_distance_f32", "mlrs_pairwise_distance_f64", "mlrs_row_sqnorms_f32",
              "mlrs_row_sqnorms_f64", "mlrs_last_error", "mlrs_status_string"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for s in declared_symbols():
        assert hasattr(lib, s), s
        assert s in _lib.SIGNATURES, "binding missing for " + s


def test_abi_version_and_status_strings():
    lib = _lib.load()
    assert lib.mlrs_abi_version() == 5
    assert lib.mlrs_status_string(0) == b"ok"
    assert lib.mlrs_status_string(-7) == b"invalid parameter value"
    assert lib.mlrs_status_string(-1) == b"shape mismatch"
    assert lib.mlrs_status_string(-2) == b"dimension mismatch"


# Dummy non-null "device" pointers: validation fails before any dereference or launch.
P = ctypes.c_void_p(0x1000)


def _knn32(xq_len, nq, d, xt_len, nt, k, metric=0, out_len=None):
    lib = _lib.load()
    out_len = nq * k if out_len is None else out_len
    return lib.mlrs_knn_topk_f32(P, xq_len, nq, d, P, xt_len, nt, k, metric, 2.0, P, P, out_len, None)


def _info():
    e = _lib.ErrorInfo()
    _lib.load().mlrs_last_error(ctypes.byref(e))
    return e


@pytest.mark.parametrize("args,operand,fields", [
    ((10 * 4 - 1, 10, 4, 20 * 4, 20, 3), "x", (10, 4, 39)),
    ((10 * 4, 10, 4, 20 * 4 + 1, 20, 3), "y", (20, 4, 81)),
    ((10 * 4, 10, 4, 20 * 4, 20, 0), "k", (1, 0, 20)),
    ((10 * 4, 10, 4, 20 * 4, 20, 21), "k", (1, 21, 20)),
    ((0, 10, 0, 0, 20, 3), "features", (0, 0, 0)),
])
def test_knn_validation_is_prim_error(args, operand, fields):
    rc = _knn32(*args)
    assert rc == _lib.MLRS_ERR_SHAPE_MISMATCH
    e = _info()
    assert e.operand.decode() == operand
    assert (e.rows, e.cols, e.len) == fields
    assert b"shape mismatch" in e.message


def test_knn_out_and_metric_validation():
    assert _knn32(40, 10, 4, 80, 20, 3, out_len=29) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert _info().operand == b"out"
    assert _knn32(40, 10, 4, 80, 20, 3, metric=7) == _lib.MLRS_ERR_UNSUPPORTED


def test_kmeans_validation():
    lib = _lib.load()
    f = lib.mlrs_kmeans_assign_f32
    assert f(P, 99, 10, 10, P, 30, 3, P, 10, P, 10, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert _info().operand == b"x"
    assert f(P, 100, 10, 10, P, 110, 11, P, 10, P, 10, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert _info().operand == b"k"
    assert f(P, 100, 10, 10, P, 29, 3, P, 10, P, 10, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert _info().operand == b"centers"
    assert f(P, 100, 10, 10, P, 30, 3, P, 9, P, 10, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert _info().operand == b"labels"


def test_pairwise_validation():
    lib = _lib.load()
    f = lib.mlrs_pairwise_distance_f64
    assert f(P, 14, 5, 3, P, 12, 4, 3, 0, 0, 2.0, P, 20, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert (_info().operand, _info().len) == (b"x", 14)
    assert f(P, 15, 5, 3, P, 13, 4, 3, 0, 0, 2.0, P, 20, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert _info().operand == b"y"


def test_pairwise_dim_mismatch_and_out():
    lib = _lib.load()
    f = lib.mlrs_pairwise_distance_f32
    assert f(P, 15, 5, 3, P, 16, 4, 4, 0, 0, 2.0, P, 20, None) == _lib.MLRS_ERR_DIM_MISMATCH
    e = _info()
    assert (e.operand, e.rows, e.cols) == (b"cols", 3, 4)
    assert f(P, 15, 5, 3, P, 12, 4, 3, 0, 0, 2.0, P, 19, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert _info().operand == b"out"


def test_python_error_mapping():
    with pytest.raises(_lib.ShapeMismatch) as ei:
        _lib.check(_knn32(39, 10, 4, 80, 20, 3))
    assert ei.value.operand == "x" and ei.value.len == 39


def test_estimator_parameter_validation_needs_no_gpu():
    from mlrs_amd.neighbors import NearestNeighbors, _resolve_metric
    with pytest.raises(ValueError, match="Algorithm is not supported"):
        NearestNeighbors(algorithm="lsh").fit(np.zeros((3, 2)))
    with pytest.raises(ValueError, match="Metric 'cosine' not valid"):
        NearestNeighbors(algorithm="kd_tree", metric="cosine").fit(np.zeros((3, 2)))
    with pytest.raises(ValueError, match="p must be greater or equal to one"):
        NearestNeighbors(p=0.5).fit(np.zeros((3, 2)))
    assert _resolve_metric("minkowski", 2, None)[0] == "euclidean"
    assert _resolve_metric("minkowski", 1, None)[0] == "manhattan"
    assert _resolve_metric("minkowski", float("inf"), None)[0] == "chebyshev"


def test_self_drop_by_index_identity():
    from mlrs_amd.neighbors import _drop_self_column
    dist = np.array([[0.0, 0.0, 1.0], [0.0, 0.0, 2.0], [0.5, 0.7, 0.9]])
    idx = np.array([[1, 0, 2], [0, 1, 2], [0, 1, 3]])
    d, i = _drop_self_column(dist, idx, 2)
    assert i.tolist() == [[1, 2], [0, 2], [0, 1]]
    assert d.tolist() == [[0.0, 1.0], [0.0, 2.0], [0.5, 0.7]]


def test_force_path_validation():
    """The kernel-family override validates its argument without touching a GPU."""
    from mlrs_amd import _lib, prims
    lib = _lib.load()
    assert lib.mlrs_force_path(7) == -3
    assert lib.mlrs_force_path(0) == 0
    with pytest.raises(ValueError):
        prims.force_path("mfma")
    prims.force_path("auto")


def test_metric_family_validation():
    """Unknown metrics and Minkowski p < 1 are rejected before any launch."""
    lib = _lib.load()
    f = lib.mlrs_knn_topk_f32
    assert f(P, 30, 10, 3, P, 30, 10, 2, 9, 2.0, P, P, 20, None) == _lib.MLRS_ERR_UNSUPPORTED
    assert _info().operand == b"metric"
    assert f(P, 30, 10, 3, P, 30, 10, 2, 4, 0.5, P, P, 20, None) == _lib.MLRS_ERR_UNSUPPORTED
    assert _info().operand == b"p"
    g = lib.mlrs_pairwise_distance_f64
    assert g(P, 15, 5, 3, P, 12, 4, 3, 4, 0, float("nan"), P, 20, None) == _lib.MLRS_ERR_UNSUPPORTED
    assert _info().operand == b"p"


def _radius32(xq_len=40, nq=10, d=4, xt_len=80, nt=20, dt=4, metric=0, p=2.0, radius=1.0, counts_len=10,
              out=None, cap=0):
    total = ctypes.c_int64(-1)
    rc = _lib.load().mlrs_radius_neighbors_f32(P, xq_len, nq, d, P, xt_len, nt, dt, metric, p, radius, P,
                                              counts_len, out, out, cap, ctypes.byref(total), None)
    return rc


@pytest.mark.parametrize("kw,code,operand", [
    (dict(radius=-1.0), _lib.MLRS_ERR_INVALID_PARAM, b"radius"),
    (dict(radius=float("nan")), _lib.MLRS_ERR_INVALID_PARAM, b"radius"),
    (dict(nq=0, xq_len=0), _lib.MLRS_ERR_SHAPE_MISMATCH, b"xq"),
    (dict(d=0, xq_len=0, dt=0, xt_len=0), _lib.MLRS_ERR_SHAPE_MISMATCH, b"xq"),
    (dict(xq_len=39), _lib.MLRS_ERR_SHAPE_MISMATCH, b"xq"),
    (dict(dt=5, xt_len=100), _lib.MLRS_ERR_DIM_MISMATCH, b"n_features"),
    (dict(xt_len=81), _lib.MLRS_ERR_SHAPE_MISMATCH, b"y"),
    (dict(metric=5), _lib.MLRS_ERR_UNSUPPORTED, b"metric"),
    (dict(metric=4, p=0.5), _lib.MLRS_ERR_UNSUPPORTED, b"p"),
    (dict(counts_len=9), _lib.MLRS_ERR_SHAPE_MISMATCH, b"counts"),
])
def test_radius_validation(kw, code, operand):
    """radius_neighbors rejects bad radii and geometry before any launch, in
    validate_radius_query's order (nearest.rs:755-797)."""
    assert _radius32(**kw) == code
    assert _info().operand == operand


def test_radius_error_text_and_python_mapping():
    assert _radius32(radius=-0.5) == _lib.MLRS_ERR_INVALID_PARAM
    assert b"eps = -0.5 is invalid (must be >= 0)" in _info().message
    with pytest.raises(_lib.InvalidParam) as ei:
        _lib.check(_radius32(radius=-0.5))
    assert ei.value.operand == "radius"


def test_graph_validation():
    """knn_graph's validate_geometry order (knn_graph.rs:475-539) before any launch."""
    lib = _lib.load()
    f = lib.mlrs_knn_graph_f32
    assert f(P, 29, 10, 3, 3, 0, 2.0, 0, P, P, 30, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert _info().operand == b"x"
    assert f(P, 30, 10, 3, 10, 0, 2.0, 0, P, P, 100, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    e = _info()
    assert (e.operand, e.rows, e.cols, e.len) == (b"k", 1, 10, 9)
    assert f(P, 30, 10, 3, 0, 0, 2.0, 1, P, P, 0, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert f(P, 30, 10, 3, 3, 4, 0.5, 0, P, P, 30, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert (_info().operand, _info().len) == (b"p", 1)
    assert f(P, 30, 10, 3, 3, 6, 2.0, 0, P, P, 30, None) == _lib.MLRS_ERR_UNSUPPORTED
    assert f(P, 30, 10, 3, 3, 0, 2.0, 0, P, P, 29, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert _info().operand == b"out"
    g = lib.mlrs_hdbscan_core_distances_f64
    assert g(P, 30, 10, 3, 1, 2.0, 5, P, 10, None) == _lib.MLRS_ERR_UNSUPPORTED
    assert g(P, 30, 10, 3, 0, 2.0, 5, P, 9, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
    assert _info().operand == b"out"


def test_kmeans_fit_validation():
    lib = _lib.load()
    f = lib.mlrs_kmeans_fit_f32
    inertia, n_iter = ctypes.c_double(), ctypes.c_int64()

    def call(n=10, d=3, k=3, kind=1, init_len=0, n_init=1, max_iter=10, tol=1e-4, x_len=None, c_len=None,
             l_len=None, algorithm=0):
        return f(P, n * d if x_len is None else x_len, n, d, k, kind, P, init_len, 0, n_init, max_iter, tol, algorithm, P,
                 k * d if c_len is None else c_len, P, n if l_len is None else l_len, ctypes.byref(inertia),
                 ctypes.byref(n_iter), None)
    assert call(k=11) == _lib.MLRS_ERR_INVALID_PARAM and _info().operand == b"k"
    assert b"out of range" in _info().message
    assert call(k=0) == _lib.MLRS_ERR_INVALID_PARAM
    assert call(x_len=29) == _lib.MLRS_ERR_SHAPE_MISMATCH and _info().operand == b"x"
    assert call(kind=0, init_len=8) == _lib.MLRS_ERR_SHAPE_MISMATCH and _info().operand == b"init"
    assert call(kind=5) == _lib.MLRS_ERR_UNSUPPORTED
    assert call(n_init=0) == _lib.MLRS_ERR_INVALID_PARAM and _info().operand == b"n_init"
    assert call(tol=-1.0) == _lib.MLRS_ERR_INVALID_PARAM and _info().operand == b"tol"
    assert call(algorithm=2) == _lib.MLRS_ERR_INVALID_PARAM and _info().operand == b"algorithm"
    assert call(c_len=8) == _lib.MLRS_ERR_SHAPE_MISMATCH and _info().operand == b"centers"
    assert call(l_len=9) == _lib.MLRS_ERR_SHAPE_MISMATCH and _info().operand == b"labels"


def test_noalloc_entry_validates_like_the_allocating_one():
    lib = _lib.load()
    for name in ("mlrs_knn_topk_f32", "mlrs_knn_topk_f32_noalloc"):
        f = getattr(lib, name)
        assert f(P, 39, 10, 4, P, 80, 20, 3, 0, 2.0, P, P, 30, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
        assert _info().operand == b"x"
        assert f(P, 40, 10, 4, P, 80, 20, 21, 0, 2.0, P, P, 210, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
        e = _info()
        assert (e.operand, e.rows, e.cols, e.len) == (b"k", 1, 21, 20)
        assert f(P, 40, 10, 4, P, 80, 20, 3, 9, 2.0, P, P, 30, None) == _lib.MLRS_ERR_UNSUPPORTED
        # no queries: nothing to do, no device touched
        assert f(P, 0, 0, 4, P, 80, 20, 3, 0, 2.0, P, P, 0, None) == _lib.MLRS_OK


def test_every_k_up_to_n_train_is_served():
    assert _lib.load().mlrs_knn_max_k(4, 128, 0) == 2**31 - 1


def test_device_copy_validation():
    lib = _lib.load()
    for f in (lib.mlrs_device_copy_f32, lib.mlrs_device_copy_f64):
        assert f(P, 10, P, 9, None) == _lib.MLRS_ERR_SHAPE_MISMATCH
        e = _info()
        assert (e.operand, e.rows, e.cols, e.len) == (b"dst", 10, 1, 9)
        assert f(P, -1, P, -1, None) == _lib.MLRS_ERR_SHAPE_MISMATCH and _info().operand == b"src"
        assert f(None, 4, P, 4, None) == _lib.MLRS_ERR_NULL_POINTER
        assert f(None, 0, None, 0, None) == _lib.MLRS_OK


def test_pool_stats_without_a_device():
    st = _lib.PoolStats()
    assert _lib.load().mlrs_pool_stats_get(ctypes.byref(st)) == _lib.MLRS_OK
    assert _lib.load().mlrs_pool_stats_get(None) == _lib.MLRS_ERR_NULL_POINTER
