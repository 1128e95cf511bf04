"""ctypes binding of libmlrs_hip_knn.so (the C ABI in include/mlrs_hip_knn.h).

The library is loaded from this package directory only.  If it is missing the
import of any compute entry point raises -- there is no CPU fallback.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmlrs_hip_knn.so")

MLRS_OK = 0
MLRS_ERR_SHAPE_MISMATCH = -1
MLRS_ERR_DIM_MISMATCH = -2
MLRS_ERR_UNSUPPORTED = -3
MLRS_ERR_NULL_POINTER = -4
MLRS_ERR_HIP = -5
MLRS_ERR_ALLOC = -6
MLRS_ERR_INVALID_PARAM = -7

# Size of the allocation-free entry point's static scratch (MLRS_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 128 << 20

METRIC_EUCLIDEAN = 0
METRIC_COSINE = 1
METRIC_MANHATTAN = 2
METRIC_CHEBYSHEV = 3
METRIC_MINKOWSKI = 4


class ErrorInfo(ctypes.Structure):
    _fields_ = [
        ("code", ctypes.c_int32),
        ("operand", ctypes.c_char * 32),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("len", ctypes.c_int64),
        ("hip_error", ctypes.c_int32),
        ("message", ctypes.c_char * 160),
    ]


class PoolStats(ctypes.Structure):
    """mlrs_pool_stats: the reference's PoolStats counters over the library's
    cached device buffers (crates/mlrs-backend/src/pool.rs:27-56)."""
    _fields_ = [
        ("allocations", ctypes.c_uint64),
        ("reuses", ctypes.c_uint64),
        ("peak_bytes", ctypes.c_uint64),
        ("live_bytes", ctypes.c_uint64),
        ("read_backs", ctypes.c_uint64),
    ]


class PrimError(ValueError):
    """A geometry violation rejected before any launch (mlrs_core::PrimError)."""

    def __init__(self, info):
        self.code = info.code
        self.operand = info.operand.decode()
        self.rows = info.rows
        self.cols = info.cols
        self.len = info.len
        super().__init__(info.message.decode())


class ShapeMismatch(PrimError):
    """PrimError::ShapeMismatch{operand, rows, cols, len}."""


class DimMismatch(PrimError):
    """PrimError::DimMismatch{dim, lhs, rhs}; `rows`/`cols` carry lhs/rhs."""


class InvalidParam(PrimError):
    """A scalar parameter outside its domain (AlgoError::InvalidEps and its like);
    ``operand`` names it."""


class UnsupportedError(NotImplementedError):
    pass


class HipError(RuntimeError):
    pass


# (name, restype, argtypes) of every exported symbol in include/mlrs_hip_knn.h
_i32, _i64, _vp, _f64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_double
SIGNATURES = {
    "mlrs_last_error": (_i32, [ctypes.POINTER(ErrorInfo)]),
    "mlrs_status_string": (ctypes.c_char_p, [_i32]),
    "mlrs_abi_version": (_i32, []),
    "mlrs_knn_topk_f32": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _i32, _f64, _vp, _vp, _i64, _vp]),
    "mlrs_knn_topk_f64": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _i32, _f64, _vp, _vp, _i64, _vp]),
    "mlrs_knn_max_k": (_i32, [_i32, _i64, _i32]),
    "mlrs_knn_topk_f32_noalloc": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _i32, _f64, _vp, _vp, _i64,
                                         _vp]),
    "mlrs_kmeans_assign_f32": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "mlrs_kmeans_assign_f64": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "mlrs_pairwise_distance_f32": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _i32, _f64, _vp, _i64,
                                          _vp]),
    "mlrs_pairwise_distance_f64": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _i32, _f64, _vp, _i64,
                                          _vp]),
    "mlrs_row_sqnorms_f32": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp]),
    "mlrs_row_sqnorms_f64": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp]),
    "mlrs_knn_regress_f32": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp]),
    "mlrs_knn_regress_f64": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp]),
    "mlrs_knn_classify_f32": (_i32, [_vp, _i64, _i32, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp, _i64,
                                     _vp]),
    "mlrs_knn_classify_f64": (_i32, [_vp, _i64, _i32, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp, _i64,
                                     _vp]),
    "mlrs_radius_neighbors_f32": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _f64, _f64, _vp, _i64,
                                         _vp, _vp, _i64, ctypes.POINTER(_i64), _vp]),
    "mlrs_radius_neighbors_f64": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _f64, _f64, _vp, _i64,
                                         _vp, _vp, _i64, ctypes.POINTER(_i64), _vp]),
    "mlrs_knn_graph_f32": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _f64, _i32, _vp, _vp, _i64, _vp]),
    "mlrs_knn_graph_f64": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _f64, _i32, _vp, _vp, _i64, _vp]),
    "mlrs_hdbscan_core_distances_f32": (_i32, [_vp, _i64, _i64, _i64, _i32, _f64, _i64, _vp, _i64, _vp]),
    "mlrs_hdbscan_core_distances_f64": (_i32, [_vp, _i64, _i64, _i64, _i32, _f64, _i64, _vp, _i64, _vp]),
    "mlrs_kmeans_fit_f32": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _i64, ctypes.c_uint64, _i64, _i64, _f64,
                                   _i32, _vp, _i64, _vp, _i64, ctypes.POINTER(_f64), ctypes.POINTER(_i64), _vp]),
    "mlrs_kmeans_fit_f64": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _i64, ctypes.c_uint64, _i64, _i64, _f64,
                                   _i32, _vp, _i64, _vp, _i64, ctypes.POINTER(_f64), ctypes.POINTER(_i64), _vp]),
    "mlrs_release_workspace": (_i32, []),
    "mlrs_device_copy_f32": (_i32, [_vp, _i64, _vp, _i64, _vp]),
    "mlrs_device_copy_f64": (_i32, [_vp, _i64, _vp, _i64, _vp]),
    "mlrs_pool_stats_get": (_i32, [ctypes.POINTER(PoolStats)]),
    "mlrs_pool_stats_reset": (_i32, []),
    "mlrs_timing_enable": (_i32, [_i32]),
    "mlrs_probe_peak": (_i32, [_i32, _i32, ctypes.POINTER(_f64), _vp]),
    "mlrs_force_path": (_i32, [_i32]),
    "mlrs_timing_read": (_i32, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64), ctypes.c_char_p, _i32]),
}

_lib = None


def load():
    """Load the engine library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            "mlrs_amd: HIP engine %s is not built; run `python -c \"import __graft_entry__ as g; g.build()\"` "
            "(or python mlrs_amd/build.py) first" % LIB_PATH)
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


def check(rc):
    """Raise the Python twin of a non-zero status."""
    if rc == MLRS_OK:
        return
    info = ErrorInfo()
    load().mlrs_last_error(ctypes.byref(info))
    if rc == MLRS_ERR_SHAPE_MISMATCH:
        raise ShapeMismatch(info)
    if rc == MLRS_ERR_DIM_MISMATCH:
        raise DimMismatch(info)
    if rc == MLRS_ERR_INVALID_PARAM:
        raise InvalidParam(info)
    if rc == MLRS_ERR_UNSUPPORTED:
        raise UnsupportedError(info.message.decode())
    if rc == MLRS_ERR_NULL_POINTER:
        raise ValueError(info.message.decode())
    raise HipError("%s (hip error %d)" % (info.message.decode(), info.hip_error))
