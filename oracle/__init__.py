"""CPU oracle for the brute-force kNN path -- TEST INFRASTRUCTURE ONLY.

A ctypes front for ``ref_cpu.c`` (the plain-C restatement of mlrs's cpu-backend
kNN, k-means assignment and pairwise-distance arithmetic; see that file's header
for the reference citations).  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg may import this package, and only as the
checker or the timed CPU baseline -- never as part of the product path.

Parity status of each function (how it is pinned) is listed in
``tests/test_oracle.py``; every function here is pinned by at least one of: the
reference's sklearn fixtures, an exact-arithmetic brute force on small inputs,
or a known-answer invariant from the reference's own tests.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATHS = {"x86-64-v3": os.path.join(_HERE, "libmlrs_oracle.so"),
              "x86-64-v4": os.path.join(_HERE, "libmlrs_oracle_v4.so")}
_V4_FLAGS = ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl")


def host_isa():
    """The widest oracle build this CPU runs: x86-64-v4 when /proc/cpuinfo
    lists the AVX-512 subsets it needs, else x86-64-v3.  MLRS_ORACLE_ISA
    overrides."""
    forced = os.environ.get("MLRS_ORACLE_ISA")
    if forced in _LIB_PATHS:
        return forced
    try:
        flags = set()
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    break
        if all(x in flags for x in _V4_FLAGS):
            return "x86-64-v4"
    except OSError:
        pass
    return "x86-64-v3"


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def build_info():
    """What the loaded oracle is: {"isa", "flags", "cpu_model"}."""
    from . import build as _build
    isa = host_isa()
    return {"isa": isa, "flags": _build.flags_of(isa), "cpu_model": cpu_model()}

METRIC_EUCLIDEAN = 0
METRIC_COSINE = 1
METRIC_MANHATTAN = 2
METRIC_CHEBYSHEV = 3
METRIC_MINKOWSKI = 4
METRICS = {"euclidean": METRIC_EUCLIDEAN, "cosine": METRIC_COSINE, "manhattan": METRIC_MANHATTAN,
           "chebyshev": METRIC_CHEBYSHEV, "minkowski": METRIC_MINKOWSKI}

ARM_DIRECT = 0
ARM_METRIC = 1
ARM_HOST = 2

_lib = None


def _load():
    global _lib
    if _lib is not None:
        return _lib
    path = _LIB_PATHS[host_isa()]
    if not os.path.exists(path):
        from . import build as _build  # noqa: F401  (oracle/build.py)
        _build.build()
    lib = ctypes.CDLL(path)
    i64, i32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
    lib.orc_knn_arm.argtypes = [i64, i64, i32]
    lib.orc_knn_arm.restype = i32
    lib.orc_max_threads.argtypes = []
    lib.orc_max_threads.restype = i32
    for s_ in ("f32", "f64"):
        f = getattr(lib, "orc_kmeans_fit_" + s_)
        f.argtypes = [vp, i64, i64, i64, i32, vp, ctypes.c_uint64, i64, i64, ctypes.c_double, vp, vp, vp, vp]
        f.restype = i32
        f = getattr(lib, "orc_kmeans_init_" + s_)
        f.argtypes = [vp, i64, i64, i64, i32, ctypes.c_uint64, vp]
        f.restype = i32
        f = getattr(lib, "orc_feature_mean_var_" + s_)
        f.argtypes = [vp, i64, i64]
        f.restype = ctypes.c_double
    lib.orc_splitmix64_stream.argtypes = [ctypes.c_uint64, i64, vp]
    lib.orc_splitmix64_stream.restype = None
    lib.orc_knn_graph_f64.argtypes = [vp, i64, i64, i64, i32, ctypes.c_double, i32, vp, vp]
    lib.orc_knn_graph_f64.restype = i32
    lib.orc_core_distances_f64.argtypes = [vp, i64, i64, i32, ctypes.c_double, i64, vp]
    lib.orc_core_distances_f64.restype = i32
    for s in ("f32", "f64"):
        f = getattr(lib, "orc_knn_topk_" + s)
        f.argtypes = [vp, i64, vp, i64, i64, i64, i32, ctypes.c_double, vp, vp, i32]
        f.restype = i32
        f = getattr(lib, "orc_kmeans_assign_" + s)
        f.argtypes = [vp, i64, vp, i64, i64, vp, vp, i32]
        f.restype = i32
        f = getattr(lib, "orc_pairwise_" + s)
        f.argtypes = [vp, i64, vp, i64, i64, i32, i32, ctypes.c_double, vp, i32]
        f.restype = i32
        f = getattr(lib, "orc_row_sqnorms_" + s)
        f.argtypes = [vp, i64, i64, vp]
        f.restype = None
        f = getattr(lib, "orc_radius_scan_" + s)
        f.argtypes = [vp, i64, vp, i64, i64, i32, ctypes.c_double, ctypes.c_double, vp, vp, vp, vp, i32]
        f.restype = i32
        f = getattr(lib, "orc_knn_regress_mean_" + s)
        f.argtypes = [vp, i64, vp, i64, i64, vp, vp]
        f.restype = None
        f = getattr(lib, "orc_knn_regress_gather_" + s)
        f.argtypes = [vp, i64, i64, vp, vp, i64, i64, i32, vp, vp]
        f.restype = None
        f = getattr(lib, "orc_knn_classify_" + s)
        f.argtypes = [vp, i64, i64, vp, vp, i64, i64, i32, vp, vp, vp, vp, vp]
        f.restype = i32
    _lib = lib
    return lib


def _suffix(dtype):
    if dtype == np.float32:
        return "f32"
    if dtype == np.float64:
        return "f64"
    raise TypeError("oracle supports float32/float64, got %s" % dtype)


def _metric_id(metric):
    if isinstance(metric, str):
        return METRICS[metric]
    return int(metric)


def knn_arm(d, k, metric="euclidean"):
    """Which reference cpu arm serves (d, k, metric): ARM_DIRECT/METRIC/HOST."""
    return _load().orc_knn_arm(int(d), int(k), _metric_id(metric))


def max_threads():
    return _load().orc_max_threads()


def knn_topk(xq, xt, k, metric="euclidean", nthreads=0, p=2.0):
    """(distances, uint32 indices), each (n_query, k), ascending (value, index).
    ``p`` is the Minkowski exponent (metric "minkowski" only)."""
    lib = _load()
    xq = np.ascontiguousarray(xq)
    xt = np.ascontiguousarray(xt, dtype=xq.dtype)
    nq, d = xq.shape
    nt, d2 = xt.shape
    assert d == d2
    s = _suffix(xq.dtype)
    out_v = np.empty((nq, k), dtype=xq.dtype)
    out_i = np.empty((nq, k), dtype=np.uint32)
    rc = getattr(lib, "orc_knn_topk_" + s)(
        xq.ctypes.data, nq, xt.ctypes.data, nt, d, int(k), _metric_id(metric), float(p),
        out_v.ctypes.data, out_i.ctypes.data, int(nthreads))
    if rc != 0:
        raise ValueError("oracle knn_topk rejected k=%d for n_train=%d" % (k, nt))
    return out_v, out_i


def kmeans_assign(x, centers, nthreads=0):
    """(uint32 labels, squared distances) of the nearest centre per row."""
    lib = _load()
    x = np.ascontiguousarray(x)
    centers = np.ascontiguousarray(centers, dtype=x.dtype)
    n, d = x.shape
    kc = centers.shape[0]
    s = _suffix(x.dtype)
    labels = np.empty(n, dtype=np.uint32)
    dist = np.empty(n, dtype=x.dtype)
    rc = getattr(lib, "orc_kmeans_assign_" + s)(
        x.ctypes.data, n, centers.ctypes.data, kc, d, labels.ctypes.data,
        dist.ctypes.data, int(nthreads))
    if rc != 0:
        raise ValueError("oracle kmeans_assign rejected k=%d for n=%d" % (kc, n))
    return labels, dist


def pairwise(x, y, metric="euclidean", sqrt=False, nthreads=0, p=2.0):
    lib = _load()
    x = np.ascontiguousarray(x)
    y = np.ascontiguousarray(y, dtype=x.dtype)
    nx, d = x.shape
    ny = y.shape[0]
    out = np.empty((nx, ny), dtype=x.dtype)
    rc = getattr(lib, "orc_pairwise_" + _suffix(x.dtype))(
        x.ctypes.data, nx, y.ctypes.data, ny, d, _metric_id(metric), int(bool(sqrt)), float(p),
        out.ctypes.data, int(nthreads))
    if rc != 0:
        raise ValueError("oracle pairwise rejected d=%d" % d)
    return out


def radius_neighbors(xq, xt, radius, metric="euclidean", nthreads=0, p=2.0):
    """(distances, int32 indices, uint32 counts): every training row within
    ``radius`` of each query row, concatenated row by row in ascending training
    index (a CSR layout without indptr), distances through the metric's
    boundary transform."""
    lib = _load()
    xq = np.ascontiguousarray(xq)
    xt = np.ascontiguousarray(xt, dtype=xq.dtype)
    nq, d = xq.shape
    nt = xt.shape[0]
    f = getattr(lib, "orc_radius_scan_" + _suffix(xq.dtype))
    counts = np.zeros(nq, dtype=np.uint32)
    rc = f(xq.ctypes.data, nq, xt.ctypes.data, nt, d, _metric_id(metric), float(p), float(radius),
           counts.ctypes.data, None, None, None, int(nthreads))
    if rc != 0:
        raise ValueError("oracle radius_neighbors rejected radius=%r, d=%d" % (radius, d))
    offsets = np.zeros(nq, dtype=np.int64)
    if nq > 1:
        np.cumsum(counts[:-1], dtype=np.int64, out=offsets[1:])
    total = int(counts.sum(dtype=np.int64))
    dist = np.empty(total, dtype=xq.dtype)
    idx = np.empty(total, dtype=np.int32)
    f(xq.ctypes.data, nq, xt.ctypes.data, nt, d, _metric_id(metric), float(p), float(radius),
      counts.ctypes.data, offsets.ctypes.data, dist.ctypes.data, idx.ctypes.data, int(nthreads))
    return dist, idx, counts


def knn_graph(x, k, metric="euclidean", p=2.0, include_self=False):
    """(uint32 indices, f64 distances), each (n, k): the directed k-nearest
    graph of the rows of ``x`` against themselves in the reference's host f64
    arithmetic (``x`` is widened to f64 first, as the reference does)."""
    lib = _load()
    x = np.ascontiguousarray(x, dtype=np.float64)
    n, d = x.shape
    idx = np.empty((n, k), dtype=np.uint32)
    dist = np.empty((n, k), dtype=np.float64)
    rc = lib.orc_knn_graph_f64(x.ctypes.data, n, d, int(k), _metric_id(metric), float(p), int(bool(include_self)),
                               idx.ctypes.data, dist.ctypes.data)
    if rc != 0:
        raise ValueError("oracle knn_graph rejected k=%d for n=%d" % (k, n))
    return idx, dist


def core_distances(x, min_samples, metric="euclidean", p=2.0):
    """HDBSCAN core distances (f64): the (k-1)-th smallest distance of each row
    to the whole set, self included, k = clamp(min_samples, 1, n)."""
    lib = _load()
    x = np.ascontiguousarray(x, dtype=np.float64)
    n, d = x.shape
    out = np.empty(n, dtype=np.float64)
    rc = lib.orc_core_distances_f64(x.ctypes.data, n, d, _metric_id(metric), float(p), int(min_samples),
                                    out.ctypes.data)
    if rc != 0:
        raise ValueError("oracle core_distances rejected the input")
    return out


KMEANS_INIT = {"array": 0, "k-means++": 1, "random": 2}


def kmeans_fit(x, k, init="k-means++", init_centers=None, seed=0, n_init=1, max_iter=300, tol=1e-4):
    """KMeans.fit as the reference's cpu backend runs it: ``(centers (k, d) in
    x's dtype, uint32 labels, inertia (f64), n_iter)``."""
    lib = _load()
    x = np.ascontiguousarray(x)
    n, d = x.shape
    s = _suffix(x.dtype)
    ini = None
    if init == "array":
        ini = np.ascontiguousarray(init_centers, dtype=x.dtype)
    centers = np.empty((k, d), dtype=x.dtype)
    labels = np.empty(n, dtype=np.uint32)
    inertia = ctypes.c_double()
    n_iter = ctypes.c_int64()
    rc = getattr(lib, "orc_kmeans_fit_" + s)(
        x.ctypes.data, n, d, int(k), KMEANS_INIT[init], ini.ctypes.data if ini is not None else None,
        int(seed), int(n_init), int(max_iter), float(tol), centers.ctypes.data, labels.ctypes.data,
        ctypes.byref(inertia), ctypes.byref(n_iter))
    if rc != 0:
        raise ValueError("oracle kmeans_fit failed (%d)" % rc)
    return centers, labels, inertia.value, n_iter.value


def kmeans_init(x, k, init="k-means++", seed=0):
    """The row indices k-means++ / random initialisation picks (SplitMix64)."""
    lib = _load()
    x = np.ascontiguousarray(x)
    n, d = x.shape
    out = np.empty(k, dtype=np.int64)
    rc = getattr(lib, "orc_kmeans_init_" + _suffix(x.dtype))(x.ctypes.data, n, d, int(k), KMEANS_INIT[init],
                                                              int(seed), out.ctypes.data)
    if rc != 0:
        raise ValueError("oracle kmeans_init failed")
    return out


def splitmix64(seed, n):
    out = np.empty(n, dtype=np.uint64)
    _load().orc_splitmix64_stream(int(seed), int(n), out.ctypes.data)
    return out


def feature_mean_var(x):
    x = np.ascontiguousarray(x)
    n, d = x.shape
    return getattr(_load(), "orc_feature_mean_var_" + _suffix(x.dtype))(x.ctypes.data, n, d)


def row_sqnorms(x):
    lib = _load()
    x = np.ascontiguousarray(x)
    n, d = x.shape
    out = np.empty(n, dtype=x.dtype)
    getattr(lib, "orc_row_sqnorms_" + _suffix(x.dtype))(x.ctypes.data, n, d, out.ctypes.data)
    return out


def _sfx(dtype):
    return "f32" if np.dtype(dtype) == np.float32 else "f64"


def knn_regress(y_train, idx, dist=None, weighted=False):
    """Neighbour-target prediction (knn_regress_mean for the uniform
    single-output case, knn_regress_gather otherwise).  ``y_train`` is
    (n_train,) or (n_train, n_outputs); ``idx``/``dist`` are (n_query, k).
    Returns (prediction, oob_flags)."""
    lib = _load()
    y = np.ascontiguousarray(y_train)
    multi = y.ndim == 2
    n_train = y.shape[0]
    n_out = y.shape[1] if multi else 1
    idx = np.ascontiguousarray(idx, dtype=np.uint32)
    nq, k = idx.shape
    out = np.empty((nq, n_out), dtype=y.dtype)
    oob = np.empty(nq, dtype=np.uint32)
    s = _sfx(y.dtype)
    if not weighted and not multi:
        getattr(lib, "orc_knn_regress_mean_" + s)(y.ctypes.data, n_train, idx.ctypes.data, nq, k,
                                                  out.ctypes.data, oob.ctypes.data)
    else:
        d = None if dist is None else np.ascontiguousarray(dist, dtype=y.dtype)
        getattr(lib, "orc_knn_regress_gather_" + s)(y.ctypes.data, n_train, n_out, idx.ctypes.data,
                                                    None if d is None else d.ctypes.data, nq, k,
                                                    int(bool(weighted)), out.ctypes.data, oob.ctypes.data)
    return (out if multi else out.ravel()), oob


def knn_classify(y_class, n_classes, idx, dist=None, weighted=False, dtype=np.float32):
    """The classifier vote: (proba (n_query, n_classes) in ``dtype``, dense
    labels (n_query,) int32).  Raises IndexError on a bad neighbour index or
    class id, naming (kind, value, query, slot)."""
    lib = _load()
    yc = np.ascontiguousarray(y_class, dtype=np.int32)
    idx = np.ascontiguousarray(idx, dtype=np.uint32)
    nq, k = idx.shape
    proba = np.empty((nq, n_classes), dtype=dtype)
    labels = np.empty(nq, dtype=np.int32)
    acc = np.empty(max(n_classes, 1), dtype=np.float64)
    w = np.empty(max(k, 1), dtype=np.float64)
    err = np.zeros(4, dtype=np.int64)
    d = None if dist is None else np.ascontiguousarray(dist, dtype=dtype)
    rc = getattr(lib, "orc_knn_classify_" + _sfx(dtype))(
        yc.ctypes.data, yc.size, n_classes, idx.ctypes.data, None if d is None else d.ctypes.data, nq, k,
        int(bool(weighted)), proba.ctypes.data, labels.ctypes.data, acc.ctypes.data, w.ctypes.data,
        err.ctypes.data)
    if rc:
        raise IndexError(("train_idx" if err[0] == 1 else "class_id", int(err[1]), int(err[2]), int(err[3])))
    return proba, labels
