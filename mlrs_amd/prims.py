"""Device-level primitives over torch tensors -- the mirror of mlrs-backend's
prims for the brute-force kNN path.

Each function takes and returns device-resident ``torch`` tensors (HIP memory
on ``cuda:N``), launches on the current torch stream and does not synchronize.
Geometry is validated by the C ABI before any launch; a violation raises
``ShapeMismatch`` / ``DimMismatch`` carrying the same fields as
``mlrs_core::PrimError``.

| function            | reference prim it replaces (file:line)                          |
|---------------------|-----------------------------------------------------------------|
| ``knn_topk``        | metric_topk's arms, crates/mlrs-algos/src/neighbors/nearest.rs:891-953 |
| ``kmeans_assign``   | assign_min, crates/mlrs-backend/src/prims/kmeans.rs:635-750      |
| ``pairwise_distance`` | distance_direct / metric_distance, prims/distance.rs:428-727 |
| ``row_sqnorms``     | row_sqnorms, crates/mlrs-backend/src/prims/kmeans.rs:805-832     |
| ``radius_neighbors`` | radius_neighbor_indices_metric, crates/mlrs-algos/src/neighbors/nearest.rs:609-749 |
| ``knn_graph``       | knn_graph via host_knn, crates/mlrs-algos/src/manifold/umap_host_knn.rs:212-515 |
| ``core_distances``  | HDBSCAN core distances, crates/mlrs-algos/src/cluster/hdbscan/host_core.rs:253-540 |
| ``kmeans_fit``      | KMeans::fit, crates/mlrs-algos/src/cluster/kmeans.rs:1353-1580 |
| ``knn_regress``     | knn_regress_mean / knn_regress_gather, crates/mlrs-kernels/src/knn.rs:95-316 |
| ``knn_classify``    | KNeighborsClassifier's host vote, crates/mlrs-algos/src/neighbors/classifier.rs:782-930 |
| ``device_copy``     | device_copy, crates/mlrs-backend/src/prims/knn.rs:358-386         |
| ``pool_stats``      | BufferPool::stats (PoolStats), crates/mlrs-backend/src/pool.rs:27-56,97 |
"""
import ctypes

import torch

from . import _lib

METRICS = {"euclidean": _lib.METRIC_EUCLIDEAN, "cosine": _lib.METRIC_COSINE, "manhattan": _lib.METRIC_MANHATTAN,
           "chebyshev": _lib.METRIC_CHEBYSHEV, "minkowski": _lib.METRIC_MINKOWSKI}
_DT = {torch.float32: "f32", torch.float64: "f64"}


def _suffix(t):
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError("mlrs_amd supports float32/float64 tensors, got %s" % t.dtype)


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _metric_id(metric):
    if isinstance(metric, str):
        try:
            return METRICS[metric]
        except KeyError:
            raise _lib.UnsupportedError("metric %r is not served by the HIP engine" % metric)
    return int(metric)


def _dev_check(*ts):
    for t in ts:
        if not t.is_cuda:
            raise ValueError("mlrs_amd prims take device tensors (got a %s tensor)" % t.device)
        if not t.is_contiguous():
            raise ValueError("mlrs_amd prims take contiguous row-major tensors")
    if any(t.device != ts[0].device for t in ts[1:]):
        raise ValueError("mlrs_amd prims take operands on one device (got %s)" % sorted({str(t.device) for t in ts}))
    # the library works on the current HIP device
    if ts and ts[0].device.index != torch.cuda.current_device():
        raise ValueError("operands are on %s but the current device is cuda:%d (use torch.cuda.device(...))"
                         % (ts[0].device, torch.cuda.current_device()))


# Index / label buffers hold uint32 values; int32 (and uint32 where torch has
# it) tensors have that width.
_IDX_DTYPES = tuple(d for d in (torch.int32, getattr(torch, "uint32", None)) if d is not None)


def _check_out(t, name, dtypes, numel, device):
    """A caller-supplied output buffer: the C ABI counts elements, not bytes,
    and writes through the raw pointer, so the buffer must be a contiguous
    tensor on the operands' device with the element type and count the call
    writes.  Raises before anything is launched."""
    if not isinstance(t, torch.Tensor):
        raise TypeError("%s must be a tensor, got %s" % (name, type(t).__name__))
    if t.device != device:
        raise ValueError("%s must be on %s (got %s)" % (name, device, t.device))
    if t.dtype not in dtypes:
        raise TypeError("%s must be %s, got %s" % (name, " or ".join(str(d) for d in dtypes), t.dtype))
    if not t.is_contiguous():
        raise ValueError("%s must be contiguous" % name)
    if t.numel() != numel:
        raise ValueError("%s must hold %d elements, got %d" % (name, numel, t.numel()))


_PATHS = {"auto": 0, "fused": 1, "lowd": 2, "generic": 3}


def force_path(name):
    """Kernel-family override for tests and benchmarks (mlrs_force_path):
    "auto" (default), "fused" (Gram-MFMA), "lowd" (low-d ALU) or "generic"
    (exact tiles + selection).  Every family returns the same bits."""
    if name not in _PATHS:
        raise ValueError("unknown kernel family %r (expected one of %s)" % (name, sorted(_PATHS)))
    _lib.check(_lib.load().mlrs_force_path(_PATHS[name]))


def knn_topk(xq, x_train, k, metric="euclidean", p=2.0, out=None):
    """k nearest rows of ``x_train`` for every row of ``xq``.

    Returns ``(distances, indices)``: ``(n_query, k)`` tensors, distances in
    the input dtype (true distances), indices ``int64`` by default (``uint32``
    values widened; pass ``out=(dist, idx_int32_or_uint32)`` to supply buffers).
    """
    _dev_check(xq, x_train)
    if x_train.dtype != xq.dtype:
        raise TypeError("query and training dtypes differ")
    s = _suffix(xq)
    nq = xq.shape[0] if xq.dim() == 2 else 0
    d = xq.shape[1] if xq.dim() == 2 else 0
    nt = x_train.shape[0] if x_train.dim() == 2 else 0
    if out is None:
        dist = torch.empty((nq, int(k)), dtype=xq.dtype, device=xq.device)
        idx = torch.empty((nq, int(k)), dtype=torch.int32, device=xq.device)
        widen = True
    else:
        dist, idx = out
        _check_out(dist, "out distances", (xq.dtype,), nq * int(k), xq.device)
        _check_out(idx, "out indices", _IDX_DTYPES, nq * int(k), xq.device)
        widen = False
    lib = _lib.load()
    rc = getattr(lib, "mlrs_knn_topk_" + s)(
        _ptr(xq), xq.numel(), nq, d, _ptr(x_train), x_train.numel(), nt, int(k),
        _metric_id(metric), float(p), _ptr(dist), _ptr(idx), dist.numel(), _stream(xq.device))
    _lib.check(rc)
    if widen:
        # uint32 values below 2^31 (n_train <= UINT32_MAX is validated; the
        # int32 view is exact for n_train < 2^31, which covers every shape here)
        idx = idx.to(torch.int64) & 0xFFFFFFFF
    return dist, idx


def kmeans_assign(x, centers, labels=None, sqdist=None):
    """Nearest centre of every row: ``(labels int64, squared distances)``."""
    _dev_check(x, centers)
    if centers.dtype != x.dtype:
        raise TypeError("points and centres dtypes differ")
    s = _suffix(x)
    n, d = x.shape
    kc = centers.shape[0]
    if labels is not None:
        _check_out(labels, "labels", _IDX_DTYPES, n, x.device)
    if sqdist is not None:
        _check_out(sqdist, "sqdist", (x.dtype,), n, x.device)
    lab = torch.empty(n, dtype=torch.int32, device=x.device) if labels is None else labels
    dist = torch.empty(n, dtype=x.dtype, device=x.device) if sqdist is None else sqdist
    lib = _lib.load()
    rc = getattr(lib, "mlrs_kmeans_assign_" + s)(
        _ptr(x), x.numel(), n, d, _ptr(centers), centers.numel(), kc, _ptr(lab), lab.numel(),
        _ptr(dist), dist.numel(), _stream(x.device))
    _lib.check(rc)
    if labels is None:
        lab = lab.to(torch.int64) & 0xFFFFFFFF
    return lab, dist


def pairwise_distance(x, y, metric="euclidean", sqrt=False, out=None, p=2.0):
    """Full ``rows_x x rows_y`` distance matrix (squared Euclidean unless
    ``sqrt``; ``p`` is the Minkowski exponent)."""
    _dev_check(x, y)
    if y.dtype != x.dtype:
        raise TypeError("x and y dtypes differ")
    s = _suffix(x)
    rx, cx = x.shape
    ry, cy = y.shape
    if out is not None:
        _check_out(out, "out", (x.dtype,), rx * ry, x.device)
    o = torch.empty((rx, ry), dtype=x.dtype, device=x.device) if out is None else out
    lib = _lib.load()
    rc = getattr(lib, "mlrs_pairwise_distance_" + s)(
        _ptr(x), x.numel(), rx, cx, _ptr(y), y.numel(), ry, cy, _metric_id(metric), int(bool(sqrt)), float(p),
        _ptr(o), o.numel(), _stream(x.device))
    _lib.check(rc)
    return o


def row_sqnorms(x, out=None):
    _dev_check(x)
    s = _suffix(x)
    n, d = x.shape
    if out is not None:
        _check_out(out, "out", (x.dtype,), n, x.device)
    o = torch.empty(n, dtype=x.dtype, device=x.device) if out is None else out
    lib = _lib.load()
    rc = getattr(lib, "mlrs_row_sqnorms_" + s)(_ptr(x), x.numel(), n, d, _ptr(o), o.numel(),
                                               _stream(x.device))
    _lib.check(rc)
    return o


def device_copy(x, out=None):
    """The fit-time ownership copy (mlrs_device_copy_*, the reference's
    device_copy): a new device tensor holding ``x``'s values, or ``out``
    filled with them."""
    _dev_check(x)
    s = _suffix(x)
    if out is not None:
        _check_out(out, "out", (x.dtype,), x.numel(), x.device)
    o = torch.empty_like(x) if out is None else out
    rc = getattr(_lib.load(), "mlrs_device_copy_" + s)(_ptr(x), x.numel(), _ptr(o), o.numel(), _stream(x.device))
    _lib.check(rc)
    return o


def pool_stats():
    """The library's buffer counters on the current device (mlrs_pool_stats_get):
    a dict with allocations, reuses, peak_bytes, live_bytes, read_backs."""
    st = _lib.PoolStats()
    _lib.check(_lib.load().mlrs_pool_stats_get(ctypes.byref(st)))
    return {name: int(getattr(st, name)) for name, _ in _lib.PoolStats._fields_}


def pool_stats_reset():
    """Zero the allocation, reuse and read-back counters (peak := live)."""
    _lib.check(_lib.load().mlrs_pool_stats_reset())


# Last match total per search shape (device, dtype, sizes, metric, p, radius):
# sizes the buffers of the next search of that shape.
_RADIUS_TOTAL_HINT = {}


def _remember_radius_total(key, n):
    if key not in _RADIUS_TOTAL_HINT and len(_RADIUS_TOTAL_HINT) >= 64:
        _RADIUS_TOTAL_HINT.clear()
    _RADIUS_TOTAL_HINT[key] = n


def radius_neighbors(xq, x_train, radius, metric="euclidean", p=2.0):
    """Every row of ``x_train`` within ``radius`` of each row of ``xq``
    (mlrs_radius_neighbors_*).

    Returns ``(distances, indices, counts)`` on the device: the matches of
    query row 0, then row 1, ... concatenated, each row's in ascending
    training index (the reference's RadiusNeighbors layout, a CSR matrix
    without its indptr), ``indices`` int32, ``counts`` int64 per query row.
    Synchronizes: the match total sizes the outputs.  A search of a shape
    searched before passes buffers sized from that search's total, so one
    call (one matrix-core pass when every strip's matches fit the library's
    staging) returns the matches."""
    _dev_check(xq, x_train)
    if x_train.dtype != xq.dtype:
        raise TypeError("query and training dtypes differ")
    s = _suffix(xq)
    nq = xq.shape[0] if xq.dim() == 2 else 0
    d = xq.shape[1] if xq.dim() == 2 else 0
    nt = x_train.shape[0] if x_train.dim() == 2 else 0
    dt = x_train.shape[1] if x_train.dim() == 2 else 0
    counts = torch.empty(nq, dtype=torch.int32, device=xq.device)
    total = ctypes.c_int64(0)
    f = getattr(_lib.load(), "mlrs_radius_neighbors_" + s)
    args = (_ptr(xq), xq.numel(), nq, d, _ptr(x_train), x_train.numel(), nt, dt, _metric_id(metric), float(p),
            float(radius), _ptr(counts), counts.numel())
    stream = _stream(xq.device)
    key = (xq.device.index, xq.dtype, nq, nt, d, metric, float(p), float(radius))
    hint = _RADIUS_TOTAL_HINT.get(key)
    if hint is not None:
        # One call with buffers sized from the last search of this shape: the
        # library then counts and keeps the matches in the same pass and
        # copies them into place.  Too small, and the call returns the total
        # with its counts kept for the exact-size call below.
        cap = hint + hint // 8 + 1024
        dist = torch.empty(cap, dtype=xq.dtype, device=xq.device)
        idx = torch.empty(cap, dtype=torch.int32, device=xq.device)
        rc = f(*args, _ptr(dist), _ptr(idx), cap, ctypes.byref(total), stream)
        if rc == 0:
            n = int(total.value)
            _remember_radius_total(key, n)
            return dist[:n], idx[:n], counts.to(torch.int64)
        if rc != _lib.MLRS_ERR_SHAPE_MISMATCH or int(total.value) <= cap:
            _lib.check(rc)
    _lib.check(f(*args, None, None, 0, ctypes.byref(total), stream))
    n = int(total.value)
    _remember_radius_total(key, n)
    dist = torch.empty(n, dtype=xq.dtype, device=xq.device)
    idx = torch.empty(n, dtype=torch.int32, device=xq.device)
    if n:
        _lib.check(f(*args, _ptr(dist), _ptr(idx), n, ctypes.byref(total), stream))
    return dist, idx, counts.to(torch.int64)


def knn_graph(x, k, metric="euclidean", p=2.0, include_self=False):
    """Directed k-nearest graph of the rows of ``x`` against themselves in the
    reference host scan's f64 arithmetic (mlrs_knn_graph_*): ``(indices int64
    (n, k), distances float64 (n, k))``; ``include_self=False`` leaves out each
    row's own index by identity."""
    _dev_check(x)
    s = _suffix(x)
    n, d = x.shape
    idx = torch.empty((n, int(k)), dtype=torch.int32, device=x.device)
    dist = torch.empty((n, int(k)), dtype=torch.float64, device=x.device)
    rc = getattr(_lib.load(), "mlrs_knn_graph_" + s)(
        _ptr(x), x.numel(), n, d, int(k), _metric_id(metric), float(p), int(bool(include_self)), _ptr(idx),
        _ptr(dist), dist.numel(), _stream(x.device))
    _lib.check(rc)
    return idx.to(torch.int64) & 0xFFFFFFFF, dist


def core_distances(x, min_samples, metric="euclidean", p=2.0):
    """HDBSCAN core distances (mlrs_hdbscan_core_distances_*): float64 (n,),
    the (k-1)-th smallest distance of each row to the set, itself included,
    k = clamp(min_samples, 1, n)."""
    _dev_check(x)
    s = _suffix(x)
    n, d = x.shape
    out = torch.empty(n, dtype=torch.float64, device=x.device)
    rc = getattr(_lib.load(), "mlrs_hdbscan_core_distances_" + s)(
        _ptr(x), x.numel(), n, d, _metric_id(metric), float(p), int(min_samples), _ptr(out), out.numel(),
        _stream(x.device))
    _lib.check(rc)
    return out


_KMEANS_INIT = {"array": 0, "k-means++": 1, "random": 2}


_KMEANS_ALGORITHM = {"lloyd": 0, "elkan": 1}


def kmeans_fit(x, n_clusters, init="k-means++", init_centers=None, seed=0, n_init=1, max_iter=300, tol=1e-4,
               algorithm="lloyd"):
    """k-means fit on the device (mlrs_kmeans_fit_*): ``(centers (k, d) in
    x's dtype, labels int64 (n,), inertia float, n_iter int)`` of the winning
    restart.  ``init`` is "k-means++", "random" or "array" (then
    ``init_centers`` is a (k, d) device tensor of x's dtype).  ``algorithm``
    "lloyd" (every row assigned each iteration) or "elkan" (the bound-pruned
    assignment): the same fit either way."""
    if algorithm not in _KMEANS_ALGORITHM:
        raise ValueError("algorithm should be 'lloyd' or 'elkan', got %r" % (algorithm,))
    _dev_check(x)
    s = _suffix(x)
    n, d = x.shape
    k = int(n_clusters)
    ini = None
    if init == "array":
        ini = init_centers.to(device=x.device, dtype=x.dtype).contiguous()
    centers = torch.empty((k, d), dtype=x.dtype, device=x.device)
    labels = torch.empty(n, dtype=torch.int32, device=x.device)
    inertia = ctypes.c_double()
    n_iter = ctypes.c_int64()
    rc = getattr(_lib.load(), "mlrs_kmeans_fit_" + s)(
        _ptr(x), x.numel(), n, d, k, _KMEANS_INIT[init], _ptr(ini), ini.numel() if ini is not None else 0,
        int(seed) & 0xFFFFFFFFFFFFFFFF, int(n_init), int(max_iter), float(tol), _KMEANS_ALGORITHM[algorithm],
        _ptr(centers), centers.numel(),
        _ptr(labels), labels.numel(), ctypes.byref(inertia), ctypes.byref(n_iter), _stream(x.device))
    _lib.check(rc)
    return centers, labels.to(torch.int64), inertia.value, int(n_iter.value)


def _as_u32_idx(idx):
    """Neighbour indices as a contiguous int32 tensor holding the uint32 bits."""
    if idx.dtype == torch.int32:
        return idx.contiguous()
    if idx.dtype == torch.int64:
        return (idx & 0xFFFFFFFF).to(torch.int32).contiguous() if idx.numel() else idx.to(torch.int32)
    raise TypeError("neighbour indices must be int32 or int64, got %s" % idx.dtype)


def knn_regress(y_train, idx, dist=None, weighted=False):
    """Neighbour-target prediction on the device (mlrs_knn_regress_*).

    ``y_train``: (n_train,) or (n_train, n_outputs); ``idx``/``dist``: the
    (n_query, k) indices and true distances of a search (``dist`` needed only
    when ``weighted``).  Returns (n_query,) or (n_query, n_outputs)."""
    _dev_check(y_train)
    s = _suffix(y_train)
    multi = y_train.dim() == 2
    n_train = y_train.shape[0]
    n_out = y_train.shape[1] if multi else 1
    idx32 = _as_u32_idx(idx)
    nq, k = idx32.shape
    d = None
    if dist is not None:
        d = dist.to(y_train.dtype).contiguous()
        _dev_check(d)
    out = torch.empty((nq, n_out) if multi else (nq,), dtype=y_train.dtype, device=y_train.device)
    lib = _lib.load()
    rc = getattr(lib, "mlrs_knn_regress_" + s)(
        _ptr(y_train), y_train.numel(), n_train, n_out, _ptr(idx32), idx32.numel(), _ptr(d),
        d.numel() if d is not None else 0, nq, int(k), int(bool(weighted)), _ptr(out), out.numel(),
        _stream(y_train.device))
    _lib.check(rc)
    return out


def knn_classify(y_class, n_classes, idx, dist=None, weighted=False, dtype=torch.float32):
    """The classifier vote on the device (mlrs_knn_classify_*): ``y_class``
    holds each training row's dense class index; returns
    ``(proba (n_query, n_classes) in dtype, dense labels int64)``."""
    yc = y_class.to(torch.int32).contiguous()
    _dev_check(yc)
    idx32 = _as_u32_idx(idx)
    nq, k = idx32.shape
    d = None
    if dist is not None:
        d = dist.to(dtype).contiguous()
        _dev_check(d)
    proba = torch.empty((nq, int(n_classes)), dtype=dtype, device=yc.device)
    labels = torch.empty(nq, dtype=torch.int32, device=yc.device)
    s = "f32" if dtype == torch.float32 else "f64"
    lib = _lib.load()
    rc = getattr(lib, "mlrs_knn_classify_" + s)(
        _ptr(yc), yc.numel(), int(n_classes), _ptr(idx32), idx32.numel(), _ptr(d),
        d.numel() if d is not None else 0, nq, int(k), int(bool(weighted)), _ptr(proba), proba.numel(),
        _ptr(labels), labels.numel(), _stream(yc.device))
    _lib.check(rc)
    return proba, labels.to(torch.int64)
