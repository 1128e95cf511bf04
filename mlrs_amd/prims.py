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
"""
import torch

from . import _lib

METRICS = {"euclidean": _lib.METRIC_EUCLIDEAN, "cosine": _lib.METRIC_COSINE}
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
    s = _suffix(x)
    n, d = x.shape
    kc = centers.shape[0]
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


def pairwise_distance(x, y, metric="euclidean", sqrt=False, out=None):
    """Full ``rows_x x rows_y`` distance matrix (squared Euclidean unless ``sqrt``)."""
    _dev_check(x, y)
    s = _suffix(x)
    rx, cx = x.shape
    ry, cy = y.shape
    o = torch.empty((rx, ry), dtype=x.dtype, device=x.device) if out is None else out
    lib = _lib.load()
    rc = getattr(lib, "mlrs_pairwise_distance_" + s)(
        _ptr(x), x.numel(), rx, cx, _ptr(y), y.numel(), ry, cy, _metric_id(metric), int(bool(sqrt)),
        _ptr(o), o.numel(), _stream(x.device))
    _lib.check(rc)
    return o


def row_sqnorms(x, out=None):
    _dev_check(x)
    s = _suffix(x)
    n, d = x.shape
    o = torch.empty(n, dtype=x.dtype, device=x.device) if out is None else out
    lib = _lib.load()
    rc = getattr(lib, "mlrs_row_sqnorms_" + s)(_ptr(x), x.numel(), n, d, _ptr(o), o.numel(),
                                               _stream(x.device))
    _lib.check(rc)
    return o
