"""``NearestNeighbors`` over the HIP engine -- the brute-force kNN estimator
surface of ``mlrs.neighbors`` (crates/mlrs-py/python/mlrs/neighbors.py).

Same parameter names, metric resolution, validation order and error messages
as the reference shim for the metrics the engine serves (Euclidean and its
aliases, cosine); ``kneighbors(X=None)`` queries the training set with k+1 and
drops each row's own index by identity, not by position or distance
(neighbors.py:217-238, 622-647).

Inputs may be numpy arrays or torch tensors; the training matrix is uploaded
once at ``fit`` and stays resident in HBM.  Results come back as numpy arrays
for numpy input and as device tensors for tensor input.
"""
import warnings

import numpy as np
import torch

from . import prims

_NEIGHBORS_ALGORITHMS = ("auto", "ball_tree", "kd_tree", "brute")
_SUPPORTED_METRICS = ("minkowski", "euclidean", "l2", "manhattan", "l1", "cityblock", "chebyshev",
                      "infinity", "cosine")
_ALGORITHM_VALID_METRICS = {
    "brute": ("minkowski", "euclidean", "l2", "manhattan", "l1", "cityblock", "chebyshev", "cosine"),
    "kd_tree": ("minkowski", "euclidean", "l2", "manhattan", "l1", "cityblock", "chebyshev", "infinity"),
}
_ALGORITHM_VALID_METRICS["ball_tree"] = _ALGORITHM_VALID_METRICS["kd_tree"]
_ALGORITHM_VALID_METRICS["auto"] = _SUPPORTED_METRICS

# metric_from_str (crates/mlrs-py/src/estimators/neighbors.rs:900-923)
_ENGINE_METRIC = {"euclidean": "euclidean", "l2": "euclidean", "cosine": "cosine",
                  "manhattan": "manhattan", "l1": "manhattan", "cityblock": "manhattan",
                  "chebyshev": "chebyshev", "infinity": "chebyshev"}


def _resolve_metric(metric, p, metric_params):
    """sklearn's metric resolution as the shim implements it (neighbors.py:106-171)."""
    params = {} if metric_params is None else dict(metric_params)
    if metric_params is not None and "p" in metric_params:
        warnings.warn("Parameter p is found in metric_params. "
                      "The corresponding parameter from __init__ is ignored.", SyntaxWarning, stacklevel=3)
    effective_metric = metric
    effective_p = None
    if metric == "minkowski":
        effective_p = params.pop("p", p)
        w = params.pop("w", None)
        if effective_p is None or effective_p < 1:
            raise ValueError("p must be greater or equal to one for minkowski metric")
        if w is not None:
            raise ValueError("weighted minkowski (metric_params['w']) is not supported")
        if effective_p == 1:
            effective_metric = "manhattan"
        elif effective_p == 2:
            effective_metric = "euclidean"
        elif effective_p == float("inf"):
            effective_metric = "chebyshev"
        else:
            params["p"] = effective_p
            params["w"] = w
    return effective_metric, params, effective_p


def _drop_self_column(dist, idx, k):
    """Remove each row's own index from a k+1-wide result (neighbors.py:217-238).

    Works on numpy arrays; when the self index is absent the LAST column goes.
    """
    rows = dist.shape[0]
    keep = np.ones(dist.shape, dtype=bool)
    eq = idx == np.arange(rows)[:, None]
    self_col = np.argmax(eq, axis=1)
    has_self = np.any(eq, axis=1)
    self_col = np.where(has_self, self_col, dist.shape[1] - 1)
    keep[np.arange(rows), self_col] = False
    return dist[keep].reshape(rows, k), idx[keep].reshape(rows, k)


def _as_device_matrix(X, dtype=None, device=None):
    """(device tensor, was_numpy) for a 2-D float32/float64 input."""
    if isinstance(X, torch.Tensor):
        t = X
        was_numpy = False
    else:
        a = np.asarray(X)
        if a.dtype not in (np.float32, np.float64):
            a = a.astype(np.float64)
        t = torch.from_numpy(np.ascontiguousarray(a))
        was_numpy = True
    if t.dim() != 2:
        raise ValueError("Expected 2D array, got %dD array instead" % t.dim())
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    if t.dtype not in (torch.float32, torch.float64):
        t = t.to(torch.float64)
    dev = device if device is not None else (t.device if t.is_cuda else torch.device("cuda", torch.cuda.current_device()))
    return t.to(dev).contiguous(), was_numpy


def _check_finite(t):
    if bool(torch.isnan(t).any()):
        raise ValueError("Input contains NaN.")
    if bool(torch.isinf(t).any()):
        raise ValueError("Input contains infinity or a value too large for dtype('%s')."
                         % str(t.dtype).replace("torch.", ""))


class NearestNeighbors:
    """Brute-force neighbour search (mlrs.neighbors.NearestNeighbors)."""

    def __init__(self, n_neighbors=5, output_type="input", *, radius=1.0, algorithm="auto", leaf_size=30,
                 metric="minkowski", p=2, metric_params=None, n_jobs=None, device="auto"):
        self.n_neighbors = n_neighbors
        self.output_type = output_type
        self.radius = radius
        self.algorithm = algorithm
        self.leaf_size = leaf_size
        self.metric = metric
        self.p = p
        self.metric_params = metric_params
        self.n_jobs = n_jobs
        self.device = device

    # -- validation (neighbors.py:285-338) --
    def _validate_params_for_fit(self):
        if self.algorithm not in _NEIGHBORS_ALGORITHMS:
            raise ValueError("Algorithm is not supported: %s. Supported algorithms are %s"
                             % (self.algorithm, list(_NEIGHBORS_ALGORITHMS)))
        if callable(self.metric) or self.metric not in _SUPPORTED_METRICS:
            raise ValueError("Metric is not supported: %s. Supported metrics are %s"
                             % (self.metric, list(_SUPPORTED_METRICS)))
        if not isinstance(self.leaf_size, (int, np.integer)) or self.leaf_size < 1:
            raise ValueError("leaf_size == %s, must be >= 1." % (self.leaf_size,))
        if not isinstance(self.n_neighbors, (int, np.integer)) or self.n_neighbors < 1:
            raise ValueError("n_neighbors == %s, must be >= 1." % (self.n_neighbors,))
        if self.n_jobs is not None and not isinstance(self.n_jobs, (int, np.integer)):
            raise ValueError("n_jobs == %s, must be an integer or None." % (self.n_jobs,))
        if self.metric not in _ALGORITHM_VALID_METRICS[self.algorithm]:
            raise ValueError("Metric '%s' not valid. Use sorted(sklearn.neighbors.VALID_METRICS['%s']) "
                             "to get valid options. Metric can also be a callable function."
                             % (self.metric, self.algorithm))
        if not isinstance(self.radius, (int, float, np.integer, np.floating)) or self.radius < 0:
            raise ValueError("radius must be non-negative, got %r" % (self.radius,))

    def fit(self, X, y=None):
        self._validate_params_for_fit()
        eff, params, eff_p = _resolve_metric(self.metric, self.p, self.metric_params)
        engine_metric = _ENGINE_METRIC.get(eff)
        if engine_metric not in prims.METRICS:
            raise NotImplementedError("metric %r is not served by the HIP engine" % eff)
        t, _ = _as_device_matrix(X)
        _check_finite(t)
        self._fit_X_dev = t
        self._engine_metric = engine_metric
        self.n_features_in_ = t.shape[1]
        self.n_samples_fit_ = t.shape[0]
        self.effective_metric_ = eff
        self.effective_metric_params_ = params
        return self

    def _check_fitted(self):
        if not hasattr(self, "_fit_X_dev"):
            raise ValueError("This NearestNeighbors instance is not fitted yet. Call 'fit' with "
                             "appropriate arguments before using this estimator.")

    @property
    def _fit_X(self):
        self._check_fitted()
        return self._fit_X_dev.cpu().numpy()

    def _resolve_k(self, n_neighbors, query_is_train):
        """neighbors.py:605-620: X=None needs k+1 so the self match can be dropped."""
        k = self.n_neighbors if n_neighbors is None else n_neighbors
        if not isinstance(k, (int, np.integer)) or k < 1:
            raise ValueError("Expected n_neighbors > 0. Got %s" % (k,))
        k_query = k + 1 if query_is_train else k
        if k_query > self.n_samples_fit_:
            raise ValueError("Expected n_neighbors <= n_samples_fit, but n_neighbors = %d, "
                             "n_samples_fit = %d" % (k, self.n_samples_fit_))
        return int(k), int(k_query)

    def _raw_kneighbors(self, Xq, k):
        dist, idx = prims.knn_topk(Xq, self._fit_X_dev, k, self._engine_metric)
        return dist, idx.to(torch.int32)

    def kneighbors(self, X=None, n_neighbors=None, return_distance=True):
        self._check_fitted()
        query_is_train = X is None
        k, k_query = self._resolve_k(n_neighbors, query_is_train)
        if query_is_train:
            q, was_numpy = self._fit_X_dev, True
        else:
            q, was_numpy = _as_device_matrix(X, dtype=self._fit_X_dev.dtype, device=self._fit_X_dev.device)
            if q.shape[1] != self.n_features_in_:
                raise ValueError("X has %d features, but NearestNeighbors is expecting %d features as input"
                                 % (q.shape[1], self.n_features_in_))
            _check_finite(q)
        dist, idx = self._raw_kneighbors(q, k_query)
        if query_is_train or was_numpy:
            dist_np = dist.cpu().numpy()
            idx_np = idx.cpu().numpy()
            if query_is_train:
                dist_np, idx_np = _drop_self_column(dist_np, idx_np, k)
            if not return_distance:
                return idx_np
            return dist_np, idx_np
        if not return_distance:
            return idx
        return dist, idx


def kneighbors(X_train, X_query, k, metric="euclidean"):
    """Functional form: ``(distances, int64 indices)`` as device tensors."""
    t, _ = _as_device_matrix(X_train)
    q, _ = _as_device_matrix(X_query, dtype=t.dtype, device=t.device)
    return prims.knn_topk(q, t, k, metric)
