"""``NearestNeighbors``, ``KNeighborsRegressor`` and ``KNeighborsClassifier``
over the HIP engine -- the brute-force kNN estimator surface of
``mlrs.neighbors`` (crates/mlrs-py/python/mlrs/neighbors.py).

Same parameter names, metric resolution, validation order and error messages
as the reference shim for the metrics the engine serves (Euclidean, Manhattan,
Chebyshev, Minkowski-p and their aliases, cosine); ``kneighbors(X=None)`` queries the training set with k+1 and
drops each row's own index by identity, not by position or distance
(neighbors.py:217-238, 622-647).

Inputs may be numpy arrays or torch tensors; the training matrix is uploaded
once at ``fit`` and stays resident in HBM.  Results come back as numpy arrays
for numpy input and as device tensors for tensor input.

The regressor and classifier predict on the device end to end: the search,
then the neighbour-target gather (knn_regress_mean / knn_regress_gather) or
the class vote (the reference's host f64 vote, restated as a kernel).  A
callable ``weights`` and a multi-output classification target are served on
the host from the same neighbour set, as the reference shim does
(neighbors.py:914-1036).
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
                  "chebyshev": "chebyshev", "infinity": "chebyshev", "minkowski": "minkowski"}


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


class _NeighborsBase:
    """Shared fit / kneighbors machinery (neighbors.py:241-688)."""

    radius = 1.0

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

    def _fit_X_only(self, X):
        self._validate_params_for_fit()
        eff, params, eff_p = _resolve_metric(self.metric, self.p, self.metric_params)
        engine_metric = _ENGINE_METRIC.get(eff)
        if engine_metric not in prims.METRICS:
            raise NotImplementedError("metric %r is not served by the HIP engine" % eff)
        t, _ = _as_device_matrix(X)
        _check_finite(t)
        if isinstance(X, torch.Tensor) and t.data_ptr() == X.data_ptr():
            # Fit::fit keeps its own copy of the training rows
            # (crates/mlrs-backend/src/prims/knn.rs:358-386 device_copy): a
            # device tensor of the caller is copied, not aliased
            t = prims.device_copy(t)
        self._fit_X_dev = t
        self._engine_metric = engine_metric
        self._engine_p = float(eff_p) if engine_metric == "minkowski" else 2.0
        self.n_features_in_ = t.shape[1]
        self.n_samples_fit_ = t.shape[0]
        self.effective_metric_ = eff
        self.effective_metric_params_ = params
        return t

    def _check_fitted(self):
        if not hasattr(self, "_fit_X_dev"):
            raise ValueError("This %s instance is not fitted yet. Call 'fit' with "
                             "appropriate arguments before using this estimator." % type(self).__name__)

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
        dist, idx = prims.knn_topk(Xq, self._fit_X_dev, k, self._engine_metric, p=self._engine_p)
        return dist, idx.to(torch.int32)

    def _check_query(self, q):
        if q.shape[1] != self.n_features_in_:
            raise ValueError("X has %d features, but %s is expecting %d features as input"
                             % (q.shape[1], type(self).__name__, self.n_features_in_))
        _check_finite(q)

    def _query(self, X):
        """(device query matrix, was_numpy) for a predict call."""
        self._check_fitted()
        q, was_numpy = _as_device_matrix(X, dtype=self._fit_X_dev.dtype, device=self._fit_X_dev.device)
        self._check_query(q)
        return q, was_numpy

    def kneighbors(self, X=None, n_neighbors=None, return_distance=True):
        self._check_fitted()
        query_is_train = X is None
        k, k_query = self._resolve_k(n_neighbors, query_is_train)
        if query_is_train:
            q, was_numpy = self._fit_X_dev, True
        else:
            q, was_numpy = _as_device_matrix(X, dtype=self._fit_X_dev.dtype, device=self._fit_X_dev.device)
            self._check_query(q)
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

    def kneighbors_graph(self, X=None, n_neighbors=None, mode="connectivity"):
        """The ``(n_query, n_samples_fit_)`` sparse neighbour graph as a scipy
        CSR matrix (neighbors.py:649-688): 1 per neighbour for
        ``mode='connectivity'``, the distance for ``mode='distance'``."""
        from scipy.sparse import csr_matrix

        self._check_fitted()
        if mode not in ("connectivity", "distance"):
            raise ValueError('Unsupported mode, must be one of "connectivity" or "distance" but got "%s" instead'
                             % (mode,))
        dist, idx = self.kneighbors(X, n_neighbors, return_distance=True)
        dist = dist.cpu().numpy() if isinstance(dist, torch.Tensor) else dist
        idx = idx.cpu().numpy() if isinstance(idx, torch.Tensor) else idx
        n_query, k = idx.shape
        data = np.ones(n_query * k, dtype=np.float64) if mode == "connectivity" else \
            np.asarray(dist, dtype=np.float64).ravel()
        indptr = np.arange(0, n_query * k + 1, k)
        return csr_matrix((data, idx.ravel(), indptr), shape=(n_query, self.n_samples_fit_))

    # -- radius queries (neighbors.py:443-603) --
    def _resolve_radius(self, radius):
        r = self.radius if radius is None else radius
        if not isinstance(r, (int, float, np.integer, np.floating)) or r < 0:
            raise ValueError("radius must be non-negative, got %r" % (r,))
        return float(r)

    def _raw_radius_neighbors(self, X, radius):
        """``(dist_list, idx_list, rows)``: each query row's matches, ascending
        training index, from the device scan (mlrs_radius_neighbors_*)."""
        if X is None:
            q = self._fit_X_dev
        else:
            q, _ = _as_device_matrix(X, dtype=self._fit_X_dev.dtype, device=self._fit_X_dev.device)
            self._check_query(q)
        dist, idx, counts = prims.radius_neighbors(q, self._fit_X_dev, radius, self._engine_metric,
                                                   p=self._engine_p)
        dist = dist.cpu().numpy()
        idx = idx.cpu().numpy()
        counts = counts.cpu().numpy()
        offsets = np.concatenate([[0], np.cumsum(counts)])
        rows = counts.shape[0]
        return ([dist[offsets[r]:offsets[r + 1]] for r in range(rows)],
                [idx[offsets[r]:offsets[r + 1]] for r in range(rows)], rows)

    @staticmethod
    def _drop_self_ragged(dist_list, idx_list, rows):
        """Drop each row's own index by identity (neighbors.py:493-510): a
        duplicate training point at distance 0 stays."""
        new_dist, new_idx = [], []
        for i in range(rows):
            keep = idx_list[i] != i
            new_dist.append(dist_list[i][keep])
            new_idx.append(idx_list[i][keep])
        return new_dist, new_idx

    @staticmethod
    def _sort_ragged_by_distance(dist_list, idx_list, rows):
        for i in range(rows):
            order = np.argsort(dist_list[i], kind="stable")
            dist_list[i] = dist_list[i][order]
            idx_list[i] = idx_list[i][order]
        return dist_list, idx_list

    def _radius_lists(self, X, radius, sort_results):
        self._check_fitted()
        r = self._resolve_radius(radius)
        dist_list, idx_list, rows = self._raw_radius_neighbors(X, r)
        if X is None:
            dist_list, idx_list = self._drop_self_ragged(dist_list, idx_list, rows)
        if sort_results:
            dist_list, idx_list = self._sort_ragged_by_distance(dist_list, idx_list, rows)
        return dist_list, idx_list, rows

    def radius_neighbors(self, X=None, radius=None, return_distance=True, sort_results=False):
        """Every training point within ``radius`` of each row of ``X``
        (neighbors.py:528-563): numpy object arrays with one sub-array per
        query row, ascending training index unless ``sort_results``.
        ``X=None`` queries the training set without each row's own index."""
        self._check_fitted()
        if sort_results and not return_distance:
            raise ValueError("return_distance must be True if sort_results is True.")
        dist_list, idx_list, rows = self._radius_lists(X, radius, sort_results)
        indices = np.empty(rows, dtype=object)
        for i in range(rows):
            indices[i] = idx_list[i]
        if not return_distance:
            return indices
        distances = np.empty(rows, dtype=object)
        for i in range(rows):
            distances[i] = dist_list[i]
        return distances, indices

    def radius_neighbors_graph(self, X=None, radius=None, mode="connectivity", sort_results=False):
        """The ``(n_query, n_samples_fit_)`` sparse radius graph as a scipy CSR
        matrix (neighbors.py:565-603)."""
        from scipy.sparse import csr_matrix

        self._check_fitted()
        if mode not in ("connectivity", "distance"):
            raise ValueError('Unsupported mode, must be one of "connectivity" or "distance" but got "%s" instead'
                             % (mode,))
        dist_list, idx_list, rows = self._radius_lists(X, radius, sort_results)
        counts = np.array([len(a) for a in idx_list], dtype=np.int64)
        indptr = np.concatenate([[0], np.cumsum(counts)])
        all_idx = np.concatenate(idx_list) if rows else np.array([], dtype=np.int32)
        if mode == "connectivity":
            data = np.ones(all_idx.shape[0], dtype=np.float64)
        else:
            data = np.concatenate(dist_list).astype(np.float64) if rows else np.array([], dtype=np.float64)
        return csr_matrix((data, all_idx, indptr), shape=(rows, self.n_samples_fit_))


class NearestNeighbors(_NeighborsBase):
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

    def fit(self, X, y=None):
        self._fit_X_only(X)
        return self


def _get_weights(dist, weights):
    """sklearn ``_get_weights`` on host arrays (neighbors.py:174-199): None for
    uniform, 1/d with the coincident-row indicator rule, or the callable's."""
    if weights == "uniform":
        return None
    if weights == "distance":
        with np.errstate(divide="ignore"):
            w = 1.0 / dist
        inf_mask = np.isinf(w)
        inf_row = np.any(inf_mask, axis=1)
        w[inf_row] = inf_mask[inf_row]
        return w
    return weights(dist)


def _check_weights(weights):
    if weights in ("uniform", "distance") or callable(weights):
        return weights
    raise ValueError("weights not recognized: should be 'uniform', 'distance', or a callable function")


def _out(t, was_numpy):
    return t.cpu().numpy() if was_numpy else t


class KNeighborsRegressor(_NeighborsBase):
    """k-NN regression (mlrs.neighbors.KNeighborsRegressor, neighbors.py:1036-1156):
    the weighted mean of each query's k neighbour targets, formed on the device."""

    def __init__(self, n_neighbors=5, output_type="input", *, weights="uniform", algorithm="auto", leaf_size=30,
                 p=2, metric="minkowski", metric_params=None, n_jobs=None, device="auto"):
        self.n_neighbors = n_neighbors
        self.output_type = output_type
        self.weights = weights
        self.algorithm = algorithm
        self.leaf_size = leaf_size
        self.p = p
        self.metric = metric
        self.metric_params = metric_params
        self.n_jobs = n_jobs
        self.device = device

    def fit(self, X, y):
        _check_weights(self.weights)
        t = self._fit_X_only(X)
        yt = y if isinstance(y, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(y)))
        if yt.dim() == 2 and yt.shape[1] == 1:
            yt = yt.reshape(-1)
        if yt.dim() not in (1, 2) or yt.shape[0] != t.shape[0]:
            raise ValueError("Found input variables with inconsistent numbers of samples: [%d, %d]"
                             % (t.shape[0], yt.shape[0]))
        self._y_dev = yt.to(device=t.device, dtype=t.dtype).contiguous()
        _check_finite(self._y_dev.reshape(-1, 1))
        return self

    @property
    def _y(self):
        self._check_fitted()
        return self._y_dev.cpu().numpy()

    def predict(self, X):
        q, was_numpy = self._query(X)
        k = int(self.n_neighbors)
        if k > self.n_samples_fit_:
            raise ValueError("Expected n_neighbors <= n_samples_fit, but n_neighbors = %d, n_samples_fit = %d"
                             % (k, self.n_samples_fit_))
        dist, idx = self._raw_kneighbors(q, k)
        if callable(self.weights):
            d = dist.double().cpu().numpy()
            i = (idx.to(torch.int64) & 0xFFFFFFFF).cpu().numpy()
            w = _get_weights(d, self.weights)
            yn = self._y[i]
            if w is None:
                pred = np.mean(yn, axis=1)
            elif yn.ndim == 3:
                pred = np.sum(yn * w[:, :, None], axis=1) / np.sum(w, axis=1)[:, None]
            else:
                pred = np.sum(yn * w, axis=1) / np.sum(w, axis=1)
            pred = torch.from_numpy(np.ascontiguousarray(pred.astype(self._y.dtype))).to(q.device)
        else:
            pred = prims.knn_regress(self._y_dev, idx, dist, weighted=self.weights == "distance")
        return _out(pred, was_numpy)


class KNeighborsClassifier(_NeighborsBase):
    """k-NN classification (mlrs.neighbors.KNeighborsClassifier, neighbors.py:767-1033):
    labels are encoded to dense codes here (np.unique), the vote runs on the
    device and the argmax code is mapped back through ``classes_``."""

    def __init__(self, n_neighbors=5, output_type="input", *, weights="uniform", algorithm="auto", leaf_size=30,
                 p=2, metric="minkowski", metric_params=None, n_jobs=None, device="auto"):
        self.n_neighbors = n_neighbors
        self.output_type = output_type
        self.weights = weights
        self.algorithm = algorithm
        self.leaf_size = leaf_size
        self.p = p
        self.metric = metric
        self.metric_params = metric_params
        self.n_jobs = n_jobs
        self.device = device

    def fit(self, X, y):
        _check_weights(self.weights)
        t = self._fit_X_only(X)
        y = np.asarray(y.cpu().numpy() if isinstance(y, torch.Tensor) else y)
        if y.ndim == 2 and y.shape[1] == 1:
            warnings.warn("A column-vector y was passed when a 1d array was expected. Please change the shape "
                          "of y to (n_samples,), for example using ravel().", UserWarning, stacklevel=2)
            y = y.ravel()
        if y.shape[0] != t.shape[0]:
            raise ValueError("Found input variables with inconsistent numbers of samples: [%d, %d]"
                             % (t.shape[0], y.shape[0]))
        self.outputs_2d_ = y.ndim == 2
        y2 = y.reshape(-1, 1) if not self.outputs_2d_ else y
        classes, codes = [], np.empty(y2.shape, dtype=np.int64)
        for col in range(y2.shape[1]):
            cls, inv = np.unique(y2[:, col], return_inverse=True)
            classes.append(cls)
            codes[:, col] = np.asarray(inv).ravel()
        self.classes_ = classes if self.outputs_2d_ else classes[0]
        self._codes = codes if self.outputs_2d_ else codes.ravel()
        self._codes_dev = torch.from_numpy(np.ascontiguousarray(codes[:, 0].astype(np.int32))).to(t.device)
        return self

    @property
    def _y(self):
        self._check_fitted()
        return self._codes

    def _neighbours(self, q):
        k = int(self.n_neighbors)
        if k > self.n_samples_fit_:
            raise ValueError("Expected n_neighbors <= n_samples_fit, but n_neighbors = %d, n_samples_fit = %d"
                             % (k, self.n_samples_fit_))
        return self._raw_kneighbors(q, k)

    def _host_proba(self, dist, idx):
        """sklearn's predict_proba body on host arrays (neighbors.py:914-955)."""
        d = dist.double().cpu().numpy()
        i = (idx.to(torch.int64) & 0xFFFFFFFF).cpu().numpy()
        w = _get_weights(d, self.weights)
        if w is None:
            w = np.ones_like(i, dtype=np.float64)
        elif np.any(np.all(w == 0, axis=1)):
            raise ValueError("All neighbors of some sample is getting zero weights. "
                             "Please modify 'weights' to avoid this case.")
        classes_ = self.classes_ if self.outputs_2d_ else [self.classes_]
        codes = self._codes if self.outputs_2d_ else self._codes.reshape(-1, 1)
        rows = np.arange(i.shape[0])
        out = []
        for kk, classes_k in enumerate(classes_):
            lab = codes[:, kk][i]
            proba = np.zeros((i.shape[0], classes_k.size), dtype=np.float64)
            for j, col in enumerate(lab.T):
                proba[rows, col] += w[:, j]
            norm = proba.sum(axis=1)[:, None]
            norm[norm == 0.0] = 1.0
            out.append(proba / norm)
        return out

    def _needs_host_vote(self):
        return self.outputs_2d_ or callable(self.weights)

    def predict(self, X):
        q, was_numpy = self._query(X)
        dist, idx = self._neighbours(q)
        if self._needs_host_vote():
            probas = self._host_proba(dist, idx)
            classes_ = self.classes_ if self.outputs_2d_ else [self.classes_]
            out = np.stack([c.take(np.argmax(pk, axis=1)) for c, pk in zip(classes_, probas)], axis=1)
            return out if self.outputs_2d_ else out.ravel()
        _, labels = prims.knn_classify(self._codes_dev, len(self.classes_), idx, dist,
                                       weighted=self.weights == "distance", dtype=q.dtype)
        return self.classes_.take(labels.cpu().numpy())

    def predict_proba(self, X):
        q, was_numpy = self._query(X)
        dist, idx = self._neighbours(q)
        if self._needs_host_vote():
            probas = self._host_proba(dist, idx)
            if self.outputs_2d_:
                return probas
            return probas[0].astype(np.float32 if q.dtype == torch.float32 else np.float64)
        proba, _ = prims.knn_classify(self._codes_dev, len(self.classes_), idx, dist,
                                      weighted=self.weights == "distance", dtype=q.dtype)
        return _out(proba, was_numpy)


def knn_graph(X, k, metric="euclidean", p=2.0, include_self=False):
    """Directed k-nearest graph of the rows of ``X`` against themselves, as the
    reference builds it for UMAP (include_self=False) and HDBSCAN
    (include_self=True): ``(indices int64 (n, k), distances float64 (n, k))``
    as device tensors, in the reference host scan's f64 arithmetic."""
    t, _ = _as_device_matrix(X)
    return prims.knn_graph(t, k, metric, p=p, include_self=include_self)


def hdbscan_core_distances(X, min_samples, metric="euclidean", p=2.0):
    """HDBSCAN core distances (float64 device tensor of n): the distance from
    each row to its ``min_samples``-th nearest row, itself included."""
    t, _ = _as_device_matrix(X)
    return prims.core_distances(t, min_samples, metric, p=p)


def kneighbors(X_train, X_query, k, metric="euclidean"):
    """Functional form: ``(distances, int64 indices)`` as device tensors."""
    t, _ = _as_device_matrix(X_train)
    q, _ = _as_device_matrix(X_query, dtype=t.dtype, device=t.device)
    return prims.knn_topk(q, t, k, metric)
