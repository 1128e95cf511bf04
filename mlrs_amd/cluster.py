"""k-means over the HIP engine: ``KMeans.fit`` / ``predict`` of mlrs
(crates/mlrs-algos/src/cluster/kmeans.rs, python/mlrs/cluster.py:18-183).

``fit`` runs the whole loop on the device (mlrs_kmeans_fit_*): k-means++ /
random / explicit initialisation on SplitMix64, the fused nearest-centre
assignment, the centroid sums over the reference's row blocks, empty-cluster
relocation, the f64 mean update and the reference's stopping rules, restarts
kept by lowest inertia.  ``predict`` is the fused k=1 assignment: labels are
the index of the nearest centre under squared Euclidean distance accumulated
as (x-c)*(x-c) with separate multiply and add, ties to the lowest centre.
"""
import numpy as np
import torch

from . import prims
from .neighbors import _as_device_matrix, _check_finite


def assign(X, centers):
    """``(labels int64, squared distances)`` as device tensors."""
    x, _ = _as_device_matrix(X)
    c, _ = _as_device_matrix(centers, dtype=x.dtype, device=x.device)
    return prims.kmeans_assign(x, c)


class KMeans:
    """k-means clustering with sklearn's parameter set (python/mlrs/cluster.py:18-183).

    ``init``: "k-means++", "random", an array of shape (n_clusters, n_features)
    or a callable ``init(X, k, random_state=...)`` (evaluated once at ``fit``
    and used as an explicit init).  ``n_init="auto"`` resolves to 1 for
    k-means++ and explicit inits, 10 for "random".  ``algorithm`` "lloyd" or
    "elkan" -- the bound-pruned assignment, which returns the same fit as
    Lloyd (as the reference's Elkan does).  ``random_state=None`` is seed 0.
    ``verbose`` / ``copy_x`` are accepted and have no effect.
    ``cluster_centers=`` sets fitted centres directly (``predict`` without ``fit``).
    """

    def __init__(self, n_clusters=8, init="k-means++", n_init="auto", max_iter=300, tol=1e-4, verbose=0,
                 random_state=None, copy_x=True, algorithm="lloyd", output_type="input", *, cluster_centers=None):
        self.n_clusters = n_clusters
        self.init = init
        self.n_init = n_init
        self.max_iter = max_iter
        self.tol = tol
        self.verbose = verbose
        self.random_state = random_state
        self.copy_x = copy_x
        self.algorithm = algorithm
        self.output_type = output_type
        if cluster_centers is not None:
            self.set_centers(cluster_centers)

    def set_centers(self, centers):
        c, _ = _as_device_matrix(centers)
        _check_finite(c)
        self._centers_dev = c
        self.cluster_centers_ = c.cpu().numpy()
        self.n_clusters = c.shape[0]
        self.n_features_in_ = c.shape[1]
        return self

    def _check_fitted(self):
        if not hasattr(self, "_centers_dev"):
            raise ValueError("This KMeans instance is not fitted yet.")

    def _resolve_init(self, X_np, cols):
        init = self.init
        if isinstance(init, str):
            if init not in ("k-means++", "random"):
                raise ValueError("init should be 'k-means++', 'random', an array or a callable, got %r" % (init,))
            return init, None
        if callable(init):
            rs = np.random.RandomState(0 if self.random_state is None else int(self.random_state))
            init = init(X_np, self.n_clusters, random_state=rs)
        arr = np.ascontiguousarray(init, dtype=np.float64)
        if arr.shape != (self.n_clusters, cols):
            raise ValueError("init has shape %s, expected (%d, %d)" % (arr.shape, self.n_clusters, cols))
        return "array", arr

    def _resolve_n_init(self, init_kind):
        n_init = self.n_init
        if isinstance(n_init, str):
            if n_init != "auto":
                raise ValueError("unknown n_init %r (the only legal string is 'auto')" % (n_init,))
            return 10 if init_kind == "random" else 1
        if int(n_init) < 1:
            raise ValueError("n_init should be > 0, got %r instead." % (n_init,))
        return int(n_init)

    def fit(self, X, y=None):
        x, _ = _as_device_matrix(X)
        _check_finite(x)
        n, d = x.shape
        k = int(self.n_clusters)
        if self.algorithm not in ("lloyd", "elkan"):
            raise ValueError("algorithm should be 'lloyd' or 'elkan', got %r" % (self.algorithm,))
        if not (float(self.tol) >= 0.0):
            raise ValueError("tol should be >= 0, got %r" % (self.tol,))
        if int(self.max_iter) < 1:
            raise ValueError("max_iter should be > 0, got %r" % (self.max_iter,))
        x_np = None
        if callable(self.init):
            x_np = x.cpu().numpy()
        init_kind, arr = self._resolve_init(x_np, d)
        n_init = self._resolve_n_init(init_kind)
        ini = torch.from_numpy(arr).to(device=x.device, dtype=x.dtype) if arr is not None else None
        seed = 0 if self.random_state is None else int(self.random_state)
        algorithm = "lloyd" if k == 1 else self.algorithm
        centers, labels, inertia, n_iter = prims.kmeans_fit(x, k, init_kind, ini, seed=seed, n_init=n_init,
                                                            max_iter=int(self.max_iter), tol=float(self.tol),
                                                            algorithm=algorithm)
        self._centers_dev = centers
        self.cluster_centers_ = centers.cpu().numpy()
        self.labels_ = labels.to(torch.int32).cpu().numpy()
        np_dtype = np.float32 if x.dtype == torch.float32 else np.float64
        self.inertia_ = np_dtype(inertia)
        self.n_iter_ = n_iter
        self.n_features_in_ = d
        self._n_init = n_init
        self._algorithm = algorithm
        return self

    def fit_predict(self, X, y=None):
        return self.fit(X).labels_

    def predict(self, X):
        self._check_fitted()
        x, was_numpy = _as_device_matrix(X, dtype=self._centers_dev.dtype, device=self._centers_dev.device)
        if x.shape[1] != self.n_features_in_:
            raise ValueError("X has %d features, but KMeans is expecting %d features as input"
                             % (x.shape[1], self.n_features_in_))
        _check_finite(x)
        labels, _ = prims.kmeans_assign(x, self._centers_dev)
        labels = labels.to(torch.int32)
        return labels.cpu().numpy() if was_numpy else labels

    def transform_min_sqdist(self, X):
        """Per-row squared distance to the assigned centre (the inertia terms)."""
        self._check_fitted()
        x, was_numpy = _as_device_matrix(X, dtype=self._centers_dev.dtype, device=self._centers_dev.device)
        _, d = prims.kmeans_assign(x, self._centers_dev)
        return d.cpu().numpy() if was_numpy else d


def predict_labels(X, centers):
    labels, _ = assign(X, centers)
    return labels.to(torch.int32).cpu().numpy() if not isinstance(X, torch.Tensor) else labels.to(torch.int32)


__all__ = ["KMeans", "assign", "predict_labels"]
