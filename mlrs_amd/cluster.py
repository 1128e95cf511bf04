"""k-means nearest-centre assignment over the HIP engine.

``KMeans.predict`` / ``predict_labels`` of mlrs
(crates/mlrs-algos/src/cluster/kmeans.rs:1583-1649, python/mlrs/cluster.py:
142-144): labels are the index of the nearest centre under squared Euclidean
distance accumulated as (x-c)*(x-c) with separate multiply and add, ties to
the lowest centre index -- one fused k=1 search, no n x n_centers staging.
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
    """Assignment half of ``mlrs.cluster.KMeans``: ``predict`` against set centres."""

    def __init__(self, n_clusters=8, *, cluster_centers=None):
        self.n_clusters = n_clusters
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
