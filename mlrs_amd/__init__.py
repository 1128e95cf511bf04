"""mlrs_amd -- MI355X (gfx950) brute-force k-nearest-neighbour engine for mlrs.

The compute lives in ``libmlrs_hip_knn.so`` (hand-written HIP, C ABI in
``include/mlrs_hip_knn.h``); this package is the host-side mirror of the mlrs
interface for that path:

* ``mlrs_amd.prims``      -- device-tensor primitives: knn_topk, radius_neighbors,
                             knn_graph, core_distances, kmeans_assign,
                             kmeans_fit, pairwise_distance, row_sqnorms,
                             knn_regress / knn_classify, device_copy, pool_stats
* ``mlrs_amd.neighbors``  -- ``NearestNeighbors`` (fit / kneighbors /
                             kneighbors_graph / radius_neighbors[_graph]),
                             ``KNeighborsRegressor``, ``KNeighborsClassifier``,
                             ``knn_graph``, ``hdbscan_core_distances``
* ``mlrs_amd.cluster``    -- ``KMeans`` (fit / predict / fit_predict)
* ``mlrs_amd.synthetic``  -- the seeded benchmark/test workloads
* ``mlrs_amd.build``      -- the hipcc build of the library (gfx950)
"""
from . import _lib  # noqa: F401

__version__ = "0.1.0"


def library_path():
    return _lib.LIB_PATH
