"""mlrs_amd -- MI355X (gfx950) brute-force k-nearest-neighbour engine for mlrs.

The compute lives in ``libmlrs_hip_knn.so`` (hand-written HIP, C ABI in
``include/mlrs_hip_knn.h``); this package is the host-side mirror of the mlrs
interface for that path:

* ``mlrs_amd.prims``      -- device-tensor primitives (knn_topk, kmeans_assign,
                             pairwise_distance, row_sqnorms)
* ``mlrs_amd.neighbors``  -- ``NearestNeighbors`` (fit / kneighbors)
* ``mlrs_amd.cluster``    -- ``KMeans.predict`` (nearest-centre assignment)
* ``mlrs_amd.synthetic``  -- the seeded benchmark/test workloads
"""
from . import _lib  # noqa: F401

__version__ = "0.1.0"


def library_path():
    return _lib.LIB_PATH
