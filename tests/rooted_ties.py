"""Constructed X-vs-X data whose graph depends on ranking by the root.

The host scans (crates/mlrs-algos/src/manifold/umap_host_knn.rs:171-198, 494)
push the final distance, so two rows whose aggregates differ by one ulp but
root to the same double are ordered by index.  Each group below is a query
row c = (100 g, 0) with rows at offsets whose squared (or fourth-power)
differences are exact:

  L  = c + (a, y)   aggregate a^2 + y^2 = A + 1 ulp   (the lower index)
  H  = c + (a, 0)   aggregate a^2 = A                (the higher index)

Euclidean: a = 1.25, y = 2^-26, so A = 1.5625 (ulp 2^-52) and A + 2^-52 both
have the square root 1.25 (the second is 0.4 ulp above it).  Minkowski p = 4:
a = 1, y = 2^-13, so A = 1 and A + 2^-52 both have the fourth root 1 (the
second is 0.25 ulp above it).  Ranking by the aggregate puts H first; ranking
by the root puts L first.  Every coordinate is an f32 value, so the f32 entry
points (which widen to f64) see the same aggregates.

Groups (each at its own c, 100 apart, so groups never meet):
  boundary  k - 1 nearer rows, then L and H: the k-th neighbour is L
  inside    k - 3 nearer rows, L and H, then farther rows: L before H
  heavy     4 L rows (lower indices) and 60 copies of H: more ties of one
            root than a list keeps, so the device's lists drop some of them
"""
import numpy as np

CASES = {"euclidean": (1.25, 2.0 ** -26, 2.0), "minkowski": (1.0, 2.0 ** -13, 4.0)}


def build(metric, k):
    """Rows (n x 2, f64 holding f32 values) and the Minkowski p; 6 <= k <= 32."""
    assert 6 <= k <= 32
    a, y, p = CASES[metric]
    rows = []
    g = 0

    def center():
        return 100.0 * g

    # boundary group
    c = center()
    rows += [(c + a, y)]                     # L (lower index)
    rows += [(c, 0.0)]                       # the query
    rows += [(c + (j + 1) / 32.0, 0.0) for j in range(k - 1)]  # nearer (k - 1 rows, below a)
    rows += [(c + a, 0.0)]                   # H
    rows += [(c + 3.0 + j, 0.0) for j in range(4)]  # far
    g += 1
    # inside group
    c = center()
    rows += [(c + a, y), (c, 0.0)]
    rows += [(c + (j + 1) / 32.0, 0.0) for j in range(k - 3)]
    rows += [(c + a, 0.0)]
    rows += [(c + 1.5 + 0.25 * j, 0.0) for j in range(6)]
    g += 1
    # heavy group
    c = center()
    rows += [(c + a, y) for _ in range(4)]
    rows += [(c, 0.0)]
    rows += [(c + (j + 1) / 32.0, 0.0) for j in range(max(k - 6, 0))]
    rows += [(c + a, 0.0) for _ in range(60)]
    rows += [(c + 3.0 + j, 0.0) for j in range(4)]
    x = np.array(rows, dtype=np.float64)
    assert np.array_equal(x.astype(np.float32).astype(np.float64), x), "coordinates must be f32 values"
    return x, p


def brute_graph(x, k, metric, p, by_root, include_self=False):
    """(index, distance) lists from plain numpy f64 arithmetic in the host
    scan's operation order, ranked by (root, index) or, for contrast, by
    (aggregate, index)."""
    n = x.shape[0]
    idx = np.zeros((n, k), dtype=np.int64)
    dist = np.zeros((n, k))
    for i in range(n):
        agg = np.zeros(n)
        for c in range(x.shape[1]):
            diff = x[i, c] - x[:, c]
            agg = agg + (diff * diff if metric == "euclidean" else np.abs(diff) ** p)
        root = np.sqrt(agg) if metric == "euclidean" else agg ** (1.0 / p)
        order = np.lexsort((np.arange(n), root if by_root else agg))
        if not include_self:
            order = order[order != i]
        idx[i] = order[:k]
        dist[i] = root[order[:k]]
    return idx, dist
