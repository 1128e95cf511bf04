/*
 * mlrs_hip_knn.h -- C ABI of the MI355X (gfx950) brute-force kNN engine.
 *
 * Drop-in replacement for the kernel launches behind mlrs-backend's
 * brute-force kNN / k-means-assignment / pairwise-distance prims.  Every entry
 * point:
 *   - takes DEVICE pointers (HIP, owned by the caller) plus each buffer's
 *     element count, so the geometry checks of the Rust prims can run here;
 *   - validates everything BEFORE any launch and returns 0 or a negative
 *     MLRS_ERR_* code; mlrs_last_error() then describes the failure with the
 *     same fields as mlrs_core::PrimError (crates/mlrs-core/src/error.rs:62);
 *   - enqueues its work on `stream` (a hipStream_t; NULL = the null stream)
 *     and returns without synchronizing, except when it must grow one of its
 *     cached device buffers: growth synchronizes the WHOLE device (every
 *     stream, other libraries' work included) before freeing the old buffer;
 *   - is callable from any thread, one call at a time per process (the
 *     Rust side serializes through its global pool mutex,
 *     crates/mlrs-py/src/lib.rs:104-186); calls are serialized internally;
 *   - runs after the previous call on the same device even when the two
 *     calls name different streams: the cached buffers are shared, so a call
 *     on another stream than the last call's first makes its stream wait for
 *     the last call's work (an event recorded at the end of every call), as
 *     the reference's single stream orders them
 *     (crates/mlrs-backend/src/stream_cap.rs:69).  The caller still orders
 *     its own reads of the outputs after the call's stream.
 * Results equal mlrs's cpu-backend arithmetic bit for bit: the same arm
 * (direct / metric / host) the cpu dispatch would pick for the shape
 * (crates/mlrs-algos/src/neighbors/nearest.rs:891-953) is evaluated in the same
 * operation order, and selection uses the (value, index) order with the lowest
 * index winning ties.
 */
#ifndef MLRS_HIP_KNN_H
#define MLRS_HIP_KNN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define MLRS_OK 0
#define MLRS_ERR_SHAPE_MISMATCH (-1) /* PrimError::ShapeMismatch{operand, rows, cols, len} */
#define MLRS_ERR_DIM_MISMATCH (-2)   /* PrimError::DimMismatch{dim(operand), lhs(rows), rhs(cols)} */
#define MLRS_ERR_UNSUPPORTED (-3)    /* metric or shape this build does not serve */
#define MLRS_ERR_NULL_POINTER (-4)   /* a required pointer was NULL */
#define MLRS_ERR_HIP (-5)            /* a HIP runtime call failed (hip_error holds it) */
#define MLRS_ERR_ALLOC (-6)          /* device workspace allocation failed */
#define MLRS_ERR_INVALID_PARAM (-7)  /* AlgoError::InvalidEps-style rejection of a scalar (operand names it) */

/* ---- metrics: the variants of the Metric enum of crates/mlrs-backend/src/prims/knn_graph.rs:61-75
 *      (numbered here, not in the enum's declaration order) ---- */
#define MLRS_METRIC_EUCLIDEAN 0
#define MLRS_METRIC_COSINE 1
#define MLRS_METRIC_MANHATTAN 2
#define MLRS_METRIC_CHEBYSHEV 3
#define MLRS_METRIC_MINKOWSKI 4 /* exponent in the `p` argument, p >= 1 */

typedef struct mlrs_error_info {
    int32_t code;        /* the MLRS_ERR_* value returned */
    char operand[32];    /* PrimError operand / dim name, e.g. "x", "y", "k", "out" */
    int64_t rows;        /* ShapeMismatch rows   | DimMismatch lhs */
    int64_t cols;        /* ShapeMismatch cols   | DimMismatch rhs */
    int64_t len;         /* ShapeMismatch len */
    int32_t hip_error;   /* hipError_t for MLRS_ERR_HIP / MLRS_ERR_ALLOC */
    char message[160];   /* human-readable, PrimError's Display text */
} mlrs_error_info;

/* Details of the calling thread's last failed call. Returns its code. */
int32_t mlrs_last_error(mlrs_error_info *out);
/* Static description of a status code. */
const char *mlrs_status_string(int32_t code);
/* ABI version of this header (bumped on any signature change). */
int32_t mlrs_abi_version(void);
#define MLRS_ABI_VERSION 5

/*
 * Brute-force k nearest training rows of every query row.
 *
 * Replaces: the arm chosen by metric_topk (nearest.rs:891-953) --
 *   cpu_rows_topk (crates/mlrs-backend/src/prims/knn.rs:491-671),
 *   cpu_metric_rows_topk (prims/knn.rs:732-898),
 *   knn_host_topk (crates/mlrs-backend/src/prims/knn_host.rs:210-304),
 *   fused_distance_topk (prims/knn.rs:1070-1323) and
 *   tiled_distance_topk / tiled_metric_distance_topk (nearest.rs:1058-1512).
 * Layout: xq is n_query x n_features, x_train n_train x n_features, both
 *   row-major; out_dist / out_idx are n_query x k row-major, each row ascending
 *   by (distance, index).  Distances are TRUE distances (Euclidean: the root of
 *   the selected squared values; cosine: 1 - cos, clamped to [0, 2];
 *   Manhattan: sum |x-y|; Chebyshev: max |x-y| by select, NaN never replacing;
 *   Minkowski: (sum |x-y|^p)^(1/p), |x-y|^p by a multiply chain for an integer
 *   p in 3..8 (minkowski_powi, prims/knn.rs:680-687), pow otherwise, and the
 *   root pow(v, (F)(1/p)) on the selected values).  A slot no admissible
 *   (non-NaN) candidate filled holds (+inf, 0).
 * Errors (checked in this order, before any launch, mirroring
 *   cpu_metric_rows_topk / knn_host_topk):
 *   ShapeMismatch "x"        n_query*n_features != xq_len
 *   ShapeMismatch "y"        n_train*n_features != xt_len
 *   ShapeMismatch "k"        k < 1 or k > n_train           (rows=1, cols=k, len=n_train)
 *   ShapeMismatch "features" n_features < 1
 *   ShapeMismatch "rows"     n_query or n_train > UINT32_MAX
 *   ShapeMismatch "out"      out_len != n_query*k
 *   MLRS_ERR_UNSUPPORTED     metric not served, or a Minkowski p below 1 (or NaN)
 * Every 1 <= k <= n_train is served (knn_host_possible,
 *   crates/mlrs-backend/src/prims/knn_host.rs:182-184; top_k,
 *   crates/mlrs-backend/src/prims/topk.rs:208-212).
 * `p` is the Minkowski exponent, ignored by the other metrics.
 */
int32_t mlrs_knn_topk_f32(const float *xq, int64_t xq_len, int64_t n_query, int64_t n_features,
                          const float *x_train, int64_t xt_len, int64_t n_train, int32_t k,
                          int32_t metric, double p, float *out_dist, uint32_t *out_idx,
                          int64_t out_len, void *stream);
int32_t mlrs_knn_topk_f64(const double *xq, int64_t xq_len, int64_t n_query, int64_t n_features,
                          const double *x_train, int64_t xt_len, int64_t n_train, int32_t k,
                          int32_t metric, double p, double *out_dist, uint32_t *out_idx,
                          int64_t out_len, void *stream);
/* Largest k served for (dtype_bytes, n_features, metric): INT32_MAX, i.e.
 * every k up to n_train (the arguments are kept for ABI stability). */
int32_t mlrs_knn_max_k(int32_t dtype_bytes, int64_t n_features, int32_t metric);

/*
 * mlrs_knn_topk_f32 for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, validation,
 * kernels and bits as mlrs_knn_topk_f32; the only difference is where the
 * kernels' scratch (norms, per-segment lists, queued screen values, exact
 * tiles) lives: in a static device array of MLRS_NOALLOC_SCRATCH_BYTES per
 * GPU, held until the process ends, instead of the library's cached
 * workspace.  The call makes no hipMalloc / hipFree / allocating library
 * call; its first call on a device looks the array's device address
 * (hipGetSymbolAddress) and the CU count up once: make that first call, which
 * may have n_query = 0, outside a graph capture.  After it, calls can be
 * captured into a HIP graph (every step is a kernel launch: no memset, no
 * copy, no event) and replayed with new data in the same buffers.  A search
 * whose scratch would exceed the array
 * returns MLRS_ERR_UNSUPPORTED, operand "scratch" {rows = bytes needed,
 * len = MLRS_NOALLOC_SCRATCH_BYTES}, before any launch (the exact-tile path
 * sizes its tiles to fit; the Gram path at n_train = 1M, d = 128, k = 32
 * needs ~64 MiB for 10k queries).  Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (two streams, no ordering between
 * them) RACE -- order them yourself.  Not ordered against the other entry
 * points' calls (they use other memory), and no timing events are recorded.
 */
#define MLRS_NOALLOC_SCRATCH_BYTES 134217728 /* 128 MiB */
int32_t mlrs_knn_topk_f32_noalloc(const float *xq, int64_t xq_len, int64_t n_query, int64_t n_features,
                                  const float *x_train, int64_t xt_len, int64_t n_train, int32_t k,
                                  int32_t metric, double p, float *out_dist, uint32_t *out_idx,
                                  int64_t out_len, void *stream);

/*
 * Nearest-centre assignment (the k-means assignment step, k = 1 search).
 *
 * Replaces: assign_min (crates/mlrs-backend/src/prims/kmeans.rs:635-750) --
 *   dist_direct_2d_c4 + argmin_dist_rows (crates/mlrs-kernels/src/kmeans.rs:
 *   206-310) -- without its n x n_centers staging matrix.
 * Writes labels[i] = argmin_c ||x_i - c||^2 (lowest index on a tie; a NaN
 *   distance to centre 0 wins with label 0, as argmin_dist_rows seeds from
 *   centre 0) and sqdist[i] = that SQUARED distance.
 * Errors (validate_geometry, prims/kmeans.rs:1416-1454, then assign_min):
 *   ShapeMismatch "x"        n*n_features != x_len
 *   ShapeMismatch "k"        n_centers < 1 or n_centers > n
 *   ShapeMismatch "n"/"d"/"k" a dimension > UINT32_MAX
 *   ShapeMismatch "centers"  n_centers*n_features != centers_len
 *   ShapeMismatch "labels"   labels_len != n or dist_len != n
 * The reference's extra guard n*n_centers <= UINT32_MAX existed only for its
 * staging matrix, which this kernel does not have; it is not enforced.
 */
int32_t mlrs_kmeans_assign_f32(const float *x, int64_t x_len, int64_t n, int64_t n_features,
                               const float *centers, int64_t centers_len, int64_t n_centers,
                               uint32_t *labels, int64_t labels_len, float *sqdist, int64_t dist_len,
                               void *stream);
int32_t mlrs_kmeans_assign_f64(const double *x, int64_t x_len, int64_t n, int64_t n_features,
                               const double *centers, int64_t centers_len, int64_t n_centers,
                               uint32_t *labels, int64_t labels_len, double *sqdist, int64_t dist_len,
                               void *stream);

/*
 * Full pairwise distance matrix out[i*rows_y + j].
 *
 * Replaces: distance_direct (crates/mlrs-backend/src/prims/distance.rs:428-551,
 *   kernel euclidean_sq_dist, crates/mlrs-kernels/src/distance.rs:411-440) for
 *   MLRS_METRIC_EUCLIDEAN -- SQUARED distance, with the boundary root of
 *   sqrt_elem (crates/mlrs-kernels/src/elementwise.rs:131-136) when
 *   do_sqrt != 0 -- and metric_distance's cosine_dist
 *   (crates/mlrs-kernels/src/distance.rs:257-310) for MLRS_METRIC_COSINE.
 *   MLRS_METRIC_MANHATTAN / _CHEBYSHEV / _MINKOWSKI are manhattan_dist,
 *   chebyshev_dist and minkowski_dist (distance.rs:67-227; Minkowski with pow
 *   per feature and the root pow(acc, 1/p) with 1/p formed in F); do_sqrt is
 *   ignored for them, p is read for Minkowski only.
 * Errors (validate_geometry, prims/distance.rs:260-302):
 *   ShapeMismatch "x" / "y", DimMismatch "cols", ShapeMismatch "out".
 */
int32_t mlrs_pairwise_distance_f32(const float *x, int64_t x_len, int64_t rows_x, int64_t cols,
                                   const float *y, int64_t y_len, int64_t rows_y, int64_t cols_y,
                                   int32_t metric, int32_t do_sqrt, double p, float *out, int64_t out_len,
                                   void *stream);
int32_t mlrs_pairwise_distance_f64(const double *x, int64_t x_len, int64_t rows_x, int64_t cols,
                                   const double *y, int64_t y_len, int64_t rows_y, int64_t cols_y,
                                   int32_t metric, int32_t do_sqrt, double p, double *out, int64_t out_len,
                                   void *stream);

/*
 * Per-row squared L2 norms, out[r] = sum_c x[r,c]^2 accumulated in column
 * order with separate multiply and add.
 *
 * Replaces: row_sqnorms (crates/mlrs-backend/src/prims/kmeans.rs:805-832,
 *   kernel row_sqnorm, crates/mlrs-kernels/src/kmeans.rs:610) and the
 *   row_sumsq norm feeder (crates/mlrs-kernels/src/knn.rs:2130-2149).
 * Errors: ShapeMismatch "x" (n*n_features != x_len), ShapeMismatch "out".
 */
int32_t mlrs_row_sqnorms_f32(const float *x, int64_t x_len, int64_t n, int64_t n_features, float *out,
                             int64_t out_len, void *stream);
int32_t mlrs_row_sqnorms_f64(const double *x, int64_t x_len, int64_t n, int64_t n_features,
                             double *out, int64_t out_len, void *stream);

/*
 * kNN regressor prediction from a neighbour set (device-resident predict).
 *
 * Replaces: knn_regress_mean_gather (crates/mlrs-backend/src/prims/knn.rs:59-
 *   150, kernel knn_regress_mean, crates/mlrs-kernels/src/knn.rs:95-147) for
 *   weighted == 0 and n_outputs == 1, and knn_regress_gather_weighted
 *   (prims/knn.rs:151-323, kernel knn_regress_gather, knn.rs:197-316)
 *   otherwise.
 * Layout: y_train is n_train x n_outputs row-major; idx / dist are the
 *   n_query x k neighbour indices and TRUE distances of a search (dist is read
 *   only when weighted != 0 and may be NULL otherwise); out is n_query x
 *   n_outputs.  out = sum_j w_j y[idx_j] / sum_j w_j with w = 1 (uniform) or
 *   1/d (weighted; a row with a zero distance weighs its zero-distance
 *   neighbours 1 and the rest 0), both sums Neumaier-compensated.
 * Errors, before any launch: ShapeMismatch "k" (k < 1, n_query < 1,
 *   n_outputs < 1 or n_train < 1), "idx", "dist", "y_train", "n_query" /
 *   "n_train" / "n_outputs" (> UINT32_MAX), "out".  After the gather (the call
 *   synchronizes on `stream` to check): ShapeMismatch "knn.train_idx"
 *   {rows = first query row holding an index >= n_train, cols = k,
 *   len = n_train}; such an index contributes nothing.
 */
int32_t mlrs_knn_regress_f32(const float *y_train, int64_t y_len, int64_t n_train, int64_t n_outputs,
                             const uint32_t *idx, int64_t idx_len, const float *dist, int64_t dist_len,
                             int64_t n_query, int32_t k, int32_t weighted, float *out, int64_t out_len,
                             void *stream);
int32_t mlrs_knn_regress_f64(const double *y_train, int64_t y_len, int64_t n_train, int64_t n_outputs,
                             const uint32_t *idx, int64_t idx_len, const double *dist, int64_t dist_len,
                             int64_t n_query, int32_t k, int32_t weighted, double *out, int64_t out_len,
                             void *stream);

/*
 * kNN classifier vote from a neighbour set (device-resident predict).
 *
 * Replaces: KNeighborsClassifier::predict_proba_host / predict_labels_host
 *   (crates/mlrs-algos/src/neighbors/classifier.rs:782-930), the host f64
 *   vote after the search.
 * y_class holds each training row's DENSE class index (0..n_classes-1).
 *   proba (n_query x n_classes) = per-class sums of the f64 weights (1, or 1/d
 *   with the zero-distance indicator rule), divided by the row total (an
 *   all-zero row is left at zero), cast to F; labels (n_query) = the argmax
 *   over the F probabilities, lowest class index on a tie.
 * Errors, before any launch: ShapeMismatch "k", "idx", "dist", "n_classes",
 *   "proba", "labels".  After the vote (synchronizes on `stream`): the first
 *   bad neighbour in row-major order gives ShapeMismatch "knn.train_idx"
 *   {rows = the index, cols = 1, len = n_train} or "knn.class_id" {rows =
 *   max(class, 0), cols = 1, len = n_classes}.
 */
int32_t mlrs_knn_classify_f32(const int32_t *y_class, int64_t n_train, int32_t n_classes, const uint32_t *idx,
                              int64_t idx_len, const float *dist, int64_t dist_len, int64_t n_query, int32_t k,
                              int32_t weighted, float *proba, int64_t proba_len, int32_t *labels,
                              int64_t labels_len, void *stream);
int32_t mlrs_knn_classify_f64(const int32_t *y_class, int64_t n_train, int32_t n_classes, const uint32_t *idx,
                              int64_t idx_len, const double *dist, int64_t dist_len, int64_t n_query, int32_t k,
                              int32_t weighted, double *proba, int64_t proba_len, int32_t *labels,
                              int64_t labels_len, void *stream);

/*
 * Every training row within `radius` of each query row.
 *
 * Replaces: radius_neighbor_indices_metric (crates/mlrs-algos/src/neighbors/
 *   nearest.rs:609-749) with its default arm, radius_host_scan
 *   (crates/mlrs-backend/src/prims/radius_host.rs:140-234); the result is the
 *   RadiusNeighbors layout (nearest.rs:564-582): counts[q] (n_query, device)
 *   is row q's match count, and out_dist / out_idx (device) hold the matches
 *   of row 0, then row 1, ..., each row's in ascending training index -- a CSR
 *   matrix without its indptr.  Values are the host scan's: the knn_host lane
 *   arithmetic compared as `v <= th` against th = (F)(radius^2 | radius^p |
 *   radius) formed in f64 (NaN never matches), then sqrt (Euclidean),
 *   pow(v, (F)(1/p)) (Minkowski) or identity on the matches; indices are the
 *   training row numbers as int32.
 * Sizes: *total (host) receives the number of matches.  With out_dist and
 *   out_idx both NULL the call only counts (counts and *total filled).  With
 *   buffers of `capacity` entries and *total > capacity nothing is written to
 *   them and the call returns ShapeMismatch "out" {rows = total, cols = 1,
 *   len = capacity}.  The usual sequence is a counting call, then a call with
 *   buffers of the returned size and otherwise the same arguments, which
 *   starts from the first call's counts (the second call re-checks them and
 *   counts again if the data changed in between).  A call that brings
 *   buffers without a counting call before it (a caller that knows a bound
 *   on the total, e.g. from an earlier search) is served by one pass when
 *   the f32 matrix-core path keeps every strip's matches (at most 1,024 per
 *   strip and row): they are counted, kept and copied into place in the
 *   same call.  Buffers too small: as above, and the counts are kept for
 *   the next call.
 * Errors, before any launch: InvalidParam "radius" (radius not >= 0, NaN
 *   included; the text of AlgoError::InvalidEps), ShapeMismatch "xq" (n_query
 *   or n_features zero, or a length mismatch), DimMismatch "n_features",
 *   ShapeMismatch "y" / "rows" (n_train above u32::MAX) / "counts",
 *   Unsupported "metric" / "p" (Minkowski p < 1).
 * Synchronous: returns after `stream` has finished the call's work.
 */
int32_t mlrs_radius_neighbors_f32(const float *xq, int64_t xq_len, int64_t n_query, int64_t n_features,
                                  const float *x_train, int64_t x_train_len, int64_t n_train,
                                  int64_t train_features, int32_t metric, double p, double radius, uint32_t *counts,
                                  int64_t counts_len, float *out_dist, int32_t *out_idx, int64_t capacity,
                                  int64_t *total, void *stream);
int32_t mlrs_radius_neighbors_f64(const double *xq, int64_t xq_len, int64_t n_query, int64_t n_features,
                                  const double *x_train, int64_t x_train_len, int64_t n_train,
                                  int64_t train_features, int32_t metric, double p, double radius, uint32_t *counts,
                                  int64_t counts_len, double *out_dist, int32_t *out_idx, int64_t capacity,
                                  int64_t *total, void *stream);

/*
 * Directed k-nearest-neighbour graph of a row set against itself.
 *
 * Replaces: knn_graph (crates/mlrs-backend/src/prims/knn_graph.rs:180-311) as
 *   the cpu backend serves its callers, through host_knn (crates/mlrs-algos/src/
 *   manifold/umap_host_knn.rs:212-515, UMAP, include_self = 0) and the
 *   self-inclusive graph HDBSCAN reads (include_self = 1).  The arithmetic is
 *   that host scan's, in f64 (f32 rows are widened first): Euclidean
 *   sqrt(sum diff*diff), cosine 0.5*|x^ - y^|^2 over L2-normalised rows,
 *   Manhattan, Chebyshev (NaN never replaces the running max), Minkowski
 *   pow(sum pow(|diff|, p), 1/p).  out_idx / out_dist (n x k, device): per row
 *   ascending (distance, index); include_self = 0 leaves out the row's own
 *   index (by identity, not by distance: a duplicate point stays); an entry
 *   the scan cannot fill is (0, 0.0).  As in the host scan's KNearest
 *   (umap_host_knn.rs:171-198, pushing the final distance at :494), the lists
 *   are ranked by the final distance, not by the aggregate before the root:
 *   two aggregates that root to the same double are ordered by index.
 * Errors (knn_graph.rs:475-539): ShapeMismatch "x" {n, d, len} (or a
 *   dimension above u32::MAX), "k" {1, k, max_k} with max_k = n - 1 (n with
 *   include_self), "p" {1, 0, 1} (Minkowski p < 1), "out"; Unsupported
 *   "metric".  Every k up to max_k is served.
 */
int32_t mlrs_knn_graph_f32(const float *x, int64_t x_len, int64_t n, int64_t n_features, int64_t k, int32_t metric,
                           double p, int32_t include_self, uint32_t *out_idx, double *out_dist, int64_t out_len,
                           void *stream);
int32_t mlrs_knn_graph_f64(const double *x, int64_t x_len, int64_t n, int64_t n_features, int64_t k,
                           int32_t metric, double p, int32_t include_self, uint32_t *out_idx, double *out_dist,
                           int64_t out_len, void *stream);

/*
 * HDBSCAN core distances: out[i] (n, device, f64) = the (k-1)-th smallest
 *   distance from row i to every row, itself included, k = clamp(min_samples,
 *   1, n); +inf when fewer than k distances are finite.
 * Replaces: the core-distance step of feature_metric_single_linkage
 *   (crates/mlrs-algos/src/cluster/hdbscan.rs:1495-1566), served on the cpu
 *   backend by core_distances_host (cluster/hdbscan/host_core.rs:253-540); same
 *   f64 arithmetic as mlrs_knn_graph_*.  Cosine is not served (the reference
 *   takes cosine core distances from a dense matrix): Unsupported "metric".
 */
int32_t mlrs_hdbscan_core_distances_f32(const float *x, int64_t x_len, int64_t n, int64_t n_features,
                                        int32_t metric, double p, int64_t min_samples, double *out, int64_t out_len,
                                        void *stream);
int32_t mlrs_hdbscan_core_distances_f64(const double *x, int64_t x_len, int64_t n, int64_t n_features,
                                        int32_t metric, double p, int64_t min_samples, double *out, int64_t out_len,
                                        void *stream);

/*
 * k-means fit: restarts, initialisation and the Lloyd loop around the fused
 * nearest-centre assignment.
 *
 * Replaces: KMeans::fit (crates/mlrs-algos/src/cluster/kmeans.rs:1353-1580)
 *   with single_run (:929-1155) and the prims it drives (crates/mlrs-backend/
 *   src/prims/kmeans.rs): feature_mean_var (tol scaled by the mean feature
 *   variance), kmeanspp_sample / random_sample on SplitMix64 seeded
 *   seed + restart, assign_min, centroid_sums_dev (F sums over the reference's
 *   row blocks, block partials summed in order, widened to f64),
 *   relocate_empty_clusters, the f64 mean update, the strict label-equality
 *   break then the tol break, inertia_rows + sum_device, and the restart rule
 *   (strictly lower inertia on a partition that is not a relabelling).
 * algorithm: MLRS_KMEANS_LLOYD runs the fused k = 1 assignment over every row
 *   each iteration (assign_min); MLRS_KMEANS_ELKAN the bound-pruned one
 *   (elkan_init_bounds / elkan_assign_device / elkan_relax_bounds,
 *   prims/kmeans.rs:1523-1717), without the reference's n x k lower bounds:
 *   per row an upper bound on its centre distance, the sorted k x k half
 *   centre distances, and the fused search for the rows those cannot settle.
 *   Both return the same fit, bit for bit (labels, centres, inertia, n_iter),
 *   as the reference pins for its two arms; 'elkan' serves k <= 4096 with
 *   finite rows and runs Lloyd otherwise.
 * init_kind: 0 explicit centres (init, device, k x n_features; one run), 1
 *   k-means++, 2 random.  out_centers (k x n_features, device, F),
 *   out_labels (n, device), *out_inertia and *out_n_iter (host) of the
 *   winning restart.  Synchronous.
 * Errors: InvalidParam "k" (AlgoError::InvalidK text), "n_init", "max_iter",
 *   "tol", "algorithm"; ShapeMismatch "x", "init", "centers", "labels", and "labels"
 *   {n, k, empty clusters} when an empty cluster finds no donor row;
 *   Unsupported "init".
 */
#define MLRS_KMEANS_LLOYD 0
#define MLRS_KMEANS_ELKAN 1
int32_t mlrs_kmeans_fit_f32(const float *x, int64_t x_len, int64_t n, int64_t n_features, int64_t n_clusters,
                            int32_t init_kind, const float *init, int64_t init_len, uint64_t seed, int64_t n_init,
                            int64_t max_iter, double tol, int32_t algorithm, float *out_centers, int64_t centers_len,
                            uint32_t *out_labels, int64_t labels_len, double *out_inertia, int64_t *out_n_iter,
                            void *stream);
int32_t mlrs_kmeans_fit_f64(const double *x, int64_t x_len, int64_t n, int64_t n_features, int64_t n_clusters,
                            int32_t init_kind, const double *init, int64_t init_len, uint64_t seed, int64_t n_init,
                            int64_t max_iter, double tol, int32_t algorithm, double *out_centers,
                            int64_t centers_len,
                            uint32_t *out_labels, int64_t labels_len, double *out_inertia, int64_t *out_n_iter,
                            void *stream);

/*
 * Fit-time ownership copy: dst[0..len) = src[0..len) on `stream` (device
 * pointers, any alignment; 16-byte vectors when both are 16-byte aligned).
 * Replaces: device_copy (crates/mlrs-backend/src/prims/knn.rs:358-386) with
 *   its copy_elem / copy_elem_cpu_chunked kernels (crates/mlrs-kernels/src/
 *   elementwise.rs:71-125), which NearestNeighbors' Rust Fit::fit runs to own
 *   the training matrix.  The reference's u32 element ceiling (a CubeCL launch
 *   limit) does not apply.
 * Errors: ShapeMismatch "src" (len < 0), "dst" {len, 1, dst_len} when
 *   dst_len != len; NullPointer when len > 0 and a pointer is NULL.
 */
int32_t mlrs_device_copy_f32(const float *src, int64_t len, float *dst, int64_t dst_len, void *stream);
int32_t mlrs_device_copy_f64(const double *src, int64_t len, double *dst, int64_t dst_len, void *stream);

/*
 * Buffer counters of the current device: PoolStats (crates/mlrs-backend/src/
 * pool.rs:27-56) over the library's cached device buffers (the main and
 * auxiliary workspaces and the radius plan memory).  allocations: buffers
 * grown with hipMalloc; reuses: requests the held buffer already covered;
 * live_bytes: capacity currently held; peak_bytes: its high-water mark;
 * read_backs: device-to-host copies the library made (radius totals and
 * flags, the consumers' error checks, the k-means fit's per-iteration state)
 * -- the search, assignment, pairwise, norm and graph paths make none, so a
 * memory gate can assert read_backs does not move across them.
 * mlrs_pool_stats_reset zeroes allocations, reuses and read_backs and sets
 * peak_bytes to live_bytes.  The allocation-free entry point's static
 * scratch is not a cached buffer and is not counted.
 */
typedef struct mlrs_pool_stats {
    uint64_t allocations;
    uint64_t reuses;
    uint64_t peak_bytes;
    uint64_t live_bytes;
    uint64_t read_backs;
} mlrs_pool_stats;
int32_t mlrs_pool_stats_get(mlrs_pool_stats *out);
int32_t mlrs_pool_stats_reset(void);

/* Release the cached device workspace of the current device. */
int32_t mlrs_release_workspace(void);

/*
 * Measurement hook (no counterpart in the reference; for benchmarks).
 * While enabled, every call records a pair of HIP events on its own stream
 * around the launch of its dominant kernel (the Gram-MFMA kernel, the low-d
 * ALU kernel, or the generic path's distance tile; k-means fit also times
 * its centroid-sum pass).  mlrs_timing_read waits for the recorded events,
 * picks the name with the largest summed time, and returns that sum, the
 * number of launches timed under the name and the name; enabling again
 * clears the records.
 */
int32_t mlrs_timing_enable(int32_t on);
int32_t mlrs_timing_read(double *total_ms, int64_t *launches, char *kernel_name, int32_t name_len);

/*
 * Peak probe (no counterpart in the reference; the basis of the roofline
 * fractions the benchmark reports).  Runs register-only chains on every CU
 * with `waves_per_simd` waves on each SIMD (1..8) and returns the achieved
 * TFLOP/s (an FMA counts two flops) of the second of two launches, timed with
 * HIP events on `stream`:
 *   kind 0: v_fma_f32 (eight independent chains per lane, no packed math)
 *   kind 1: v_fma_f64 (likewise)
 *   kind 2: v_mfma_f32_32x32x2f32 (two independent accumulator chains)
 *   kind 3: v_mfma_f64_16x16x4f64 (four independent accumulator chains)
 * Synchronous.  Errors: Unsupported "kind" / "waves_per_simd".
 */
int32_t mlrs_probe_peak(int32_t kind, int32_t waves_per_simd, double *tflops, void *stream);

/*
 * Kernel-family override (no counterpart in the reference; for tests and
 * benchmarks).  Every family returns the same bits, so this only changes
 * speed: 0 = automatic choice (default); 1 = the fused Gram-MFMA kernels
 * wherever they serve the shape (d <= 256, k <= 128; the f32 knn_host
 * cosine arm only at d > 128; k-means: d <= 256);
 * 2 = the
 * low-d ALU kernel wherever it serves the shape (f32 and f64, Euclidean
 * and cosine, d <= 16, k <= 32); 3 = the generic exact-tile path.  A family that does not serve
 * a shape falls back to the automatic choice.  radius_neighbors: 1 = the
 * matrix-core screen wherever it serves (f32 Euclidean / cosine, d <= 128),
 * 3 = the host-scan kernel.  Process-wide.
 */
#define MLRS_PATH_AUTO 0
#define MLRS_PATH_FUSED 1
#define MLRS_PATH_LOWD 2
#define MLRS_PATH_GENERIC 3
int32_t mlrs_force_path(int32_t path);

#ifdef __cplusplus
}
#endif

#endif /* MLRS_HIP_KNN_H */
