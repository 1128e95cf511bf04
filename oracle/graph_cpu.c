/*
 * oracle/graph_cpu.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * Plain-C restatement of the X-vs-X neighbour scans the reference's cpu backend
 * runs for UMAP and HDBSCAN, for checking the HIP engine's device versions:
 *
 *   orc_knn_graph_f64     host_knn (crates/mlrs-algos/src/manifold/
 *                         umap_host_knn.rs:212-500): the directed k-nearest
 *                         graph of a row set against itself, all arithmetic in
 *                         f64; include_self = 0 skips the row's own index (the
 *                         KNearest `skip`, :125-198), include_self = 1 keeps it
 *                         (knn_graph's include_self, crates/mlrs-backend/src/
 *                         prims/knn_graph.rs:180-311).
 *   orc_core_distances_f64  HDBSCAN's core distances (crates/mlrs-algos/src/
 *                         cluster/hdbscan/host_core.rs:253-540): the
 *                         (k-1)-th smallest distance of each row to the whole
 *                         set, self included, k = clamp(min_samples, 1, n).
 *
 * Per pair the aggregate is the screened accumulators' (cluster/hdbscan/
 * distance.rs:39-117; the screen only skips pairs that cannot enter, so it is
 * left out): Euclidean and cosine s += diff*diff, Manhattan s += |diff|,
 * Chebyshev a running max that a NaN never replaces, Minkowski s +=
 * pow(|diff|, p) (always pow).  A pair whose aggregate is not finite is never
 * offered.  The kept value is the final distance: sqrt(s) (Euclidean), 0.5*s
 * over L2-normalised rows (cosine, l2_normalize_rows :504-515), s (Manhattan,
 * Chebyshev), pow(s, 1/p) (Minkowski); lists are ordered by (distance, index),
 * NaN never enters, and a row with fewer than k entries is padded with
 * (distance 0, index 0) in the graph and reads +inf as its core distance.
 *
 * Built into the same library as ref_cpu.c with -ffp-contract=off.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define G_EUCLIDEAN 0
#define G_COSINE 1
#define G_MANHATTAN 2
#define G_CHEBYSHEV 3
#define G_MINKOWSKI 4

static double g_aggregate(const double *a, const double *b, int64_t d, int metric, double p)
{
    double s = 0.0;
    for (int64_t c = 0; c < d; c++) {
        double diff = a[c] - b[c];
        if (metric == G_EUCLIDEAN || metric == G_COSINE) {
            s += diff * diff;
        } else if (metric == G_MANHATTAN) {
            s += fabs(diff);
        } else if (metric == G_CHEBYSHEV) {
            double v = fabs(diff);
            if (v > s)
                s = v;
        } else {
            s += pow(fabs(diff), p);
        }
    }
    return s;
}

static double g_final(double s, int metric, double p)
{
    if (metric == G_EUCLIDEAN)
        return sqrt(s);
    if (metric == G_COSINE)
        return 0.5 * s;
    if (metric == G_MINKOWSKI)
        return pow(s, 1.0 / p);
    return s;
}

/* KNearest::push (umap_host_knn.rs:170-197): ascending (distance, index). */
static void g_push(double *ld, uint32_t *li, int64_t *len, int64_t k, double v, uint32_t idx)
{
    if (isnan(v))
        return;
    int full = (*len == k);
    if (full && (v > ld[k - 1] || (v == ld[k - 1] && idx >= li[k - 1])))
        return;
    int64_t pos = *len;
    while (pos > 0) {
        if (ld[pos - 1] < v || (ld[pos - 1] == v && li[pos - 1] < idx))
            break;
        pos--;
    }
    int64_t last = full ? k - 1 : *len;
    for (int64_t m = last; m > pos; m--) {
        ld[m] = ld[m - 1];
        li[m] = li[m - 1];
    }
    ld[pos] = v;
    li[pos] = idx;
    if (!full)
        (*len)++;
}

static double *g_prepare(const double *x, int64_t n, int64_t d, int metric)
{
    if (metric != G_COSINE)
        return NULL;
    double *xn = (double *)malloc(sizeof(double) * (size_t)(n * d > 0 ? n * d : 1));
    for (int64_t i = 0; i < n; i++) {
        double ss = 0.0;
        for (int64_t c = 0; c < d; c++)
            ss = ss + x[i * d + c] * x[i * d + c];
        double norm = sqrt(ss);
        double inv = norm > 0.0 ? 1.0 / norm : 0.0;
        for (int64_t c = 0; c < d; c++)
            xn[i * d + c] = x[i * d + c] * inv;
    }
    return xn;
}

/* Returns 0, or -1 for k outside [1, n - 1] (include_self = 0) / [1, n]. */
int orc_knn_graph_f64(const double *x, int64_t n, int64_t d, int64_t k, int metric, double p,
                      int include_self, uint32_t *out_idx, double *out_dist)
{
    int64_t max_k = include_self ? n : n - 1;
    if (k < 1 || k > max_k || d < 1)
        return -1;
    double *xn = g_prepare(x, n, d, metric);
    const double *data = xn ? xn : x;
    #pragma omp parallel
    {
        double *ld = (double *)malloc(sizeof(double) * (size_t)k);
        uint32_t *li = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)k);
        #pragma omp for schedule(dynamic, 16)
        for (int64_t i = 0; i < n; i++) {
            int64_t len = 0;
            for (int64_t j = 0; j < n; j++) {
                if (!include_self && j == i)
                    continue;
                double a = g_aggregate(data + i * d, data + j * d, d, metric, p);
                if (isfinite(a))
                    g_push(ld, li, &len, k, g_final(a, metric, p), (uint32_t)j);
            }
            for (int64_t c = 0; c < k; c++) {
                out_dist[i * k + c] = c < len ? ld[c] : 0.0;
                out_idx[i * k + c] = c < len ? li[c] : 0u;
            }
        }
        free(ld);
        free(li);
    }
    free(xn);
    return 0;
}

/* Core distances, k = clamp(min_samples, 1, n) (hdbscan.rs:1512-1566);
 * cosine is not served (the reference takes it from a dense matrix). */
int orc_core_distances_f64(const double *x, int64_t n, int64_t d, int metric, double p, int64_t min_samples,
                           double *out)
{
    if (n < 1 || d < 1 || metric == G_COSINE)
        return -1;
    int64_t k = min_samples < 1 ? 1 : (min_samples > n ? n : min_samples);
    #pragma omp parallel
    {
        double *ld = (double *)malloc(sizeof(double) * (size_t)k);
        uint32_t *li = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)k);
        #pragma omp for schedule(dynamic, 16)
        for (int64_t i = 0; i < n; i++) {
            int64_t len = 0;
            for (int64_t j = 0; j < n; j++) {
                double a = g_aggregate(x + i * d, x + j * d, d, metric, p);
                if (isfinite(a))
                    g_push(ld, li, &len, k, g_final(a, metric, p), (uint32_t)j);
            }
            out[i] = len == k ? ld[k - 1] : INFINITY;
        }
        free(ld);
        free(li);
    }
    return 0;
}
