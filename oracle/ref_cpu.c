/*
 * oracle/ref_cpu.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A plain-C restatement of the arithmetic and selection rules of mlrs's
 * cpu-backend brute-force kNN, k-means assignment and pairwise-distance paths.
 * It exists to check the HIP engine (tests/, __graft_entry__.smoke) and to be
 * timed as the CPU baseline (bench.py's cpu_baseline leg).  Nothing in the
 * product (mlrs_amd/) may link, load or call it.
 *
 * Build: oracle/build.py (gcc -O3 -march=native -ffp-contract=off -fopenmp).
 * -ffp-contract=off is load-bearing: every multiply and add below rounds
 * separately, and a fused multiply-add appears ONLY where the reference writes
 * one (`fma(...)`), exactly as in the Rust/CubeCL sources cited per function.
 *
 * Arm dispatch (which arithmetic serves which shape) follows
 * crates/mlrs-algos/src/neighbors/nearest.rs:891-953 (`metric_topk`) on the cpu
 * backend with Device::Auto:
 *   1. Euclidean, d <= 32 and k <= 16  -> euclidean_topk_rows_cpu_direct
 *      (crates/mlrs-backend/src/prims/knn.rs:400-412 cpu_rows_applicable,
 *       crates/mlrs-kernels/src/knn.rs:2968-3227): acc = fma(x-y, x-y, acc).
 *   2. else d <= 128 and k <= 128      -> *_topk_rows_cpu_metric
 *      (prims/knn.rs:703-720, kernels/knn.rs:3265-3375, 3646-3661):
 *      Euclidean fma(x-y, x-y, acc); cosine fma(x, y, dot) folded by
 *      cosine_fold with row_sumsq squared norms.
 *   3. else                             -> knn_host_topk
 *      (crates/mlrs-backend/src/prims/knn_host.rs:418-851): Euclidean
 *      acc + diff*diff; cosine acc + x*y with reciprocal norms.
 * Selection is THE admission rule of kernels/knn.rs:2655-2706 (`insert_lane`)
 * and knn_host.rs:777-810 (`insert`): (value, index) order, lowest index wins a
 * tie, NaN is never admitted, lists are prefilled with (+inf, UINT32_MAX) and
 * a surviving sentinel index is emitted as 0 (kernels/knn.rs:2931-2961).
 * Because that order is total on admitted pairs, the k kept pairs do not
 * depend on the order candidates are offered, so this file is free to walk
 * query blocks in parallel (the reference makes the same argument,
 * crates/mlrs-backend/tests/knn_test.rs:881-884).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_METRIC_EUCLIDEAN 0
#define ORC_METRIC_COSINE 1
#define ORC_METRIC_MANHATTAN 2
#define ORC_METRIC_CHEBYSHEV 3
#define ORC_METRIC_MINKOWSKI 4

/* The integer-exponent Minkowski path: p an integer in 3..=8 runs a multiply
 * chain instead of powf (minkowski_powi, crates/mlrs-backend/src/prims/
 * knn.rs:680-687 and knn_host.rs:358-365). */
static int minkowski_powi(double p)
{
    unsigned pi = (p >= 0.0 && p < 4294967296.0) ? (unsigned)p : 0u;
    return (p == (double)pi && pi >= 3 && pi <= 8) ? (int)pi : 0;
}

#define ORC_ARM_DIRECT 0
#define ORC_ARM_METRIC 1
#define ORC_ARM_HOST 2

#define ORC_QB 32

/* Which cpu arm the reference dispatch picks for this shape
 * (nearest.rs:910-947; caps CPU_MAX_COLS=32 / CPU_K_CAP=16 at
 * kernels/knn.rs:2206-2210, CPU_METRIC_MAX_COLS=128 / CPU_METRIC_K_CAP=128 at
 * kernels/knn.rs:3240-3257). */
int orc_knn_arm(int64_t d, int64_t k, int metric)
{
    if (metric == ORC_METRIC_EUCLIDEAN && d >= 1 && d <= 32 && k >= 1 && k <= 16)
        return ORC_ARM_DIRECT;
    if (d >= 1 && d <= 128 && k >= 1 && k <= 128)
        return ORC_ARM_METRIC;
    return ORC_ARM_HOST;
}

static void set_threads(int nthreads)
{
#ifdef _OPENMP
    if (nthreads > 0)
        omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
}

int orc_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/*
 * The template below is instantiated for float and double.  T is the element
 * type, S the symbol suffix, FMA/SQRT the matching libm routines.
 */
#define ORC_DEFINE(T, S, FMA, SQRT, POW, FABS)                                             \
                                                                                           \
/* row_sumsq / row_sqnorm: acc += v*v over ascending c (kernels/knn.rs:2130-2149,         \
 * kernels/kmeans.rs:610). */                                                              \
void orc_row_sqnorms_##S(const T *x, int64_t n, int64_t d, T *out)                         \
{                                                                                          \
    for (int64_t r = 0; r < n; r++) {                                                      \
        T acc = (T)0;                                                                      \
        const T *row = x + r * d;                                                          \
        for (int64_t c = 0; c < d; c++) {                                                  \
            T v = row[c];                                                                  \
            acc = acc + v * v;                                                             \
        }                                                                                  \
        out[r] = acc;                                                                      \
    }                                                                                      \
}                                                                                          \
                                                                                           \
/* row_inv_norm_host (knn_host.rs:382-397): 1/sqrt(sum v*v), 0 for a zero row. */          \
static void inv_norms_##S(const T *x, int64_t n, int64_t d, T *out)                        \
{                                                                                          \
    for (int64_t r = 0; r < n; r++) {                                                      \
        T acc = (T)0;                                                                      \
        const T *row = x + r * d;                                                          \
        for (int64_t c = 0; c < d; c++)                                                    \
            acc = acc + row[c] * row[c];                                                   \
        out[r] = (acc > (T)0) ? (T)1 / SQRT(acc) : (T)0;                                   \
    }                                                                                      \
}                                                                                          \
                                                                                           \
/* insert_lane / insert: fold (v, t) into a sorted k-list or reject it. */                 \
static inline void insert_##S(T *lval, uint32_t *lidx, int64_t k, T v, uint32_t t)         \
{                                                                                          \
    T w = lval[k - 1];                                                                     \
    if (!(v < w || (v == w && t < lidx[k - 1])))                                           \
        return;                                                                            \
    T cav = v;                                                                             \
    uint32_t cai = t;                                                                      \
    for (int64_t j = 0; j < k; j++) {                                                      \
        T jv = lval[j];                                                                    \
        uint32_t ji = lidx[j];                                                             \
        if (cav < jv || (cav == jv && cai < ji)) {                                         \
            lval[j] = cav;                                                                 \
            lidx[j] = cai;                                                                 \
            cav = jv;                                                                      \
            cai = ji;                                                                      \
        }                                                                                  \
    }                                                                                      \
}                                                                                          \
                                                                                           \
/* The lane loop: one training row y against the QB staged query lanes, in the             \
 * arm's arithmetic; acc[a] receives lane a's pre-boundary value.  Shared by the           \
 * k-nearest scan and the radius scan, as lane_distances is shared by knn_host             \
 * and radius_host (knn_host.rs:693-760, radius_host.rs:51-60).  ynt is the                \
 * training row's cosine norm operand. */                                                  \
static inline void lane_dist_##S(const T *xt, const T *y, int64_t d, int metric, int arm,  \
                                 const T *qn, T ynt, T pe, int pi, T *acc)                 \
{                                                                                          \
    for (int a = 0; a < ORC_QB; a++)                                                       \
        acc[a] = (T)0;                                                                     \
    if (metric == ORC_METRIC_EUCLIDEAN) {                                                  \
        if (arm == ORC_ARM_HOST) {                                                         \
            for (int64_t c = 0; c < d; c++) {                                              \
                T yc = y[c];                                                               \
                const T *xc = xt + c * ORC_QB;                                             \
                for (int a = 0; a < ORC_QB; a++) {                                         \
                    T diff = xc[a] - yc;                                                   \
                    acc[a] = acc[a] + diff * diff;                                         \
                }                                                                          \
            }                                                                              \
        } else {                                                                           \
            for (int64_t c = 0; c < d; c++) {                                              \
                T yc = y[c];                                                               \
                const T *xc = xt + c * ORC_QB;                                             \
                for (int a = 0; a < ORC_QB; a++) {                                         \
                    T diff = xc[a] - yc;                                                   \
                    acc[a] = FMA(diff, diff, acc[a]);                                      \
                }                                                                          \
            }                                                                              \
        }                                                                                  \
    } else if (metric == ORC_METRIC_MANHATTAN) {                                           \
        /* acc + |x - y| (knn.rs:3277-3286, knn_host.rs:715-718) */                        \
        for (int64_t c = 0; c < d; c++) {                                                  \
            T yc = y[c];                                                                   \
            const T *xc = xt + c * ORC_QB;                                                 \
            for (int a = 0; a < ORC_QB; a++)                                               \
                acc[a] = acc[a] + FABS(xc[a] - yc);                                        \
        }                                                                                  \
    } else if (metric == ORC_METRIC_CHEBYSHEV) {                                           \
        /* running max as a select: NaN never replaces (knn.rs:3288-3312) */               \
        for (int64_t c = 0; c < d; c++) {                                                  \
            T yc = y[c];                                                                   \
            const T *xc = xt + c * ORC_QB;                                                 \
            for (int a = 0; a < ORC_QB; a++) {                                             \
                T v = FABS(xc[a] - yc);                                                    \
                acc[a] = (v > acc[a]) ? v : acc[a];                                        \
            }                                                                              \
        }                                                                                  \
    } else if (metric == ORC_METRIC_MINKOWSKI) {                                           \
        /* acc + |x - y|^p: multiply chain for integer p in 3..8, else powf                \
         * (knn.rs:3314-3360, knn_host.rs:728-742) */                                      \
        for (int64_t c = 0; c < d; c++) {                                                  \
            T yc = y[c];                                                                   \
            const T *xc = xt + c * ORC_QB;                                                 \
            for (int a = 0; a < ORC_QB; a++) {                                             \
                T ad = FABS(xc[a] - yc);                                                   \
                T r;                                                                       \
                if (pi > 0) {                                                              \
                    r = ad;                                                                \
                    for (int i = 1; i < pi; i++)                                           \
                        r = r * ad;                                                        \
                } else {                                                                   \
                    r = POW(ad, pe);                                                       \
                }                                                                          \
                acc[a] = acc[a] + r;                                                       \
            }                                                                              \
        }                                                                                  \
    } else {                                                                               \
        if (arm == ORC_ARM_HOST) {                                                         \
            for (int64_t c = 0; c < d; c++) {                                              \
                T yc = y[c];                                                               \
                const T *xc = xt + c * ORC_QB;                                             \
                for (int a = 0; a < ORC_QB; a++)                                           \
                    acc[a] = acc[a] + xc[a] * yc;                                          \
            }                                                                              \
            T iy = ynt;                                                                    \
            for (int a = 0; a < ORC_QB; a++) {                                             \
                T dv = (T)1 - acc[a] * qn[a] * iy;                                         \
                dv = (dv < (T)0) ? (T)0 : dv;                                              \
                dv = (dv > (T)2) ? (T)2 : dv;                                              \
                acc[a] = dv;                                                               \
            }                                                                              \
        } else {                                                                           \
            for (int64_t c = 0; c < d; c++) {                                              \
                T yc = y[c];                                                               \
                const T *xc = xt + c * ORC_QB;                                             \
                for (int a = 0; a < ORC_QB; a++)                                           \
                    acc[a] = FMA(xc[a], yc, acc[a]);                                       \
            }                                                                              \
            for (int a = 0; a < ORC_QB; a++) {                                             \
                T denom = SQRT(qn[a] * ynt);                                               \
                T sim = (denom > (T)0) ? acc[a] / denom : (T)0;                            \
                T dv = (T)1 - sim;                                                         \
                dv = (dv < (T)0) ? (T)0 : dv;                                              \
                dv = (dv > (T)2) ? (T)2 : dv;                                              \
                acc[a] = dv;                                                               \
            }                                                                              \
        }                                                                                  \
    }                                                                                      \
}                                                                                          \
                                                                                           \
/* One 32-query block against every training row, under `arm`/`metric`.                 \
 * xt is the transposed tile xt[c*QB + a]; lanes >= active stage zeros and are            \
 * never emitted.  qn / yn are the cosine norm operands of the arm (squared              \
 * norms for the metric family, reciprocal norms for the host arm). */                     \
static void scan_block_##S(const T *xt, int64_t active, const T *xtrain, int64_t nt,       \
                           int64_t d, int64_t k, int metric, int arm, const T *qn,         \
                           const T *yn, T pe, int pi, T *lval, uint32_t *lidx)             \
{                                                                                          \
    T acc[ORC_QB];                                                                         \
    T worst[ORC_QB];                                                                       \
    for (int a = 0; a < ORC_QB; a++)                                                       \
        worst[a] = (a < active) ? (T)INFINITY : (T)-INFINITY;                              \
    for (int64_t t = 0; t < nt; t++) {                                                     \
        const T *y = xtrain + t * d;                                                       \
        lane_dist_##S(xt, y, d, metric, arm, qn, yn ? yn[t] : (T)0, pe, pi, acc);          \
        int hit = 0;                                                                       \
        for (int a = 0; a < ORC_QB; a++)                                                   \
            hit |= (acc[a] <= worst[a]);                                                   \
        if (hit) {                                                                         \
            for (int a = 0; a < active; a++) {                                             \
                insert_##S(lval + a * k, lidx + a * k, k, acc[a], (uint32_t)t);            \
                worst[a] = lval[a * k + k - 1];                                            \
            }                                                                              \
        }                                                                                  \
    }                                                                                      \
}                                                                                          \
                                                                                           \
/* Brute-force kNN under the reference's cpu dispatch.  Returns true distances            \
 * (sqrt applied to the k selected Euclidean values, prims/knn.rs:877-883 and            \
 * knn_host.rs:826-851), indices as uint32 with the sentinel clamped to 0.               \
 * Returns 0, or -1 for a k outside [1, nt]. */                                            \
int orc_knn_topk_##S(const T *xq, int64_t nq, const T *xtrain, int64_t nt, int64_t d,      \
                     int64_t k, int metric, double p, T *out_val, uint32_t *out_idx,       \
                     int nthreads)                                                         \
{                                                                                          \
    if (k < 1 || k > nt || nq < 0 || d < 1)                                                \
        return -1;                                                                         \
    const int pi = (metric == ORC_METRIC_MINKOWSKI) ? minkowski_powi(p) : 0;               \
    const T pe = (T)p;                                                                     \
    /* powf_elem's exponent: f64_to_host(1.0 / p) (prims/knn.rs:882-888) */                \
    const T inv_p = (T)(1.0 / p);                                                          \
    int arm = orc_knn_arm(d, k, metric);                                                   \
    T *qn = NULL, *yn = NULL;                                                              \
    if (metric == ORC_METRIC_COSINE) {                                                     \
        qn = (T *)malloc(sizeof(T) * (size_t)(nq > 0 ? nq : 1));                           \
        yn = (T *)malloc(sizeof(T) * (size_t)nt);                                          \
        if (arm == ORC_ARM_HOST) {                                                         \
            inv_norms_##S(xq, nq, d, qn);                                                  \
            inv_norms_##S(xtrain, nt, d, yn);                                              \
        } else {                                                                           \
            orc_row_sqnorms_##S(xq, nq, d, qn);                                            \
            orc_row_sqnorms_##S(xtrain, nt, d, yn);                                        \
        }                                                                                  \
    }                                                                                      \
    int64_t nblocks = (nq + ORC_QB - 1) / ORC_QB;                                          \
    set_threads(nthreads);                                                                 \
    _Pragma("omp parallel")                                                                \
    {                                                                                      \
        T *xt = (T *)malloc(sizeof(T) * (size_t)(d * ORC_QB));                             \
        T *lval = (T *)malloc(sizeof(T) * (size_t)(k * ORC_QB));                           \
        uint32_t *lidx = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(k * ORC_QB));      \
        T qblk[ORC_QB];                                                                    \
        _Pragma("omp for schedule(dynamic, 1)")                                            \
        for (int64_t b = 0; b < nblocks; b++) {                                            \
            int64_t q0 = b * ORC_QB;                                                       \
            int64_t active = nq - q0 < ORC_QB ? nq - q0 : ORC_QB;                          \
            for (int64_t c = 0; c < d; c++)                                                \
                for (int a = 0; a < ORC_QB; a++)                                           \
                    xt[c * ORC_QB + a] = (a < active) ? xq[(q0 + a) * d + c] : (T)0;       \
            for (int a = 0; a < ORC_QB; a++)                                               \
                qblk[a] = (qn && a < active) ? qn[q0 + a] : (T)0;                          \
            for (int64_t j = 0; j < k * ORC_QB; j++) {                                     \
                lval[j] = (T)INFINITY;                                                     \
                lidx[j] = UINT32_MAX;                                                      \
            }                                                                              \
            scan_block_##S(xt, active, xtrain, nt, d, k, metric, arm, qblk, yn, pe, pi,    \
                           lval, lidx);                                                    \
            for (int64_t a = 0; a < active; a++)                                           \
                for (int64_t j = 0; j < k; j++) {                                          \
                    T v = lval[a * k + j];                                                 \
                    uint32_t ix = lidx[a * k + j];                                         \
                    out_val[(q0 + a) * k + j] = (metric == ORC_METRIC_EUCLIDEAN) ? SQRT(v) \
                        : (metric == ORC_METRIC_MINKOWSKI) ? POW(v, inv_p) : v;            \
                    out_idx[(q0 + a) * k + j] = (ix == UINT32_MAX) ? 0u : ix;              \
                }                                                                          \
        }                                                                                  \
        free(xt);                                                                          \
        free(lval);                                                                        \
        free(lidx);                                                                        \
    }                                                                                      \
    free(qn);                                                                              \
    free(yn);                                                                              \
    return 0;                                                                              \
}                                                                                          \
                                                                                           \
/* radius_neighbors under the reference's default arm, the fused host scan                 \
 * (radius_host.rs:239-299 scan_typed, :302-420 scan, :488-528 threshold_block,            \
 * :531-569 emit / transform), over the same lane loop as the k-nearest host arm.          \
 * The threshold is formed in double -- radius*radius for Euclidean,                       \
 * pow(radius, p) for Minkowski, radius otherwise -- then rounded to T once;               \
 * a lane matches when its pre-boundary value is <= it (NaN never matches).                \
 * counts[q] receives each query row's match count.  When out_val is given the             \
 * matches are also written, row q's at offsets[q] on (the caller's exclusive              \
 * prefix sum of counts), in ascending training index, each value through the              \
 * boundary transform chosen by p_tr (2 Euclidean, p Minkowski, 1 otherwise):              \
 * identity for 1, SQRT for 2, else POW(v, (T)(1/p_tr)).  Indices are written              \
 * as int32, as the reference's `t as i32`.                                                \
 * Returns 0, or -1 for d < 1 or a radius that is not >= 0. */                             \
int orc_radius_scan_##S(const T *xq, int64_t nq, const T *xtrain, int64_t nt, int64_t d,   \
                        int metric, double p, double radius, uint32_t *counts,             \
                        const int64_t *offsets, T *out_val, int32_t *out_idx, int nthreads)\
{                                                                                          \
    if (d < 1 || nq < 0 || nt < 0 || !(radius >= 0.0))                                     \
        return -1;                                                                         \
    const int pi = (metric == ORC_METRIC_MINKOWSKI) ? minkowski_powi(p) : 0;               \
    const T pe = (T)p;                                                                     \
    const double thresh = (metric == ORC_METRIC_EUCLIDEAN) ? radius * radius               \
                        : (metric == ORC_METRIC_MINKOWSKI) ? pow(radius, p) : radius;      \
    const T th = (T)thresh;                                                                \
    const double p_tr = (metric == ORC_METRIC_EUCLIDEAN) ? 2.0                             \
                      : (metric == ORC_METRIC_MINKOWSKI) ? p : 1.0;                        \
    const T inv_p = (T)(1.0 / p_tr);                                                       \
    T *qn = NULL, *yn = NULL;                                                              \
    if (metric == ORC_METRIC_COSINE) {                                                     \
        qn = (T *)malloc(sizeof(T) * (size_t)(nq > 0 ? nq : 1));                           \
        yn = (T *)malloc(sizeof(T) * (size_t)(nt > 0 ? nt : 1));                           \
        inv_norms_##S(xq, nq, d, qn);                                                      \
        inv_norms_##S(xtrain, nt, d, yn);                                                  \
    }                                                                                      \
    int64_t nblocks = (nq + ORC_QB - 1) / ORC_QB;                                          \
    set_threads(nthreads);                                                                 \
    _Pragma("omp parallel")                                                                \
    {                                                                                      \
        T *xt = (T *)malloc(sizeof(T) * (size_t)(d * ORC_QB));                             \
        T acc[ORC_QB];                                                                     \
        T qblk[ORC_QB];                                                                    \
        int64_t cnt[ORC_QB];                                                               \
        _Pragma("omp for schedule(dynamic, 1)")                                            \
        for (int64_t b = 0; b < nblocks; b++) {                                            \
            int64_t q0 = b * ORC_QB;                                                       \
            int64_t active = nq - q0 < ORC_QB ? nq - q0 : ORC_QB;                          \
            for (int64_t c = 0; c < d; c++)                                                \
                for (int a = 0; a < ORC_QB; a++)                                           \
                    xt[c * ORC_QB + a] = (a < active) ? xq[(q0 + a) * d + c] : (T)0;       \
            for (int a = 0; a < ORC_QB; a++) {                                             \
                qblk[a] = (qn && a < active) ? qn[q0 + a] : (T)0;                          \
                cnt[a] = 0;                                                                \
            }                                                                              \
            for (int64_t t = 0; t < nt; t++) {                                             \
                lane_dist_##S(xt, xtrain + t * d, d, metric, ORC_ARM_HOST, qblk,           \
                              yn ? yn[t] : (T)0, pe, pi, acc);                             \
                for (int64_t a = 0; a < active; a++) {                                     \
                    if (!(acc[a] <= th))                                                   \
                        continue;                                                          \
                    if (out_val) {                                                         \
                        T v = acc[a];                                                      \
                        v = (p_tr == 1.0) ? v : (p_tr == 2.0) ? SQRT(v) : POW(v, inv_p);   \
                        int64_t at = offsets[q0 + a] + cnt[a];                             \
                        out_val[at] = v;                                                   \
                        out_idx[at] = (int32_t)(uint32_t)t;                                \
                    }                                                                      \
                    cnt[a]++;                                                              \
                }                                                                          \
            }                                                                              \
            for (int64_t a = 0; a < active; a++)                                           \
                counts[q0 + a] = (uint32_t)cnt[a];                                         \
        }                                                                                  \
        free(xt);                                                                          \
    }                                                                                      \
    free(qn);                                                                              \
    free(yn);                                                                              \
    return 0;                                                                              \
}                                                                                          \
                                                                                           \
/* k-means assignment (prims/kmeans.rs:635-750): dist_direct_2d_c4                        \
 * (kernels/kmeans.rs:206-274, a += d*d) then argmin_dist_rows (:284-310): best           \
 * seeded from centre 0, strict `<` afterwards. Writes squared distances. */               \
int orc_kmeans_assign_##S(const T *x, int64_t n, const T *centers, int64_t kc, int64_t d,  \
                          uint32_t *labels, T *dist, int nthreads)                         \
{                                                                                          \
    if (kc < 1 || kc > n || d < 1)                                                         \
        return -1;                                                                         \
    set_threads(nthreads);                                                                 \
    _Pragma("omp parallel for schedule(static)")                                           \
    for (int64_t i = 0; i < n; i++) {                                                      \
        const T *xr = x + i * d;                                                           \
        T best = (T)0;                                                                     \
        uint32_t best_c = 0;                                                               \
        for (int64_t c = 0; c < kc; c++) {                                                 \
            const T *cr = centers + c * d;                                                 \
            T acc = (T)0;                                                                  \
            for (int64_t j = 0; j < d; j++) {                                              \
                T diff = xr[j] - cr[j];                                                    \
                acc = acc + diff * diff;                                                   \
            }                                                                              \
            if (c == 0) {                                                                  \
                best = acc;                                                                \
            } else if (acc < best) {                                                       \
                best = acc;                                                                \
                best_c = (uint32_t)c;                                                      \
            }                                                                              \
        }                                                                                  \
        labels[i] = best_c;                                                                \
        dist[i] = best;                                                                    \
    }                                                                                      \
    return 0;                                                                              \
}                                                                                          \
                                                                                           \
/* Pairwise distance matrix.  Euclidean = distance_direct / euclidean_sq_dist             \
 * (prims/distance.rs:428-551, kernels/distance.rs:411-440: acc += diff*diff),            \
 * optional boundary sqrt (sqrt_elem, kernels/elementwise.rs:131-136).                    \
 * Cosine = metric_distance / cosine_dist (kernels/distance.rs:257-310):                  \
 * dot += x*y, denom = sqrt(xn*yn) over row_sumsq norms, sim = dot/denom when             \
 * denom > 0 else 0, then the [0, 2] clamp. */                                             \
int orc_pairwise_##S(const T *x, int64_t nx, const T *y, int64_t ny, int64_t d,            \
                     int metric, int do_sqrt, double p, T *out, int nthreads)              \
{                                                                                          \
    if (d < 1)                                                                             \
        return -1;                                                                         \
    T *xn = NULL, *yn = NULL;                                                              \
    if (metric == ORC_METRIC_COSINE) {                                                     \
        xn = (T *)malloc(sizeof(T) * (size_t)(nx > 0 ? nx : 1));                           \
        yn = (T *)malloc(sizeof(T) * (size_t)(ny > 0 ? ny : 1));                           \
        orc_row_sqnorms_##S(x, nx, d, xn);                                                 \
        orc_row_sqnorms_##S(y, ny, d, yn);                                                 \
    }                                                                                      \
    set_threads(nthreads);                                                                 \
    _Pragma("omp parallel for schedule(static)")                                           \
    for (int64_t i = 0; i < nx; i++) {                                                     \
        const T *xr = x + i * d;                                                           \
        for (int64_t j = 0; j < ny; j++) {                                                 \
            const T *yr = y + j * d;                                                       \
            T acc = (T)0;                                                                  \
            if (metric == ORC_METRIC_MANHATTAN || metric == ORC_METRIC_CHEBYSHEV ||        \
                metric == ORC_METRIC_MINKOWSKI) {                                          \
                /* manhattan_dist / chebyshev_dist / minkowski_dist                        \
                 * (crates/mlrs-kernels/src/distance.rs:67-227): the Minkowski            \
                 * pairwise form always uses powf, with the root 1/p formed in F */        \
                const T pe = (T)p;                                                         \
                for (int64_t c = 0; c < d; c++) {                                          \
                    T diff = FABS(xr[c] - yr[c]);                                          \
                    if (metric == ORC_METRIC_MANHATTAN)                                    \
                        acc = acc + diff;                                                  \
                    else if (metric == ORC_METRIC_CHEBYSHEV)                               \
                        acc = (diff > acc) ? diff : acc;                                   \
                    else                                                                   \
                        acc = acc + POW(diff, pe);                                         \
                }                                                                          \
                if (metric == ORC_METRIC_MINKOWSKI)                                        \
                    acc = POW(acc, (T)1 / pe);                                             \
                out[i * ny + j] = acc;                                                     \
            } else if (metric == ORC_METRIC_EUCLIDEAN) {                                   \
                for (int64_t c = 0; c < d; c++) {                                          \
                    T diff = xr[c] - yr[c];                                                \
                    acc = acc + diff * diff;                                               \
                }                                                                          \
                out[i * ny + j] = do_sqrt ? SQRT(acc) : acc;                               \
            } else {                                                                       \
                for (int64_t c = 0; c < d; c++)                                            \
                    acc = acc + xr[c] * yr[c];                                             \
                T denom = SQRT(xn[i] * yn[j]);                                             \
                T sim = (T)0;                                                              \
                if (denom > (T)0)                                                          \
                    sim = acc / denom;                                                     \
                T dv = (T)1 - sim;                                                         \
                if (dv < (T)0)                                                             \
                    dv = (T)0;                                                             \
                if (dv > (T)2)                                                             \
                    dv = (T)2;                                                             \
                out[i * ny + j] = dv;                                                      \
            }                                                                              \
        }                                                                                  \
    }                                                                                      \
    free(xn);                                                                              \
    free(yn);                                                                              \
    return 0;                                                                              \
}

ORC_DEFINE(float, f32, fmaf, sqrtf, powf, fabsf)
ORC_DEFINE(double, f64, fma, sqrt, pow, fabs)
