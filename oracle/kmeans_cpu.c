/*
 * oracle/kmeans_cpu.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * Plain-C restatement of mlrs's KMeans fit as the cpu backend runs it, for
 * checking the HIP engine's device loop:
 *
 *   orc_kmeans_fit_*       KMeans::fit (crates/mlrs-algos/src/cluster/kmeans.rs:
 *                          1353-1580) with single_run (:929-1155): restarts,
 *                          init, the Lloyd loop, the final inertia.
 *   orc_feature_mean_var_* feature_mean_var (crates/mlrs-backend/src/prims/
 *                          kmeans.rs:1222-1307): mean over features of the
 *                          population variance, two blocked passes.
 *   orc_kmeans_init_*      init_centers (kmeans.rs:893-920): k-means++
 *                          (kmeanspp_sample, prims/kmeans.rs:381-491) or random
 *                          (random_sample, :1769-1786) row indices, SplitMix64
 *                          (prims/rng.rs:58-110) seeded per restart.
 *
 * Each piece keeps the reference's element type and order:
 *   - assignment: orc_kmeans_assign_* (ref_cpu.c, assign_min's arithmetic);
 *   - centroid sums: per row block (nb = clamp(ceil(n/256), 1, max(8M/(k*d), 64)),
 *     rpb = ceil(n/nb)) an F sum over the block's rows in order, then an F sum
 *     of the blocks in order (centroid_sumcount_blocked + centroid_reduce_
 *     partials, crates/mlrs-kernels/src/kmeans.rs:329-479), widened to f64;
 *   - empty clusters: relocate_empty_clusters (prims/kmeans.rs:1323-1410), the
 *     farthest rows by (distance desc, index asc) moved into them;
 *   - new centres: f64 sum * (1/count), shift = sum of squared f64 changes,
 *     centres handed to the assignment as F;
 *   - stop: the labels did not change (strict), else shift <= tol * mean_var;
 *   - inertia: per row F sum of (x - c)^2 (inertia_rows, kernels/kmeans.rs:123-
 *     145), F sums over blocks of ceil(n/clamp(ceil(n/256), 1, 256)) rows
 *     (block_sum_f, :523-545), widened and added in f64 (sum_device, prims/
 *     kmeans.rs:1137-1176);
 *   - restarts: a later run wins only with a strictly lower inertia and a
 *     partition that is not the same up to relabelling (is_same_clustering,
 *     cluster/kmeans.rs:827-838).
 *
 * Built into the same library as ref_cpu.c with -ffp-contract=off.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

int orc_kmeans_assign_f32(const float *x, int64_t n, const float *centers, int64_t kc, int64_t d,
                          uint32_t *labels, float *dist, int nthreads);
int orc_kmeans_assign_f64(const double *x, int64_t n, const double *centers, int64_t kc, int64_t d,
                          uint32_t *labels, double *dist, int nthreads);

/* ---- SplitMix64 (prims/rng.rs:58-110) ---- */
typedef struct {
    uint64_t state;
} km_rng;

static uint64_t km_next_u64(km_rng *r)
{
    r->state += 0x9E3779B97F4A7C15ull;
    uint64_t z = r->state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double km_next_f64(km_rng *r)
{
    return (double)(km_next_u64(r) >> 11) / 9007199254740992.0;
}

/* The raw stream, for pinning the generator against published values. */
void orc_splitmix64_stream(uint64_t seed, int64_t n, uint64_t *out)
{
    km_rng r = {seed};
    for (int64_t i = 0; i < n; i++)
        out[i] = km_next_u64(&r);
}

static uint64_t km_next_below(km_rng *r, uint64_t bound)
{
    if (bound <= 1)
        return 0;
    uint64_t zone = UINT64_MAX - (UINT64_MAX % bound);
    for (;;) {
        uint64_t v = km_next_u64(r);
        if (v < zone)
            return v % bound;
    }
}

/* ---- relocation ranking: (distance desc, index asc) ----
 * A total order for qsort: a NaN distance ranks above every number, NaNs and
 * equal values by index.  On numbers it is the reference's
 * (prims/kmeans.rs:1347-1359). */
static const double *km_rank_dist;
static int km_rank_cmp(const void *pa, const void *pb)
{
    int64_t a = *(const int64_t *)pa, b = *(const int64_t *)pb;
    double da = km_rank_dist[a], db = km_rank_dist[b];
    int na = da != da, nb = db != db;
    if (na != nb)
        return na ? -1 : 1;
    if (!na) {
        if (db < da)
            return -1;
        if (da < db)
            return 1;
    }
    return (a < b) ? -1 : (a > b);
}

static int km_same_clustering(const uint32_t *a, const uint32_t *b, int64_t n, int64_t k)
{
    int64_t *map = (int64_t *)malloc(sizeof(int64_t) * (size_t)k);
    for (int64_t c = 0; c < k; c++)
        map[c] = -1;
    int same = 1;
    for (int64_t i = 0; i < n && same; i++) {
        if (map[a[i]] < 0)
            map[a[i]] = b[i];
        else if (map[a[i]] != (int64_t)b[i])
            same = 0;
    }
    free(map);
    return same;
}

#define ORC_KMEANS(T, S)                                                                    \
double orc_feature_mean_var_##S(const T *x, int64_t n, int64_t d)                           \
{                                                                                           \
    int64_t cap = ((int64_t)4 << 20) / (d > 0 ? d : 1);                                     \
    if (cap < 64)                                                                           \
        cap = 64;                                                                           \
    int64_t nb = (n + 255) / 256;                                                           \
    if (nb < 1)                                                                             \
        nb = 1;                                                                             \
    if (nb > cap)                                                                           \
        nb = cap;                                                                           \
    int64_t rpb = (n + nb - 1) / nb;                                                        \
    nb = (n + rpb - 1) / rpb;                                                               \
    double inv_n = 1.0 / (double)n;                                                         \
    double *means = (double *)calloc((size_t)d, sizeof(double));                            \
    T *parts = (T *)malloc(sizeof(T) * (size_t)(nb * d));                                   \
    for (int64_t b = 0; b < nb; b++)                                                        \
        for (int64_t j = 0; j < d; j++) {                                                   \
            T acc = (T)0;                                                                   \
            int64_t end = (b + 1) * rpb < n ? (b + 1) * rpb : n;                            \
            for (int64_t i = b * rpb; i < end; i++)                                         \
                acc += x[i * d + j];                                                        \
            parts[b * d + j] = acc;                                                         \
        }                                                                                   \
    for (int64_t b = 0; b < nb; b++)                                                        \
        for (int64_t j = 0; j < d; j++)                                                     \
            means[j] += (double)parts[b * d + j];                                           \
    for (int64_t j = 0; j < d; j++)                                                         \
        means[j] *= inv_n;                                                                  \
    double var_sum = 0.0;                                                                   \
    for (int64_t b = 0; b < nb; b++)                                                        \
        for (int64_t j = 0; j < d; j++) {                                                   \
            T mj = (T)means[j];                                                             \
            T acc = (T)0;                                                                   \
            int64_t end = (b + 1) * rpb < n ? (b + 1) * rpb : n;                            \
            for (int64_t i = b * rpb; i < end; i++) {                                       \
                T diff = x[i * d + j] - mj;                                                 \
                acc += diff * diff;                                                         \
            }                                                                               \
            parts[b * d + j] = acc;                                                         \
        }                                                                                   \
    for (int64_t q = 0; q < nb * d; q++)                                                    \
        var_sum += (double)parts[q];                                                        \
    free(means);                                                                            \
    free(parts);                                                                            \
    return (var_sum * inv_n) / (double)d;                                                   \
}                                                                                           \
                                                                                            \
/* kind 1: k-means++ (kmeanspp_sample), kind 2: random (random_sample). */                  \
int orc_kmeans_init_##S(const T *x, int64_t n, int64_t d, int64_t k, int kind, uint64_t seed, \
                        int64_t *chosen)                                                    \
{                                                                                           \
    if (k < 1 || k > n)                                                                     \
        return -1;                                                                          \
    km_rng r = {seed};                                                                      \
    if (kind == 2) {                                                                        \
        int64_t *idx = (int64_t *)malloc(sizeof(int64_t) * (size_t)n);                      \
        for (int64_t i = 0; i < n; i++)                                                     \
            idx[i] = i;                                                                     \
        for (int64_t i = 0; i < k; i++) {                                                   \
            int64_t j = i + (int64_t)km_next_below(&r, (uint64_t)(n - i));                  \
            int64_t t = idx[i];                                                             \
            idx[i] = idx[j];                                                                \
            idx[j] = t;                                                                     \
        }                                                                                   \
        memcpy(chosen, idx, sizeof(int64_t) * (size_t)k);                                   \
        free(idx);                                                                          \
        return 0;                                                                           \
    }                                                                                       \
    char *is_chosen = (char *)calloc((size_t)n, 1);                                         \
    T *mind2 = (T *)malloc(sizeof(T) * (size_t)n);                                          \
    double *w = (double *)malloc(sizeof(double) * (size_t)n);                               \
    int64_t first = (int64_t)km_next_below(&r, (uint64_t)n);                                \
    chosen[0] = first;                                                                      \
    is_chosen[first] = 1;                                                                   \
    int64_t cur = first;                                                                    \
    int rc = 0;                                                                             \
    for (int64_t m = 0; m < k; m++) {                                                       \
        /* kmeanspp_mind2 (kernels/kmeans.rs:576-603) */                                    \
        for (int64_t i = 0; i < n; i++) {                                                   \
            T acc = (T)0;                                                                   \
            for (int64_t j = 0; j < d; j++) {                                               \
                T diff = x[i * d + j] - x[cur * d + j];                                     \
                acc += diff * diff;                                                         \
            }                                                                               \
            if (m == 0 || acc < mind2[i])                                                   \
                mind2[i] = acc;                                                             \
        }                                                                                   \
        if (m + 1 == k)                                                                     \
            break;                                                                          \
        double total = 0.0;                                                                 \
        for (int64_t i = 0; i < n; i++) {                                                   \
            w[i] = (double)mind2[i];                                                        \
            total += w[i];                                                                  \
        }                                                                                   \
        int64_t next = -1;                                                                  \
        if (total <= 0.0) {                                                                 \
            for (int64_t i = 0; i < n; i++)                                                 \
                if (!is_chosen[i]) {                                                        \
                    next = i;                                                               \
                    break;                                                                  \
                }                                                                           \
            if (next < 0) {                                                                 \
                rc = -1;                                                                    \
                break;                                                                      \
            }                                                                               \
        } else {                                                                            \
            double target = km_next_f64(&r) * total;                                        \
            double acc = 0.0;                                                               \
            int64_t pick = n - 1;                                                           \
            for (int64_t i = 0; i < n; i++) {                                               \
                acc += w[i];                                                                \
                if (acc >= target) {                                                        \
                    pick = i;                                                               \
                    break;                                                                  \
                }                                                                           \
            }                                                                               \
            if (w[pick] <= 0.0) {                                                           \
                for (int64_t i = n - 1; i >= 0; i--)                                        \
                    if (w[i] > 0.0) {                                                       \
                        pick = i;                                                           \
                        break;                                                              \
                    }                                                                       \
            }                                                                               \
            if (is_chosen[pick]) {                                                          \
                for (int64_t i = 0; i < n; i++)                                             \
                    if (!is_chosen[i]) {                                                    \
                        pick = i;                                                           \
                        break;                                                              \
                    }                                                                       \
            }                                                                               \
            next = pick;                                                                    \
        }                                                                                   \
        chosen[m + 1] = next;                                                               \
        is_chosen[next] = 1;                                                                \
        cur = next;                                                                         \
    }                                                                                       \
    free(is_chosen);                                                                        \
    free(mind2);                                                                            \
    free(w);                                                                                \
    return rc;                                                                              \
}                                                                                           \
                                                                                            \
/* One restart (single_run).  centers_f64 holds the starting centres (k*d) on              \
 * entry and the final f64 centres on exit. */                                              \
static int km_single_run_##S(const T *x, int64_t n, int64_t d, int64_t k, int64_t max_iter, \
                             double tol_scaled, double *centers_f64, uint32_t *labels,      \
                             double *inertia, int64_t *n_iter)                              \
{                                                                                           \
    const int64_t kd = k * d;                                                               \
    int64_t cap = ((int64_t)8 << 20) / (kd > 0 ? kd : 1);                                   \
    if (cap < 64)                                                                           \
        cap = 64;                                                                           \
    int64_t nb = (n + 255) / 256;                                                           \
    if (nb < 1)                                                                             \
        nb = 1;                                                                             \
    if (nb > cap)                                                                           \
        nb = cap;                                                                           \
    int64_t rpb = (n + nb - 1) / nb;                                                        \
    nb = (n + rpb - 1) / rpb;                                                               \
    T *cf = (T *)malloc(sizeof(T) * (size_t)kd);                                            \
    T *dist = (T *)malloc(sizeof(T) * (size_t)n);                                           \
    uint32_t *old = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)n);                       \
    T *psum = (T *)malloc(sizeof(T) * (size_t)kd);                                          \
    T *sums = (T *)malloc(sizeof(T) * (size_t)kd);                                          \
    double *sf = (double *)malloc(sizeof(double) * (size_t)kd);                             \
    double *nc = (double *)malloc(sizeof(double) * (size_t)kd);                             \
    int64_t *cnt = (int64_t *)malloc(sizeof(int64_t) * (size_t)k);                          \
    int64_t *order = (int64_t *)malloc(sizeof(int64_t) * (size_t)n);                       \
    char *moved = (char *)malloc((size_t)n);                                                \
    double *dd = (double *)malloc(sizeof(double) * (size_t)n);                              \
    int rc = 0;                                                                             \
    for (int64_t q = 0; q < kd; q++)                                                        \
        cf[q] = (T)centers_f64[q];                                                          \
    orc_kmeans_assign_##S(x, n, cf, k, d, labels, dist, 0);                                 \
    int64_t iters = 0;                                                                      \
    for (int64_t it = 0; it < max_iter; it++) {                                             \
        iters++;                                                                            \
        for (int64_t q = 0; q < kd; q++)                                                    \
            sums[q] = (T)0;                                                                 \
        for (int64_t c = 0; c < k; c++)                                                     \
            cnt[c] = 0;                                                                     \
        for (int64_t b = 0; b < nb; b++) {                                                  \
            int64_t end = (b + 1) * rpb < n ? (b + 1) * rpb : n;                            \
            for (int64_t q = 0; q < kd; q++)                                                \
                psum[q] = (T)0;                                                             \
            for (int64_t i = b * rpb; i < end; i++) {                                       \
                uint32_t c = labels[i];                                                     \
                cnt[c]++;                                                                   \
                for (int64_t j = 0; j < d; j++)                                             \
                    psum[c * d + j] += x[i * d + j];                                        \
            }                                                                               \
            for (int64_t q = 0; q < kd; q++)                                                \
                sums[q] += psum[q];                                                         \
        }                                                                                   \
        for (int64_t q = 0; q < kd; q++)                                                    \
            sf[q] = (double)sums[q];                                                        \
        int64_t n_empty = 0;                                                                \
        for (int64_t c = 0; c < k; c++)                                                     \
            n_empty += (cnt[c] == 0);                                                       \
        if (n_empty) {                                                                      \
            for (int64_t i = 0; i < n; i++) {                                               \
                order[i] = i;                                                               \
                moved[i] = 0;                                                               \
                dd[i] = (double)dist[i];                                                    \
            }                                                                               \
            km_rank_dist = dd;                                                              \
            qsort(order, (size_t)n, sizeof(int64_t), km_rank_cmp);                          \
            int64_t cursor = 0;                                                             \
            for (int64_t c = 0; c < k && rc == 0; c++) {                                    \
                if (cnt[c] != 0)                                                            \
                    continue;                                                               \
                int ok = 0;                                                                 \
                while (cursor < n) {                                                        \
                    int64_t i = order[cursor++];                                            \
                    if (moved[i])                                                           \
                        continue;                                                           \
                    uint32_t donor = labels[i];                                             \
                    if (cnt[donor] <= 1)                                                    \
                        continue;                                                           \
                    for (int64_t j = 0; j < d; j++) {                                       \
                        double xij = (double)x[i * d + j];                                  \
                        sf[c * d + j] += xij;                                               \
                        sf[donor * d + j] -= xij;                                           \
                    }                                                                       \
                    cnt[c]++;                                                               \
                    cnt[donor]--;                                                           \
                    moved[i] = 1;                                                           \
                    ok = 1;                                                                 \
                    break;                                                                  \
                }                                                                           \
                if (!ok)                                                                    \
                    rc = -2;                                                                \
            }                                                                               \
            if (rc)                                                                         \
                break;                                                                      \
        }                                                                                   \
        for (int64_t c = 0; c < k; c++) {                                                   \
            double inv = 1.0 / (double)cnt[c];                                              \
            for (int64_t j = 0; j < d; j++)                                                 \
                nc[c * d + j] = sf[c * d + j] * inv;                                        \
        }                                                                                   \
        double shift = 0.0;                                                                 \
        for (int64_t q = 0; q < kd; q++) {                                                  \
            double diff = nc[q] - centers_f64[q];                                           \
            shift += diff * diff;                                                           \
        }                                                                                   \
        memcpy(centers_f64, nc, sizeof(double) * (size_t)kd);                               \
        for (int64_t q = 0; q < kd; q++)                                                    \
            cf[q] = (T)nc[q];                                                               \
        memcpy(old, labels, sizeof(uint32_t) * (size_t)n);                                  \
        orc_kmeans_assign_##S(x, n, cf, k, d, labels, dist, 0);                             \
        int64_t changed = 0;                                                                \
        for (int64_t i = 0; i < n; i++)                                                     \
            changed += (labels[i] != old[i]);                                               \
        if (changed == 0)                                                                   \
            break;                                                                          \
        if (shift <= tol_scaled)                                                            \
            break;                                                                          \
    }                                                                                       \
    if (rc == 0) {                                                                          \
        /* inertia_rows + block_sum_f + f64 fold */                                         \
        int64_t ib = (n + 255) / 256;                                                       \
        if (ib < 1)                                                                         \
            ib = 1;                                                                         \
        if (ib > 256)                                                                       \
            ib = 256;                                                                       \
        int64_t irpb = (n + ib - 1) / ib;                                                   \
        ib = (n + irpb - 1) / irpb;                                                         \
        double tot = 0.0;                                                                   \
        for (int64_t b = 0; b < ib; b++) {                                                  \
            int64_t end = (b + 1) * irpb < n ? (b + 1) * irpb : n;                          \
            T acc = (T)0;                                                                   \
            for (int64_t i = b * irpb; i < end; i++) {                                      \
                T r = (T)0;                                                                 \
                for (int64_t j = 0; j < d; j++) {                                           \
                    T diff = x[i * d + j] - cf[(int64_t)labels[i] * d + j];                 \
                    r += diff * diff;                                                       \
                }                                                                           \
                acc += r;                                                                   \
            }                                                                               \
            tot += (double)acc;                                                             \
        }                                                                                   \
        *inertia = tot;                                                                     \
        *n_iter = iters;                                                                    \
    }                                                                                       \
    free(cf); free(dist); free(old); free(psum); free(sums); free(sf); free(nc);            \
    free(cnt); free(order); free(moved); free(dd);                                          \
    return rc;                                                                              \
}                                                                                           \
                                                                                            \
/* init_kind 0: init (k*d, F) given; 1 k-means++; 2 random.  Returns 0, -1 for a            \
 * bad k, -2 when an empty cluster finds no donor. */                                       \
int orc_kmeans_fit_##S(const T *x, int64_t n, int64_t d, int64_t k, int init_kind, const T *init, \
                       uint64_t seed, int64_t n_init, int64_t max_iter, double tol,         \
                       T *out_centers, uint32_t *out_labels, double *out_inertia,           \
                       int64_t *out_n_iter)                                                 \
{                                                                                           \
    if (k < 1 || k > n || d < 1)                                                            \
        return -1;                                                                          \
    const int64_t kd = k * d;                                                               \
    double tol_scaled = tol * orc_feature_mean_var_##S(x, n, d);                            \
    double *cen = (double *)malloc(sizeof(double) * (size_t)kd);                            \
    double *best_c = (double *)malloc(sizeof(double) * (size_t)kd);                         \
    uint32_t *lab = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)n);                       \
    int64_t *chosen = (int64_t *)malloc(sizeof(int64_t) * (size_t)k);                       \
    int have = 0, rc = 0;                                                                   \
    double best_inertia = 0.0;                                                              \
    int64_t best_iter = 0;                                                                  \
    for (int64_t restart = 0; restart < n_init && rc == 0; restart++) {                     \
        if (init_kind == 0) {                                                               \
            for (int64_t q = 0; q < kd; q++)                                                \
                cen[q] = (double)init[q];                                                   \
        } else {                                                                            \
            rc = orc_kmeans_init_##S(x, n, d, k, init_kind, seed + (uint64_t)restart, chosen); \
            if (rc)                                                                         \
                break;                                                                      \
            for (int64_t c = 0; c < k; c++)                                                 \
                for (int64_t j = 0; j < d; j++)                                             \
                    cen[c * d + j] = (double)x[chosen[c] * d + j];                          \
        }                                                                                   \
        double inertia;                                                                     \
        int64_t it;                                                                         \
        rc = km_single_run_##S(x, n, d, k, max_iter, tol_scaled, cen, lab, &inertia, &it);  \
        if (rc)                                                                             \
            break;                                                                          \
        if (!have || (inertia < best_inertia && !km_same_clustering(lab, out_labels, n, k))) { \
            have = 1;                                                                       \
            best_inertia = inertia;                                                         \
            best_iter = it;                                                                 \
            memcpy(best_c, cen, sizeof(double) * (size_t)kd);                               \
            memcpy(out_labels, lab, sizeof(uint32_t) * (size_t)n);                          \
        }                                                                                   \
    }                                                                                       \
    if (rc == 0) {                                                                          \
        for (int64_t q = 0; q < kd; q++)                                                    \
            out_centers[q] = (T)best_c[q];                                                  \
        *out_inertia = best_inertia;                                                        \
        *out_n_iter = best_iter;                                                            \
    }                                                                                       \
    free(cen); free(best_c); free(lab); free(chosen);                                       \
    return rc;                                                                              \
}

ORC_KMEANS(float, f32)
ORC_KMEANS(double, f64)
