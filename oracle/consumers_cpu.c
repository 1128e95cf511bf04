/*
 * oracle/consumers_cpu.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * Plain-C restatement of the kNN consumers that turn a neighbour set into a
 * prediction, for checking the HIP engine's device versions:
 *
 *   orc_knn_regress_mean_*   knn_regress_mean (crates/mlrs-kernels/src/knn.rs:
 *                            95-147): Neumaier-compensated sum of the k
 *                            neighbour targets divided by k, in F arithmetic.
 *   orc_knn_regress_gather_* knn_regress_gather (knn.rs:197-316): uniform or
 *                            1/d weights with the coincident-row indicator rule,
 *                            Neumaier sums of w*y and of w, multi-output.
 *   orc_knn_classify_*       KNeighborsClassifier::predict_proba_host /
 *                            predict_labels_host (crates/mlrs-algos/src/
 *                            neighbors/classifier.rs:782-930): f64 weights and
 *                            class sums, row normalisation, argmax with the
 *                            lowest class index on a tie.
 *
 * Index errors follow the reference: the regressor kernels skip an index
 * outside [0, n_train) and flag the row (oob[q] = 1, the host then raises);
 * the classifier stops at the first bad (query, neighbour) in row-major order
 * and reports it through err[0..3] = {kind (1 train index, 2 class id), value,
 * query row, neighbour slot}.
 *
 * Built into the same library as ref_cpu.c with -ffp-contract=off: every
 * operation rounds on its own, in the order written.
 */
#include <stdint.h>
#include <string.h>

#define ORC_CONSUMERS(T, S)                                                               \
/* one Neumaier step: fold `term` into (acc, comp) -- knn.rs:115-131 */                   \
static inline void neumaier_##S(T *acc, T *comp, T term)                                  \
{                                                                                         \
    const T zero = (T)0;                                                                  \
    T sum = *acc + term;                                                                  \
    T a_mag = *acc;                                                                       \
    if (a_mag < zero)                                                                     \
        a_mag = zero - a_mag;                                                             \
    T t_mag = term;                                                                       \
    if (t_mag < zero)                                                                     \
        t_mag = zero - t_mag;                                                             \
    if (a_mag >= t_mag)                                                                   \
        *comp = *comp + ((*acc - sum) + term);                                            \
    else                                                                                  \
        *comp = *comp + ((term - sum) + *acc);                                            \
    *acc = sum;                                                                           \
}                                                                                         \
                                                                                          \
void orc_knn_regress_mean_##S(const T *y, int64_t n_train, const uint32_t *idx, int64_t nq, \
                              int64_t k, T *out, uint32_t *oob)                           \
{                                                                                         \
    for (int64_t q = 0; q < nq; q++) {                                                    \
        T acc = (T)0, comp = (T)0;                                                        \
        uint32_t bad = 0;                                                                 \
        for (int64_t j = 0; j < k; j++) {                                                 \
            uint32_t t = idx[q * k + j];                                                  \
            if ((int64_t)t < n_train)                                                     \
                neumaier_##S(&acc, &comp, y[t]);                                          \
            else                                                                          \
                bad = 1;                                                                  \
        }                                                                                 \
        out[q] = (acc + comp) / (T)k;                                                     \
        oob[q] = bad;                                                                     \
    }                                                                                     \
}                                                                                         \
                                                                                          \
void orc_knn_regress_gather_##S(const T *y, int64_t n_train, int64_t n_out,               \
                                const uint32_t *idx, const T *dist, int64_t nq, int64_t k, \
                                int weighted, T *out, uint32_t *oob)                      \
{                                                                                         \
    const T zero = (T)0, one = (T)1;                                                      \
    for (int64_t q = 0; q < nq; q++) {                                                    \
        const int64_t base = q * k;                                                       \
        T dmin = dist ? dist[base] : zero;                                                \
        for (int64_t z = 1; dist && z < k; z++)                                           \
            if (dist[base + z] < dmin)                                                    \
                dmin = dist[base + z];                                                    \
        uint32_t bad = 0;                                                                 \
        for (int64_t o = 0; o < n_out; o++) {                                             \
            T acc = zero, acc_c = zero, ws = zero, ws_c = zero;                           \
            for (int64_t j = 0; j < k; j++) {                                             \
                uint32_t t = idx[base + j];                                               \
                if ((int64_t)t < n_train) {                                               \
                    T v = y[(int64_t)t * n_out + o];                                      \
                    T w = one;                                                            \
                    if (weighted) {                                                       \
                        T d = dist[base + j];                                             \
                        if (dmin <= zero) {                                               \
                            w = zero;                                                     \
                            if (d <= zero)                                                \
                                w = one;                                                  \
                        } else {                                                          \
                            w = one / d;                                                  \
                        }                                                                 \
                    }                                                                     \
                    T term = w * v;                                                       \
                    neumaier_##S(&acc, &acc_c, term);                                     \
                    neumaier_##S(&ws, &ws_c, w);                                          \
                } else {                                                                  \
                    bad = 1;                                                              \
                }                                                                         \
            }                                                                             \
            out[q * n_out + o] = (acc + acc_c) / (ws + ws_c);                             \
        }                                                                                 \
        oob[q] = bad;                                                                     \
    }                                                                                     \
}                                                                                         \
                                                                                          \
int orc_knn_classify_##S(const int32_t *y_class, int64_t n_train, int64_t n_classes,      \
                         const uint32_t *idx, const T *dist, int64_t nq, int64_t k,       \
                         int weighted, T *proba, int32_t *labels, double *acc,            \
                         double *w, int64_t *err)                                         \
{                                                                                         \
    for (int64_t q = 0; q < nq; q++) {                                                    \
        if (!weighted) {                                                                  \
            for (int64_t j = 0; j < k; j++)                                               \
                w[j] = 1.0;                                                               \
        } else {                                                                          \
            int coincident = 0;                                                           \
            for (int64_t j = 0; j < k; j++)                                               \
                if ((double)dist[q * k + j] == 0.0)                                       \
                    coincident = 1;                                                       \
            for (int64_t j = 0; j < k; j++) {                                             \
                double d = (double)dist[q * k + j];                                       \
                w[j] = !coincident ? 1.0 / d : (d == 0.0 ? 1.0 : 0.0);                    \
            }                                                                             \
        }                                                                                 \
        for (int64_t c = 0; c < n_classes; c++)                                           \
            acc[c] = 0.0;                                                                 \
        for (int64_t j = 0; j < k; j++) {                                                 \
            uint32_t t = idx[q * k + j];                                                  \
            if ((int64_t)t >= n_train) {                                                  \
                err[0] = 1; err[1] = t; err[2] = q; err[3] = j;                           \
                return -1;                                                                \
            }                                                                             \
            int32_t cls = y_class[t];                                                     \
            if (cls < 0 || (int64_t)cls >= n_classes) {                                   \
                err[0] = 2; err[1] = cls; err[2] = q; err[3] = j;                         \
                return -1;                                                                \
            }                                                                             \
            acc[cls] += w[j];                                                             \
        }                                                                                 \
        double total = 0.0;                                                               \
        for (int64_t c = 0; c < n_classes; c++)                                           \
            total += acc[c];                                                              \
        double denom = (total == 0.0) ? 1.0 : total;                                      \
        for (int64_t c = 0; c < n_classes; c++)                                           \
            proba[q * n_classes + c] = (T)(acc[c] / denom);                               \
        int64_t best = 0;                                                                 \
        double best_v = (double)proba[q * n_classes];                                     \
        for (int64_t c = 1; c < n_classes; c++) {                                         \
            double v = (double)proba[q * n_classes + c];                                  \
            if (v > best_v) {                                                             \
                best_v = v;                                                               \
                best = c;                                                                 \
            }                                                                             \
        }                                                                                 \
        labels[q] = (int32_t)best;                                                        \
    }                                                                                     \
    return 0;                                                                             \
}

ORC_CONSUMERS(float, f32)
ORC_CONSUMERS(double, f64)
