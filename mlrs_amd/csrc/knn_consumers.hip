// kNN consumers on the device: the regressor's neighbour-target gathers and
// the classifier's vote, so a predict never leaves the GPU between the
// search and the prediction.
//
//  * knn_regress_mean_kernel    knn_regress_mean (crates/mlrs-kernels/src/
//    knn.rs:95-147): Neumaier-compensated sum of the k targets, / k.
//  * knn_regress_gather_kernel  knn_regress_gather (knn.rs:197-316): uniform
//    or 1/d weights (a row with a zero distance switches to the indicator
//    weighting), Neumaier sums of w*y and of w, multi-output.
//  * knn_classify_kernel        KNeighborsClassifier::predict_proba_host /
//    predict_labels_host (crates/mlrs-algos/src/neighbors/classifier.rs:
//    782-930), whose host f64 loop becomes one lane per query: f64 weights
//    and class sums in neighbour order, row normalisation, the cast to F,
//    argmax with the lowest class index on a tie.
// One lane per query row; every operation rounds on its own, in the
// reference's order, so the results are its bits.
//
// Index errors: the regressor kernels skip an index outside [0, n_train) and
// flag the row, the classifier records the first bad (neighbour slot) of the
// row; each kernel also keeps the lowest flagged row in one 64-bit word, which
// the host reads back to raise the reference's error for that row.
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

template <typename T>
__device__ __forceinline__ void neumaier(T& acc, T& comp, T term) {
    const T zero = T(0);
    const T sum = acc + term;
    T a_mag = acc;
    if (a_mag < zero) a_mag = zero - a_mag;
    T t_mag = term;
    if (t_mag < zero) t_mag = zero - t_mag;
    if (a_mag >= t_mag)
        comp = comp + ((acc - sum) + term);
    else
        comp = comp + ((term - sum) + acc);
    acc = sum;
}

template <typename T>
__global__ __launch_bounds__(256) void knn_regress_mean_kernel(const T* __restrict__ y, int64_t n_train,
                                                               const uint32_t* __restrict__ idx, int64_t nq,
                                                               int64_t k, T* __restrict__ out,
                                                               unsigned long long* first_bad) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= nq) return;
    T acc = T(0), comp = T(0);
    bool bad = false;
    for (int64_t j = 0; j < k; ++j) {
        const uint32_t t = idx[q * k + j];
        if ((int64_t)t < n_train)
            neumaier<T>(acc, comp, y[t]);
        else
            bad = true;
    }
    out[q] = (acc + comp) / (T)k;
    if (bad) atomicMin(first_bad, (unsigned long long)q);
}

template <typename T>
__global__ __launch_bounds__(256) void knn_regress_gather_kernel(const T* __restrict__ y, int64_t n_train,
                                                                 int64_t n_out, const uint32_t* __restrict__ idx,
                                                                 const T* __restrict__ dist, int64_t nq, int64_t k,
                                                                 int weighted, T* __restrict__ out,
                                                                 unsigned long long* first_bad) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= nq) return;
    const T zero = T(0), one = T(1);
    const int64_t base = q * k;
    T dmin = zero;
    if (weighted) {
        dmin = dist[base];
        for (int64_t z = 1; z < k; ++z)
            if (dist[base + z] < dmin) dmin = dist[base + z];
    }
    bool bad = false;
    for (int64_t o = 0; o < n_out; ++o) {
        T acc = zero, acc_c = zero, ws = zero, ws_c = zero;
        for (int64_t j = 0; j < k; ++j) {
            const uint32_t t = idx[base + j];
            if ((int64_t)t < n_train) {
                const T v = y[(int64_t)t * n_out + o];
                T w = one;
                if (weighted) {
                    const T d = dist[base + j];
                    if (dmin <= zero) {
                        w = zero;
                        if (d <= zero) w = one;
                    } else {
                        w = one / d;
                    }
                }
                const T term = w * v;
                neumaier<T>(acc, acc_c, term);
                neumaier<T>(ws, ws_c, w);
            } else {
                bad = true;
            }
        }
        out[q * n_out + o] = (acc + acc_c) / (ws + ws_c);
    }
    if (bad) atomicMin(first_bad, (unsigned long long)q);
}

// err[q] = {kind (1: neighbour index >= n_train, 2: class id out of range),
// the offending value, the neighbour slot}; acc is this query's row of the
// f64 class-sum scratch.
template <typename T>
__global__ __launch_bounds__(256) void knn_classify_kernel(const int32_t* __restrict__ y_class, int64_t n_train,
                                                           int64_t n_classes, const uint32_t* __restrict__ idx,
                                                           const T* __restrict__ dist, int64_t q0, int64_t nq,
                                                           int64_t k, int weighted, T* __restrict__ proba,
                                                           int32_t* __restrict__ labels, double* __restrict__ acc_all,
                                                           int64_t* __restrict__ err,
                                                           unsigned long long* first_bad) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // row within the chunk
    const int64_t q = q0 + r;
    if (q >= nq) return;
    double* acc = acc_all + r * n_classes;
    const int64_t base = q * k;
    bool coincident = false;
    if (weighted)
        for (int64_t j = 0; j < k; ++j)
            if ((double)dist[base + j] == 0.0) coincident = true;
    for (int64_t c = 0; c < n_classes; ++c) acc[c] = 0.0;
    for (int64_t j = 0; j < k; ++j) {
        const uint32_t t = idx[base + j];
        int kind = 0;
        int64_t val = 0;
        if ((int64_t)t >= n_train) {
            kind = 1;
            val = t;
        } else {
            const int32_t cls = y_class[t];
            if (cls < 0 || (int64_t)cls >= n_classes) {
                kind = 2;
                val = cls;
            } else {
                double w = 1.0;
                if (weighted) {
                    const double d = (double)dist[base + j];
                    w = !coincident ? 1.0 / d : (d == 0.0 ? 1.0 : 0.0);
                }
                acc[cls] += w;
            }
        }
        if (kind) {
            err[3 * q + 0] = kind;
            err[3 * q + 1] = val;
            err[3 * q + 2] = j;
            atomicMin(first_bad, (unsigned long long)q);
            return;
        }
    }
    double total = 0.0;
    for (int64_t c = 0; c < n_classes; ++c) total += acc[c];
    const double denom = (total == 0.0) ? 1.0 : total;
    int64_t best = 0;
    double best_v = 0.0;
    for (int64_t c = 0; c < n_classes; ++c) {
        const T p = (T)(acc[c] / denom);
        proba[q * n_classes + c] = p;
        const double v = (double)p;
        if (c == 0 || v > best_v) {
            best_v = v;
            best = c;
        }
    }
    labels[q] = (int32_t)best;
}

__global__ void fill_u64_max_kernel(unsigned long long* p) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *p = ~0ull;
}

}  // namespace

hipError_t launch_first_bad_reset(unsigned long long* first_bad, hipStream_t s) {
    hipLaunchKernelGGL(fill_u64_max_kernel, dim3(1), dim3(64), 0, s, first_bad);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_knn_regress(const T* y, int64_t n_train, int64_t n_out, const uint32_t* idx, const T* dist,
                              int64_t nq, int64_t k, int weighted, T* out, unsigned long long* first_bad,
                              hipStream_t s) {
    const dim3 grid((unsigned)((nq + 255) / 256));
    if (!weighted && n_out == 1)
        hipLaunchKernelGGL((knn_regress_mean_kernel<T>), grid, dim3(256), 0, s, y, n_train, idx, nq, k, out,
                           first_bad);
    else
        hipLaunchKernelGGL((knn_regress_gather_kernel<T>), grid, dim3(256), 0, s, y, n_train, n_out, idx, dist, nq,
                           k, weighted, out, first_bad);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_knn_classify(const int32_t* y_class, int64_t n_train, int64_t n_classes, const uint32_t* idx,
                               const T* dist, int64_t q0, int64_t rows, int64_t nq, int64_t k, int weighted,
                               T* proba, int32_t* labels, double* acc, int64_t* err, unsigned long long* first_bad,
                               hipStream_t s) {
    const dim3 grid((unsigned)((rows + 255) / 256));
    hipLaunchKernelGGL((knn_classify_kernel<T>), grid, dim3(256), 0, s, y_class, n_train, n_classes, idx, dist, q0,
                       q0 + rows < nq ? q0 + rows : nq, k, weighted, proba, labels, acc, err, first_bad);
    return hipGetLastError();
}

template hipError_t launch_knn_regress<float>(const float*, int64_t, int64_t, const uint32_t*, const float*, int64_t,
                                              int64_t, int, float*, unsigned long long*, hipStream_t);
template hipError_t launch_knn_regress<double>(const double*, int64_t, int64_t, const uint32_t*, const double*,
                                               int64_t, int64_t, int, double*, unsigned long long*, hipStream_t);
template hipError_t launch_knn_classify<float>(const int32_t*, int64_t, int64_t, const uint32_t*, const float*,
                                               int64_t, int64_t, int64_t, int64_t, int, float*, int32_t*, double*,
                                               int64_t*, unsigned long long*, hipStream_t);
template hipError_t launch_knn_classify<double>(const int32_t*, int64_t, int64_t, const uint32_t*, const double*,
                                                int64_t, int64_t, int64_t, int64_t, int, double*, int32_t*, double*,
                                                int64_t*, unsigned long long*, hipStream_t);

}  // namespace mlrs
