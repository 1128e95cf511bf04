// X-vs-X neighbour graphs: the directed k-nearest graph UMAP consumes and the
// HDBSCAN core distances, in the f64 arithmetic of the reference's host scans
// (crates/mlrs-algos/src/manifold/umap_host_knn.rs:212-515,
// crates/mlrs-algos/src/cluster/hdbscan/host_core.rs:253-540).  The search
// itself is the engine's f64 kNN (Gram-MFMA with exact rescoring, or exact
// tiles); these kernels prepare its operand and finish its lists:
//
//  * widen_kernel          the f32 rows as f64 (the reference widens x to its
//                          f64 host domain before the scan)
//  * normalize_rows_kernel cosine: x * (1/sqrt(sum x*x)), 0 for a zero row --
//                          l2_normalize_rows (umap_host_knn.rs:504-515) with the
//                          row norm from row_norms_kernel (ascending sum)
//  * graph_finish_kernel   drops each row's own index by identity (the last
//                          column when it is absent), halves the cosine value
//                          (0.5 * |x^ - y^|^2) and writes (0, 0) for a
//                          non-finite entry, which the host scan never offers
//  * core_column_kernel    column k-1 of the self-inclusive lists
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

__global__ __launch_bounds__(256) void widen_kernel(const float* __restrict__ x, int64_t n,
                                                    double* __restrict__ y) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) y[i] = (double)x[i];
}

__global__ __launch_bounds__(256) void normalize_rows_kernel(const double* __restrict__ x, int64_t n, int64_t d,
                                                             const double* __restrict__ inv,
                                                             double* __restrict__ y) {
    const int64_t total = n * d;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) y[i] = x[i] * inv[i / d];
}

__global__ __launch_bounds__(256) void graph_finish_kernel(const double* __restrict__ val,
                                                           const uint32_t* __restrict__ idx, int64_t n, int kk,
                                                           int k, int drop_self, int halve,
                                                           double* __restrict__ out_dist,
                                                           uint32_t* __restrict__ out_idx) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= n) return;
    const double* v = val + r * kk;
    const uint32_t* ix = idx + r * kk;
    int skip = kk;  // column left out
    if (drop_self) {
        skip = kk - 1;
        for (int c = 0; c < kk; ++c)
            if ((int64_t)ix[c] == r) {
                skip = c;
                break;
            }
    }
    int o = 0;
    for (int c = 0; c < kk && o < k; ++c) {
        if (c == skip) continue;
        double dv = v[c];
        uint32_t iv = ix[c];
        if (!__builtin_isfinite(dv)) {  // inf or NaN: never offered by the host scan
            dv = 0.0;
            iv = 0u;
        } else if (halve) {
            dv = 0.5 * dv;
        }
        out_dist[r * k + o] = dv;
        out_idx[r * k + o] = iv;
        ++o;
    }
}

__global__ __launch_bounds__(256) void core_column_kernel(const double* __restrict__ val, int64_t n, int k,
                                                          double* __restrict__ out) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r < n) out[r] = val[r * k + (k - 1)];
}

unsigned grid_for(int64_t n, int64_t cap) {
    int64_t b = (n + 255) / 256;
    if (b < 1) b = 1;
    if (b > cap) b = cap;
    return (unsigned)b;
}

}  // namespace

hipError_t launch_widen(const float* x, int64_t n, double* y, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(widen_kernel, dim3(grid_for(n, 16384)), dim3(256), 0, s, x, n, y);
    return hipGetLastError();
}

hipError_t launch_normalize_rows(const double* x, int64_t n, int64_t d, const double* inv, double* y,
                                 hipStream_t s) {
    if (n * d <= 0) return hipSuccess;
    hipLaunchKernelGGL(normalize_rows_kernel, dim3(grid_for(n * d, 16384)), dim3(256), 0, s, x, n, d, inv, y);
    return hipGetLastError();
}

hipError_t launch_graph_finish(const double* val, const uint32_t* idx, int64_t n, int kk, int k, int drop_self,
                               int halve, double* out_dist, uint32_t* out_idx, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(graph_finish_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, val, idx, n, kk, k,
                       drop_self, halve, out_dist, out_idx);
    return hipGetLastError();
}

hipError_t launch_core_column(const double* val, int64_t n, int k, double* out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(core_column_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, val, n, k, out);
    return hipGetLastError();
}

}  // namespace mlrs
