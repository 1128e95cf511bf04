// Peak probe behind mlrs_probe_peak: register-only chains that measure what
// the vector and matrix units deliver on this part with a given number of
// waves per SIMD (the basis of the benchmark's roofline fractions).  Each
// lane keeps several independent chains so that one wave's dependent
// latency does not set the rate; the results are summed into one store per
// lane so that nothing is dead code.
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef double f64x4 __attribute__((ext_vector_type(4)));

template <typename T>
__global__ __launch_bounds__(256) void probe_fma_kernel(T* __restrict__ out, int iters, T a, T b) {
    constexpr int C = 8;
    T v[C];
#pragma unroll
    for (int c = 0; c < C; ++c) v[c] = (T)(threadIdx.x + c);
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int u = 0; u < 16; ++u)
#pragma unroll
            for (int c = 0; c < C; ++c) {
                if constexpr (sizeof(T) == 4)
                    v[c] = __builtin_fmaf(v[c], a, b);
                else
                    v[c] = __builtin_fma(v[c], a, b);
            }
    }
    T acc = T(0);
#pragma unroll
    for (int c = 0; c < C; ++c) acc += v[c];
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

__global__ __launch_bounds__(256) void probe_mfma_f32_kernel(float* __restrict__ out, int iters, float a, float b) {
    f32x16 c0, c1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        c0[r] = 0.0f;
        c1[r] = 0.0f;
    }
    const float x = a + (float)threadIdx.x * 1e-7f, y = b;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(y, x, c1, 0, 0, 0);
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc += c0[r] + c1[r];
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

__global__ __launch_bounds__(256) void probe_mfma_f64_kernel(double* __restrict__ out, int iters, double a, double b) {
    f64x4 c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) c[j][r] = 0.0;
    const double x = a + (double)threadIdx.x * 1e-9, y = b;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_mfma_f64_16x16x4f64(x, y, c[j], 0, 0, 0);
    }
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc += c[j][r];
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

}  // namespace

// Flops one launch performs, for `blocks` workgroups of 256 threads.
double probe_flops(int kind, int64_t blocks, int iters) {
    const double lanes = (double)blocks * 256.0;
    const double waves = (double)blocks * 4.0;
    switch (kind) {
    case 0:
    case 1: return lanes * iters * 16.0 * 8.0 * 2.0;          // 8 chains x 16 FMAs per iteration
    case 2: return waves * iters * 32.0 * (32.0 * 32.0 * 2.0 * 2.0);  // 32 MFMAs of 32x32x2
    default: return waves * iters * 32.0 * (16.0 * 16.0 * 4.0 * 2.0);  // 32 MFMAs of 16x16x4
    }
}

hipError_t launch_probe(int kind, int64_t blocks, int iters, void* out, hipStream_t s) {
    const dim3 grid((unsigned)blocks), block(256);
    switch (kind) {
    case 0:
        hipLaunchKernelGGL((probe_fma_kernel<float>), grid, block, 0, s, static_cast<float*>(out), iters, 0.999999f,
                           1e-3f);
        break;
    case 1:
        hipLaunchKernelGGL((probe_fma_kernel<double>), grid, block, 0, s, static_cast<double*>(out), iters,
                           0.999999999, 1e-3);
        break;
    case 2:
        hipLaunchKernelGGL(probe_mfma_f32_kernel, grid, block, 0, s, static_cast<float*>(out), iters, 1e-3f, 1e-3f);
        break;
    default:
        hipLaunchKernelGGL(probe_mfma_f64_kernel, grid, block, 0, s, static_cast<double*>(out), iters, 1e-3, 1e-3);
        break;
    }
    return hipGetLastError();
}

}  // namespace mlrs
