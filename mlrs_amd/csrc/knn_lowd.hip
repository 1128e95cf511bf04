// Low-dimension kNN on the vector ALUs (d <= 16), exact direct form.
//
// The MI355X counterpart of euclidean_topk_rows_cpu_direct
// (crates/mlrs-kernels/src/knn.rs:2968-3227): one lane owns one query row,
// keeps its sorted k-list in VGPRs and walks every index row of its strip,
// accumulating fma(x-y, x-y, acc) (or acc + d*d for the host arm) over
// ascending columns.  At d <= 16 a Gram tile would spend as many VALU cycles
// in its epilogue as the direct form spends on the whole pair, and the direct
// form is exact by construction (duplicates score exactly 0), so this path
// uses no MFMA.
//
// Index rows are staged through LDS (4-float padded rows); every lane of a
// wave reads the same row at the same time, so the reads are LDS broadcasts.
// Admission is insert_lane's rule (knn.rs:2655-2706): reject with one compare
// against the kept worst, else a shift-insertion by (value, index).
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

constexpr int kRt = 512;        // index rows per LDS tile
constexpr int kMaxD = 16;
constexpr int kMaxK = 32;

template <int D, int K, int ARM>
__global__ __launch_bounds__(256) void knn_lowd_kernel(LowdArgs32 a) {
    constexpr int DP = (D + 3) & ~3;  // padded row length in LDS
    __shared__ __attribute__((aligned(16))) float tile[kRt * DP];

    const int tid = threadIdx.x;
    const int64_t q = (int64_t)blockIdx.x * 256 + tid;
    const bool qvalid = q < a.nq;
    const int64_t t_begin = (int64_t)blockIdx.y * a.rows_per_strip;
    int64_t t_end = t_begin + a.rows_per_strip;
    if (t_end > a.nt) t_end = a.nt;
    const int k = a.k;
    const float inf = __builtin_huge_valf();

    float qv[D];
#pragma unroll
    for (int c = 0; c < D; ++c) qv[c] = qvalid ? a.q[q * D + c] : 0.0f;

    float lv[K];
    uint32_t li[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        lv[j] = inf;
        li[j] = kSentinelIdx;
    }
    // An inactive lane can never admit (prefill_lists' -inf bound, knn.rs:2875-2905).
    float worst = qvalid ? inf : -inf;
    uint32_t worst_i = kSentinelIdx;

    for (int64_t t0 = t_begin; t0 < t_end; t0 += kRt) {
        const int nrows = (int)((t_end - t0) < kRt ? (t_end - t0) : kRt);
        __syncthreads();
        for (int e = tid; e < kRt * DP; e += 256) {
            int r = e / DP, c = e % DP;
            tile[e] = (r < nrows && c < D) ? a.x[(t0 + r) * D + c] : 0.0f;
        }
        __syncthreads();
        for (int r = 0; r < nrows; ++r) {
            const float* yr = &tile[r * DP];
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < D; ++c) {
                float diff = qv[c] - yr[c];
                if (ARM == ARM_EUCLID_FMA)
                    acc = __builtin_fmaf(diff, diff, acc);
                else
                    acc = acc + diff * diff;
            }
            const uint32_t t = (uint32_t)(t0 + r);
            if (acc <= worst) {
                if (acc < worst || t < worst_i) {
                    float cav = acc;
                    uint32_t cai = t;
#pragma unroll
                    for (int j = 0; j < K; ++j) {
                        if (j < k) {
                            float jv = lv[j];
                            uint32_t ji = li[j];
                            if (cav < jv || (cav == jv && cai < ji)) {
                                lv[j] = cav;
                                li[j] = cai;
                                cav = jv;
                                cai = ji;
                            }
                        }
                    }
                    // the new worst kept pair is slot k-1
#pragma unroll
                    for (int j = 0; j < K; ++j)
                        if (j == k - 1) {
                            worst = lv[j];
                            worst_i = li[j];
                        }
                }
            }
        }
    }

    if (!qvalid) return;
#pragma unroll
    for (int j = 0; j < K; ++j) {
        if (j < k) {
            if (a.nstrips > 1) {
                int64_t o = ((int64_t)blockIdx.y * a.nq + q) * k + j;
                a.part_val[o] = lv[j];
                a.part_idx[o] = li[j];
            } else {
                int64_t o = q * k + j;
                a.out_val[o] = (a.mode == EMIT_SQRT) ? __builtin_sqrtf(lv[j]) : lv[j];
                a.out_idx[o] = (li[j] == kSentinelIdx) ? 0u : li[j];
            }
        }
    }
}

// Strip merge, one wave per query (lists are sorted; k <= 32 <= 64 lanes).
__global__ __launch_bounds__(256) void lowd_merge_kernel(LowdArgs32 a) {
    const int lane = threadIdx.x & 63;
    const int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (q >= a.nq) return;
    const int k = a.k;
    const float inf = __builtin_huge_valf();
    float lv = inf;
    uint32_t li = kSentinelIdx;
    if (lane < k) {
        lv = a.part_val[q * k + lane];
        li = a.part_idx[q * k + lane];
    }
    for (int s = 1; s < a.nstrips; ++s) {
        float v = inf;
        uint32_t ix = kSentinelIdx;
        if (lane < k) {
            int64_t o = ((int64_t)s * a.nq + q) * k + lane;
            v = a.part_val[o];
            ix = a.part_idx[o];
        }
        wave_merge64<float>(lv, li, v, ix, lane);
    }
    if (lane < k) {
        a.out_val[q * k + lane] = (a.mode == EMIT_SQRT) ? __builtin_sqrtf(lv) : lv;
        a.out_idx[q * k + lane] = (li == kSentinelIdx) ? 0u : li;
    }
}

template <int D, int K, int ARM>
hipError_t launch3(const LowdArgs32& a, hipStream_t s) {
    dim3 grid((unsigned)((a.nq + 255) / 256), (unsigned)a.nstrips);
    hipLaunchKernelGGL((knn_lowd_kernel<D, K, ARM>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int D, int ARM>
hipError_t launch_k(const LowdArgs32& a, hipStream_t s) {
    if (a.k <= 1) return launch3<D, 1, ARM>(a, s);
    if (a.k <= 4) return launch3<D, 4, ARM>(a, s);
    if (a.k <= 8) return launch3<D, 8, ARM>(a, s);
    if (a.k <= 16) return launch3<D, 16, ARM>(a, s);
    return launch3<D, 32, ARM>(a, s);
}

template <int ARM>
hipError_t launch_d(const LowdArgs32& a, hipStream_t s) {
    switch (a.d) {
    case 1: return launch_k<1, ARM>(a, s);
    case 2: return launch_k<2, ARM>(a, s);
    case 3: return launch_k<3, ARM>(a, s);
    case 4: return launch_k<4, ARM>(a, s);
    case 5: return launch_k<5, ARM>(a, s);
    case 6: return launch_k<6, ARM>(a, s);
    case 7: return launch_k<7, ARM>(a, s);
    case 8: return launch_k<8, ARM>(a, s);
    case 9: return launch_k<9, ARM>(a, s);
    case 10: return launch_k<10, ARM>(a, s);
    case 11: return launch_k<11, ARM>(a, s);
    case 12: return launch_k<12, ARM>(a, s);
    case 13: return launch_k<13, ARM>(a, s);
    case 14: return launch_k<14, ARM>(a, s);
    case 15: return launch_k<15, ARM>(a, s);
    case 16: return launch_k<16, ARM>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

int lowd_max_d() { return kMaxD; }
int lowd_max_k() { return kMaxK; }

hipError_t launch_lowd_f32(const LowdArgs32& a, int arm, hipStream_t s) {
    if (a.d < 1 || a.d > kMaxD || a.k < 1 || a.k > kMaxK) return hipErrorInvalidValue;
    hipError_t e;
    if (arm == ARM_EUCLID_FMA)
        e = launch_d<ARM_EUCLID_FMA>(a, s);
    else if (arm == ARM_EUCLID_MULADD)
        e = launch_d<ARM_EUCLID_MULADD>(a, s);
    else
        return hipErrorInvalidValue;
    if (e != hipSuccess || a.nstrips <= 1) return e;
    hipLaunchKernelGGL(lowd_merge_kernel, dim3((unsigned)((a.nq + 3) / 4)), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace mlrs
