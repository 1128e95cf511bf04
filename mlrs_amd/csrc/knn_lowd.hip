// Low-dimension kNN on the vector ALUs (d <= 16), no MFMA.
//
// The MI355X counterpart of euclidean_topk_rows_cpu_direct
// (crates/mlrs-kernels/src/knn.rs:2968-3227).  Each lane owns QL query rows
// (QL = 2 for k <= 16, 1 above), keeps their sorted k-lists in
// VGPRs and walks every index row of its strip.  Per (query, row) pair the
// screen costs d FMAs: the expansion ||x||^2 - 2 x.q accumulated from the
// row's precomputed squared norm, against the threshold derived from the
// query's exact k-th value (the same rigorous rounding bound as the Gram
// kernels).  A pair that passes is evaluated exactly, right there, in the
// reference arm's order -- fma(q-x, q-x, acc) (or acc + d*d for the host
// arm) over ascending columns, from the query in registers and the row in
// LDS -- and offered to the list with insert_lane's rule (knn.rs:2655-2706):
// (value, index) order, NaN never admitted.  The exact direct form is what
// the list holds, so results are the reference's bit for bit.
//
// Index rows are staged through LDS with their norm appended ((d+1) floats
// padded to a multiple of 4); every lane of a wave reads the same row at the
// same time, so the reads are LDS broadcasts.
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

constexpr int kMaxD = 16;
constexpr int kMaxK = 32;

template <int D, int K, int QL, int ARM>
__global__ __launch_bounds__(256) void knn_lowd_kernel(LowdArgs32 a) {
    constexpr int DPN = (D + 1 + 3) & ~3;  // row + norm, padded to float4
#ifndef MLRS_LOWD_RU4
#define MLRS_LOWD_RU4 8
#endif
    constexpr int RU = DPN <= 4 ? MLRS_LOWD_RU4 : (DPN <= 8 ? 4 : 2);  // rows per screening step
    constexpr int RT = 64 * RU;            // index rows per LDS tile: 64 steps
    __shared__ __attribute__((aligned(16))) float tile[RT * DPN];

    const int tid = threadIdx.x;
    const int64_t qbase = (int64_t)blockIdx.x * (256 * QL) + tid;
    const int64_t t_begin = (int64_t)blockIdx.y * a.rows_per_strip;
    int64_t t_end = t_begin + a.rows_per_strip;
    if (t_end > a.nt) t_end = a.nt;
    const int k = a.k;
    const float inf = __builtin_huge_valf();
    const float* __restrict__ X = a.x;
    const float* __restrict__ XSQ = a.xsq;

    float qv[QL][D];    // the queries
    float qm2[QL][D];   // -2 * the queries (exact scaling) for the screen
    float qsq[QL], eps[QL], thr[QL], worst[QL];
    uint32_t worst_i[QL];
    float lv[QL][K];
    uint32_t li[QL][K];
    const double xmax = (double)a.stats->xsq_max;
#pragma unroll
    for (int i = 0; i < QL; ++i) {
        const int64_t q = qbase + 256 * i;
        const bool ok = q < a.nq;
#pragma unroll
        for (int c = 0; c < D; ++c) {
            qv[i][c] = ok ? a.q[q * D + c] : 0.0f;
            qm2[i][c] = -2.0f * qv[i][c];
        }
        qsq[i] = ok ? a.qsq[q] : 0.0f;
        eps[i] = (float)(a.eps_rel * ((double)qsq[i] + xmax) + a.eps_abs);
        // An inactive lane can never admit (prefill_lists' -inf bound, knn.rs:2875-2905).
        worst[i] = ok ? inf : -inf;
        thr[i] = ok ? inf : -inf;
        worst_i[i] = kSentinelIdx;
        // A later strip starts from the k-th value the earlier strips of this
        // query reached (strips are dispatched in order, so the first strips
        // have usually finished by then); any k real rows bound the answer.
        if (ok && a.shared_r && blockIdx.y > 0) {
            const float R0 = __uint_as_float(__hip_atomic_load(&a.shared_r[q], __ATOMIC_RELAXED,
                                                               __HIP_MEMORY_SCOPE_AGENT));
            if (R0 < inf) thr[i] = round_up_f((double)R0 - (double)qsq[i] + (double)eps[i]);
        }
#pragma unroll
        for (int j = 0; j < K; ++j) {
            lv[i][j] = inf;
            li[i][j] = kSentinelIdx;
        }
    }

    // The tile's rows are screened first, each step of RU rows recording one
    // bit when any value of the lane passes; the recorded steps are rescored
    // at the tile's end (the rows still in LDS), against the thresholds as
    // they tighten.  A wave enters rescoring once per tile instead of at every
    // step where one of its lanes passes (about one step in five at c4),
    // and the screen loop carries no rescoring code.
    constexpr int STEPS = RT / RU;            // steps per tile (64)
    for (int64_t t0 = t_begin; t0 < t_end; t0 += RT) {
        const int nrows = (int)((t_end - t0) < RT ? (t_end - t0) : RT);
        __syncthreads();
        for (int e = tid; e < RT * DPN; e += 256) {
            const int r = e / DPN, c = e % DPN;
            float v = 0.0f;
            if (r < nrows) {
                if (c < D)
                    v = X[(t0 + r) * D + c];
                else if (c == D)
                    v = XSQ[t0 + r];
            }
            tile[e] = v;
        }
        __syncthreads();
        // screen: acc = ||x||^2 - 2 x.q, the group's smallest against the
        // threshold (one min per pair instead of a compare).  fminf drops
        // a NaN value unless the whole group is NaN (which then passes);
        // a NaN screen value means a NaN or infinite input, whose exact
        // value is NaN (never admitted) or +inf (admitted only while the
        // list is not full, when thr is +inf and every finite value
        // passes too), so dropping it here never loses a pair.  The
        // padding rows of a partial tile are zeros: they may pass, and
        // rescoring skips them.
        uint64_t pend = 0;
        for (int st = 0; st < STEPS && st * RU < nrows; ++st) {
            const int r0 = st * RU;
            // RU rows per step: their LDS reads are issued together, so one
            // LDS latency is paid per RU rows, not per row
            float row[RU][DPN];
#pragma unroll
            for (int rr = 0; rr < RU; ++rr)
#pragma unroll
                for (int c4 = 0; c4 < DPN / 4; ++c4) {
                    const float4 v = *reinterpret_cast<const float4*>(&tile[(r0 + rr) * DPN + 4 * c4]);
                    row[rr][4 * c4 + 0] = v.x;
                    row[rr][4 * c4 + 1] = v.y;
                    row[rr][4 * c4 + 2] = v.z;
                    row[rr][4 * c4 + 3] = v.w;
                }
            bool any = false;
#pragma unroll
            for (int i = 0; i < QL; ++i) {
                float mn = __builtin_huge_valf();
#pragma unroll
                for (int rr = 0; rr < RU; ++rr) {
                    float s_ = row[rr][D];
#pragma unroll
                    for (int c = 0; c < D; ++c) s_ = __builtin_fmaf(qm2[i][c], row[rr][c], s_);
                    mn = (rr == 0) ? s_ : __builtin_fminf(mn, s_);
                }
                any |= !(mn > thr[i]);
            }
            pend |= (uint64_t)any << st;
        }
        // rescoring of the recorded steps: the screen again, now against the
        // current thresholds, and an exact evaluation of each passing pair
        // in the reference's order, offered to the list with insert_lane's
        // rule (value, index), NaN never admitted
        while (pend) {
            const int st = __builtin_ctzll(pend);
            pend &= pend - 1;
            const int r0 = st * RU;
            const int rmax = (nrows - r0) < RU ? (nrows - r0) : RU;  // padding rows of the last step
#pragma unroll
            for (int i = 0; i < QL; ++i) {
                uint32_t m = 0;
#pragma unroll
                for (int rr = 0; rr < RU; ++rr) {
                    const float* yr = &tile[(r0 + rr) * DPN];
                    float s_ = yr[D];
#pragma unroll
                    for (int c = 0; c < D; ++c) s_ = __builtin_fmaf(qm2[i][c], yr[c], s_);
                    m |= (uint32_t)!(s_ > thr[i]) << rr;
                }
                m &= (rmax >= 32) ? 0xFFFFFFFFu : ((1u << rmax) - 1u);
                while (m) {
                    const int rr = __builtin_ctz(m);
                    m &= m - 1;
                    const float* yr = &tile[(r0 + rr) * DPN];
                    const uint32_t t = (uint32_t)(t0 + r0 + rr);
                    float e = 0.0f;
#pragma unroll
                    for (int c = 0; c < D; ++c) {
                        const float diff = qv[i][c] - yr[c];
                        if (ARM == ARM_EUCLID_FMA)
                            e = __builtin_fmaf(diff, diff, e);
                        else
                            e = e + diff * diff;
                    }
                    if (!(e <= worst[i]) || (e == worst[i] && t > worst_i[i])) continue;
                    float cav = e;
                    uint32_t cai = t;
                    // positions k..K-1 only ever receive pairs pushed out of the
                    // first k, so they never influence the kept ones
#pragma unroll
                    for (int j = 0; j < K; ++j) {
                        const float jv = lv[i][j];
                        const uint32_t ji = li[i][j];
                        if (cav < jv || (cav == jv && cai < ji)) {
                            lv[i][j] = cav;
                            li[i][j] = cai;
                            cav = jv;
                            cai = ji;
                        }
                    }
#pragma unroll
                    for (int j = 0; j < K; ++j)
                        if (j == k - 1) {
                            worst[i] = lv[i][j];
                            worst_i[i] = li[i][j];
                        }
                    // exact <= R  =>  ||x||^2 - 2 x.q <= R - ||q||^2 + eps:
                    // (R + eps) - ||q||^2 in f32, raised by four times its
                    // rounding bound (2^-126 near zero) -- an upper bound
                    if (worst[i] < inf) {
                        const float we_ = worst[i] + eps[i];
                        const float s_ = we_ - qsq[i];
                        thr[i] = s_ + ((we_ + __builtin_fabsf(s_)) * 0x1p-22f + 0x1p-126f);
                    }
                }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < QL; ++i) {
        const int64_t q = qbase + 256 * i;
        if (q >= a.nq) continue;
        if (a.shared_r && worst[i] < inf) atomicMin(&a.shared_r[q], __float_as_uint(worst[i]));
#pragma unroll
        for (int j = 0; j < K; ++j) {
            if (j < k) {
                if (a.nstrips > 1) {
                    const int64_t o = ((int64_t)blockIdx.y * a.nq + q) * k + j;
                    a.part_val[o] = lv[i][j];
                    a.part_idx[o] = li[i][j];
                } else {
                    const int64_t o = q * k + j;
                    a.out_val[o] = (a.mode == EMIT_SQRT) ? __builtin_sqrtf(lv[i][j]) : lv[i][j];
                    a.out_idx[o] = (li[i][j] == kSentinelIdx) ? 0u : li[i][j];
                }
            }
        }
    }
}

// Strip merge, one lane per query: the query's list and each strip's list
// (sorted, k <= K entries, padded with sentinels) are merged in registers.
// The K smallest of two sorted lists by the (value, index) order are
// min(A[j], B[K-1-j]), a bitonic sequence; K log2(K) / 2 compare-exchanges
// sort it.  The order is total (indices are distinct across strips), so the
// result is the first k of the union, whatever the network.
template <int K>
__global__ __launch_bounds__(256) void lowd_merge_kernel(LowdArgs32 a) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= a.nq) return;
    const int k = a.k;
    const float inf = __builtin_huge_valf();
    float lv[K];
    uint32_t li[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        lv[j] = (j < k) ? a.part_val[q * k + j] : inf;
        li[j] = (j < k) ? a.part_idx[q * k + j] : kSentinelIdx;
    }
    for (int s = 1; s < a.nstrips; ++s) {
        const int64_t o = ((int64_t)s * a.nq + q) * k;
        float bv[K];
        uint32_t bi[K];
#pragma unroll
        for (int j = 0; j < K; ++j) {
            bv[j] = (j < k) ? a.part_val[o + j] : inf;
            bi[j] = (j < k) ? a.part_idx[o + j] : kSentinelIdx;
        }
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const bool t = pair_less<float>(bv[K - 1 - j], bi[K - 1 - j], lv[j], li[j]);
            lv[j] = t ? bv[K - 1 - j] : lv[j];
            li[j] = t ? bi[K - 1 - j] : li[j];
        }
#pragma unroll
        for (int m = K / 2; m > 0; m >>= 1) {
#pragma unroll
            for (int j = 0; j < K; ++j) {
                if ((j & m) == 0) {
                    const bool t = pair_less<float>(lv[j + m], li[j + m], lv[j], li[j]);
                    const float v0 = lv[j], v1 = lv[j + m];
                    const uint32_t i0 = li[j], i1 = li[j + m];
                    lv[j] = t ? v1 : v0;
                    li[j] = t ? i1 : i0;
                    lv[j + m] = t ? v0 : v1;
                    li[j + m] = t ? i0 : i1;
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < K; ++j) {
        if (j < k) {
            a.out_val[q * k + j] = (a.mode == EMIT_SQRT) ? __builtin_sqrtf(lv[j]) : lv[j];
            a.out_idx[q * k + j] = (li[j] == kSentinelIdx) ? 0u : li[j];
        }
    }
}

__global__ void lowd_fill_inf_kernel(unsigned int* p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0x7F800000u;
}

template <int D, int K, int ARM>
hipError_t launch3(const LowdArgs32& a, hipStream_t s) {
    constexpr int QL = lowd_queries_per_lane(K);
    dim3 grid((unsigned)((a.nq + 256 * QL - 1) / (256 * QL)), (unsigned)a.nstrips);
    hipLaunchKernelGGL((knn_lowd_kernel<D, K, QL, ARM>), grid, dim3(256), 0, s, a);
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
int lowd_queries_per_block(int k) { return 256 * lowd_queries_per_lane(k <= 1 ? 1 : k <= 4 ? 4 : k <= 8 ? 8 : k <= 16 ? 16 : 32); }
int lowd_max_k() { return kMaxK; }

hipError_t launch_lowd_f32(const LowdArgs32& a, int arm, hipStream_t s) {
    if (a.d < 1 || a.d > kMaxD || a.k < 1 || a.k > kMaxK) return hipErrorInvalidValue;
    if (a.shared_r) {
        hipLaunchKernelGGL(lowd_fill_inf_kernel, dim3((unsigned)((a.nq + 255) / 256)), dim3(256), 0, s, a.shared_r,
                           a.nq);
        if (hipGetLastError() != hipSuccess) return hipErrorLaunchFailure;
    }
    hipError_t e;
    if (arm == ARM_EUCLID_FMA)
        e = launch_d<ARM_EUCLID_FMA>(a, s);
    else if (arm == ARM_EUCLID_MULADD)
        e = launch_d<ARM_EUCLID_MULADD>(a, s);
    else
        return hipErrorInvalidValue;
    if (e != hipSuccess || a.nstrips <= 1) return e;
    const dim3 mg((unsigned)((a.nq + 255) / 256));
    if (a.k <= 1)
        hipLaunchKernelGGL(lowd_merge_kernel<1>, mg, dim3(256), 0, s, a);
    else if (a.k <= 4)
        hipLaunchKernelGGL(lowd_merge_kernel<4>, mg, dim3(256), 0, s, a);
    else if (a.k <= 8)
        hipLaunchKernelGGL(lowd_merge_kernel<8>, mg, dim3(256), 0, s, a);
    else if (a.k <= 16)
        hipLaunchKernelGGL(lowd_merge_kernel<16>, mg, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(lowd_merge_kernel<32>, mg, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace mlrs
