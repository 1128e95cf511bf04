// Low-dimension kNN on the vector ALUs (d <= 16), no MFMA, f32 and f64,
// Euclidean and cosine.
//
// The MI355X counterpart of euclidean_topk_rows_cpu_direct
// (crates/mlrs-kernels/src/knn.rs:2968-3227).  Each lane owns QL query rows
// (lowd_queries_per_lane), keeps their sorted k-lists in VGPRs and walks
// every index row of its strip.  Per (query, row) pair the screen costs d
// FMAs: the expansion ||x||^2 - 2 x.q accumulated from the row's precomputed
// squared norm, against the threshold derived from the query's exact k-th
// value (the same rigorous rounding bound as the Gram kernels, in the
// element type).  A pair that passes is evaluated exactly, right there, in
// the reference arm's order -- fma(q-x, q-x, acc) (or acc + d*d for the host
// arm) over ascending columns, from the query in registers and the row in
// LDS -- and offered to the list with insert_lane's rule (knn.rs:2655-2706):
// (value, index) order, NaN never admitted.  The exact direct form is what
// the list holds, so results are the reference's bit for bit.
//
// Index rows are staged through LDS with their norm appended ((d+1) values
// padded to 16 bytes); every lane of a wave reads the same row at the same
// time, so the reads are LDS broadcasts.
//
// Cosine (the metric arm, ARM_COS_FOLD: d <= 128, k <= 128 always holds
// here) screens by the Gram kernels' cosine screen, the dot product scaled
// by the row's -1/||x|| (staged after the row, then its squared norm),
// against ((R + eps) - 1) ||q||, eps the absolute cosine bound; a passing
// pair is evaluated as the arm does (fma dot product over ascending
// columns, sqrt(||q||^2 ||x||^2), divide, clamp to [0, 2]).  Zero queries
// and queries whose norm sums may overflow are never screened (every row is
// evaluated exactly), as in the Gram kernels.  f64 runs the same code in double:
// MI355X issues v_fma_f64 at the rate of a non-packed v_fma_f32, so the f64
// screen costs what the f32 one does, and only the LDS reads double.
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

constexpr int kMaxD = 16;
constexpr int kMaxK = 32;

// Element-type arithmetic of the low-d kernel.
template <typename T>
struct LowdNum;
template <>
struct LowdNum<float> {
    typedef float4 vec;  // one 16-byte LDS read
    static constexpr int kVec = 4;
    static __device__ __forceinline__ float fma_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
    static __device__ __forceinline__ float min_(float a, float b) { return __builtin_fminf(a, b); }
    static __device__ __forceinline__ float abs_(float a) { return __builtin_fabsf(a); }
    static __device__ __forceinline__ float sqrt_(float a) { return __builtin_sqrtf(a); }
    static __device__ __forceinline__ float inf() { return __builtin_huge_valf(); }
    // four unit roundoffs and the smallest normal: the threshold's margin
    static __device__ __forceinline__ float margin(float we, float s) {
        return (we + __builtin_fabsf(s)) * 0x1p-22f + 0x1p-126f;
    }
    static __device__ __forceinline__ unsigned int bits(float v) { return __float_as_uint(v); }
    static __device__ __forceinline__ float from_bits(unsigned int b) { return __uint_as_float(b); }
    static __device__ __forceinline__ double xmax(const NormStats* st) { return (double)st->xsq_max; }
    static __device__ __forceinline__ void unpack(const vec& v, float* o) {
        o[0] = v.x;
        o[1] = v.y;
        o[2] = v.z;
        o[3] = v.w;
    }
};
template <>
struct LowdNum<double> {
    typedef double2 vec;
    static constexpr int kVec = 2;
    static __device__ __forceinline__ double fma_(double a, double b, double c) { return __builtin_fma(a, b, c); }
    static __device__ __forceinline__ double min_(double a, double b) { return __builtin_fmin(a, b); }
    static __device__ __forceinline__ double abs_(double a) { return __builtin_fabs(a); }
    static __device__ __forceinline__ double sqrt_(double a) { return __builtin_sqrt(a); }
    static __device__ __forceinline__ double inf() { return __builtin_huge_val(); }
    static __device__ __forceinline__ double margin(double we, double s) {
        return (we + __builtin_fabs(s)) * 0x1p-51 + 0x1p-1022;
    }
    static __device__ __forceinline__ unsigned long long bits(double v) {
        return (unsigned long long)__double_as_longlong(v);
    }
    static __device__ __forceinline__ double from_bits(unsigned long long b) {
        return __longlong_as_double((long long)b);
    }
    static __device__ __forceinline__ double xmax(const NormStats* st) { return st->xsq_max64; }
    static __device__ __forceinline__ void unpack(const vec& v, double* o) {
        o[0] = v.x;
        o[1] = v.y;
    }
};

// NV staged values per row (the row, then its norm operands), padded to
// whole 16-byte reads.
template <typename T, int NV>
constexpr int lowd_row_width() {
    return (NV + LowdNum<T>::kVec - 1) / LowdNum<T>::kVec * LowdNum<T>::kVec;
}

// Cosine screen threshold: exact <= R  =>  1 + acc/||q|| <= R + eps  =>
// acc <= (R + eps - 1) ||q||; f32 rounded up from double, f64 in double with
// its rounding inside eps (the Gram kernels' forms).
__device__ __forceinline__ float lowd_cos_threshold(float R, float qs, float eps) {
    return round_up_f(((double)R + (double)eps - 1.0) * (double)qs);
}
__device__ __forceinline__ double lowd_cos_threshold(double R, double qs, double eps) {
    return ((R + eps) - 1.0) * qs;
}

template <typename T, int D, int K, int QL, int ARM>
__global__ __launch_bounds__(256) void knn_lowd_kernel(LowdArgs<T> a) {
    typedef LowdNum<T> N;
    constexpr bool COS = ARM == ARM_COS_FOLD;
    // staged per row: Euclidean ||x||^2; cosine -1/||x||, then ||x||^2
    constexpr int DPN = lowd_row_width<T, D + (COS ? 2 : 1)>();
#ifndef MLRS_LOWD_RU4
#define MLRS_LOWD_RU4 8
#endif
    // rows per screening step: 8 for rows of at most four values (d <= 3),
    // else by the padded row width in floats (f64 d <= 3 at 8 rows measured
    // faster than at 4: 36.6 -> 33.2 ms at d = 2, 145 -> 115 ms at d = 3,
    // k = 32; wider f64 rows slower at 4 rows than at 2)
    constexpr int W4 = DPN * (int)sizeof(T) / 4;
    constexpr int RU = DPN <= 4 ? MLRS_LOWD_RU4 : (W4 <= 8 ? 4 : 2);
    constexpr int RT = 64 * RU;            // index rows per LDS tile: 64 steps
    __shared__ __attribute__((aligned(16))) T tile[RT * DPN];

    const int tid = threadIdx.x;
    const int64_t qbase = (int64_t)blockIdx.x * (256 * QL) + tid;
    const int64_t t_begin = (int64_t)blockIdx.y * a.rows_per_strip;
    int64_t t_end = t_begin + a.rows_per_strip;
    if (t_end > a.nt) t_end = a.nt;
    const int k = a.k;
    const T inf = N::inf();
    const T* __restrict__ X = a.x;
    const T* __restrict__ XSQ = a.xsq;
    const T* __restrict__ XSCALE = a.xscale;

    T qv[QL][D];    // the queries
    T qm2[QL][D];   // Euclidean: -2 * the queries (exact scaling) for the screen
    T qsq[QL], eps[QL], thr[QL], worst[QL];
    T qs[QL];       // cosine: ||q||, the screen's scale
    bool screened[QL];  // cosine: the screen bound holds for this query
    uint32_t worst_i[QL];
    T lv[QL][K];
    uint32_t li[QL][K];
    const double xmax = N::xmax(a.stats);
#pragma unroll
    for (int i = 0; i < QL; ++i) {
        const int64_t q = qbase + 256 * i;
        const bool ok = q < a.nq;
#pragma unroll
        for (int c = 0; c < D; ++c) {
            qv[i][c] = ok ? a.q[q * D + c] : T(0);
            qm2[i][c] = T(-2) * qv[i][c];
        }
        qsq[i] = ok ? a.qsq[q] : T(0);
        eps[i] = (T)(a.eps_rel * ((double)qsq[i] + xmax) + a.eps_abs);
        qs[i] = N::sqrt_(qsq[i]);
        // cosine: a zero query ties every row (never screened), and the
        // bound needs norm sums well inside the range
        screened[i] = !COS || (qs[i] > T(0) && (double)qsq[i] + xmax <= (sizeof(T) == 4 ? 0x1p124 : 0x1p1020));
        // An inactive lane can never admit (prefill_lists' -inf bound, knn.rs:2875-2905).
        worst[i] = ok ? inf : -inf;
        thr[i] = ok ? inf : -inf;
        worst_i[i] = kSentinelIdx;
        // A later strip starts from the k-th value the earlier strips of this
        // query reached (strips are dispatched in order, so the first strips
        // have usually finished by then); any k real rows bound the answer.
        if (ok && a.shared_r && blockIdx.y > 0) {
            const T R0 = N::from_bits(__hip_atomic_load(&a.shared_r[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            if (R0 < inf && screened[i]) {
                if constexpr (COS) {
                    thr[i] = lowd_cos_threshold(R0, qs[i], eps[i]);
                } else if constexpr (sizeof(T) == 4) {
                    thr[i] = round_up_f((double)R0 - (double)qsq[i] + (double)eps[i]);
                } else {
                    const T we_ = R0 + eps[i];
                    const T s_ = we_ - qsq[i];
                    thr[i] = s_ + N::margin(we_, s_);
                }
            }
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
            T v = T(0);
            if (r < nrows) {
                if (c < D)
                    v = X[(t0 + r) * D + c];
                else if (c == D)
                    v = COS ? XSCALE[t0 + r] : XSQ[t0 + r];
                else if (COS && c == D + 1)
                    v = XSQ[t0 + r];
            }
            tile[e] = v;
        }
        __syncthreads();
        // screen: acc = ||x||^2 - 2 x.q, the group's smallest against the
        // threshold (one min per pair instead of a compare).  fmin drops
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
            T row[RU][DPN];
#pragma unroll
            for (int rr = 0; rr < RU; ++rr)
#pragma unroll
                for (int c4 = 0; c4 < DPN / N::kVec; ++c4) {
                    const typename N::vec v =
                        *reinterpret_cast<const typename N::vec*>(&tile[(r0 + rr) * DPN + N::kVec * c4]);
                    N::unpack(v, &row[rr][N::kVec * c4]);
                }
            bool any = false;
#pragma unroll
            for (int i = 0; i < QL; ++i) {
                T mn = inf;
#pragma unroll
                for (int rr = 0; rr < RU; ++rr) {
                    T s_;
                    if constexpr (COS) {
                        s_ = T(0);
#pragma unroll
                        for (int c = 0; c < D; ++c) s_ = N::fma_(qv[i][c], row[rr][c], s_);
                        s_ = s_ * row[rr][D];
                    } else {
                        s_ = row[rr][D];
#pragma unroll
                        for (int c = 0; c < D; ++c) s_ = N::fma_(qm2[i][c], row[rr][c], s_);
                    }
                    mn = (rr == 0) ? s_ : N::min_(mn, s_);
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
                    const T* yr = &tile[(r0 + rr) * DPN];
                    T s_;
                    if constexpr (COS) {
                        s_ = T(0);
#pragma unroll
                        for (int c = 0; c < D; ++c) s_ = N::fma_(qv[i][c], yr[c], s_);
                        s_ = s_ * yr[D];
                    } else {
                        s_ = yr[D];
#pragma unroll
                        for (int c = 0; c < D; ++c) s_ = N::fma_(qm2[i][c], yr[c], s_);
                    }
                    m |= (uint32_t)!(s_ > thr[i]) << rr;
                }
                m &= (rmax >= 32) ? 0xFFFFFFFFu : ((1u << rmax) - 1u);
                while (m) {
                    const int rr = __builtin_ctz(m);
                    m &= m - 1;
                    const T* yr = &tile[(r0 + rr) * DPN];
                    const uint32_t t = (uint32_t)(t0 + r0 + rr);
                    T e = T(0);
                    if constexpr (COS) {
                        // the metric arm's cosine (exact_pair, ARM_COS_FOLD)
                        T dot = T(0);
#pragma unroll
                        for (int c = 0; c < D; ++c) dot = N::fma_(qv[i][c], yr[c], dot);
                        const T denom = N::sqrt_(qsq[i] * yr[D + 1]);
                        const T sim = (denom > T(0)) ? dot / denom : T(0);
                        e = clamp02<T>(T(1) - sim);
                    } else {
#pragma unroll
                        for (int c = 0; c < D; ++c) {
                            const T diff = qv[i][c] - yr[c];
                            if (ARM == ARM_EUCLID_FMA)
                                e = N::fma_(diff, diff, e);
                            else
                                e = e + diff * diff;
                        }
                    }
                    if (!(e <= worst[i]) || (e == worst[i] && t > worst_i[i])) continue;
                    T cav = e;
                    uint32_t cai = t;
                    // positions k..K-1 only ever receive pairs pushed out of the
                    // first k, so they never influence the kept ones
#pragma unroll
                    for (int j = 0; j < K; ++j) {
                        const T jv = lv[i][j];
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
                    // (R + eps) - ||q||^2 in the element type, raised by four
                    // times its rounding bound (the smallest normal near
                    // zero) -- an upper bound
                    if (worst[i] < inf && screened[i]) {
                        if constexpr (COS) {
                            thr[i] = lowd_cos_threshold(worst[i], qs[i], eps[i]);
                        } else {
                            const T we_ = worst[i] + eps[i];
                            const T s_ = we_ - qsq[i];
                            thr[i] = s_ + N::margin(we_, s_);
                        }
                    }
                }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < QL; ++i) {
        const int64_t q = qbase + 256 * i;
        if (q >= a.nq) continue;
        if (a.shared_r && worst[i] < inf) atomicMin(&a.shared_r[q], N::bits(worst[i]));
#pragma unroll
        for (int j = 0; j < K; ++j) {
            if (j < k) {
                if (a.nstrips > 1) {
                    const int64_t o = ((int64_t)blockIdx.y * a.nq + q) * k + j;
                    a.part_val[o] = lv[i][j];
                    a.part_idx[o] = li[i][j];
                } else {
                    const int64_t o = q * k + j;
                    a.out_val[o] = (a.mode == EMIT_SQRT) ? N::sqrt_(lv[i][j]) : lv[i][j];
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
template <typename T, int K>
__global__ __launch_bounds__(256) void lowd_merge_kernel(LowdArgs<T> a) {
    typedef LowdNum<T> N;
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= a.nq) return;
    const int k = a.k;
    const T inf = N::inf();
    T lv[K];
    uint32_t li[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        lv[j] = (j < k) ? a.part_val[q * k + j] : inf;
        li[j] = (j < k) ? a.part_idx[q * k + j] : kSentinelIdx;
    }
    for (int s = 1; s < a.nstrips; ++s) {
        const int64_t o = ((int64_t)s * a.nq + q) * k;
        T bv[K];
        uint32_t bi[K];
#pragma unroll
        for (int j = 0; j < K; ++j) {
            bv[j] = (j < k) ? a.part_val[o + j] : inf;
            bi[j] = (j < k) ? a.part_idx[o + j] : kSentinelIdx;
        }
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const bool t = pair_less<T>(bv[K - 1 - j], bi[K - 1 - j], lv[j], li[j]);
            lv[j] = t ? bv[K - 1 - j] : lv[j];
            li[j] = t ? bi[K - 1 - j] : li[j];
        }
#pragma unroll
        for (int m = K / 2; m > 0; m >>= 1) {
#pragma unroll
            for (int j = 0; j < K; ++j) {
                if ((j & m) == 0) {
                    const bool t = pair_less<T>(lv[j + m], li[j + m], lv[j], li[j]);
                    const T v0 = lv[j], v1 = lv[j + m];
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
            a.out_val[q * k + j] = (a.mode == EMIT_SQRT) ? N::sqrt_(lv[j]) : lv[j];
            a.out_idx[q * k + j] = (li[j] == kSentinelIdx) ? 0u : li[j];
        }
    }
}

// The shared bounds start at +inf (as bits of the element type).
template <typename B>
__global__ void lowd_fill_inf_kernel(B* p, int64_t n, B inf_bits) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = inf_bits;
}

// List capacity of a k (the kernels are instantiated for these).
constexpr int lowd_list_cap(int k) { return k <= 1 ? 1 : k <= 4 ? 4 : k <= 8 ? 8 : k <= 16 ? 16 : 32; }

template <typename T, int D, int K, int ARM>
hipError_t launch3(const LowdArgs<T>& a, hipStream_t s) {
    constexpr int QL = lowd_queries_per_lane<T>(K, D);
    dim3 grid((unsigned)((a.nq + 256 * QL - 1) / (256 * QL)), (unsigned)a.nstrips);
    hipLaunchKernelGGL((knn_lowd_kernel<T, D, K, QL, ARM>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

template <typename T, int D, int ARM>
hipError_t launch_k(const LowdArgs<T>& a, hipStream_t s) {
    switch (lowd_list_cap(a.k)) {
    case 1: return launch3<T, D, 1, ARM>(a, s);
    case 4: return launch3<T, D, 4, ARM>(a, s);
    case 8: return launch3<T, D, 8, ARM>(a, s);
    case 16: return launch3<T, D, 16, ARM>(a, s);
    default: return launch3<T, D, 32, ARM>(a, s);
    }
}

template <typename T, int ARM>
hipError_t launch_d(const LowdArgs<T>& a, hipStream_t s) {
    switch (a.d) {
    case 1: return launch_k<T, 1, ARM>(a, s);
    case 2: return launch_k<T, 2, ARM>(a, s);
    case 3: return launch_k<T, 3, ARM>(a, s);
    case 4: return launch_k<T, 4, ARM>(a, s);
    case 5: return launch_k<T, 5, ARM>(a, s);
    case 6: return launch_k<T, 6, ARM>(a, s);
    case 7: return launch_k<T, 7, ARM>(a, s);
    case 8: return launch_k<T, 8, ARM>(a, s);
    case 9: return launch_k<T, 9, ARM>(a, s);
    case 10: return launch_k<T, 10, ARM>(a, s);
    case 11: return launch_k<T, 11, ARM>(a, s);
    case 12: return launch_k<T, 12, ARM>(a, s);
    case 13: return launch_k<T, 13, ARM>(a, s);
    case 14: return launch_k<T, 14, ARM>(a, s);
    case 15: return launch_k<T, 15, ARM>(a, s);
    case 16: return launch_k<T, 16, ARM>(a, s);
    default: return hipErrorInvalidValue;
    }
}

template <typename T>
hipError_t launch_lowd(const LowdArgs<T>& a, int arm, hipStream_t s) {
    if (a.d < 1 || a.d > kMaxD || a.k < 1 || a.k > kMaxK) return hipErrorInvalidValue;
    if (a.shared_r) {
        typedef typename LowdBits<T>::type B;
        const B inf_bits = sizeof(T) == 4 ? (B)0x7F800000u : (B)0x7FF0000000000000ull;
        hipLaunchKernelGGL(lowd_fill_inf_kernel<B>, dim3((unsigned)((a.nq + 255) / 256)), dim3(256), 0, s,
                           a.shared_r, a.nq, inf_bits);
        if (hipGetLastError() != hipSuccess) return hipErrorLaunchFailure;
    }
    hipError_t e;
    if (arm == ARM_EUCLID_FMA)
        e = launch_d<T, ARM_EUCLID_FMA>(a, s);
    else if (arm == ARM_EUCLID_MULADD)
        e = launch_d<T, ARM_EUCLID_MULADD>(a, s);
    else if (arm == ARM_COS_FOLD && a.xscale)
        e = launch_d<T, ARM_COS_FOLD>(a, s);
    else
        return hipErrorInvalidValue;
    if (e != hipSuccess || a.nstrips <= 1) return e;
    const dim3 mg((unsigned)((a.nq + 255) / 256));
    switch (lowd_list_cap(a.k)) {
    case 1: hipLaunchKernelGGL((lowd_merge_kernel<T, 1>), mg, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((lowd_merge_kernel<T, 4>), mg, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((lowd_merge_kernel<T, 8>), mg, dim3(256), 0, s, a); break;
    case 16: hipLaunchKernelGGL((lowd_merge_kernel<T, 16>), mg, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((lowd_merge_kernel<T, 32>), mg, dim3(256), 0, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace

int lowd_max_d() { return kMaxD; }
int lowd_max_k() { return kMaxK; }

int lowd_queries_per_block(int k, int64_t d, int elem_bytes) {
    const int K = lowd_list_cap(k);
    return 256 * (elem_bytes == 8 ? lowd_queries_per_lane<double>(K, (int)d) : lowd_queries_per_lane<float>(K, (int)d));
}

hipError_t launch_lowd_f32(const LowdArgs32& a, int arm, hipStream_t s) { return launch_lowd<float>(a, arm, s); }
hipError_t launch_lowd_f64(const LowdArgs64& a, int arm, hipStream_t s) { return launch_lowd<double>(a, arm, s); }

}  // namespace mlrs
