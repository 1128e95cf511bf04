// Device-side building blocks shared by the kNN kernels (gfx950, wave64).
//
// Everything here is compiled with -ffp-contract=off: each multiply and add
// rounds on its own, and a fused multiply-add appears only where the mlrs
// cpu-backend arithmetic writes one, so the exact distance routines below are
// bit-for-bit the reference's (see the per-routine citations).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "knn_kernels.hpp"  // EmitMode

namespace mlrs {

// Arithmetic arms of the reference cpu backend (the ones results are compared
// against), selected by the host exactly as metric_topk
// (crates/mlrs-algos/src/neighbors/nearest.rs:891-953) selects the cpu arm.
enum Arm : int {
    // euclidean_topk_rows_cpu_direct / _cpu_metric
    // (crates/mlrs-kernels/src/knn.rs:3042-3075, :3265-3275): fma(x-y, x-y, acc)
    ARM_EUCLID_FMA = 0,
    // knn_host lane_distances (crates/mlrs-backend/src/prims/knn_host.rs:703-708),
    // dist_direct_2d_c4 (crates/mlrs-kernels/src/kmeans.rs:206-274),
    // euclidean_sq_dist (crates/mlrs-kernels/src/distance.rs:411-440): acc + d*d
    ARM_EUCLID_MULADD = 1,
    // cosine_topk_rows_cpu_metric: fma dot then cosine_fold over row_sumsq
    // squared norms (crates/mlrs-kernels/src/knn.rs:3366-3375, :3646-3661)
    ARM_COS_FOLD = 2,
    // knn_host cosine: acc + x*y, 1 - dot*ix*iy over reciprocal norms, clamp
    // (crates/mlrs-backend/src/prims/knn_host.rs:382-397, :750-764)
    ARM_COS_HOST = 3,
    // cosine_dist (crates/mlrs-kernels/src/distance.rs:257-310): acc + x*y,
    // sqrt(xn*yn) over row_sumsq norms, divide, clamp
    ARM_COS_PAIRWISE = 4,
    // metric_step_manhattan / knn_host / manhattan_dist (knn.rs:3277-3286,
    // knn_host.rs:715-718, distance.rs:67-91): acc + |x - y|
    ARM_MANHATTAN = 5,
    // metric_step_chebyshev / chebyshev_dist (knn.rs:3288-3312, distance.rs:
    // 154-180): acc = (|x - y| > acc) ? |x - y| : acc, so NaN never replaces
    ARM_CHEBYSHEV = 6,
    // metric_step_minkowski_int (knn.rs:3330-3356): acc + |x - y|^pi by a
    // multiply chain, integer pi in 3..8
    ARM_MINKOWSKI_INT = 7,
    // metric_step_minkowski / minkowski_dist (knn.rs:3314-3328, distance.rs:
    // 201-227): acc + pow(|x - y|, p)
    ARM_MINKOWSKI_POW = 8,
};

template <typename T> struct FloatTraits;
template <> struct FloatTraits<float> {
    static __device__ __forceinline__ float inf() { return __builtin_huge_valf(); }
    static __device__ __forceinline__ float fma_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
    static __device__ __forceinline__ float sqrt_(float a) { return __builtin_sqrtf(a); }
    static __device__ __forceinline__ float abs_(float a) { return __builtin_fabsf(a); }
    static __device__ __forceinline__ float pow_(float a, float b) { return powf(a, b); }
};
template <> struct FloatTraits<double> {
    static __device__ __forceinline__ double inf() { return __builtin_huge_val(); }
    static __device__ __forceinline__ double fma_(double a, double b, double c) { return __builtin_fma(a, b, c); }
    static __device__ __forceinline__ double sqrt_(double a) { return __builtin_sqrt(a); }
    static __device__ __forceinline__ double abs_(double a) { return __builtin_fabs(a); }
    static __device__ __forceinline__ double pow_(double a, double b) { return pow(a, b); }
};

static constexpr uint32_t kSentinelIdx = 0xFFFFFFFFu;

// (value, index) total order of insert_lane (crates/mlrs-kernels/src/knn.rs:
// 2655-2706): smaller value first, lower index on an equal value.
template <typename T>
__device__ __forceinline__ bool pair_less(T va, uint32_t ia, T vb, uint32_t ib) {
    // bitwise, not short-circuit: evaluated as lane masks with no branches
    return (va < vb) | ((va == vb) & (ia < ib));
}

// The reference clamp written in statement form: NaN passes through.
template <typename T>
__device__ __forceinline__ T clamp02(T v) {
    v = (v < T(0)) ? T(0) : v;
    v = (v > T(2)) ? T(2) : v;
    return v;
}

// Sum of squares in ascending column order with separate multiply and add
// (row_sumsq, crates/mlrs-kernels/src/knn.rs:2130-2149; row_sqnorm,
// crates/mlrs-kernels/src/kmeans.rs:610).
template <typename T>
__device__ __forceinline__ T row_sumsq(const T* __restrict__ row, int64_t d) {
    T acc = T(0);
    for (int64_t c = 0; c < d; ++c) {
        T v = row[c];
        acc = acc + v * v;
    }
    return acc;
}

// Exact per-pair value of one arm, in the reference's operation order.
// q is the query row, y the training row.  `qa`/`ya` are the arm's per-row
// norm operands: squared norms for ARM_COS_FOLD / ARM_COS_PAIRWISE,
// reciprocal norms for ARM_COS_HOST, unused otherwise.
template <typename T, int ARM>
__device__ __forceinline__ T exact_pair(const T* __restrict__ q, const T* __restrict__ y, int64_t d,
                                        T qa, T ya) {
    using F = FloatTraits<T>;
    if (ARM == ARM_EUCLID_FMA) {
        T acc = T(0);
        for (int64_t c = 0; c < d; ++c) {
            T diff = q[c] - y[c];
            acc = F::fma_(diff, diff, acc);
        }
        return acc;
    } else if (ARM == ARM_EUCLID_MULADD) {
        T acc = T(0);
        for (int64_t c = 0; c < d; ++c) {
            T diff = q[c] - y[c];
            acc = acc + diff * diff;
        }
        return acc;
    } else if (ARM == ARM_COS_FOLD) {
        T dot = T(0);
        for (int64_t c = 0; c < d; ++c) dot = F::fma_(q[c], y[c], dot);
        T denom = F::sqrt_(qa * ya);
        T sim = (denom > T(0)) ? dot / denom : T(0);
        return clamp02<T>(T(1) - sim);
    } else if (ARM == ARM_COS_HOST) {
        T dot = T(0);
        for (int64_t c = 0; c < d; ++c) dot = dot + q[c] * y[c];
        return clamp02<T>(T(1) - dot * qa * ya);
    } else {  // ARM_COS_PAIRWISE
        T dot = T(0);
        for (int64_t c = 0; c < d; ++c) dot = dot + q[c] * y[c];
        T denom = F::sqrt_(qa * ya);
        T sim = T(0);
        if (denom > T(0)) sim = dot / denom;
        return clamp02<T>(T(1) - sim);
    }
}

// Smallest float >= t (screen thresholds are rounded up, never down).
__device__ __forceinline__ float round_up_f(double t) {
    float f = (float)t;
    if ((double)f < t) {  // step one ulp towards +inf
        uint32_t b = __float_as_uint(f);
        if (f == 0.0f)
            f = __uint_as_float(1u);
        else
            f = __uint_as_float(f > 0.0f ? b + 1u : b - 1u);
    }
    return f;
}

// ---------------------------------------------------------------------------
// Wave64 bitonic machinery over (value, index) pairs, one pair per lane.
// ---------------------------------------------------------------------------

// Lane exchanges.  The partner lane ^ m of a constant m comes from DPP (quad
// permutations for m = 1, 2; row shifts left and right for m = 4, 8) or from
// v_permlane{16,32}_swap (m = 16, 32): VALU operations, no round trip
// through the LDS crossbar as ds_bpermute (the generic __shfl_xor) takes.
// Every lane of the wave must be active.  The bitonic loops below are fully
// unrolled, so m is a constant by the time these are inlined.
__device__ __forceinline__ uint32_t lane_id_u() {
    return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}
__device__ __forceinline__ uint32_t xor_lane_u(uint32_t v, int m) {
    const uint32_t lane = lane_id_u();
    switch (m) {
    case 1: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    case 2: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    case 4: {
        const uint32_t up = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x104, 0xF, 0xF, false);  // row_shl:4
        const uint32_t dn = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
        return (lane & 4u) ? dn : up;
    }
    case 8: {
        const uint32_t up = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x108, 0xF, 0xF, false);  // row_shl:8
        const uint32_t dn = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x118, 0xF, 0xF, false);  // row_shr:8
        return (lane & 8u) ? dn : up;
    }
    case 16: {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16u) ? r[0] : r[1];
    }
    case 32: {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane & 32u) ? r[0] : r[1];
    }
    default: return (uint32_t)__shfl_xor((int)v, m, 64);
    }
}
// Value of lane 63 - lane: the mirror inside each 16-lane row, then the rows
// reversed (rows 0..3 -> 3..0 is lane ^ 48).
__device__ __forceinline__ uint32_t reverse_lane_u(uint32_t v) {
    const uint32_t r = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);  // row_mirror
    return xor_lane_u(xor_lane_u(r, 16), 32);
}

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __uint_as_float(xor_lane_u(__float_as_uint(v), m)); }
__device__ __forceinline__ double shfl_xor_f(double v, int m) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = xor_lane_u((uint32_t)b, m), hi = xor_lane_u((uint32_t)(b >> 32), m);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ uint32_t shfl_xor_u(uint32_t v, int m) { return xor_lane_u(v, m); }
__device__ __forceinline__ float reverse_f(float v) { return __uint_as_float(reverse_lane_u(__float_as_uint(v))); }
__device__ __forceinline__ double reverse_f(double v) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = reverse_lane_u((uint32_t)b), hi = reverse_lane_u((uint32_t)(b >> 32));
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ uint32_t reverse_u(uint32_t v) { return reverse_lane_u(v); }
__device__ __forceinline__ float shfl_f(float v, int src) { return __shfl(v, src, 64); }
__device__ __forceinline__ double shfl_f(double v, int src) { return __shfl(v, src, 64); }
__device__ __forceinline__ uint32_t shfl_u(uint32_t v, int src) { return (uint32_t)__shfl((int)v, src, 64); }
// Value of lane `src`, the same lane for the whole wave (v_readlane).
__device__ __forceinline__ float bcast_f(float v, int src) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), src));
}
__device__ __forceinline__ double bcast_f(double v, int src) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, src);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), src);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ uint32_t bcast_u(uint32_t v, int src) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, src);
}

// One compare-exchange step with the partner lane^m.  `up` says whether this
// lane's sub-sequence sorts ascending.
template <typename T>
__device__ __forceinline__ void bitonic_step(T& v, uint32_t& ix, int lane, int m, bool up) {
    T ov = shfl_xor_f(v, m);
    uint32_t oi = shfl_xor_u(ix, m);
    const bool lower = (lane & m) == 0;
    // The lower lane of an ascending pair keeps the smaller element, the upper
    // lane the larger; a descending pair the reverse.  Selects, no branches.
    const bool first = (lower == up);
    const bool take = (first & pair_less<T>(ov, oi, v, ix)) | (!first & pair_less<T>(v, ix, ov, oi));
    v = take ? ov : v;
    ix = take ? oi : ix;
}

// Full ascending bitonic sort of 64 lanes.
template <typename T>
__device__ __forceinline__ void wave_sort64(T& v, uint32_t& ix, int lane) {
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1) {
        bool up = (lane & size) == 0 || size == 64;
#pragma unroll
        for (int m = size >> 1; m > 0; m >>= 1) bitonic_step<T>(v, ix, lane, m, up);
    }
}

// Merge the ascending 64-lane sequence (v, ix) with the ascending list
// (lv, li): afterwards lanes 0..63 hold the 64 smallest pairs of the union,
// ascending.  Both inputs must be sorted.
template <typename T>
__device__ __forceinline__ void wave_merge64(T& lv, uint32_t& li, T v, uint32_t ix, int lane) {
    T rv = reverse_f(v);
    uint32_t ri = reverse_u(ix);
    const bool take = pair_less<T>(rv, ri, lv, li);
    lv = take ? rv : lv;
    li = take ? ri : li;
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) bitonic_step<T>(lv, li, lane, m, true);
}

// wave_merge64 that also returns the smallest value it discards (the upper
// half of the union), +inf when only sentinels are discarded.  Values must
// not be NaN.
template <typename T>
__device__ __forceinline__ T wave_merge64_drop(T& lv, uint32_t& li, T v, uint32_t ix, int lane) {
    T rv = reverse_f(v);
    uint32_t ri = reverse_u(ix);
    const bool take = pair_less<T>(rv, ri, lv, li);
    const T dv0 = take ? lv : rv;
    lv = take ? rv : lv;
    li = take ? ri : li;
    T dv = dv0;
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) bitonic_step<T>(lv, li, lane, m, true);
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
        const T o = shfl_xor_f(dv, m);
        dv = (o < dv) ? o : dv;
    }
    return dv;
}

// ---------------------------------------------------------------------------
// The same machinery on 64-bit keys: for f32 values the (value, index) order
// is the unsigned order of (orderable value bits << 32 | index), so one
// 64-bit compare replaces the two-part comparison.
// ---------------------------------------------------------------------------

// Order-preserving map of float bits to unsigned (negative values flipped).
__device__ __forceinline__ uint32_t f32_order_bits(float v) {
    const uint32_t u = __float_as_uint(v + 0.0f);  // -0 -> +0: equal values order by index
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float f32_from_order_bits(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
__device__ __forceinline__ unsigned long long pair_key(float v, uint32_t ix) {
    return ((unsigned long long)f32_order_bits(v) << 32) | ix;
}
__device__ __forceinline__ float key_value(unsigned long long key) { return f32_from_order_bits((uint32_t)(key >> 32)); }
__device__ __forceinline__ uint32_t key_index(unsigned long long key) { return (uint32_t)key; }
constexpr unsigned long long kKeyEmpty = 0xFF800000FFFFFFFFull;  // (+inf, sentinel index)

__device__ __forceinline__ unsigned long long xor_lane_key(unsigned long long v, int m) {
    return ((unsigned long long)xor_lane_u((uint32_t)(v >> 32), m) << 32) | xor_lane_u((uint32_t)v, m);
}

// Compare-exchange with lane ^ m.  Equal keys may be exchanged: they are
// the same pair (or both empty), so the sequence is unchanged.
__device__ __forceinline__ void bitonic_step_key(unsigned long long& v, int lane, int m, bool up) {
    const unsigned long long o = xor_lane_key(v, m);
    const bool first = (((lane & m) == 0) == up);
    const bool take = (o < v) == first;
    v = take ? o : v;
}

__device__ __forceinline__ void wave_sort64_key(unsigned long long& v, int lane) {
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1) {
        const bool up = (lane & size) == 0 || size == 64;
#pragma unroll
        for (int m = size >> 1; m > 0; m >>= 1) bitonic_step_key(v, lane, m, up);
    }
}

// Merge the ascending sequence v into the ascending list lv (the 64 smallest
// keys of the union stay in lv) and return the smallest key discarded.
__device__ __forceinline__ unsigned long long wave_merge64_key_drop(unsigned long long& lv, unsigned long long v,
                                                                    int lane) {
    const unsigned long long r =
        ((unsigned long long)reverse_lane_u((uint32_t)(v >> 32)) << 32) | reverse_lane_u((uint32_t)v);
    unsigned long long dv = (r < lv) ? lv : r;
    lv = (r < lv) ? r : lv;
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) bitonic_step_key(lv, lane, m, true);
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
        const unsigned long long o = xor_lane_key(dv, m);
        dv = (o < dv) ? o : dv;
    }
    return dv;
}
__device__ __forceinline__ void wave_merge64_key(unsigned long long& lv, unsigned long long v, int lane) {
    const unsigned long long r =
        ((unsigned long long)reverse_lane_u((uint32_t)(v >> 32)) << 32) | reverse_lane_u((uint32_t)v);
    lv = (r < lv) ? r : lv;
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) bitonic_step_key(lv, lane, m, true);
}

// ---------------------------------------------------------------------------
// Lists longer than a wave: NB blocks, element 64 r + lane in block r, the
// whole list ascending.  A sorted 64-lane sequence is merged in block by
// block: the 64 smallest of (block r, carry) stay in block r and the 64
// largest carry on into block r + 1 (every element of block r + 1 is >= all
// of block r, so the smallest 64 of everything from block r on lie in block r
// or the carry).  Each step is a half-cleaner of the bitonic union.
// ---------------------------------------------------------------------------
__device__ __forceinline__ unsigned long long reverse_key(unsigned long long v) {
    return ((unsigned long long)reverse_lane_u((uint32_t)(v >> 32)) << 32) | reverse_lane_u((uint32_t)v);
}
__device__ __forceinline__ void bitonic_clean_key(unsigned long long& v, int lane) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) bitonic_step_key(v, lane, m, true);
}
__device__ __forceinline__ uint32_t key_hi_u(unsigned long long v) { return (uint32_t)(v >> 32); }

// Merge the ascending 64-lane sequence v into the NB-block list lv; the
// 64 NB smallest keys stay, ascending, and the smallest discarded key is
// returned (kKeyEmpty-like keys when only empties are discarded).  A block
// whose largest key is below the carry's smallest is left as it is.
template <int NB>
__device__ __forceinline__ unsigned long long wave_merge_blocks_key_drop(unsigned long long (&lv)[NB],
                                                                         unsigned long long v, int lane) {
    unsigned long long carry = v;
#pragma unroll
    for (int r = 0; r < NB; ++r) {
        if (NB > 1) {
            // both keys are wave-uniform after the readlanes: a uniform branch
            const unsigned long long cmin = ((unsigned long long)bcast_u(key_hi_u(carry), 0) << 32) |
                                            bcast_u((uint32_t)carry, 0);
            const unsigned long long bmax = ((unsigned long long)bcast_u(key_hi_u(lv[r]), 63) << 32) |
                                            bcast_u((uint32_t)lv[r], 63);
            if (bmax < cmin) continue;
        }
        const unsigned long long rc = reverse_key(carry);
        const bool t = rc < lv[r];
        const unsigned long long lo = t ? rc : lv[r];
        carry = t ? lv[r] : rc;
        lv[r] = lo;
        bitonic_clean_key(lv[r], lane);
        if (r + 1 < NB) bitonic_clean_key(carry, lane);
    }
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
        const unsigned long long o = xor_lane_key(carry, m);
        carry = (o < carry) ? o : carry;
    }
    return carry;
}

// The order bits of list element `pos` (wave-uniform pos), from its block.
template <int NB>
__device__ __forceinline__ uint32_t list_hi_at(const unsigned long long (&lv)[NB], int pos) {
    const int b = pos >> 6;
    uint32_t v = key_hi_u(lv[0]);
#pragma unroll
    for (int r = 1; r < NB; ++r)
        if (b == r) v = key_hi_u(lv[r]);
    return bcast_u(v, pos & 63);
}

// The same block merge on (value, index) pairs (the seeds' lists, the f64
// kernel's lists); returns the smallest value discarded.  A block whose
// largest pair is below the carry's smallest is left as it is (a uniform
// test, NB > 1 only).
template <typename T, int NB>
__device__ __forceinline__ T wave_merge_blocks_drop(T (&lv)[NB], uint32_t (&li)[NB], T v, uint32_t ix, int lane) {
    T cv = v;
    uint32_t ci = ix;
#pragma unroll
    for (int r = 0; r < NB; ++r) {
        if (NB > 1) {
            const T cmin = bcast_f(cv, 0), bmax = bcast_f(lv[r], 63);
            const uint32_t cmi = bcast_u(ci, 0), bmi = bcast_u(li[r], 63);
            if (pair_less<T>(bmax, bmi, cmin, cmi)) continue;
        }
        const T rv = reverse_f(cv);
        const uint32_t ri = reverse_u(ci);
        const bool t = pair_less<T>(rv, ri, lv[r], li[r]);
        const T lov = t ? rv : lv[r];
        const uint32_t loi = t ? ri : li[r];
        cv = t ? lv[r] : rv;
        ci = t ? li[r] : ri;
        lv[r] = lov;
        li[r] = loi;
#pragma unroll
        for (int m = 32; m > 0; m >>= 1) bitonic_step<T>(lv[r], li[r], lane, m, true);
        if (r + 1 < NB) {
#pragma unroll
            for (int m = 32; m > 0; m >>= 1) bitonic_step<T>(cv, ci, lane, m, true);
        }
    }
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
        const T o = shfl_xor_f(cv, m);
        cv = (o < cv) ? o : cv;
    }
    return cv;
}
template <typename T, int NB>
__device__ __forceinline__ void wave_merge_blocks(T (&lv)[NB], uint32_t (&li)[NB], T v, uint32_t ix, int lane) {
    (void)wave_merge_blocks_drop<T, NB>(lv, li, v, ix, lane);
}

// Value of list element `pos` (wave-uniform pos), from its block.
template <typename T, int NB>
__device__ __forceinline__ T list_value_at(const T (&lv)[NB], int pos) {
    const int b = pos >> 6;
    T v = lv[0];
#pragma unroll
    for (int r = 1; r < NB; ++r)
        if (b == r) v = lv[r];
    return bcast_f(v, pos & 63);
}

// A 16-byte load through the global address space.  A pointer the compiler
// cannot prove global (one walked in a register array) is otherwise loaded
// with a flat instruction, which also counts against the LDS wait counter:
// every later wait for an LDS read would then wait for this load as well.
__device__ __forceinline__ float4 gload4(const float* p) {
    typedef float f4v_t __attribute__((ext_vector_type(4)));
    const f4v_t v = *(const __attribute__((address_space(1))) f4v_t*)p;
    return make_float4(v.x, v.y, v.z, v.w);
}

// Element r of a 16-float accumulator for a lane-varying r: a v_bfi_b32
// select tree on the bits of r (15 bitfield selects).  Written in asm: as
// C++ selects the compiler rebuilds a dynamic extract and expands it into a
// compare chain per element.
typedef float f32x16_t __attribute__((ext_vector_type(16)));
__device__ __forceinline__ float pick16(const f32x16_t& a, int r) {
    const uint32_t s0 = 0u - ((uint32_t)r & 1u), s1 = 0u - (((uint32_t)r >> 1) & 1u),
                   s2 = 0u - (((uint32_t)r >> 2) & 1u), s3 = 0u - (((uint32_t)r >> 3) & 1u);
    uint32_t l1[8], l2[4], l3[2], v;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(l1[i]) : "v"(s0), "v"(__float_as_uint(a[2 * i + 1])),
            "v"(__float_as_uint(a[2 * i])));
#pragma unroll
    for (int i = 0; i < 4; ++i)
        asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(l2[i]) : "v"(s1), "v"(l1[2 * i + 1]), "v"(l1[2 * i]));
#pragma unroll
    for (int i = 0; i < 2; ++i)
        asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(l3[i]) : "v"(s2), "v"(l2[2 * i + 1]), "v"(l2[2 * i]));
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(v) : "v"(s3), "v"(l3[1]), "v"(l3[0]));
    return __uint_as_float(v);
}

// Rotating wave priority for the kernels that run several workgroups per CU.
// The SIMD's instruction arbiter favours older waves, so with equal
// priorities the workgroups sharing a CU finish in dispatch order and the
// youngest runs its tail alone (c2: 20.3, 21.8 and 23.1 ms).  Every 64 tiles
// of a segment (tiles_done counts them) a wave moves to the next of `levels`
// priorities, offset by its
// workgroup's dispatch rank on the CU (the CU-mates of a grid of one
// resident round are gridDim.x / levels block ids apart), so each spends a
// third (a half) of its tiles at every level and the CU-mates finish
// together.
__device__ __forceinline__ void rotate_wave_priority(uint32_t tiles_done, int levels) {
    if ((tiles_done & 63u) != 0u || levels < 2) return;
    const uint32_t rank = (uint32_t)((uint64_t)blockIdx.x * (uint64_t)levels / gridDim.x);
    const uint32_t p = ((tiles_done >> 6) + rank) % (uint32_t)levels;
    if (p == 0)
        __builtin_amdgcn_s_setprio(0);
    else if (p == 1)
        __builtin_amdgcn_s_setprio(1);
    else
        __builtin_amdgcn_s_setprio(2);
}

// 16 bytes per lane from global memory straight into LDS (gfx950's
// global_load_lds_dwordx4, counted by vmcnt): lane i's bytes land at
// lds_wave_base + 16 i, lds_wave_base uniform over the wave.  The builtin
// exists only for the device target; the host pass, which never runs a
// kernel body, compiles the call away (it would otherwise drop the kernel's
// launch stub).
__device__ __forceinline__ void global_to_lds16(const void* g, void* lds_wave_base) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(g, lds_wave_base, 16, 0, 0);
#else
    (void)g;
    (void)lds_wave_base;
#endif
}

// Element r (0..7) of the pair (a0, a1) = (a0[0..3], a1[0..3]), by the same
// v_bfi_b32 select tree as pick16.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float pick8(const f32x4_t& a0, const f32x4_t& a1, int r) {
    const uint32_t s0 = 0u - ((uint32_t)r & 1u), s1 = 0u - (((uint32_t)r >> 1) & 1u),
                   s2 = 0u - (((uint32_t)r >> 2) & 1u);
    const float e[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
    uint32_t l1[4], l2[2], v;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(l1[i]) : "v"(s0), "v"(__float_as_uint(e[2 * i + 1])),
            "v"(__float_as_uint(e[2 * i])));
#pragma unroll
    for (int i = 0; i < 2; ++i)
        asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(l2[i]) : "v"(s1), "v"(l1[2 * i + 1]), "v"(l1[2 * i]));
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(v) : "v"(s2), "v"(l2[1]), "v"(l2[0]));
    return __uint_as_float(v);
}

// The Gram kernels' seed: for the kSeedQpb queries of one workgroup (four
// waves, kSeedQpw each), the k-th smallest EXACT value (the arm's operation
// order) over nsamp evenly spaced index rows, stored as the bits of its type
// into shared_r; any k rows bound the final k-th value from above.  Each
// batch of 64 sampled rows is staged through LDS in column chunks of 512
// bytes (coalesced loads, each row read once per workgroup); lane l of every
// wave continues its row's running sums, one per query, chunk by chunk, in
// ascending column order.  qop / yop: the arm's per-query / per-row operand
// arrays (squared norms for the fold arm, reciprocal norms for the knn_host
// arm, unused for Euclidean).
constexpr int kSeedQpw = 4;
constexpr int kSeedQpb = 4 * kSeedQpw;
constexpr int kSeedInsertMax = 8;  // batches with at most this many rows below the k-th insert them one by one
template <typename T, int ARM, typename Bits, int SB = 1>
__device__ __forceinline__ void seed_kth_block(const T* __restrict__ Q, const T* __restrict__ X, int64_t nq,
                                               int64_t nt, int64_t d, int k, int64_t nsamp,
                                               const T* __restrict__ qop, const T* __restrict__ yop,
                                               Bits* __restrict__ shared_r) {
    using F = FloatTraits<T>;
    constexpr int CH = 512 / (int)sizeof(T);  // columns per chunk (a power of two)
    constexpr int CH_LOG = sizeof(T) == 4 ? 7 : 6;
    constexpr int V = 16 / (int)sizeof(T);     // elements per 16-byte LDS read
    // LDS row stride: an odd number of 16-byte chunks, so the 16-byte reads of
    // 64 lanes (lane l: row l) spread over the banks
    constexpr int STR = CH + V;
    __shared__ __attribute__((aligned(16))) T rows[64][STR];
    __shared__ __attribute__((aligned(16))) T qch[kSeedQpb][CH];  // the workgroup's queries, same columns
    __shared__ uint32_t srow[64];              // the batch's sampled index rows
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const T inf = F::inf();
    const int64_t qb0 = (int64_t)blockIdx.x * kSeedQpb;
    const int64_t q0 = qb0 + (int64_t)w * kSeedQpw;
    const bool vec = (d % V == 0) && ((reinterpret_cast<uintptr_t>(Q) & 15) == 0) &&
                     ((reinterpret_cast<uintptr_t>(X) & 15) == 0);
    T qa[kSeedQpw], lv[kSeedQpw][SB];
    uint32_t li[kSeedQpw][SB];
#pragma unroll
    for (int j = 0; j < kSeedQpw; ++j) {
        const int64_t qg = (q0 + j < nq) ? q0 + j : nq - 1;  // past the end: repeats a query, not written
        qa[j] = (ARM == ARM_COS_FOLD || ARM == ARM_COS_HOST) ? qop[qg] : T(0);
#pragma unroll
        for (int b = 0; b < SB; ++b) {
            lv[j][b] = inf;
            li[j][b] = kSentinelIdx;
        }
    }
    for (int64_t s0 = 0; s0 < nsamp; s0 += 64) {
        const int64_t s = s0 + lane;
        const bool on = s < nsamp;
        const uint32_t t = on ? (uint32_t)((s * nt) / nsamp) : kSentinelIdx;
        __syncthreads();  // the previous batch's rows are no longer read
        if (tid < 64) srow[tid] = t;
        T acc[kSeedQpw];
#pragma unroll
        for (int j = 0; j < kSeedQpw; ++j) acc[j] = T(0);
        for (int64_t c0 = 0; c0 < d; c0 += CH) {
            const int cw = (d - c0 < CH) ? (int)(d - c0) : CH;
            __syncthreads();  // srow written; the previous chunk is no longer read
            // rows s0 .. s0+63 of the sample, columns c0 .. c0+CH: thread i
            // copies elements i, i+256, ... of the 64 x CH block (row-major;
            // consecutive threads read consecutive columns of one row), 16
            // bytes at a time where rows are 16-byte aligned (cw is then a
            // multiple of V), all of a thread's loads issued together
            if (vec) {
                constexpr int CV = CH / V;  // 16-byte pieces per chunk row (32)
#pragma unroll
                for (int i = 0; i < 64 * CV / 256; ++i) {
                    const int e = tid + 256 * i;
                    const int r = e / CV, c = (e % CV) * V;
                    const uint32_t tr = srow[r];
                    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (tr != kSentinelIdx && c < cw)
                        v = *reinterpret_cast<const float4*>(X + (int64_t)tr * d + c0 + c);
                    *reinterpret_cast<float4*>(&rows[r][c]) = v;
                }
#pragma unroll
                for (int i = 0; i < (kSeedQpb * CV + 255) / 256; ++i) {
                    const int e = tid + 256 * i;
                    if (e < kSeedQpb * CV) {
                        const int j = e / CV, c = (e % CV) * V;
                        const int64_t qg = (qb0 + j < nq) ? qb0 + j : nq - 1;
                        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                        if (c < cw) v = *reinterpret_cast<const float4*>(Q + qg * d + c0 + c);
                        *reinterpret_cast<float4*>(&qch[j][c]) = v;
                    }
                }
            } else {
                for (int e = tid; e < 64 * CH; e += 256) {
                    const int r = e >> CH_LOG, c = e & (CH - 1);
                    const uint32_t tr = srow[r];
                    rows[r][c] = (tr != kSentinelIdx && c < cw) ? X[(int64_t)tr * d + c0 + c] : T(0);
                }
                for (int e = tid; e < kSeedQpb * CH; e += 256) {
                    const int j = e >> CH_LOG, c = e & (CH - 1);
                    const int64_t qg = (qb0 + j < nq) ? qb0 + j : nq - 1;
                    qch[j][c] = (c < cw) ? Q[qg * d + c0 + c] : T(0);
                }
            }
            __syncthreads();
            // V columns per step, in ascending order (the arm's operation
            // order), then the columns left over one at a time
            auto step = [&](T& acc_j, T qv, T yv) {
                if (ARM == ARM_EUCLID_FMA) {
                    const T diff = qv - yv;
                    acc_j = F::fma_(diff, diff, acc_j);
                } else if (ARM == ARM_EUCLID_MULADD) {
                    const T diff = qv - yv;
                    acc_j = acc_j + diff * diff;
                } else if (ARM == ARM_COS_FOLD) {
                    acc_j = F::fma_(qv, yv, acc_j);
                } else {  // ARM_COS_HOST
                    acc_j = acc_j + qv * yv;
                }
            };
            const int cfull = cw / V * V;
#pragma unroll 2
            for (int c = 0; c < cfull; c += V) {
                T yv[V];
                *reinterpret_cast<float4*>(yv) = *reinterpret_cast<const float4*>(&rows[lane][c]);
#pragma unroll
                for (int j = 0; j < kSeedQpw; ++j) {
                    T qv[V];  // the same address in every lane
                    *reinterpret_cast<float4*>(qv) = *reinterpret_cast<const float4*>(&qch[w * kSeedQpw + j][c]);
#pragma unroll
                    for (int e = 0; e < V; ++e) step(acc[j], qv[e], yv[e]);
                }
            }
            for (int c = cfull; c < cw; ++c) {
                const T yv = rows[lane][c];
#pragma unroll
                for (int j = 0; j < kSeedQpw; ++j) step(acc[j], qch[w * kSeedQpw + j][c], yv);
            }
        }
        const T ya = (on && (ARM == ARM_COS_FOLD || ARM == ARM_COS_HOST)) ? yop[t] : T(0);
#pragma unroll
        for (int j = 0; j < kSeedQpw; ++j) {
            T e = acc[j];
            if (ARM == ARM_COS_FOLD) {
                const T denom = F::sqrt_(qa[j] * ya);
                const T sim = (denom > T(0)) ? e / denom : T(0);
                e = clamp02<T>(T(1) - sim);
            } else if (ARM == ARM_COS_HOST) {
                e = clamp02<T>(T(1) - e * qa[j] * ya);
            }
            uint32_t tj = t;
            if (!on || e != e) {
                e = inf;
                tj = kSentinelIdx;
            }
            // Only the k-th value is kept: a batch with no value below the
            // list's k-th (+inf until k rows are listed) cannot change it.
            T kth = lv[j][0];
#pragma unroll
            for (int b = 1; b < SB; ++b)
                if (((k - 1) >> 6) == b) kth = lv[j][b];
            kth = bcast_f(kth, (k - 1) & 63);
            const uint64_t cand = __builtin_amdgcn_ballot_w64(e < kth);
            if (!cand) continue;
            if (SB == 1 && __builtin_popcountll(cand) <= kSeedInsertMax) {
                // A few rows below the k-th (later batches): each goes into
                // its place in the list, which is sorted by (value, index)
                // across the lanes, instead of sorting the batch and merging.
                // Entries past the k-th may then differ from a full merge's;
                // the k-th value does not.
                uint64_t cm = cand;
                while (cm) {
                    const int l = __builtin_ctzll(cm);
                    cm &= cm - 1;
                    const T ce = bcast_f(e, l);
                    const uint32_t ct = bcast_u(tj, l);
                    if (!(ce < bcast_f(lv[j][0], (k - 1) & 63))) continue;
                    const int p = __builtin_popcountll(
                        __builtin_amdgcn_ballot_w64(pair_less<T>(lv[j][0], li[j][0], ce, ct)));
                    const T uv = __shfl_up(lv[j][0], 1, 64);
                    const uint32_t ui = (uint32_t)__shfl_up((int)li[j][0], 1, 64);
                    if (lane > p) {
                        lv[j][0] = uv;
                        li[j][0] = ui;
                    } else if (lane == p) {
                        lv[j][0] = ce;
                        li[j][0] = ct;
                    }
                }
                continue;
            }
            wave_sort64<T>(e, tj, lane);
            if (SB == 1)
                wave_merge64<T>(lv[j][0], li[j][0], e, tj, lane);
            else
                wave_merge_blocks<T, SB>(lv[j], li[j], e, tj, lane);
        }
    }
#pragma unroll
    for (int j = 0; j < kSeedQpw; ++j) {
        // element k - 1 of the list: block (k - 1) / 64, lane (k - 1) % 64
        T kv = lv[j][0];
#pragma unroll
        for (int b = 1; b < SB; ++b)
            if (((k - 1) >> 6) == b) kv = lv[j][b];
        if (lane == ((k - 1) & 63) && q0 + j < nq) {
            if (sizeof(T) == 4)
                shared_r[q0 + j] = (Bits)__float_as_uint((float)kv);
            else
                shared_r[q0 + j] = (Bits)__double_as_longlong((double)kv);
        }
    }
}

// Output transform: the boundary root of prims/knn.rs:877-883 (Euclidean),
// identity (cosine), or the k-means (label, squared distance) pair with
// argmin_dist_rows' centre-0 seeding (crates/mlrs-kernels/src/kmeans.rs:284-310).
__device__ __forceinline__ void emit_pair(int mode, const float* __restrict__ Q, const float* __restrict__ X,
                                          const float* __restrict__ qsq, const float* __restrict__ xsq, int64_t d,
                                          int k, int64_t qg, int slot, float v, uint32_t ix,
                                          float* __restrict__ out_val, uint32_t* __restrict__ out_idx) {
    const int64_t o = qg * k + slot;
    if (mode == EMIT_KMEANS) {
        // argmin_dist_rows seeds `best` from centre 0 unconditionally, so a NaN
        // distance to centre 0 wins with label 0.  That distance can only be
        // NaN when a norm is non-finite; check those rows exactly.
        const float inf = __builtin_huge_valf();
        if (!(qsq[qg] < inf) || !(xsq[0] < inf)) {
            float e0 = exact_pair<float, ARM_EUCLID_MULADD>(Q + qg * d, X, d, 0.0f, 0.0f);
            if (e0 != e0) {
                v = e0;
                ix = 0;
            }
        }
        out_val[o] = v;
    } else {
        out_val[o] = (mode == EMIT_SQRT) ? __builtin_sqrtf(v) : v;
    }
    out_idx[o] = (ix == kSentinelIdx) ? 0u : ix;
}

}  // namespace mlrs
