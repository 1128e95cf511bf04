// Device-side building blocks shared by the kNN kernels (gfx950, wave64).
//
// Everything here is compiled with -ffp-contract=off: each multiply and add
// rounds on its own, and a fused multiply-add appears only where the mlrs
// cpu-backend arithmetic writes one, so the exact distance routines below are
// bit-for-bit the reference's (see the per-routine citations).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
    return va < vb || (va == vb && ia < ib);
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

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ double shfl_xor_f(double v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ uint32_t shfl_xor_u(uint32_t v, int m) {
    return (uint32_t)__shfl_xor((int)v, m, 64);
}
__device__ __forceinline__ float shfl_f(float v, int src) { return __shfl(v, src, 64); }
__device__ __forceinline__ double shfl_f(double v, int src) { return __shfl(v, src, 64); }
__device__ __forceinline__ uint32_t shfl_u(uint32_t v, int src) { return (uint32_t)__shfl((int)v, src, 64); }

// One compare-exchange step with the partner lane^m.  `up` says whether this
// lane's sub-sequence sorts ascending.
template <typename T>
__device__ __forceinline__ void bitonic_step(T& v, uint32_t& ix, int lane, int m, bool up) {
    T ov = shfl_xor_f(v, m);
    uint32_t oi = shfl_xor_u(ix, m);
    bool lower = (lane & m) == 0;
    // The lower lane of an ascending pair keeps the smaller element, the upper
    // lane the larger; a descending pair the reverse.
    bool take = (lower == up) ? pair_less<T>(ov, oi, v, ix) : pair_less<T>(v, ix, ov, oi);
    if (take) {
        v = ov;
        ix = oi;
    }
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
    T rv = shfl_f(v, 63 - lane);
    uint32_t ri = shfl_u(ix, 63 - lane);
    if (pair_less<T>(rv, ri, lv, li)) {
        lv = rv;
        li = ri;
    }
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) bitonic_step<T>(lv, li, lane, m, true);
}

}  // namespace mlrs
