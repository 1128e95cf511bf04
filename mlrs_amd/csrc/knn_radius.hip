// radius_neighbors on the device: every index row within `radius` of each
// query row, as the reference's CSR-without-indptr result -- matches of row 0,
// then row 1, ..., each row's in ascending index order, plus a count per row
// (RadiusNeighbors, crates/mlrs-algos/src/neighbors/nearest.rs:564-582).
//
// The values are those of the reference's default arm, the fused host scan
// (crates/mlrs-backend/src/prims/radius_host.rs:239-569): the knn_host lane
// arithmetic (knn_host.rs:693-760) -- Euclidean acc + diff*diff, cosine
// 1 - dot*(1/|q|)*(1/|x|) clamped to [0, 2], Manhattan, Chebyshev as a select,
// Minkowski as a multiply chain or pow -- compared as `v <= th` against the
// threshold in the metric's internal units (NaN never matches), and the
// boundary transform applied to the matches only.
//
// Layout: lanes are index rows, so the 64 rows of a chunk are compared with
// one query row at a time and a wave ballot orders that row's matches -- the
// popcount of the lower lanes' hits is a match's place, the popcount of all
// of them advances the row's cursor.  A wave carries RQ query rows (their
// transposed features are uniform loads) and walks one strip of index rows.
// COUNT fixes each (strip, row) count; a scan turns the counts into output
// positions; FILL recomputes and writes the pre-boundary values; a last pass
// applies the boundary transform to the matches.  FILL checks that every
// strip ends where its count said and never writes at or past the caller's
// capacity.
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

template <typename T> struct RadiusShape;
template <> struct RadiusShape<float> { static constexpr int RQ = 32; };
template <> struct RadiusShape<double> { static constexpr int RQ = 16; };

// qT[g][c][r] = xq[g*RQ + r][c], zero past nq.
template <typename T, int RQ>
__global__ __launch_bounds__(256) void radius_stage_kernel(const T* __restrict__ xq, int64_t nq, int64_t d,
                                                           T* __restrict__ qT, int64_t total) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
        const int64_t r = i % RQ;
        const int64_t c = (i / RQ) % d;
        const int64_t q = (i / ((int64_t)RQ * d)) * RQ + r;
        qT[i] = q < nq ? xq[q * d + c] : T(0);
    }
}

template <typename T, int ARM>
__device__ __forceinline__ T radius_step(T acc, T q, T x, T pexp, int pint) {
    using F = FloatTraits<T>;
    if (ARM == ARM_EUCLID_MULADD) {
        const T diff = q - x;
        return acc + diff * diff;
    } else if (ARM == ARM_MANHATTAN) {
        return acc + F::abs_(q - x);
    } else if (ARM == ARM_CHEBYSHEV) {
        const T v = F::abs_(q - x);
        return (v > acc) ? v : acc;
    } else if (ARM == ARM_MINKOWSKI_INT) {
        const T ad = F::abs_(q - x);
        T r = ad;
#pragma unroll
        for (int i = 1; i < 8; ++i)
            if (i < pint) r = r * ad;
        return acc + r;
    } else if (ARM == ARM_MINKOWSKI_POW) {
        return acc + F::pow_(F::abs_(q - x), pexp);
    } else {  // ARM_COS_HOST: the plain dot product
        return acc + q * x;
    }
}

// qT and the outputs come as their own restrict-qualified arguments: with
// them the compiler knows the match stores cannot touch the query groups and
// keeps the uniform query loads on the scalar unit.
template <typename T, int RQ, int ARM, bool VEC, bool FILL>
__global__ __launch_bounds__(256) void radius_scan_kernel(RadiusArgs<T> a, const T* __restrict__ qT,
                                                          T* __restrict__ out_dist, int32_t* __restrict__ out_idx) {
    constexpr int V = VEC ? 16 / (int)sizeof(T) : 1;
    const int lane = threadIdx.x & 63;
    const int s = (int)blockIdx.y * 4 + (threadIdx.x >> 6);
    if (s >= a.nstrips) return;
    const int64_t g = blockIdx.x;
    const int64_t q0 = g * RQ;
    const int active = (a.nq - q0) < RQ ? (int)(a.nq - q0) : RQ;
    const int64_t t_begin = (int64_t)s * a.strip_len;
    const int64_t t_end = (t_begin + a.strip_len) < a.nt ? t_begin + a.strip_len : a.nt;
    const int64_t d = a.d;
    const T* __restrict__ qg = qT + g * d * RQ;
    const uint64_t below = (1ull << lane) - 1ull;

    // rel[r]: row r's matches so far in this strip (wave-uniform).  FILL:
    // lane r holds row r's first output position for this strip.
    uint32_t rel[RQ];
#pragma unroll
    for (int r = 0; r < RQ; ++r) rel[r] = 0u;
    unsigned long long basev = 0ull;
    if (FILL && lane < active) basev = a.qoff[q0 + lane] + a.cnt[(int64_t)s * a.nq + q0 + lane];

    for (int64_t t0 = t_begin; t0 < t_end; t0 += 64) {
        const int64_t t = t0 + lane;
        const bool valid = t < t_end;
        const int64_t tr = valid ? t : t_end - 1;
        const T* __restrict__ xr = a.x + tr * d;
        T acc[RQ];
#pragma unroll
        for (int r = 0; r < RQ; ++r) acc[r] = T(0);
        for (int64_t c = 0; c < d; c += V) {
            T xv[V];
            if (VEC) {
                if (sizeof(T) == 4) {
                    const float4 v4 = *reinterpret_cast<const float4*>(xr + c);
                    xv[0] = (T)v4.x;
                    xv[V > 1 ? 1 : 0] = (T)v4.y;
                    xv[V > 2 ? 2 : 0] = (T)v4.z;
                    xv[V > 3 ? 3 : 0] = (T)v4.w;
                } else {
                    const double2 v2 = *reinterpret_cast<const double2*>(xr + c);
                    xv[0] = (T)v2.x;
                    xv[V > 1 ? 1 : 0] = (T)v2.y;
                }
            } else {
                xv[0] = xr[c];
            }
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const T* __restrict__ qc = qg + (c + e) * RQ;
#pragma unroll
                for (int r = 0; r < RQ; ++r) acc[r] = radius_step<T, ARM>(acc[r], qc[r], xv[e], a.pexp, a.pint);
            }
        }
        const T xi = (ARM == ARM_COS_HOST) ? a.xinv[tr] : T(0);
#pragma unroll
        for (int r = 0; r < RQ; ++r) {
            if (r < active) {
                T v = acc[r];
                if (ARM == ARM_COS_HOST) v = clamp02<T>(T(1) - v * a.qinv[q0 + r] * xi);
                const bool hit = valid && (v <= a.th);
                const uint64_t m = __ballot(hit);
                if (FILL && m != 0ull) {
                    const unsigned long long b =
                        ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(basev >> 32), r)
                         << 32) |
                        (unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)basev, r);
                    if (hit) {
                        const unsigned long long pos = b + rel[r] + (unsigned long long)__popcll(m & below);
                        if (pos < (unsigned long long)a.capacity) {
                            out_dist[pos] = v;
                            out_idx[pos] = (int32_t)(uint32_t)t;
                        }
                    }
                }
                rel[r] += (uint32_t)__popcll(m);
            }
        }
    }

    // lane r reports row r
    uint32_t mine = 0u;
#pragma unroll
    for (int r = 0; r < RQ; ++r)
        if (lane == r) mine = rel[r];
    if (lane < active) {
        const int64_t q = q0 + lane;
        if (!FILL) {
            a.cnt[(int64_t)s * a.nq + q] = mine;
        } else {
            const unsigned long long want =
                a.qoff[q] + (s + 1 < a.nstrips ? (unsigned long long)a.cnt[(int64_t)(s + 1) * a.nq + q]
                                               : (unsigned long long)a.row_cnt[q]);
            if (basev + mine != want) atomicOr(a.mismatch, 1u);
        }
    }
}

// The boundary transform on the matches: 1 sqrt, 2 pow(v, e).
template <typename T>
__global__ __launch_bounds__(256) void radius_transform_kernel(T* __restrict__ v, int64_t n, int mode, T e) {
    using F = FloatTraits<T>;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        v[i] = mode == 1 ? F::sqrt_(v[i]) : F::pow_(v[i], e);
}

// 256-thread exclusive scan of one u64 per thread; *sum receives the total.
__device__ unsigned long long block_exclusive_scan(unsigned long long v, unsigned long long* sum) {
    __shared__ unsigned long long wave_tot[4];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    unsigned long long inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long u = (unsigned long long)__shfl_up((long long)inc, o, 64);
        if (lane >= o) inc += u;
    }
    if (lane == 63) wave_tot[w] = inc;
    __syncthreads();
    unsigned long long before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (i < w) before += wave_tot[i];
        all += wave_tot[i];
    }
    __syncthreads();
    *sum = all;
    return before + inc - v;
}

// One thread per row: the in-row exclusive prefix over the strips (in place)
// and the row total; one partial sum per 256-row block.
__global__ __launch_bounds__(256) void radius_rows_kernel(uint32_t* __restrict__ cnt, int64_t nq, int nstrips,
                                                          uint32_t* __restrict__ row_cnt,
                                                          unsigned long long* __restrict__ block_sum) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    unsigned long long run = 0;
    if (q < nq) {
        for (int s = 0; s < nstrips; ++s) {
            const uint32_t c = cnt[(int64_t)s * nq + q];
            cnt[(int64_t)s * nq + q] = (uint32_t)run;
            run += c;
        }
        row_cnt[q] = (uint32_t)run;
    }
    unsigned long long tot;
    (void)block_exclusive_scan(run, &tot);
    if (threadIdx.x == 0) block_sum[blockIdx.x] = tot;
}

// One block: exclusive scan of the block sums in place, and the grand total.
__global__ __launch_bounds__(256) void radius_top_kernel(unsigned long long* __restrict__ block_sum, int64_t nb,
                                                         unsigned long long* __restrict__ total) {
    unsigned long long carry = 0;
    for (int64_t b0 = 0; b0 < nb; b0 += 256) {
        const int64_t i = b0 + threadIdx.x;
        const unsigned long long v = i < nb ? block_sum[i] : 0ull;
        unsigned long long tot;
        const unsigned long long ex = block_exclusive_scan(v, &tot);
        if (i < nb) block_sum[i] = carry + ex;
        carry += tot;
    }
    if (threadIdx.x == 0) *total = carry;
}

__global__ __launch_bounds__(256) void radius_qoff_kernel(const uint32_t* __restrict__ row_cnt, int64_t nq,
                                                          const unsigned long long* __restrict__ block_sum,
                                                          unsigned long long* __restrict__ qoff) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const unsigned long long v = q < nq ? (unsigned long long)row_cnt[q] : 0ull;
    unsigned long long tot;
    const unsigned long long ex = block_exclusive_scan(v, &tot);
    if (q < nq) qoff[q] = block_sum[blockIdx.x] + ex;
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) p[i] = v;
}

template <typename T, int RQ, int ARM, bool VEC>
hipError_t launch_scan_arm(const RadiusArgs<T>& a, bool fill, hipStream_t s) {
    const dim3 grid((unsigned)((a.nq + RQ - 1) / RQ), (unsigned)((a.nstrips + 3) / 4));
    if (fill)
        hipLaunchKernelGGL((radius_scan_kernel<T, RQ, ARM, VEC, true>), grid, dim3(256), 0, s, a, a.qT, a.out_dist,
                           a.out_idx);
    else
        hipLaunchKernelGGL((radius_scan_kernel<T, RQ, ARM, VEC, false>), grid, dim3(256), 0, s, a, a.qT, a.out_dist,
                           a.out_idx);
    return hipGetLastError();
}

template <typename T, int RQ, bool VEC>
hipError_t launch_scan_vec(const RadiusArgs<T>& a, int arm, bool fill, hipStream_t s) {
    switch (arm) {
        case ARM_EUCLID_MULADD: return launch_scan_arm<T, RQ, ARM_EUCLID_MULADD, VEC>(a, fill, s);
        case ARM_COS_HOST: return launch_scan_arm<T, RQ, ARM_COS_HOST, VEC>(a, fill, s);
        case ARM_MANHATTAN: return launch_scan_arm<T, RQ, ARM_MANHATTAN, VEC>(a, fill, s);
        case ARM_CHEBYSHEV: return launch_scan_arm<T, RQ, ARM_CHEBYSHEV, VEC>(a, fill, s);
        case ARM_MINKOWSKI_INT: return launch_scan_arm<T, RQ, ARM_MINKOWSKI_INT, VEC>(a, fill, s);
        case ARM_MINKOWSKI_POW: return launch_scan_arm<T, RQ, ARM_MINKOWSKI_POW, VEC>(a, fill, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

template <typename T>
int radius_queries_per_wave() {
    return RadiusShape<T>::RQ;
}

template <typename T>
hipError_t launch_radius_stage(const T* xq, int64_t nq, int64_t d, T* qT, hipStream_t s) {
    constexpr int RQ = RadiusShape<T>::RQ;
    const int64_t total = ((nq + RQ - 1) / RQ) * RQ * d;
    if (total == 0) return hipSuccess;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL((radius_stage_kernel<T, RQ>), dim3((unsigned)blocks), dim3(256), 0, s, xq, nq, d, qT, total);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_radius_scan(const RadiusArgs<T>& a, int arm, bool fill, hipStream_t s) {
    constexpr int RQ = RadiusShape<T>::RQ;
    constexpr int V = 16 / (int)sizeof(T);
    if (a.nq == 0 || a.nstrips == 0) return hipSuccess;
    const bool vec = (a.d % V == 0) && ((reinterpret_cast<uintptr_t>(a.x) & 15u) == 0);
    return vec ? launch_scan_vec<T, RQ, true>(a, arm, fill, s) : launch_scan_vec<T, RQ, false>(a, arm, fill, s);
}

hipError_t launch_radius_offsets(uint32_t* cnt, int64_t nq, int nstrips, uint32_t* row_cnt,
                                 unsigned long long* block_sum, unsigned long long* qoff,
                                 unsigned long long* total, hipStream_t s) {
    const int64_t nb = (nq + 255) / 256;
    if (nb > 0) {
        hipLaunchKernelGGL(radius_rows_kernel, dim3((unsigned)nb), dim3(256), 0, s, cnt, nq, nstrips, row_cnt,
                           block_sum);
    }
    hipLaunchKernelGGL(radius_top_kernel, dim3(1), dim3(256), 0, s, block_sum, nb, total);
    if (nb > 0) hipLaunchKernelGGL(radius_qoff_kernel, dim3((unsigned)nb), dim3(256), 0, s, row_cnt, nq, block_sum, qoff);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_radius_transform(T* v, int64_t n, int mode, T e, hipStream_t s) {
    if (n <= 0 || mode == 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL((radius_transform_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, s, v, n, mode, e);
    return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

template int radius_queries_per_wave<float>();
template int radius_queries_per_wave<double>();
template hipError_t launch_radius_stage<float>(const float*, int64_t, int64_t, float*, hipStream_t);
template hipError_t launch_radius_stage<double>(const double*, int64_t, int64_t, double*, hipStream_t);
template hipError_t launch_radius_scan<float>(const RadiusArgs<float>&, int, bool, hipStream_t);
template hipError_t launch_radius_scan<double>(const RadiusArgs<double>&, int, bool, hipStream_t);
template hipError_t launch_radius_transform<float>(float*, int64_t, int, float, hipStream_t);
template hipError_t launch_radius_transform<double>(double*, int64_t, int, double, hipStream_t);

}  // namespace mlrs
