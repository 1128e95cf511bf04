// Exact building blocks: row norms, the tiled exact pairwise-value kernel and
// the per-row (value, index) top-k selection over a materialized matrix.
//
// Together the last two are the engine's generic path -- any d, any k up to
// the row length, any arm, f32 or f64 -- the MI355X counterpart of the
// reference's two-kernel distance_direct -> top_k composition
// (crates/mlrs-algos/src/neighbors/nearest.rs:1117-1343,
// crates/mlrs-backend/src/prims/distance.rs:428-551, prims/topk.rs:62-186).
// The pairwise kernel alone is the pairwise-distance entry point.
#include <algorithm>

#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

// ---------------------------------------------------------------------------
// Row norms (row_sumsq order) + device-side max for the Gram screen bound.
// ---------------------------------------------------------------------------
// 256 rows per block.  Each 32-element (f32) / 16-element (f64) column chunk
// of the block's rows is staged in LDS with coalesced loads (consecutive
// threads read consecutive columns of one row), then each thread continues
// its own row's sum over the chunk in column order -- the row_sumsq order.
// VEC: rows 16-byte aligned with d a multiple of the 16-byte vector; each
// thread then issues all eight of its 16-byte loads of a chunk before the
// barrier, so a block keeps 32 KB in flight.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void row_norms_kernel(const T* __restrict__ x, int64_t n, int64_t d,
                                                        T* __restrict__ sq, T* __restrict__ inv,
                                                        T* __restrict__ neg_inv, NormStats* stats) {
    constexpr int CW = 128 / sizeof(T);  // columns per chunk: one 128-byte segment per row
    constexpr int V = 16 / sizeof(T);    // elements per 16-byte vector
    constexpr int VPR = CW / V;          // vectors per row chunk (8)
    constexpr int RPP = 256 / VPR;       // rows per load pass (32)
    __shared__ T stage[256][CW + 1];
    const int tid = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * 256;
    const int64_t r = r0 + tid;
    const bool valid = r < n;
    T s = T(0);
    for (int64_t c0 = 0; c0 < d; c0 += CW) {
        const int cw = (d - c0) < CW ? (int)(d - c0) : CW;
        if (VEC) {
            const int vr = tid / VPR, vc = tid % VPR;
            T buf[256 / RPP][V];
#pragma unroll
            for (int p = 0; p < 256 / RPP; ++p) {
                const int64_t gr = r0 + vr + RPP * p;
#pragma unroll
                for (int e = 0; e < V; ++e) buf[p][e] = T(0);
                if (gr < n && vc * V < cw) {
                    if (sizeof(T) == 4) {
                        const float4 v = *reinterpret_cast<const float4*>(x + gr * d + c0 + vc * V);
                        buf[p][0] = (T)v.x;
                        buf[p][1] = (T)v.y;
                        if (V > 2) {
                            buf[p][V > 2 ? 2 : 0] = (T)v.z;
                            buf[p][V > 2 ? 3 : 0] = (T)v.w;
                        }
                    } else {
                        const double2 v = *reinterpret_cast<const double2*>(x + gr * d + c0 + vc * V);
                        buf[p][0] = (T)v.x;
                        buf[p][1] = (T)v.y;
                    }
                }
            }
#pragma unroll
            for (int p = 0; p < 256 / RPP; ++p)
#pragma unroll
                for (int e = 0; e < V; ++e) stage[vr + RPP * p][vc * V + e] = buf[p][e];
        } else {
#pragma unroll 4
            for (int m = 0; m < CW; ++m) {
                const int e = tid + 256 * m;  // element of the 256 x CW chunk
                const int rr = e / CW, cc = e % CW;
                const int64_t gr = r0 + rr;
                if (cc < cw && gr < n) stage[rr][cc] = x[gr * d + c0 + cc];
            }
        }
        __syncthreads();
        if (valid) {
            for (int cc = 0; cc < cw; ++cc) {
                T v = stage[tid][cc];
                s = s + v * v;
            }
        }
        __syncthreads();
    }
    if (valid) {
        sq[r] = s;
        T iv = (s > T(0)) ? T(1) / FloatTraits<T>::sqrt_(s) : T(0);
        if (inv) inv[r] = iv;
        if (neg_inv) neg_inv[r] = -iv;
    }
    if (stats) {
        // Max over non-NaN squared norms; non-negative floats order like their bits.
        unsigned long long bits = 0;
        if (valid && !(s != s)) {
            if (sizeof(T) == 4) {
                float f = (float)s;
                bits = (unsigned long long)__float_as_uint(f);
            } else {
                bits = (unsigned long long)__double_as_longlong((double)s);
            }
        }
        // Wave-level max, then the workgroup's in LDS, then at most one
        // atomic per workgroup, skipped when the running max is already as
        // large (the atomics on one word serialise: one per wave cost ~0.15 ms
        // over 1M rows).
        for (int m = 32; m > 0; m >>= 1) {
            unsigned long long o = (unsigned long long)__shfl_xor((long long)bits, m, 64);
            bits = o > bits ? o : bits;
        }
        __shared__ unsigned long long wmax[4];
        if ((tid & 63) == 0) wmax[tid >> 6] = bits;
        __syncthreads();
        if (tid == 0) {
            unsigned long long b = wmax[0];
#pragma unroll
            for (int i = 1; i < 4; ++i) b = wmax[i] > b ? wmax[i] : b;
            if (b > __hip_atomic_load(&stats->xsq_max_bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                atomicMax(&stats->xsq_max_bits, b);
        }
    }
}

template <typename T>
__global__ void stats_reset_kernel(NormStats* stats) {
    if (threadIdx.x == 0) stats->xsq_max_bits = 0ull;
}

template <typename T>
__global__ void stats_finalize_kernel(NormStats* stats) {
    if (threadIdx.x == 0) {
        unsigned long long b = stats->xsq_max_bits;
        if (sizeof(T) == 4) {
            float f = __uint_as_float((uint32_t)b);
            stats->xsq_max = f;
            stats->xsq_max64 = (double)f;
        } else {
            double v = __longlong_as_double((long long)b);
            stats->xsq_max64 = v;
            stats->xsq_max = (float)v;
        }
    }
}

// ---------------------------------------------------------------------------
// Tiled exact pairwise values.  A 16x16 thread block computes a 64x64 output
// tile, 4x4 per thread; 16-column chunks of both operands are staged in LDS.
// Each pair still accumulates over ascending columns one step at a time, so
// the value is the arm's exact reference value.
// ---------------------------------------------------------------------------
constexpr int PT = 64;   // output tile edge
constexpr int PC = 16;   // staged columns per chunk

// `root`: 0 none, 1 sqrt, 2 pow(v, root_exp) on the stored value; `pexp` /
// `pint` are the Minkowski exponent of the pow and integer arms.
template <typename T, int ARM>
__global__ __launch_bounds__(256) void pairwise_tile_kernel(const T* __restrict__ x, int64_t nx,
                                                            const T* __restrict__ y, int64_t ny,
                                                            int64_t d, const T* __restrict__ xa,
                                                            const T* __restrict__ ya, T* __restrict__ out,
                                                            int64_t ldo, int root, T pexp, int pint, T root_exp) {
    using F = FloatTraits<T>;
    __shared__ T xs[PC][PT + 1];
    __shared__ T ys[PC][PT + 1];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int64_t i0 = (int64_t)blockIdx.y * PT, j0 = (int64_t)blockIdx.x * PT;
    T acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = T(0);

    for (int64_t c0 = 0; c0 < d; c0 += PC) {
        // Stage x[i0..i0+64)[c0..c0+16) and y[j0..)[c0..) transposed.
        for (int e = threadIdx.x; e < PT * PC; e += 256) {
            int r = e / PC, c = e % PC;
            int64_t gi = i0 + r, gj = j0 + r, gc = c0 + c;
            xs[c][r] = (gi < nx && gc < d) ? x[gi * d + gc] : T(0);
            ys[c][r] = (gj < ny && gc < d) ? y[gj * d + gc] : T(0);
        }
        __syncthreads();
        int cn = (d - c0) < PC ? (int)(d - c0) : PC;
        for (int c = 0; c < cn; ++c) {
            T xv[4], yv[4];
#pragma unroll
            for (int a = 0; a < 4; ++a) xv[a] = xs[c][ty + 16 * a];
#pragma unroll
            for (int b = 0; b < 4; ++b) yv[b] = ys[c][tx + 16 * b];
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    if (ARM == ARM_EUCLID_FMA) {
                        T diff = xv[a] - yv[b];
                        acc[a][b] = F::fma_(diff, diff, acc[a][b]);
                    } else if (ARM == ARM_EUCLID_MULADD) {
                        T diff = xv[a] - yv[b];
                        acc[a][b] = acc[a][b] + diff * diff;
                    } else if (ARM == ARM_COS_FOLD) {
                        acc[a][b] = F::fma_(xv[a], yv[b], acc[a][b]);
                    } else if (ARM == ARM_MANHATTAN) {
                        acc[a][b] = acc[a][b] + F::abs_(xv[a] - yv[b]);
                    } else if (ARM == ARM_CHEBYSHEV) {
                        const T v = F::abs_(xv[a] - yv[b]);
                        acc[a][b] = (v > acc[a][b]) ? v : acc[a][b];
                    } else if (ARM == ARM_MINKOWSKI_INT) {
                        const T ad = F::abs_(xv[a] - yv[b]);
                        T r = ad;
                        for (int i = 1; i < pint; ++i) r = r * ad;
                        acc[a][b] = acc[a][b] + r;
                    } else if (ARM == ARM_MINKOWSKI_POW) {
                        acc[a][b] = acc[a][b] + F::pow_(F::abs_(xv[a] - yv[b]), pexp);
                    } else {
                        acc[a][b] = acc[a][b] + xv[a] * yv[b];
                    }
                }
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        int64_t gi = i0 + ty + 16 * a;
        if (gi >= nx) continue;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            int64_t gj = j0 + tx + 16 * b;
            if (gj >= ny) continue;
            T v = acc[a][b];
            if (ARM == ARM_COS_FOLD || ARM == ARM_COS_PAIRWISE) {
                T denom = F::sqrt_(xa[gi] * ya[gj]);
                T sim = T(0);
                if (denom > T(0)) sim = v / denom;
                v = clamp02<T>(T(1) - sim);
            } else if (ARM == ARM_COS_HOST) {
                v = clamp02<T>(T(1) - v * xa[gi] * ya[gj]);
            } else if (root == 1) {
                v = F::sqrt_(v);
            } else if (root == 2) {
                v = F::pow_(v, root_exp);
            }
            out[gi * ldo + gj] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Per-row top-k selection by radix select over order-preserving keys.
// ---------------------------------------------------------------------------
template <typename T> struct KeyOf;
template <> struct KeyOf<float> {
    typedef uint32_t K;
    static constexpr int BITS = 32;
    static __device__ __forceinline__ K key(float v) {
        if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal: one key
        uint32_t b = __float_as_uint(v);
        return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    }
    static __device__ __forceinline__ float val(K k) {
        uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
        return __uint_as_float(b);
    }
};
template <> struct KeyOf<double> {
    typedef unsigned long long K;
    static constexpr int BITS = 64;
    static __device__ __forceinline__ K key(double v) {
        if (v == 0.0) v = 0.0;
        unsigned long long b = (unsigned long long)__double_as_longlong(v);
        return (b & 0x8000000000000000ull) ? ~b : (b | 0x8000000000000000ull);
    }
    static __device__ __forceinline__ double val(K k) {
        unsigned long long b = (k & 0x8000000000000000ull) ? (k & 0x7FFFFFFFFFFFFFFFull) : ~k;
        return __longlong_as_double((long long)b);
    }
};

// LDS-resident selection serves k up to SEL_MAXK; larger k collects into the
// output rows and sorts there (select_collect_kernel and below).
constexpr int SEL_MAXK = 256;

// Loads in flight per thread in the row scans below.
constexpr int kRadixBatch = 8;

// Shared state of one row's radix select (one 256-thread workgroup per row).
template <typename K>
struct RadixShared {
    uint32_t hist[256];
    uint32_t cnt_less, cnt_eq, nvalid;
    uint32_t wave_less[4], wave_eq[4];
    K prefix;
    uint32_t want;
};

// Number of admissible (non-NaN) values of the row.
template <typename T>
__device__ uint32_t row_count_valid(const T* __restrict__ dr, int64_t cols, RadixShared<typename KeyOf<T>::K>& sh) {
    const int tid = threadIdx.x;
    if (tid == 0) sh.nvalid = 0;
    __syncthreads();
    uint32_t local = 0;
    // kRadixBatch loads in flight per thread (a long row read by one
    // workgroup is bound by the load latency otherwise)
    for (int64_t c0 = 0; c0 < cols; c0 += 256 * kRadixBatch) {
        T v[kRadixBatch];
#pragma unroll
        for (int u = 0; u < kRadixBatch; ++u) {
            const int64_t c = c0 + u * 256 + tid;
            v[u] = (c < cols) ? dr[c] : T(0) / T(0);
        }
#pragma unroll
        for (int u = 0; u < kRadixBatch; ++u) local += (v[u] == v[u]) ? 1u : 0u;
    }
    atomicAdd(&sh.nvalid, local);
    __syncthreads();
    return sh.nvalid;
}

// Radix select, 8 bits per pass from the top: `prefix` becomes the kk-th
// smallest key of the row (NaN excluded) and `want` how many of its copies
// belong to the kk smallest (the lowest-index ones).
template <typename T>
__device__ void row_radix_kth(const T* __restrict__ dr, int64_t cols, uint32_t kk,
                              RadixShared<typename KeyOf<T>::K>& sh, typename KeyOf<T>::K& prefix,
                              uint32_t& want) {
    typedef typename KeyOf<T>::K K;
    const int tid = threadIdx.x;
    K pmask = 0;
    prefix = 0;
    want = kk;
    for (int shift = KeyOf<T>::BITS - 8; shift >= 0; shift -= 8) {
        sh.hist[tid] = 0;
        __syncthreads();
        for (int64_t c0 = 0; c0 < cols; c0 += 256 * kRadixBatch) {
            T v[kRadixBatch];
#pragma unroll
            for (int u = 0; u < kRadixBatch; ++u) {
                const int64_t c = c0 + u * 256 + tid;
                v[u] = (c < cols) ? dr[c] : T(0) / T(0);  // past the row: NaN, never counted
            }
#pragma unroll
            for (int u = 0; u < kRadixBatch; ++u) {
                if (v[u] != v[u]) continue;
                const K key = KeyOf<T>::key(v[u]);
                if ((key & pmask) == prefix) atomicAdd(&sh.hist[(uint32_t)(key >> shift) & 255u], 1u);
            }
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t w = want;
            int b = 0;
            for (; b < 255; ++b) {
                if (sh.hist[b] >= w) break;
                w -= sh.hist[b];
            }
            sh.prefix = prefix | ((K)b << shift);
            sh.want = w;
        }
        __syncthreads();
        prefix = sh.prefix;
        want = sh.want;
        pmask |= ((K)255 << shift);
        __syncthreads();
    }
}

// The kk smallest pairs of the row, in ascending column order within each
// class: every key below `prefix` goes to slot [0, kk - want) and the first
// `want` copies of `prefix` to [kk - want, kk).  put(slot, key, column).
template <typename T, typename Put>
__device__ void row_collect(const T* __restrict__ dr, int64_t cols, uint32_t kk, typename KeyOf<T>::K prefix,
                            uint32_t want, RadixShared<typename KeyOf<T>::K>& sh, Put put) {
    typedef typename KeyOf<T>::K K;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const uint32_t n_less = kk - want;
    if (tid == 0) {
        sh.cnt_less = 0;
        sh.cnt_eq = 0;
    }
    __syncthreads();
    // kRadixBatch chunks' values loaded together, then compacted in order
    for (int64_t b0 = 0; b0 < cols; b0 += 256 * kRadixBatch) {
        T vv[kRadixBatch];
#pragma unroll
        for (int u = 0; u < kRadixBatch; ++u) {
            const int64_t c = b0 + (int64_t)u * 256 + tid;
            vv[u] = (c < cols) ? dr[c] : T(0);
        }
#pragma unroll
        for (int u = 0; u < kRadixBatch; ++u) {
            const int64_t base = b0 + (int64_t)u * 256;
            if (base >= cols) break;  // uniform
            const int64_t c = base + tid;
            bool is_less = false, is_eq = false;
            K key = 0;
            if (c < cols) {
                const T v = vv[u];
                if (v == v) {
                    key = KeyOf<T>::key(v);
                    is_less = key < prefix;
                    is_eq = key == prefix;
                }
            }
            const uint64_t bl = __builtin_amdgcn_ballot_w64(is_less);
            const uint64_t be = __builtin_amdgcn_ballot_w64(is_eq);
            if (lane == 0) {
                sh.wave_less[wv] = (uint32_t)__builtin_popcountll(bl);
                sh.wave_eq[wv] = (uint32_t)__builtin_popcountll(be);
            }
            __syncthreads();
            uint32_t before_l = sh.cnt_less, before_e = sh.cnt_eq;
            for (int w2 = 0; w2 < wv; ++w2) {
                before_l += sh.wave_less[w2];
                before_e += sh.wave_eq[w2];
            }
            if (is_less) {
                const uint32_t r = before_l + (uint32_t)__builtin_popcountll(bl & below);
                if (r < n_less) put(r, key, (uint32_t)c);  // always true: kk - want keys lie below prefix
            }
            if (is_eq) {
                const uint32_t r = before_e + (uint32_t)__builtin_popcountll(be & below);
                if (r < want) put(n_less + r, key, (uint32_t)c);
            }
            __syncthreads();
            if (tid == 0) {
                sh.cnt_less += sh.wave_less[0] + sh.wave_less[1] + sh.wave_less[2] + sh.wave_less[3];
                sh.cnt_eq += sh.wave_eq[0] + sh.wave_eq[1] + sh.wave_eq[2] + sh.wave_eq[3];
            }
            __syncthreads();
        }
    }
}

// k <= SEL_MAXK: the kk pairs are collected and bitonic-sorted in LDS.
template <typename T>
__global__ __launch_bounds__(256) void select_rows_kernel(const T* __restrict__ dist, int64_t rows,
                                                          int64_t cols, int64_t ld, int k, int mode,
                                                          T* __restrict__ out_val,
                                                          uint32_t* __restrict__ out_idx) {
    typedef typename KeyOf<T>::K K;
    __shared__ RadixShared<K> sh;
    __shared__ K skey[SEL_MAXK];
    __shared__ uint32_t sidx[SEL_MAXK];

    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const T* dr = dist + row * ld;
    const int tid = threadIdx.x;

    const uint32_t nvalid = row_count_valid<T>(dr, cols, sh);
    const int kk = (int)((uint32_t)k < nvalid ? (uint32_t)k : nvalid);

    if (kk > 0) {
        K prefix;
        uint32_t want;
        row_radix_kth<T>(dr, cols, (uint32_t)kk, sh, prefix, want);
        row_collect<T>(dr, cols, (uint32_t)kk, prefix, want, sh, [&](uint32_t slot, K key, uint32_t c) {
            skey[slot] = key;
            sidx[slot] = c;
        });
        // bitonic sort of the kk kept pairs by (key, index)
        int n2 = 1;
        while (n2 < kk) n2 <<= 1;
        for (int e = kk + tid; e < n2; e += 256) {
            skey[e] = ~(K)0;
            sidx[e] = kSentinelIdx;
        }
        __syncthreads();
        for (int size = 2; size <= n2; size <<= 1) {
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                for (int e = tid; e < n2; e += 256) {
                    int p = e ^ stride;
                    if (p > e) {
                        bool up = (e & size) == 0;
                        K ka = skey[e], kb = skey[p];
                        uint32_t ia = sidx[e], ib = sidx[p];
                        bool a_gt = (ka > kb) || (ka == kb && ia > ib);
                        if (a_gt == up) {
                            skey[e] = kb;
                            skey[p] = ka;
                            sidx[e] = ib;
                            sidx[p] = ia;
                        }
                    }
                }
                __syncthreads();
            }
        }
    }
    // emit (value recovered from the key: exact, since the key map is a bijection)
    for (int s = tid; s < k; s += 256) {
        T v;
        uint32_t ix;
        if (s < kk) {
            v = KeyOf<T>::val(skey[s]);
            ix = sidx[s];
        } else {
            v = FloatTraits<T>::inf();
            ix = 0;  // sentinel index emitted as 0 (crates/mlrs-kernels/src/knn.rs:2931-2961)
        }
        if (mode == EMIT_SQRT) v = FloatTraits<T>::sqrt_(v);
        out_val[row * k + s] = v;
        out_idx[row * k + s] = ix;
    }
}

// ---------------------------------------------------------------------------
// k > SEL_MAXK (any k up to the row length, the reference's top_k contract,
// crates/mlrs-backend/src/prims/topk.rs:208-212): the same radix select, the
// kk pairs collected straight into the row's output slots (keys in the value
// slots, which have the key's width), then sorted by (key, index) -- in LDS
// when kk fits one chunk, else chunk sorts in LDS followed by merge passes
// through a scratch copy -- and finally mapped back to values.  (key, index)
// pairs are distinct, so every step is a total order with no ties.
// ---------------------------------------------------------------------------
template <typename T> struct SortChunk;
template <> struct SortChunk<float> { static constexpr int N = 8192; };   // 64 KB of (key, index)
template <> struct SortChunk<double> { static constexpr int N = 4096; };  // 48 KB

template <typename K>
__device__ __forceinline__ bool pair_gt(K ka, uint32_t ia, K kb, uint32_t ib) {
    return (ka > kb) || (ka == kb && ia > ib);
}

// One workgroup per row: kk = min(k, admissible values) pairs into
// okey/oidx[row*k + 0..kk), and nk[row] = kk.
template <typename T>
__global__ __launch_bounds__(256) void select_collect_kernel(const T* __restrict__ dist, int64_t rows,
                                                             int64_t cols, int64_t ld, int k,
                                                             typename KeyOf<T>::K* __restrict__ okey,
                                                             uint32_t* __restrict__ oidx, uint32_t* __restrict__ nk) {
    typedef typename KeyOf<T>::K K;
    __shared__ RadixShared<K> sh;
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const T* dr = dist + row * ld;
    const uint32_t nvalid = row_count_valid<T>(dr, cols, sh);
    const uint32_t kk = (uint32_t)k < nvalid ? (uint32_t)k : nvalid;
    if (threadIdx.x == 0) nk[row] = kk;
    if (kk == 0) return;
    K prefix;
    uint32_t want;
    row_radix_kth<T>(dr, cols, kk, sh, prefix, want);
    K* rk = okey + row * (int64_t)k;
    uint32_t* ri = oidx + row * (int64_t)k;
    row_collect<T>(dr, cols, kk, prefix, want, sh, [&](uint32_t slot, K key, uint32_t c) {
        rk[slot] = key;
        ri[slot] = c;
    });
}

// Sort chunk `ch` ([ch*N, min((ch+1)*N, kk)) of row r) in LDS, in place.
// Workgroup b = r * nchunks + ch.
template <typename T>
__global__ __launch_bounds__(512) void select_sort_chunk_kernel(typename KeyOf<T>::K* __restrict__ key,
                                                                uint32_t* __restrict__ idx,
                                                                const uint32_t* __restrict__ nk, int64_t rows,
                                                                int k, int nchunks) {
    typedef typename KeyOf<T>::K K;
    constexpr int N = SortChunk<T>::N;
    __shared__ K sk[N];
    __shared__ uint32_t si[N];
    const int64_t r = (int64_t)blockIdx.x / nchunks;
    const int ch = (int)((int64_t)blockIdx.x - r * nchunks);
    if (r >= rows) return;
    const int64_t kk = nk[r];
    const int64_t lo = (int64_t)ch * N;
    if (lo >= kk) return;
    const int n = (int)((kk - lo) < N ? (kk - lo) : N);
    int n2 = 1;
    while (n2 < n) n2 <<= 1;
    K* rk = key + r * (int64_t)k + lo;
    uint32_t* ri = idx + r * (int64_t)k + lo;
    const int tid = threadIdx.x;
    for (int e = tid; e < n2; e += 512) {
        sk[e] = e < n ? rk[e] : ~(K)0;
        si[e] = e < n ? ri[e] : kSentinelIdx;
    }
    __syncthreads();
    for (int size = 2; size <= n2; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int e = tid; e < n2; e += 512) {
                const int p = e ^ stride;
                if (p > e) {
                    const bool up = (e & size) == 0;
                    const K ka = sk[e], kb = sk[p];
                    const uint32_t ia = si[e], ib = si[p];
                    if (pair_gt<K>(ka, ia, kb, ib) == up) {
                        sk[e] = kb;
                        sk[p] = ka;
                        si[e] = ib;
                        si[p] = ia;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (int e = tid; e < n; e += 512) {
        rk[e] = sk[e];
        ri[e] = si[e];
    }
}

// One merge pass: sorted runs of length L within [0, kk) of every row are
// merged pairwise into runs of 2L (src -> dst).  An element's place is its
// rank in its own run plus the number of smaller elements of the partner run
// (binary search).  Workgroup b covers elements [c*256, c*256+256) of row
// b / nblk, c = b % nblk.
template <typename K>
__global__ __launch_bounds__(256) void select_merge_kernel(const K* __restrict__ skey, const uint32_t* __restrict__ sidx,
                                                           K* __restrict__ dkey, uint32_t* __restrict__ didx,
                                                           const uint32_t* __restrict__ nk, int64_t rows, int k,
                                                           int64_t L, int64_t nblk) {
    const int64_t r = (int64_t)blockIdx.x / nblk;
    const int64_t c = (int64_t)blockIdx.x - r * nblk;
    if (r >= rows) return;
    const int64_t kk = nk[r];
    const int64_t i = c * 256 + threadIdx.x;
    if (i >= kk) return;
    const K* rk = skey + r * (int64_t)k;
    const uint32_t* ri = sidx + r * (int64_t)k;
    const K ek = rk[i];
    const uint32_t ei = ri[i];
    const int64_t s = (i / (2 * L)) * (2 * L);
    const bool in_a = i < s + L;
    // the partner run [plo, phi)
    const int64_t plo = in_a ? s + L : s;
    int64_t phi = in_a ? s + 2 * L : s + L;
    if (phi > kk) phi = kk;
    int64_t lo = plo, hi = phi > plo ? phi : plo;  // first partner element greater than (ek, ei)
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (pair_gt<K>(ek, ei, rk[mid], ri[mid])) lo = mid + 1;
        else hi = mid;
    }
    const int64_t own = in_a ? i - s : i - s - L;
    const int64_t pos = s + own + (lo - plo);
    dkey[r * (int64_t)k + pos] = ek;
    didx[r * (int64_t)k + pos] = ei;
}

// Keys back to values with the output transform; slots past kk get (+inf, 0).
template <typename T>
__global__ __launch_bounds__(256) void select_finish_kernel(const typename KeyOf<T>::K* __restrict__ skey,
                                                            const uint32_t* __restrict__ sidx,
                                                            const uint32_t* __restrict__ nk, int64_t rows, int k,
                                                            int mode, int64_t nblk, T* __restrict__ out_val,
                                                            uint32_t* __restrict__ out_idx) {
    const int64_t r = (int64_t)blockIdx.x / nblk;
    const int64_t c = (int64_t)blockIdx.x - r * nblk;
    if (r >= rows) return;
    const int64_t i = c * 256 + threadIdx.x;
    if (i >= k) return;
    const int64_t o = r * (int64_t)k + i;
    T v;
    uint32_t ix;
    if (i < (int64_t)nk[r]) {
        v = KeyOf<T>::val(skey[o]);
        ix = sidx[o];
    } else {
        v = FloatTraits<T>::inf();
        ix = 0;
    }
    if (mode == EMIT_SQRT) v = FloatTraits<T>::sqrt_(v);
    out_val[o] = v;
    out_idx[o] = ix;
}

// argmin_dist_rows (crates/mlrs-kernels/src/kmeans.rs:284-310) over a
// materialized rows x cols block: best seeded from column 0, strict `<`
// afterwards (so a NaN in column 0 wins and NaN elsewhere never does).
template <typename T>
__global__ void argmin_rows_kernel(const T* __restrict__ dist, int64_t rows, int64_t cols, int64_t ld,
                                   uint32_t* __restrict__ labels, T* __restrict__ best_out) {
    int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const T* dr = dist + r * ld;
    T best = dr[0];
    uint32_t bc = 0;
    for (int64_t c = 1; c < cols; ++c) {
        T v = dr[c];
        if (v < best) {
            best = v;
            bc = (uint32_t)c;
        }
    }
    labels[r] = bc;
    best_out[r] = best;
}

// k <= 64: one wave per row, two streaming passes.  Pass 1: each lane keeps
// the smallest (value, column) pair of its strided share of the row; the
// k-th smallest of those 64 pairs is a bound B on the row's k-th pair (k
// distinct pairs are <= B).  Pass 2 re-reads the row (L2-resident) and
// compacts the pairs <= B into LDS (ballot + popcount, columns ascending),
// sorting and merging them into the row's list 64 at a time -- typically
// once.  NaN is never admitted; +inf is a value like any other; -0 is
// emitted as +0 (as the radix kernel's key map does).  The same
// (value, index) top-k as select_rows_kernel.
template <typename T>
__global__ __launch_bounds__(256) void select_small_kernel(const T* __restrict__ dist, int64_t rows, int64_t cols,
                                                           int64_t ld, int k, int mode, T* __restrict__ out_val,
                                                           uint32_t* __restrict__ out_idx) {
    constexpr int U = 8;
    __shared__ T cv[4][128];
    __shared__ uint32_t ci[4][128];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * 4 + wv;
    if (row >= rows) return;
    const T* __restrict__ dr = dist + row * ld;
    const T inf = FloatTraits<T>::inf();
    const uint64_t below = (1ull << lane) - 1ull;

    // pass 1: per-lane smallest pair
    T mv = inf;
    uint32_t mi = kSentinelIdx;
    for (int64_t base = 0; base < cols; base += 64 * U) {
        T vv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c = base + 64 * u + lane;
            vv[u] = (c < cols) ? dr[c] : inf;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c = base + 64 * u + lane;
            const bool take = (c < cols) && pair_less<T>(vv[u], (uint32_t)c, mv, mi);
            mv = take ? vv[u] : mv;
            mi = take ? (uint32_t)c : mi;
        }
    }
    wave_sort64<T>(mv, mi, lane);
    const T bv = bcast_f(mv, k - 1);
    const uint32_t bi = bcast_u(mi, k - 1);

    // pass 2: the pairs <= (bv, bi), compacted and merged 64 at a time
    T lv = inf;
    uint32_t li = kSentinelIdx;
    uint32_t nc = 0;
    auto merge_batch = [&](uint32_t count) {
        T e = ((uint32_t)lane < count) ? cv[wv][lane] : inf;
        uint32_t t = ((uint32_t)lane < count) ? ci[wv][lane] : kSentinelIdx;
        wave_sort64<T>(e, t, lane);
        wave_merge64<T>(lv, li, e, t, lane);
    };
    for (int64_t base = 0; base < cols; base += 64 * U) {
        T vv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c = base + 64 * u + lane;
            vv[u] = (c < cols) ? dr[c] : inf;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c = base + 64 * u + lane;
            const T v = vv[u];
            const bool in = (c < cols) && !pair_less<T>(bv, bi, v, (uint32_t)c) && (v == v);
            const uint64_t bal = __builtin_amdgcn_ballot_w64(in);
            if (bal) {
                const uint32_t pos = nc + (uint32_t)__builtin_popcountll(bal & below);
                if (in) {
                    cv[wv][pos] = v;
                    ci[wv][pos] = (uint32_t)c;
                }
                nc += (uint32_t)__builtin_popcountll(bal);
                if (nc >= 64) {
                    merge_batch(64);
                    const uint32_t rest = nc - 64;
                    const T mvv = ((uint32_t)lane < rest) ? cv[wv][64 + lane] : inf;
                    const uint32_t mii = ((uint32_t)lane < rest) ? ci[wv][64 + lane] : 0u;
                    if ((uint32_t)lane < rest) {
                        cv[wv][lane] = mvv;
                        ci[wv][lane] = mii;
                    }
                    nc = rest;
                }
            }
        }
    }
    if (nc > 0) merge_batch(nc);
    if (lane < k) {
        T v = lv + T(0);  // -0 -> +0
        const uint32_t ix = (li == kSentinelIdx) ? 0u : li;
        if (li == kSentinelIdx) v = inf;
        if (mode == EMIT_SQRT) v = FloatTraits<T>::sqrt_(v);
        out_val[row * k + lane] = v;
        out_idx[row * k + lane] = ix;
    }
}

}  // namespace

template <typename T>
hipError_t launch_argmin_rows(const T* dist, int64_t rows, int64_t cols, int64_t ld, uint32_t* labels,
                              T* best, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL((argmin_rows_kernel<T>), dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s,
                       dist, rows, cols, ld, labels, best);
    return hipGetLastError();
}
template hipError_t launch_argmin_rows<float>(const float*, int64_t, int64_t, int64_t, uint32_t*, float*,
                                              hipStream_t);
template hipError_t launch_argmin_rows<double>(const double*, int64_t, int64_t, int64_t, uint32_t*,
                                               double*, hipStream_t);

template <typename T>
hipError_t launch_row_norms(const T* x, int64_t n, int64_t d, T* sq, T* inv, T* neg_inv,
                            NormStats* stats, hipStream_t s) {
    if (stats) hipLaunchKernelGGL((stats_reset_kernel<T>), dim3(1), dim3(64), 0, s, stats);
    if (n > 0) {
        unsigned blocks = (unsigned)((n + 255) / 256);
        const int vec = 16 / (int)sizeof(T);
        if (d % vec == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0)
            hipLaunchKernelGGL((row_norms_kernel<T, true>), dim3(blocks), dim3(256), 0, s, x, n, d, sq, inv,
                               neg_inv, stats);
        else
            hipLaunchKernelGGL((row_norms_kernel<T, false>), dim3(blocks), dim3(256), 0, s, x, n, d, sq, inv,
                               neg_inv, stats);
    }
    if (stats) hipLaunchKernelGGL((stats_finalize_kernel<T>), dim3(1), dim3(64), 0, s, stats);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_pairwise_tile(const T* x, int64_t nx, const T* y, int64_t ny, int64_t d, int arm,
                                const T* xa, const T* ya, T* out, int64_t ldo, int root, hipStream_t s,
                                T pexp, int pint, T root_exp) {
    if (nx == 0 || ny == 0) return hipSuccess;
    dim3 grid((unsigned)((ny + PT - 1) / PT), (unsigned)((nx + PT - 1) / PT));
#define MLRS_PT_CASE(A)                                                                                   \
    case A:                                                                                               \
        hipLaunchKernelGGL((pairwise_tile_kernel<T, A>), grid, dim3(256), 0, s, x, nx, y, ny, d, xa, ya, out, \
                           ldo, root, pexp, pint, root_exp);                                              \
        break;
    switch (arm) {
        MLRS_PT_CASE(ARM_EUCLID_FMA)
        MLRS_PT_CASE(ARM_EUCLID_MULADD)
        MLRS_PT_CASE(ARM_COS_FOLD)
        MLRS_PT_CASE(ARM_COS_HOST)
        MLRS_PT_CASE(ARM_COS_PAIRWISE)
        MLRS_PT_CASE(ARM_MANHATTAN)
        MLRS_PT_CASE(ARM_CHEBYSHEV)
        MLRS_PT_CASE(ARM_MINKOWSKI_INT)
        MLRS_PT_CASE(ARM_MINKOWSKI_POW)
    default:
        return hipErrorInvalidValue;
    }
#undef MLRS_PT_CASE
    return hipGetLastError();
}

// out[i] = pow(out[i], e): the Minkowski boundary root over the n emitted
// values (powf_elem, crates/mlrs-kernels/src/elementwise.rs:139-152).
template <typename T>
__global__ void pow_inplace_kernel(T* __restrict__ v, int64_t n, T e) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) v[i] = FloatTraits<T>::pow_(v[i], e);
}

// copy_elem (crates/mlrs-kernels/src/elementwise.rs:71-125): dst = src.
// 16-byte vectors when both pointers are 16-byte aligned, each thread moving
// four of them per pass; the remainder (fewer than 16 bytes) and unaligned
// buffers go element by element.
__global__ __launch_bounds__(256) void copy_vec16_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                         int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * 1024;
    for (int64_t b = (int64_t)blockIdx.x * 1024 + threadIdx.x; b < n16; b += stride) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (b + 256 * u < n16) v[u] = src[b + 256 * u];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (b + 256 * u < n16) dst[b + 256 * u] = v[u];
    }
}

template <typename T>
__global__ __launch_bounds__(256) void copy_elems_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

template <typename T>
hipError_t launch_device_copy(const T* src, T* dst, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int64_t done = 0;
    if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0) {
        const int64_t n16 = (n * (int64_t)sizeof(T)) / 16;
        if (n16 > 0) {
            const int64_t blocks = std::min<int64_t>((n16 + 1023) / 1024, 8192);
            hipLaunchKernelGGL(copy_vec16_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                               reinterpret_cast<const uint4*>(src), reinterpret_cast<uint4*>(dst), n16);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            done = n16 * 16 / (int64_t)sizeof(T);
        }
    }
    if (done < n) {
        const int64_t rest = n - done;
        const int64_t blocks = std::min<int64_t>((rest + 255) / 256, 8192);
        hipLaunchKernelGGL((copy_elems_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, s, src + done, dst + done,
                           rest);
        return hipGetLastError();
    }
    return hipSuccess;
}
template hipError_t launch_device_copy<float>(const float*, float*, int64_t, hipStream_t);
template hipError_t launch_device_copy<double>(const double*, double*, int64_t, hipStream_t);

template <typename T>
hipError_t launch_pow_inplace(T* v, int64_t n, T e, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL((pow_inplace_kernel<T>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, v, n, e);
    return hipGetLastError();
}

size_t select_rows_scratch_bytes(int64_t rows, int k, int elem_bytes) {
    if (k <= SEL_MAXK || rows <= 0) return 0;
    const int chunk = elem_bytes == 4 ? SortChunk<float>::N : SortChunk<double>::N;
    size_t b = ((size_t)rows * 4 + 255) & ~(size_t)255;
    if (k > chunk) {
        b += (((size_t)rows * k * elem_bytes + 255) & ~(size_t)255);
        b += (((size_t)rows * k * 4 + 255) & ~(size_t)255);
    }
    return b;
}

template <typename T>
hipError_t launch_select_rows(const T* dist, int64_t rows, int64_t cols, int64_t ld, int k, int mode,
                              T* out_val, uint32_t* out_idx, void* scratch, hipStream_t s) {
    typedef typename KeyOf<T>::K K;
    if (rows == 0) return hipSuccess;
    if (k < 1) return hipErrorInvalidValue;
    if (k <= 64) {
        hipLaunchKernelGGL((select_small_kernel<T>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, dist, rows,
                           cols, ld, k, mode, out_val, out_idx);
        return hipGetLastError();
    }
    if (k <= SEL_MAXK) {
        hipLaunchKernelGGL((select_rows_kernel<T>), dim3((unsigned)rows), dim3(256), 0, s, dist, rows, cols,
                           ld, k, mode, out_val, out_idx);
        return hipGetLastError();
    }
    // k > SEL_MAXK: collect into the outputs (keys in the value slots), sort, finish
    if (!scratch) return hipErrorInvalidValue;
    constexpr int N = SortChunk<T>::N;
    char* sp = static_cast<char*>(scratch);
    uint32_t* nk = reinterpret_cast<uint32_t*>(sp);
    sp += ((size_t)rows * 4 + 255) & ~(size_t)255;
    K* okey = reinterpret_cast<K*>(out_val);
    hipLaunchKernelGGL((select_collect_kernel<T>), dim3((unsigned)rows), dim3(256), 0, s, dist, rows, cols, ld, k,
                       okey, out_idx, nk);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nchunks = (k + N - 1) / N;
    hipLaunchKernelGGL((select_sort_chunk_kernel<T>), dim3((unsigned)(rows * nchunks)), dim3(512), 0, s, okey,
                       out_idx, nk, rows, k, nchunks);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t nblk = (k + 255) / 256;
    const K* src_k = okey;
    const uint32_t* src_i = out_idx;
    if (nchunks > 1) {
        K* tk = reinterpret_cast<K*>(sp);
        sp += ((size_t)rows * k * sizeof(K) + 255) & ~(size_t)255;
        uint32_t* ti = reinterpret_cast<uint32_t*>(sp);
        K* bufk[2] = {okey, tk};
        uint32_t* bufi[2] = {out_idx, ti};
        int cur = 0;
        for (int64_t L = N; L < k; L *= 2) {
            hipLaunchKernelGGL((select_merge_kernel<K>), dim3((unsigned)(rows * nblk)), dim3(256), 0, s, bufk[cur],
                               bufi[cur], bufk[cur ^ 1], bufi[cur ^ 1], nk, rows, k, L, nblk);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
            cur ^= 1;
        }
        src_k = bufk[cur];
        src_i = bufi[cur];
    }
    hipLaunchKernelGGL((select_finish_kernel<T>), dim3((unsigned)(rows * nblk)), dim3(256), 0, s, src_k, src_i, nk,
                       rows, k, mode, nblk, out_val, out_idx);
    return hipGetLastError();
}

template hipError_t launch_row_norms<float>(const float*, int64_t, int64_t, float*, float*, float*,
                                            NormStats*, hipStream_t);
template hipError_t launch_row_norms<double>(const double*, int64_t, int64_t, double*, double*, double*,
                                             NormStats*, hipStream_t);
template hipError_t launch_pow_inplace<float>(float*, int64_t, float, hipStream_t);
template hipError_t launch_pow_inplace<double>(double*, int64_t, double, hipStream_t);
template hipError_t launch_pairwise_tile<float>(const float*, int64_t, const float*, int64_t, int64_t, int,
                                                const float*, const float*, float*, int64_t, int, hipStream_t,
                                                float, int, float);
template hipError_t launch_pairwise_tile<double>(const double*, int64_t, const double*, int64_t, int64_t,
                                                 int, const double*, const double*, double*, int64_t, int,
                                                 hipStream_t, double, int, double);
template hipError_t launch_select_rows<float>(const float*, int64_t, int64_t, int64_t, int, int, float*,
                                              uint32_t*, void*, hipStream_t);
template hipError_t launch_select_rows<double>(const double*, int64_t, int64_t, int64_t, int, int, double*,
                                               uint32_t*, void*, hipStream_t);

}  // namespace mlrs
