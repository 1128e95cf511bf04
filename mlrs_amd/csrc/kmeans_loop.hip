// Device pieces of the k-means fit loop around the fused assignment
// (crates/mlrs-algos/src/cluster/kmeans.rs:929-1155, prims/kmeans.rs).
//
// Centroid sums.  The reference forms, for every row block b of its layout
// (nb = clamp(ceil(n/256), 1, max(8M/(k*d), 64)), rpb = ceil(n/nb)), the F sum
// of x[i][j] over the block's rows i with label c in ascending i, then the F
// sum of the nb partials in block order (centroid_sumcount_blocked +
// centroid_reduce_partials, crates/mlrs-kernels/src/kmeans.rs:329-479).  It
// evaluates that with one thread per (b, c, j) scanning the whole block, n*k*d
// label tests.  Here the rows are first bucketed by (block, label) -- a
// per-block label histogram, offsets, and a stable scatter of the row
// numbers -- so the thread of (b, c, j) walks exactly the rows of its bucket,
// in ascending order: the same sums in the same order for O(n*d) work.
//
// Each block is cut into S sub-blocks of consecutive rows, one wave each, so
// the scatter fills the chip whatever the block count:
//   km_subhist_kernel       cursor[b][s][c]: label counts of sub-block (b, s)
//   km_subprefix_kernel     per (b, c): counts -> exclusive prefix over s, and
//                           pcount[b][c], the bucket size
//   km_label_totals_kernel  per label: its total and each (b, c) bucket's
//   km_label_starts_kernel  start in the label-major permutation (a prefix
//   km_add_starts_kernel    over blocks, then over labels)
//   km_scatter_kernel       stable scatter of each sub-block's rows: row i of
//                           label c goes to seg[b][c] + cursor[b][s][c] + its
//                           rank among the sub-block's earlier rows of c
//   km_psum_kernel          psum[b][c][j] over the bucket, ascending rows
//   km_reduce_kernel        sums[c][j] = sum over b in order
//
// Also: km_changed_kernel (labels that differ), km_inertia_rows_kernel and
// km_block_sum_kernel (inertia_rows + block_sum_f, kernels/kmeans.rs:123-145,
// 523-545), km_mean_kernel (the mean divide), km_col_sum_kernel (col_sum_blocked and, given the means,
// col_sqdiff_blocked, :704-762), km_mind2_kernel (kmeanspp_mind2, :576-603) and
// km_gather_kernel (gather_rows_idx, :552-570).  Every sum is the reference's
// element type and order.
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

// The lanes of the wave whose label equals this lane's (a label-match ballot
// over the label bits), among the lanes in `active`.
__device__ __forceinline__ uint64_t same_label_lanes(uint32_t lab, int nbits, uint64_t active) {
    uint64_t m = active;
    for (int bit = 0; bit < nbits; ++bit) {
        const bool one = (lab >> bit) & 1u;
        const uint64_t bal = __builtin_amdgcn_ballot_w64(one);
        m &= one ? bal : ~bal;
    }
    return m;
}

// acc + p[0] + p[stride] + ... in order; the loads are issued 16 at a time
// ahead of the dependent adds, so a long strided sum is not latency-bound.
template <typename T>
__device__ __forceinline__ T ordered_sum(const T* __restrict__ p, int64_t count, int64_t stride) {
    T acc = T(0);
    int64_t b = 0;
    for (; b + 16 <= count; b += 16) {
        T v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = p[(b + u) * stride];
#pragma unroll
        for (int u = 0; u < 16; ++u) acc = acc + v[u];
    }
    for (; b < count; ++b) acc = acc + p[b * stride];
    return acc;
}

// One wave per sub-block (b, s): its label counts into cursor[b][s][.]
// (zeroed by the caller).  Each chunk of 64 rows adds one count per distinct
// label, from the group's lowest lane; the wave owns the counts, so the adds
// need no atomics.
__global__ __launch_bounds__(256) void km_subhist_kernel(const uint32_t* __restrict__ labels, int64_t n,
                                                         int64_t rpb, int64_t k, int64_t nsub, int64_t srows,
                                                         int nbits, uint32_t* __restrict__ cursor) {
    const int64_t wv = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t b = wv / nsub, sb = wv - b * nsub;
    const int64_t bend = ((b + 1) * rpb < n) ? (b + 1) * rpb : n;
    const int64_t start = b * rpb + sb * srows;
    const int64_t end = (start + srows < bend) ? start + srows : bend;
    if (b * rpb >= n || start >= end) return;
    uint32_t* cur = cursor + wv * k;
    const uint64_t below = (1ull << lane) - 1ull;
    for (int64_t i0 = start; i0 < end; i0 += 64) {
        const int64_t i = i0 + lane;
        const bool on = i < end;
        const uint32_t lab = on ? labels[i] : 0u;
        const uint64_t grp = same_label_lanes(lab, nbits, __builtin_amdgcn_ballot_w64(on));
        if (on && (grp & below) == 0) cur[lab] += (uint32_t)__builtin_popcountll(grp);
        // the next chunk may read a count another lane just wrote
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
}

// One thread per (b, c): the sub-blocks' counts become their exclusive prefix
// (the label's rows before sub-block s within the block), and the total is the
// (b, c) bucket's size.
__global__ __launch_bounds__(256) void km_subprefix_kernel(uint32_t* __restrict__ cursor, int64_t nb, int64_t k,
                                                           int64_t nsub, uint32_t* __restrict__ pcount) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= nb * k) return;
    const int64_t b = t / k, c = t - b * k;
    uint32_t run = 0;
    for (int64_t sb = 0; sb < nsub; ++sb) {
        uint32_t* p = cursor + ((b * nsub + sb) * k + c);
        const uint32_t v = *p;
        *p = run;
        run += v;
    }
    pcount[t] = run;
}

// One thread per label: counts[c], and seg[b][c] = the bucket's first slot
// relative to the label's own start (the label offsets come next).
__global__ __launch_bounds__(256) void km_label_totals_kernel(const uint32_t* __restrict__ pcount, int64_t nb,
                                                              int64_t k, uint32_t* __restrict__ seg,
                                                              uint32_t* __restrict__ counts) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= k) return;
    uint32_t run = 0;
    int64_t b = 0;
    for (; b + 16 <= nb; b += 16) {
        uint32_t v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = pcount[(b + u) * k + c];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            seg[(b + u) * k + c] = run;
            run += v[u];
        }
    }
    for (; b < nb; ++b) {
        seg[b * k + c] = run;
        run += pcount[b * k + c];
    }
    counts[c] = run;
}

// One block: exclusive scan of the label totals (label starts in the permutation).
__global__ __launch_bounds__(256) void km_label_starts_kernel(const uint32_t* __restrict__ counts, int64_t k,
                                                              uint32_t* __restrict__ starts) {
    __shared__ uint32_t wsum[4];
    __shared__ uint32_t carry_s;
    if (threadIdx.x == 0) carry_s = 0;
    __syncthreads();
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int64_t c0 = 0; c0 < k; c0 += 256) {
        const int64_t c = c0 + threadIdx.x;
        const uint32_t v = c < k ? counts[c] : 0u;
        uint32_t inc = v;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t u = (uint32_t)__shfl_up((int)inc, o, 64);
            if (lane >= o) inc += u;
        }
        if (lane == 63) wsum[w] = inc;
        __syncthreads();
        uint32_t before = carry_s;
        for (int i = 0; i < w; ++i) before += wsum[i];
        if (c < k) starts[c] = before + inc - v;
        __syncthreads();
        if (threadIdx.x == 0) carry_s += wsum[0] + wsum[1] + wsum[2] + wsum[3];
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void km_add_starts_kernel(uint32_t* __restrict__ seg, int64_t nb, int64_t k,
                                                            const uint32_t* __restrict__ starts) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < nb * k; t += stride) seg[t] += starts[t % k];
}

// One wave per sub-block (b, s), its rows in order, 64 at a time: a row goes
// to its bucket's start seg[b][c], plus the label's rows in earlier
// sub-blocks and earlier chunks (cursor[b][s][c], advanced by the group's
// highest lane), plus its rank among the chunk's earlier rows of the label.
__global__ __launch_bounds__(256) void km_scatter_kernel(const uint32_t* __restrict__ labels, int64_t n,
                                                         int64_t rpb, int64_t k, int64_t nsub, int64_t srows,
                                                         int nbits, const uint32_t* __restrict__ seg,
                                                         uint32_t* __restrict__ cursor, uint32_t* __restrict__ perm) {
    const int64_t wv = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t b = wv / nsub, sb = wv - b * nsub;
    const int64_t bend = ((b + 1) * rpb < n) ? (b + 1) * rpb : n;
    const int64_t start = b * rpb + sb * srows;
    const int64_t end = (start + srows < bend) ? start + srows : bend;
    if (b * rpb >= n || start >= end) return;
    uint32_t* cur = cursor + wv * k;
    const uint32_t* bseg = seg + b * k;
    const uint64_t below = (1ull << lane) - 1ull;
    for (int64_t i0 = start; i0 < end; i0 += 64) {
        const int64_t i = i0 + lane;
        const bool on = i < end;
        const uint32_t lab = on ? labels[i] : 0u;
        const uint64_t grp = same_label_lanes(lab, nbits, __builtin_amdgcn_ballot_w64(on));
        if (on) {
            const uint32_t rank = (uint32_t)__builtin_popcountll(grp & below);
            const uint32_t base = cur[lab];
            perm[bseg[lab] + base + rank] = (uint32_t)i;
            if ((grp >> lane) == 1ull) cur[lab] = base + (uint32_t)__builtin_popcountll(grp);  // highest lane
        }
        // the next chunk may read a cursor another lane just wrote
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
}

template <typename T>
__global__ __launch_bounds__(256) void km_psum_kernel(const T* __restrict__ x, int64_t d, int64_t nb, int64_t k,
                                                      const uint32_t* __restrict__ pcount,
                                                      const uint32_t* __restrict__ seg,
                                                      const uint32_t* __restrict__ perm, T* __restrict__ psum) {
    const int64_t total = nb * k * d;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += stride) {
        const int64_t bc = t / d, j = t - bc * d;
        const uint32_t s0 = seg[bc], m = pcount[bc];
        const uint32_t* __restrict__ pp = perm + s0;
        // the bucket's rows in ascending order; eight row numbers, then eight
        // elements, are loaded ahead of the dependent adds
        T acc = T(0);
        uint32_t p = 0;
        for (; p + 8 <= m; p += 8) {
            uint32_t r[8];
            T v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) r[u] = pp[p + u];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = x[(int64_t)r[u] * d + j];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = acc + v[u];
        }
        for (; p < m; ++p) acc = acc + x[(int64_t)pp[p] * d + j];
        psum[t] = acc;
    }
}

// The same sums with one wave per (bucket, 64-feature chunk), for d a
// multiple of 64: the bucket is wave-uniform, so its row numbers come through
// scalar loads, eight at a time with the next eight requested while this
// eight's row loads are in flight, and lane j adds feature chunk * 64 + j of
// each row in ascending order (the same order and operations as
// km_psum_kernel).
template <typename T>
__global__ __launch_bounds__(256) void km_psum_wave_kernel(const T* __restrict__ x, int64_t d, int64_t nb,
                                                           int64_t k, const uint32_t* __restrict__ pcount,
                                                           const uint32_t* __restrict__ seg,
                                                           const uint32_t* __restrict__ perm,
                                                           T* __restrict__ psum) {
    const int lane = threadIdx.x & 63;
    const int64_t nch = d >> 6;
    const int64_t total = nb * k * nch;
    const int64_t step = (int64_t)gridDim.x * 4;
    for (int64_t wv = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); wv < total;
         wv += step) {
        const int64_t bc = wv / nch;
        const int64_t j = (wv - bc * nch) * 64 + lane;
        const uint32_t s0 = seg[bc], m = pcount[bc];
        const uint32_t* __restrict__ pp = perm + s0;
        const T* __restrict__ xj = x + j;
        T acc = T(0);
        uint32_t p = 0;
        uint32_t r[8];
        if (m >= 8) {
#pragma unroll
            for (int u = 0; u < 8; ++u) r[u] = pp[u];
        }
        for (; p + 8 <= m; p += 8) {
            T v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = xj[(int64_t)r[u] * d];
            if (p + 16 <= m) {
#pragma unroll
                for (int u = 0; u < 8; ++u) r[u] = pp[p + 8 + u];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = acc + v[u];
        }
        for (; p < m; ++p) acc = acc + xj[(int64_t)pp[p] * d];
        psum[bc * d + j] = acc;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void km_reduce_kernel(const T* __restrict__ psum, int64_t nb, int64_t kd,
                                                        T* __restrict__ sums) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= kd) return;
    sums[t] = ordered_sum<T>(psum + t, nb, kd);
}

// Labels that differ: 16 bytes (four labels) per load where both arrays are
// 16-byte aligned, the workgroup's count summed in LDS and added to `count`
// with one atomic per workgroup (one per wave made 5M labels cost 0.14 ms:
// the atomics on one word serialise).
__global__ __launch_bounds__(256) void km_changed_kernel(const uint32_t* __restrict__ a,
                                                         const uint32_t* __restrict__ b, int64_t n,
                                                         unsigned int* __restrict__ count) {
    __shared__ unsigned int part[4];
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t first = (int64_t)blockIdx.x * 256 + threadIdx.x;
    unsigned int local = 0;
    int64_t tail = 0;
    if (((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0) {
        const uint4* a4 = reinterpret_cast<const uint4*>(a);
        const uint4* b4 = reinterpret_cast<const uint4*>(b);
        const int64_t n4 = n / 4;
        for (int64_t i = first; i < n4; i += stride) {
            const uint4 x = a4[i], y = b4[i];
            local += (x.x != y.x ? 1u : 0u) + (x.y != y.y ? 1u : 0u) + (x.z != y.z ? 1u : 0u) + (x.w != y.w ? 1u : 0u);
        }
        tail = 4 * n4;
    }
    for (int64_t i = tail + first; i < n; i += stride) local += (a[i] != b[i]) ? 1u : 0u;
    for (int o = 32; o > 0; o >>= 1) local += (unsigned int)__shfl_xor((int)local, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = local;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned int sum = part[0] + part[1] + part[2] + part[3];
        if (sum) atomicAdd(count, sum);
    }
}

// sum over j of (x[j] - c[j])^2 as acc + diff * diff in ascending j.  VEC:
// both rows 16-byte aligned and d a multiple of 16 / sizeof(T), so they are
// read 16 bytes at a time, eight pieces in flight.
template <typename T, bool VEC>
__device__ __forceinline__ T row_sqdist(const T* __restrict__ xr, const T* __restrict__ cr, int64_t d) {
    T acc = T(0);
    if constexpr (VEC) {
        constexpr int V = 16 / (int)sizeof(T);
        constexpr int U = 8;
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        const float4* c4 = reinterpret_cast<const float4*>(cr);
        const int64_t n4 = d / V;
        int64_t p = 0;
        for (; p + U <= n4; p += U) {
            float4 a[U], b[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                a[u] = x4[p + u];
                b[u] = c4[p + u];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const T* av = reinterpret_cast<const T*>(&a[u]);
                const T* bv = reinterpret_cast<const T*>(&b[u]);
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const T diff = av[e] - bv[e];
                    acc = acc + diff * diff;
                }
            }
        }
        for (; p < n4; ++p) {
            const float4 a = x4[p], b = c4[p];
            const T* av = reinterpret_cast<const T*>(&a);
            const T* bv = reinterpret_cast<const T*>(&b);
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const T diff = av[e] - bv[e];
                acc = acc + diff * diff;
            }
        }
    } else {
        for (int64_t j = 0; j < d; ++j) {
            const T diff = xr[j] - cr[j];
            acc = acc + diff * diff;
        }
    }
    return acc;
}

template <typename T>
bool rows_vec(const T* x, const T* c, int64_t d) {
    return (d % (16 / (int64_t)sizeof(T)) == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0) &&
           ((reinterpret_cast<uintptr_t>(c) & 15) == 0);
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void km_inertia_rows_kernel(const T* __restrict__ x, const T* __restrict__ c,
                                                              const uint32_t* __restrict__ labels, int64_t n,
                                                              int64_t d, T* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    out[i] = row_sqdist<T, VEC>(x + i * d, c + (int64_t)labels[i] * d, d);
}

// block_sum_f: out[b] = ((v[b rpb] + v[b rpb + 1]) + ...) in order, one
// dependent chain per block (a few hundred blocks of ~20,000 rows at the
// reference's sum_device layout).  A workgroup per block stages its values
// through LDS in 16 KB chunks, double-buffered: lane 0 adds one chunk while
// waves 1-3 load the next, so the chain runs at the add latency rather than
// behind one thread's loads.
template <typename T>
__global__ __launch_bounds__(256) void km_block_sum_kernel(const T* __restrict__ v, int64_t n, int64_t rpb,
                                                           T* __restrict__ out) {
    constexpr int CH = 16384 / (int)sizeof(T);
    constexpr int V = 16 / (int)sizeof(T);
    __shared__ __attribute__((aligned(16))) T buf[2][CH];
    const int64_t start = (int64_t)blockIdx.x * rpb;
    const int64_t len = ((start + rpb) < n ? start + rpb : n) - start;
    const int nch = (int)((len + CH - 1) / CH);
    const int tid = threadIdx.x;
    auto chunk_len = [&](int c) -> int {
        const int64_t left = len - (int64_t)c * CH;
        return left < CH ? (int)left : CH;
    };
    auto load = [&](int c, T* dst, int first, int step) {
        const T* src = v + start + (int64_t)c * CH;
        const int cnt = chunk_len(c);
        for (int i = first; i < cnt; i += step) dst[i] = src[i];
    };
    if (nch > 0) load(0, buf[0], tid, 256);
    __syncthreads();
    T acc = T(0);
    for (int c = 0; c < nch; ++c) {
        if (tid >= 64 && c + 1 < nch) load(c + 1, buf[(c + 1) & 1], tid - 64, 192);
        if (tid == 0) {
            const T* p = buf[c & 1];
            const int cnt = chunk_len(c);
            const int nv = cnt / V;
            int i = 0;
            // 16-byte reads eight ahead of the adds (they are independent of them)
            for (; i + 8 <= nv; i += 8) {
                float4 w[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) w[u] = reinterpret_cast<const float4*>(p)[i + u];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const T* e = reinterpret_cast<const T*>(&w[u]);
#pragma unroll
                    for (int j = 0; j < V; ++j) acc = acc + e[j];
                }
            }
            for (int j = i * V; j < cnt; ++j) acc = acc + p[j];
        }
        __syncthreads();  // chunk c read; chunk c + 1 stored
    }
    if (tid == 0) out[blockIdx.x] = acc;
}

// The new centres from the sums and counts: (T)((double)sums * (1.0 /
// (double)count)), the host's mean divide (single_run, cluster/kmeans.rs
// :1010-1030) operation for operation; every step is correctly rounded on the
// device as on the host, so the centres are the same bits.  A label without
// rows gives NaN or inf here; the host then relocates and uploads its own.
template <typename T>
__global__ __launch_bounds__(256) void km_mean_kernel(const T* __restrict__ sums, const uint32_t* __restrict__ counts,
                                                      int64_t k, int64_t d, T* __restrict__ out) {
    const int64_t total = k * d;
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < total; q += (int64_t)gridDim.x * 256) {
        const double inv = 1.0 / (double)counts[q / d];
        out[q] = (T)((double)sums[q] * inv);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void km_col_sum_kernel(const T* __restrict__ x, int64_t n, int64_t d, int64_t nb,
                                                         int64_t rpb, const T* __restrict__ means,
                                                         T* __restrict__ out) {
    const int64_t total = nb * d;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += stride) {
        const int64_t b = t / d, j = t - b * d;
        const int64_t start = b * rpb;
        const int64_t end = (start + rpb) < n ? start + rpb : n;
        T acc = T(0);
        if (means) {
            const T m = means[j];
            for (int64_t i = start; i < end; ++i) {
                const T diff = x[i * d + j] - m;
                acc = acc + diff * diff;
            }
        } else {
            acc = ordered_sum<T>(x + start * d + j, end - start, d);
        }
        out[t] = acc;
    }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void km_mind2_kernel(const T* __restrict__ x, int64_t n, int64_t d, int64_t cidx,
                                                       int first, T* __restrict__ mind2) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const T acc = row_sqdist<T, VEC>(x + i * d, x + cidx * d, d);
    if (first || acc < mind2[i]) mind2[i] = acc;
}

template <typename T>
__global__ __launch_bounds__(256) void km_gather_kernel(const T* __restrict__ x, const int64_t* __restrict__ idx,
                                                        int64_t k, int64_t d, T* __restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= k * d) return;
    const int64_t c = t / d, j = t - c * d;
    out[t] = x[idx[c] * d + j];
}

unsigned blocks_for(int64_t n, int64_t cap) {
    int64_t b = (n + 255) / 256;
    if (b < 1) b = 1;
    if (b > cap) b = cap;
    return (unsigned)b;
}

}  // namespace

int64_t km_sub_blocks(int64_t nb, int64_t rpb, int64_t k) {
    // about 2,048 waves in all, at least 64 rows each, and the per-(sub-block,
    // label) cursors within 256 MB
    int64_t sb = (2048 + nb - 1) / nb;
    const int64_t by_rows = (rpb + 63) / 64;
    if (sb > by_rows) sb = by_rows;
    const int64_t by_mem = ((int64_t)64 << 20) / (nb * (k > 0 ? k : 1));
    if (sb > by_mem) sb = by_mem;
    return sb < 1 ? 1 : sb;
}

template <typename T>
hipError_t launch_km_centroid_sums(const T* x, const uint32_t* labels, int64_t n, int64_t d, int64_t k, int64_t nb,
                                   int64_t rpb, const KmScratch<T>& w, hipStream_t s) {
    const int64_t nsub = km_sub_blocks(nb, rpb, k);
    const int64_t srows = (rpb + nsub - 1) / nsub;
    int nbits = 0;
    while (nbits < 32 && ((int64_t)1 << nbits) < k) ++nbits;
    const int64_t waves = nb * nsub;
    hipError_t e = launch_fill_u32(w.cursor, waves * k, 0u, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(km_subhist_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, labels, n, rpb, k, nsub,
                       srows, nbits, w.cursor);
    hipLaunchKernelGGL(km_subprefix_kernel, dim3(blocks_for(nb * k, 1 << 30)), dim3(256), 0, s, w.cursor, nb, k, nsub,
                       w.pcount);
    hipLaunchKernelGGL(km_label_totals_kernel, dim3(blocks_for(k, 1 << 20)), dim3(256), 0, s, w.pcount, nb, k, w.seg,
                       w.counts);
    hipLaunchKernelGGL(km_label_starts_kernel, dim3(1), dim3(256), 0, s, w.counts, k, w.starts);
    hipLaunchKernelGGL(km_add_starts_kernel, dim3(blocks_for(nb * k, 4096)), dim3(256), 0, s, w.seg, nb, k, w.starts);
    hipLaunchKernelGGL(km_scatter_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, labels, n, rpb, k, nsub,
                       srows, nbits, w.seg, w.cursor, w.perm);
    if (d % 64 == 0)
        hipLaunchKernelGGL((km_psum_wave_kernel<T>), dim3(blocks_for(nb * k * (d / 64) * 64, 65536)), dim3(256), 0, s,
                           x, d, nb, k, w.pcount, w.seg, w.perm, w.psum);
    else
        hipLaunchKernelGGL((km_psum_kernel<T>), dim3(blocks_for(nb * k * d, 65536)), dim3(256), 0, s, x, d, nb, k,
                           w.pcount, w.seg, w.perm, w.psum);
    hipLaunchKernelGGL((km_reduce_kernel<T>), dim3(blocks_for(k * d, 1 << 20)), dim3(256), 0, s, w.psum, nb, k * d,
                       w.sums);
    return hipGetLastError();
}

hipError_t launch_km_changed(const uint32_t* a, const uint32_t* b, int64_t n, unsigned int* count, hipStream_t s) {
    hipError_t e = launch_fill_u32(count, 1, 0u, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(km_changed_kernel, dim3(blocks_for((n + 3) / 4, 1024)), dim3(256), 0, s, a, b, n, count);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_km_inertia(const T* x, const T* c, const uint32_t* labels, int64_t n, int64_t d, T* rows,
                             int64_t nb, int64_t rpb, T* parts, hipStream_t s) {
    if (rows_vec(x, c, d))
        hipLaunchKernelGGL((km_inertia_rows_kernel<T, true>), dim3(blocks_for(n, 1 << 30)), dim3(256), 0, s, x, c,
                           labels, n, d, rows);
    else
        hipLaunchKernelGGL((km_inertia_rows_kernel<T, false>), dim3(blocks_for(n, 1 << 30)), dim3(256), 0, s, x, c,
                           labels, n, d, rows);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? launch_km_block_sum<T>(rows, n, nb, rpb, parts, s) : e;
}

template <typename T>
hipError_t launch_km_block_sum(const T* v, int64_t n, int64_t nb, int64_t rpb, T* parts, hipStream_t s) {
    if (nb <= 0) return hipSuccess;
    hipLaunchKernelGGL((km_block_sum_kernel<T>), dim3((unsigned)nb), dim3(256), 0, s, v, n, rpb, parts);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_km_mean(const T* sums, const uint32_t* counts, int64_t k, int64_t d, T* out, hipStream_t s) {
    if (k * d <= 0) return hipSuccess;
    hipLaunchKernelGGL((km_mean_kernel<T>), dim3(blocks_for(k * d, 4096)), dim3(256), 0, s, sums, counts, k, d, out);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_km_col_sums(const T* x, int64_t n, int64_t d, int64_t nb, int64_t rpb, const T* means, T* out,
                              hipStream_t s) {
    hipLaunchKernelGGL((km_col_sum_kernel<T>), dim3(blocks_for(nb * d, 65536)), dim3(256), 0, s, x, n, d, nb, rpb,
                       means, out);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_km_mind2(const T* x, int64_t n, int64_t d, int64_t cidx, int first, T* mind2, hipStream_t s) {
    if (rows_vec(x, x, d))
        hipLaunchKernelGGL((km_mind2_kernel<T, true>), dim3(blocks_for(n, 1 << 30)), dim3(256), 0, s, x, n, d, cidx,
                           first, mind2);
    else
        hipLaunchKernelGGL((km_mind2_kernel<T, false>), dim3(blocks_for(n, 1 << 30)), dim3(256), 0, s, x, n, d, cidx,
                           first, mind2);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_km_gather(const T* x, const int64_t* idx, int64_t k, int64_t d, T* out, hipStream_t s) {
    hipLaunchKernelGGL((km_gather_kernel<T>), dim3(blocks_for(k * d, 1 << 30)), dim3(256), 0, s, x, idx, k, d, out);
    return hipGetLastError();
}

// Relocation ranking (relocate_empty_clusters, prims/kmeans.rs:1323-1410):
// the keys -distance, so that ascending (key, index) is the reference's
// (distance desc, index asc) order, padded with +inf up to `padded` entries,
// and the number of NaN distances (the reference ranks those first, which the
// keys cannot express).
template <typename T>
__global__ __launch_bounds__(256) void km_neg_kernel(const T* __restrict__ dist, int64_t n, int64_t padded,
                                                     T* __restrict__ neg, unsigned int* __restrict__ nans) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    bool nan = false;
    if (i < n) {
        const T v = dist[i];
        neg[i] = -v;
        nan = v != v;
    } else if (i < padded) {
        neg[i] = FloatTraits<T>::inf();
    }
    const uint64_t b = __builtin_amdgcn_ballot_w64(nan);
    if (b != 0 && (int)(threadIdx.x & 63) == __builtin_ctzll(b)) atomicAdd(nans, (unsigned int)__builtin_popcountll(b));
}

// Global row numbers of the first stage's picks: pick j of chunk r (column
// idx[r m + j] of the chunk) is row r C + idx.
__global__ __launch_bounds__(256) void km_chunk_rows_kernel(const uint32_t* __restrict__ idx, int64_t nchunks,
                                                            int64_t m, int64_t C, uint32_t* __restrict__ rows) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < nchunks * m) rows[i] = (uint32_t)((i / m) * C + idx[i]);
}

// out[i] = src[idx[i]], i < m (0 for an index past the n_src entries).
__global__ __launch_bounds__(256) void km_take_u32_kernel(const uint32_t* __restrict__ src, int64_t n_src,
                                                          const uint32_t* __restrict__ idx, int64_t m,
                                                          uint32_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < m) out[i] = ((int64_t)idx[i] < n_src) ? src[idx[i]] : 0u;
}

template <typename T>
hipError_t launch_km_neg(const T* dist, int64_t n, int64_t padded, T* neg, unsigned int* nans, hipStream_t s) {
    hipError_t e = launch_fill_u32(nans, 1, 0u, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((km_neg_kernel<T>), dim3((unsigned)((padded + 255) / 256)), dim3(256), 0, s, dist, n, padded,
                       neg, nans);
    return hipGetLastError();
}

hipError_t launch_km_chunk_rows(const uint32_t* idx, int64_t nchunks, int64_t m, int64_t C, uint32_t* rows,
                                hipStream_t s) {
    hipLaunchKernelGGL(km_chunk_rows_kernel, dim3((unsigned)((nchunks * m + 255) / 256)), dim3(256), 0, s, idx,
                       nchunks, m, C, rows);
    return hipGetLastError();
}

hipError_t launch_km_take_u32(const uint32_t* src, int64_t n_src, const uint32_t* idx, int64_t m, uint32_t* out,
                              hipStream_t s) {
    hipLaunchKernelGGL(km_take_u32_kernel, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, src, n_src, idx, m,
                       out);
    return hipGetLastError();
}

namespace {

// ---------------------------------------------------------------------------
// Bound-pruned assignment (algorithm = 'elkan'; the reference's
// elkan_init_bounds / elkan_assign_device / elkan_relax_bounds,
// crates/mlrs-backend/src/prims/kmeans.rs:1523-1717, carry an n x k lower-bound
// matrix, 20 GB and as many bytes of traffic per iteration at 5M x 1,024).
// Here: one upper bound U[i] >= |x_i - c_a| per row (a its label), the k x k
// half centre distances h(a, c) = |c_a - c_c| / 2 (lower bounds) with each
// centre's row sorted, and dnc[a] = min over c != a of h(a, c).  By the
// triangle inequality |x_i - c_c| >= 2 h(a, c) - U, so every centre with
// h(a, c) >= K U lies strictly farther than c_a -- strictly also for the
// COMPUTED distances (F arithmetic, the assignment's operation order): with
// gamma bounding their relative error and eta the absolute error of
// underflowing terms, K = (1 + gamma) / (1 - gamma) (1 + 2^-30) and U >= umin =
// sqrt(2^30 eta) leave a margin U^2 (1 + gamma) 2^-29 > 2 eta.  A row with
// dnc[a] >= K U keeps its label without a distance; else its own distance
// tightens U, and the centres with h(a, c) < K U (a prefix of a's sorted row)
// are evaluated exactly and ranked by (distance, index) with c_a; a row with
// more than maxcand such centres goes to the fused k = 1 search instead
// (compacted into fb_list).  Labels are therefore the assignment's own.
// Bounds are kept in f64: after a centre update U += delta[a] (an upper
// bound of the centre's move), and every fresh distance v resets
// U = sqrt((v + eta) / (1 - gamma)).
template <typename T>
__global__ __launch_bounds__(256) void km_half_dist_kernel(const T* __restrict__ c, int64_t k, int64_t d,
                                                           double* __restrict__ hcd, double* __restrict__ dnc) {
    const int64_t a = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (a >= k) return;
    const double inf = __builtin_huge_val();
    double best = inf;
    for (int64_t c0 = 0; c0 < k; c0 += 64) {
        const int64_t cc = c0 + lane;
        if (cc < k) {
            double acc = 0.0;
            for (int64_t j = 0; j < d; ++j) {
                const double diff = (double)c[a * d + j] - (double)c[cc * d + j];
                acc += diff * diff;
            }
            // a lower bound: the f64 sum's relative error is far below 2^-40
            const double h = 0.5 * __builtin_sqrt(acc) * (1.0 - 0x1p-40);
            hcd[a * k + cc] = (cc == a) ? 0.0 : h;
            if (cc != a) best = fmin(best, h);
        }
    }
    for (int m = 32; m > 0; m >>= 1) best = fmin(best, __shfl_xor(best, m, 64));
    if (lane == 0) dnc[a] = best;
}

__device__ __forceinline__ double km_upper(double v, double gamma, double eta) {
    // |x - c|^2 <= (v + eta) / (1 - gamma); NaN or inf gives +inf
    const double u = __builtin_sqrt((v + eta) / (1.0 - gamma)) * (1.0 + 0x1p-50);
    return (u == u && u < __builtin_huge_val()) ? u : __builtin_huge_val();
}

template <typename T>
__global__ __launch_bounds__(256) void km_bound_init_kernel(const T* __restrict__ dist, int64_t n, double gamma,
                                                            double eta, double* __restrict__ U) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) U[i] = km_upper((double)dist[i], gamma, eta);
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void km_elkan_kernel(const T* __restrict__ x, int64_t n, int64_t d,
                                                       const T* __restrict__ c, int64_t k,
                                                       const uint32_t* __restrict__ lab_old,
                                                       uint32_t* __restrict__ lab_new, T* __restrict__ dist,
                                                       double* __restrict__ U, const double* __restrict__ delta,
                                                       const double* __restrict__ dnc,
                                                       const double* __restrict__ sv,
                                                       const uint32_t* __restrict__ si, KmPruneConsts pc,
                                                       uint32_t* __restrict__ fb_list,
                                                       unsigned int* __restrict__ fb_count) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int lane = threadIdx.x & 63;
    bool fallback = false;
    if (i < n) {
        uint32_t a = lab_old[i];
        double u = (U[i] + delta[a]) * (1.0 + 0x1p-50);
        if (!(u == u)) u = __builtin_huge_val();
        if (!(u >= pc.umin && dnc[a] >= pc.K * u)) {
            const T* xr = x + i * d;
            const T da = row_sqdist<T, VEC>(xr, c + (int64_t)a * d, d);
            const double ut = km_upper((double)da, pc.gamma, pc.eta);
            if (ut < u) u = ut;
            T bv = da;
            uint32_t bi = a;
            if (!(u >= pc.umin && dnc[a] >= pc.K * u)) {
                // the centres that may lie nearer: a prefix of a's sorted row
                const double lim = (u >= pc.umin) ? pc.K * u : __builtin_huge_val();
                const double* hrow = sv + (int64_t)a * k;
                const uint32_t* crow = si + (int64_t)a * k;
                int cnt = 0;
                for (int64_t j = 0; j < k; ++j) {
                    if (!(hrow[j] < lim)) break;
                    const uint32_t cc = crow[j];
                    if (cc == a) continue;
                    if (++cnt > pc.maxcand) {
                        fallback = true;
                        break;
                    }
                    const T dc = row_sqdist<T, VEC>(xr, c + (int64_t)cc * d, d);
                    if (dc < bv || (dc == bv && cc < bi)) {
                        bv = dc;
                        bi = cc;
                    }
                }
            }
            if (!fallback) {
                a = bi;
                dist[i] = bv;
                u = km_upper((double)bv, pc.gamma, pc.eta);
            }
        }
        if (!fallback) {
            lab_new[i] = a;
            U[i] = u;
        }
    }
    // rows for the fused search: one atomic per wave
    const uint64_t bal = __builtin_amdgcn_ballot_w64(fallback);
    if (bal) {
        const int first = __builtin_ctzll(bal);
        unsigned int base = 0;
        if (lane == first) base = atomicAdd(fb_count, (unsigned int)__builtin_popcountll(bal));
        base = (unsigned int)__shfl((int)base, first, 64);
        if (fallback) fb_list[base + (unsigned int)__builtin_popcountll(bal & ((1ull << lane) - 1ull))] = (uint32_t)i;
    }
}

// The same assignment over rows taken in the label-major order of the
// centroid sums' permutation (perm, for the labels lab_old), with the rows
// staged through LDS: a workgroup takes 256 consecutive perm entries, so its
// rows arrive with coalesced 16-byte loads (16-byte rows of at most 512
// bytes: RC chunks, row stride RC + 1 chunks so that the threads' 16-byte
// reads of one chunk column hit distinct bank groups) and its threads mostly
// share one centre, whose row and sorted half-distance row they read
// together.  Each row's distances are still one thread's ascending sum.
template <typename T, int RC>
__global__ __launch_bounds__(256) void km_elkan_lds_kernel(const T* __restrict__ x, int64_t n, int64_t d,
                                                           const T* __restrict__ c, int64_t k,
                                                           const uint32_t* __restrict__ perm,
                                                           const uint32_t* __restrict__ lab_old,
                                                           uint32_t* __restrict__ lab_new, T* __restrict__ dist,
                                                           double* __restrict__ U, const double* __restrict__ delta,
                                                           const double* __restrict__ dnc,
                                                           const double* __restrict__ sv,
                                                           const uint32_t* __restrict__ si, KmPruneConsts pc,
                                                           uint32_t* __restrict__ fb_list,
                                                           unsigned int* __restrict__ fb_count) {
    constexpr int V = 16 / (int)sizeof(T);  // elements per 16-byte chunk
    constexpr int RS = (RC + 1) * V;        // row stride (elements)
    __shared__ __attribute__((aligned(16))) T xs[256 * RS];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int64_t p0 = (int64_t)blockIdx.x * 256;
    const int64_t pos = p0 + tid;
    const bool valid = pos < n;
    const uint32_t i = valid ? perm[pos] : 0u;
    uint32_t a = valid ? lab_old[i] : 0u;
    double u = 0.0;
    bool need = false;
    if (valid) {
        u = (U[i] + delta[a]) * (1.0 + 0x1p-50);
        if (!(u == u)) u = __builtin_huge_val();
        need = !(u >= pc.umin && dnc[a] >= pc.K * u);
    }
    bool fallback = false;
    if (__syncthreads_or(need)) {
        const int cpr = (int)(d / V);  // 16-byte chunks per row (<= RC)
        for (int e = tid; e < 256 * cpr; e += 256) {
            const int r = e / cpr, ch = e - r * cpr;
            if (p0 + r < n) {
                const float4 v = *reinterpret_cast<const float4*>(x + (int64_t)perm[p0 + r] * d + (int64_t)ch * V);
                *reinterpret_cast<float4*>(&xs[r * RS + ch * V]) = v;
            }
        }
        __syncthreads();
        if (need) {
            const T* xr = &xs[tid * RS];
            auto sqd = [&](uint32_t cc) -> T {
                const T* cr = c + (int64_t)cc * d;
                T acc = T(0);
                for (int ch = 0; ch < cpr; ++ch) {
                    const float4 xv = *reinterpret_cast<const float4*>(xr + ch * V);
                    const float4 cv = *reinterpret_cast<const float4*>(cr + ch * V);
                    const T* xa = reinterpret_cast<const T*>(&xv);
                    const T* ca = reinterpret_cast<const T*>(&cv);
#pragma unroll
                    for (int e = 0; e < V; ++e) {
                        const T diff = xa[e] - ca[e];
                        acc = acc + diff * diff;
                    }
                }
                return acc;
            };
            const T da = sqd(a);
            const double ut = km_upper((double)da, pc.gamma, pc.eta);
            if (ut < u) u = ut;
            T bv = da;
            uint32_t bi = a;
            if (!(u >= pc.umin && dnc[a] >= pc.K * u)) {
                const double lim = (u >= pc.umin) ? pc.K * u : __builtin_huge_val();
                const double* hrow = sv + (int64_t)a * k;
                const uint32_t* crow = si + (int64_t)a * k;
                int cnt = 0;
                for (int64_t j = 0; j < k; ++j) {
                    if (!(hrow[j] < lim)) break;
                    const uint32_t cc = crow[j];
                    if (cc == a) continue;
                    if (++cnt > pc.maxcand) {
                        fallback = true;
                        break;
                    }
                    const T dc = sqd(cc);
                    if (dc < bv || (dc == bv && cc < bi)) {
                        bv = dc;
                        bi = cc;
                    }
                }
            }
            if (!fallback) {
                a = bi;
                dist[i] = bv;
                u = km_upper((double)bv, pc.gamma, pc.eta);
            }
        }
    }
    if (valid && !fallback) {
        lab_new[i] = a;
        U[i] = u;
    }
    const uint64_t bal = __builtin_amdgcn_ballot_w64(fallback);
    if (bal) {
        const int first = __builtin_ctzll(bal);
        unsigned int base = 0;
        if (lane == first) base = atomicAdd(fb_count, (unsigned int)__builtin_popcountll(bal));
        base = (unsigned int)__shfl((int)base, first, 64);
        if (fallback) fb_list[base + (unsigned int)__builtin_popcountll(bal & ((1ull << lane) - 1ull))] = i;
    }
}

// The rows (and their row_sumsq) of fb_list[0..m) into dense buffers.
template <typename T>
__global__ __launch_bounds__(256) void km_gather_list_kernel(const T* __restrict__ x, const T* __restrict__ xsq,
                                                             const uint32_t* __restrict__ list, int64_t m,
                                                             int64_t d, T* __restrict__ out,
                                                             T* __restrict__ out_sq) {
    const int64_t total = m * d;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += stride) {
        const int64_t r = e / d;
        out[e] = x[(int64_t)list[r] * d + (e - r * d)];
        if (e - r * d == 0) out_sq[r] = xsq[list[r]];
    }
}

template <typename T>
__global__ __launch_bounds__(256) void km_scatter_list_kernel(const uint32_t* __restrict__ list, int64_t m,
                                                              const uint32_t* __restrict__ lab_sub,
                                                              const T* __restrict__ dist_sub, double gamma,
                                                              double eta, uint32_t* __restrict__ lab_new,
                                                              T* __restrict__ dist, double* __restrict__ U) {
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= m) return;
    const uint32_t i = list[j];
    lab_new[i] = lab_sub[j];
    dist[i] = dist_sub[j];
    U[i] = km_upper((double)dist_sub[j], gamma, eta);
}

// Rows whose row_sumsq is not finite (inf or NaN entries, or an overflowing
// sum): the pruned assignment serves finite data only.
template <typename T>
__global__ __launch_bounds__(256) void km_count_nonfinite_kernel(const T* __restrict__ v, int64_t n,
                                                                 unsigned int* __restrict__ count) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool bad = i < n && !(v[i] == v[i] && v[i] < (T)__builtin_huge_val() && v[i] > -(T)__builtin_huge_val());
    const uint64_t bal = __builtin_amdgcn_ballot_w64(bad);
    if (bal && (threadIdx.x & 63) == __builtin_ctzll(bal)) atomicAdd(count, (unsigned int)__builtin_popcountll(bal));
}

}  // namespace

template <typename T>
hipError_t launch_km_half_dist(const T* c, int64_t k, int64_t d, double* hcd, double* dnc, hipStream_t s) {
    hipLaunchKernelGGL((km_half_dist_kernel<T>), dim3((unsigned)((k + 3) / 4)), dim3(256), 0, s, c, k, d, hcd, dnc);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_km_bound_init(const T* dist, int64_t n, double gamma, double eta, double* U, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL((km_bound_init_kernel<T>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dist, n, gamma,
                       eta, U);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_km_elkan(const T* x, int64_t n, int64_t d, const T* c, int64_t k, const uint32_t* perm,
                           const uint32_t* lab_old, uint32_t* lab_new, T* dist, double* U, const double* delta,
                           const double* dnc, const double* sv, const uint32_t* si, const KmPruneConsts& pc,
                           uint32_t* fb_list, unsigned int* fb_count, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 255) / 256));
    const int64_t chunks = d * (int64_t)sizeof(T) / 16;  // 16-byte chunks per row
    if (perm && rows_vec<T>(x, c, d) && chunks <= 32) {
        if (chunks <= 16)
            hipLaunchKernelGGL((km_elkan_lds_kernel<T, 16>), grid, dim3(256), 0, s, x, n, d, c, k, perm, lab_old,
                               lab_new, dist, U, delta, dnc, sv, si, pc, fb_list, fb_count);
        else
            hipLaunchKernelGGL((km_elkan_lds_kernel<T, 32>), grid, dim3(256), 0, s, x, n, d, c, k, perm, lab_old,
                               lab_new, dist, U, delta, dnc, sv, si, pc, fb_list, fb_count);
        return hipGetLastError();
    }
    if (rows_vec<T>(x, c, d))
        hipLaunchKernelGGL((km_elkan_kernel<T, true>), grid, dim3(256), 0, s, x, n, d, c, k, lab_old, lab_new, dist,
                           U, delta, dnc, sv, si, pc, fb_list, fb_count);
    else
        hipLaunchKernelGGL((km_elkan_kernel<T, false>), grid, dim3(256), 0, s, x, n, d, c, k, lab_old, lab_new,
                           dist, U, delta, dnc, sv, si, pc, fb_list, fb_count);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_km_gather_list(const T* x, const T* xsq, const uint32_t* list, int64_t m, int64_t d, T* out,
                                 T* out_sq, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    int64_t b = (m * d + 255) / 256;
    if (b > 65536) b = 65536;
    hipLaunchKernelGGL((km_gather_list_kernel<T>), dim3((unsigned)b), dim3(256), 0, s, x, xsq, list, m, d, out,
                       out_sq);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_km_scatter_list(const uint32_t* list, int64_t m, const uint32_t* lab_sub, const T* dist_sub,
                                  double gamma, double eta, uint32_t* lab_new, T* dist, double* U, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    hipLaunchKernelGGL((km_scatter_list_kernel<T>), dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, list, m,
                       lab_sub, dist_sub, gamma, eta, lab_new, dist, U);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_km_count_nonfinite(const T* v, int64_t n, unsigned int* count, hipStream_t s) {
    hipError_t e = launch_fill_u32(count, 1, 0u, s);
    if (e != hipSuccess || n <= 0) return e;
    hipLaunchKernelGGL((km_count_nonfinite_kernel<T>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, v, n,
                       count);
    return hipGetLastError();
}

#define MLRS_KM_INST(T)                                                                                            \
    template hipError_t launch_km_centroid_sums<T>(const T*, const uint32_t*, int64_t, int64_t, int64_t, int64_t,   \
                                                   int64_t, const KmScratch<T>&, hipStream_t);                     \
    template hipError_t launch_km_inertia<T>(const T*, const T*, const uint32_t*, int64_t, int64_t, T*, int64_t,    \
                                             int64_t, T*, hipStream_t);                                            \
    template hipError_t launch_km_block_sum<T>(const T*, int64_t, int64_t, int64_t, T*, hipStream_t);              \
    template hipError_t launch_km_mean<T>(const T*, const uint32_t*, int64_t, int64_t, T*, hipStream_t);          \
    template hipError_t launch_km_col_sums<T>(const T*, int64_t, int64_t, int64_t, int64_t, const T*, T*,           \
                                              hipStream_t);                                                        \
    template hipError_t launch_km_mind2<T>(const T*, int64_t, int64_t, int64_t, int, T*, hipStream_t);              \
    template hipError_t launch_km_gather<T>(const T*, const int64_t*, int64_t, int64_t, T*, hipStream_t);        \
    template hipError_t launch_km_neg<T>(const T*, int64_t, int64_t, T*, unsigned int*, hipStream_t);                \
    template hipError_t launch_km_half_dist<T>(const T*, int64_t, int64_t, double*, double*, hipStream_t);       \
    template hipError_t launch_km_bound_init<T>(const T*, int64_t, double, double, double*, hipStream_t);        \
    template hipError_t launch_km_elkan<T>(const T*, int64_t, int64_t, const T*, int64_t, const uint32_t*,         \
                                           const uint32_t*, uint32_t*, T*, double*, const double*, const double*, \
                                           const double*,                                                        \
                                           const uint32_t*, const KmPruneConsts&, uint32_t*, unsigned int*,      \
                                           hipStream_t);                                                          \
    template hipError_t launch_km_gather_list<T>(const T*, const T*, const uint32_t*, int64_t, int64_t, T*, T*,   \
                                                 hipStream_t);                                                    \
    template hipError_t launch_km_scatter_list<T>(const uint32_t*, int64_t, const uint32_t*, const T*, double,   \
                                                  double, uint32_t*, T*, double*, hipStream_t);                   \
    template hipError_t launch_km_count_nonfinite<T>(const T*, int64_t, unsigned int*, hipStream_t);
MLRS_KM_INST(float)
MLRS_KM_INST(double)
#undef MLRS_KM_INST

}  // namespace mlrs
