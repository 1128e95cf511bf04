// radius_neighbors with the Gram contraction on the matrix cores (f32,
// 16 < d <= 128, Euclidean and cosine): the same results as the host-scan
// kernel of knn_radius.hip -- matches in ascending index order per query row,
// values in the reference's host-scan arithmetic (knn_host.rs:693-760,
// radius_host.rs:239-569) -- with the d-long distance loops of every pair
// replaced by a screen.
//
// Shape: a workgroup is 4 waves x 32 query rows (128) and walks one strip of
// index rows 32 at a time, as the fused kNN kernel does (knn_gram_f32.hip):
// the 32-row tile sits in LDS, the next one prefetched into registers under
// the MFMAs, and each wave keeps its 32 query rows as the B operand of
// v_mfma_f32_32x32x2f32.  One tile buffer (two barriers per tile) leaves room
// for three workgroups per CU (52 KB LDS, 168 VGPRs): at c2 with radius 14.8
// that ran the scan in 20.75 ms against 22.11 ms for two double-buffered
// workgroups per CU.
//  * Euclidean: acc = ||x||^2 - 2 x.q; a pair passes when
//    acc <= th - ||q||^2 + eps.  Cosine: acc = x.q scaled by 1/||x|| after the
//    contraction; a pair passes when 1 - acc/||q|| <= th + eps.  eps bounds
//    the expansion's rounding error plus the reference arithmetic's own (the
//    bounds of the fused kNN screen), so every pair whose exact value is
//    <= th passes; NaN passes too.  A query whose squared norm plus the
//    largest index squared norm is not well inside the float range is not
//    screened (every pair is evaluated exactly).
//  * A passing pair is queued in LDS in ascending index order (the two lanes
//    holding a query's tile rows combine their row masks, so each row's place
//    is a popcount).  When a queue could overflow, and at the end of the
//    strip, the wave evaluates all queued pairs exactly, 64 at a time one per
//    lane, in the host arm's operation order; the exact matches (v <= th)
//    take their places with one ballot per batch.
//  * COUNT writes each (strip, query) match count; FILL writes the
//    pre-boundary values and indices at the offsets the count pass produced,
//    never at or past the caller's capacity, and flags a strip whose matches
//    differ from its count.  STAGE counts as COUNT does and also keeps each
//    (strip, query)'s first stage_cap matches, in order, in a staging area
//    (flagging a strip with more), so that a call which already holds its
//    output buffers copies them into place instead of running FILL.
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

constexpr int kWaves = 4;
constexpr int kQpw = 32;               // query rows per wave (MFMA N dimension)
constexpr int kQpb = kWaves * kQpw;    // query rows per workgroup
constexpr int kBn = 32;                // index rows per tile (MFMA M dimension)
constexpr int kQcap = 64;              // queued pairs per query row
constexpr int kFlushAt = kQcap - kBn;  // flush when a queue could overflow on the next tile
constexpr int kWgsPerCu = 3;           // resident workgroups per CU (one wave per SIMD each)

typedef float f32x16 __attribute__((ext_vector_type(16)));

struct RgWaveLds {
    uint32_t qidx[kQpw][kQcap];
    uint32_t off[kQpw + 1];
    uint32_t rel[kQpw];               // matches of each query row in this strip so far
    unsigned long long base[kQpw];    // FILL: first output position of the row's matches in this strip
    float qa[kQpw];                   // cosine: the row's reciprocal norm
};

// The host arm's value of one pair: Euclidean acc + diff*diff, cosine
// clamp(1 - dot*qinv*xinv) with dot = acc + q*x (knn_host.rs:703-708, :750-764).
template <bool COS, bool VEC4>
__device__ __forceinline__ float host_value(const float* __restrict__ q, const float* __restrict__ y, int64_t d,
                                            float qa, float ya) {
    constexpr int ARM = COS ? ARM_COS_HOST : ARM_EUCLID_MULADD;
    if (!VEC4) return exact_pair<float, ARM>(q, y, d, qa, ya);
    const float4* q4 = reinterpret_cast<const float4*>(q);
    const float4* y4 = reinterpret_cast<const float4*>(y);
    const int n4 = (int)(d >> 2);
    float acc = 0.0f;
    constexpr int U = 4;
    int c = 0;
    for (; c < n4; c += U) {
        float4 a[U], b[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            a[u] = (c + u < n4) ? q4[c + u] : make_float4(0.f, 0.f, 0.f, 0.f);
            b[u] = (c + u < n4) ? y4[c + u] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c + u >= n4) break;
            if (!COS) {
                const float d0 = a[u].x - b[u].x, d1 = a[u].y - b[u].y, d2 = a[u].z - b[u].z, d3 = a[u].w - b[u].w;
                acc = acc + d0 * d0;
                acc = acc + d1 * d1;
                acc = acc + d2 * d2;
                acc = acc + d3 * d3;
            } else {
                acc = acc + a[u].x * b[u].x;
                acc = acc + a[u].y * b[u].y;
                acc = acc + a[u].z * b[u].z;
                acc = acc + a[u].w * b[u].w;
            }
        }
    }
    if (COS) return clamp02<float>(1.0f - acc * qa * ya);
    return acc;
}

template <int NG, bool COS, bool VEC4, bool FILL, bool STAGE>
__global__ __launch_bounds__(256, kWgsPerCu) void radius_gram_kernel(RadiusArgs<float> a, float* __restrict__ out_dist,
                                                             int32_t* __restrict__ out_idx) {
    constexpr int DP = NG * 8;        // padded feature count
    constexpr int STRIDE = DP + 4;    // LDS row stride (floats)
    constexpr int TILE_F4 = kBn * DP / 4;
    constexpr int PF = (TILE_F4 + 255) / 256;

    __shared__ __attribute__((aligned(16))) float tile[kBn][STRIDE];
    __shared__ __attribute__((aligned(16))) float tnorm[kBn];
    __shared__ RgWaveLds wl[kWaves];

    const float* __restrict__ Q = a.q;
    const float* __restrict__ X = a.x;
    const float* __restrict__ XNORM = COS ? a.xinv : a.xsq;  // per-row tile scalar
    const int64_t nq = a.nq, nt = a.nt, d = a.d;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int h = lane >> 5;
    const int jl = lane & 31;
    RgWaveLds& L = wl[w];
    const float inf = __builtin_huge_valf();
    const uint64_t below = (1ull << lane) - 1ull;

    // (query block, strip) from the XCD-grouped number of this workgroup:
    // the query blocks of one strip (the same index rows) run on one XCD.
    const int64_t gx = gridDim.x;
    const int64_t gid = xcd_grouped_wg((int64_t)blockIdx.y * gx + blockIdx.x, gx * (int64_t)gridDim.y);
    const int64_t s = gid / gx;
    const int64_t qwave = (gid % gx) * kQpb + w * kQpw;
    const int64_t qmine = qwave + jl;
    const bool qvalid = qmine < nq;
    const int64_t t_begin = s * a.strip_len;
    int64_t t_end = t_begin + a.strip_len;
    if (t_end > nt) t_end = nt;
    const uint32_t t_end32 = (uint32_t)t_end;

    // ---- per-query screen thresholds, counters, output bases.  thr: a pair
    //      whose exact value can be <= th passes it.  thr_lo (count pass): a
    //      pair at or below it is a match for certain (exact <= screen + eps
    //      <= th) and is counted without evaluation; only the pairs between
    //      the two are evaluated. ----
    float thr = -inf, thr_lo = -inf;
    if (qvalid) {
        const float qsq = a.qsq[qmine];
        const bool bounded = (double)qsq + (double)a.stats->xsq_max <= 0x1p124;  // false for NaN / inf too
        double lo = -__builtin_huge_val();
        if (!bounded) {
            thr = inf;
        } else if (!COS) {
            const double eps = a.eps_rel * ((double)qsq + (double)a.stats->xsq_max) + a.eps_abs;
            thr = round_up_f((double)a.th - (double)qsq + eps);
            lo = (double)a.th - (double)qsq - eps;
        } else {
            thr = round_up_f((double)a.th + a.eps_abs);
            lo = (double)a.th - a.eps_abs;
        }
        if (!FILL && lo > -__builtin_huge_val()) thr_lo = -round_up_f(-(lo - __builtin_fabs(lo) * 0x1p-40));
    }
    uint32_t sure = 0u;  // count pass: this lane's certain matches
    if (lane < kQpw) {
        L.rel[lane] = 0u;
        L.qa[lane] = (COS && qvalid) ? a.qinv[qmine] : 0.0f;
        L.base[lane] = (FILL && qvalid) ? a.qoff[qmine] + a.cnt[s * nq + qmine] : 0ull;
    }
    const float qa_mine = (COS && qvalid) ? a.qinv[qmine] : 0.0f;

    // ---- query operand: qreg[g] = scale * q[8g+4h .. 8g+4h+3] ----
    float4 qreg[NG];
    {
        const float scale = COS ? 1.0f : -2.0f;
        const float* qp = Q + qmine * d;
        if (VEC4) {  // one 16-byte load per group, all issued before use
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                const int64_t c = 8 * g + 4 * h;
                qreg[g] = (qvalid && c < d) ? *reinterpret_cast<const float4*>(qp + c) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                qreg[g].x *= scale;
                qreg[g].y *= scale;
                qreg[g].z *= scale;
                qreg[g].w *= scale;
            }
        } else {
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t c = 8 * g + 4 * h + e;
                    v[e] = (qvalid && c < d) ? qp[c] * scale : 0.0f;
                }
                qreg[g] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }

    // ---- tile prefetch into registers: PF fixed 16-byte chunks per thread ----
    int pf_r[PF];
    bool pf_on[PF];
    const float* pf_src[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        const int f = tid + 256 * p;
        pf_r[p] = f / (DP / 4);
        const int c4 = f % (DP / 4);
        pf_on[p] = (f < TILE_F4) && (4 * c4 < d);
        pf_src[p] = X + (t_begin + pf_r[p]) * d + 4 * c4;
    }
    float4 pf[PF];
    float pfn = 0.0f;
    // Whole tiles of rows without padded columns load unconditionally.
    const bool pf_fast = VEC4 && (PF * 256 == TILE_F4) && (d == DP);
#define MLRS_RG_PREFETCH(T0)                                                                 \
    do {                                                                                     \
        const uint32_t t0_ = (uint32_t)(T0);                                                 \
        if (pf_fast && t_end32 - t0_ >= (uint32_t)kBn) { /* not t0 + kBn: no wrap */        \
            _Pragma("unroll") for (int p = 0; p < PF; ++p) {                                 \
                pf[p] = gload4(pf_src[p]);                                                   \
                pf_src[p] += kBn * d;                                                        \
            }                                                                                \
        } else {                                                                             \
        _Pragma("unroll") for (int p = 0; p < PF; ++p) {                                     \
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);                                      \
            const uint32_t t = t0_ + (uint32_t)pf_r[p];                                      \
            if (pf_on[p] && t < t_end32) {                                                   \
                const float* src = pf_src[p];                                                \
                if (VEC4) {                                                                  \
                    v = gload4(src);                                                         \
                } else {                                                                     \
                    const int c0_ = (int)((tid + 256 * p) % (DP / 4)) * 4;                   \
                    float e4[4];                                                             \
                    _Pragma("unroll") for (int e = 0; e < 4; ++e) e4[e] =                    \
                        (c0_ + e < d) ? src[e] : 0.0f;                                       \
                    v = make_float4(e4[0], e4[1], e4[2], e4[3]);                             \
                }                                                                            \
            }                                                                                \
            pf[p] = v;                                                                       \
            pf_src[p] += kBn * d;                                                            \
        }                                                                                    \
        }                                                                                    \
        if (tid < kBn) {                                                                     \
            const uint32_t t = t0_ + (uint32_t)tid;                                          \
            pfn = (t < t_end32) ? XNORM[t] : (COS ? 0.0f : inf);                             \
        }                                                                                    \
    } while (0)

    // ---- flush: every queued pair of the wave evaluated exactly, 64 per
    //      batch; a query's pairs are contiguous and in index order, so a
    //      match's place is its query's count so far plus the ballot popcount
    //      of the query's earlier lanes in the batch ----
#define MLRS_RG_FLUSH()                                                                      \
    do {                                                                                     \
        const uint32_t c_ = (lane < kQpw) ? cntr : 0u;                                       \
        uint32_t incl_ = c_;                                                                 \
        _Pragma("unroll") for (int m_ = 1; m_ < kQpw; m_ <<= 1) {                            \
            const uint32_t o_ = (uint32_t)__shfl_up((int)incl_, m_, 64);                     \
            if ((lane & 31) >= m_) incl_ += o_;                                              \
        }                                                                                    \
        const uint32_t total_ = bcast_u(incl_, kQpw - 1);                                    \
        if (lane < kQpw) L.off[lane] = incl_ - c_;                                           \
        if (lane == 0) L.off[kQpw] = total_;                                                 \
        for (uint32_t b_ = 0; b_ < total_; b_ += 64) {                                       \
            const uint32_t e_ = b_ + (uint32_t)lane;                                         \
            const bool act_ = e_ < total_;                                                   \
            int j_ = 0;                                                                      \
            float v_ = inf;                                                                  \
            uint32_t t_ = 0u;                                                                \
            if (act_) {                                                                      \
                _Pragma("unroll") for (int m_ = 16; m_ >= 1; m_ >>= 1) if (L.off[j_ + m_] <= e_) \
                    j_ += m_;                                                                \
                t_ = L.qidx[j_][e_ - L.off[j_]];                                             \
                v_ = host_value<COS, VEC4>(Q + (qwave + j_) * d, X + (int64_t)t_ * d, d, L.qa[j_], \
                                           COS ? a.xinv[t_] : 0.0f);                         \
            }                                                                                \
            const bool hit_ = act_ && (v_ <= a.th);                                          \
            const uint64_t H_ = __builtin_amdgcn_ballot_w64(hit_);                           \
            uint32_t lo_ = 0u, hi_ = 64u, r0_ = 0u;                                          \
            if (act_) {                                                                      \
                const uint32_t o0_ = L.off[j_], o1_ = L.off[j_ + 1];                         \
                lo_ = (o0_ > b_) ? o0_ - b_ : 0u;                                            \
                hi_ = (o1_ - b_ < 64u) ? o1_ - b_ : 64u;                                     \
                r0_ = L.rel[j_];                                                             \
            }                                                                                \
            const uint64_t from_ = ~((1ull << lo_) - 1ull);                                  \
            if (FILL && hit_) {                                                              \
                const unsigned long long pos_ =                                              \
                    L.base[j_] + r0_ + (unsigned long long)__popcll(H_ & below & from_);     \
                if (pos_ < (unsigned long long)a.capacity) {                                 \
                    out_dist[pos_] = v_;                                                     \
                    out_idx[pos_] = (int32_t)t_;                                             \
                }                                                                            \
            }                                                                                \
            if (STAGE && hit_) {                                                             \
                const uint32_t rk_ = r0_ + (uint32_t)__popcll(H_ & below & from_);           \
                if (rk_ < (uint32_t)a.stage_cap) {                                           \
                    const int64_t so_ = (s * nq + qwave + j_) * a.stage_cap + rk_;           \
                    a.stage_val[so_] = v_;                                                   \
                    a.stage_idx[so_] = (int32_t)t_;                                          \
                }                                                                            \
            }                                                                                \
            if (act_ && (uint32_t)lane == hi_ - 1u) {                                        \
                const uint64_t upto_ = (hi_ >= 64u) ? ~0ull : ((1ull << hi_) - 1ull);        \
                L.rel[j_] = r0_ + (uint32_t)__popcll(H_ & from_ & upto_);                    \
            }                                                                                \
        }                                                                                    \
        cntr = 0u;                                                                           \
    } while (0)

    if (t_begin < t_end) MLRS_RG_PREFETCH(t_begin);
    __syncthreads();  // per-wave LDS state visible to the wave

    uint32_t cntr = 0u;  // queued pairs of query jl (equal in lanes jl and jl + 32)
    for (int64_t t0 = t_begin; t0 < t_end; t0 += kBn) {
        // publish the prefetched tile once every wave is done with the last one
        __syncthreads();
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int f = tid + 256 * p;
            if (f < TILE_F4) {
                const int r = f / (DP / 4);
                const int c4 = f % (DP / 4);
                *reinterpret_cast<float4*>(&tile[r][4 * c4]) = pf[p];
            }
        }
        if (tid < kBn) tnorm[tid] = pfn;
        __syncthreads();
        if (t0 + kBn < t_end) MLRS_RG_PREFETCH(t0 + kBn);

        f32x16 acc;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const float4 n4 = *reinterpret_cast<const float4*>(&tnorm[8 * g4 + 4 * h]);
            acc[4 * g4 + 0] = COS ? 0.0f : n4.x;
            acc[4 * g4 + 1] = COS ? 0.0f : n4.y;
            acc[4 * g4 + 2] = COS ? 0.0f : n4.z;
            acc[4 * g4 + 3] = COS ? 0.0f : n4.w;
        }
        const float* arow = &tile[jl][4 * h];
        float4 av = *reinterpret_cast<const float4*>(arow);
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            float4 an = av;
            if (g + 1 < NG) an = *reinterpret_cast<const float4*>(arow + 8 * (g + 1));
            __builtin_amdgcn_sched_barrier(0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, qreg[g].x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, qreg[g].y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, qreg[g].z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, qreg[g].w, acc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            av = an;
        }

        // ---- screen: lane (jl, h) holds rows 8*(r/4) + 4h + (r%4) of the tile ----
        uint32_t m = 0, dm = 0;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            float sc[4] = {1.f, 1.f, 1.f, 1.f};
            if (COS) {
                const float4 s4 = *reinterpret_cast<const float4*>(&tnorm[8 * g4 + 4 * h]);
                sc[0] = s4.x;
                sc[1] = s4.y;
                sc[2] = s4.z;
                sc[3] = s4.w;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * g4 + e;
                const float wv = COS ? 1.0f - (acc[r] * sc[e]) * qa_mine : acc[r];
                m |= (uint32_t)!(wv > thr) << r;
                if (!FILL && !STAGE) dm |= (uint32_t)(wv <= thr_lo) << r;
            }
        }
        if (!qvalid) m = 0;
        if (t0 + kBn > t_end) {  // partial tile: rows past the strip are not candidates
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if ((uint32_t)t0 + (uint32_t)(8 * (r >> 2) + 4 * h + (r & 3)) >= t_end32) m &= ~(1u << r);
        }
        if (!FILL && !STAGE) {  // staging needs every match's value: no certain-match shortcut
            dm &= m;
            sure += (uint32_t)__builtin_popcount(dm);
            m &= ~dm;
        }
        if (__builtin_amdgcn_ballot_w64(m != 0)) {
            // row-ordered 32-bit mask of the query's passing tile rows
            uint32_t rowm = 0u;
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) rowm |= ((m >> (4 * g4)) & 0xFu) << (8 * g4 + 4 * h);
            const uint32_t full = rowm | shfl_xor_u(rowm, 32);
            while (m) {
                const int r = __builtin_ctz(m);
                m &= m - 1;
                const int rho = 8 * (r >> 2) + 4 * h + (r & 3);
                L.qidx[jl][cntr + (uint32_t)__builtin_popcount(full & ((1u << rho) - 1u))] = (uint32_t)t0 + (uint32_t)rho;
            }
            cntr += (uint32_t)__builtin_popcount(full);
        }
        if (__builtin_amdgcn_ballot_w64(lane < kQpw && cntr > (uint32_t)kFlushAt)) MLRS_RG_FLUSH();
    }
    if (__builtin_amdgcn_ballot_w64(lane < kQpw && cntr > 0u)) MLRS_RG_FLUSH();
#undef MLRS_RG_FLUSH
#undef MLRS_RG_PREFETCH

    // ---- per (strip, query): the count, or the end check of the fill ----
    if (!FILL) sure += shfl_xor_u(sure, 32);  // the query's two lanes
    if (lane < kQpw && qvalid) {
        const uint32_t mine = L.rel[lane] + sure;
        if (!FILL) {
            a.cnt[s * nq + qmine] = mine;
            if (STAGE && mine > (uint32_t)a.stage_cap) atomicOr(a.stage_over, 1u);
        } else {
            const unsigned long long want =
                a.qoff[qmine] + (s + 1 < a.nstrips ? (unsigned long long)a.cnt[(s + 1) * nq + qmine]
                                                   : (unsigned long long)a.row_cnt[qmine]);
            if (L.base[lane] + mine != want) atomicOr(a.mismatch, 1u);
        }
    }
}

template <int NG, bool COS, bool VEC4>
hipError_t launch_rg(const RadiusArgs<float>& a, int mode, hipStream_t s) {
    const dim3 grid((unsigned)((a.nq + kQpb - 1) / kQpb), (unsigned)a.nstrips);
    if (mode == RADIUS_FILL)
        hipLaunchKernelGGL((radius_gram_kernel<NG, COS, VEC4, true, false>), grid, dim3(256), 0, s, a, a.out_dist,
                           a.out_idx);
    else if (mode == RADIUS_STAGE)
        hipLaunchKernelGGL((radius_gram_kernel<NG, COS, VEC4, false, true>), grid, dim3(256), 0, s, a, a.out_dist,
                           a.out_idx);
    else
        hipLaunchKernelGGL((radius_gram_kernel<NG, COS, VEC4, false, false>), grid, dim3(256), 0, s, a, a.out_dist,
                           a.out_idx);
    return hipGetLastError();
}

template <bool COS, bool VEC4>
hipError_t launch_rg_ng(const RadiusArgs<float>& a, int mode, hipStream_t s) {
    const int ng = (int)((a.d + 7) / 8);
    if (ng <= 4) return launch_rg<4, COS, VEC4>(a, mode, s);
    if (ng <= 8) return launch_rg<8, COS, VEC4>(a, mode, s);
    if (ng <= 12) return launch_rg<12, COS, VEC4>(a, mode, s);
    return launch_rg<16, COS, VEC4>(a, mode, s);
}

// The staged matches of every (strip, row) copied to the row's output
// offset plus the strip's in-row prefix: one wave per (strip, row).
__global__ __launch_bounds__(256) void radius_unstage_kernel(RadiusArgs<float> a) {
    const int64_t sq = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // strip * nq + row
    const int lane = threadIdx.x & 63;
    if (sq >= (int64_t)a.nstrips * a.nq) return;
    const int64_t q = sq % a.nq, st = sq / a.nq;
    const uint32_t beg = a.cnt[sq];
    const uint32_t end = (st + 1 < a.nstrips) ? a.cnt[sq + a.nq] : a.row_cnt[q];
    const int64_t n = (int64_t)(end - beg) < a.stage_cap ? (int64_t)(end - beg) : a.stage_cap;
    const unsigned long long base = a.qoff[q] + beg;
    const int64_t src = sq * a.stage_cap;
    for (int64_t r = lane; r < n; r += 64) {
        const unsigned long long pos = base + (unsigned long long)r;
        if (pos < (unsigned long long)a.capacity) {
            a.out_dist[pos] = a.stage_val[src + r];
            a.out_idx[pos] = a.stage_idx[src + r];
        }
    }
}

}  // namespace

bool radius_gram_serves(int arm, int64_t d) {
    return (arm == ARM_EUCLID_MULADD || arm == ARM_COS_HOST) && d > 0 && d <= 128;
}
int64_t radius_gram_rows_per_tile() { return kBn; }
int64_t radius_gram_queries_per_block() { return kQpb; }
int64_t radius_gram_wgs_per_cu() { return kWgsPerCu; }

hipError_t launch_radius_gram(const RadiusArgs<float>& a, int arm, int mode, hipStream_t s) {
    if (a.nq == 0 || a.nstrips == 0) return hipSuccess;
    if (mode == RADIUS_STAGE && (a.stage_cap <= 0 || !a.stage_val || !a.stage_idx || !a.stage_over))
        return hipErrorInvalidValue;
    const bool vec4 = (a.d % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0);
    if (arm == ARM_EUCLID_MULADD)
        return vec4 ? launch_rg_ng<false, true>(a, mode, s) : launch_rg_ng<false, false>(a, mode, s);
    if (arm == ARM_COS_HOST)
        return vec4 ? launch_rg_ng<true, true>(a, mode, s) : launch_rg_ng<true, false>(a, mode, s);
    return hipErrorInvalidValue;
}

hipError_t launch_radius_unstage(const RadiusArgs<float>& a, hipStream_t s) {
    const int64_t n = (int64_t)a.nstrips * a.nq;
    if (n == 0 || a.stage_cap <= 0) return hipSuccess;
    hipLaunchKernelGGL(radius_unstage_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace mlrs
