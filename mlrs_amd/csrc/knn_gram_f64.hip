// Fused f64 Gram-MFMA kNN with exact rescoring (gfx950).
//
// The f64 counterpart of knn_gram_f32.hip: serves every cpu arm
// (direct / metric / knn_host, Euclidean and cosine) for d <= 256, k <= 128,
// replacing the materialized-matrix paths tiled_distance_topk /
// tiled_metric_distance_topk (crates/mlrs-algos/src/neighbors/nearest.rs:
// 1058-1512) and the host scan of knn_host_topk (crates/mlrs-backend/src/
// prims/knn_host.rs:418-851) for f64.
//
// Shape of one workgroup: 4 waves x 16 queries = 64 queries, walking one
// segment of index rows 16 at a time with v_mfma_f64_16x16x4f64.
//  * Lane l of a wave owns query l%16 and lane group g = l/16.  The K
//    dimension is split into four contiguous quarters of NS columns: at
//    k-step s, group g supplies column g*NS + s of both operands, so each
//    lane's A operand is a contiguous run of its tile row (ds_read_b128
//    feeds two k-steps) and its B operand (the query, pre-scaled by -2 for
//    Euclidean) is held in VGPRs for the whole segment.
//  * The MFMA result layout is D[l/16 + 4r][l%16], r = 0..3: lane l scores
//    tile rows g, g+4, g+8, g+12 against its query.
//  * The screen, the per-query queues, the exact rescoring in the reference
//    arm's operation order, the (value, index) lists and the stream-K split
//    with a shared per-query bound are those of the f32 kernel, in double.
// The thresholds are computed in double with a margin for their own
// rounding folded into the error bound (the f32 kernel rounds up in double
// instead).
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

constexpr int kWaves = 4;
constexpr int kQpw = 16;               // queries per wave (MFMA N dimension)
constexpr int kQpb = kWaves * kQpw;    // queries per workgroup
constexpr int kBn = 16;                // index rows per tile (MFMA M dimension)
constexpr int kKcap = 128;             // largest k kept
constexpr int kQcap = 48;              // queued candidates per query (two workgroups still fit a CU's LDS)
constexpr int kFlushAt = kQcap - kBn;  // flush when a queue may overflow on the next tile
constexpr int kShareEvery = 32;        // tiles between reads of the shared bound
constexpr int kMaxD = 256;

typedef double f64x4 __attribute__((ext_vector_type(4)));

struct WaveLds64 {
    uint32_t qidx[kQpw][kQcap];
    double thr[kQpw];
    double qa[kQpw];   // exact arm's query operand (squared or reciprocal norm)
    double qs[kQpw];   // screen operand: ||q||^2 (Euclidean) or ||q|| (cosine)
    double eps[kQpw];  // screen error bound
    uint32_t mode[kQpw];  // 0 = screen-value list, 1 = exact list
};

constexpr unsigned long long kInfBits64 = 0x7FF0000000000000ull;

template <bool COS>
__device__ __forceinline__ double screen_threshold64(double R, double qs, double eps) {
    const double inf = __builtin_huge_val();
    if (!(R < inf)) return inf;
    // Euclidean: R widened by a relative 2^-48, so that every pair whose root
    // equals the root of a value <= R passes too (the X-vs-X graph ranks by
    // the root, and sqrt maps at most a few consecutive doubles to one)
    if (!COS) return ((R + __builtin_fabs(R) * 0x1p-48) - qs) + eps;
    if (qs == 0.0) return inf;  // a zero query ties every row: never screened
    return ((R + eps) - 1.0) * qs;
}

// Exact value of one (query, row) pair in the arm's operation order; loads
// issued U 16-byte pairs at a time when rows are 16-byte aligned (inside the
// Gram kernel U = 2: the d = 256 kernel holds 128 VGPRs of query operand;
// the merge kernel has registers for more in flight).
template <int ARM, bool VEC2, int U = 2>
__device__ __forceinline__ double exact_f64(const double* __restrict__ q, const double* __restrict__ y,
                                            int64_t d, double qa, double ya) {
    if (!VEC2) return exact_pair<double, ARM>(q, y, d, qa, ya);
    const double2* q2 = reinterpret_cast<const double2*>(q);
    const double2* y2 = reinterpret_cast<const double2*>(y);
    const int n2 = (int)(d >> 1);
    double acc = 0.0;
    int c = 0;
    for (; c < n2; c += U) {
        double2 a[U], b[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c + u < n2) {
                a[u] = q2[c + u];
                b[u] = y2[c + u];
            } else {
                a[u] = make_double2(0.0, 0.0);
                b[u] = make_double2(0.0, 0.0);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c + u >= n2) break;
            const double e0a = a[u].x, e1a = a[u].y, e0b = b[u].x, e1b = b[u].y;
            if (ARM == ARM_EUCLID_FMA) {
                const double d0 = e0a - e0b, d1 = e1a - e1b;
                acc = __builtin_fma(d0, d0, acc);
                acc = __builtin_fma(d1, d1, acc);
            } else if (ARM == ARM_EUCLID_MULADD) {
                const double d0 = e0a - e0b, d1 = e1a - e1b;
                acc = acc + d0 * d0;
                acc = acc + d1 * d1;
            } else if (ARM == ARM_COS_FOLD) {
                acc = __builtin_fma(e0a, e0b, acc);
                acc = __builtin_fma(e1a, e1b, acc);
            } else {  // ARM_COS_HOST: mul + add
                acc = acc + e0a * e0b;
                acc = acc + e1a * e1b;
            }
        }
    }
    if (ARM == ARM_COS_FOLD) {
        const double denom = __builtin_sqrt(qa * ya);
        const double sim = (denom > 0.0) ? acc / denom : 0.0;
        return clamp02<double>(1.0 - sim);
    }
    if (ARM == ARM_COS_HOST) return clamp02<double>(1.0 - acc * qa * ya);
    return acc;
}

// KL: 64-entry blocks of a (segment, query) list during a flush (1 for
// k <= 64, 3 for k <= 128: k + 32 entries).
template <int NS, int ARM, bool COS, bool VEC2, int KL>
__global__ __launch_bounds__(256, 2) void knn_gram_f64_kernel(GramArgs64 a) {
    constexpr int DP = 4 * NS;             // padded feature count
    constexpr int STRIDE = DP + 2;         // LDS row stride (doubles): rows 16 bytes apart in the banks
    constexpr int CPT = DP / 2;            // 16-byte column pairs per tile row
    constexpr int RPG = 256 / CPT;         // tile rows one pass of the workgroup loads
    constexpr int PF = kBn / RPG;          // passes per tile
    static_assert(RPG >= 1 && kBn % RPG == 0, "tile fill shape");
    // Rows of whole kilobytes (d padded to 128 or 256) with 16-byte aligned
    // operands load the next tile straight into LDS (global_load_lds_dwordx4:
    // each wave instruction fills one contiguous kilobyte, half or all of a
    // row), so no registers hold it in flight; other shapes stage it through
    // registers.
    constexpr bool DIRECT = VEC2 && (DP % 128 == 0);
    constexpr int KB_PER_ROW = DP >= 128 ? DP / 128 : 1;  // 1 KB wave loads per tile row (DIRECT)
    constexpr int LOADS_PER_WAVE = kBn * KB_PER_ROW / kWaves;

    // The two tile buffers are distinct objects, so the compiler can tell the
    // direct loads into one from the reads of the other.
    __shared__ __attribute__((aligned(16))) double tileA[kBn][STRIDE];
    __shared__ __attribute__((aligned(16))) double tileB[kBn][STRIDE];
    __shared__ __attribute__((aligned(16))) double tnA[kBn];
    __shared__ __attribute__((aligned(16))) double tnB[kBn];
    __shared__ WaveLds64 wl[kWaves];

    const double* __restrict__ Q = a.q;
    const double* __restrict__ X = a.x;
    const double* __restrict__ QSQ = a.qsq;
    const double* __restrict__ XSQ = a.xsq;
    const double* __restrict__ QINV = a.qinv;
    const double* __restrict__ XINV = a.xinv;
    const double* __restrict__ XSCALE = a.xscale;
    unsigned long long* __restrict__ SHARED_R = a.shared_r;
    const int64_t nq = a.nq, nt = a.nt, d = a.d;
    const int k = a.k;
    const int K2 = gram_list_cap(k);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: tile rows and LDS slots in SGPRs
    const int g = lane >> 4;   // lane group: K quarter / first tile row of the lane
    const int jl = lane & 15;  // query of the lane within the wave
    WaveLds64& L = wl[w];
    const double inf = __builtin_huge_val();
    // screen values of this wave's queued pairs, [query][queue position]
    double* __restrict__ QVw = a.qval + ((int64_t)blockIdx.x * kWaves + w) * (kQpw * kQcap);

    // ---- work split (StreamSplit), as in the f32 kernel ----
    const StreamSplit sp(nq, nt, kQpb, kBn, a.grid_wgs);
    const int64_t wg = xcd_grouped_wg(blockIdx.x, gridDim.x);
    const int64_t u_hi = ((wg + 1) * sp.P < sp.T) ? (wg + 1) * sp.P : sp.T;
    for (int64_t u = wg * sp.P; u < u_hi;) {
    int64_t panel, qblock, tile0, left;
    sp.decode(u, panel, qblock, tile0, left);
    const int64_t tile1 = tile0 + ((left < u_hi - u) ? left : (u_hi - u));
    const int64_t slot = sp.slot(wg, panel, qblock);
    double* __restrict__ LV = a.part_val + slot * nq * K2;
    uint32_t* __restrict__ LI = a.part_idx + slot * nq * K2;

    const int64_t qwave = qblock * kQpb + w * kQpw;
    const int64_t qmine = qwave + jl;
    const bool qvalid = qmine < nq;
    const int64_t t_begin = tile0 * kBn;
    int64_t t_end = tile1 * kBn;
    if (t_end > nt) t_end = nt;
    const uint32_t t_end32 = (uint32_t)t_end;

    uint32_t cntr = 0u;  // queued candidates of query jl (equal in the four lanes of the query)
    if (lane < kQpw) {
        const double qsq = qvalid ? QSQ[qmine] : 0.0;
        L.thr[lane] = qvalid ? inf : -inf;
        if (!COS) {
            L.qs[lane] = qsq;
            L.qa[lane] = 0.0;
            L.eps[lane] = a.eps_rel * (qsq + a.stats->xsq_max64) + a.eps_abs;
        } else {
            L.qs[lane] = __builtin_sqrt(qsq);
            L.qa[lane] = (ARM == ARM_COS_HOST) ? (qvalid ? QINV[qmine] : 0.0) : qsq;
            L.eps[lane] = a.eps_abs;
        }
        // Screen-value lists need |screen distance - exact| <= eps for every
        // pair: norms well inside the double range (a nonzero query for
        // cosine), and k > 1 (a one-entry list has no room for near ties).
        bool sv = qvalid && k > 1 && (qsq + a.stats->xsq_max64 <= 0x1p1020) && (L.eps[lane] < inf);
        if (COS) sv = sv && (L.qs[lane] > 0.0);
        L.mode[lane] = sv ? 0u : 1u;
    }
    for (int j = 0; j < kQpw; ++j) {
        const int64_t qg = qwave + j;
#pragma unroll
        for (int r = 0; r < KL; ++r) {
            const int p = 64 * r + lane;
            if (qg < nq && p < K2) {
                LV[qg * K2 + p] = inf;
                LI[qg * K2 + p] = kSentinelIdx;
            }
        }
    }
    if (SHARED_R && lane < kQpw && qvalid) {
        const double R0 = __longlong_as_double((long long)SHARED_R[qmine]);
        L.thr[lane] = fmin(L.thr[lane], screen_threshold64<COS>(R0, L.qs[lane], L.eps[lane]));
    }

    // ---- query operand: qreg[s] = scale * q[g*NS + s] ----
    double qreg[NS];
    {
        const double scale = COS ? 1.0 : -2.0;
        const double* qp = Q + qmine * d;
        if (VEC2) {  // 16-byte loads, all issued before use (NS and d even)
#pragma unroll
            for (int s = 0; s < NS; s += 2) {
                const int64_t c = (int64_t)g * NS + s;
                const double2 v = (qvalid && c < d) ? *reinterpret_cast<const double2*>(qp + c) : make_double2(0.0, 0.0);
                qreg[s] = v.x;
                qreg[s + 1] = v.y;
            }
#pragma unroll
            for (int s = 0; s < NS; ++s) qreg[s] *= scale;
        } else {
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const int64_t c = (int64_t)g * NS + s;
                qreg[s] = (qvalid && c < d) ? qp[c] * scale : 0.0;
            }
        }
    }

    // ---- tile prefetch into registers.  Thread tid owns column pair c2 =
    //      tid % CPT of rows r0 + RPG*p (r0 = tid / CPT), p < PF: one walking
    //      row pointer, constant row and LDS offsets. ----
    const int pc2 = tid % CPT;
    const int pr0 = tid / CPT;
    const bool pon = (pr0 < RPG) && (2 * pc2 < d);
    const double* pfp = X + (t_begin + pr0) * d + 2 * pc2;
    const int64_t prow = (int64_t)RPG * d;  // elements between a thread's rows
    double2 pf[PF];
    double pfn = 0.0;
#define MLRS_PREFETCH64(T0)                                                                  \
    do {                                                                                     \
        const uint32_t t0_ = (uint32_t)(T0);                                                 \
        _Pragma("unroll") for (int p = 0; p < PF; ++p) {                                     \
            double2 v = make_double2(0.0, 0.0);                                              \
            const uint32_t t = t0_ + (uint32_t)(pr0 + RPG * p);                              \
            if (pon && t < t_end32) {                                                        \
                const double* src = pfp + p * prow;                                          \
                if (VEC2) {                                                                  \
                    v = *reinterpret_cast<const double2*>(src);                              \
                } else {                                                                     \
                    v.x = src[0];                                                            \
                    v.y = (2 * pc2 + 1 < d) ? src[1] : 0.0;                                  \
                }                                                                            \
            }                                                                                \
            pf[p] = v;                                                                       \
        }                                                                                    \
        pfp += kBn * d;                                                                      \
        if (tid < kBn) {                                                                     \
            const uint32_t t = t0_ + (uint32_t)tid;                                          \
            if (COS)                                                                         \
                pfn = (t < t_end32) ? XSCALE[t] : 0.0;                                       \
            else                                                                             \
                pfn = (t < t_end32) ? XSQ[t] : inf;                                          \
        }                                                                                    \
    } while (0)

// Flush: one query's queue sorted and merged into its list.  Screen-value
// mode: a queued pair enters with its screen value mapped back to a
// distance, within eps of its exact value; the list keeps the K2 smallest and
// the segment's bound is its k-th + eps.  A pair whose screen value is NaN,
// and every pair of an exact-mode query, is evaluated exactly in the arm's
// operation order.  When a discarded pair lies within 2 eps of the k-th, the
// old list and the queue are re-evaluated exactly and the query's list stays
// exact from then on.
#define MLRS_EXACT64_AT(T_)                                                                  \
    exact_f64<ARM, VEC2>(Q + qg_ * d, X + (int64_t)(T_) * d, d, L.qa[j_],                    \
                         (ARM == ARM_COS_FOLD) ? XSQ[(T_)] : (ARM == ARM_COS_HOST) ? XINV[(T_)] : 0.0)
#define MLRS_FLUSH64(J)                                                                      \
    do {                                                                                     \
        const int j_ = (J);                                                                  \
        const int64_t qg_ = qwave + j_;                                                      \
        const uint32_t n_ = bcast_u(cntr, j_);                                                \
        const bool exact_ = L.mode[j_] != 0u;                                                \
        double lv_[KL];                                                                      \
        uint32_t li_[KL];                                                                    \
        _Pragma("unroll") for (int r_ = 0; r_ < KL; ++r_) {                                  \
            const int p_ = 64 * r_ + lane;                                                   \
            lv_[r_] = (p_ < K2) ? LV[qg_ * K2 + p_] : inf;                                   \
            li_[r_] = (p_ < K2) ? LI[qg_ * K2 + p_] : kSentinelIdx;                          \
        }                                                                                    \
        double e_ = inf;                                                                     \
        uint32_t t_ = kSentinelIdx;                                                          \
        if ((uint32_t)lane < n_) {                                                           \
            t_ = L.qidx[j_][lane];                                                           \
            const double s_ = exact_ ? 0.0 : QVw[j_ * kQcap + lane];                         \
            if (exact_ || s_ != s_)                                                          \
                e_ = MLRS_EXACT64_AT(t_);                                                    \
            else                                                                             \
                e_ = COS ? 1.0 + s_ / L.qs[j_] : s_ + L.qs[j_];                              \
            if (e_ != e_) {                                                                  \
                e_ = inf;                                                                    \
                t_ = kSentinelIdx;                                                           \
            }                                                                                \
        }                                                                                    \
        wave_sort64<double>(e_, t_, lane);                                                   \
        const uint32_t oi_ = li_[0];                                                         \
        double dm_;                                                                          \
        if constexpr (KL == 1)                                                               \
            dm_ = wave_merge64_drop<double>(lv_[0], li_[0], e_, t_, lane);                   \
        else                                                                                 \
            dm_ = wave_merge_blocks_drop<double, KL>(lv_, li_, e_, t_, lane);                \
        double R_ = list_value_at<double, KL>(lv_, k - 1);                                   \
        /* the smallest exact value the list drops (exact lists only) */                     \
        double dx_ = exact_ ? ((K2 < 64 * KL) ? list_value_at<double, KL>(lv_, K2) : dm_) : inf; \
        if (!exact_) {                                                                       \
            const double dr_ = (K2 < 64 * KL) ? list_value_at<double, KL>(lv_, K2) : dm_;    \
            double w_ = R_ + 2.0 * L.eps[j_];                                                \
            w_ += __builtin_fabs(w_) * 0x1p-40;                                              \
            if (dr_ < inf && dr_ <= w_) {                                                    \
              if constexpr (KL == 1) {                                                       \
                double x1_ = inf, x2_ = inf;                                                 \
                uint32_t i1_ = oi_, i2_ = t_;                                                \
                if (i1_ != kSentinelIdx) x1_ = MLRS_EXACT64_AT(i1_);                         \
                if (i2_ != kSentinelIdx) x2_ = MLRS_EXACT64_AT(i2_);                         \
                if (x1_ != x1_) { x1_ = inf; i1_ = kSentinelIdx; }                           \
                if (x2_ != x2_) { x2_ = inf; i2_ = kSentinelIdx; }                           \
                wave_sort64<double>(x1_, i1_, lane);                                         \
                wave_sort64<double>(x2_, i2_, lane);                                         \
                dx_ = wave_merge64_drop<double>(x1_, i1_, x2_, i2_, lane);                   \
                lv_[0] = x1_;                                                                \
                li_[0] = i1_;                                                                \
              } else {                                                                       \
                /* the old list (still in memory) and the queue, exactly */                  \
                _Pragma("unroll") for (int r_ = 0; r_ < KL; ++r_) {                          \
                    lv_[r_] = inf;                                                           \
                    li_[r_] = kSentinelIdx;                                                  \
                }                                                                            \
                _Pragma("unroll") for (int r_ = 0; r_ <= KL; ++r_) {                         \
                    uint32_t i_ = kSentinelIdx;                                              \
                    if (r_ < KL) {                                                           \
                        const int p_ = 64 * r_ + lane;                                       \
                        if (p_ < K2) i_ = LI[qg_ * K2 + p_];                                 \
                    } else if ((uint32_t)lane < n_) {                                        \
                        i_ = L.qidx[j_][lane];                                               \
                    }                                                                        \
                    double x_ = inf;                                                         \
                    if (i_ != kSentinelIdx) x_ = MLRS_EXACT64_AT(i_);                        \
                    if (x_ != x_) { x_ = inf; i_ = kSentinelIdx; }                           \
                    wave_sort64<double>(x_, i_, lane);                                       \
                    dx_ = fmin(dx_, wave_merge_blocks_drop<double, KL>(lv_, li_, x_, i_, lane)); \
                }                                                                            \
              }                                                                              \
                if (K2 < 64 * KL) dx_ = fmin(dx_, list_value_at<double, KL>(lv_, K2));       \
                R_ = list_value_at<double, KL>(lv_, k - 1);                                  \
                if (lane == 0) L.mode[j_] = 1u;                                              \
            } else if (R_ < inf) {                                                           \
                R_ = R_ + L.eps[j_];                                                         \
            }                                                                                \
        }                                                                                    \
        _Pragma("unroll") for (int r_ = 0; r_ < KL; ++r_) {                                  \
            const int p_ = 64 * r_ + lane;                                                   \
            if (p_ < K2) {                                                                   \
                LV[qg_ * K2 + p_] = lv_[r_];                                                 \
                LI[qg_ * K2 + p_] = li_[r_];                                                 \
            }                                                                                \
        }                                                                                    \
        /* a dropped exact value whose root may equal the k-th's: the merge */               \
        /* cannot rank that root's ties by index, the root fill will */                      \
        if (a.root_flag && lane == 0 && dx_ < inf && dx_ <= R_ + __builtin_fabs(R_) * 0x1p-48) \
            a.root_flag[qg_] = 1u;                                                           \
        if (lane == 0) {                                                                     \
            if (SHARED_R && R_ < inf && R_ >= 0.0) {                                         \
                const unsigned long long old_ =                                              \
                    atomicMin(&SHARED_R[qg_], (unsigned long long)__double_as_longlong(R_)); \
                R_ = fmin(R_, __longlong_as_double((long long)old_));                        \
            }                                                                                \
            L.thr[j_] = fmin(L.thr[j_], screen_threshold64<COS>(R_, L.qs[j_], L.eps[j_]));   \
        }                                                                                    \
        if (jl == j_) cntr = 0u;                                                             \
    } while (0)

#define MLRS_STORE64(DST, TN)                                                                \
    do {                                                                                     \
        if (pr0 < RPG) {                                                                     \
            double* dst_ = &(DST)[pr0][2 * pc2];                                             \
            _Pragma("unroll") for (int p = 0; p < PF; ++p)                                   \
                *reinterpret_cast<double2*>(dst_ + p * RPG * STRIDE) = pf[p];                \
        }                                                                                    \
        if (tid < kBn) (TN)[tid] = pfn;                                                      \
    } while (0)

    // Direct loads of tile T0's rows into DST: wave w fills kilobytes
    // w*LOADS_PER_WAVE + i of the tile (row kb / KB_PER_ROW, its half kb %
    // KB_PER_ROW); a row past the segment is not loaded (its values are masked
    // out of the screen).  The row norms go through a register as in the
    // staged path.
    auto direct_load = [&](double (&dst)[kBn][STRIDE], uint32_t t0) {
        if constexpr (DIRECT) {
            // the row (and kilobyte) of each load is wave-uniform: a scalar
            // base plus the lane's 16-byte offset.  A whole tile of rows
            // without padded columns loads unconditionally (t0 + kBn could
            // wrap, so the rows left are compared).
            if (t_end32 - t0 >= (uint32_t)kBn && d == DP) {
#pragma unroll
                for (int i = 0; i < LOADS_PER_WAVE; ++i) {
                    const int kb = w * LOADS_PER_WAVE + i;
                    const int r = kb / KB_PER_ROW, half = kb % KB_PER_ROW;
                    const double* row = X + ((int64_t)(t0 + (uint32_t)r) * d + half * 128);
                    global_to_lds16(row + 2 * lane, &dst[r][half * 128]);
                }
            } else {
#pragma unroll
                for (int i = 0; i < LOADS_PER_WAVE; ++i) {
                    const int kb = w * LOADS_PER_WAVE + i;
                    const int r = kb / KB_PER_ROW, half = kb % KB_PER_ROW;
                    const double* row = X + ((int64_t)(t0 + (uint32_t)r) * d + half * 128);
                    if (t0 + (uint32_t)r < t_end32 && half * 128 + 2 * lane < d)
                        global_to_lds16(row + 2 * lane, &dst[r][half * 128]);
                }
            }
        }
        if (tid < kBn) {
            const uint32_t t = t0 + (uint32_t)tid;
            if (COS)
                pfn = (t < t_end32) ? XSCALE[t] : 0.0;
            else
                pfn = (t < t_end32) ? XSQ[t] : inf;
        }
    };
    if (DIRECT && d < DP) {
        // columns past d are never loaded: zero them once in both buffers
        // (they meet the query operand's zeros, and garbage could be NaN)
        const int pad = (int)(DP - d);
        for (int e = tid; e < kBn * pad; e += 256) {
            tileA[e / pad][d + e % pad] = 0.0;
            tileB[e / pad][d + e % pad] = 0.0;
        }
    }

    // The next tile is loaded (into registers, or straight into the other LDS
    // buffer) before this tile's MFMAs; staged registers are stored into the
    // other buffer right after them, so they are free again during the screen
    // and the rescoring.
    if (t_begin < t_end) {
        if (DIRECT) {
            direct_load(tileA, (uint32_t)t_begin);
            if (tid < kBn) tnA[tid] = pfn;
        } else {
            MLRS_PREFETCH64(t_begin);
            MLRS_STORE64(tileA, tnA);
        }
    }

    double thr = L.thr[jl];
    int tiles = 0;
    auto tile_step = [&](double (&cur)[kBn][STRIDE], double* tncur, double (&nxt)[kBn][STRIDE], double* tnnxt,
                         int64_t t0) {
        // this wave's direct loads into cur are done; the barrier makes every
        // wave's visible and ends every wave's reads of nxt
        if (DIRECT) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        const bool more = t0 + kBn < t_end;
        if (more) {
            if (DIRECT)
                direct_load(nxt, (uint32_t)(t0 + kBn));
            else
                MLRS_PREFETCH64(t0 + kBn);
        }

        // two accumulator chains (even and odd k-steps): one dependent chain
        // of f64 MFMAs leaves the matrix unit idle between its instructions
        f64x4 acc0, acc1;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            acc0[r] = COS ? 0.0 : tncur[g + 4 * r];
            acc1[r] = 0.0;
        }
        // A operand: this lane's tile row jl, columns g*NS + s; one 16-byte
        // read feeds two k-steps, the next pair is read one step ahead.
        const double* arow = &cur[jl][g * NS];
        double2 av = *reinterpret_cast<const double2*>(arow);
#pragma unroll
        for (int p = 0; p < NS / 2; ++p) {
            double2 an = av;
            if (p + 1 < NS / 2) an = *reinterpret_cast<const double2*>(arow + 2 * (p + 1));
            __builtin_amdgcn_sched_barrier(0);
            acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64(av.x, qreg[2 * p], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64(av.y, qreg[2 * p + 1], acc1, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            av = an;
        }
        f64x4 acc;
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = acc0[r] + acc1[r];
        if (COS) {
            // rows scaled by -1/||x_t|| after the contraction (the scales ride
            // in tnorm), so the prefetched loads need no arithmetic until the
            // LDS store after the MFMAs
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] *= tncur[g + 4 * r];
        }
        if (more) {
            if (DIRECT) {
                if (tid < kBn) tnnxt[tid] = pfn;
            } else {
                MLRS_STORE64(nxt, tnnxt);
            }
        }

        // ---- screen: lane holds tile rows g + 4r for query jl ----
        uint32_t m = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) m |= (uint32_t)!(acc[r] > thr) << r;
        if (!qvalid) m = 0;
        if (t0 + kBn > t_end) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if ((uint32_t)t0 + (uint32_t)(g + 4 * r) >= t_end32) m &= ~(1u << r);
        }
        if (__builtin_amdgcn_ballot_w64(m != 0)) {
            // the query's four lanes (groups 0..3) append in group order
            const uint32_t c = (uint32_t)__builtin_popcount(m);
            // the counts of the query's other three lanes: groups g^1, g^2, g^3
            const uint32_t x1 = shfl_xor_u(c, 16), x2 = shfl_xor_u(c, 32), x3 = shfl_xor_u(x1, 32);
            const uint32_t c0 = (g == 0) ? c : (g == 1) ? x1 : (g == 2) ? x2 : x3;
            const uint32_t c1 = (g == 1) ? c : (g == 0) ? x1 : (g == 3) ? x2 : x3;
            const uint32_t c2 = (g == 2) ? c : (g == 3) ? x1 : (g == 0) ? x2 : x3;
            const uint32_t c3 = (g == 3) ? c : (g == 2) ? x1 : (g == 1) ? x2 : x3;
            uint32_t pos = cntr + (g > 0 ? c0 : 0u) + (g > 1 ? c1 : 0u) + (g > 2 ? c2 : 0u);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (m & (1u << r)) {
                    L.qidx[jl][pos] = (uint32_t)t0 + (uint32_t)(g + 4 * r);
                    QVw[jl * kQcap + pos] = acc[r];
                    ++pos;
                }
            }
            cntr += c0 + c1 + c2 + c3;
        }
        uint64_t mask = __builtin_amdgcn_ballot_w64(lane < kQpw && cntr > (uint32_t)kFlushAt);
        if (mask) {
            if (lane < kQpw) L.thr[lane] = fmin(L.thr[lane], thr);
            // the queued screen values were stored by other lanes of this wave
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            while (mask) {
                const int j = __builtin_ctzll(mask);
                mask &= mask - 1;
                MLRS_FLUSH64(j);
            }
            thr = L.thr[jl];
        }
        rotate_wave_priority((uint32_t)tiles + 1u, 2);
        if (SHARED_R && (++tiles % kShareEvery) == 0) {
            if (lane < kQpw && qvalid) {
                const double R = __longlong_as_double((long long)SHARED_R[qmine]);
                L.thr[lane] = fmin(fmin(L.thr[lane], thr), screen_threshold64<COS>(R, L.qs[lane], L.eps[lane]));
            }
            thr = L.thr[jl];
        }
    };
    for (int64_t t0 = t_begin; t0 < t_end;) {
        tile_step(tileA, tnA, tileB, tnB, t0);
        t0 += kBn;
        if (t0 >= t_end) break;
        tile_step(tileB, tnB, tileA, tnA, t0);
        t0 += kBn;
    }
    {
        uint64_t mask = __builtin_amdgcn_ballot_w64(lane < kQpw && cntr > 0u);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        while (mask) {
            const int j = __builtin_ctzll(mask);
            mask &= mask - 1;
            MLRS_FLUSH64(j);
        }
    }
#undef MLRS_FLUSH64
#undef MLRS_EXACT64_AT
#undef MLRS_STORE64
#undef MLRS_PREFETCH64
    u += tile1 - tile0;
    __syncthreads();  // LDS state and tile buffers are reused by the next segment
    }
}

// Merge the per-segment lists of one query per wave and emit the output
// transform (boundary sqrt, identity, or the k-means pair with the centre-0
// NaN rule of argmin_dist_rows, crates/mlrs-kernels/src/kmeans.rs:284-310).
// Every list entry's value lies within eps of its pair's exact value (exact
// entries equal it) and the segments hold disjoint index rows, so with V the
// k-th smallest value over all lists a pair can be among the k best only if
// its value is <= V + 2 eps: exactly those pairs are evaluated in the arm's
// operation order and ranked by (exact value, index), NaN never admitted.
// EMIT_ROOT_RANKED ranks by (sqrt(exact value), index) instead: every pair
// whose root equals the k-th root lies within V + 2 eps too (its aggregate
// exceeds the k-th by a relative 2^-50 at most), and the kernel's screen and
// drops keep all of them listed unless root_flag says otherwise.
template <int ARM, bool VEC2>
__global__ __launch_bounds__(256) void knn_merge_f64_kernel(GramArgs64 a) {
    __shared__ uint32_t cand[4][128];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int64_t qg = (int64_t)blockIdx.x * 4 + wv;
    if (qg >= a.nq) return;
    const int k = a.k;
    const int K2 = gram_list_cap(k);
    const int64_t d = a.d;
    const double inf = __builtin_huge_val();
    const StreamSplit sp(a.nq, a.nt, kQpb, kBn, a.grid_wgs);
    const int64_t nsl = sp.slots_of(qg / kQpb);
    double uv = inf;
    uint32_t ui = kSentinelIdx;
    for (int64_t s = 0; s < nsl; ++s) {
        double v = inf;
        uint32_t ix = kSentinelIdx;
        if (lane < K2) {
            const int64_t o = (s * a.nq + qg) * K2 + lane;
            v = a.part_val[o];
            ix = a.part_idx[o];
        }
        wave_merge64<double>(uv, ui, v, ix, lane);
    }
    const double qsq = a.qsq[qg];
    const bool cos = (ARM == ARM_COS_FOLD || ARM == ARM_COS_HOST);
    const double eps = cos ? a.eps_abs : a.eps_rel * (qsq + a.stats->xsq_max64) + a.eps_abs;
    double W = bcast_f(uv, k - 1) + 2.0 * eps;
    W += __builtin_fabs(W) * 0x1p-40;
    const double qa = (ARM == ARM_COS_HOST) ? a.qinv[qg] : qsq;
    double lv = inf;
    uint32_t li = kSentinelIdx;
    uint32_t nc = 0;
    auto evaluate = [&](uint32_t count) {
        double e = inf;
        uint32_t t = kSentinelIdx;
        if ((uint32_t)lane < count) {
            t = cand[wv][lane];
            const double ya = (ARM == ARM_COS_FOLD) ? a.xsq[t] : (ARM == ARM_COS_HOST) ? a.xinv[t] : 0.0;
            e = exact_f64<ARM, VEC2, 8>(a.q + qg * d, a.x + (int64_t)t * d, d, qa, ya);
            if (e != e) {
                e = inf;
                t = kSentinelIdx;
            } else if (a.mode == EMIT_ROOT_RANKED) {
                e = __builtin_sqrt(e);  // ranked by (root, index)
            }
        }
        wave_sort64<double>(e, t, lane);
        wave_merge64<double>(lv, li, e, t, lane);
    };
    for (int64_t s = 0; s < nsl; ++s) {
        bool in = false;
        uint32_t ix = kSentinelIdx;
        if (lane < K2) {
            const int64_t o = (s * a.nq + qg) * K2 + lane;
            ix = a.part_idx[o];
            in = (ix != kSentinelIdx) && !(a.part_val[o] > W);
        }
        const uint64_t bal = __builtin_amdgcn_ballot_w64(in);
        const uint32_t pre = (uint32_t)__builtin_popcountll(bal & ((1ull << lane) - 1ull));
        if (in) cand[wv][nc + pre] = ix;
        nc += (uint32_t)__builtin_popcountll(bal);
        if (nc >= 64) {
            evaluate(64);
            const uint32_t rest = nc - 64;
            const uint32_t mv = ((uint32_t)lane < rest) ? cand[wv][64 + lane] : 0u;
            if ((uint32_t)lane < rest) cand[wv][lane] = mv;
            nc = rest;
        }
    }
    if (nc > 0) evaluate(nc);
    if (lane < k) {
        const int64_t o = qg * k + lane;
        if (a.mode == EMIT_KMEANS) {
            if (!(a.qsq[qg] < inf) || !(a.xsq[0] < inf)) {
                const double e0 = exact_pair<double, ARM_EUCLID_MULADD>(a.q + qg * a.d, a.x, a.d, 0.0, 0.0);
                if (e0 != e0) {
                    lv = e0;
                    li = 0;
                }
            }
            a.out_val[o] = lv;
        } else {
            a.out_val[o] = (a.mode == EMIT_SQRT) ? __builtin_sqrt(lv) : lv;
        }
        a.out_idx[o] = (li == kSentinelIdx) ? 0u : li;
    }
}

// 64 < k <= 128: the same merge over lists of up to three 64-entry blocks
// (k + 32 entries); the union and the result are two-block lists (the k
// smallest fit in 128 entries), merged block by block.  k-means assignment
// (k = 1) never comes here, so the output transform is the root or identity.
template <int ARM, bool VEC2>
__global__ __launch_bounds__(256) void knn_merge_blocks_f64_kernel(GramArgs64 a) {
    constexpr int SLB = 3;  // blocks of a segment list
    constexpr int UB = 2;   // blocks of the union and of the result
    __shared__ uint32_t cand[4][128];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int64_t qg = (int64_t)blockIdx.x * 4 + wv;
    if (qg >= a.nq) return;
    const int k = a.k;
    const int K2 = gram_list_cap(k);
    const int64_t d = a.d;
    const double inf = __builtin_huge_val();
    const StreamSplit sp(a.nq, a.nt, kQpb, kBn, a.grid_wgs);
    const int64_t nsl = sp.slots_of(qg / kQpb);
    double uv[UB];
    uint32_t ui[UB];
#pragma unroll
    for (int r = 0; r < UB; ++r) {
        uv[r] = inf;
        ui[r] = kSentinelIdx;
    }
    for (int64_t s = 0; s < nsl; ++s) {
#pragma unroll
        for (int r = 0; r < SLB; ++r) {
            if (64 * r >= K2) break;
            const int p = 64 * r + lane;
            double v = inf;
            uint32_t ix = kSentinelIdx;
            if (p < K2) {
                const int64_t o = (s * a.nq + qg) * K2 + p;
                v = a.part_val[o];
                ix = a.part_idx[o];
            }
            wave_merge_blocks<double, UB>(uv, ui, v, ix, lane);
        }
    }
    const double qsq = a.qsq[qg];
    const bool cos = (ARM == ARM_COS_FOLD || ARM == ARM_COS_HOST);
    const double eps = cos ? a.eps_abs : a.eps_rel * (qsq + a.stats->xsq_max64) + a.eps_abs;
    double W = list_value_at<double, UB>(uv, k - 1) + 2.0 * eps;
    W += __builtin_fabs(W) * 0x1p-40;
    const double qa = (ARM == ARM_COS_HOST) ? a.qinv[qg] : qsq;
    double lv[UB];
    uint32_t li[UB];
#pragma unroll
    for (int r = 0; r < UB; ++r) {
        lv[r] = inf;
        li[r] = kSentinelIdx;
    }
    uint32_t nc = 0;
    auto evaluate = [&](uint32_t count) {
        double e = inf;
        uint32_t t = kSentinelIdx;
        if ((uint32_t)lane < count) {
            t = cand[wv][lane];
            const double ya = (ARM == ARM_COS_FOLD) ? a.xsq[t] : (ARM == ARM_COS_HOST) ? a.xinv[t] : 0.0;
            e = exact_f64<ARM, VEC2, 8>(a.q + qg * d, a.x + (int64_t)t * d, d, qa, ya);
            if (e != e) {
                e = inf;
                t = kSentinelIdx;
            } else if (a.mode == EMIT_ROOT_RANKED) {
                e = __builtin_sqrt(e);  // ranked by (root, index)
            }
        }
        wave_sort64<double>(e, t, lane);
        wave_merge_blocks<double, UB>(lv, li, e, t, lane);
    };
    for (int64_t s = 0; s < nsl; ++s) {
        for (int r = 0; r < SLB; ++r) {
            if (64 * r >= K2) break;
            const int p = 64 * r + lane;
            bool in = false;
            uint32_t ix = kSentinelIdx;
            if (p < K2) {
                const int64_t o = (s * a.nq + qg) * K2 + p;
                ix = a.part_idx[o];
                in = (ix != kSentinelIdx) && !(a.part_val[o] > W);
            }
            const uint64_t bal = __builtin_amdgcn_ballot_w64(in);
            const uint32_t pre = (uint32_t)__builtin_popcountll(bal & ((1ull << lane) - 1ull));
            if (in) cand[wv][nc + pre] = ix;
            nc += (uint32_t)__builtin_popcountll(bal);
            if (nc >= 64) {
                evaluate(64);
                const uint32_t rest = nc - 64;
                const uint32_t mv = ((uint32_t)lane < rest) ? cand[wv][64 + lane] : 0u;
                if ((uint32_t)lane < rest) cand[wv][lane] = mv;
                nc = rest;
            }
        }
    }
    if (nc > 0) evaluate(nc);
#pragma unroll
    for (int r = 0; r < UB; ++r) {
        const int slot = 64 * r + lane;
        if (slot < k) {
            const int64_t o = qg * k + slot;
            a.out_val[o] = (a.mode == EMIT_SQRT) ? __builtin_sqrt(lv[r]) : lv[r];
            a.out_idx[o] = (li[r] == kSentinelIdx) ? 0u : li[r];
        }
    }
}

// EMIT_ROOT_RANKED, queries with root_flag set (an exact list dropped a pair
// whose root may equal the k-th root, so ties of that root may be missing
// from the merge): the emitted row keeps its m entries below the k-th root
// r (all pairs with a smaller root: their aggregates are below the k-th, so
// the merge saw them) and slots m..k-1 get r with the lowest-index rows whose
// root is r, found by evaluating every index row in ascending order, 64 at a
// time (one wave per query; unflagged queries return at once).  This is the
// host scan's KNearest order (crates/mlrs-algos/src/manifold/
// umap_host_knn.rs:171-198): (root, index).
template <int ARM, bool VEC2>
__global__ __launch_bounds__(256) void knn_root_fill_f64_kernel(GramArgs64 a) {
    const int lane = threadIdx.x & 63;
    const int64_t qg = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (qg >= a.nq || a.root_flag[qg] == 0u) return;
    const int k = a.k;
    double* ov = a.out_val + qg * k;
    uint32_t* oi = a.out_idx + qg * k;
    const double r = ov[k - 1];
    if (!(r < __builtin_huge_val())) return;
    uint32_t m = 0;
    for (int j0 = 0; j0 < k; j0 += 64)
        m += (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(j0 + lane < k && ov[j0 + lane] < r));
    const uint32_t need = (uint32_t)k - m;
    const int64_t d = a.d;
    uint32_t found = 0;
    for (int64_t t0 = 0; t0 < a.nt && found < need; t0 += 64) {
        const int64_t t = t0 + lane;
        bool hit = false;
        if (t < a.nt) {
            const double e = exact_f64<ARM, VEC2, 8>(a.q + qg * d, a.x + t * d, d, 0.0, 0.0);
            hit = (e == e) && __builtin_sqrt(e) == r;
        }
        const uint64_t bal = __builtin_amdgcn_ballot_w64(hit);
        const uint32_t pos = found + (uint32_t)__builtin_popcountll(bal & ((1ull << lane) - 1ull));
        if (hit && pos < need) {
            ov[m + pos] = r;
            oi[m + pos] = (uint32_t)t;
        }
        found += (uint32_t)__builtin_popcountll(bal);
    }
}

// Initial per-query bound: the k-th smallest exact value over an evenly
// spaced sample of index rows (seed_kth_block): any k distinct rows bound the
// final k-th value from above, so each segment's screen starts tight instead
// of at +inf.
// SB: 64-entry blocks of the running sample list (k <= 64 SB).
template <int ARM, int SB>
__global__ __launch_bounds__(256) void knn_seed_f64_kernel(GramArgs64 a, int64_t nsamp) {
    const double* qop = (ARM == ARM_COS_FOLD) ? a.qsq : a.qinv;
    const double* yop = (ARM == ARM_COS_FOLD) ? a.xsq : a.xinv;
    seed_kth_block<double, ARM, unsigned long long, SB>(a.q, a.x, a.nq, a.nt, a.d, a.k, nsamp, qop, yop,
                                                        a.shared_r);
}

__global__ void fill_u64_kernel(unsigned long long* p, int64_t n, unsigned long long v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

template <int NS, int ARM, bool COS>
hipError_t launch_ns(const GramArgs64& a, bool vec2, hipStream_t s) {
    dim3 grid((unsigned)StreamSplit(a.nq, a.nt, kQpb, kBn, a.grid_wgs).G);
    if (a.k <= 64) {
        if (vec2)
            hipLaunchKernelGGL((knn_gram_f64_kernel<NS, ARM, COS, true, 1>), grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((knn_gram_f64_kernel<NS, ARM, COS, false, 1>), grid, dim3(256), 0, s, a);
    } else {
        if (vec2)
            hipLaunchKernelGGL((knn_gram_f64_kernel<NS, ARM, COS, true, 3>), grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((knn_gram_f64_kernel<NS, ARM, COS, false, 3>), grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

template <int ARM, bool COS>
hipError_t launch_arm64(const GramArgs64& a, bool vec2, hipStream_t s) {
    // k-steps per lane group, even (one 16-byte LDS read feeds two)
    const int64_t ns = ((a.d + 3) / 4 + 1) / 2 * 2;
    if (ns <= 8) return launch_ns<8, ARM, COS>(a, vec2, s);
    if (ns <= 16) return launch_ns<16, ARM, COS>(a, vec2, s);
    if (ns <= 32) return launch_ns<32, ARM, COS>(a, vec2, s);
    if (ns <= 48) return launch_ns<48, ARM, COS>(a, vec2, s);
    return launch_ns<64, ARM, COS>(a, vec2, s);
}

}  // namespace

void gram_f64_split(int64_t nq, int64_t nt, int cus, int64_t* grid_wgs, int* nslots) {
    const StreamSplit full(nq, nt, kQpb, kBn, 1);
    // one resident round (two workgroups per CU), but at least 16 tiles each
    int64_t g0 = 2 * (int64_t)(cus > 0 ? cus : 1);
    if (g0 > full.T / 16) g0 = full.T / 16;
    if (g0 < 1) g0 = 1;
    *grid_wgs = g0;
    *nslots = (int)StreamSplit(nq, nt, kQpb, kBn, g0).nslots();
}

int gram_f64_max_k() { return kKcap; }
int gram_f64_max_d() { return kMaxD; }

// Seed on the matrix cores (16-byte rows): the screen value of every
// (query, sampled row) pair on v_mfma_f64_16x16x4f64 (Euclidean: acc =
// ||x||^2 - 2 x.q; cosine: acc = -(x.q)/||x||), turned into the distance it
// stands for, u = max(acc + ||q||^2, 0) or clamp(1 + acc/||q||, 0, 2) (NaN
// kept), written to S[q][s].  The screen bound eps holds for any summation
// order, so k sampled rows have exact <= u + eps <= u_k + eps.  A wave takes
// 16 queries (lane l: query l % 16; k-slot g = l / 16 supplies feature
// g KS + s at k-step s, so each lane's query operand and tile reads are
// contiguous runs, loaded 16 bytes at a time), a workgroup 64 queries and a
// slice of the sample's 16-row tiles (blockIdx.y); sampled row s is index row
// s * n / m.  The next tile's rows are loaded into registers while the
// current tile's MFMA chain runs (two accumulator chains: the even and odd
// k-steps), and stored into the one LDS tile between two barriers.
template <int KS, bool COS>
__global__ __launch_bounds__(256, 2) void knn_seed_screen_f64_kernel(GramArgs64 a, int64_t nsamp,
                                                                     double* __restrict__ S, int64_t ld) {
    static_assert(KS % 2 == 0, "k-steps come in 16-byte pairs");
    constexpr int DP = 4 * KS;
    constexpr int STR = DP + 2;               // rows 16 bytes apart in the banks
    constexpr int CPR = DP / 2;               // 16-byte chunks per tile row
    constexpr int PF = kBn * CPR / 256;       // chunks each thread stages per tile
    static_assert(kBn * CPR % 256 == 0, "whole chunks per thread");
    __shared__ __attribute__((aligned(16))) double tile[kBn * STR];
    __shared__ double tn[kBn];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, j = lane & 15;
    const int64_t nq = a.nq, nt = a.nt, d = a.d;
    const double inf = __builtin_huge_val();
    const int64_t q = (int64_t)blockIdx.x * kQpb + (int64_t)w * kQpw + j;
    const bool qvalid = q < nq;
    const int64_t qrow = qvalid ? q : nq - 1;
    const double qsq = a.qsq[qrow];
    const double qs = COS ? __builtin_sqrt(qsq) : qsq;
    double qreg[KS];
#pragma unroll
    for (int st = 0; st < KS; st += 2) {
        const int64_t c = (int64_t)g * KS + st;  // c and d even: c < d covers c + 1
        double2 v = make_double2(0.0, 0.0);
        if (c < d) v = *reinterpret_cast<const double2*>(a.q + qrow * d + c);
        qreg[st] = v.x * (COS ? 1.0 : -2.0);
        qreg[st + 1] = v.y * (COS ? 1.0 : -2.0);
    }
    const int64_t ntiles = (nsamp + kBn - 1) / kBn;
    const int64_t per = (ntiles + gridDim.y - 1) / gridDim.y;
    const int64_t s_lo = (int64_t)blockIdx.y * per * kBn;
    int64_t s_hi = s_lo + per * kBn;
    if (s_hi > nsamp) s_hi = nsamp;
    // staging: chunk f = tid + 256 p is column pair f % CPR of tile row f / CPR
    double2 pf[PF];
    double pfn = 0.0;
    auto load_tile = [&](int64_t s0) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int f = tid + 256 * p;
            const int r = f / CPR, c2 = f % CPR;
            const int64_t sr = s0 + r;
            double2 v = make_double2(0.0, 0.0);
            if (sr < nsamp && 2 * c2 < d)
                v = *reinterpret_cast<const double2*>(a.x + ((sr * nt) / nsamp) * d + 2 * c2);
            pf[p] = v;
        }
        if (tid < kBn) {
            const int64_t sr = s0 + tid;
            const int64_t t = (sr < nsamp) ? (sr * nt) / nsamp : 0;
            pfn = (sr < nsamp) ? (COS ? a.xscale[t] : a.xsq[t]) : (COS ? 0.0 : inf);
        }
    };
    if (s_lo < s_hi) load_tile(s_lo);
    for (int64_t s0 = s_lo; s0 < s_hi; s0 += kBn) {
        __syncthreads();  // the previous tile is no longer read
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int f = tid + 256 * p;
            *reinterpret_cast<double2*>(&tile[(f / CPR) * STR + 2 * (f % CPR)]) = pf[p];
        }
        if (tid < kBn) tn[tid] = pfn;
        __syncthreads();
        if (s0 + kBn < s_hi) load_tile(s0 + kBn);  // in flight under the chain
        f64x4 acc0, acc1;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            acc0[r] = COS ? 0.0 : tn[g + 4 * r];
            acc1[r] = 0.0;
        }
        const double* arow = &tile[j * STR + g * KS];
#pragma unroll
        for (int st = 0; st < KS; st += 2) {
            const double2 av = *reinterpret_cast<const double2*>(arow + st);
            acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64(av.x, qreg[st], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64(av.y, qreg[st + 1], acc1, 0, 0, 0);
        }
        if (qvalid) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t sr = s0 + g + 4 * r;
                if (sr < nsamp) {
                    const double acc = acc0[r] + acc1[r];
                    const double v = COS ? acc * tn[g + 4 * r] : acc;
                    double u = __builtin_nan("");
                    if (v == v) {
                        if (COS) {
                            u = 1.0 + v / qs;
                            u = u < 0.0 ? 0.0 : (u > 2.0 ? 2.0 : u);
                        } else {
                            u = v + qsq;
                            u = u < 0.0 ? 0.0 : u;
                        }
                    }
                    S[q * ld + sr] = u;
                }
            }
        }
    }
}

// The seed bound from each query's k-th smallest u: (u_k + eps) rounded
// up by a relative 2^-50, for queries in screen-value mode; +inf otherwise.
__global__ void seed_screen_finalize64_kernel(GramArgs64 a, const double* __restrict__ kv, int k, int cos) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= a.nq) return;
    const double inf = __builtin_huge_val();
    const double qsq = a.qsq[q], xmax = a.stats->xsq_max64;
    const double eps = cos ? a.eps_abs : a.eps_rel * (qsq + xmax) + a.eps_abs;
    const bool sv = (qsq + xmax <= 0x1p1020) && (eps < inf) && (!cos || qsq > 0.0);
    const double vk = kv[q * k + (k - 1)];
    double R = inf;
    if (sv && vk < inf) R = (vk + eps) * (1.0 + 0x1p-50);
    a.shared_r[q] = (unsigned long long)__double_as_longlong(R);
}

// Rows the matrix-core seed samples: 128 k, at most 8192 and nt / 64, at
// least 512.  With the tile loads under the MFMA chain the launch is cheap
// enough for four times the exact seed's sample at c3 (k = 16, 2048 rows):
// kernel 9.15 -> 9.01 ms and step 9.43 -> 9.41 ms against 512 rows (A/B of
// two builds on one box; 4096 rows: kernel 8.96 ms, step 9.53 ms).
static int64_t seed_screen_rows64(int64_t nt, int k) {
    int64_t n = 128 * (int64_t)k;
    if (n > 8192) n = 8192;
    if (n > nt / 64) n = nt / 64;
    if (n < 512) n = 512;
    return nt < n ? nt : n;
}

size_t gram_f64_seed_screen_bytes(int64_t nq, int64_t nt, int64_t d, int k, bool vec2) {
    if (k <= 1 || k > kKcap || d > kMaxD || !vec2) return 0;
    const int64_t nsamp = seed_screen_rows64(nt, k);
    if (nsamp < k) return 0;
    const int64_t ld = (nsamp + 1) / 2 * 2;
    const size_t bytes = (size_t)nq * (size_t)ld * 8 + (((size_t)nq * (size_t)k * 8 + 255) & ~(size_t)255) +
                         (((size_t)nq * (size_t)k * 4 + 255) & ~(size_t)255) + 512;
    return bytes <= ((size_t)512 << 20) ? bytes : 0;
}

template <int KS, bool COS>
static void launch_seed_screen64_ks(const GramArgs64& a, int64_t nsamp, double* S, int64_t ld, dim3 grid,
                                    hipStream_t s) {
    hipLaunchKernelGGL((knn_seed_screen_f64_kernel<KS, COS>), grid, dim3(256), 0, s, a, nsamp, S, ld);
}

template <int ARM>
hipError_t launch_seed64(const GramArgs64& a, int64_t nsamp, hipStream_t s) {
    const dim3 grid((unsigned)((a.nq + kSeedQpb - 1) / kSeedQpb));
    if (a.k <= 64)
        hipLaunchKernelGGL((knn_seed_f64_kernel<ARM, 1>), grid, dim3(256), 0, s, a, nsamp);
    else
        hipLaunchKernelGGL((knn_seed_f64_kernel<ARM, 2>), grid, dim3(256), 0, s, a, nsamp);
    return hipGetLastError();
}

hipError_t launch_gram_f64_prep(const GramArgs64& a, int arm, hipStream_t s, void* seed_buf) {
    if (a.root_flag) {
        const hipError_t e = launch_fill_u32(a.root_flag, a.nq, 0u, s);
        if (e != hipSuccess) return e;
    }
    if (!a.shared_r) return hipSuccess;
    if (seed_buf && a.k > 1) {
        const bool cos = (arm == ARM_COS_FOLD || arm == ARM_COS_HOST);
        const int64_t nsamp = seed_screen_rows64(a.nt, a.k);
        const int64_t ld = (nsamp + 1) / 2 * 2;
        double* S = static_cast<double*>(seed_buf);
        char* p = reinterpret_cast<char*>(S + (size_t)a.nq * (size_t)ld);
        p = reinterpret_cast<char*>(((uintptr_t)p + 255) & ~(uintptr_t)255);
        double* kv = reinterpret_cast<double*>(p);
        p += ((size_t)a.nq * (size_t)a.k * 8 + 255) & ~(size_t)255;
        uint32_t* ki = reinterpret_cast<uint32_t*>(p);
        // about four workgroups per CU: the sample's tiles split over blockIdx.y
        const int64_t nqb = (a.nq + kQpb - 1) / kQpb;
        const int64_t ntiles = (nsamp + kBn - 1) / kBn;
        int64_t ys = (1024 + nqb - 1) / nqb;
        if (ys > ntiles) ys = ntiles;
        if (ys > 65535) ys = 65535;
        if (ys < 1) ys = 1;
        const dim3 grid((unsigned)nqb, (unsigned)ys);
        const int64_t ks = (a.d + 3) / 4;
        if (cos) {
            if (ks <= 16) launch_seed_screen64_ks<16, true>(a, nsamp, S, ld, grid, s);
            else if (ks <= 32) launch_seed_screen64_ks<32, true>(a, nsamp, S, ld, grid, s);
            else if (ks <= 48) launch_seed_screen64_ks<48, true>(a, nsamp, S, ld, grid, s);
            else launch_seed_screen64_ks<64, true>(a, nsamp, S, ld, grid, s);
        } else {
            if (ks <= 16) launch_seed_screen64_ks<16, false>(a, nsamp, S, ld, grid, s);
            else if (ks <= 32) launch_seed_screen64_ks<32, false>(a, nsamp, S, ld, grid, s);
            else if (ks <= 48) launch_seed_screen64_ks<48, false>(a, nsamp, S, ld, grid, s);
            else launch_seed_screen64_ks<64, false>(a, nsamp, S, ld, grid, s);
        }
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = launch_select_rows<double>(S, a.nq, nsamp, ld, a.k, EMIT_IDENTITY, kv, ki, nullptr, s);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(seed_screen_finalize64_kernel, dim3((unsigned)((a.nq + 255) / 256)), dim3(256), 0, s, a,
                           kv, a.k, cos ? 1 : 0);
        return hipGetLastError();
    }
    const int64_t nsamp = gram_seed_rows(a.nt, a.k);
    if (nsamp >= a.k) {
        if (arm == ARM_EUCLID_FMA) return launch_seed64<ARM_EUCLID_FMA>(a, nsamp, s);
        if (arm == ARM_EUCLID_MULADD) return launch_seed64<ARM_EUCLID_MULADD>(a, nsamp, s);
        if (arm == ARM_COS_FOLD) return launch_seed64<ARM_COS_FOLD>(a, nsamp, s);
        if (arm == ARM_COS_HOST) return launch_seed64<ARM_COS_HOST>(a, nsamp, s);
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(fill_u64_kernel, dim3((unsigned)((a.nq + 255) / 256)), dim3(256), 0, s, a.shared_r, a.nq,
                       kInfBits64);
    return hipGetLastError();
}

hipError_t launch_gram_f64(const GramArgs64& a, int arm, hipStream_t s) {
    const bool vec2 = (a.d % 2 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0);
    if (arm == ARM_EUCLID_FMA) return launch_arm64<ARM_EUCLID_FMA, false>(a, vec2, s);
    if (arm == ARM_EUCLID_MULADD) return launch_arm64<ARM_EUCLID_MULADD, false>(a, vec2, s);
    if (arm == ARM_COS_FOLD) return launch_arm64<ARM_COS_FOLD, true>(a, vec2, s);
    if (arm == ARM_COS_HOST) return launch_arm64<ARM_COS_HOST, true>(a, vec2, s);
    return hipErrorInvalidValue;
}

template <int ARM>
hipError_t launch_merge64(const GramArgs64& a, bool vec2, hipStream_t s) {
    const dim3 grid((unsigned)((a.nq + 3) / 4));
    if (a.k > 64) {
        if (vec2)
            hipLaunchKernelGGL((knn_merge_blocks_f64_kernel<ARM, true>), grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((knn_merge_blocks_f64_kernel<ARM, false>), grid, dim3(256), 0, s, a);
    } else if (vec2) {
        hipLaunchKernelGGL((knn_merge_f64_kernel<ARM, true>), grid, dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL((knn_merge_f64_kernel<ARM, false>), grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_gram_f64_merge(const GramArgs64& a, int arm, hipStream_t s) {
    const bool vec2 = (a.d % 2 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0);
    if (arm == ARM_EUCLID_FMA) return launch_merge64<ARM_EUCLID_FMA>(a, vec2, s);
    if (arm == ARM_EUCLID_MULADD) return launch_merge64<ARM_EUCLID_MULADD>(a, vec2, s);
    if (arm == ARM_COS_FOLD) return launch_merge64<ARM_COS_FOLD>(a, vec2, s);
    if (arm == ARM_COS_HOST) return launch_merge64<ARM_COS_HOST>(a, vec2, s);
    return hipErrorInvalidValue;
}

hipError_t launch_gram_f64_root_fill(const GramArgs64& a, int arm, hipStream_t s) {
    if (!a.root_flag || a.mode != EMIT_ROOT_RANKED) return hipSuccess;
    const bool vec2 = (a.d % 2 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0);
    const dim3 grid((unsigned)((a.nq + 3) / 4));
    if (arm == ARM_EUCLID_MULADD) {
        if (vec2)
            hipLaunchKernelGGL((knn_root_fill_f64_kernel<ARM_EUCLID_MULADD, true>), grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((knn_root_fill_f64_kernel<ARM_EUCLID_MULADD, false>), grid, dim3(256), 0, s, a);
        return hipGetLastError();
    }
    if (arm == ARM_EUCLID_FMA) {
        if (vec2)
            hipLaunchKernelGGL((knn_root_fill_f64_kernel<ARM_EUCLID_FMA, true>), grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((knn_root_fill_f64_kernel<ARM_EUCLID_FMA, false>), grid, dim3(256), 0, s, a);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;  // the roots are sqrt: Euclidean arms only
}

}  // namespace mlrs
