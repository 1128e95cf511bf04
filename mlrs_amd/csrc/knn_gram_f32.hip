// Fused f32 Gram-MFMA kNN with exact rescoring (gfx950).
//
// Replaces the GPU arm euclidean_topk_fused{,_dot,_dot_vec,_dot_vec8}
// (crates/mlrs-kernels/src/knn.rs:377-2112) and the two-kernel
// distance_direct -> top_k fallback (crates/mlrs-algos/src/neighbors/
// nearest.rs:1058-1343) for f32, d <= 256, k <= 128, Euclidean and cosine.
//
// Two register shapes (GramShape below): d <= 128, 4 waves x 32 queries =
// 128 queries per workgroup on v_mfma_f32_32x32x2f32; 128 < d <= 256, 4 waves
// x 16 queries = 64 per workgroup on v_mfma_f32_16x16x4f32.  Either walks one
// strip of index rows 32 at a time.
//  * Each wave keeps its query rows in VGPRs as the B operand (pre-scaled by
//    -2 for Euclidean), loaded once per segment.
//  * The 32-row index tile is staged in LDS (row stride d_pad + 4 floats, so
//    16 consecutive rows fall on distinct bank groups; rows of 128 floats in
//    pairs that share one 1 KB slot), double-buffered in two distinct LDS
//    objects.  Aligned rows of at least 64 floats are loaded one tile ahead
//    straight from global memory into LDS (global_load_lds_dwordx4); other
//    shapes, and k = 1, prefetch into registers.
//  * Euclidean: the accumulator starts at ||x_t||^2, so after the contraction
//    acc = ||x_t||^2 - 2 x_t.q_j, the expansion minus the per-query constant.
//    Cosine: the contraction is scaled by -1/||x_t|| per row afterwards,
//    acc = -x_t.q_j/||x_t||.
//  * Screen: acc is compared against a per-query threshold derived from the
//    best bound known on the query's k-th exact value (its own list, any
//    segment's, shared through a per-query word and per-segment list
//    summaries in global memory) plus a rigorous bound eps on the expansion's
//    rounding error and the reference's own.  A pair that can still enter the
//    exact top-k always passes; the comparison is !(acc > thr), so NaN passes
//    too.  For k = 1 the bound is tightened every tile with the tile's
//    smallest expansion value.
//  * For k > 1 the per-query bound starts from a seed launch: the k-th
//    smallest exact value over evenly spaced index rows (gram_seed_rows).
//  * Passing (query, row) pairs are queued in a per-wave global array (index
//    rows and screen values; queue lengths live in registers; the lanes
//    screening a query append with a popcount prefix, no atomics), which
//    leaves the LDS small enough for three workgroups per CU at d <= 128.
//    Before a queue could overflow, the wave sorts it and merges it into the
//    query's list for this segment (global memory, one per query and
//    segment): a queued pair enters with its screen value mapped back to a
//    distance, which is within eps of its exact value, and the list keeps
//    the k + 32 (at most 64) smallest.  No pair is evaluated exactly during
//    the scan, except in the rare lists that turn exact (a dropped pair
//    inside the 2 eps window of the k-th, NaN screen values, norms that could
//    overflow).  k = 1 queues index rows in LDS and keeps one exact
//    (value, index) pair per query there.
//  * The merge kernel takes each query's lists from all segments, finds the
//    k-th value V of their union and evaluates EXACTLY, in the reference
//    arm's operation order, every listed pair whose screen value is within
//    2 eps of V (window rescoring), then ranks by (exact value, index).
//  * Work split: StreamSplit (knn_kernels.hpp), panel-major, with XCD-grouped
//    workgroup numbering, so the workgroups on one XCD stream the same index
//    panel in lockstep.
// The kept lists are therefore the reference's own top-k: the full distance
// matrix never reaches HBM and no tolerance is involved.
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

constexpr int kWaves = 4;                // waves per workgroup, narrow shape (the wide shape: 6)
constexpr int kBn = 32;                  // index rows per tile
constexpr int kKcap = 128;               // largest k this kernel keeps
constexpr int kQcapK1 = 48;              // k = 1: the screen tightens every tile, queues stay short
constexpr int kShareEvery = 64;          // tiles between reads of the shared thresholds
// The narrow shape's k <= 64 lists (k > 1) read them every 128 tiles: c2
// kernel 20.38 -> 20.29 ms; the three-block lists and the wide shape keep 64
// (at 128: c2k128 +0.1 ms, d256 +0.07 ms; 96, not a power of two, was slower
// for both narrow kernels; 256: c2 +0.15 ms)
constexpr int share_every(bool k1, int kl, bool w16) {
    return (!k1 && kl == 1 && !w16) ? 2 * kShareEvery : kShareEvery;
}
constexpr int kSumSlots = 16;            // segment summaries read per refresh (k > 1)

// The two register shapes of a wave's block of (row, query) values.
//  d <= 128 (W16 = false): 32 queries per wave, v_mfma_f32_32x32x2f32 over
//    the 32-row tile; lane (h = lane / 32, jl = lane % 32) holds 16 of query
//    jl's rows, and the query operand is d/2 VGPRs.
//  128 < d <= 256 (W16 = true): 16 queries per wave, v_mfma_f32_16x16x4f32
//    on the tile's two 16-row halves; lane (g = lane / 16, jl = lane % 16)
//    holds 8 of query jl's rows, and lane group g contracts the g-th quarter
//    of the feature axis, so the query operand is d/4 VGPRs (64 at d = 256).
//  Both shapes run 4 waves per workgroup.  (For the wide shape, whose two
//  33 KB tiles leave room for only two workgroups per CU, a third wave per
//  SIMD from larger workgroups did not pay: two 6-wave workgroups are seldom
//  placed so that both fit a CU (d256 7.0 ms), and one 12-wave workgroup runs
//  its waves in lockstep behind one barrier (5.6 ms against 5.3-5.4).)
template <bool W16>
struct GramShape {
    static constexpr int qpw = W16 ? 16 : 32;      // queries per wave
    static constexpr int waves = kWaves;           // waves per workgroup
    static constexpr int threads = 64 * waves;
    static constexpr int qpb = waves * qpw;        // queries per workgroup
    static constexpr int vals = W16 ? 8 : 16;      // tile values per lane
    // queued candidates per query (k > 1): the wide shape 128 (flushed as two
    // 64-entry blocks: d256 kernel 4.83 -> 4.59 ms against 48; 64: 4.64,
    // 96: 4.60); the narrow k <= 64 kernel 64 (128 measured slower there)
    static constexpr int qcap = W16 ? 128 : 64;
    // three-block lists (k > 64): longer queues, about half as many flushes
    // (c2k128 kernel 24.5 -> 23.0 ms; 96 entries 24.0, 192 23.4, 256 23.2)
    static constexpr int qcap3 = 128;
};
constexpr int kQpbNarrow = GramShape<false>::qpb;
constexpr int kQpbWide = GramShape<true>::qpb;
constexpr int kQvalPerWave = 32 * 128;            // pairs a wave may queue (any shape), k > 1
// Per wave in a.qval: the kernel's QPW x QCAP screen values, then as many
// index-row numbers, both [queue position][query] (gram_f32_qval_elems sizes
// the buffer for the launch's list length).

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Per-wave LDS state.  Only k = 1 queues its candidates' indices here (QCAP
// per query); k > 1 queues them in global memory beside their screen values,
// which leaves room for a third workgroup per CU.
template <int QCAP, int QPW>
struct WaveLds {
    uint32_t qidx[QPW][QCAP];
    float thr[QPW];
    float qa[QPW];   // exact arm's query operand (row_sumsq for the fold arm)
    float qs[QPW];   // screen operand: ||q||^2 (Euclidean) or ||q|| (cosine)
    float eps[QPW];  // screen error bound
    uint32_t off[QPW];                 // k = 1: queue offsets of the batched flush
    uint32_t mode[QPW];                // 0: screen values lie within eps of exact values (k > 1: screen-value list); 1: not (exact list)
    unsigned long long best[QPW];      // k = 1: (value bits << 32 | index) of the kept pair
};

// (value, index) packed so that unsigned order is the (value, index) order
// for the non-negative values every served arm produces.
constexpr unsigned long long kBestEmpty = (0x7F800000ull << 32) | 0xFFFFFFFFull;

template <bool COS>
__device__ __forceinline__ float screen_threshold(float R, float qs, float eps) {
    const float inf = __builtin_huge_valf();
    if (!(R < inf)) return inf;  // no finite k-th value known yet
    if (!COS) {
        // exact <= R  =>  ||x||^2 - 2 x.q <= R - ||q||^2 + eps
        return round_up_f((double)R - (double)qs + (double)eps);
    } else {
        // exact <= R  =>  1 + acc/||q|| <= R + eps  =>  acc <= (R + eps - 1)||q||
        // A zero query scores exactly 1 against every row: all rows tie, and a
        // bound published by another segment cannot tell which of them win
        // (lower indices may lie in a segment that has not run yet), so such a
        // query is never screened.
        if (qs == 0.0f) return inf;
        return round_up_f(((double)R + (double)eps - 1.0) * (double)qs);
    }
}

// The arms' per-row and per-query operands of the exact evaluation: the
// squared norm (cosine fold: sqrt(||q||^2 ||x||^2)), the reciprocal norm
// (knn_host cosine) or nothing (Euclidean).
template <int ARM>
__device__ __forceinline__ float row_operand(const GramArgs32& a, int64_t t) {
    return (ARM == ARM_COS_FOLD) ? a.xsq[t] : (ARM == ARM_COS_HOST) ? a.xinv[t] : 0.0f;
}
template <int ARM>
__device__ __forceinline__ float query_operand(const GramArgs32& a, int64_t q) {
    return (ARM == ARM_COS_FOLD) ? a.qsq[q] : (ARM == ARM_COS_HOST) ? a.qinv[q] : 0.0f;
}

// Exact value of one (query, row) pair in the arm's operation order, loads
// issued U 16-byte chunks at a time.
template <int ARM, bool VEC4, int U = 4>
__device__ __forceinline__ float exact_f32(const float* __restrict__ q, const float* __restrict__ y,
                                           int64_t d, float qa, float ya) {
    if (!VEC4) return exact_pair<float, ARM>(q, y, d, qa, ya);
    const float4* q4 = reinterpret_cast<const float4*>(q);
    const float4* y4 = reinterpret_cast<const float4*>(y);
    const int n4 = (int)(d >> 2);
    float acc = 0.0f;
    int c = 0;
    for (; c + U <= n4; c += U) {
        float4 a[U], b[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            a[u] = q4[c + u];
            b[u] = y4[c + u];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (ARM == ARM_EUCLID_FMA) {
                float d0 = a[u].x - b[u].x, d1 = a[u].y - b[u].y, d2 = a[u].z - b[u].z, d3 = a[u].w - b[u].w;
                acc = __builtin_fmaf(d0, d0, acc);
                acc = __builtin_fmaf(d1, d1, acc);
                acc = __builtin_fmaf(d2, d2, acc);
                acc = __builtin_fmaf(d3, d3, acc);
            } else if (ARM == ARM_EUCLID_MULADD) {
                float d0 = a[u].x - b[u].x, d1 = a[u].y - b[u].y, d2 = a[u].z - b[u].z, d3 = a[u].w - b[u].w;
                acc = acc + d0 * d0;
                acc = acc + d1 * d1;
                acc = acc + d2 * d2;
                acc = acc + d3 * d3;
            } else if (ARM == ARM_COS_HOST) {  // mul + add dot
                acc = acc + a[u].x * b[u].x;
                acc = acc + a[u].y * b[u].y;
                acc = acc + a[u].z * b[u].z;
                acc = acc + a[u].w * b[u].w;
            } else {  // ARM_COS_FOLD: fma dot
                acc = __builtin_fmaf(a[u].x, b[u].x, acc);
                acc = __builtin_fmaf(a[u].y, b[u].y, acc);
                acc = __builtin_fmaf(a[u].z, b[u].z, acc);
                acc = __builtin_fmaf(a[u].w, b[u].w, acc);
            }
        }
    }
    for (; c < n4; ++c) {
        float4 a = q4[c], b = y4[c];
        if (ARM == ARM_EUCLID_FMA) {
            float d0 = a.x - b.x, d1 = a.y - b.y, d2 = a.z - b.z, d3 = a.w - b.w;
            acc = __builtin_fmaf(d0, d0, acc);
            acc = __builtin_fmaf(d1, d1, acc);
            acc = __builtin_fmaf(d2, d2, acc);
            acc = __builtin_fmaf(d3, d3, acc);
        } else if (ARM == ARM_EUCLID_MULADD) {
            float d0 = a.x - b.x, d1 = a.y - b.y, d2 = a.z - b.z, d3 = a.w - b.w;
            acc = acc + d0 * d0;
            acc = acc + d1 * d1;
            acc = acc + d2 * d2;
            acc = acc + d3 * d3;
        } else if (ARM == ARM_COS_HOST) {
            acc = acc + a.x * b.x;
            acc = acc + a.y * b.y;
            acc = acc + a.z * b.z;
            acc = acc + a.w * b.w;
        } else {
            acc = __builtin_fmaf(a.x, b.x, acc);
            acc = __builtin_fmaf(a.y, b.y, acc);
            acc = __builtin_fmaf(a.z, b.z, acc);
            acc = __builtin_fmaf(a.w, b.w, acc);
        }
    }
    if (ARM == ARM_COS_FOLD) {
        float denom = __builtin_sqrtf(qa * ya);
        float sim = (denom > 0.0f) ? acc / denom : 0.0f;
        return clamp02<float>(1.0f - sim);
    }
    // knn_host cosine (crates/mlrs-backend/src/prims/knn_host.rs:749-760):
    // reciprocal norms, 1 - dot * (1/||q||) * (1/||x||), clamped
    if (ARM == ARM_COS_HOST) return clamp02<float>(1.0f - acc * qa * ya);
    return acc;
}

// Workgroups per CU.  Three (at most 168 VGPRs, 53 KB LDS) wherever they
// fit: k = 1 with d <= 64 (its LDS queues allow no more), the narrow shape
// (d <= 128) with k > 1, whose queues live in global memory (k <= 128: the
// compiler spills a little of the three-block lists), and the wide shape
// with k > 1 and 16-byte rows, which then keeps one tile buffer (33 KB at
// d = 256; two barriers per tile).  A third wave per SIMD keeps the matrix
// core fed while the other two wait at a tile barrier or merge a queue into
// a list.
__host__ __device__ constexpr int gram_f32_wgs_per_cu(int ng, bool k1, int kl, bool vec4) {
    return (k1 && ng <= 8) || (!k1 && (ng <= 16 || vec4)) ? 3 : 2;
}
template <int NG, bool K1, int KL, bool VEC4>
struct GramOcc {
    static constexpr int wgs = gram_f32_wgs_per_cu(NG, K1, KL, VEC4);
};

// KL: 64-entry blocks of a (segment, query) list in registers during a flush
// (1 for k <= 64, 3 for k <= 128: k + 32 entries).
// FULLW: every row is exactly DP = 8 NG floats wide (d = DP), launched for the
// paired-row kernels (d = 128) so that their tile loads need no runtime
// stride.
template <int NG, int ARM, bool COS, bool VEC4, bool K1, int KL, bool FULLW = false>
// (__launch_bounds__' second argument is waves per SIMD: workgroups per CU x
// waves per workgroup / 4.)
__global__ __launch_bounds__(GramShape<(NG > 16)>::threads,
                             (GramOcc<NG, K1, KL, VEC4>::wgs * GramShape<(NG > 16)>::waves / 4)) void knn_gram_f32_kernel(
    GramArgs32 a) {
    constexpr bool W16 = NG > 16;     // the wide shape (GramShape)
    typedef GramShape<W16> SH;
    constexpr int QPW = SH::qpw;
    constexpr int QPB = SH::qpb;
    constexpr int WV = SH::waves;     // waves per workgroup
    constexpr int NT = SH::threads;   // threads per workgroup
    constexpr int DP = NG * 8;        // padded feature count
    constexpr int CPR = DP / 4;       // 16-byte chunks per tile row
    // LDS row stride (floats): DP + 4, an odd number of 16-byte chunks, so
    // the A-operand ds_read_b128 of 16 consecutive rows (one chunk column)
    // hit 16 distinct groups of four banks.  Narrow rows of 128 floats are
    // kept in pairs instead: slot s (0..15) holds rows s and s + 16 back to
    // back (1 KB, one wave-wide direct load) and slots are 2 DP + 4 floats
    // apart, so rows 0..15 (and 16..31) still fall on distinct bank groups.
    constexpr int STRIDE = DP + 4;
    constexpr bool PAIRS = !W16 && NG == 16;
    constexpr int SLOT = 2 * DP + 4;
    constexpr int TILE_FL = PAIRS ? 16 * SLOT : kBn * STRIDE;
    constexpr int TILE_F4 = kBn * DP / 4;
    constexpr int PF = (TILE_F4 + NT - 1) / NT;
    // 16-byte aligned rows of at least 64 floats go from global memory
    // straight into LDS (gfx950's global_load_lds_dwordx4, one instruction per
    // row, or per slot of two rows, with the first CPR (2 CPR) lanes active:
    // lane i's 16 bytes land 16 i bytes after the row start), so no registers
    // hold the next tile in flight and no ds_write stores it; other shapes
    // stage it through registers.  The k = 1 kernel (short segments, three
    // workgroups per CU already) runs faster staged.
    constexpr bool DIRECT = VEC4 && NG >= 8 && !K1;
    // Wide shape, direct loads: one tile buffer, refilled once every wave's
    // MFMA chain has read it, so that three workgroups fit a CU.
    constexpr bool SINGLE = W16 && DIRECT;
    constexpr int RPW = (kBn + WV - 1) / WV;  // tile rows each wave fills (direct): w, w + WV, ...
    constexpr int QQ = DP / 4;        // wide: features per lane-group quarter
    constexpr int NQR = W16 ? QQ / 4 : NG;  // 16-byte query-operand chunks per lane

    // The two tile buffers are distinct objects, so the compiler can tell the
    // direct loads into one from the reads of the other.
    __shared__ __attribute__((aligned(16))) float tileA[TILE_FL];
    __shared__ __attribute__((aligned(16))) float tileB[SINGLE ? 4 : TILE_FL];
    __shared__ __attribute__((aligned(16))) float tnA[kBn];
    __shared__ __attribute__((aligned(16))) float tnB[kBn];
    constexpr int QCAP = K1 ? kQcapK1 : (KL > 1 ? SH::qcap3 : SH::qcap);
    constexpr int QB = (QCAP + 63) / 64;  // 64-entry blocks of a flushed queue
    constexpr int kFlushAt = QCAP - kBn;  // flush when a queue may overflow next tile
    __shared__ WaveLds<K1 ? QCAP : 1, QPW> wl[WV];

    // Kernel arguments as locals: they stay in SGPRs.
    const float* __restrict__ Q = a.q;
    const float* __restrict__ X = a.x;
    const float* __restrict__ QSQ = a.qsq;
    const float* __restrict__ XSQ = a.xsq;
    const float* __restrict__ XSCALE = a.xscale;
    unsigned int* __restrict__ SHARED_R = a.shared_r;
    const int64_t nq = a.nq, nt = a.nt, d = a.d;
    const int k = a.k;
    const int K2 = gram_list_cap(k);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    // narrow: h = lane / 32 picks the 4-row group of each 8-row slab;
    // wide: g = lane / 16 picks the 4-row group of each 16-row half and the
    // feature quarter.  jl: the lane's query within the wave.
    const int h = W16 ? (lane >> 4) : (lane >> 5);
    const int jl = lane & (QPW - 1);
    WaveLds<K1 ? QCAP : 1, QPW>& L = wl[w];
    const float inf = __builtin_huge_valf();
    // screen values and index rows of this wave's queued pairs (k > 1),
    // [queue position][query]
    constexpr int QVW = QPW * QCAP;  // this kernel's pairs per wave (<= kQvalPerWave)
    static_assert(QVW <= (KL > 1 ? 32 * 128 : 32 * 64), "gram_f32_qval_elems sizes the queues");
    float* __restrict__ QVw = K1 ? nullptr : a.qval + ((int64_t)blockIdx.x * WV + w) * (2 * QVW);
    uint32_t* __restrict__ QIw = K1 ? nullptr : reinterpret_cast<uint32_t*>(QVw + QVW);

    // Tile row of value r of this lane.
    auto row_of = [&](int r) -> int {
        return W16 ? 16 * (r >> 2) + 4 * h + (r & 3) : 8 * (r >> 2) + 4 * h + (r & 3);
    };
    // LDS float offset of 16-byte chunk c of tile row r.
    auto row_at = [&](int r) -> int { return PAIRS ? (r & 15) * SLOT + (r >> 4) * DP : r * STRIDE; };
    auto chunk_at = [&](int r, int c) -> int { return row_at(r) + 4 * c; };

    // Direct fills never write the columns past d (d < DP): zero them once in
    // both buffers, as they meet the query operand's zeros and left alone
    // could hold NaN.
    if (DIRECT && d < DP) {
        const int pad = (int)(DP - d);
        for (int e = tid; e < kBn * pad; e += NT) {
            tileA[row_at(e / pad) + d + e % pad] = 0.0f;
            if constexpr (!SINGLE) tileB[row_at(e / pad) + d + e % pad] = 0.0f;
        }
    }

    // ---- work split (StreamSplit): this workgroup's range of (query block,
    //      tile) units, panel-major; each piece of a job in the range is a
    //      segment with its own exact lists [slot][nq][k], merged at the end
    //      by knn_merge_f32_kernel. ----
    const StreamSplit sp(nq, nt, QPB, kBn, a.grid_wgs);
    const int64_t wg = xcd_grouped_wg(blockIdx.x, gridDim.x);
    const int64_t u_hi = ((wg + 1) * sp.P < sp.T) ? (wg + 1) * sp.P : sp.T;
    for (int64_t u = wg * sp.P; u < u_hi;) {
    int64_t panel, qblock, tile0, left;
    sp.decode(u, panel, qblock, tile0, left);
    const int64_t tile1 = tile0 + ((left < u_hi - u) ? left : (u_hi - u));
    const int64_t slot = sp.slot(wg, panel, qblock);
    float* __restrict__ LV = a.part_val + slot * nq * K2;
    uint32_t* __restrict__ LI = a.part_idx + slot * nq * K2;
    // Summaries of the query block's segment lists: segment s holds at least
    // rank_i pairs whose exact value is <= summ[s][q].i (rank_i = ceil(i k/4));
    // the union over segments (disjoint rows) bounds the query's k-th value.
    float4* __restrict__ SUMM = a.summ;
    const int64_t nsum = SUMM ? (sp.slots_of(qblock) < kSumSlots ? sp.slots_of(qblock) : kSumSlots) : 0;
    const int rk1 = (k + 3) / 4, rk2 = (k + 1) / 2, rk3 = (3 * k + 3) / 4;

    const int64_t qwave = qblock * QPB + w * QPW;  // first query of this wave
    const int64_t qmine = qwave + jl;
    const bool qvalid = qmine < nq;
    const int64_t t_begin = tile0 * kBn;
    int64_t t_end = tile1 * kBn;
    if (t_end > nt) t_end = nt;

    // Feature of chunk element e of the lane's query-operand chunk i.
    auto qfeat = [&](int i, int e) -> int64_t {
        return W16 ? (int64_t)h * QQ + 4 * i + e : (int64_t)8 * i + 4 * h + e;
    };

    // ---- segment start: the loads first, from clamped rows so that they are
    //      unconditional and all in flight together (a segment of k-means
    //      assignment lasts only 32 tiles), then the per-query state.  Wide
    //      rows (NG > 8) load the operand later: early it would spill. ----
    constexpr bool kEarlyQ = NG <= 8;
    const int64_t qrow = qvalid ? qmine : nq - 1;
    const float qsq_l = QSQ[qrow];
    const float r0_l = SHARED_R ? __uint_as_float(SHARED_R[qrow]) : inf;
    float4 qreg[NQR];
    if (VEC4 && kEarlyQ) {
        const float* qp = Q + qrow * d;
#pragma unroll
        for (int g = 0; g < NQR; ++g) {
            const int64_t c = qfeat(g, 0);
            const float4 v = *reinterpret_cast<const float4*>(qp + (c < d ? c : d - 4));
            qreg[g] = (qvalid && c < d) ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }

    // ---- per-query constants, lists, queues ----
    uint32_t cntr = 0u;  // queued candidates of query jl
    if (lane < QPW) {
        const float qsq = qvalid ? qsq_l : 0.0f;
        L.thr[lane] = qvalid ? inf : -inf;
        if (!COS) {
            L.qs[lane] = qsq;
            L.qa[lane] = 0.0f;
            L.eps[lane] = (float)(a.eps_rel * ((double)qsq + (double)a.stats->xsq_max) + a.eps_abs);
        } else {
            L.qs[lane] = __builtin_sqrtf(qsq);
            L.qa[lane] = (ARM == ARM_COS_HOST) ? (qvalid ? a.qinv[qrow] : 0.0f) : qsq;
            L.eps[lane] = (float)a.eps_abs;
        }
        // Screen-value lists need |screen distance - exact| <= eps for every
        // pair, which the error bound gives while no sum can overflow: norms
        // well inside the float range (and a nonzero query for cosine).
        // Other queries keep exact lists.
        bool sv = qvalid && ((double)qsq + (double)a.stats->xsq_max <= 0x1p124) && (L.eps[lane] < inf);
        if (COS) sv = sv && (L.qs[lane] > 0.0f);
        L.mode[lane] = sv ? 0u : 1u;
    }
    if (K1) {
        if (lane < QPW) L.best[lane] = kBestEmpty;
    } else {
        for (int j = 0; j < QPW; ++j) {
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
    }
    // Strips that start late begin from the bound earlier strips have reached.
    if (SHARED_R && lane < QPW && qvalid)
        L.thr[lane] = fminf(L.thr[lane], screen_threshold<COS>(r0_l, L.qs[lane], L.eps[lane]));

    // ---- query operand: qreg[i] = scale * q[qfeat(i, 0..3)] (aligned rows:
    //      one 16-byte load per chunk) ----
    {
        const float scale = COS ? 1.0f : -2.0f;
        const float* qp = Q + qmine * d;
        if (VEC4) {
            if (!kEarlyQ) {
#pragma unroll
                for (int g = 0; g < NQR; ++g) {
                    const int64_t c = qfeat(g, 0);
                    qreg[g] = (qvalid && c < d) ? *reinterpret_cast<const float4*>(qp + c)
                                                : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
#pragma unroll
            for (int g = 0; g < NQR; ++g) {
                qreg[g].x *= scale;
                qreg[g].y *= scale;
                qreg[g].z *= scale;
                qreg[g].w *= scale;
            }
        } else {
#pragma unroll
            for (int g = 0; g < NQR; ++g) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t c = qfeat(g, e);
                    v[e] = (qvalid && c < d) ? qp[c] * scale : 0.0f;
                }
                qreg[g] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }

    // ---- tile prefetch into registers (rows past the strip: zeros, norm +inf) ----
    // Each thread owns PF fixed 16-byte chunks of the tile: row pf_r[p], column
    // chunk pf_c[p]; its source pointer walks down one tile (kBn rows) per step.
    const uint32_t t_end32 = (uint32_t)t_end;
    int pf_r[PF];
    bool pf_on[PF];
    const float* pf_src[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        const int f = tid + NT * p;
        pf_r[p] = f / (DP / 4);
        const int c4 = f % (DP / 4);
        pf_on[p] = (f < TILE_F4) && (4 * c4 < d);
        pf_src[p] = X + (t_begin + pf_r[p]) * d + 4 * c4;
    }
    // Whole tiles of rows without padded columns load unconditionally.
    const bool pf_fast = VEC4 && (PF * NT == TILE_F4) && (d == DP);
    // Wide rows: a thread's chunks lie in one column, PF_RPP rows apart, so one
    // pointer and uniform offsets address them (eight live 64-bit pointers
    // would not fit next to the 64-register query operand).
    constexpr int PF_RPP = (NT % (DP / 4) == 0) ? NT / (DP / 4) : 0;
    constexpr bool PF_ONE_PTR = W16 && PF_RPP > 0;
    // The address, row and on-flag of prefetch chunk p (wide rows: derived
    // from chunk 0's).
#define MLRS_PF_SRC(p) (PF_ONE_PTR ? pf_src[0] + (int64_t)(p) * PF_RPP * d : pf_src[p])
#define MLRS_PF_ROW(p) (PF_ONE_PTR ? pf_r[0] + (p) * PF_RPP : pf_r[p])
#define MLRS_PF_ON(p) (PF_ONE_PTR ? pf_on[0] : pf_on[p])
#define MLRS_PREFETCH(T0)                                                                    \
    do {                                                                                     \
        const uint32_t t0_ = (uint32_t)(T0);                                                 \
        if (pf_fast && t_end32 - t0_ >= (uint32_t)kBn) { /* not t0 + kBn: no wrap */        \
            _Pragma("unroll") for (int p = 0; p < PF; ++p) pf[p] = gload4(MLRS_PF_SRC(p));   \
        } else {                                                                             \
        _Pragma("unroll") for (int p = 0; p < PF; ++p) {                                     \
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);                                      \
            const uint32_t t = t0_ + (uint32_t)MLRS_PF_ROW(p);                               \
            if (MLRS_PF_ON(p) && t < t_end32) {                                              \
                const float* src = MLRS_PF_SRC(p);                                           \
                if (VEC4) {                                                                  \
                    v = gload4(src);                                                         \
                } else {                                                                     \
                    const int c0_ = (int)((tid + NT * p) % (DP / 4)) * 4;                    \
                    float e4[4];                                                             \
                    _Pragma("unroll") for (int e = 0; e < 4; ++e) e4[e] =                    \
                        (c0_ + e < d) ? src[e] : 0.0f;                                       \
                    v = make_float4(e4[0], e4[1], e4[2], e4[3]);                             \
                }                                                                            \
            }                                                                                \
            pf[p] = v;                                                                       \
        }                                                                                    \
        }                                                                                    \
        _Pragma("unroll") for (int p = 0; p < (PF_ONE_PTR ? 1 : PF); ++p) pf_src[p] += kBn * d; \
        if (tid < kBn) {                                                                     \
            const uint32_t t = t0_ + (uint32_t)tid;                                          \
            if (COS)                                                                         \
                pfn = (t < t_end32) ? XSCALE[t] : 0.0f;                                      \
            else                                                                             \
                pfn = (t < t_end32) ? XSQ[t] : inf;                                          \
        }                                                                                    \
    } while (0)

    // ---- flush (k > 1): one query's queue sorted and merged into its list.
    //      Screen-value mode: a queued pair enters with its screen value
    //      mapped back to a distance, within eps of its exact value; the list
    //      keeps the K2 smallest, and the segment's bound is its k-th + eps.
    //      A pair whose screen value is NaN, and every pair of an exact-mode
    //      query, is evaluated exactly in the arm's operation order.  When a
    //      discarded pair lies within 2 eps of the k-th (it could still be
    //      among the k best), the old list and the queue are re-evaluated
    //      exactly and the query's list stays exact from then on. ----
#define MLRS_EXACT_AT(T_)                                                                    \
    exact_f32<ARM, VEC4>(Q + qg_ * d, X + (int64_t)(T_) * d, d, L.qa[j_], row_operand<ARM>(a, (T_)))
#define MLRS_FLUSH(J)                                                                        \
    do {                                                                                     \
        const int j_ = (J);                                                                  \
        const int64_t qg_ = qwave + j_;                                                      \
        const uint32_t n_ = bcast_u(cntr, j_);                                               \
        const bool exact_ = L.mode[j_] != 0u;                                                \
        unsigned long long lk_[KL];                                                          \
        _Pragma("unroll") for (int r_ = 0; r_ < KL; ++r_) {                                  \
            const int p_ = 64 * r_ + lane;                                                   \
            lk_[r_] = kKeyEmpty;                                                             \
            if (p_ < K2) lk_[r_] = pair_key(LV[qg_ * K2 + p_], LI[qg_ * K2 + p_]);           \
        }                                                                                    \
        const unsigned long long ok_ = lk_[0];                                               \
        unsigned long long dk_ = kKeyEmpty;                                                  \
        unsigned long long ek_ = kKeyEmpty;                                                  \
        if constexpr (QB == 1) {                                                             \
            float e_ = inf;                                                                  \
            uint32_t t_ = kSentinelIdx;                                                      \
            if ((uint32_t)lane < n_) {                                                       \
                t_ = QIw[lane * QPW + j_];                                                   \
                const float s_ = exact_ ? 0.0f : QVw[lane * QPW + j_];                       \
                if (exact_ || s_ != s_)                                                      \
                    e_ = MLRS_EXACT_AT(t_);                                                  \
                else                                                                         \
                    e_ = COS ? 1.0f + s_ / L.qs[j_] : s_ + L.qs[j_];                         \
                if (e_ != e_) { /* NaN is never admitted */                                  \
                    e_ = inf;                                                                \
                    t_ = kSentinelIdx;                                                       \
                }                                                                            \
            }                                                                                \
            ek_ = pair_key(e_, t_);                                                          \
            wave_sort64_key(ek_, lane);                                                      \
            if constexpr (KL == 1)                                                           \
                dk_ = wave_merge64_key_drop(lk_[0], ek_, lane);                              \
            else                                                                             \
                dk_ = wave_merge_blocks_key_drop<KL>(lk_, ek_, lane);                        \
        } else {                                                                             \
          _Pragma("unroll") for (int b_ = 0; b_ < QB; ++b_) {                                \
            if (b_ == 0 || n_ > 64u * (uint32_t)b_) {                                        \
              float e_ = inf;                                                                \
              uint32_t t_ = kSentinelIdx;                                                    \
              const uint32_t qi_ = 64u * (uint32_t)b_ + (uint32_t)lane;                      \
              if (qi_ < n_) {                                                                \
                  t_ = QIw[qi_ * QPW + j_];                                                  \
                  const float s_ = exact_ ? 0.0f : QVw[qi_ * QPW + j_];                      \
                  if (exact_ || s_ != s_)                                                    \
                      e_ = MLRS_EXACT_AT(t_);                                                \
                  else                                                                       \
                      e_ = COS ? 1.0f + s_ / L.qs[j_] : s_ + L.qs[j_];                       \
                  if (e_ != e_) { /* NaN is never admitted */                                \
                      e_ = inf;                                                              \
                      t_ = kSentinelIdx;                                                     \
                  }                                                                          \
              }                                                                              \
              ek_ = pair_key(e_, t_);                                                        \
              wave_sort64_key(ek_, lane);                                                    \
              const unsigned long long d_ = wave_merge_blocks_key_drop<KL>(lk_, ek_, lane);  \
              dk_ = (b_ == 0 || d_ < dk_) ? d_ : dk_; /* the smallest dropped */           \
            }                                                                                \
          }                                                                                  \
        }                                                                                    \
        float R_ = f32_from_order_bits(list_hi_at<KL>(lk_, k - 1));                          \
        if (!exact_) {                                                                       \
            const float dr_ = (K2 < 64 * KL) ? f32_from_order_bits(list_hi_at<KL>(lk_, K2))  \
                                             : key_value(dk_);                               \
            double w_ = (double)R_ + 2.0 * (double)L.eps[j_];                                \
            w_ += __builtin_fabs(w_) * 0x1p-40;                                              \
            if (dr_ < inf && (double)dr_ <= w_) {                                            \
              if constexpr (KL == 1 && QB == 1) {                                            \
                /* the old list and the queue, exactly */                                    \
                float x1_ = inf, x2_ = inf;                                                  \
                uint32_t i1_ = key_index(ok_), i2_ = key_index(ek_);                         \
                if (i1_ != kSentinelIdx) x1_ = MLRS_EXACT_AT(i1_);                           \
                if (i2_ != kSentinelIdx) x2_ = MLRS_EXACT_AT(i2_);                           \
                if (x1_ != x1_) { x1_ = inf; i1_ = kSentinelIdx; }                           \
                if (x2_ != x2_) { x2_ = inf; i2_ = kSentinelIdx; }                           \
                unsigned long long k1_ = pair_key(x1_, i1_), k2_ = pair_key(x2_, i2_);       \
                wave_sort64_key(k1_, lane);                                                  \
                wave_sort64_key(k2_, lane);                                                  \
                wave_merge64_key(k1_, k2_, lane);                                            \
                lk_[0] = k1_;                                                                \
              } else {                                                                       \
                /* the old list (still in memory) and the queue, exactly */                  \
                _Pragma("unroll") for (int r_ = 0; r_ < KL; ++r_) lk_[r_] = kKeyEmpty;       \
                _Pragma("unroll") for (int r_ = 0; r_ < KL + QB; ++r_) {                     \
                    uint32_t i_ = kSentinelIdx;                                              \
                    if (r_ < KL) {                                                           \
                        const int p_ = 64 * r_ + lane;                                       \
                        if (p_ < K2) i_ = LI[qg_ * K2 + p_];                                 \
                    } else if (64u * (uint32_t)(r_ - KL) + (uint32_t)lane < n_) {            \
                        i_ = QIw[(64u * (uint32_t)(r_ - KL) + (uint32_t)lane) * QPW + j_];   \
                    }                                                                        \
                    float x_ = inf;                                                          \
                    if (i_ != kSentinelIdx) x_ = MLRS_EXACT_AT(i_);                          \
                    if (x_ != x_) { x_ = inf; i_ = kSentinelIdx; }                           \
                    unsigned long long b_ = pair_key(x_, i_);                                \
                    wave_sort64_key(b_, lane);                                               \
                    (void)wave_merge_blocks_key_drop<KL>(lk_, b_, lane);                     \
                }                                                                            \
              }                                                                              \
                R_ = f32_from_order_bits(list_hi_at<KL>(lk_, k - 1));                        \
                if (lane == 0) L.mode[j_] = 1u;                                              \
            } else if (R_ < inf) {                                                           \
                R_ = round_up_f((double)R_ + (double)L.eps[j_]);                             \
            }                                                                                \
        }                                                                                    \
        _Pragma("unroll") for (int r_ = 0; r_ < KL; ++r_) {                                  \
            const int p_ = 64 * r_ + lane;                                                   \
            if (p_ < K2) {                                                                   \
                LV[qg_ * K2 + p_] = key_value(lk_[r_]);                                      \
                LI[qg_ * K2 + p_] = key_index(lk_[r_]);                                      \
            }                                                                                \
        }                                                                                    \
        if (SUMM) {                                                                          \
            const bool sv_ = !exact_ && L.mode[j_] == 0u;                                    \
            float p_[4] = {f32_from_order_bits(list_hi_at<KL>(lk_, rk1 - 1)),                \
                           f32_from_order_bits(list_hi_at<KL>(lk_, rk2 - 1)),                \
                           f32_from_order_bits(list_hi_at<KL>(lk_, rk3 - 1)),                \
                           f32_from_order_bits(list_hi_at<KL>(lk_, k - 1))};                 \
            if (lane == 0) {                                                                 \
                _Pragma("unroll") for (int i_ = 0; i_ < 4; ++i_)                             \
                    if (sv_ && p_[i_] < inf) p_[i_] = round_up_f((double)p_[i_] + (double)L.eps[j_]); \
                SUMM[slot * nq + qg_] = make_float4(p_[0], p_[1], p_[2], p_[3]);             \
            }                                                                                \
        }                                                                                    \
        if (lane == 0) {                                                                     \
            if (SHARED_R && R_ < inf) {                                                      \
                /* published without waiting for the old value: other segments' */           \
                /* bounds reach this one at its next refresh */                              \
                __hip_atomic_fetch_min(&SHARED_R[qg_], __float_as_uint(R_), __ATOMIC_RELAXED, \
                                       __HIP_MEMORY_SCOPE_AGENT);                            \
            }                                                                                \
            L.thr[j_] = fminf(L.thr[j_], screen_threshold<COS>(R_, L.qs[j_], L.eps[j_]));    \
        }                                                                                    \
        if (jl == j_) cntr = 0u;                                                             \
    } while (0)

    // ---- k = 1: every queued pair of the wave evaluated in lane-parallel
    //      batches, kept with a 64-bit LDS atomicMin on (value, index) ----
#define MLRS_FLUSH_K1()                                                                      \
    do {                                                                                     \
        const uint32_t c_ = (lane < QPW) ? cntr : 0u;                                        \
        uint32_t incl_ = c_;                                                                 \
        _Pragma("unroll") for (int m_ = 1; m_ < QPW; m_ <<= 1) {                             \
            const uint32_t o_ = (uint32_t)__shfl_up((int)incl_, m_, 64);                     \
            if ((lane & (QPW - 1)) >= m_) incl_ += o_;                                       \
        }                                                                                    \
        const uint32_t total_ = (uint32_t)__shfl((int)incl_, QPW - 1, 64);                   \
        if (lane < QPW) L.off[lane] = incl_ - c_;                                            \
        for (uint32_t base_ = 0; base_ < total_; base_ += 64) {                              \
            const uint32_t e_ = base_ + (uint32_t)lane;                                      \
            if (e_ < total_) {                                                               \
                int j_ = 0;                                                                  \
                _Pragma("unroll") for (int m_ = QPW / 2; m_ >= 1; m_ >>= 1) if (L.off[j_ + m_] <= e_) \
                    j_ += m_;                                                                \
                const uint32_t t_ = L.qidx[j_][e_ - L.off[j_]];                              \
                const float ya_ = row_operand<ARM>(a, t_);                                   \
                const float v_ = exact_f32<ARM, VEC4>(Q + (qwave + j_) * d, X + (int64_t)t_ * d, d, \
                                                       L.qa[j_], ya_);                       \
                if (v_ == v_)                                                                \
                    atomicMin(&L.best[j_], ((unsigned long long)__float_as_uint(v_) << 32) | t_); \
            }                                                                                \
        }                                                                                    \
        cntr = 0u;                                                                           \
        qlo = qlo0;                                                                          \
        if (lane < QPW) {                                                                    \
            float R_ = __uint_as_float((uint32_t)(L.best[lane] >> 32));                      \
            if (SHARED_R && qvalid && R_ < inf) {                                            \
                const unsigned int old_ = atomicMin(&SHARED_R[qmine], __float_as_uint(R_));  \
                R_ = fminf(R_, __uint_as_float(old_));                                       \
            }                                                                                \
            L.thr[lane] = fminf(L.thr[lane], screen_threshold<COS>(R_, L.qs[lane], L.eps[lane])); \
        }                                                                                    \
    } while (0)

    float4 pf[PF];
    float pfn = 0.0f;
    // Direct fill of tile T0 into DST: wave w's instruction i fills chunks
    // 64 (w PF + i) .. + 63 of the contiguous tile; chunk f is position f % CPR
    // of row f / CPR, which holds the row's column chunk position ^ (row & 15).
    // Rows past the segment are not loaded (their values are masked out of the
    // screen); the row norms go through a register as in the staged path.
    // pair layout: lane l loads chunk l % 32 of slot row 16 (l / 32)
    const uint32_t pair_off = (uint32_t)(16 * (lane >> 5) * DP + 4 * (lane & 31));
    auto direct_load = [&](float (&dst)[TILE_FL], uint32_t t0) {
        if constexpr (DIRECT && PAIRS) {
            // slots 4w .. 4w + 3: lane l loads chunk l % 32 of row slot + 16 (l / 32)
            if (FULLW && t_end32 - t0 >= (uint32_t)kBn) {
                // unpadded rows, whole tile (t0 + kBn could wrap): a
                // wave-uniform row base plus the lane's constant offset, so no
                // per-slot runtime strides are kept (they were scalar
                // registers spilled to VGPR lanes, read back every tile)
                const float* base = X + (int64_t)(t0 + (uint32_t)(4 * w)) * DP;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    global_to_lds16(base + (uint32_t)(i * DP + pair_off), &dst[(4 * w + i) * SLOT]);
            } else {
                const int rl = 16 * (lane >> 5);
                const float* xw = X + (int64_t)(t0 + (uint32_t)(4 * w)) * d + (int64_t)rl * d + 4 * (lane & 31);
                const int di = (int)d;
                if (4 * (lane & 31) < di) {
                    if (t_end32 - t0 >= (uint32_t)kBn) {  // whole tile (t0 + kBn could wrap)
#pragma unroll
                        for (int i = 0; i < 4; ++i) global_to_lds16(xw + i * di, &dst[(4 * w + i) * SLOT]);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (t0 + (uint32_t)(4 * w + i + rl) < t_end32)
                                global_to_lds16(xw + i * di, &dst[(4 * w + i) * SLOT]);
                    }
                }
            }
        } else if constexpr (DIRECT) {
            // rows w, w + WV, ... of the tile: this wave's first row
            // (wave-uniform) + the lane's chunk
            const float* xw = X + (int64_t)(t0 + (uint32_t)w) * d + 4 * lane;
            const int di = (int)d;
            if (lane < CPR && 4 * lane < di) {
                if (t_end32 - t0 >= (uint32_t)kBn) {  // whole tile (t0 + kBn could wrap)
#pragma unroll
                    for (int i = 0; i < RPW; ++i)
                        if (kBn % WV == 0 || w + WV * i < kBn)
                            global_to_lds16(xw + (int64_t)WV * i * di, &dst[(w + WV * i) * STRIDE]);
                } else {
#pragma unroll
                    for (int i = 0; i < RPW; ++i)
                        if ((kBn % WV == 0 || w + WV * i < kBn) && t0 + (uint32_t)(w + WV * i) < t_end32)
                            global_to_lds16(xw + (int64_t)WV * i * di, &dst[(w + WV * i) * STRIDE]);
                }
            }
        }
        // the tile's row norms, one per lane of wave 0 (the three-block-list
        // kernel tests the wave index and the lane, which measured faster
        // there: c2k128 25.04 -> 24.51 ms; the others test tid)
        if (KL > 1 ? (w == 0 && lane < kBn) : (tid < kBn)) {
            const uint32_t t = t0 + (uint32_t)(KL > 1 ? lane : tid);
            if (COS)
                pfn = (t < t_end32) ? XSCALE[t] : 0.0f;
            else
                pfn = (t < t_end32) ? XSQ[t] : inf;
        }
    };
    // the tile at T0: into registers (staged) or straight into DST (direct)
    auto load_tile = [&](float (&dst)[TILE_FL], int64_t t0) {
        if constexpr (DIRECT)
            direct_load(dst, (uint32_t)t0);
        else
            MLRS_PREFETCH(t0);
    };
    if (t_begin < t_end) load_tile(tileA, t_begin);
    __syncthreads();  // per-wave LDS init visible to the wave
    // Sign-bit screen (below): Euclidean waves whose valid queries are all in
    // screen-value mode (L.mode 0: no screen sum can overflow), where a NaN
    // screen value comes only from a row holding a NaN, whose exact value is
    // NaN and never kept, so the screen may drop it.  Used by the k = 1 and
    // three-block-list kernels; the k <= 64 narrow kernel and the wide shape
    // measured no faster with it (c2 +0.9%).
    constexpr bool kSignScreen = !COS && !W16 && (K1 || KL > 1);
    const bool nan_free =
        kSignScreen && __builtin_amdgcn_ballot_w64(lane < QPW && qvalid && L.mode[lane] != 0u) == 0;

    float thr = L.thr[jl];
    const float eps2 = 2.0f * L.eps[jl];  // k = 1 tightening (exact doubling)
    // k = 1: a lower bound on the screen values of the rows in query jl's
    // queue.  A NaN screen value can hide a finite exact value only where a
    // sum may overflow, so queries without screen-value mode (L.mode) keep
    // -inf and never drop queued rows; with it, NaN screen values come from
    // rows holding a NaN, whose exact values are NaN and never kept.
    const float qlo0 = (L.mode[jl] == 0u) ? inf : -inf;
    float qlo = qlo0;
    int tiles = 0;
    // One tile: CUR holds (or receives from the staging registers) the rows
    // at T0, the next tile is loaded towards NXT.
    auto tile_step = [&](float (&cur)[TILE_FL], float* __restrict__ tncur, float (&nxt)[TILE_FL],
                         int64_t t0) {
        // publish the tile: the staged registers are stored into CUR; the
        // direct loads into CUR are waited for, and the barrier makes every
        // wave's visible (and ends every wave's reads of NXT)
        if constexpr (DIRECT) {
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        } else {
#pragma unroll
            for (int p = 0; p < PF; ++p) {
                const int f = tid + NT * p;
                if (f < TILE_F4) {
                    const int r = f / (DP / 4);
                    const int c4 = f % (DP / 4);
                    *reinterpret_cast<float4*>(&cur[0] + chunk_at(r, c4)) = pf[p];
                }
            }
        }
        if (KL > 1 ? (w == 0 && lane < kBn) : (tid < kBn)) tncur[KL > 1 ? lane : tid] = pfn;
        __syncthreads();
        if (!SINGLE && t_end32 - (uint32_t)t0 > (uint32_t)kBn) load_tile(nxt, t0 + kBn);

        // The lane's tile values: narrow, acc[r] = row row_of(r); wide, r < 4
        // in acc0 (the first 16-row half) and r >= 4 in acc1.
        f32x16 acc;
        f32x4 acc0, acc1;
        if constexpr (!W16) {
            if (!COS) {
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    float4 n4 = *reinterpret_cast<const float4*>(&tncur[8 * g4 + 4 * h]);
                    acc[4 * g4 + 0] = n4.x;
                    acc[4 * g4 + 1] = n4.y;
                    acc[4 * g4 + 2] = n4.z;
                    acc[4 * g4 + 3] = n4.w;
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
            }
            // A operands double-buffered: the next group's LDS read is issued
            // before the current group's four MFMAs (the scheduling barriers keep
            // that order), so its latency hides under ~256 MFMA cycles.
            const float* arow = &cur[row_at(jl) + 4 * h];
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
            if (COS) {
                // rows scaled by -1/||x_t|| after the contraction (the scales ride
                // in tnorm), so the prefetched loads need no arithmetic before the
                // next tile's LDS store
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const float4 s4 = *reinterpret_cast<const float4*>(&tncur[8 * g4 + 4 * h]);
                    acc[4 * g4 + 0] *= s4.x;
                    acc[4 * g4 + 1] *= s4.y;
                    acc[4 * g4 + 2] *= s4.z;
                    acc[4 * g4 + 3] *= s4.w;
                }
            }
        } else {
            const float4 n0 = *reinterpret_cast<const float4*>(&tncur[4 * h]);
            const float4 n1 = *reinterpret_cast<const float4*>(&tncur[16 + 4 * h]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc0[r] = COS ? 0.0f : (&n0.x)[r];
                acc1[r] = COS ? 0.0f : (&n1.x)[r];
            }
            // A operands: this lane's rows jl and 16 + jl, its quarter's chunk
            // i, one group ahead; each chunk feeds eight MFMAs (four k-steps
            // on each half).
            const float* t0p = &cur[0];
            const int c0 = h * (QQ / 4);
            float4 av0 = *reinterpret_cast<const float4*>(t0p + chunk_at(jl, c0));
            float4 av1 = *reinterpret_cast<const float4*>(t0p + chunk_at(16 + jl, c0));
#pragma unroll
            for (int i = 0; i < NQR; ++i) {
                float4 an0 = av0, an1 = av1;
                if (i + 1 < NQR) {
                    an0 = *reinterpret_cast<const float4*>(t0p + chunk_at(jl, c0 + i + 1));
                    an1 = *reinterpret_cast<const float4*>(t0p + chunk_at(16 + jl, c0 + i + 1));
                }
                __builtin_amdgcn_sched_barrier(0);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(av0.x, qreg[i].x, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(av1.x, qreg[i].x, acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(av0.y, qreg[i].y, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(av1.y, qreg[i].y, acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(av0.z, qreg[i].z, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(av1.z, qreg[i].z, acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(av0.w, qreg[i].w, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(av1.w, qreg[i].w, acc1, 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                av0 = an0;
                av1 = an1;
            }
            if (COS) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc0[r] *= (&n0.x)[r];
                    acc1[r] *= (&n1.x)[r];
                }
            }
        }
        if constexpr (SINGLE) {
            // every wave's chain has read the tile (and its norms): refill it
            // under this tile's screen
            __syncthreads();
            if (t_end32 - (uint32_t)t0 > (uint32_t)kBn) load_tile(nxt, t0 + kBn);
        }
        auto val = [&](int r) -> float {
            if constexpr (W16) return r < 4 ? acc0[r] : acc1[r - 4];
            else return acc[r];
        };

        // ---- k = 1: tighten with this tile's smallest expansion value ----
        if (K1 && !COS) {  // the k = 1 kernel (every k = 1 search launches it)
            float m = inf;
#pragma unroll
            for (int r = 0; r < SH::vals; ++r) m = fminf(m, val(r));  // NaN ignored; past-end rows are +inf
            if (W16) m = fminf(m, shfl_xor_f(m, 16));
            m = fminf(m, shfl_xor_f(m, 32));
            if (m < inf) {
                // m + 2 eps rounded to nearest, then stepped up by at least one
                // ulp (2^-126 near zero): an upper bound of the exact sum
                const float s_ = m + eps2;
                thr = fminf(thr, s_ + (__builtin_fabsf(s_) * 0x1p-23f + 0x1p-126f));
            }
            if constexpr (K1) {
                // Rows queued on earlier tiles whose screen values all exceed
                // the tightened threshold cannot be the nearest row (nor tie
                // with it): the queue restarts before this tile's rows join it.
                // Each new running minimum used to leave its predecessors queued
                // (about ln(tiles) rows per query at each flush).
                if (qlo > thr) {
                    cntr = 0u;
                    qlo = inf;
                }
                qlo = fminf(qlo, m);
            }
        }

        // ---- screen: value r of the lane is tile row row_of(r) for query jl.
        //      Passing rows are appended to the query's queue at cntr (kept in
        //      registers, equal in every lane of the query); the lanes of a
        //      query write in lane order, each after the earlier lanes' entries. ----
        uint32_t m = 0;
        if (kSignScreen && nan_free) {
            // pass <=> thr - value >= +0: the rounded difference has the sign
            // of the exact one (x - x = +0), thr + 0 turns a -0 threshold into
            // +0, and v_alignbit shifts each sign bit into the fail mask:
            // two instructions per value and no compare-mask hazards
            const float t_ = thr + 0.0f;
            uint32_t f = 0;
#pragma unroll
            for (int r = SH::vals - 1; r >= 0; --r)
                f = __builtin_amdgcn_alignbit(f, __float_as_uint(t_ - val(r)), 31);
            m = f ^ ((1u << SH::vals) - 1u);
        } else {
#pragma unroll
            for (int r = 0; r < SH::vals; ++r) m |= (uint32_t)!(val(r) > thr) << r;
        }
        if (!qvalid) m = 0;
        // Partial tile (the segment's last): rows past the segment are not
        // candidates.  Rows left are compared in 32 bits, a scalar branch; a
        // 64-bit ordered compare is a vector instruction, and the compiler
        // then computed this mask on every tile.
        if (t_end32 - (uint32_t)t0 < (uint32_t)kBn) {
#pragma unroll
            for (int r = 0; r < SH::vals; ++r)
                if ((uint32_t)t0 + (uint32_t)row_of(r) >= t_end32) m &= ~(1u << r);
        }
        if (__builtin_amdgcn_ballot_w64(m != 0)) {
            const uint32_t c = (uint32_t)__builtin_popcount(m);
            uint32_t before, total;
            if constexpr (W16) {
                // exclusive prefix and total over the query's four lanes (h = 0..3)
                const uint32_t u1 = (uint32_t)__shfl_up((int)c, 16, 64);
                const uint32_t s1 = c + (h >= 1 ? u1 : 0u);
                const uint32_t u2 = (uint32_t)__shfl_up((int)s1, 32, 64);
                const uint32_t incl = s1 + (h >= 2 ? u2 : 0u);
                before = incl - c;
                total = (uint32_t)__shfl((int)incl, 48 + jl, 64);
            } else {
                const uint32_t co = shfl_xor_u(c, 32);
                before = h ? co : 0u;
                total = c + co;
            }
            uint32_t pos = cntr + before;
            const uint32_t tb = (uint32_t)t0;
            if (K1) {
                while (m) {
                    const int r = __builtin_ctz(m);
                    m &= m - 1;
                    L.qidx[jl][pos++] = tb + (uint32_t)row_of(r);
                }
            } else {
                // one iteration per admitted row of the lane (usually one)
                while (m) {
                    const int r = __builtin_ctz(m);
                    m &= m - 1;
                    QIw[pos * QPW + jl] = tb + (uint32_t)row_of(r);
                    if constexpr (W16) QVw[pos * QPW + jl] = pick8(acc0, acc1, r);
                    else QVw[pos * QPW + jl] = pick16(acc, r);
                    ++pos;
                }
            }
            cntr += total;
        }
        // ---- flush queries whose queue could overflow on the next tile ----
        uint64_t mask = __builtin_amdgcn_ballot_w64(lane < QPW && cntr > (uint32_t)kFlushAt);
        if (mask) {
            if (lane < QPW) L.thr[lane] = fminf(L.thr[lane], thr);
            if (K1) {
                MLRS_FLUSH_K1();
            } else {
                // the queued screen values were stored by other lanes of this wave
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
                while (mask) {
                    const int j = __builtin_ctzll(mask);
                    mask &= mask - 1;
                    MLRS_FLUSH(j);
                }
            }
            thr = L.thr[jl];
        }
        // ---- pick up thresholds tightened by other strips of these queries ----
        rotate_wave_priority((uint32_t)tiles + 1u, GramOcc<NG, K1, KL, VEC4>::wgs);
        if (SHARED_R && (++tiles % share_every(K1, KL, W16)) == 0) {
            if (lane < QPW && qvalid) {
                float R = __uint_as_float(SHARED_R[qmine]);
                if (nsum > 0) {
                    // the smallest T with at least k pairs <= T over the
                    // segment summaries: the four smallest (value, rank
                    // increment) pairs, accumulated in order
                    float b0 = inf, b1 = inf, b2 = inf, b3 = inf;
                    int i0 = 0, i1 = 0, i2 = 0, i3 = 0;
                    const int inc[4] = {rk1, rk2 - rk1, rk3 - rk2, k - rk3};
                    for (int64_t s0 = 0; s0 < nsum; s0 += 4) {
                        // four summaries in flight, then folded in
                        float4 v4s[4];
#pragma unroll
                        for (int u = 0; u < 4; ++u)
                            v4s[u] = (s0 + u < nsum) ? SUMM[(s0 + u) * nq + qmine] : make_float4(inf, inf, inf, inf);
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            const float4 v4 = v4s[i >> 2];
                            const float v = ((i & 3) == 0) ? v4.x : ((i & 3) == 1) ? v4.y : ((i & 3) == 2) ? v4.z : v4.w;
                            const int n = inc[i & 3];
                            const bool c0 = v < b0, c1 = v < b1, c2 = v < b2, c3 = v < b3;
                            b3 = c2 ? b2 : (c3 ? v : b3);
                            i3 = c2 ? i2 : (c3 ? n : i3);
                            b2 = c1 ? b1 : (c2 ? v : b2);
                            i2 = c1 ? i1 : (c2 ? n : i2);
                            b1 = c0 ? b0 : (c1 ? v : b1);
                            i1 = c0 ? i0 : (c1 ? n : i1);
                            b0 = c0 ? v : b0;
                            i0 = c0 ? n : i0;
                        }
                    }
                    float T = inf;
                    int got = i0;
                    if (got >= k) {
                        T = b0;
                    } else {
                        got += i1;
                        if (got >= k) {
                            T = b1;
                        } else {
                            got += i2;
                            if (got >= k) {
                                T = b2;
                            } else {
                                got += i3;
                                if (got >= k) T = b3;
                            }
                        }
                    }
                    R = fminf(R, T);
                }
                L.thr[lane] = fminf(fminf(L.thr[lane], thr), screen_threshold<COS>(R, L.qs[lane], L.eps[lane]));
            }
            thr = L.thr[jl];
        }
    };
    if constexpr (SINGLE) {
        for (int64_t t0 = t_begin; t0 < t_end; t0 += kBn) tile_step(tileA, tnA, tileA, t0);
    } else {
        for (int64_t t0 = t_begin; t0 < t_end; t0 += 2 * kBn) {
            tile_step(tileA, tnA, tileB, t0);
            if (t0 + kBn < t_end) tile_step(tileB, tnB, tileA, t0 + kBn);
        }
    }

    // ---- final flush of every non-empty queue ----
    {
        uint64_t mask = __builtin_amdgcn_ballot_w64(lane < QPW && cntr > 0u);
        if (K1) {
            if (mask) MLRS_FLUSH_K1();
        } else {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            while (mask) {
                const int j = __builtin_ctzll(mask);
                mask &= mask - 1;
                MLRS_FLUSH(j);
            }
        }
    }
#undef MLRS_FLUSH_K1
#undef MLRS_FLUSH
#undef MLRS_EXACT_AT
#undef MLRS_PREFETCH
#undef MLRS_PF_SRC
#undef MLRS_PF_ROW
#undef MLRS_PF_ON

    // ---- k = 1: the kept pair becomes this segment's one-entry list ----
    if (K1 && lane < QPW && qvalid) {
        const unsigned long long b = L.best[lane];
        LV[qmine] = __uint_as_float((uint32_t)(b >> 32));
        LI[qmine] = (uint32_t)b;
    }
    u += tile1 - tile0;
    __syncthreads();  // LDS state and tile buffers are reused by the next segment
    }
}

// Initial per-query bound: the k-th smallest exact value over an evenly
// spaced sample of index rows (seed_kth_block).  Any k distinct rows bound the
// final k-th value from above, so the screen starts tight instead of at +inf.
// SB: 64-entry blocks of the running sample list (k <= 64 SB).
template <int ARM, int SB>
__global__ __launch_bounds__(256) void knn_seed_f32_kernel(GramArgs32 a, int64_t nsamp) {
    const float* qop = (ARM == ARM_COS_FOLD) ? a.qsq : a.qinv;
    const float* yop = (ARM == ARM_COS_FOLD) ? a.xsq : a.xinv;
    seed_kth_block<float, ARM, unsigned int, SB>(a.q, a.x, a.nq, a.nt, a.d, a.k, nsamp, qop, yop, a.shared_r);
}

// Merge the per-segment lists of one query per wave and emit the output
// transform (the strip merge of select_k_onepass_indexed,
// crates/mlrs-kernels/src/topk.rs:612-758, here over sorted lists).  Every
// list entry's value lies within eps of its pair's exact value (exact-mode
// entries equal it), and the segments hold disjoint index rows.  So with V
// the k-th smallest value over all lists, k distinct pairs are exactly <=
// V + eps, and a pair can be among the k best only if its value is
// <= V + 2 eps: exactly those pairs are evaluated in the reference arm's
// operation order and ranked by (exact value, index), NaN never admitted.
template <int ARM, bool VEC4>
__global__ __launch_bounds__(256) void knn_merge_f32_kernel(GramArgs32 a) {
    __shared__ uint32_t cand[4][128];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int64_t qg = (int64_t)blockIdx.x * 4 + wv;
    if (qg >= a.nq) return;
    const int k = a.k;
    const int K2 = gram_list_cap(k);
    const int64_t d = a.d;
    const float inf = __builtin_huge_valf();
    const StreamSplit sp(a.nq, a.nt, a.qpb, kBn, a.grid_wgs);
    const int64_t nsl = sp.slots_of(qg / a.qpb);
    // the k-th smallest value over the union of the lists
    float uv = inf;
    uint32_t ui = kSentinelIdx;
    for (int64_t s = 0; s < nsl; ++s) {
        float v = inf;
        uint32_t ix = kSentinelIdx;
        if (lane < K2) {
            const int64_t o = (s * a.nq + qg) * K2 + lane;
            v = a.part_val[o];
            ix = a.part_idx[o];
        }
        wave_merge64<float>(uv, ui, v, ix, lane);
    }
    const float qsq = a.qsq[qg];
    const float eps = (ARM == ARM_COS_FOLD || ARM == ARM_COS_HOST)
                          ? (float)a.eps_abs
                          : (float)(a.eps_rel * ((double)qsq + (double)a.stats->xsq_max) + a.eps_abs);
    double W = (double)bcast_f(uv, k - 1) + 2.0 * (double)eps;
    W += __builtin_fabs(W) * 0x1p-40;
    // exact evaluation of the window's pairs, compacted 64 at a time
    float lv = inf;
    uint32_t li = kSentinelIdx;
    uint32_t nc = 0;
    auto evaluate = [&](uint32_t count) {
        float e = inf;
        uint32_t t = kSentinelIdx;
        if ((uint32_t)lane < count) {
            t = cand[wv][lane];
            e = exact_f32<ARM, VEC4, 8>(a.q + qg * d, a.x + (int64_t)t * d, d, query_operand<ARM>(a, qg),
                                        row_operand<ARM>(a, t));
            if (e != e) {
                e = inf;
                t = kSentinelIdx;
            }
        }
        wave_sort64<float>(e, t, lane);
        wave_merge64<float>(lv, li, e, t, lane);
    };
    for (int64_t s = 0; s < nsl; ++s) {
        bool in = false;
        uint32_t ix = kSentinelIdx;
        if (lane < K2) {
            const int64_t o = (s * a.nq + qg) * K2 + lane;
            ix = a.part_idx[o];
            in = (ix != kSentinelIdx) && !((double)a.part_val[o] > W);
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
    if (lane < k) emit_pair(a.mode, a.q, a.x, a.qsq, a.xsq, a.d, k, qg, lane, lv, li, a.out_val, a.out_idx);
}

// 64 < k <= 128: the same merge over lists of up to three 64-entry blocks
// (k + 32 entries).  The union and the result are kept as two-block lists
// (the k smallest fit in 128 entries), merged block by block on 64-bit
// (value bits, index) keys.
template <int ARM, bool VEC4>
__global__ __launch_bounds__(256) void knn_merge_blocks_f32_kernel(GramArgs32 a) {
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
    const StreamSplit sp(a.nq, a.nt, a.qpb, kBn, a.grid_wgs);
    const int64_t nsl = sp.slots_of(qg / a.qpb);
    // the k-th smallest value over the union of the lists
    unsigned long long u[UB];
#pragma unroll
    for (int r = 0; r < UB; ++r) u[r] = kKeyEmpty;
    for (int64_t s = 0; s < nsl; ++s) {
#pragma unroll
        for (int r = 0; r < SLB; ++r) {
            if (64 * r >= K2) break;
            const int p = 64 * r + lane;
            unsigned long long key = kKeyEmpty;
            if (p < K2) {
                const int64_t o = (s * a.nq + qg) * K2 + p;
                key = pair_key(a.part_val[o], a.part_idx[o]);
            }
            (void)wave_merge_blocks_key_drop<UB>(u, key, lane);
        }
    }
    const float qsq = a.qsq[qg];
    const float eps = (ARM == ARM_COS_FOLD || ARM == ARM_COS_HOST)
                          ? (float)a.eps_abs
                          : (float)(a.eps_rel * ((double)qsq + (double)a.stats->xsq_max) + a.eps_abs);
    double W = (double)f32_from_order_bits(list_hi_at<UB>(u, k - 1)) + 2.0 * (double)eps;
    W += __builtin_fabs(W) * 0x1p-40;
    // exact evaluation of the window's pairs, compacted 64 at a time
    unsigned long long res[UB];
#pragma unroll
    for (int r = 0; r < UB; ++r) res[r] = kKeyEmpty;
    uint32_t nc = 0;
    auto evaluate = [&](uint32_t count) {
        float e = __builtin_huge_valf();
        uint32_t t = kSentinelIdx;
        if ((uint32_t)lane < count) {
            t = cand[wv][lane];
            e = exact_f32<ARM, VEC4, 8>(a.q + qg * d, a.x + (int64_t)t * d, d, query_operand<ARM>(a, qg),
                                        row_operand<ARM>(a, t));
            if (e != e) {
                e = __builtin_huge_valf();
                t = kSentinelIdx;
            }
        }
        unsigned long long ek = pair_key(e, t);
        wave_sort64_key(ek, lane);
        (void)wave_merge_blocks_key_drop<UB>(res, ek, lane);
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
                in = (ix != kSentinelIdx) && !((double)a.part_val[o] > W);
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
        if (slot < k)
            emit_pair(a.mode, a.q, a.x, a.qsq, a.xsq, a.d, k, qg, slot, key_value(res[r]), key_index(res[r]),
                      a.out_val, a.out_idx);
    }
}

// k = 1: the same merge with one lane per query (the segment lists are one
// pair each, so the merge is a (value, index) minimum).
__global__ __launch_bounds__(256) void knn_merge1_f32_kernel(GramArgs32 a) {
    const int64_t qg = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (qg >= a.nq) return;
    float lv = a.part_val[qg];
    uint32_t li = a.part_idx[qg];
    const StreamSplit sp(a.nq, a.nt, a.qpb, kBn, a.grid_wgs);
    const int64_t nsl = sp.slots_of(qg / a.qpb);
    for (int64_t s = 1; s < nsl; ++s) {
        const float v = a.part_val[s * a.nq + qg];
        const uint32_t ix = a.part_idx[s * a.nq + qg];
        if (pair_less<float>(v, ix, lv, li)) {
            lv = v;
            li = ix;
        }
    }
    emit_pair(a.mode, a.q, a.x, a.qsq, a.xsq, a.d, 1, qg, 0, lv, li, a.out_val, a.out_idx);
}

// Seed on the matrix cores (d <= 256, 16-byte rows): the screen value of
// every (query, sampled row) pair, formed as the narrow main kernel forms it
// (Euclidean: acc = ||x||^2, then v_mfma_f32_32x32x2f32 over -2 q; cosine:
// the contraction over q scaled by -1/||x|| afterwards; above d = 128 too,
// where the main kernel contracts on 16x16x4 tiles: the screen bound holds
// for any summation order), turned into the distance it stands for, rounded
// up -- u = max(acc + ||q||^2, 0) or clamp(1 + acc/||q||, 0, 2) -- and
// written to S[q][s] (NaN for a NaN screen value, which the selection never
// admits).  The k-th smallest u then bounds the query's k-th exact value
// once eps is added (k sampled rows have exact <= u + eps <= u_k + eps).  A
// workgroup takes 128 queries and one contiguous range of the sample's
// 32-row tiles (blockIdx.y: the tiles are split so that the launch fills the
// chip); sampled row s is index row s * n / m.  The next tile's rows are
// loaded into registers while the current tile's MFMA chain runs.
template <int NG, bool COS>
__global__ __launch_bounds__(256, 2) void knn_seed_screen_f32_kernel(GramArgs32 a, int64_t nsamp,
                                                                     float* __restrict__ S, int64_t ld) {
    constexpr int DP = NG * 8;
    constexpr int STRIDE = DP + 4;
    __shared__ __attribute__((aligned(16))) float tile[kBn * STRIDE];
    __shared__ __attribute__((aligned(16))) float tn[kBn];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, jl = lane & 31;
    const int64_t nq = a.nq, nt = a.nt, d = a.d;
    const float inf = __builtin_huge_valf();
    const int64_t q = (int64_t)blockIdx.x * kQpbNarrow + (int64_t)w * 32 + jl;
    const bool qvalid = q < nq;
    const int64_t qrow = qvalid ? q : nq - 1;
    const float qsq = a.qsq[qrow];
    const float qs = COS ? __builtin_sqrtf(qsq) : qsq;  // the main kernel's screen operand
    const float scale = COS ? 1.0f : -2.0f;
    float4 qreg[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int64_t c = 8 * g + 4 * h;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < d) v = *reinterpret_cast<const float4*>(a.q + qrow * d + c);
        qreg[g] = make_float4(scale * v.x, scale * v.y, scale * v.z, scale * v.w);
    }
    const int64_t ntiles = (nsamp + kBn - 1) / kBn;
    const int64_t per = (ntiles + gridDim.y - 1) / gridDim.y;
    const int64_t s_lo = (int64_t)blockIdx.y * per * kBn;
    int64_t s_hi = s_lo + per * kBn;
    if (s_hi > nsamp) s_hi = nsamp;
    // staging: chunk f = tid + 256 p is column chunk f % (DP / 4) of tile row
    // f / (DP / 4); the next tile is loaded into registers under the chain
    constexpr int PF = (kBn * DP / 4 + 255) / 256;
    float4 pf[PF];
    float pfn = 0.0f;
    auto load_tile = [&](int64_t s0) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int f = tid + 256 * p;
            const int r = f / (DP / 4), c4 = f % (DP / 4);
            const int64_t sr = s0 + r;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (f < kBn * DP / 4 && sr < nsamp && 4 * c4 < d)
                v = *reinterpret_cast<const float4*>(a.x + ((sr * nt) / nsamp) * d + 4 * c4);
            pf[p] = v;
        }
        if (tid < kBn) {
            const int64_t sr = s0 + tid;
            const int64_t t = (sr < nsamp) ? (sr * nt) / nsamp : 0;
            pfn = (sr < nsamp) ? (COS ? a.xscale[t] : a.xsq[t]) : (COS ? 0.0f : inf);
        }
    };
    if (s_lo < s_hi) load_tile(s_lo);
    for (int64_t s0 = s_lo; s0 < s_hi; s0 += kBn) {
        __syncthreads();  // the previous tile is no longer read
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int f = tid + 256 * p;
            if (f < kBn * DP / 4)
                *reinterpret_cast<float4*>(&tile[(f / (DP / 4)) * STRIDE + 4 * (f % (DP / 4))]) = pf[p];
        }
        if (tid < kBn) tn[tid] = pfn;
        __syncthreads();
        if (s0 + kBn < s_hi) load_tile(s0 + kBn);  // in flight under the chain
        f32x16 acc;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const float4 n4 = *reinterpret_cast<const float4*>(&tn[8 * g4 + 4 * h]);
            acc[4 * g4 + 0] = COS ? 0.0f : n4.x;
            acc[4 * g4 + 1] = COS ? 0.0f : n4.y;
            acc[4 * g4 + 2] = COS ? 0.0f : n4.z;
            acc[4 * g4 + 3] = COS ? 0.0f : n4.w;
        }
        const float* arow = &tile[jl * STRIDE + 4 * h];
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const float4 av = *reinterpret_cast<const float4*>(arow + 8 * g);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, qreg[g].x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, qreg[g].y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, qreg[g].z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, qreg[g].w, acc, 0, 0, 0);
        }
        if (qvalid) {
            // values r = 4 g4 .. 4 g4 + 3 are four consecutive sampled rows:
            // one 16-byte store (ld and s0 are multiples of 4)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                float u4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * g4 + e;
                    // cosine: the contraction scaled by -1/||x|| afterwards, as
                    // in the main kernel
                    const float v = COS ? acc[r] * tn[8 * g4 + 4 * h + e] : acc[r];
                    float u = __builtin_nanf("");
                    if (v == v) {
                        if (COS) {
                            u = round_up_f(1.0 + (double)v / (double)qs);
                            u = u < 0.0f ? 0.0f : (u > 2.0f ? 2.0f : u);
                        } else {
                            u = round_up_f((double)v + (double)qs);
                            u = u < 0.0f ? 0.0f : u;
                        }
                    }
                    u4[e] = u;
                }
                const int64_t sr0 = s0 + 8 * g4 + 4 * h;
                if (sr0 + 3 < nsamp) {
                    *reinterpret_cast<float4*>(S + q * ld + sr0) = make_float4(u4[0], u4[1], u4[2], u4[3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (sr0 + e < nsamp) S[q * ld + sr0 + e] = u4[e];
                }
            }
        }
    }
}

// The seed bound from each query's k-th smallest u (out_val[q][k - 1]):
// round_up(u_k + eps), for queries in screen-value mode (norms well inside
// the float range); +inf otherwise.
__global__ void seed_screen_finalize_kernel(GramArgs32 a, const float* __restrict__ kv, int k, int cos) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= a.nq) return;
    const float inf = __builtin_huge_valf();
    const double qsq = (double)a.qsq[q], xmax = (double)a.stats->xsq_max;
    const double eps = cos ? a.eps_abs : a.eps_rel * (qsq + xmax) + a.eps_abs;
    const float vk = kv[q * k + (k - 1)];
    float R = inf;
    // cosine: a zero query ties every row and is never screened
    if (qsq + xmax <= 0x1p124 && eps < 0x1p120 && vk < inf && (!cos || qsq > 0.0))
        R = round_up_f((double)vk + eps);
    a.shared_r[q] = __float_as_uint(R);
}

// The shared per-query threshold words start at +inf (as float bits).
__global__ void fill_inf_bits_kernel(unsigned int* p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0x7F800000u;
}

template <int NG, int ARM, bool COS, bool VEC4>
hipError_t launch_ng(const GramArgs32& a, int64_t nblocks, hipStream_t s) {
    dim3 grid((unsigned)StreamSplit(a.nq, a.nt, a.qpb, kBn, a.grid_wgs).G);
    const dim3 block(GramShape<(NG > 16)>::threads);
    (void)nblocks;
    // rows exactly 128 floats wide take the paired-row kernels' fixed-stride
    // instance (k > 1: the k = 1 kernel stages its tiles)
    constexpr bool kPairs = NG == 16 && VEC4;
    const bool fullw = kPairs && a.d == 8 * NG;
    if (a.k == 1)
        hipLaunchKernelGGL((knn_gram_f32_kernel<NG, ARM, COS, VEC4, true, 1>), grid, block, 0, s, a);
    else if (a.k <= 64 && fullw)
        hipLaunchKernelGGL((knn_gram_f32_kernel<NG, ARM, COS, VEC4, false, 1, kPairs>), grid, block, 0, s, a);
    else if (a.k <= 64)
        hipLaunchKernelGGL((knn_gram_f32_kernel<NG, ARM, COS, VEC4, false, 1>), grid, block, 0, s, a);
    else if (fullw)
        hipLaunchKernelGGL((knn_gram_f32_kernel<NG, ARM, COS, VEC4, false, 3, kPairs>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((knn_gram_f32_kernel<NG, ARM, COS, VEC4, false, 3>), grid, block, 0, s, a);
    return hipGetLastError();
}

template <int ARM, bool COS, bool VEC4>
hipError_t launch_arm(const GramArgs32& a, int64_t nblocks, hipStream_t s) {
    const int ng = (int)((a.d + 7) / 8);
    // the split and the merge must see the query-block size of the shape
    if (a.qpb != (ng > 16 ? kQpbWide : kQpbNarrow)) return hipErrorInvalidValue;
    if (ng <= 2) return launch_ng<2, ARM, COS, VEC4>(a, nblocks, s);
    if (ng <= 4) return launch_ng<4, ARM, COS, VEC4>(a, nblocks, s);
    if (ng <= 8) return launch_ng<8, ARM, COS, VEC4>(a, nblocks, s);
    if (ng <= 12) return launch_ng<12, ARM, COS, VEC4>(a, nblocks, s);
    if (ng <= 16) return launch_ng<16, ARM, COS, VEC4>(a, nblocks, s);
    if (ng <= 24) return launch_ng<24, ARM, COS, VEC4>(a, nblocks, s);
    return launch_ng<32, ARM, COS, VEC4>(a, nblocks, s);
}

template <int ARM, bool COS, bool VEC4>
hipError_t launch_wide(const GramArgs32& a, int64_t nblocks, hipStream_t s) {
    const int ng = (int)((a.d + 7) / 8);
    if (ng <= 16 || a.qpb != kQpbWide) return hipErrorInvalidValue;
    if (ng <= 24) return launch_ng<24, ARM, COS, VEC4>(a, nblocks, s);
    return launch_ng<32, ARM, COS, VEC4>(a, nblocks, s);
}

template <int ARM>
hipError_t launch_seed(const GramArgs32& a, int64_t nsamp, hipStream_t s) {
    const dim3 grid((unsigned)((a.nq + kSeedQpb - 1) / kSeedQpb));
    if (a.k <= 64)
        hipLaunchKernelGGL((knn_seed_f32_kernel<ARM, 1>), grid, dim3(256), 0, s, a, nsamp);
    else
        hipLaunchKernelGGL((knn_seed_f32_kernel<ARM, 2>), grid, dim3(256), 0, s, a, nsamp);
    return hipGetLastError();
}

}  // namespace

int gram_f32_queries_per_block(int64_t d) { return d > 128 ? kQpbWide : kQpbNarrow; }


void gram_f32_split(int64_t nq, int64_t nt, int64_t d, int k, int cus, bool vec4, int64_t* grid_wgs, int* nslots) {
    const int64_t qpb = gram_f32_queries_per_block(d);
    const StreamSplit full(nq, nt, qpb, kBn, 1);
    // one resident round (gram_f32_wgs_per_cu workgroups per CU), but at
    // least 16 tiles each
    const int per_cu = gram_f32_wgs_per_cu((int)((d + 7) / 8), k == 1, k <= 64 ? 1 : 3, vec4);
    int64_t g0 = per_cu * (int64_t)(cus > 0 ? cus : 1);
    if (g0 > full.T / 16) g0 = full.T / 16;
    if (g0 < 1) g0 = 1;
    *grid_wgs = g0;
    *nslots = (int)StreamSplit(nq, nt, qpb, kBn, g0).nslots();
}

int gram_f32_max_k() { return kKcap; }
int gram_f32_max_d() { return 256; }
int gram_f32_rows_per_tile() { return kBn; }

// Rows the matrix-core seed samples: 128 k, at most 8192 and nt / 128, at
// least 512 -- more than the exact seed's cap, since a sampled pair costs a
// few MFMA cycles here instead of a d-long FMA chain.  c2 with k = 128: 7812
// rows, step 27.2 -> 26.6 ms against the exact seed's 1953 (kernel 26.3 ->
// 25.2 ms); k = 32 takes 4096: kernel 20.76 -> 20.68 ms against 2048 at the
// same step (8192 rows at k = 32: kernel 20.59 ms, step +0.1 ms).
static int64_t seed_screen_rows(int64_t nt, int k) {
    int64_t n = 128 * (int64_t)k;
    if (n > 8192) n = 8192;
    if (n > nt / 128) n = nt / 128;
    if (n < 512) n = 512;
    return nt < n ? nt : n;
}

template <bool COS>
static void launch_seed_screen_ng(const GramArgs32& a, int64_t nsamp, float* S, int64_t ld, dim3 grid, int ng,
                                  hipStream_t s) {
    if (ng <= 4)
        hipLaunchKernelGGL((knn_seed_screen_f32_kernel<4, COS>), grid, dim3(256), 0, s, a, nsamp, S, ld);
    else if (ng <= 8)
        hipLaunchKernelGGL((knn_seed_screen_f32_kernel<8, COS>), grid, dim3(256), 0, s, a, nsamp, S, ld);
    else if (ng <= 12)
        hipLaunchKernelGGL((knn_seed_screen_f32_kernel<12, COS>), grid, dim3(256), 0, s, a, nsamp, S, ld);
    else if (ng <= 16)
        hipLaunchKernelGGL((knn_seed_screen_f32_kernel<16, COS>), grid, dim3(256), 0, s, a, nsamp, S, ld);
    else if (ng <= 24)
        hipLaunchKernelGGL((knn_seed_screen_f32_kernel<24, COS>), grid, dim3(256), 0, s, a, nsamp, S, ld);
    else
        hipLaunchKernelGGL((knn_seed_screen_f32_kernel<32, COS>), grid, dim3(256), 0, s, a, nsamp, S, ld);
}

size_t gram_f32_seed_screen_bytes(int64_t nq, int64_t nt, int64_t d, int k, int arm, bool vec4) {
    if (k <= 1 || k > kKcap || d > 256 || !vec4) return 0;
    const int64_t nsamp = seed_screen_rows(nt, k);
    if (nsamp < k) return 0;
    const int64_t ld = (nsamp + 3) / 4 * 4;
    const size_t bytes = (size_t)nq * (size_t)ld * 4 + 2 * (((size_t)nq * (size_t)k * 4 + 255) & ~(size_t)255) + 512;
    return bytes <= ((size_t)512 << 20) ? bytes : 0;  // larger searches keep the exact seed
}

hipError_t launch_gram_f32_prep(const GramArgs32& a, int arm, hipStream_t s, void* seed_buf) {
    if (!a.shared_r) return hipSuccess;
    if (a.summ) {
        const int64_t n = (int64_t)a.nslots * a.nq * 4;
        hipLaunchKernelGGL(fill_inf_bits_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                           reinterpret_cast<unsigned int*>(a.summ), n);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (a.k > 1) {
        const int64_t nsamp = seed_buf ? seed_screen_rows(a.nt, a.k) : gram_seed_rows(a.nt, a.k);
        if (seed_buf) {
            const int64_t ld = (nsamp + 3) / 4 * 4;
            float* S = static_cast<float*>(seed_buf);
            char* p = reinterpret_cast<char*>(S + (size_t)a.nq * (size_t)ld);
            p = reinterpret_cast<char*>(((uintptr_t)p + 255) & ~(uintptr_t)255);
            float* kv = reinterpret_cast<float*>(p);
            p += ((size_t)a.nq * (size_t)a.k * 4 + 255) & ~(size_t)255;
            uint32_t* ki = reinterpret_cast<uint32_t*>(p);
            // about four workgroups per CU: the sample's tiles split over blockIdx.y
            const int64_t nqb = (a.nq + kQpbNarrow - 1) / kQpbNarrow;
            const int64_t ntiles = (nsamp + kBn - 1) / kBn;
            int64_t ys = (1024 + nqb - 1) / nqb;
            if (ys > ntiles) ys = ntiles;
            if (ys > 65535) ys = 65535;
            if (ys < 1) ys = 1;
            const dim3 grid((unsigned)nqb, (unsigned)ys);
            const int ng = (int)((a.d + 7) / 8);
            const bool cos = (arm == ARM_COS_FOLD || arm == ARM_COS_HOST);
            if (cos)
                launch_seed_screen_ng<true>(a, nsamp, S, ld, grid, ng, s);
            else
                launch_seed_screen_ng<false>(a, nsamp, S, ld, grid, ng, s);
            hipError_t e = hipGetLastError();
            if (e == hipSuccess) e = launch_select_rows<float>(S, a.nq, nsamp, ld, a.k, EMIT_IDENTITY, kv, ki, nullptr, s);
            if (e != hipSuccess) return e;
            hipLaunchKernelGGL(seed_screen_finalize_kernel, dim3((unsigned)((a.nq + 255) / 256)), dim3(256), 0, s, a,
                               kv, a.k, cos ? 1 : 0);
            return hipGetLastError();
        }
        if (arm == ARM_EUCLID_FMA) return launch_seed<ARM_EUCLID_FMA>(a, nsamp, s);
        if (arm == ARM_EUCLID_MULADD) return launch_seed<ARM_EUCLID_MULADD>(a, nsamp, s);
        if (arm == ARM_COS_FOLD) return launch_seed<ARM_COS_FOLD>(a, nsamp, s);
        if (arm == ARM_COS_HOST) return launch_seed<ARM_COS_HOST>(a, nsamp, s);
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(fill_inf_bits_kernel, dim3((unsigned)((a.nq + 255) / 256)), dim3(256), 0, s, a.shared_r, a.nq);
    return hipGetLastError();
}

template <int ARM, bool VEC4>
hipError_t launch_merge(const GramArgs32& a, hipStream_t s) {
    const dim3 grid((unsigned)((a.nq + 3) / 4));
    if (a.k <= 64)
        hipLaunchKernelGGL((knn_merge_f32_kernel<ARM, VEC4>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((knn_merge_blocks_f32_kernel<ARM, VEC4>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_gram_f32_merge(const GramArgs32& a, int arm, hipStream_t s) {
    if (a.k == 1) {
        hipLaunchKernelGGL(knn_merge1_f32_kernel, dim3((unsigned)((a.nq + 255) / 256)), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    const bool vec4 = (a.d % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0);
    if (arm == ARM_EUCLID_FMA)
        return vec4 ? launch_merge<ARM_EUCLID_FMA, true>(a, s) : launch_merge<ARM_EUCLID_FMA, false>(a, s);
    if (arm == ARM_EUCLID_MULADD)
        return vec4 ? launch_merge<ARM_EUCLID_MULADD, true>(a, s) : launch_merge<ARM_EUCLID_MULADD, false>(a, s);
    if (arm == ARM_COS_FOLD)
        return vec4 ? launch_merge<ARM_COS_FOLD, true>(a, s) : launch_merge<ARM_COS_FOLD, false>(a, s);
    if (arm == ARM_COS_HOST)
        return vec4 ? launch_merge<ARM_COS_HOST, true>(a, s) : launch_merge<ARM_COS_HOST, false>(a, s);
    return hipErrorInvalidValue;
}

hipError_t launch_gram_f32(const GramArgs32& a, int arm, hipStream_t s) {
    const int64_t nblocks = (a.nq + a.qpb - 1) / a.qpb;
    const bool vec4 = (a.d % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0);
    hipError_t e;
    if (arm == ARM_EUCLID_FMA)
        e = vec4 ? launch_arm<ARM_EUCLID_FMA, false, true>(a, nblocks, s)
                 : launch_arm<ARM_EUCLID_FMA, false, false>(a, nblocks, s);
    else if (arm == ARM_EUCLID_MULADD)
        e = vec4 ? launch_arm<ARM_EUCLID_MULADD, false, true>(a, nblocks, s)
                 : launch_arm<ARM_EUCLID_MULADD, false, false>(a, nblocks, s);
    else if (arm == ARM_COS_FOLD)
        e = vec4 ? launch_arm<ARM_COS_FOLD, true, true>(a, nblocks, s)
                 : launch_arm<ARM_COS_FOLD, true, false>(a, nblocks, s);
    else if (arm == ARM_COS_HOST)  // the knn_host arm serves cosine above d = 128 only: wide shapes
        e = vec4 ? launch_wide<ARM_COS_HOST, true, true>(a, nblocks, s)
                 : launch_wide<ARM_COS_HOST, true, false>(a, nblocks, s);
    else
        return hipErrorInvalidValue;
    return e;
}

}  // namespace mlrs
