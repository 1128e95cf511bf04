// k = 1 Euclidean search with the index resident in LDS (gfx950).
//
// Serves what the fused f32 Gram kernel serves for k = 1 (the k-means
// assignment argmin_dist_rows, crates/mlrs-kernels/src/kmeans.rs:284-310, and
// the k = 1 nearest neighbour of metric_topk, crates/mlrs-algos/src/neighbors/
// nearest.rs:1058-1343) when the index is small: its rows are cut into
// chunks that fit one workgroup's LDS, and each workgroup loads one chunk
// once and keeps it for the whole launch.
//  * One workgroup of 12 waves per CU (three per SIMD).  Every wave works on
//    its own blocks of 32 queries against the resident chunk: the query block
//    is the MFMA B operand in VGPRs (pre-scaled by -2), the chunk's 32-row
//    tiles the A operand read from LDS, as in the fused kernel's narrow shape
//    (v_mfma_f32_32x32x2f32; the accumulator starts at ||x_t||^2).  Nothing
//    is written to LDS in the loop, so the waves never wait for each other:
//    no tile barrier, no tile loads.
//  * Per tile, the k = 1 steps of the fused kernel: the threshold tightened
//    with the tile's smallest expansion value + 2 eps, the screen (the sign
//    of threshold - value where the wave's screen sums cannot overflow, the
//    compare elsewhere), passing rows queued per query (16-bit chunk rows, in
//    global memory: admissions are rare at k = 1, and the LDS goes to the
//    chunk), a queue whose rows all screen above the tightened threshold
//    emptied before the tile's rows join it.
//  * The queued rows are evaluated exactly, in the reference arm's operation
//    order, with the query row from global memory and the index row from the
//    resident chunk; the best (value, index) per query is kept with a 64-bit
//    LDS atomicMin, and written as the (chunk, query) list.
//  * knn_merge1_chunks_f32_kernel takes each query's best over the chunks
//    (value, then index) and applies the output transform.
// The results are the fused kernel's, bit for bit: the same screen, error
// bound and exact rescoring.
#include "knn_common.hpp"
#include "knn_kernels.hpp"

namespace mlrs {

namespace {

constexpr int kResWaves = 16;             // waves per workgroup (one workgroup per CU)
constexpr int kResThreads = 64 * kResWaves;
constexpr int kResQpw = 32;               // queries per wave block
constexpr int kResBn = 32;                // rows per tile
constexpr int kResQcap = 48;              // queued rows per query (flushed above 16)
constexpr int kResLdsBytes = 163840;      // gfx950's LDS per workgroup

struct ResWave {
    float thr[kResQpw];
    float qs[kResQpw];
    float eps[kResQpw];
    uint32_t off[kResQpw];
    uint32_t mode[kResQpw];             // 0: screen values within eps of exact values (finite sums)
    unsigned long long best[kResQpw];   // (value bits << 32 | global row) of the kept pair
};

constexpr unsigned long long kResEmpty = (0x7F800000ull << 32) | 0xFFFFFFFFull;

// Rows of a chunk at a padded feature count DP: what LDS holds after the
// wave state, in whole tiles.
__host__ __device__ constexpr int res_rows_max(int dp) {
    return ((kResLdsBytes - kResWaves * (int)sizeof(ResWave) - 256) / ((dp + 4) * 4 + 4)) / kResBn * kResBn;
}

template <int NG, int ARM>
__global__ __launch_bounds__(kResThreads) void knn_k1_resident_f32_kernel(GramArgs32 a, int chunk_rows,
                                                                          int nchunks,
                                                                          uint16_t* __restrict__ queues,
                                                                          float* __restrict__ qsq_out) {
    constexpr int DP = NG * 8;
    constexpr int STRIDE = DP + 4;  // an odd number of 16-byte chunks: 16 consecutive rows on distinct bank groups
    constexpr int RMAX = res_rows_max(DP);
    constexpr int kFlushAt = kResQcap - kResBn;
    __shared__ __attribute__((aligned(16))) float chunk[RMAX * STRIDE];
    __shared__ __attribute__((aligned(16))) float cnorm[RMAX];
    __shared__ ResWave wl[kResWaves];

    const float* __restrict__ Q = a.q;
    const float* __restrict__ X = a.x;
    const float* __restrict__ QSQ = a.qsq;
    const float* __restrict__ XSQ = a.xsq;
    const int64_t nq = a.nq, nt = a.nt, d = a.d;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int jl = lane & 31;
    const float inf = __builtin_huge_valf();
    ResWave& L = wl[w];
    // this wave's queues in global memory, [query][position]: chunk rows
    uint16_t* __restrict__ QI = queues + ((int64_t)blockIdx.x * kResWaves + w) * (kResQpw * kResQcap);

    // ---- the chunk: rows [row0, row0 + rows), zero columns past d, padded
    //      to whole tiles with zero rows of norm +inf ----
    const int cidx = (int)(blockIdx.x % (unsigned)nchunks);
    const int64_t grp = blockIdx.x / (unsigned)nchunks;
    const int64_t ngrp = gridDim.x / (unsigned)nchunks;
    const int64_t row0 = (int64_t)cidx * chunk_rows;
    const int rows = (int)((nt - row0) < chunk_rows ? (nt - row0) : chunk_rows);
    const int tiles = (rows + kResBn - 1) / kResBn;
    for (int e = tid; e < tiles * kResBn * (DP / 4); e += kResThreads) {
        const int r = e / (DP / 4), c4 = e % (DP / 4);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < rows && 4 * c4 < d) v = *reinterpret_cast<const float4*>(X + (row0 + r) * d + 4 * c4);
        *reinterpret_cast<float4*>(&chunk[r * STRIDE + 4 * c4]) = v;
    }
    for (int r = tid; r < tiles * kResBn; r += kResThreads) cnorm[r] = r < rows ? XSQ[row0 + r] : inf;
    __syncthreads();  // the chunk is read-only from here on

    float* __restrict__ LV = a.part_val + (int64_t)cidx * nq;
    uint32_t* __restrict__ LI = a.part_idx + (int64_t)cidx * nq;
    const int64_t nqb = (nq + kResQpw - 1) / kResQpw;
    for (int64_t qb = grp * kResWaves + w; qb < nqb; qb += ngrp * kResWaves) {
        const int64_t qwave = qb * kResQpw;
        const int64_t qmine = qwave + jl;
        const bool qvalid = qmine < nq;
        const int64_t qrow = qvalid ? qmine : nq - 1;

        // ---- per-query state (lanes 0..31 of the wave) ----
        float4 qreg[NG];
        {
            const float* qp = Q + qrow * d;
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                const int64_t c = (int64_t)8 * g + 4 * h;
                const float4 v = *reinterpret_cast<const float4*>(qp + (c < d ? c : d - 4));
                qreg[g] = (qvalid && c < d) ? make_float4(-2.0f * v.x, -2.0f * v.y, -2.0f * v.z, -2.0f * v.w)
                                            : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        float qsq_l;
        if (qsq_out) {
            // ||q||^2 from the operand: qreg = -2 q exactly, so the sum of its
            // squares is 4 ||q||^2 in some order (within the screen bound's
            // allowance for the norm's rounding, as a sum in any order is);
            // chunk 0 keeps it for the merge's k-means rule
            float s2 = 0.0f;
#pragma unroll
            for (int g = 0; g < NG; ++g)
                s2 = s2 + qreg[g].x * qreg[g].x + qreg[g].y * qreg[g].y + qreg[g].z * qreg[g].z +
                     qreg[g].w * qreg[g].w;
            qsq_l = (s2 + shfl_xor_f(s2, 32)) * 0.25f;
            if (cidx == 0 && h == 0 && qvalid) qsq_out[qmine] = qsq_l;
        } else {
            qsq_l = QSQ[qrow];
        }
        if (lane < kResQpw) {
            const float qsq = qvalid ? qsq_l : 0.0f;
            L.thr[lane] = qvalid ? inf : -inf;
            L.qs[lane] = qsq;
            L.eps[lane] = (float)(a.eps_rel * ((double)qsq + (double)a.stats->xsq_max) + a.eps_abs);
            const bool sv = qvalid && ((double)qsq + (double)a.stats->xsq_max <= 0x1p124) && (L.eps[lane] < inf);
            L.mode[lane] = sv ? 0u : 1u;
            L.best[lane] = kResEmpty;
        }
        // (LDS operations of one wave complete in order: the lanes' stores
        // above are seen by the reads below)
        float thr = L.thr[jl];
        const float eps2 = 2.0f * L.eps[jl];
        const bool nan_free = __builtin_amdgcn_ballot_w64(lane < kResQpw && qvalid && L.mode[lane] != 0u) == 0;
        // a lower bound on the screen values of the query's queued rows (the
        // fused kernel's qlo; -inf where a NaN screen value could hide a
        // finite exact one)
        const float qlo0 = (L.mode[jl] == 0u) ? inf : -inf;
        float qlo = qlo0;
        uint32_t cntr = 0u;

        // every queued (query, row) pair evaluated exactly in lane-parallel
        // batches, the best kept with a 64-bit LDS atomicMin
        auto flush = [&]() {
            const uint32_t c_ = (lane < kResQpw) ? cntr : 0u;
            uint32_t incl = c_;
#pragma unroll
            for (int m_ = 1; m_ < kResQpw; m_ <<= 1) {
                const uint32_t o_ = (uint32_t)__shfl_up((int)incl, m_, 64);
                if ((lane & (kResQpw - 1)) >= m_) incl += o_;
            }
            const uint32_t total = (uint32_t)__shfl((int)incl, kResQpw - 1, 64);
            if (lane < kResQpw) L.off[lane] = incl - c_;
            // the queued rows were stored by other lanes of this wave
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            for (uint32_t base = 0; base < total; base += 64) {
                const uint32_t e_ = base + (uint32_t)lane;
                if (e_ < total) {
                    int j_ = 0;
#pragma unroll
                    for (int m_ = kResQpw / 2; m_ >= 1; m_ >>= 1)
                        if (L.off[j_ + m_] <= e_) j_ += m_;
                    const uint32_t t_ = QI[j_ * kResQcap + (e_ - L.off[j_])];
                    const float* qp = Q + (qwave + j_) * d;
                    const float* yp = &chunk[(int)t_ * STRIDE];
                    float acc = 0.0f;
                    for (int c4 = 0; c4 < (int)(d >> 2); ++c4) {
                        const float4 qv = *reinterpret_cast<const float4*>(qp + 4 * c4);
                        const float4 yv = *reinterpret_cast<const float4*>(yp + 4 * c4);
                        const float d0 = qv.x - yv.x, d1 = qv.y - yv.y, d2 = qv.z - yv.z, d3 = qv.w - yv.w;
                        if (ARM == ARM_EUCLID_FMA) {
                            acc = __builtin_fmaf(d0, d0, acc);
                            acc = __builtin_fmaf(d1, d1, acc);
                            acc = __builtin_fmaf(d2, d2, acc);
                            acc = __builtin_fmaf(d3, d3, acc);
                        } else {
                            acc = acc + d0 * d0;
                            acc = acc + d1 * d1;
                            acc = acc + d2 * d2;
                            acc = acc + d3 * d3;
                        }
                    }
                    if (acc == acc)
                        atomicMin(&L.best[j_], ((unsigned long long)__float_as_uint(acc) << 32) |
                                                   (uint32_t)(row0 + (int64_t)t_));
                }
            }
            cntr = 0u;
            qlo = qlo0;
            if (lane < kResQpw) {
                const float R_ = __uint_as_float((uint32_t)(L.best[lane] >> 32));
                if (R_ < inf) {
                    // exact <= R  =>  ||x||^2 - 2 x.q <= R - ||q||^2 + eps
                    L.thr[lane] = fminf(L.thr[lane], round_up_f((double)R_ - (double)L.qs[lane] + (double)L.eps[lane]));
                }
            }
        };

        for (int t = 0; t < tiles; ++t) {
            // A operands from the resident chunk: lane (h, jl) reads row jl's
            // chunk 2g + h; the next group's read issued before this group's
            // four MFMAs
            f32x16_t acc;
            {
                const float* nrm = &cnorm[t * kResBn];
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const float4 n4 = *reinterpret_cast<const float4*>(nrm + 8 * g4 + 4 * h);
                    acc[4 * g4 + 0] = n4.x;
                    acc[4 * g4 + 1] = n4.y;
                    acc[4 * g4 + 2] = n4.z;
                    acc[4 * g4 + 3] = n4.w;
                }
            }
            const float* arow = &chunk[(t * kResBn + jl) * STRIDE + 4 * h];
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

            // ---- tighten with this tile's smallest expansion value ----
            float m = inf;
#pragma unroll
            for (int r = 0; r < 16; ++r) m = fminf(m, acc[r]);  // NaN ignored; padding rows are +inf
            m = fminf(m, shfl_xor_f(m, 32));
            if (m < inf) {
                const float s_ = m + eps2;
                thr = fminf(thr, s_ + (__builtin_fabsf(s_) * 0x1p-23f + 0x1p-126f));
            }
            if (qlo > thr) {
                cntr = 0u;
                qlo = inf;
            }
            qlo = fminf(qlo, m);

            // ---- screen; value r of the lane is tile row 8 (r / 4) + 4 h + r % 4 ----
            uint32_t msk = 0;
            if (nan_free) {
                const float t_ = thr + 0.0f;
                uint32_t f = 0;
#pragma unroll
                for (int r = 15; r >= 0; --r) f = __builtin_amdgcn_alignbit(f, __float_as_uint(t_ - acc[r]), 31);
                msk = f ^ 0xFFFFu;
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) msk |= (uint32_t)!(acc[r] > thr) << r;
            }
            if (!qvalid) msk = 0;
            if ((t + 1) * kResBn > rows) {  // the padded tail of the chunk is never a candidate
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (t * kResBn + 8 * (r >> 2) + 4 * h + (r & 3) >= rows) msk &= ~(1u << r);
            }
            if (__builtin_amdgcn_ballot_w64(msk != 0)) {
                const uint32_t c = (uint32_t)__builtin_popcount(msk);
                const uint32_t co = shfl_xor_u(c, 32);
                uint32_t pos = cntr + (h ? co : 0u);
                const int tb = t * kResBn;
                while (msk) {
                    const int r = __builtin_ctz(msk);
                    msk &= msk - 1;
                    QI[jl * kResQcap + pos++] = (uint16_t)(tb + 8 * (r >> 2) + 4 * h + (r & 3));
                }
                cntr += c + co;
            }
            if (__builtin_amdgcn_ballot_w64(lane < kResQpw && cntr > (uint32_t)kFlushAt)) {
                if (lane < kResQpw) L.thr[lane] = fminf(L.thr[lane], thr);
                flush();
                thr = L.thr[jl];
            }
        }
        if (__builtin_amdgcn_ballot_w64(lane < kResQpw && cntr > 0u)) flush();
        if (lane < kResQpw && qvalid) {
            const unsigned long long b = L.best[lane];
            LV[qmine] = __uint_as_float((uint32_t)(b >> 32));
            LI[qmine] = (uint32_t)b;
        }
    }
}

// Each query's best (value, index) over the chunks, then the output transform.
__global__ __launch_bounds__(256) void knn_merge1_chunks_f32_kernel(GramArgs32 a, int nchunks) {
    const int64_t qg = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (qg >= a.nq) return;
    float lv = a.part_val[qg];
    uint32_t li = a.part_idx[qg];
    for (int s = 1; s < nchunks; ++s) {
        const float v = a.part_val[(int64_t)s * a.nq + qg];
        const uint32_t ix = a.part_idx[(int64_t)s * a.nq + qg];
        if (pair_less<float>(v, ix, lv, li)) {
            lv = v;
            li = ix;
        }
    }
    emit_pair(a.mode, a.q, a.x, a.qsq, a.xsq, a.d, 1, qg, 0, lv, li, a.out_val, a.out_idx);
}

template <int NG, int ARM>
hipError_t launch_res_ng(const GramArgs32& a, int cus, float* qsq_out, hipStream_t s) {
    const int rmax = res_rows_max(NG * 8);
    const int nchunks = (int)((a.nt + rmax - 1) / rmax);
    // balanced chunks in whole tiles
    int chunk_rows = (int)((a.nt + nchunks - 1) / nchunks);
    chunk_rows = (chunk_rows + kResBn - 1) / kResBn * kResBn;
    const int64_t nqb = (a.nq + kResQpw - 1) / kResQpw;
    int64_t ngrp = cus / nchunks;
    if (ngrp < 1) ngrp = 1;
    const int64_t need = (nqb + kResWaves - 1) / kResWaves;  // groups that still get a block per wave
    if (ngrp > need) ngrp = need;
    hipLaunchKernelGGL((knn_k1_resident_f32_kernel<NG, ARM>), dim3((unsigned)(ngrp * nchunks)), dim3(kResThreads), 0,
                       s, a, chunk_rows, nchunks, reinterpret_cast<uint16_t*>(a.qval), qsq_out);
    return hipGetLastError();
}

}  // namespace

size_t gram_f32_k1_resident_queue_bytes(int cus) {
    return (size_t)(cus > 0 ? cus : 1) * kResWaves * kResQpw * kResQcap * sizeof(uint16_t);
}

int gram_f32_k1_resident_chunks(int64_t nq, int64_t nt, int64_t d, int k, int arm, bool vec4) {
    if (k != 1 || !vec4 || d > 64 || nq < 1 || nt < 1) return 0;
    if (arm != ARM_EUCLID_FMA && arm != ARM_EUCLID_MULADD) return 0;
    const int ng = d <= 32 ? 4 : 8;
    const int rmax = res_rows_max(ng * 8);
    const int64_t nchunks = (nt + rmax - 1) / rmax;
    return nchunks <= 8 ? (int)nchunks : 0;
}

hipError_t launch_gram_f32_k1_resident_merge(const GramArgs32& a, int nchunks, hipStream_t s) {
    hipLaunchKernelGGL(knn_merge1_chunks_f32_kernel, dim3((unsigned)((a.nq + 255) / 256)), dim3(256), 0, s, a,
                       nchunks);
    return hipGetLastError();
}

hipError_t launch_gram_f32_k1_resident(const GramArgs32& a, int arm, int cus, float* qsq_out, hipStream_t s) {
    if (!gram_f32_k1_resident_chunks(a.nq, a.nt, a.d, a.k, arm, true)) return hipErrorInvalidValue;
    if (a.d <= 32)
        return arm == ARM_EUCLID_FMA ? launch_res_ng<4, ARM_EUCLID_FMA>(a, cus, qsq_out, s)
                                     : launch_res_ng<4, ARM_EUCLID_MULADD>(a, cus, qsq_out, s);
    return arm == ARM_EUCLID_FMA ? launch_res_ng<8, ARM_EUCLID_FMA>(a, cus, qsq_out, s)
                                 : launch_res_ng<8, ARM_EUCLID_MULADD>(a, cus, qsq_out, s);
}

}  // namespace mlrs
