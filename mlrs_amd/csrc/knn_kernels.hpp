// Launch-side declarations shared by the kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlrs {

enum EmitMode : int {
    EMIT_SQRT = 0,      // Euclidean kNN: boundary sqrt of the k kept squared values
    EMIT_IDENTITY = 1,  // cosine kNN: values as kept
    EMIT_KMEANS = 2,    // k-means assignment: squared value + argmin centre-0 rule
    // X-vs-X graph (the host scans' KNearest): the values are the roots
    // (sqrt for the Euclidean arms, pow(v, 1/p) for Minkowski) and the lists
    // are ranked by (root, index), so two aggregates that root to the same
    // value are ordered by index
    EMIT_ROOT_RANKED = 3,
};

// Device-resident summary of the index rows' squared norms, written by the
// norm kernel and read by the Gram kernels' screen bound (no host sync).
struct NormStats {
    unsigned long long xsq_max_bits;  // max finite-or-inf squared norm (NaN rows ignored), as bits
    float xsq_max;                    // f32 view filled by the finalize kernel
    double xsq_max64;                 // f64 view
};

// Work split of the Gram kernels.  The (query block b, index tile t) units
// are ordered panel-major: the index is cut into S panels of P tiles (the
// last one L tiles), and the units run panel by panel, query block by query
// block, tile by tile.  Workgroup w takes units [w*P, (w+1)*P): in every
// panel but the last that is exactly one (panel, query block) job, so the
// workgroups of one panel start on the same tile and stream the same index
// rows together (one L2 fill serves all of them on an XCD).  In the last
// panel a range may hold pieces of several jobs and a job may be split in
// two.  Each piece keeps its own exact lists in list slot slot(w, j, b);
// a query block has slots_of(b) <= S + 1 of them.  With many query blocks
// S = 1 and this is a plain balanced split over query blocks.
struct StreamSplit {
    int64_t nqb, ntiles, T, P, S, L, G;
    __host__ __device__ StreamSplit(int64_t nq, int64_t nt, int64_t qpb, int64_t bn, int64_t g0) {
        nqb = (nq + qpb - 1) / qpb;
        ntiles = (nt + bn - 1) / bn;
        T = nqb * ntiles;
        if (g0 < 1) g0 = 1;
        P = (T + g0 - 1) / g0;
        S = (ntiles + P - 1) / P;
        L = ntiles - (S - 1) * P;
        G = (T + P - 1) / P;
    }
    // unit u -> panel j, query block b, tile t, units left in its job from u
    __host__ __device__ void decode(int64_t u, int64_t& j, int64_t& b, int64_t& t, int64_t& left) const {
        const int64_t full = (S - 1) * nqb * P;
        if (u < full) {
            j = u / (nqb * P);
            const int64_t r = u - j * nqb * P;
            b = r / P;
            const int64_t o = r - b * P;
            t = j * P + o;
            left = P - o;
        } else {
            j = S - 1;
            const int64_t r = u - full;
            b = r / L;
            const int64_t o = r - b * L;
            t = j * P + o;
            left = L - o;
        }
    }
    __host__ __device__ int64_t slot(int64_t w, int64_t j, int64_t b) const {
        if (j < S - 1) return j;
        const int64_t u0 = (S - 1) * nqb * P + b * L;
        return (S - 1) + (w - u0 / P);
    }
    __host__ __device__ int64_t slots_of(int64_t b) const {
        const int64_t u0 = (S - 1) * nqb * P + b * L;
        const int64_t u1 = u0 + L;
        return (S - 1) + ((u1 - 1) / P - u0 / P + 1);
    }
    __host__ __device__ int64_t nslots() const { return S + 1; }
};

// XCD-aware workgroup numbering.  Consecutive workgroup ids are handed to
// the eight XCDs in turn, and each XCD has its own L2.  Renumbering so that
// the workgroups resident on one XCD take one contiguous range of the
// StreamSplit order puts the workgroups that stream one index panel on the
// same XCD, where one L2 fill serves all of them.  A bijection of [0, G).
__device__ __forceinline__ int64_t xcd_grouped_wg(int64_t b, int64_t G) {
    constexpr int64_t kXcds = 8;
    const int64_t x = b % kXcds, i = b / kXcds, per = G / kXcds, rem = G % kXcds;
    return x * per + (x < rem ? x : rem) + i;
}

struct GramArgs32 {
    const float* q;
    int64_t nq;
    const float* x;
    int64_t nt;
    int64_t d;
    int k;
    int mode;          // EmitMode
    const float* qsq;  // query row_sumsq
    const float* xsq;  // index row_sumsq
    const float* xscale;  // cosine: -1/||x_t|| (0 for zero rows)
    const float* qinv;    // knn_host cosine: query reciprocal norms (0 for zero rows)
    const float* xinv;    // knn_host cosine: index reciprocal norms
    const NormStats* stats;
    double eps_rel;    // Euclidean screen bound: eps = eps_rel*(||q||^2 + max||x||^2) + eps_abs
    double eps_abs;    // cosine screen bound (absolute)
    int64_t grid_wgs;  // the G0 the StreamSplit is built from (<= one resident round)
    int nslots;        // list slots per query (StreamSplit::nslots)
    int qpb;           // queries per workgroup: gram_f32_queries_per_block(d)
    float* part_val;   // [nslots][nq][gram_list_cap(k)] lists, one per (segment, query)
    uint32_t* part_idx;
    float* qval;       // [grid_wgs][4 waves][2][2048]: screen values, then index rows, of the queued pairs (k > 1)
    float4* summ;      // [nslots][nq]: per-(segment, query) list summaries (k > 1), or null
    float* out_val;    // [nq][k]
    uint32_t* out_idx;
    unsigned int* shared_r;  // [nq] best known exact k-th value per query (float bits), or null
};

// Entries of one (segment, query) list of the Gram kernels: the k best plus
// room for the pairs whose screen values lie within the error window of the
// k-th (k = 1 keeps the single best pair, exactly): one 64-entry block for
// k <= 64, k + 32 (at most 160, three blocks) above.
__host__ __device__ inline int gram_list_cap(int k) {
    return k == 1 ? 1 : k <= 64 ? (k + 32 < 64 ? k + 32 : 64) : k + 32;
}

// Queued (screen value, index row) pairs of the f32 Gram kernel, 2 words
// each, per workgroup of 4 waves: narrow shape 32 queries x 64 (k <= 64) or
// 128 (k > 64) entries; the wide shape's 16 x 128 fits either.
inline size_t gram_f32_qval_elems(int64_t grid_wgs, int k) {
    return (size_t)grid_wgs * 4 * 32 * (k > 64 ? 128 : 64) * 2;
}
// The f64 kernel's queued screen values: 4 waves x 16 queries x 48 entries.
inline size_t gram_f64_qval_elems(int64_t grid_wgs) { return (size_t)grid_wgs * 4 * 16 * 48; }

// Index rows the seed launch samples for k > 1 (evenly spaced): 64 k, at
// most 2048 and at most nt / 512 (the seed's exact vector work stays near
// 0.2% of the scan's), but at least 512, so the k-th of the sample sits near
// the same quantile for every k (at k = 128, 512 rows left the bound near the
// 25% quantile).  Measured: c2 (1M rows, k = 32) steps fastest with the
// 1953-row cap (1024 rows: +0.1 ms; 4096: the kernel gains 0.1 ms more but
// the seed launch costs more), k = 128 likewise (4096 and 8192 rows cut the
// scan by 0.6 and 1.1 ms and cost more in the seed), d256 (200k rows) with
// 512; never more than the index.
inline int64_t gram_seed_rows(int64_t nt, int k) {
    int64_t n = 64 * (int64_t)k;
    if (n > 2048) n = 2048;
    if (n > nt / 512) n = nt / 512;
    if (n < 512) n = 512;
    return nt < n ? nt : n;
}

// G0, launched workgroups and per-query list slots of the Gram kernel's split.
// vec4: the launch's 16-byte row test (d % 4 == 0, both bases 16-byte aligned),
// which picks the kernel and with it the workgroups per CU the split assumes.
void gram_f32_split(int64_t nq, int64_t nt, int64_t d, int k, int cus, bool vec4, int64_t* grid_wgs, int* nslots);

// Three launches per search: prep (the shared per-query bound: seeded from a
// row sample for k > 1, else reset), the Gram kernel, the strip merge +
// output transform.
// seed_buf: gram_f32_seed_screen_bytes(...) bytes of workspace when that is
// nonzero (the seed then runs on the matrix cores), else null.
hipError_t launch_gram_f32_prep(const GramArgs32& a, int arm, hipStream_t s, void* seed_buf);
size_t gram_f32_seed_screen_bytes(int64_t nq, int64_t nt, int64_t d, int k, int arm, bool vec4);
hipError_t launch_gram_f32(const GramArgs32& a, int arm, hipStream_t s);
// k = 1 Euclidean searches whose index fits a few workgroups' LDS
// (knn_k1_resident.hip): the chunk count the launch uses (each chunk one
// (chunk, query) list slot), or 0 where it does not serve the shape.
int gram_f32_k1_resident_chunks(int64_t nq, int64_t nt, int64_t d, int k, int arm, bool vec4);
// The resident search (part_val / part_idx: one slot per chunk), then the
// merge of the chunks' lists with the output transform.
// a.qval must hold gram_f32_k1_resident_queue_bytes(cus) (the waves' queues).
// qsq_out non-null: the kernel forms the queries' squared norms itself and
// writes them there (a.qsq must then point at the same array, for the merge).
hipError_t launch_gram_f32_k1_resident(const GramArgs32& a, int arm, int cus, float* qsq_out, hipStream_t s);
size_t gram_f32_k1_resident_queue_bytes(int cus);
hipError_t launch_gram_f32_k1_resident_merge(const GramArgs32& a, int nchunks, hipStream_t s);
hipError_t launch_gram_f32_merge(const GramArgs32& a, int arm, hipStream_t s);
int gram_f32_max_k();
int gram_f32_max_d();
// 128 queries per workgroup for d <= 128 (32 per wave), 64 above (16 per wave)
int gram_f32_queries_per_block(int64_t d);
int gram_f32_rows_per_tile();

struct GramArgs64 {
    const double* q;
    int64_t nq;
    const double* x;
    int64_t nt;
    int64_t d;
    int k;
    int mode;             // EmitMode
    const double* qsq;    // query row_sumsq
    const double* xsq;    // index row_sumsq
    const double* qinv;   // knn_host cosine: query reciprocal norms
    const double* xinv;   // knn_host cosine: index reciprocal norms
    const double* xscale; // cosine: -1/||x_t|| (0 for zero rows)
    const NormStats* stats;
    double eps_rel;       // Euclidean screen bound: eps = eps_rel*(||q||^2 + max||x||^2) + eps_abs
    double eps_abs;       // cosine screen bound (absolute)
    int64_t grid_wgs;
    int nslots;
    double* part_val;     // [nslots][nq][gram_list_cap(k)]
    uint32_t* part_idx;
    double* qval;         // [grid_wgs][4 waves][16 queries][48]: screen values of the queued pairs
    double* out_val;      // [nq][k]
    uint32_t* out_idx;
    unsigned long long* shared_r;  // [nq] best known exact k-th value per query (double bits)
    // EMIT_ROOT_RANKED only, else null: [nq], set to 1 where an exact list
    // dropped a pair whose root may equal the k-th root (the merge cannot
    // then rank that root's ties by index; launch_gram_f64_root_fill does)
    unsigned int* root_flag;
};

void gram_f64_split(int64_t nq, int64_t nt, int cus, int64_t* grid_wgs, int* nslots);
// prep: the shared per-query bound, seeded with the k-th exact value over a
// row sample (arm: the exact arithmetic)
// seed_buf: gram_f64_seed_screen_bytes(...) bytes when that is nonzero (the
// seed then runs on the matrix cores), else null.
hipError_t launch_gram_f64_prep(const GramArgs64& a, int arm, hipStream_t s, void* seed_buf);
size_t gram_f64_seed_screen_bytes(int64_t nq, int64_t nt, int64_t d, int k, bool vec2);
hipError_t launch_gram_f64(const GramArgs64& a, int arm, hipStream_t s);
hipError_t launch_gram_f64_merge(const GramArgs64& a, int arm, hipStream_t s);
// EMIT_ROOT_RANKED (Euclidean arms): the queries root_flag marks get the
// rows whose root equals their k-th root in ascending index order
hipError_t launch_gram_f64_root_fill(const GramArgs64& a, int arm, hipStream_t s);
int gram_f64_max_k();
int gram_f64_max_d();

// Row norms: sq[r] = row_sumsq (separate multiply/add, ascending column),
// optional inv[r] = (sq > 0) ? 1/sqrt(sq) : 0 and optional neg-inverse scale.
template <typename T>
hipError_t launch_row_norms(const T* x, int64_t n, int64_t d, T* sq, T* inv, T* neg_inv,
                            NormStats* stats, hipStream_t s);

// Generic exact path: tiled exact pairwise values under one arm.
template <typename T>
// `root`: 0 none, 1 sqrt, 2 pow(v, root_exp); pexp / pint: the Minkowski
// exponent of the pow / integer arms.
hipError_t launch_pairwise_tile(const T* x, int64_t nx, const T* y, int64_t ny, int64_t d, int arm,
                                const T* xa, const T* ya, T* out, int64_t ldo, int root,
                                hipStream_t s, T pexp = T(0), int pint = 0, T root_exp = T(0));
template <typename T>
hipError_t launch_pow_inplace(T* v, int64_t n, T e, hipStream_t s);
// dst[0..n) = src[0..n) (the fit-time ownership copy).
template <typename T>
hipError_t launch_device_copy(const T* src, T* dst, int64_t n, hipStream_t s);

// Generic exact path: per-row (value, index) top-k over a materialized
// rows x cols matrix, NaN never admitted, sentinel-padded; any k >= 1.  For k
// above 256 the pairs are collected into the output rows and sorted there,
// with select_rows_scratch_bytes(rows, k, sizeof(T)) bytes of `scratch`
// (256-byte aligned; unused, and may be null, for k <= 256).
template <typename T>
hipError_t launch_select_rows(const T* dist, int64_t rows, int64_t cols, int64_t ld, int k,
                              int mode, T* out_val, uint32_t* out_idx, void* scratch, hipStream_t s);
size_t select_rows_scratch_bytes(int64_t rows, int k, int elem_bytes);

// argmin_dist_rows semantics over a materialized block (generic k-means path).
template <typename T>
hipError_t launch_argmin_rows(const T* dist, int64_t rows, int64_t cols, int64_t ld, uint32_t* labels,
                              T* best, hipStream_t s);

// Low-dimension ALU path (exact, lane per query), f32 and f64.  The shared
// per-query bound holds the k-th value's bits (non-negative values order as
// their bits): 32-bit words for f32, 64-bit for f64.
template <typename T>
struct LowdBits;
template <>
struct LowdBits<float> {
    typedef unsigned int type;
};
template <>
struct LowdBits<double> {
    typedef unsigned long long type;
};
template <typename T>
struct LowdArgs {
    const T* q;
    int64_t nq;
    const T* x;
    int64_t nt;
    int64_t d;
    int k;
    int mode;
    const T* qsq;           // query row_sumsq
    const T* xsq;           // index row_sumsq
    const T* xscale;        // cosine: -1/||x|| (0 for zero rows); null for Euclidean
    const NormStats* stats; // max index row_sumsq (screen bound)
    double eps_rel;         // screen bound eps = eps_rel*(||q||^2 + max||x||^2) + eps_abs
    double eps_abs;
    int64_t rows_per_strip;
    int nstrips;
    typename LowdBits<T>::type* shared_r;  // [nq] k-th value reached by finished strips (bits), or null
    T* part_val;
    uint32_t* part_idx;
    T* out_val;
    uint32_t* out_idx;
};
typedef LowdArgs<float> LowdArgs32;
typedef LowdArgs<double> LowdArgs64;
// Queries per lane of the low-d kernel for a list capacity K and row width D
// (f64 lanes hold twice the registers per value: two queries only up to
// D = 8).
#ifndef MLRS_LOWD_QL_SMALL_K
#define MLRS_LOWD_QL_SMALL_K 2
#endif
template <typename T>
constexpr int lowd_queries_per_lane(int K, int D) {
    return sizeof(T) == 8 ? ((K <= 16 && D <= 8) ? 2 : 1) : (K <= 8 ? MLRS_LOWD_QL_SMALL_K : (K <= 16 ? 2 : 1));
}
int lowd_queries_per_block(int k, int64_t d, int elem_bytes);
hipError_t launch_lowd_f32(const LowdArgs32& a, int arm, hipStream_t s);
hipError_t launch_lowd_f64(const LowdArgs64& a, int arm, hipStream_t s);
int lowd_max_d();
int lowd_max_k();

// kNN consumers (knn_consumers.hip).
hipError_t launch_first_bad_reset(unsigned long long* first_bad, hipStream_t s);
template <typename T>
hipError_t launch_knn_regress(const T* y, int64_t n_train, int64_t n_out, const uint32_t* idx, const T* dist,
                              int64_t nq, int64_t k, int weighted, T* out, unsigned long long* first_bad,
                              hipStream_t s);
template <typename T>
hipError_t launch_knn_classify(const int32_t* y_class, int64_t n_train, int64_t n_classes, const uint32_t* idx,
                               const T* dist, int64_t q0, int64_t rows, int64_t nq, int64_t k, int weighted,
                               T* proba, int32_t* labels, double* acc, int64_t* err, unsigned long long* first_bad,
                               hipStream_t s);

// radius_neighbors (knn_radius.hip).  A query group of radius_queries_per_wave
// rows is scanned against one strip of index rows per wave, 64 rows at a time
// (lane = index row), in the arithmetic of the reference's host arm; the
// matches of a group row within a 64-row chunk are placed by a wave ballot,
// so each row's matches come out in ascending index order.  Two passes share
// the kernel: COUNT writes each (strip, row) match count; FILL recomputes and
// writes the matches' pre-boundary values at the offsets the count pass
// fixed; launch_radius_transform then applies the boundary transform.
template <typename T>
struct RadiusArgs {
    const T* qT;       // [G][d][RQ] query groups, transposed (zero rows past nq)
    const T* x;        // [nt][d] index rows
    const T* qinv;     // cosine: [G*RQ] query reciprocal norms
    const T* xinv;     // cosine: [nt] index reciprocal norms
    int64_t nq, nt, d;
    int64_t strip_len; // index rows per strip (a multiple of 64)
    int nstrips;
    T th;              // threshold on the pre-boundary value
    T pexp;            // Minkowski exponent of the pow arm
    int pint;          // Minkowski integer exponent (3..8) of the multiply arm
    uint32_t* cnt;     // [nstrips][nq]: COUNT writes counts; FILL reads the in-row exclusive prefix
    const uint32_t* row_cnt;           // [nq] per-row totals (FILL: end check of the last strip)
    const unsigned long long* qoff;    // [nq] first output position of each row
    T* out_dist;
    int32_t* out_idx;
    int64_t capacity;                  // FILL: entries the outputs hold; no write at or past it
    unsigned int* mismatch;            // FILL: set when a strip's matches differ from its count
    // the matrix-core screen (knn_radius_gram.hip)
    const T* q;                        // [nq][d] query rows
    const T* qsq;                      // [nq] query row_sumsq
    const T* xsq;                      // [nt] index row_sumsq
    const NormStats* stats;            // largest index squared norm
    double eps_rel, eps_abs;           // screen error bound (as the fused kNN screen's)
    // STAGE (matrix-core screen): [nstrips][nq][stage_cap] first matches of
    // each (strip, row), and a flag set when a (strip, row) has more
    T* stage_val;
    int32_t* stage_idx;
    int64_t stage_cap;
    unsigned int* stage_over;
};
enum RadiusMode : int { RADIUS_COUNT = 0, RADIUS_FILL = 1, RADIUS_STAGE = 2 };
// The matrix-core radius scan: f32, Euclidean and cosine, d <= 128.
bool radius_gram_serves(int arm, int64_t d);
int64_t radius_gram_rows_per_tile();
int64_t radius_gram_queries_per_block();
int64_t radius_gram_wgs_per_cu();
hipError_t launch_radius_gram(const RadiusArgs<float>& a, int arm, int mode, hipStream_t s);
// The staged matches of a STAGE pass copied into the outputs (after the offsets).
hipError_t launch_radius_unstage(const RadiusArgs<float>& a, hipStream_t s);
template <typename T>
int radius_queries_per_wave();
template <typename T>
hipError_t launch_radius_stage(const T* xq, int64_t nq, int64_t d, T* qT, hipStream_t s);
template <typename T>
hipError_t launch_radius_scan(const RadiusArgs<T>& a, int arm, bool fill, hipStream_t s);
// Row totals, the in-row exclusive strip prefix, the row offsets and the
// match total (one u64 on the device).
hipError_t launch_radius_offsets(uint32_t* cnt, int64_t nq, int nstrips, uint32_t* row_cnt,
                                 unsigned long long* block_sum, unsigned long long* qoff,
                                 unsigned long long* total, hipStream_t s);
// mode 1: v = sqrt(v); mode 2: v = pow(v, e); mode 0: nothing.
template <typename T>
hipError_t launch_radius_transform(T* v, int64_t n, int mode, T e, hipStream_t s);
hipError_t launch_fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t s);

// X-vs-X graphs (knn_graph.hip): operand preparation and list finishing
// around the f64 kNN search.
hipError_t launch_widen(const float* x, int64_t n, double* y, hipStream_t s);
hipError_t launch_normalize_rows(const double* x, int64_t n, int64_t d, const double* inv, double* y,
                                 hipStream_t s);
hipError_t launch_graph_finish(const double* val, const uint32_t* idx, int64_t n, int kk, int k, int drop_self,
                               int halve, double* out_dist, uint32_t* out_idx, hipStream_t s);
hipError_t launch_core_column(const double* val, int64_t n, int k, double* out, hipStream_t s);

// k-means fit loop (kmeans_loop.hip).  Centroid sums over the reference's row
// blocks: buckets of rows by (block, label), then per-(block, label, feature)
// sums over each bucket in ascending row order, then the block partials summed
// in block order.
template <typename T>
struct KmScratch {
    uint32_t* pcount;  // [nb][k] rows of label c in block b
    uint32_t* seg;     // [nb][k] first slot of bucket (b, c) in perm
    uint32_t* cursor;  // [nb][km_sub_blocks(nb, rpb, k)][k] sub-block counts, then scatter cursors
    uint32_t* counts;  // [k]
    uint32_t* starts;  // [k]
    uint32_t* perm;    // [n] row numbers, bucket by bucket
    T* psum;           // [nb][k][d]
    T* sums;           // [k][d]
};
// Sub-blocks per reference block in the centroid-sum scatter (sizes KmScratch::cursor).
int64_t km_sub_blocks(int64_t nb, int64_t rpb, int64_t k);
template <typename T>
hipError_t launch_km_centroid_sums(const T* x, const uint32_t* labels, int64_t n, int64_t d, int64_t k, int64_t nb,
                                   int64_t rpb, const KmScratch<T>& w, hipStream_t s);
hipError_t launch_km_changed(const uint32_t* a, const uint32_t* b, int64_t n, unsigned int* count, hipStream_t s);

// Peak probe (probe.hip): kind 0 FMA f32, 1 FMA f64, 2 MFMA f32, 3 MFMA f64;
// `blocks` workgroups of 256 threads, iters loop trips; out holds one value
// per thread (8 bytes).
hipError_t launch_probe(int kind, int64_t blocks, int iters, void* out, hipStream_t s);
double probe_flops(int kind, int64_t blocks, int iters);

// Bound-pruned assignment (the fit's algorithm = 'elkan'): see kmeans_loop.hip.
struct KmPruneConsts {
    double gamma;  // relative error bound of a computed squared distance
    double eta;    // its absolute error bound (underflowing terms)
    double K;      // (1 + gamma) / (1 - gamma) (1 + 2^-30)
    double umin;   // sqrt(2^30 eta): below it no centre is excluded
    int maxcand;   // centres a row evaluates itself before it goes to the fused search
};
template <typename T>
hipError_t launch_km_half_dist(const T* c, int64_t k, int64_t d, double* hcd, double* dnc, hipStream_t s);
template <typename T>
hipError_t launch_km_bound_init(const T* dist, int64_t n, double gamma, double eta, double* U, hipStream_t s);
template <typename T>
// perm: the rows in the label-major order of lab_old (the centroid sums'
// permutation), or null (rows in index order)
hipError_t launch_km_elkan(const T* x, int64_t n, int64_t d, const T* c, int64_t k, const uint32_t* perm,
                           const uint32_t* lab_old, uint32_t* lab_new, T* dist, double* U, const double* delta,
                           const double* dnc, const double* sv, const uint32_t* si, const KmPruneConsts& pc,
                           uint32_t* fb_list, unsigned int* fb_count, hipStream_t s);
template <typename T>
hipError_t launch_km_gather_list(const T* x, const T* xsq, const uint32_t* list, int64_t m, int64_t d, T* out,
                                 T* out_sq, hipStream_t s);
template <typename T>
hipError_t launch_km_scatter_list(const uint32_t* list, int64_t m, const uint32_t* lab_sub, const T* dist_sub,
                                  double gamma, double eta, uint32_t* lab_new, T* dist, double* U, hipStream_t s);
template <typename T>
hipError_t launch_km_count_nonfinite(const T* v, int64_t n, unsigned int* count, hipStream_t s);
// block_sum_f over v: parts[b] = the ordered sum of rows [b rpb, (b + 1) rpb).
template <typename T>
hipError_t launch_km_block_sum(const T* v, int64_t n, int64_t nb, int64_t rpb, T* parts, hipStream_t s);
// out = (T)((double)sums * (1.0 / (double)counts[c])), element by element.
template <typename T>
hipError_t launch_km_mean(const T* sums, const uint32_t* counts, int64_t k, int64_t d, T* out, hipStream_t s);
template <typename T>
hipError_t launch_km_inertia(const T* x, const T* c, const uint32_t* labels, int64_t n, int64_t d, T* rows,
                             int64_t nb, int64_t rpb, T* parts, hipStream_t s);
// means == nullptr: column sums; else column sums of (x - means)^2.
template <typename T>
hipError_t launch_km_col_sums(const T* x, int64_t n, int64_t d, int64_t nb, int64_t rpb, const T* means, T* out,
                              hipStream_t s);
template <typename T>
hipError_t launch_km_mind2(const T* x, int64_t n, int64_t d, int64_t cidx, int first, T* mind2, hipStream_t s);
template <typename T>
hipError_t launch_km_gather(const T* x, const int64_t* idx, int64_t k, int64_t d, T* out, hipStream_t s);
// neg[i] = -dist[i] (i < n), +inf up to `padded`; *nans = the number of NaN
// distances (relocation ranking).
template <typename T>
hipError_t launch_km_neg(const T* dist, int64_t n, int64_t padded, T* neg, unsigned int* nans, hipStream_t s);
// rows[r m + j] = r C + idx[r m + j]: chunk-local picks to row numbers.
hipError_t launch_km_chunk_rows(const uint32_t* idx, int64_t nchunks, int64_t m, int64_t C, uint32_t* rows,
                                hipStream_t s);
// out[i] = src[idx[i]], i < m (0 for an index past the n_src entries).
hipError_t launch_km_take_u32(const uint32_t* src, int64_t n_src, const uint32_t* idx, int64_t m, uint32_t* out,
                              hipStream_t s);

}  // namespace mlrs
