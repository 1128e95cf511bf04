// C-ABI layer: validation (before any launch), arm selection, workspace and
// dispatch to the kernels.  See include/mlrs_hip_knn.h for the contract.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <unordered_map>
#include <mutex>
#include <type_traits>
#include <vector>

#include "../../include/mlrs_hip_knn.h"
#include "knn_common.hpp"
#include "knn_kernels.hpp"

using namespace mlrs;

// Scratch of the allocation-free entry point (mlrs_knn_topk_f32_noalloc): one
// copy per GPU, held until the process ends.  Host code never uses this name
// as an address -- it takes the device address hipGetSymbolAddress returns
// for the current device (g_scratch_dev) and passes that to the kernels.
static __device__ __align__(256) char scratch[MLRS_NOALLOC_SCRATCH_BYTES];

namespace {

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
thread_local mlrs_error_info g_err;

int32_t set_err(int32_t code, const char* operand, int64_t rows, int64_t cols, int64_t len, int hip,
                const char* fmt, ...) {
    std::memset(&g_err, 0, sizeof(g_err));
    g_err.code = code;
    std::snprintf(g_err.operand, sizeof(g_err.operand), "%s", operand ? operand : "");
    g_err.rows = rows;
    g_err.cols = cols;
    g_err.len = len;
    g_err.hip_error = hip;
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err.message, sizeof(g_err.message), fmt, ap);
    va_end(ap);
    return code;
}

// PrimError::ShapeMismatch's Display text (crates/mlrs-core/src/error.rs:66-70).
int32_t shape_err(const char* operand, int64_t rows, int64_t cols, int64_t len) {
    return set_err(MLRS_ERR_SHAPE_MISMATCH, operand, rows, cols, len, 0,
                   "primitive '%s' shape mismatch: rows(%lld) * cols(%lld) = %lld != len(%lld)", operand,
                   (long long)rows, (long long)cols, (long long)(rows * cols), (long long)len);
}

// PrimError::DimMismatch's Display text (crates/mlrs-core/src/error.rs:76).
int32_t dim_err(const char* dim, int64_t lhs, int64_t rhs) {
    return set_err(MLRS_ERR_DIM_MISMATCH, dim, lhs, rhs, 0, 0,
                   "primitive dimension mismatch (%s): lhs declares %lld, rhs declares %lld", dim,
                   (long long)lhs, (long long)rhs);
}

int32_t hip_err(hipError_t e, const char* where) {
    return set_err(MLRS_ERR_HIP, where, 0, 0, 0, (int)e, "HIP error in %s: %s", where, hipGetErrorString(e));
}

int32_t ok() {
    return MLRS_OK;
}

// rows * cols == len without overflow (checked_mul in the reference).
bool geom_ok(int64_t rows, int64_t cols, int64_t len) {
    if (rows < 0 || cols < 0 || len < 0) return false;
    if (cols != 0 && rows > INT64_MAX / cols) return false;
    return rows * cols == len;
}

constexpr int64_t kU32Max = 0xFFFFFFFFll;

// ---------------------------------------------------------------------------
// per-device cached workspace (the BufferPool role: reuse across calls)
// ---------------------------------------------------------------------------
std::mutex g_mu;
constexpr int kMaxDevices = 64;
struct Arena {
    char* base = nullptr;
    size_t cap = 0;
    int cus = 0;
    bool pooled = false;  // base came from hipMallocAsync
};
Arena g_arena[kMaxDevices];

struct Carver {
    char* p;
    size_t off = 0;
    explicit Carver(char* b) : p(b) {}
    template <typename T>
    T* take(size_t n) {
        off = (off + 255) & ~(size_t)255;
        T* r = reinterpret_cast<T*>(p + off);
        off += n * sizeof(T);
        return r;
    }
};

static size_t aligned_bytes(size_t n) { return (n + 255) & ~(size_t)255; }

// ---------------------------------------------------------------------------
// call ordering across streams
// ---------------------------------------------------------------------------
// Every call enqueues on its caller's stream and returns without waiting, and
// all calls on a device carve the same cached buffers.  So a call that runs
// on another stream than the previous call first makes its stream wait for
// the previous call's work (an event recorded at the end of every call that
// touched a cached buffer): calls on one device run in call order, as on the
// reference's single stream (crates/mlrs-backend/src/stream_cap.rs:69).
struct DevOrder {
    hipEvent_t ev = nullptr;
    bool have = false;
};
DevOrder g_order[kMaxDevices];

struct CallState {
    hipStream_t s = nullptr;
    int dev = -1;
    bool armed = false;
};
CallState* g_call = nullptr;  // the running entry-point call (under g_mu)

// The allocation-free variant runs with the static scratch in place of the
// arenas (set for the duration of such a call, under g_mu).
bool g_noalloc = false;
char* g_noalloc_base = nullptr;

// Holds the process-wide lock for one entry-point call; records the call's
// end on its stream when the call touched a cached buffer.
struct CallGuard {
    std::lock_guard<std::mutex> lk;
    CallState st;
    CallGuard() : lk(g_mu) { g_call = &st; }
    ~CallGuard() {
        if (st.armed) {
            DevOrder& O = g_order[st.dev];
            if (hipEventRecord(O.ev, st.s) == hipSuccess) O.have = true;
        }
        g_call = nullptr;
    }
    CallGuard(const CallGuard&) = delete;
    CallGuard& operator=(const CallGuard&) = delete;
};

// Before the running call first touches a cached buffer of `dev`.
int32_t order_after_last_call(int dev, hipStream_t s) {
    if (!g_call || g_call->armed || g_noalloc) return MLRS_OK;
    DevOrder& O = g_order[dev];
    hipError_t e;
    if (!O.ev) {
        e = hipEventCreateWithFlags(&O.ev, hipEventDisableTiming);
        if (e != hipSuccess) {
            O.ev = nullptr;
            return hip_err(e, "hipEventCreateWithFlags");
        }
    }
    // Waited for even when the stream handle equals the last call's: a
    // destroyed stream's handle can be handed out again while its work is
    // pending, and waiting on an event the stream itself recorded is free.
    if (O.have) {
        e = hipStreamWaitEvent(s, O.ev, 0);
        if (e != hipSuccess) return hip_err(e, "hipStreamWaitEvent");
    }
    g_call->armed = true;
    g_call->dev = dev;
    g_call->s = s;
    return MLRS_OK;
}

int32_t current_device(int* dev) {
    hipError_t e = hipGetDevice(dev);
    if (e != hipSuccess) return hip_err(e, "hipGetDevice");
    if (*dev < 0 || *dev >= kMaxDevices)
        return set_err(MLRS_ERR_UNSUPPORTED, "device", *dev, 0, 0, 0, "device ordinal %d out of range", *dev);
    return MLRS_OK;
}

// PoolStats (crates/mlrs-backend/src/pool.rs:27-56) over the library's cached
// device buffers (main and auxiliary workspaces, radius plan memory), per
// device: an allocation is a buffer grown with hipMalloc, a reuse a request
// the held buffer already covers; live bytes are the held capacities;
// read-backs count the device-to-host copies the library makes (a total, a
// flag, k-means sums) -- 0 for the search, assignment and pairwise paths.
mlrs_pool_stats g_pool[kMaxDevices];

void pool_note_grow(int dev, size_t old_cap, size_t new_cap) {
    mlrs_pool_stats& P = g_pool[dev];
    P.allocations += 1;
    P.live_bytes = P.live_bytes - old_cap + new_cap;
    if (P.live_bytes > P.peak_bytes) P.peak_bytes = P.live_bytes;
}

void pool_note_release(int dev, size_t cap) { g_pool[dev].live_bytes -= cap; }

// Counted before each device-to-host copy of the running call.
void note_read_back() {
    int dev = -1;
    if (g_call && g_call->armed) dev = g_call->dev;
    else if (hipGetDevice(&dev) != hipSuccess) return;
    if (dev >= 0 && dev < kMaxDevices) g_pool[dev].read_backs += 1;
}

// Bytes a call may carve from the workspace (the static scratch's size in the
// allocation-free variant, else unbounded).
size_t workspace_limit() { return g_noalloc ? (size_t)MLRS_NOALLOC_SCRATCH_BYTES : SIZE_MAX; }

// 1 where the device has stream-ordered memory pools, 0 where not, -1 unknown.
int g_mempools[kMaxDevices];
bool g_mempools_init = [] {
    for (int& v : g_mempools) v = -1;
    return true;
}();

// Replace a cached buffer (*base, *pooled) by one of `want` bytes.  The old
// buffer is read only by the library's own earlier work on this device, and
// the call ordering (order_after_last_call, which every grower runs first)
// has already put stream `s` after all of it.  With memory pools the old
// buffer is therefore returned and the new one taken in stream order on `s`
// (hipFreeAsync, hipMallocAsync): neither waits for other streams, nor for
// the host.  Without them (and for a buffer hipMalloc made) the old buffer
// goes after a device-wide synchronize, since hipFree waits for the device.
// On failure *base is null.
hipError_t buffer_regrow(int dev, char** base, bool* pooled, size_t want, hipStream_t s) {
    if (g_mempools[dev] < 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMemoryPoolsSupported, dev) != hipSuccess) v = 0;
        g_mempools[dev] = v ? 1 : 0;
    }
    hipError_t e = hipSuccess;
    if (*base) {
        if (*pooled) {
            e = hipFreeAsync(*base, s);
        } else {
            e = hipDeviceSynchronize();
            if (e == hipSuccess) (void)hipFree(*base);
        }
        *base = nullptr;
        if (e != hipSuccess) return e;
    }
    if (g_mempools[dev]) {
        e = hipMallocAsync((void**)base, want, s);
        *pooled = true;
    } else {
        e = hipMalloc((void**)base, want);
        *pooled = false;
    }
    if (e != hipSuccess) *base = nullptr;
    return e;
}

// Return a cached buffer at release (the caller has synchronized the device).
void buffer_free(char** base, bool* pooled) {
    if (!*base) return;
    if (*pooled) {
        (void)hipFreeAsync(*base, nullptr);
        (void)hipStreamSynchronize(nullptr);
    } else {
        (void)hipFree(*base);
    }
    *base = nullptr;
    *pooled = false;
}

// Growing a cached buffer waits for nothing but the call's own stream order
// (buffer_regrow).
int32_t workspace(size_t bytes, hipStream_t s, char** out, int* cus) {
    int dev = 0;
    int32_t rc = current_device(&dev);
    if (rc) return rc;
    hipError_t e;
    Arena& A = g_arena[dev];
    if (A.cus == 0) {
        int n = 0;
        e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return hip_err(e, "hipDeviceGetAttribute");
        A.cus = n > 0 ? n : 1;
    }
    *cus = A.cus;
    if (bytes == 0) bytes = 256;
    if (g_noalloc) {
        if (bytes > (size_t)MLRS_NOALLOC_SCRATCH_BYTES)
            return set_err(MLRS_ERR_UNSUPPORTED, "scratch", (int64_t)bytes, 0, (int64_t)MLRS_NOALLOC_SCRATCH_BYTES, 0,
                           "this search needs %zu bytes of scratch; the allocation-free entry point holds %zu",
                           bytes, (size_t)MLRS_NOALLOC_SCRATCH_BYTES);
        *out = g_noalloc_base;
        return MLRS_OK;
    }
    rc = order_after_last_call(dev, s);
    if (rc) return rc;
    if (A.cap < bytes) {
        const size_t old_cap = A.cap;
        size_t want = std::max(bytes + bytes / 4, (size_t)64 << 20);
        e = buffer_regrow(dev, &A.base, &A.pooled, want, s);
        if (e != hipSuccess) {
            A.cap = 0;
            pool_note_release(dev, old_cap);
            return set_err(MLRS_ERR_ALLOC, "workspace", (int64_t)want, 0, 0, (int)e,
                           "device workspace allocation of %zu bytes failed: %s", want, hipGetErrorString(e));
        }
        A.cap = want;
        pool_note_grow(dev, old_cap, want);
    } else {
        g_pool[dev].reuses += 1;
    }
    *out = A.base;
    return MLRS_OK;
}

// ---------------------------------------------------------------------------
// measurement hook: events around the dominant kernel launch
// ---------------------------------------------------------------------------
struct TimedLaunch {
    hipEvent_t a, b;
    const char* name;  // a string literal: the timed kernel (or region)
};
bool g_timing = false;
std::vector<TimedLaunch> g_timed;

struct KernelTimer {
    hipStream_t s;
    TimedLaunch t{nullptr, nullptr, nullptr};
    KernelTimer(hipStream_t st, const char* name) : s(st) {
        if (!g_timing || g_noalloc) return;
        if (hipEventCreate(&t.a) != hipSuccess || hipEventCreate(&t.b) != hipSuccess) {
            t.a = t.b = nullptr;
            return;
        }
        t.name = name;
        (void)hipEventRecord(t.a, s);
    }
    ~KernelTimer() {
        if (!g_timing || !t.a) return;
        (void)hipEventRecord(t.b, s);
        g_timed.push_back(t);
    }
};

void clear_timed() {
    for (auto& t : g_timed) {
        (void)hipEventDestroy(t.a);
        (void)hipEventDestroy(t.b);
    }
    g_timed.clear();
}

// ---------------------------------------------------------------------------
// arm selection: the cpu-backend dispatch of metric_topk
// ---------------------------------------------------------------------------
// crates/mlrs-algos/src/neighbors/nearest.rs:910-947 with the caps of
// cpu_rows_applicable (prims/knn.rs:400-412: d <= 32, k <= 16) and
// cpu_metric_rows_applicable (prims/knn.rs:703-720: d <= 128, k <= 128).
// minkowski_powi (crates/mlrs-backend/src/prims/knn.rs:680-687): an integer p
// in 3..8 runs a multiply chain, anything else pow.
static int minkowski_powi(double p) {
    const double pf = std::floor(p);
    return (p == pf && pf >= 3.0 && pf <= 8.0) ? (int)pf : 0;
}

int knn_arm(int64_t d, int64_t k, int metric, double p = 2.0) {
    const bool metric_family = d >= 1 && d <= 128 && k >= 1 && k <= 128;
    switch (metric) {
    case MLRS_METRIC_EUCLIDEAN: return metric_family ? ARM_EUCLID_FMA : ARM_EUCLID_MULADD;
    case MLRS_METRIC_COSINE: return metric_family ? ARM_COS_FOLD : ARM_COS_HOST;
    case MLRS_METRIC_MANHATTAN: return ARM_MANHATTAN;    // one arithmetic on every arm
    case MLRS_METRIC_CHEBYSHEV: return ARM_CHEBYSHEV;
    default: return minkowski_powi(p) ? ARM_MINKOWSKI_INT : ARM_MINKOWSKI_POW;
    }
}

// Split the index axis so the grid has enough workgroups to fill the chip,
// preferring a total that is a whole number of waves of workgroups.
int pick_strips(int64_t nblocks, int64_t nt, int64_t slots, int64_t min_rows, int max_strips) {
    int64_t best_s = 1;
    double best_cost = 1e300;
    int64_t s_hi = std::max<int64_t>(1, std::min<int64_t>(max_strips, (nt + min_rows - 1) / min_rows));
    for (int64_t s = 1; s <= s_hi; ++s) {
        int64_t wgs = nblocks * s;
        int64_t rounds = (wgs + slots - 1) / slots;
        // time ~ rounds * (work per WG) = rounds / s; penalize the merge a little
        double cost = (double)rounds / (double)s * (1.0 + 0.002 * (double)s);
        if (cost < best_cost - 1e-12) {
            best_cost = cost;
            best_s = s;
        }
    }
    return (int)best_s;
}

// The Gram kernel gives each XCD an equal contiguous range of the strip-major
// work items, so the balance that matters is per XCD: ceil(s*nblocks/8)
// workgroups over the XCD's slots.
int pick_strips_xcd(int64_t nblocks, int64_t nt, int64_t slots_per_xcd, int64_t min_rows, int max_strips) {
    int64_t best_s = 1;
    double best_cost = 1e300;
    int64_t s_hi = std::max<int64_t>(1, std::min<int64_t>(max_strips, (nt + min_rows - 1) / min_rows));
    for (int64_t s = 1; s <= s_hi; ++s) {
        int64_t per_xcd = (s * nblocks + 7) / 8;
        int64_t rounds = (per_xcd + slots_per_xcd - 1) / slots_per_xcd;
        double cost = (double)rounds / (double)s * (1.0 + 0.002 * (double)s);
        if (cost < best_cost - 1e-12) {
            best_cost = cost;
            best_s = s;
        }
    }
    return (int)best_s;
}

// ---------------------------------------------------------------------------
// generic exact path: tile of exact pairwise values + per-row selection
// ---------------------------------------------------------------------------
template <typename T>
int32_t knn_generic(const T* xq, int64_t nq, const T* xt, int64_t nt, int64_t d, int k, int arm, int mode,
                    T* out_v, uint32_t* out_i, hipStream_t s, double p = 2.0) {
    const bool cos = (arm == ARM_COS_FOLD || arm == ARM_COS_HOST);
    // per query row of a tile: its exact values plus the selection's scratch
    const size_t fixed = 4 * aligned_bytes(sizeof(T) * (nq + nt)) + 4096;
    const size_t per_row = sizeof(T) * (size_t)std::max<int64_t>(nt, 1) + select_rows_scratch_bytes(1, k, sizeof(T));
    size_t tile_budget = (size_t)256 << 20;
    const size_t limit = workspace_limit();
    if (limit != SIZE_MAX) tile_budget = std::min(tile_budget, limit > fixed ? limit - fixed : 0);
    int64_t qt = (int64_t)(tile_budget / per_row);
    qt = std::max<int64_t>(1, std::min<int64_t>(qt, nq));
    const size_t sel_bytes = select_rows_scratch_bytes(qt, k, sizeof(T));
    size_t bytes = aligned_bytes(sizeof(T) * (size_t)qt * nt) + sel_bytes + fixed;
    char* ws;
    int cus;
    int32_t rc = workspace(bytes, s, &ws, &cus);
    if (rc) return rc;
    Carver cv(ws);
    T* dist = cv.take<T>((size_t)qt * nt);
    void* sel = sel_bytes ? (void*)cv.take<char>(sel_bytes) : nullptr;
    T* qa = nullptr;
    T* xa = nullptr;
    if (cos) {
        qa = cv.take<T>(nq);
        xa = cv.take<T>(nt);
        hipError_t e;
        if (arm == ARM_COS_HOST) {
            // reciprocal norms (row_inv_norm_host), squared norms discarded
            T* qsq = cv.take<T>(nq);
            T* xsq = cv.take<T>(nt);
            e = launch_row_norms<T>(xq, nq, d, qsq, qa, nullptr, nullptr, s);
            if (e == hipSuccess) e = launch_row_norms<T>(xt, nt, d, xsq, xa, nullptr, nullptr, s);
        } else {
            // squared norms (row_sumsq)
            e = launch_row_norms<T>(xq, nq, d, qa, nullptr, nullptr, nullptr, s);
            if (e == hipSuccess) e = launch_row_norms<T>(xt, nt, d, xa, nullptr, nullptr, nullptr, s);
        }
        if (e != hipSuccess) return hip_err(e, "row_norms");
    }
    const bool minkowski = (arm == ARM_MINKOWSKI_INT || arm == ARM_MINKOWSKI_POW);
    // EMIT_ROOT_RANKED: the tile holds the roots (sqrt, or pow(v, 1/p) for
    // Minkowski), so the selection ranks by (root, index)
    const bool ranked = mode == EMIT_ROOT_RANKED;
    const int root = ranked ? (minkowski ? 2 : 1) : 0;
    for (int64_t q0 = 0; q0 < nq; q0 += qt) {
        int64_t rows = std::min<int64_t>(qt, nq - q0);
        hipError_t e;
        {
            KernelTimer timer(s, "pairwise_tile_kernel");
            e = launch_pairwise_tile<T>(xq + q0 * d, rows, xt, nt, d, arm, cos ? qa + q0 : nullptr, xa, dist,
                                        nt, root, s, (T)p, minkowski_powi(p), (T)(1.0 / p));
        }
        if (e == hipSuccess)
            e = launch_select_rows<T>(dist, rows, nt, nt, k, ranked ? EMIT_IDENTITY : mode, out_v + q0 * k,
                                      out_i + q0 * k, sel, s);
        if (e != hipSuccess) return hip_err(e, "generic kNN");
    }
    // Minkowski's boundary root over the emitted values, exponent
    // f64_to_host(1/p) (prims/knn.rs:882-888)
    if (minkowski && !ranked) {
        hipError_t e = launch_pow_inplace<T>(out_v, nq * k, (T)(1.0 / p), s);
        if (e != hipSuccess) return hip_err(e, "minkowski root");
    }
    return ok();
}

template <typename T>
int32_t kmeans_generic(const T* x, int64_t n, const T* c, int64_t kc, int64_t d, uint32_t* labels, T* dist,
                       hipStream_t s) {
    const size_t tile_budget = (size_t)256 << 20;
    int64_t qt = (int64_t)(tile_budget / (sizeof(T) * (size_t)std::max<int64_t>(kc, 1)));
    qt = std::max<int64_t>(1, std::min<int64_t>(qt, n));
    char* ws;
    int cus;
    int32_t rc = workspace(aligned_bytes(sizeof(T) * (size_t)qt * kc) + 256, s, &ws, &cus);
    if (rc) return rc;
    T* buf = reinterpret_cast<T*>(ws);
    for (int64_t r0 = 0; r0 < n; r0 += qt) {
        int64_t rows = std::min<int64_t>(qt, n - r0);
        hipError_t e = launch_pairwise_tile<T>(x + r0 * d, rows, c, kc, d, ARM_EUCLID_MULADD, nullptr, nullptr,
                                               buf, kc, 0, s);
        if (e == hipSuccess) e = launch_argmin_rows<T>(buf, rows, kc, kc, labels + r0, dist + r0, s);
        if (e != hipSuccess) return hip_err(e, "generic k-means assignment");
    }
    return ok();
}

// ---------------------------------------------------------------------------
// fast paths
// ---------------------------------------------------------------------------
// Below about 4e9 multiply-adds the whole exact distance matrix is cheaper
// than the fused kernel's fixed costs (a few flush round trips per segment
// and query): c1's 1k x 10k x 64 search takes 0.05 ms of exact tiles against
// 0.5 ms fused on an MI355X.
static bool small_search(int64_t nq, int64_t nt, int64_t d) {
    return (double)nq * (double)nt * (double)d <= 4294967296.0;
}

// f32 searches the low-d ALU kernel serves faster than the Gram kernel
// (timed on 500,000-row self-searches: the ALU kernel's cost grows with d
// and, past list capacity 16, with one query per lane instead of two; the
// Gram kernel's is nearly flat for d <= 16): every d at k <= 8, d <= 11 at
// k <= 16, and for Euclidean d <= 3 at k <= 32 (cosine at d = 3, k = 32:
// 176 ms against the Gram kernel's 149).  f64 always takes the ALU kernel
// (its Gram kernel runs 2.4-12x slower there).
static bool lowd_f32_faster(int64_t d, int64_t k, bool cos) {
    if (k <= 8) return true;
    if (k <= 16) return d <= 11;
    return !cos && d <= 3;
}

// Process-wide kernel-family override (mlrs_force_path); a family that does
// not serve the shape yields the automatic choice.
static int g_force_path = MLRS_PATH_AUTO;
static int pick_path(bool lowd_ok, bool gram_ok) {
    if (g_force_path == MLRS_PATH_FUSED && gram_ok) return MLRS_PATH_FUSED;
    if (g_force_path == MLRS_PATH_LOWD && lowd_ok) return MLRS_PATH_LOWD;
    if (g_force_path == MLRS_PATH_GENERIC) return MLRS_PATH_GENERIC;
    return MLRS_PATH_AUTO;
}

// qsq_pre: the queries' row_sumsq when the caller already holds them (the
// k-means loop assigns the same rows every iteration); Euclidean arms only.
int32_t knn_gram32(const float* xq, int64_t nq, const float* xt, int64_t nt, int64_t d, int k, int arm,
                   int mode, float* out_v, uint32_t* out_i, hipStream_t s, const float* qsq_pre = nullptr) {
    const bool cos = (arm == ARM_COS_FOLD || arm == ARM_COS_HOST);
    const bool host_cos = arm == ARM_COS_HOST;
    // sizes that do not depend on the strip count
    size_t fixed = 2 * aligned_bytes(sizeof(float) * nq) + 3 * aligned_bytes(sizeof(float) * nt) +
                   aligned_bytes(sizeof(NormStats)) + 1024;
    char* ws;
    int cus;
    int32_t rc = workspace(fixed, s, &ws, &cus);
    if (rc) return rc;
    int64_t grid_wgs = 1;
    int nslots = 1;
    const bool vec4 = (d % 4 == 0) && ((reinterpret_cast<uintptr_t>(xq) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(xt) & 15) == 0);
    gram_f32_split(nq, nt, d, k, cus, vec4, &grid_wgs, &nslots);
    // k = 1 over an index that a few workgroups' LDS holds: the resident
    // search (knn_k1_resident.hip), one list slot per chunk
    const int res_chunks = gram_f32_k1_resident_chunks(nq, nt, d, k, arm, vec4);
    // per-(segment slot, query) lists: the kernel's top-k state, merged at the end
    size_t parts = (size_t)std::max<int64_t>(nslots, res_chunks) * nq * gram_list_cap(k);
    size_t qvals = (k > 1) ? gram_f32_qval_elems(grid_wgs, k)
                 : res_chunks ? (gram_f32_k1_resident_queue_bytes(cus) + sizeof(float) - 1) / sizeof(float) : 0;
    size_t summs = (k > 1) ? (size_t)nslots * nq : 0;
    size_t bytes = fixed + aligned_bytes(parts * sizeof(float)) + aligned_bytes(parts * sizeof(uint32_t)) +
                   aligned_bytes(qvals * sizeof(float)) + aligned_bytes(summs * sizeof(float4)) +
                   aligned_bytes(sizeof(unsigned int) * nq);
    // the seed's screen values on the matrix cores, where served and where
    // the workspace allows (otherwise the exact seed, which needs none)
    size_t seed_bytes = gram_f32_seed_screen_bytes(nq, nt, d, k, arm, vec4);
    if (seed_bytes && bytes + aligned_bytes(seed_bytes) > workspace_limit()) seed_bytes = 0;
    if (seed_bytes) bytes += aligned_bytes(seed_bytes);
    rc = workspace(bytes, s, &ws, &cus);
    if (rc) return rc;
    Carver cv(ws);
    GramArgs32 a;
    std::memset(&a, 0, sizeof(a));
    float* qsq = cv.take<float>(nq);
    float* qinv = cv.take<float>(nq);
    float* xsq = cv.take<float>(nt);
    float* xinv = cv.take<float>(nt);
    float* xscale = cv.take<float>(nt);
    NormStats* stats = cv.take<NormStats>(1);
    hipError_t e = hipSuccess;
    // the resident k = 1 search forms the query norms from its operand
    const bool res_qsq = res_chunks && !qsq_pre;
    if (qsq_pre && !cos)
        qsq = const_cast<float*>(qsq_pre);  // only read
    else if (!res_qsq)
        e = launch_row_norms<float>(xq, nq, d, qsq, host_cos ? qinv : nullptr, nullptr, nullptr, s);
    if (e == hipSuccess)
        e = launch_row_norms<float>(xt, nt, d, xsq, host_cos ? xinv : nullptr, cos ? xscale : nullptr, stats, s);
    if (e != hipSuccess) return hip_err(e, "row_norms");
    a.q = xq;
    a.nq = nq;
    a.x = xt;
    a.nt = nt;
    a.d = d;
    a.k = k;
    a.mode = mode;
    a.qsq = qsq;
    a.xsq = xsq;
    a.xscale = xscale;
    a.qinv = host_cos ? qinv : nullptr;
    a.xinv = host_cos ? xinv : nullptr;
    a.stats = stats;
    // Screen bounds (see knn_gram_f32.hip): with u = 2^-23 (covers any
    // rounding mode of the matrix core) the expansion's and the reference's
    // rounding errors together stay below 6(d+3)u(||q||^2 + ||x||^2) for
    // Euclidean and (4d+11)u for cosine; the bounds used are 8(d+4)u and
    // (8d+32)u, plus an absolute floor for flushed subnormal products.
    const double u = std::ldexp(1.0, -23);
    if (!cos) {
        a.eps_rel = 8.0 * (double)(d + 4) * u;
        a.eps_abs = (double)(d + 4) * std::ldexp(1.0, -120);
    } else {
        a.eps_rel = 0.0;
        a.eps_abs = (8.0 * (double)d + 32.0) * u;
    }
    a.grid_wgs = grid_wgs;
    a.nslots = nslots;
    a.qpb = gram_f32_queries_per_block(d);
    a.part_val = cv.take<float>(parts);
    a.part_idx = cv.take<uint32_t>(parts);
    if (qvals) a.qval = cv.take<float>(qvals);
    if (summs) a.summ = cv.take<float4>(summs);
    if (nslots > 1 || k > 1) a.shared_r = cv.take<unsigned int>(nq);
    void* seed_buf = seed_bytes ? static_cast<void*>(cv.take<char>(seed_bytes)) : nullptr;
    a.out_val = out_v;
    a.out_idx = out_i;
    if (res_chunks) {
        {
            KernelTimer timer(s, "knn_k1_resident_f32_kernel");
            e = launch_gram_f32_k1_resident(a, arm, cus, res_qsq ? qsq : nullptr, s);
        }
        if (e == hipSuccess) e = launch_gram_f32_k1_resident_merge(a, res_chunks, s);
        if (e != hipSuccess) return hip_err(e, "knn_k1_resident_f32");
        return ok();
    }
    e = launch_gram_f32_prep(a, arm, s, seed_buf);
    if (e == hipSuccess) {
        KernelTimer timer(s, "knn_gram_f32_kernel");
        e = launch_gram_f32(a, arm, s);
    }
    if (e == hipSuccess) e = launch_gram_f32_merge(a, arm, s);
    if (e != hipSuccess) return hip_err(e, "knn_gram_f32");
    return ok();
}

int32_t knn_gram64(const double* xq, int64_t nq, const double* xt, int64_t nt, int64_t d, int k, int arm,
                   int mode, double* out_v, uint32_t* out_i, hipStream_t s, const double* qsq_pre = nullptr) {
    const bool cos = (arm == ARM_COS_FOLD || arm == ARM_COS_HOST);
    size_t fixed = 2 * aligned_bytes(sizeof(double) * nq) + 3 * aligned_bytes(sizeof(double) * nt) +
                   aligned_bytes(sizeof(NormStats)) + 1024;
    char* ws;
    int cus;
    int32_t rc = workspace(fixed, s, &ws, &cus);
    if (rc) return rc;
    int64_t grid_wgs = 1;
    int nslots = 1;
    gram_f64_split(nq, nt, cus, &grid_wgs, &nslots);
    size_t parts = (size_t)nslots * nq * gram_list_cap(k);
    size_t qvals = gram_f64_qval_elems(grid_wgs);
    const bool ranked = mode == EMIT_ROOT_RANKED;
    size_t bytes = fixed + aligned_bytes(parts * sizeof(double)) + aligned_bytes(parts * sizeof(uint32_t)) +
                   aligned_bytes(qvals * sizeof(double)) + aligned_bytes(sizeof(unsigned long long) * nq) +
                   (ranked ? aligned_bytes(sizeof(uint32_t) * nq) : 0);
    // the seed's screen values on the matrix cores where the workspace allows
    const bool vec2 = (d % 2 == 0) && ((reinterpret_cast<uintptr_t>(xq) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(xt) & 15) == 0);
    size_t seed_bytes = gram_f64_seed_screen_bytes(nq, nt, d, k, vec2);
    if (seed_bytes && bytes + aligned_bytes(seed_bytes) > workspace_limit()) seed_bytes = 0;
    if (seed_bytes) bytes += aligned_bytes(seed_bytes);
    rc = workspace(bytes, s, &ws, &cus);
    if (rc) return rc;
    Carver cv(ws);
    GramArgs64 a;
    std::memset(&a, 0, sizeof(a));
    double* qsq = cv.take<double>(nq);
    double* qinv = cv.take<double>(nq);
    double* xsq = cv.take<double>(nt);
    double* xinv = cv.take<double>(nt);
    double* xscale = cv.take<double>(nt);
    NormStats* stats = cv.take<NormStats>(1);
    hipError_t e = hipSuccess;
    if (qsq_pre && !cos)
        qsq = const_cast<double*>(qsq_pre);  // only read; qinv serves cosine only
    else
        e = launch_row_norms<double>(xq, nq, d, qsq, qinv, nullptr, nullptr, s);
    if (e == hipSuccess) e = launch_row_norms<double>(xt, nt, d, xsq, xinv, xscale, stats, s);
    if (e != hipSuccess) return hip_err(e, "row_norms");
    a.q = xq;
    a.nq = nq;
    a.x = xt;
    a.nt = nt;
    a.d = d;
    a.k = k;
    a.mode = mode;
    a.qsq = qsq;
    a.xsq = xsq;
    a.qinv = qinv;
    a.xinv = xinv;
    a.xscale = xscale;
    a.stats = stats;
    // Screen bounds as for f32 with u = 2^-52, plus 16u (Euclidean, relative)
    // and 16u (cosine, absolute) for the rounding of the threshold arithmetic
    // itself, which the f64 kernel does in double.
    const double u = std::ldexp(1.0, -52);
    if (!cos) {
        a.eps_rel = (8.0 * (double)(d + 4) + 16.0) * u;
        a.eps_abs = (double)(d + 4) * std::ldexp(1.0, -1000);
    } else {
        a.eps_rel = 0.0;
        a.eps_abs = (8.0 * (double)d + 48.0) * u;
    }
    a.grid_wgs = grid_wgs;
    a.nslots = nslots;
    a.part_val = cv.take<double>(parts);
    a.part_idx = cv.take<uint32_t>(parts);
    a.qval = cv.take<double>(qvals);
    a.shared_r = cv.take<unsigned long long>(nq);
    a.root_flag = ranked ? cv.take<unsigned int>(nq) : nullptr;
    void* seed_buf = seed_bytes ? static_cast<void*>(cv.take<char>(seed_bytes)) : nullptr;
    a.out_val = out_v;
    a.out_idx = out_i;
    e = launch_gram_f64_prep(a, arm, s, seed_buf);
    if (e == hipSuccess) {
        KernelTimer timer(s, "knn_gram_f64_kernel");
        e = launch_gram_f64(a, arm, s);
    }
    if (e == hipSuccess) e = launch_gram_f64_merge(a, arm, s);
    if (e == hipSuccess && ranked) e = launch_gram_f64_root_fill(a, arm, s);
    if (e != hipSuccess) return hip_err(e, "knn_gram_f64");
    return ok();
}

// The low-d ALU path (knn_lowd.hip), f32 and f64.
static hipError_t launch_lowd_t(const LowdArgs32& a, int arm, hipStream_t s) { return launch_lowd_f32(a, arm, s); }
static hipError_t launch_lowd_t(const LowdArgs64& a, int arm, hipStream_t s) { return launch_lowd_f64(a, arm, s); }

template <typename T>
int32_t knn_lowd(const T* xq, int64_t nq, const T* xt, int64_t nt, int64_t d, int k, int arm, int mode,
                 T* out_v, uint32_t* out_i, hipStream_t s) {
    typedef typename LowdBits<T>::type B;
    const bool cos = arm == ARM_COS_FOLD;
    const size_t fixed = aligned_bytes(sizeof(T) * nq) + (cos ? 2 : 1) * aligned_bytes(sizeof(T) * nt) +
                         aligned_bytes(sizeof(NormStats)) + 1024;
    char* ws;
    int cus;
    int32_t rc = workspace(fixed, s, &ws, &cus);
    if (rc) return rc;
    const int qpb = lowd_queries_per_block(k, d, (int)sizeof(T));
    const int64_t nblocks = (nq + qpb - 1) / qpb;
    // ~3 resident 256-lane workgroups per CU (the k <= 8 kernel holds ~150 VGPRs)
    int nstrips = pick_strips(nblocks, nt, (int64_t)cus * 3, 4096, 64);
    int64_t rps = (nt + nstrips - 1) / nstrips;
    nstrips = (int)((nt + rps - 1) / rps);
    size_t parts = nstrips > 1 ? (size_t)nstrips * nq * k : 0;
    if (parts) {
        rc = workspace(fixed + aligned_bytes(parts * sizeof(T)) + aligned_bytes(parts * sizeof(uint32_t)) +
                           aligned_bytes(sizeof(B) * nq),
                       s, &ws, &cus);
        if (rc) return rc;
    }
    Carver cv(ws);
    LowdArgs<T> a;
    std::memset(&a, 0, sizeof(a));
    T* qsq = cv.take<T>(nq);
    T* xsq = cv.take<T>(nt);
    T* xscale = cos ? cv.take<T>(nt) : nullptr;
    NormStats* stats = cv.take<NormStats>(1);
    hipError_t e = launch_row_norms<T>(xq, nq, d, qsq, nullptr, nullptr, nullptr, s);
    if (e == hipSuccess) e = launch_row_norms<T>(xt, nt, d, xsq, nullptr, xscale, stats, s);
    if (e != hipSuccess) return hip_err(e, "row_norms");
    a.q = xq;
    a.nq = nq;
    a.x = xt;
    a.nt = nt;
    a.d = d;
    a.k = k;
    a.mode = mode;
    a.qsq = qsq;
    a.xsq = xsq;
    a.xscale = xscale;
    a.stats = stats;
    // the Gram kernels' screen bounds (knn_gram32 / knn_gram64) with the
    // element type's unit: 2^-23 (f32) or 2^-52 (f64).  Euclidean: the
    // threshold arithmetic carries its own rounding margin; cosine: f32 rounds
    // the threshold up from double, f64 folds its rounding into eps (+16 u).
    const bool f64 = sizeof(T) == 8;
    const double u = std::ldexp(1.0, f64 ? -52 : -23);
    if (cos) {
        a.eps_rel = 0.0;
        a.eps_abs = (8.0 * (double)d + (f64 ? 48.0 : 32.0)) * u;
    } else {
        a.eps_rel = 8.0 * (double)(d + 4) * u;
        a.eps_abs = (double)(d + 4) * std::ldexp(1.0, f64 ? -1000 : -120);
    }
    a.rows_per_strip = rps;
    a.nstrips = nstrips;
    if (parts) {
        a.part_val = cv.take<T>(parts);
        a.part_idx = cv.take<uint32_t>(parts);
        a.shared_r = cv.take<B>(nq);
    }
    a.out_val = out_v;
    a.out_idx = out_i;
    {
        KernelTimer timer(s, "knn_lowd_kernel");
        e = launch_lowd_t(a, arm, s);
    }
    if (e != hipSuccess) return hip_err(e, f64 ? "knn_lowd_f64" : "knn_lowd_f32");
    return ok();
}

template <typename T>
int32_t validate_knn(const T* xq, int64_t xq_len, int64_t nq, int64_t d, const T* xt, int64_t xt_len,
                     int64_t nt, int32_t k, int32_t metric, const void* ov, const void* oi, int64_t out_len) {
    if (!geom_ok(nq, d, xq_len)) return shape_err("x", nq, d, xq_len);
    if (!geom_ok(nt, d, xt_len)) return shape_err("y", nt, d, xt_len);
    if (k < 1 || (int64_t)k > nt) return shape_err("k", 1, k, nt);
    if (d < 1) return shape_err("features", d, 0, 0);
    if (nq > kU32Max || nt > kU32Max) return shape_err("rows", std::max(nq, nt), 0, kU32Max);
    if (!geom_ok(nq, k, out_len)) return shape_err("out", nq, k, out_len);
    if (metric < MLRS_METRIC_EUCLIDEAN || metric > MLRS_METRIC_MINKOWSKI)
        return set_err(MLRS_ERR_UNSUPPORTED, "metric", metric, 0, 0, 0, "metric %d is not served", metric);
    if (nq > 0 && (!xq || !ov || !oi)) return set_err(MLRS_ERR_NULL_POINTER, "x", 0, 0, 0, 0, "null pointer");
    if (!xt) return set_err(MLRS_ERR_NULL_POINTER, "y", 0, 0, 0, 0, "null pointer");
    return MLRS_OK;
}

}  // namespace

// ===========================================================================
// exported entry points
// ===========================================================================
extern "C" {

int32_t mlrs_abi_version(void) { return MLRS_ABI_VERSION; }

int32_t mlrs_last_error(mlrs_error_info* out) {
    if (out) *out = g_err;
    return g_err.code;
}

const char* mlrs_status_string(int32_t code) {
    switch (code) {
    case MLRS_OK: return "ok";
    case MLRS_ERR_SHAPE_MISMATCH: return "shape mismatch";
    case MLRS_ERR_DIM_MISMATCH: return "dimension mismatch";
    case MLRS_ERR_UNSUPPORTED: return "unsupported metric or shape";
    case MLRS_ERR_NULL_POINTER: return "null pointer";
    case MLRS_ERR_HIP: return "HIP runtime error";
    case MLRS_ERR_ALLOC: return "device workspace allocation failed";
    case MLRS_ERR_INVALID_PARAM: return "invalid parameter value";
    default: return "unknown status";
    }
}

int32_t mlrs_knn_max_k(int32_t dtype_bytes, int64_t n_features, int32_t metric) {
    (void)dtype_bytes;
    (void)n_features;
    (void)metric;
    return INT32_MAX;  // every 1 <= k <= n_train
}

}  // extern "C"

namespace {
int32_t knn_topk_f32_dispatch(const float* xq, int64_t n_query, int64_t n_features, const float* x_train,
                              int64_t n_train, int32_t k, int32_t metric, double p, float* out_dist,
                              uint32_t* out_idx, hipStream_t s) {
    const int arm = knn_arm(n_features, k, metric, p);
    const int mode = (metric == MLRS_METRIC_EUCLIDEAN) ? EMIT_SQRT : EMIT_IDENTITY;
    const bool lowd_ok = (metric == MLRS_METRIC_EUCLIDEAN || (metric == MLRS_METRIC_COSINE && arm == ARM_COS_FOLD)) &&
                         n_features <= lowd_max_d() && k <= lowd_max_k();
    // the knn_host cosine arm on the matrix cores in the wide shape only (it
    // serves d > 128, where the wide shape runs)
    const bool gram_ok = (arm == ARM_EUCLID_FMA || arm == ARM_EUCLID_MULADD || arm == ARM_COS_FOLD ||
                          (arm == ARM_COS_HOST && n_features > 128)) &&
                         n_features <= gram_f32_max_d() && k <= gram_f32_max_k();
    const bool small = small_search(n_query, n_train, n_features);
    int path = pick_path(lowd_ok, gram_ok);
    if (path == MLRS_PATH_AUTO)
        path = (lowd_ok && (small || !gram_ok || lowd_f32_faster(n_features, k, metric == MLRS_METRIC_COSINE))) ? MLRS_PATH_LOWD
               : (gram_ok && !small)                                             ? MLRS_PATH_FUSED
                                                                                 : MLRS_PATH_GENERIC;
    if (path == MLRS_PATH_LOWD)
        return knn_lowd<float>(xq, n_query, x_train, n_train, n_features, k, arm, mode, out_dist, out_idx, s);
    if (path == MLRS_PATH_FUSED)
        return knn_gram32(xq, n_query, x_train, n_train, n_features, k, arm, mode, out_dist, out_idx, s);
    return knn_generic<float>(xq, n_query, x_train, n_train, n_features, k, arm, mode, out_dist, out_idx, s, p);
}

int32_t knn_topk_f32_validate(const float* xq, int64_t xq_len, int64_t n_query, int64_t n_features,
                              const float* x_train, int64_t xt_len, int64_t n_train, int32_t k, int32_t metric,
                              double p, float* out_dist, uint32_t* out_idx, int64_t out_len) {
    int32_t rc = validate_knn<float>(xq, xq_len, n_query, n_features, x_train, xt_len, n_train, k, metric,
                                     out_dist, out_idx, out_len);
    if (rc) return rc;
    if (metric == MLRS_METRIC_MINKOWSKI && !(p >= 1.0))
        return set_err(MLRS_ERR_UNSUPPORTED, "p", 0, 0, 0, 0, "minkowski p must be >= 1");
    return MLRS_OK;
}

// The allocation-free variant's device address of the static scratch, per
// device, taken once with that device current.
char* g_scratch_dev[kMaxDevices];

struct NoAllocScope {
    NoAllocScope(char* base) {
        g_noalloc = true;
        g_noalloc_base = base;
    }
    ~NoAllocScope() {
        g_noalloc = false;
        g_noalloc_base = nullptr;
    }
};
}  // namespace

extern "C" {

int32_t mlrs_knn_topk_f32(const float* xq, int64_t xq_len, int64_t n_query, int64_t n_features,
                          const float* x_train, int64_t xt_len, int64_t n_train, int32_t k, int32_t metric,
                          double p, float* out_dist, uint32_t* out_idx, int64_t out_len, void* stream) {
    CallGuard cg;
    int32_t rc = knn_topk_f32_validate(xq, xq_len, n_query, n_features, x_train, xt_len, n_train, k, metric, p,
                                       out_dist, out_idx, out_len);
    if (rc) return rc;
    if (n_query == 0) return MLRS_OK;
    return knn_topk_f32_dispatch(xq, n_query, n_features, x_train, n_train, k, metric, p, out_dist, out_idx,
                                 (hipStream_t)stream);
}

}  // extern "C"

// The allocation-free entry point's set-up on the current device, once: the
// scratch array's device address and the CU count the split reads.  Done by
// the first call on the device, which may have n_query = 0, so that calls
// captured into a graph afterwards make no such query.
static int32_t noalloc_setup(int* dev) {
    int32_t rc = current_device(dev);
    if (rc) return rc;
    if (g_scratch_dev[*dev]) return MLRS_OK;
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return hip_err(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress");
    if (g_arena[*dev].cus == 0) {
        int n = 0;
        e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, *dev);
        if (e != hipSuccess) return hip_err(e, "hipDeviceGetAttribute");
        g_arena[*dev].cus = n > 0 ? n : 1;
    }
    g_scratch_dev[*dev] = static_cast<char*>(ptr);
    return MLRS_OK;
}

extern "C" {

int32_t mlrs_knn_topk_f32_noalloc(const float* xq, int64_t xq_len, int64_t n_query, int64_t n_features,
                                  const float* x_train, int64_t xt_len, int64_t n_train, int32_t k, int32_t metric,
                                  double p, float* out_dist, uint32_t* out_idx, int64_t out_len, void* stream) {
    CallGuard cg;
    int32_t rc = knn_topk_f32_validate(xq, xq_len, n_query, n_features, x_train, xt_len, n_train, k, metric, p,
                                       out_dist, out_idx, out_len);
    if (rc) return rc;
    int dev = 0;
    if (n_query == 0) {
        // nothing to search: the device's set-up only, where there is a
        // device (a failure is reported by the first call with queries)
        (void)noalloc_setup(&dev);
        return MLRS_OK;
    }
    rc = noalloc_setup(&dev);
    if (rc) return rc;
    NoAllocScope scope(g_scratch_dev[dev]);
    return knn_topk_f32_dispatch(xq, n_query, n_features, x_train, n_train, k, metric, p, out_dist, out_idx,
                                 (hipStream_t)stream);
}

int32_t mlrs_knn_topk_f64(const double* xq, int64_t xq_len, int64_t n_query, int64_t n_features,
                          const double* x_train, int64_t xt_len, int64_t n_train, int32_t k, int32_t metric,
                          double p, double* out_dist, uint32_t* out_idx, int64_t out_len, void* stream) {
    CallGuard cg;
    int32_t rc = validate_knn<double>(xq, xq_len, n_query, n_features, x_train, xt_len, n_train, k, metric,
                                      out_dist, out_idx, out_len);
    if (rc) return rc;
    if (metric == MLRS_METRIC_MINKOWSKI && !(p >= 1.0))
        return set_err(MLRS_ERR_UNSUPPORTED, "p", 0, 0, 0, 0, "minkowski p must be >= 1");
    if (n_query == 0) return MLRS_OK;
    hipStream_t s = (hipStream_t)stream;
    const int arm = knn_arm(n_features, k, metric, p);
    const int mode = (metric == MLRS_METRIC_EUCLIDEAN) ? EMIT_SQRT : EMIT_IDENTITY;
    const bool lowd_ok = (metric == MLRS_METRIC_EUCLIDEAN || (metric == MLRS_METRIC_COSINE && arm == ARM_COS_FOLD)) &&
                         n_features <= lowd_max_d() && k <= lowd_max_k();
    const bool gram_ok = arm <= ARM_COS_HOST && n_features <= gram_f64_max_d() && k <= gram_f64_max_k();
    int path = pick_path(lowd_ok, gram_ok);
    if (path == MLRS_PATH_AUTO)
        path = lowd_ok ? MLRS_PATH_LOWD
                       : (gram_ok && !small_search(n_query, n_train, n_features)) ? MLRS_PATH_FUSED : MLRS_PATH_GENERIC;
    if (path == MLRS_PATH_LOWD)
        return knn_lowd<double>(xq, n_query, x_train, n_train, n_features, k, arm, mode, out_dist, out_idx, s);
    if (path == MLRS_PATH_FUSED)
        return knn_gram64(xq, n_query, x_train, n_train, n_features, k, arm, mode, out_dist, out_idx, s);
    return knn_generic<double>(xq, n_query, x_train, n_train, n_features, k, arm, mode, out_dist, out_idx, s, p);
}

extern "C++" {
template <typename T>
static int32_t validate_kmeans(const T* x, int64_t x_len, int64_t n, int64_t d, const T* c, int64_t c_len,
                               int64_t kc, const void* labels, int64_t labels_len, const void* dist,
                               int64_t dist_len) {
    // validate_geometry (prims/kmeans.rs:1416-1440) then assign_min's checks (:646-677)
    if (!geom_ok(n, d, x_len)) return shape_err("x", n, d, x_len);
    if (kc < 1 || kc > n) return shape_err("k", 1, kc, n);
    if (n > kU32Max) return shape_err("n", n, 0, kU32Max);
    if (d > kU32Max) return shape_err("d", d, 0, kU32Max);
    if (kc > kU32Max) return shape_err("k", kc, 0, kU32Max);
    if (!geom_ok(kc, d, c_len)) return shape_err("centers", kc, d, c_len);
    if (labels_len != n || dist_len != n) return shape_err("labels", n, 1, std::min(labels_len, dist_len));
    if (d < 1) return shape_err("x", n, d, x_len);
    if (!x || !c || !labels || !dist) return set_err(MLRS_ERR_NULL_POINTER, "x", 0, 0, 0, 0, "null pointer");
    return MLRS_OK;
}
}  // extern "C++"

int32_t mlrs_kmeans_assign_f32(const float* x, int64_t x_len, int64_t n, int64_t n_features, const float* centers,
                               int64_t centers_len, int64_t n_centers, uint32_t* labels, int64_t labels_len,
                               float* sqdist, int64_t dist_len, void* stream) {
    CallGuard cg;
    int32_t rc = validate_kmeans<float>(x, x_len, n, n_features, centers, centers_len, n_centers, labels,
                                        labels_len, sqdist, dist_len);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (n_features <= gram_f32_max_d() && pick_path(false, true) != MLRS_PATH_GENERIC)
        return knn_gram32(x, n, centers, n_centers, n_features, 1, ARM_EUCLID_MULADD, EMIT_KMEANS, sqdist, labels,
                          s);
    return kmeans_generic<float>(x, n, centers, n_centers, n_features, labels, sqdist, s);
}

int32_t mlrs_kmeans_assign_f64(const double* x, int64_t x_len, int64_t n, int64_t n_features,
                               const double* centers, int64_t centers_len, int64_t n_centers, uint32_t* labels,
                               int64_t labels_len, double* sqdist, int64_t dist_len, void* stream) {
    CallGuard cg;
    int32_t rc = validate_kmeans<double>(x, x_len, n, n_features, centers, centers_len, n_centers, labels,
                                         labels_len, sqdist, dist_len);
    if (rc) return rc;
    if (n_features <= gram_f64_max_d() && pick_path(false, true) != MLRS_PATH_GENERIC)
        return knn_gram64(x, n, centers, n_centers, n_features, 1, ARM_EUCLID_MULADD, EMIT_KMEANS, sqdist, labels,
                          (hipStream_t)stream);
    return kmeans_generic<double>(x, n, centers, n_centers, n_features, labels, sqdist, (hipStream_t)stream);
}

extern "C++" {
template <typename T>
static int32_t pairwise_impl(const T* x, int64_t x_len, int64_t rows_x, int64_t cols, const T* y, int64_t y_len,
                             int64_t rows_y, int64_t cols_y, int32_t metric, int32_t do_sqrt, double p, T* out,
                             int64_t out_len, void* stream) {
    CallGuard cg;
    if (!geom_ok(rows_x, cols, x_len)) return shape_err("x", rows_x, cols, x_len);
    if (!geom_ok(rows_y, cols_y, y_len)) return shape_err("y", rows_y, cols_y, y_len);
    if (cols != cols_y) return dim_err("cols", cols, cols_y);
    if (!geom_ok(rows_x, rows_y, out_len)) return shape_err("out", rows_x, rows_y, out_len);
    if (metric < MLRS_METRIC_EUCLIDEAN || metric > MLRS_METRIC_MINKOWSKI)
        return set_err(MLRS_ERR_UNSUPPORTED, "metric", metric, 0, 0, 0, "metric %d is not served", metric);
    if (metric == MLRS_METRIC_MINKOWSKI && !(p >= 1.0))
        return set_err(MLRS_ERR_UNSUPPORTED, "p", 0, 0, 0, 0, "minkowski p must be >= 1");
    if (rows_x == 0 || rows_y == 0) return MLRS_OK;
    if (!x || !y || !out) return set_err(MLRS_ERR_NULL_POINTER, "x", 0, 0, 0, 0, "null pointer");
    hipStream_t s = (hipStream_t)stream;
    const T* xa = nullptr;
    const T* ya = nullptr;
    int arm = ARM_EUCLID_MULADD;
    if (metric == MLRS_METRIC_COSINE) {
        arm = ARM_COS_PAIRWISE;
        char* ws;
        int cus;
        int32_t rc = workspace(aligned_bytes(sizeof(T) * rows_x) + aligned_bytes(sizeof(T) * rows_y) + 256, s, &ws,
                               &cus);
        if (rc) return rc;
        Carver cv(ws);
        T* xn = cv.take<T>(rows_x);
        T* yn = cv.take<T>(rows_y);
        hipError_t e = launch_row_norms<T>(x, rows_x, cols, xn, nullptr, nullptr, nullptr, s);
        if (e == hipSuccess) e = launch_row_norms<T>(y, rows_y, cols, yn, nullptr, nullptr, nullptr, s);
        if (e != hipSuccess) return hip_err(e, "row_norms");
        xa = xn;
        ya = yn;
    }
    int root = do_sqrt ? 1 : 0;
    T pe = T(0), root_exp = T(0);
    if (metric == MLRS_METRIC_MANHATTAN) {
        arm = ARM_MANHATTAN;
        root = 0;
    } else if (metric == MLRS_METRIC_CHEBYSHEV) {
        arm = ARM_CHEBYSHEV;
        root = 0;
    } else if (metric == MLRS_METRIC_MINKOWSKI) {
        // minkowski_dist: pow per feature, root exponent 1/p formed in F
        // (crates/mlrs-kernels/src/distance.rs:201-227)
        arm = ARM_MINKOWSKI_POW;
        pe = (T)p;
        root = 2;
        root_exp = T(1) / pe;
    }
    hipError_t e = launch_pairwise_tile<T>(x, rows_x, y, rows_y, cols, arm, xa, ya, out, rows_y, root, s, pe, 0,
                                           root_exp);
    if (e != hipSuccess) return hip_err(e, "pairwise_tile");
    return MLRS_OK;
}
}  // extern "C++"

int32_t mlrs_pairwise_distance_f32(const float* x, int64_t x_len, int64_t rows_x, int64_t cols, const float* y,
                                   int64_t y_len, int64_t rows_y, int64_t cols_y, int32_t metric, int32_t do_sqrt,
                                   double p, float* out, int64_t out_len, void* stream) {
    return pairwise_impl<float>(x, x_len, rows_x, cols, y, y_len, rows_y, cols_y, metric, do_sqrt, p, out, out_len,
                                stream);
}

int32_t mlrs_pairwise_distance_f64(const double* x, int64_t x_len, int64_t rows_x, int64_t cols, const double* y,
                                   int64_t y_len, int64_t rows_y, int64_t cols_y, int32_t metric, int32_t do_sqrt,
                                   double p, double* out, int64_t out_len, void* stream) {
    return pairwise_impl<double>(x, x_len, rows_x, cols, y, y_len, rows_y, cols_y, metric, do_sqrt, p, out, out_len,
                                 stream);
}

extern "C++" {
template <typename T>
static int32_t sqnorms_impl(const T* x, int64_t x_len, int64_t n, int64_t d, T* out, int64_t out_len,
                            void* stream) {
    CallGuard cg;
    if (!geom_ok(n, d, x_len)) return shape_err("x", n, d, x_len);
    if (out_len != n) return shape_err("out", n, 1, out_len);
    if (n == 0) return MLRS_OK;
    if (!x || !out) return set_err(MLRS_ERR_NULL_POINTER, "x", 0, 0, 0, 0, "null pointer");
    hipError_t e = launch_row_norms<T>(x, n, d, out, nullptr, nullptr, nullptr, (hipStream_t)stream);
    if (e != hipSuccess) return hip_err(e, "row_norms");
    return MLRS_OK;
}
}  // extern "C++"

int32_t mlrs_row_sqnorms_f32(const float* x, int64_t x_len, int64_t n, int64_t n_features, float* out,
                             int64_t out_len, void* stream) {
    return sqnorms_impl<float>(x, x_len, n, n_features, out, out_len, stream);
}

int32_t mlrs_row_sqnorms_f64(const double* x, int64_t x_len, int64_t n, int64_t n_features, double* out,
                             int64_t out_len, void* stream) {
    return sqnorms_impl<double>(x, x_len, n, n_features, out, out_len, stream);
}

// ---------------------------------------------------------------------------
// kNN consumers: regressor gathers and classifier vote
// ---------------------------------------------------------------------------
extern "C++" {
// Read back the lowest flagged row (UINT64_MAX when none) -- a synchronous
// point, as in the reference, whose host raises right after its gather.
static int32_t read_first_bad(const unsigned long long* dev_word, hipStream_t s, int64_t* row) {
    unsigned long long h = ~0ull;
    note_read_back();
    hipError_t e = hipMemcpyAsync(&h, dev_word, sizeof(h), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_err(e, "first_bad read-back");
    *row = (h == ~0ull) ? -1 : (int64_t)h;
    return MLRS_OK;
}

template <typename T>
static int32_t regress_impl(const T* y, int64_t y_len, int64_t n_train, int64_t n_out, const uint32_t* idx,
                            int64_t idx_len, const T* dist, int64_t dist_len, int64_t nq, int32_t k,
                            int32_t weighted, T* out, int64_t out_len, void* stream) {
    CallGuard cg;
    // knn_regress_gather_weighted / knn_regress_mean_gather's checks
    // (crates/mlrs-backend/src/prims/knn.rs:59-323)
    if (k < 1 || nq < 1 || n_out < 1 || n_train < 1) return shape_err("k", nq, k, idx_len);
    if (!geom_ok(nq, k, idx_len)) return shape_err("idx", nq, k, idx_len);
    const bool general = weighted || n_out != 1;
    if (general && dist_len != idx_len) return shape_err("dist", nq, k, dist_len);
    if (!geom_ok(n_train, n_out, y_len)) return shape_err("y_train", n_train, n_out, y_len);
    if (nq > kU32Max) return shape_err("n_query", nq, 0, kU32Max);
    if (n_train > kU32Max) return shape_err("n_train", n_train, 0, kU32Max);
    if (n_out > kU32Max) return shape_err("n_outputs", n_out, 0, kU32Max);
    if (!geom_ok(nq, n_out, out_len)) return shape_err("out", nq, n_out, out_len);
    if (!y || !idx || !out || (weighted && !dist)) return set_err(MLRS_ERR_NULL_POINTER, "ptr", 0, 0, 0, 0,
                                                                 "a required pointer is NULL");
    hipStream_t s = (hipStream_t)stream;
    char* ws;
    int cus;
    int32_t rc = workspace(256, s, &ws, &cus);
    if (rc) return rc;
    unsigned long long* first_bad = reinterpret_cast<unsigned long long*>(ws);
    hipError_t e = launch_first_bad_reset(first_bad, s);
    if (e == hipSuccess) e = launch_knn_regress<T>(y, n_train, n_out, idx, dist, nq, k, weighted, out, first_bad, s);
    if (e != hipSuccess) return hip_err(e, "knn_regress");
    int64_t row;
    rc = read_first_bad(first_bad, s, &row);
    if (rc) return rc;
    if (row >= 0) return shape_err("knn.train_idx", row, k, n_train);
    return ok();
}

template <typename T>
static int32_t classify_impl(const int32_t* y_class, int64_t n_train, int32_t n_classes, const uint32_t* idx,
                             int64_t idx_len, const T* dist, int64_t dist_len, int64_t nq, int32_t k,
                             int32_t weighted, T* proba, int64_t proba_len, int32_t* labels, int64_t labels_len,
                             void* stream) {
    CallGuard cg;
    if (k < 1 || nq < 1 || n_train < 1) return shape_err("k", nq, k, idx_len);
    if (!geom_ok(nq, k, idx_len)) return shape_err("idx", nq, k, idx_len);
    if (weighted && dist_len != idx_len) return shape_err("dist", nq, k, dist_len);
    if (n_classes < 1) return shape_err("n_classes", n_classes, 1, 0);
    if (!geom_ok(nq, n_classes, proba_len)) return shape_err("proba", nq, n_classes, proba_len);
    if (labels_len != nq) return shape_err("labels", nq, 1, labels_len);
    if (!y_class || !idx || !proba || !labels || (weighted && !dist))
        return set_err(MLRS_ERR_NULL_POINTER, "ptr", 0, 0, 0, 0, "a required pointer is NULL");
    hipStream_t s = (hipStream_t)stream;
    // f64 class sums for a chunk of queries (<= 64 MB) + per-row error records
    const int64_t chunk = std::max<int64_t>(256, std::min<int64_t>(nq, ((int64_t)64 << 20) / (8 * (int64_t)n_classes)));
    const size_t bytes = aligned_bytes(sizeof(double) * (size_t)chunk * n_classes) +
                         aligned_bytes(sizeof(int64_t) * 3 * (size_t)nq) + 512;
    char* ws;
    int cus;
    int32_t rc = workspace(bytes, s, &ws, &cus);
    if (rc) return rc;
    Carver cv(ws);
    unsigned long long* first_bad = cv.take<unsigned long long>(1);
    double* acc = cv.take<double>((size_t)chunk * n_classes);
    int64_t* err = cv.take<int64_t>(3 * (size_t)nq);
    hipError_t e = launch_first_bad_reset(first_bad, s);
    for (int64_t q0 = 0; e == hipSuccess && q0 < nq; q0 += chunk)
        e = launch_knn_classify<T>(y_class, n_train, n_classes, idx, dist, q0, std::min(chunk, nq - q0), nq, k,
                                   weighted, proba, labels, acc, err, first_bad, s);
    if (e != hipSuccess) return hip_err(e, "knn_classify");
    int64_t row;
    rc = read_first_bad(first_bad, s, &row);
    if (rc) return rc;
    if (row >= 0) {
        int64_t rec[3] = {0, 0, 0};
        note_read_back();
        e = hipMemcpy(rec, err + 3 * row, sizeof(rec), hipMemcpyDeviceToHost);
        if (e != hipSuccess) return hip_err(e, "knn_classify error read-back");
        // classifier.rs:850-875: the first bad (query, neighbour) in row order
        if (rec[0] == 1) return shape_err("knn.train_idx", rec[1], 1, n_train);
        return shape_err("knn.class_id", std::max<int64_t>(rec[1], 0), 1, n_classes);
    }
    return ok();
}
}  // extern "C++"

int32_t mlrs_knn_regress_f32(const float* y_train, int64_t y_len, int64_t n_train, int64_t n_outputs,
                             const uint32_t* idx, int64_t idx_len, const float* dist, int64_t dist_len,
                             int64_t n_query, int32_t k, int32_t weighted, float* out, int64_t out_len,
                             void* stream) {
    return regress_impl<float>(y_train, y_len, n_train, n_outputs, idx, idx_len, dist, dist_len, n_query, k,
                               weighted, out, out_len, stream);
}
int32_t mlrs_knn_regress_f64(const double* y_train, int64_t y_len, int64_t n_train, int64_t n_outputs,
                             const uint32_t* idx, int64_t idx_len, const double* dist, int64_t dist_len,
                             int64_t n_query, int32_t k, int32_t weighted, double* out, int64_t out_len,
                             void* stream) {
    return regress_impl<double>(y_train, y_len, n_train, n_outputs, idx, idx_len, dist, dist_len, n_query, k,
                                weighted, out, out_len, stream);
}
int32_t mlrs_knn_classify_f32(const int32_t* y_class, int64_t n_train, int32_t n_classes, const uint32_t* idx,
                              int64_t idx_len, const float* dist, int64_t dist_len, int64_t n_query, int32_t k,
                              int32_t weighted, float* proba, int64_t proba_len, int32_t* labels,
                              int64_t labels_len, void* stream) {
    return classify_impl<float>(y_class, n_train, n_classes, idx, idx_len, dist, dist_len, n_query, k, weighted,
                                proba, proba_len, labels, labels_len, stream);
}
int32_t mlrs_knn_classify_f64(const int32_t* y_class, int64_t n_train, int32_t n_classes, const uint32_t* idx,
                              int64_t idx_len, const double* dist, int64_t dist_len, int64_t n_query, int32_t k,
                              int32_t weighted, double* proba, int64_t proba_len, int32_t* labels,
                              int64_t labels_len, void* stream) {
    return classify_impl<double>(y_class, n_train, n_classes, idx, idx_len, dist, dist_len, n_query, k, weighted,
                                 proba, proba_len, labels, labels_len, stream);
}

// ---------------------------------------------------------------------------
// radius_neighbors
// ---------------------------------------------------------------------------
// The count pass's products -- the in-row strip prefix, the row totals, the
// row offsets and the match total -- are kept per device together with the
// arguments of the call that made them, until a call fills from them.  A call
// with the same arguments (the usual count-only call, then the call with
// buffers of the returned size) starts from them instead of counting again.  The queries are staged afresh
// in every call, and the fill pass checks each (strip, row) against its kept
// count, so changed data is caught: on a mismatch the plan is dropped and the
// call counts and fills again.
extern "C++" {
struct RadiusPlan {
    bool valid = false;
    const void* xq = nullptr;
    const void* xt = nullptr;
    int64_t nq = 0, nt = 0, d = 0;
    int32_t metric = -1;
    double p = 0.0, radius = 0.0;
    int elem = 0;
    void* stream = nullptr;
    int nstrips = 0;
    int64_t strip_len = 0;
    bool gram = false;
    unsigned long long total = 0;
    char* base = nullptr;
    size_t cap = 0;
    bool pooled = false;  // base came from hipMallocAsync
};
RadiusPlan g_rplan[kMaxDevices];

template <typename T>
struct RadiusBufs {
    uint32_t* cnt;
    uint32_t* row_cnt;
    unsigned long long* block_sum;
    unsigned long long* qoff;
    unsigned long long* total;
    unsigned int* mismatch;
    T* qT;
    T* qsq;
    T* qinv;
    T* xsq;
    T* xinv;
    NormStats* stats;
    unsigned int* stage_over;
    T* stage_val;
    int32_t* stage_idx;
};

// The staging area (last, so the other buffers keep their places whatever
// its size) holds stage_cap matches per (strip, row).
template <typename T>
static size_t radius_carve(char* base, int64_t nq, int64_t nt, int64_t d, int nstrips, int64_t stage_cap,
                           RadiusBufs<T>* b) {
    const int RQ = radius_queries_per_wave<T>();
    const int64_t G = (nq + RQ - 1) / RQ;
    Carver cv(base);
    b->cnt = cv.take<uint32_t>((size_t)std::max<int64_t>(1, (int64_t)nstrips * nq));
    b->row_cnt = cv.take<uint32_t>((size_t)nq);
    b->block_sum = cv.take<unsigned long long>((size_t)((nq + 255) / 256 + 1));
    b->qoff = cv.take<unsigned long long>((size_t)nq);
    b->total = cv.take<unsigned long long>(1);
    b->mismatch = cv.take<unsigned int>(1);
    b->qT = cv.take<T>((size_t)(G * RQ * d));
    b->qsq = cv.take<T>((size_t)nq);
    b->qinv = cv.take<T>((size_t)nq);
    b->xsq = cv.take<T>((size_t)std::max<int64_t>(1, nt));
    b->xinv = cv.take<T>((size_t)std::max<int64_t>(1, nt));
    b->stats = cv.take<NormStats>(1);
    b->stage_over = cv.take<unsigned int>(1);
    b->stage_val = nullptr;
    b->stage_idx = nullptr;
    if (stage_cap > 0) {
        b->stage_val = cv.take<T>((size_t)nstrips * (size_t)nq * (size_t)stage_cap);
        b->stage_idx = cv.take<int32_t>((size_t)nstrips * (size_t)nq * (size_t)stage_cap);
    }
    return cv.off + 256;
}

// (The call has run order_after_last_call on `s` through workspace().)
static int32_t radius_plan_memory(RadiusPlan& P, size_t bytes, hipStream_t s) {
    const int dev = (int)(&P - g_rplan);
    if (P.cap >= bytes) {
        g_pool[dev].reuses += 1;
        return MLRS_OK;
    }
    const size_t old_cap = P.cap;
    P.valid = false;
    size_t want = std::max(bytes + bytes / 4, (size_t)16 << 20);
    hipError_t e = buffer_regrow(dev, &P.base, &P.pooled, want, s);
    if (e != hipSuccess) {
        P.cap = 0;
        pool_note_release(dev, old_cap);
        return set_err(MLRS_ERR_ALLOC, "radius", (int64_t)want, 0, 0, (int)e,
                       "device allocation of %zu bytes for the radius scan failed: %s", want, hipGetErrorString(e));
    }
    P.cap = want;
    pool_note_grow(dev, old_cap, want);
    return MLRS_OK;
}

static int32_t read_u64(const unsigned long long* dev, hipStream_t s, unsigned long long* out) {
    note_read_back();
    hipError_t e = hipMemcpyAsync(out, dev, sizeof(*out), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_err(e, "radius read-back");
    return MLRS_OK;
}

template <typename T>
static int32_t radius_impl(const T* xq, int64_t xq_len, int64_t nq, int64_t d, const T* xt, int64_t xt_len,
                           int64_t nt, int64_t d_train, int32_t metric, double p, double radius, uint32_t* counts,
                           int64_t counts_len, T* out_dist, int32_t* out_idx, int64_t capacity, int64_t* total,
                           void* stream) {
    CallGuard cg;
    // validate_radius_query (nearest.rs:755-797) and radius_host_scan's
    // geometry checks (radius_host.rs:150-196)
    if (!(radius >= 0.0))
        return set_err(MLRS_ERR_INVALID_PARAM, "radius", 0, 0, 0, 0,
                       "estimator 'nearest_neighbors': eps = %g is invalid (must be >= 0)", radius);
    if (nq == 0 || d == 0 || !geom_ok(nq, d, xq_len)) return shape_err("xq", nq, d, xq_len);
    if (d != d_train) return dim_err("n_features", d, d_train);
    if (!geom_ok(nt, d_train, xt_len)) return shape_err("y", nt, d_train, xt_len);
    if (nt > kU32Max) return shape_err("rows", nt, 0, kU32Max);
    if (metric < MLRS_METRIC_EUCLIDEAN || metric > MLRS_METRIC_MINKOWSKI)
        return set_err(MLRS_ERR_UNSUPPORTED, "metric", metric, 0, 0, 0, "metric %d is not served", metric);
    if (metric == MLRS_METRIC_MINKOWSKI && !(p >= 1.0))
        return set_err(MLRS_ERR_UNSUPPORTED, "p", 0, 0, 0, 0, "minkowski p must be >= 1");
    if (counts_len != nq) return shape_err("counts", nq, 1, counts_len);
    if (!xq || (nt > 0 && !xt) || !counts || !total || ((out_dist == nullptr) != (out_idx == nullptr)))
        return set_err(MLRS_ERR_NULL_POINTER, "ptr", 0, 0, 0, 0, "a required pointer is NULL");
    if (out_dist && capacity < 0) return shape_err("out", 0, 1, capacity);
    *total = 0;
    hipStream_t s = (hipStream_t)stream;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_err(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return set_err(MLRS_ERR_UNSUPPORTED, "device", dev, 0, 0, 0, "device ordinal %d out of range", dev);
    char* ws;
    int cus;
    int32_t rc = workspace(256, s, &ws, &cus);  // the CU count
    if (rc) return rc;

    // arm: the host scan's lane arithmetic; threshold in the metric's internal
    // units formed in f64 (scan_typed, radius_host.rs:239-271); boundary
    // transform chosen by p as `transform` does (:559-569)
    int arm = ARM_EUCLID_MULADD;
    double thresh = radius, p_tr = 1.0;
    int pint = 0;
    switch (metric) {
    case MLRS_METRIC_EUCLIDEAN: thresh = radius * radius; p_tr = 2.0; break;
    case MLRS_METRIC_COSINE: arm = ARM_COS_HOST; break;
    case MLRS_METRIC_MANHATTAN: arm = ARM_MANHATTAN; break;
    case MLRS_METRIC_CHEBYSHEV: arm = ARM_CHEBYSHEV; break;
    default:
        pint = minkowski_powi(p);
        arm = pint ? ARM_MINKOWSKI_INT : ARM_MINKOWSKI_POW;
        thresh = std::pow(radius, p);
        p_tr = p;
    }

    // The matrix-core screen serves f32 Euclidean and cosine for 16 < d <=
    // 128 when the search is large enough to fill the matrix cores (or when
    // the fused family is forced); the host-scan kernel serves the rest.
    const bool gram_ok = sizeof(T) == 4 && radius_gram_serves(arm, d);
    const bool gram = gram_ok && (g_force_path == MLRS_PATH_FUSED ||
                                  (g_force_path == MLRS_PATH_AUTO && d > 16 &&
                                   (double)nq * (double)nt * (double)d >= 1073741824.0));

    // strips: enough waves (host scan) or workgroups (matrix cores) to fill
    // the chip several times over; strip lengths are multiples of 64 rows
    const int RQ = radius_queries_per_wave<T>();
    const int64_t G = (nq + RQ - 1) / RQ;
    const int64_t chunks = (nt + 63) / 64;
    int64_t want_strips;
    if (gram) {
        // whole resident rounds on every XCD (a workgroup per (query block,
        // strip), radius_gram_wgs_per_cu() of them per CU): at c2 the 26
        // strips of an even split left a fifth round of one or two
        // workgroups per XCD
        const int64_t nqb = (nq + radius_gram_queries_per_block() - 1) / radius_gram_queries_per_block();
        const int64_t old = ((int64_t)cus * 8 + nqb - 1) / std::max<int64_t>(1, nqb);
        want_strips = pick_strips_xcd(nqb, nt, std::max<int64_t>(1, (int64_t)cus / 8 * radius_gram_wgs_per_cu()),
                                      64, (int)std::min<int64_t>(2 * old, 65535));
    } else {
        want_strips = ((int64_t)cus * 16 + G - 1) / G;
    }
    want_strips = std::max<int64_t>(1, std::min<int64_t>(want_strips, std::max<int64_t>(1, chunks)));
    int64_t strip_len = std::max<int64_t>(64, ((chunks + want_strips - 1) / want_strips) * 64);
    if (gram) strip_len = std::max<int64_t>(strip_len, ((nt + 65534) / 65535 + 63) / 64 * 64);  // grid.y limit
    const int nstrips = nt > 0 ? (int)((nt + strip_len - 1) / strip_len) : 0;

    RadiusPlan& P = g_rplan[dev];
    const int elem = (int)sizeof(T);
    const bool same = P.valid && P.xq == xq && P.xt == xt && P.nq == nq && P.nt == nt && P.d == d &&
                      P.metric == metric && P.p == p && P.radius == radius && P.elem == elem &&
                      P.stream == stream && P.nstrips == nstrips && P.strip_len == strip_len && P.gram == gram;
    // A call that brings its output buffers and finds no kept plan counts
    // with the staged pass on the matrix-core path: each (strip, row)'s first
    // stage_cap matches are kept, so when every strip fits and the buffers
    // are large enough the matches are copied into place and no fill pass
    // runs.  Staging holds at most 1,024 matches per (strip, row) and 2 GiB
    // in all; below 64 per (strip, row) it is not used.
    int64_t stage_cap = 0;
    if (gram && out_dist && !same && nstrips > 0) {
        const double per = (double)(2ull << 30) / ((double)nstrips * (double)nq * (double)(sizeof(T) + 4));
        stage_cap = per >= 1024.0 ? 1024 : ((int64_t)per / 16) * 16;
        if (stage_cap < 64) stage_cap = 0;
    }
    RadiusBufs<T> B;
    const size_t need = radius_carve<T>(nullptr, nq, nt, d, nstrips, stage_cap, &B);
    if (!same) {
        P.valid = false;
        rc = radius_plan_memory(P, need, s);
        if (rc) return rc;
    }
    (void)radius_carve<T>(P.base, nq, nt, d, nstrips, stage_cap, &B);

    RadiusArgs<T> a{};
    a.qT = B.qT;
    a.x = xt;
    a.qinv = B.qinv;
    a.xinv = B.xinv;
    a.nq = nq;
    a.nt = nt;
    a.d = d;
    a.strip_len = strip_len;
    a.nstrips = nstrips;
    a.th = (T)thresh;
    a.pexp = (T)p;
    a.pint = pint;
    const int transform = p_tr == 1.0 ? 0 : (p_tr == 2.0 ? 1 : 2);
    a.cnt = B.cnt;
    a.row_cnt = B.row_cnt;
    a.qoff = B.qoff;
    a.out_dist = out_dist;
    a.out_idx = out_idx;
    a.capacity = capacity;
    a.mismatch = B.mismatch;
    a.q = xq;
    a.qsq = B.qsq;
    a.xsq = B.xsq;
    a.stats = B.stats;
    // the fused kNN screen's bounds (u = 2^-23): 8(d+4)u (||q||^2 + max ||x||^2)
    // plus a subnormal floor (Euclidean), (8d+32)u (cosine)
    const double u23 = std::ldexp(1.0, -23);
    a.eps_rel = (arm == ARM_COS_HOST) ? 0.0 : 8.0 * (double)(d + 4) * u23;
    a.eps_abs = (arm == ARM_COS_HOST) ? (8.0 * (double)d + 32.0) * u23 : (double)(d + 4) * std::ldexp(1.0, -120);
    a.stage_val = B.stage_val;
    a.stage_idx = B.stage_idx;
    a.stage_cap = stage_cap;
    a.stage_over = B.stage_over;

    e = gram ? hipSuccess : launch_radius_stage<T>(xq, nq, d, B.qT, s);
    if (e == hipSuccess && (arm == ARM_COS_HOST || gram)) {
        // row_inv_norm_host (knn_host.rs:382-397); the squared norms and the
        // largest index norm feed the matrix-core screen
        e = launch_row_norms<T>(xq, nq, d, B.qsq, B.qinv, nullptr, nullptr, s);
        if (e == hipSuccess && nt > 0)
            e = launch_row_norms<T>(xt, nt, d, B.xsq, B.xinv, nullptr, gram ? B.stats : nullptr, s);
    }
    if (e != hipSuccess) return hip_err(e, "radius staging");
    auto scan = [&](int mode) -> hipError_t {
        const bool fill_pass = mode == RADIUS_FILL;
        if constexpr (std::is_same<T, float>::value) {
            if (gram) {
                if (fill_pass) {
                    KernelTimer kt(s, "radius_gram_fill");
                    return launch_radius_gram(a, arm, RADIUS_FILL, s);
                }
                if (mode == RADIUS_STAGE) {
                    KernelTimer kt(s, "radius_gram_stage");
                    return launch_radius_gram(a, arm, RADIUS_STAGE, s);
                }
                return launch_radius_gram(a, arm, RADIUS_COUNT, s);
            }
        }
        if (fill_pass) {
            KernelTimer kt(s, "radius_scan_fill");
            return launch_radius_scan<T>(a, arm, true, s);
        }
        return launch_radius_scan<T>(a, arm, false, s);
    };

    auto count = [&](bool staged) -> int32_t {
        hipError_t e2 = launch_fill_u32(B.cnt, (int64_t)nstrips * nq, 0u, s);
        if (e2 == hipSuccess && staged) e2 = launch_fill_u32(B.stage_over, 1, 0u, s);
        if (e2 == hipSuccess) e2 = scan(staged ? RADIUS_STAGE : RADIUS_COUNT);
        if (e2 == hipSuccess) e2 = launch_radius_offsets(B.cnt, nq, nstrips, B.row_cnt, B.block_sum, B.qoff, B.total, s);
        if (e2 != hipSuccess) return hip_err(e2, "radius count");
        int32_t r2 = read_u64(B.total, s, &P.total);
        if (r2) return r2;
        P.valid = true;
        P.xq = xq;
        P.xt = xt;
        P.nq = nq;
        P.nt = nt;
        P.d = d;
        P.metric = metric;
        P.p = p;
        P.radius = radius;
        P.elem = elem;
        P.stream = stream;
        P.nstrips = nstrips;
        P.strip_len = strip_len;
        P.gram = gram;
        return MLRS_OK;
    };
    auto fill = [&](unsigned int* bad) -> int32_t {
        hipError_t e2 = launch_fill_u32(B.mismatch, 1, 0u, s);
        if (e2 == hipSuccess) e2 = scan(RADIUS_FILL);
        if (e2 != hipSuccess) return hip_err(e2, "radius fill");
        note_read_back();
        e2 = hipMemcpyAsync(bad, B.mismatch, sizeof(*bad), hipMemcpyDeviceToHost, s);
        if (e2 == hipSuccess) e2 = hipStreamSynchronize(s);
        if (e2 != hipSuccess) return hip_err(e2, "radius read-back");
        if (*bad) return MLRS_OK;
        e2 = launch_radius_transform<T>(out_dist, (int64_t)P.total, transform, (T)(1.0 / p_tr), s);
        if (e2 != hipSuccess) return hip_err(e2, "radius transform");
        return MLRS_OK;
    };
    auto finish_counts = [&]() -> int32_t {
        hipError_t e2 = hipMemcpyAsync(counts, B.row_cnt, sizeof(uint32_t) * (size_t)nq, hipMemcpyDeviceToDevice, s);
        if (e2 == hipSuccess) e2 = hipStreamSynchronize(s);
        if (e2 != hipSuccess) return hip_err(e2, "radius counts");
        *total = (int64_t)P.total;
        return MLRS_OK;
    };

    bool counted_now = false;
    if (!same) {
        rc = count(stage_cap > 0);
        if (rc) return rc;
        counted_now = true;
        if (stage_cap > 0 && P.total <= (unsigned long long)capacity) {
            unsigned int over = 1;
            note_read_back();
            hipError_t e2 = hipMemcpyAsync(&over, B.stage_over, sizeof(over), hipMemcpyDeviceToHost, s);
            if (e2 == hipSuccess) e2 = hipStreamSynchronize(s);
            if (e2 != hipSuccess) return hip_err(e2, "radius read-back");
            if (!over) {
                if constexpr (std::is_same<T, float>::value) {
                    e2 = launch_radius_unstage(a, s);
                    if (e2 == hipSuccess)
                        e2 = launch_radius_transform<T>(out_dist, (int64_t)P.total, transform, (T)(1.0 / p_tr), s);
                    if (e2 != hipSuccess) return hip_err(e2, "radius unstage");
                }
                P.valid = false;
                return finish_counts();
            }
        }
    }
    for (;;) {
        if (!out_dist || P.total > (unsigned long long)capacity) {
            rc = finish_counts();
            if (rc) return rc;
            if (!out_dist) return ok();
            return shape_err("out", (int64_t)P.total, 1, capacity);
        }
        unsigned int bad = 0;
        rc = fill(&bad);
        if (rc) return rc;
        if (!bad) {
            // the kept counts serve the call right after the one that made
            // them, not every later call with the same arguments
            P.valid = false;
            return finish_counts();
        }
        P.valid = false;
        if (counted_now)
            return set_err(MLRS_ERR_HIP, "radius", 0, 0, 0, 0,
                           "radius fill pass disagrees with its own count pass (inputs modified during the call)");
        rc = count(false);
        if (rc) return rc;
        counted_now = true;
    }
}
}  // extern "C++"

int32_t mlrs_radius_neighbors_f32(const float* xq, int64_t xq_len, int64_t n_query, int64_t n_features,
                                  const float* x_train, int64_t x_train_len, int64_t n_train, int64_t train_features,
                                  int32_t metric, double p, double radius, uint32_t* counts, int64_t counts_len,
                                  float* out_dist, int32_t* out_idx, int64_t capacity, int64_t* total,
                                  void* stream) {
    return radius_impl<float>(xq, xq_len, n_query, n_features, x_train, x_train_len, n_train, train_features, metric,
                              p, radius, counts, counts_len, out_dist, out_idx, capacity, total, stream);
}

int32_t mlrs_radius_neighbors_f64(const double* xq, int64_t xq_len, int64_t n_query, int64_t n_features,
                                  const double* x_train, int64_t x_train_len, int64_t n_train,
                                  int64_t train_features, int32_t metric, double p, double radius, uint32_t* counts,
                                  int64_t counts_len, double* out_dist, int32_t* out_idx, int64_t capacity,
                                  int64_t* total, void* stream) {
    return radius_impl<double>(xq, xq_len, n_query, n_features, x_train, x_train_len, n_train, train_features,
                               metric, p, radius, counts, counts_len, out_dist, out_idx, capacity, total, stream);
}

// ---------------------------------------------------------------------------
// X-vs-X graphs: the UMAP kNN graph and the HDBSCAN core distances
// ---------------------------------------------------------------------------
extern "C++" {
// A second cached device buffer for operands and lists that must survive the
// search, whose own workspace() calls may move the main arena.
Arena g_aux[kMaxDevices];

static int32_t aux_workspace(size_t bytes, hipStream_t s, char** out) {
    int dev = 0;
    int32_t rc = current_device(&dev);
    if (rc) return rc;
    rc = order_after_last_call(dev, s);
    if (rc) return rc;
    hipError_t e;
    Arena& A = g_aux[dev];
    if (A.cap < bytes) {
        const size_t old_cap = A.cap;
        size_t want = std::max(bytes + bytes / 4, (size_t)16 << 20);
        e = buffer_regrow(dev, &A.base, &A.pooled, want, s);
        if (e != hipSuccess) {
            A.cap = 0;
            pool_note_release(dev, old_cap);
            return set_err(MLRS_ERR_ALLOC, "workspace", (int64_t)want, 0, 0, (int)e,
                           "device allocation of %zu bytes failed: %s", want, hipGetErrorString(e));
        }
        A.cap = want;
        pool_note_grow(dev, old_cap, want);
    } else {
        g_pool[dev].reuses += 1;
    }
    *out = A.base;
    return MLRS_OK;
}

// Pinned host memory for the k-means fit's read-backs and uploads (grown on
// demand and kept; used under the call lock).  Copies to and from it are DMA
// transfers queued behind the kernels, where pageable memory would be staged
// by the runtime on the host's time.  Every fit waits for its own copies
// before it returns, so growing may free the old block.
char* g_pinned = nullptr;
size_t g_pinned_cap = 0;

static int32_t pinned_staging(size_t bytes, char** out) {
    if (g_pinned_cap < bytes) {
        if (g_pinned) (void)hipHostFree(g_pinned);
        g_pinned = nullptr;
        g_pinned_cap = 0;
        const size_t want = std::max(bytes + bytes / 4, (size_t)1 << 20);
        void* p = nullptr;
        hipError_t e = hipHostMalloc(&p, want, hipHostMallocDefault);
        if (e != hipSuccess)
            return set_err(MLRS_ERR_ALLOC, "pinned", (int64_t)want, 0, 0, (int)e,
                           "pinned host allocation of %zu bytes failed: %s", want, hipGetErrorString(e));
        g_pinned = static_cast<char*>(p);
        g_pinned_cap = want;
    }
    *out = g_pinned;
    return MLRS_OK;
}

// The f64 search under an explicit arm: the low-d ALU kernel for Euclidean
// arms ranked by the aggregate (d <= 16, k <= 32), the Gram-MFMA kernel where
// it serves the arm and shape, else exact tiles + selection.
static int32_t search_f64(const double* xq, int64_t nq, const double* xt, int64_t nt, int64_t d, int k, int arm,
                          int mode, double p, double* ov, uint32_t* oi, hipStream_t s) {
    const bool lowd_ok = (arm == ARM_EUCLID_FMA || arm == ARM_EUCLID_MULADD || arm == ARM_COS_FOLD) &&
                         mode != EMIT_ROOT_RANKED && d <= lowd_max_d() && k <= lowd_max_k();
    const bool gram_ok = arm <= ARM_COS_HOST && d <= gram_f64_max_d() && k <= gram_f64_max_k();
    int path = pick_path(lowd_ok, gram_ok);
    if (path == MLRS_PATH_AUTO)
        path = lowd_ok ? MLRS_PATH_LOWD : (gram_ok && !small_search(nq, nt, d)) ? MLRS_PATH_FUSED : MLRS_PATH_GENERIC;
    if (path == MLRS_PATH_LOWD) return knn_lowd<double>(xq, nq, xt, nt, d, k, arm, mode, ov, oi, s);
    if (path == MLRS_PATH_FUSED) return knn_gram64(xq, nq, xt, nt, d, k, arm, mode, ov, oi, s);
    return knn_generic<double>(xq, nq, xt, nt, d, k, arm, mode, ov, oi, s, p);
}

// knn_graph's validate_geometry (crates/mlrs-backend/src/prims/knn_graph.rs:475-539).
static int32_t validate_graph(const void* x, int64_t x_len, int64_t n, int64_t d, int64_t k, int32_t metric,
                              double p, bool include_self) {
    if (!geom_ok(n, d, x_len) || d < 1) return shape_err("x", n, d, x_len);
    const int64_t max_k = include_self ? n : std::max<int64_t>(0, n - 1);
    if (k < 1 || k > max_k) return shape_err("k", 1, k, max_k);
    if (metric < MLRS_METRIC_EUCLIDEAN || metric > MLRS_METRIC_MINKOWSKI)
        return set_err(MLRS_ERR_UNSUPPORTED, "metric", metric, 0, 0, 0, "metric %d is not served", metric);
    if (metric == MLRS_METRIC_MINKOWSKI && !(p >= 1.0)) return shape_err("p", 1, 0, 1);
    if (n > kU32Max) return shape_err("x", n, 0, kU32Max);
    if (d > kU32Max) return shape_err("x", d, 0, kU32Max);
    if (k + 1 > kU32Max) return shape_err("k", k + 1, 0, kU32Max);
    if (!x) return set_err(MLRS_ERR_NULL_POINTER, "x", 0, 0, 0, 0, "null pointer");
    return MLRS_OK;
}

// The host scans' per-metric arithmetic as engine arms (umap_host_knn.rs:318-411):
// Euclidean and cosine accumulate diff*diff with separate rounding (cosine over
// normalised rows), Minkowski always through pow.  The scans push the final
// distance, `(ops.fin)(a)` (:494), into a list ordered by (distance, index)
// (KNearest::push, :171-198): Euclidean and Minkowski are ranked by their root
// (EMIT_ROOT_RANKED), so aggregates that root to the same value are ordered
// by index; the other finals (identity, the exact halving of cosine) keep the
// aggregate's order.
static void graph_arm(int32_t metric, int* arm, int* mode) {
    switch (metric) {
    case MLRS_METRIC_EUCLIDEAN: *arm = ARM_EUCLID_MULADD; *mode = EMIT_ROOT_RANKED; break;
    case MLRS_METRIC_COSINE: *arm = ARM_EUCLID_MULADD; *mode = EMIT_IDENTITY; break;
    case MLRS_METRIC_MANHATTAN: *arm = ARM_MANHATTAN; *mode = EMIT_IDENTITY; break;
    case MLRS_METRIC_CHEBYSHEV: *arm = ARM_CHEBYSHEV; *mode = EMIT_IDENTITY; break;
    default: *arm = ARM_MINKOWSKI_POW; *mode = EMIT_ROOT_RANKED; break;
    }
}

// Operand in f64 (widened / normalised as the host scan sees it) plus the
// (n x kk) lists, carved from the auxiliary buffer.
template <typename TIn>
static int32_t graph_search(const TIn* x, int64_t n, int64_t d, int kk, int32_t metric, double p, hipStream_t s,
                            double** val, uint32_t** idx) {
    const bool widen = sizeof(TIn) == 4;
    const bool cos = metric == MLRS_METRIC_COSINE;
    size_t bytes = aligned_bytes(sizeof(double) * (size_t)n * kk) + aligned_bytes(sizeof(uint32_t) * (size_t)n * kk) +
                   2 * aligned_bytes(sizeof(double) * (size_t)n * d) + 2 * aligned_bytes(sizeof(double) * (size_t)n) +
                   1024;
    char* aux;
    int32_t rc = aux_workspace(bytes, s, &aux);
    if (rc) return rc;
    Carver cv(aux);
    *val = cv.take<double>((size_t)n * kk);
    *idx = cv.take<uint32_t>((size_t)n * kk);
    const double* xd = reinterpret_cast<const double*>(x);
    hipError_t e = hipSuccess;
    if (widen) {
        double* w = cv.take<double>((size_t)n * d);
        e = launch_widen(reinterpret_cast<const float*>(x), n * d, w, s);
        xd = w;
    }
    if (e == hipSuccess && cos) {
        double* sq = cv.take<double>((size_t)n);
        double* inv = cv.take<double>((size_t)n);
        double* xn = cv.take<double>((size_t)n * d);
        e = launch_row_norms<double>(xd, n, d, sq, inv, nullptr, nullptr, s);
        if (e == hipSuccess) e = launch_normalize_rows(xd, n, d, inv, xn, s);
        xd = xn;
    }
    if (e != hipSuccess) return hip_err(e, "graph operand");
    int arm, mode;
    graph_arm(metric, &arm, &mode);
    return search_f64(xd, n, xd, n, d, kk, arm, mode, p, *val, *idx, s);
}

template <typename TIn>
static int32_t knn_graph_impl(const TIn* x, int64_t x_len, int64_t n, int64_t d, int64_t k, int32_t metric,
                              double p, int32_t include_self, uint32_t* out_idx, double* out_dist, int64_t out_len,
                              void* stream) {
    CallGuard cg;
    int32_t rc = validate_graph(x, x_len, n, d, k, metric, p, include_self != 0);
    if (rc) return rc;
    if (!geom_ok(n, k, out_len)) return shape_err("out", n, k, out_len);
    if (!out_idx || !out_dist) return set_err(MLRS_ERR_NULL_POINTER, "out", 0, 0, 0, 0, "null pointer");
    const int64_t kk = include_self ? k : k + 1;
    if (kk > INT32_MAX) return shape_err("k", 1, k, INT32_MAX);
    hipStream_t s = (hipStream_t)stream;
    double* val;
    uint32_t* idx;
    rc = graph_search<TIn>(x, n, d, (int)kk, metric, p, s, &val, &idx);
    if (rc) return rc;
    hipError_t e = launch_graph_finish(val, idx, n, (int)kk, (int)k, include_self ? 0 : 1,
                                       metric == MLRS_METRIC_COSINE ? 1 : 0, out_dist, out_idx, s);
    if (e != hipSuccess) return hip_err(e, "graph finish");
    return ok();
}

template <typename TIn>
static int32_t core_impl(const TIn* x, int64_t x_len, int64_t n, int64_t d, int32_t metric, double p,
                         int64_t min_samples, double* out, int64_t out_len, void* stream) {
    CallGuard cg;
    // k = min_samples clamped to [1, n] (hdbscan.rs:1508-1510)
    const int64_t k = std::max<int64_t>(1, std::min<int64_t>(min_samples, n));
    int32_t rc = validate_graph(x, x_len, n, d, n >= 1 ? k : 1, metric, p, true);
    if (rc) return rc;
    if (metric == MLRS_METRIC_COSINE)
        return set_err(MLRS_ERR_UNSUPPORTED, "metric", metric, 0, 0, 0,
                       "cosine core distances come from the dense cosine matrix, not a kNN scan");
    if (out_len != n) return shape_err("out", n, 1, out_len);
    if (!out) return set_err(MLRS_ERR_NULL_POINTER, "out", 0, 0, 0, 0, "null pointer");
    if (k > INT32_MAX) return shape_err("min_samples", 1, k, INT32_MAX);
    hipStream_t s = (hipStream_t)stream;
    double* val;
    uint32_t* idx;
    rc = graph_search<TIn>(x, n, d, (int)k, metric, p, s, &val, &idx);
    if (rc) return rc;
    hipError_t e = launch_core_column(val, n, (int)k, out, s);
    if (e != hipSuccess) return hip_err(e, "core column");
    return ok();
}
}  // extern "C++"

int32_t mlrs_knn_graph_f32(const float* x, int64_t x_len, int64_t n, int64_t n_features, int64_t k, int32_t metric,
                           double p, int32_t include_self, uint32_t* out_idx, double* out_dist, int64_t out_len,
                           void* stream) {
    return knn_graph_impl<float>(x, x_len, n, n_features, k, metric, p, include_self, out_idx, out_dist, out_len,
                                 stream);
}
int32_t mlrs_knn_graph_f64(const double* x, int64_t x_len, int64_t n, int64_t n_features, int64_t k,
                           int32_t metric, double p, int32_t include_self, uint32_t* out_idx, double* out_dist,
                           int64_t out_len, void* stream) {
    return knn_graph_impl<double>(x, x_len, n, n_features, k, metric, p, include_self, out_idx, out_dist, out_len,
                                  stream);
}
int32_t mlrs_hdbscan_core_distances_f32(const float* x, int64_t x_len, int64_t n, int64_t n_features,
                                        int32_t metric, double p, int64_t min_samples, double* out, int64_t out_len,
                                        void* stream) {
    return core_impl<float>(x, x_len, n, n_features, metric, p, min_samples, out, out_len, stream);
}
int32_t mlrs_hdbscan_core_distances_f64(const double* x, int64_t x_len, int64_t n, int64_t n_features,
                                        int32_t metric, double p, int64_t min_samples, double* out, int64_t out_len,
                                        void* stream) {
    return core_impl<double>(x, x_len, n, n_features, metric, p, min_samples, out, out_len, stream);
}

// ---------------------------------------------------------------------------
// k-means fit: restarts, initialisation and the Lloyd loop around the fused
// assignment (KMeans::fit, crates/mlrs-algos/src/cluster/kmeans.rs:1353-1580;
// single_run :929-1155)
// ---------------------------------------------------------------------------
extern "C++" {
static int32_t km_assign(const float* x, int64_t n, const float* c, int64_t k, int64_t d, uint32_t* labels,
                         float* dist, hipStream_t s, const float* xsq = nullptr) {
    if (d <= gram_f32_max_d() && pick_path(false, true) != MLRS_PATH_GENERIC)
        return knn_gram32(x, n, c, k, d, 1, ARM_EUCLID_MULADD, EMIT_KMEANS, dist, labels, s, xsq);
    return kmeans_generic<float>(x, n, c, k, d, labels, dist, s);
}
static int32_t km_assign(const double* x, int64_t n, const double* c, int64_t k, int64_t d, uint32_t* labels,
                         double* dist, hipStream_t s, const double* xsq = nullptr) {
    if (d <= gram_f64_max_d() && pick_path(false, true) != MLRS_PATH_GENERIC)
        return knn_gram64(x, n, c, k, d, 1, ARM_EUCLID_MULADD, EMIT_KMEANS, dist, labels, s, xsq);
    return kmeans_generic<double>(x, n, c, k, d, labels, dist, s);
}

// The reference's row-block layout: nb = clamp(ceil(n/256), 1, cap), rpb =
// ceil(n/nb), nb = ceil(n/rpb).
static void km_layout(int64_t n, int64_t cap, int64_t* nb, int64_t* rpb) {
    int64_t b = std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, cap));
    *rpb = (n + b - 1) / b;
    *nb = (n + *rpb - 1) / *rpb;
}

// SplitMix64 (crates/mlrs-backend/src/prims/rng.rs:58-110).
struct KmRng {
    uint64_t state;
    uint64_t next_u64() {
        state += 0x9E3779B97F4A7C15ull;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double next_f64() { return (double)(next_u64() >> 11) / 9007199254740992.0; }
    uint64_t next_below(uint64_t bound) {
        if (bound <= 1) return 0;
        const uint64_t zone = UINT64_MAX - (UINT64_MAX % bound);
        for (;;) {
            const uint64_t v = next_u64();
            if (v < zone) return v % bound;
        }
    }
};

template <typename T>
static int32_t km_d2h(void* dst, const void* src, size_t bytes, hipStream_t s) {
    note_read_back();
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e == hipSuccess ? MLRS_OK : hip_err(e, "kmeans read-back");
}

// The top m rows by (distance desc, index asc) -- the prefix of the
// relocation's ranking (prims/kmeans.rs:1347-1359) -- selected on the device
// from the keys -distance (ascending (key, index) is that order), with their
// labels.  *ranked stays false when a distance is NaN: the reference ranks
// NaN above every number, which the keys cannot express, so the host ranks.
// The selection runs one workgroup per row, so a long array is cut into
// chunks of C keys (padded with +inf): each chunk's m smallest are selected
// in parallel, then the m smallest of those.  The candidates lie chunk by
// chunk, each chunk's equal keys in index order, so candidate order breaks
// ties as the row number does.
template <typename T>
static int32_t km_rank_device(const T* dist, const uint32_t* labels, int64_t n, int64_t m,
                              std::vector<uint32_t>& rows, std::vector<uint32_t>& labs, bool* ranked,
                              hipStream_t s) {
    *ranked = false;
    int64_t C = 8192;
    while (C < 4 * m || C * C < n * m) C <<= 1;
    const int64_t R = (n + C - 1) / C;
    const bool two = R > 1;
    const int64_t padded = two ? R * C : n;
    const int64_t cand = two ? R * m : 0;
    const size_t sel = std::max(select_rows_scratch_bytes(two ? R : 1, (int)m, (int)sizeof(T)),
                                select_rows_scratch_bytes(1, (int)m, (int)sizeof(T)));
    const size_t bytes = aligned_bytes(sizeof(T) * (size_t)padded) + aligned_bytes(sizeof(T) * (size_t)cand) +
                         2 * aligned_bytes(sizeof(uint32_t) * (size_t)cand) + aligned_bytes(sizeof(T) * (size_t)m) +
                         3 * aligned_bytes(sizeof(uint32_t) * (size_t)m) + aligned_bytes(sizeof(uint32_t)) +
                         aligned_bytes(sel) + 256;
    char* ws;
    int cus;
    int32_t rc = workspace(bytes, s, &ws, &cus);
    if (rc) return rc;
    Carver cv(ws);
    T* neg = cv.take<T>((size_t)padded);
    T* v1 = cv.take<T>((size_t)cand);
    uint32_t* i1 = cv.take<uint32_t>((size_t)cand);
    uint32_t* g1 = cv.take<uint32_t>((size_t)cand);
    T* v2 = cv.take<T>((size_t)m);
    uint32_t* i2 = cv.take<uint32_t>((size_t)m);
    uint32_t* orow = cv.take<uint32_t>((size_t)m);
    uint32_t* olab = cv.take<uint32_t>((size_t)m);
    unsigned int* nans = cv.take<unsigned int>(1);
    void* scratch = sel ? static_cast<void*>(cv.take<char>(sel)) : nullptr;
    hipError_t e = launch_km_neg<T>(dist, n, padded, neg, nans, s);
    if (two) {
        if (e == hipSuccess) e = launch_select_rows<T>(neg, R, C, C, (int)m, EMIT_IDENTITY, v1, i1, scratch, s);
        if (e == hipSuccess) e = launch_km_chunk_rows(i1, R, m, C, g1, s);
        if (e == hipSuccess) e = launch_select_rows<T>(v1, 1, cand, cand, (int)m, EMIT_IDENTITY, v2, i2, scratch, s);
        if (e == hipSuccess) e = launch_km_take_u32(g1, cand, i2, m, orow, s);
    } else if (e == hipSuccess) {
        e = launch_select_rows<T>(neg, 1, n, n, (int)m, EMIT_IDENTITY, v2, orow, scratch, s);
    }
    if (e == hipSuccess) e = launch_km_take_u32(labels, n, orow, m, olab, s);
    if (e != hipSuccess) return hip_err(e, "kmeans relocation ranking");
    unsigned int nn = 0;
    rc = km_d2h<T>(&nn, nans, sizeof(nn), s);
    if (rc || nn) return rc;
    rows.resize((size_t)m);
    labs.resize((size_t)m);
    rc = km_d2h<T>(rows.data(), orow, sizeof(uint32_t) * (size_t)m, s);
    if (!rc) rc = km_d2h<T>(labs.data(), olab, sizeof(uint32_t) * (size_t)m, s);
    if (rc) return rc;
    *ranked = true;
    return MLRS_OK;
}

template <typename T>
static int32_t kmeans_fit_impl(const T* x, int64_t x_len, int64_t n, int64_t d, int64_t k, int32_t init_kind,
                               const T* init, int64_t init_len, uint64_t seed, int64_t n_init, int64_t max_iter,
                               double tol, int32_t algorithm, T* out_centers, int64_t centers_len,
                               uint32_t* out_labels, int64_t labels_len, double* out_inertia, int64_t* out_n_iter,
                               void* stream) {
    CallGuard cg;
    if (k < 1 || k > n)
        return set_err(MLRS_ERR_INVALID_PARAM, "k", 1, k, n, 0,
                       "estimator 'kmeans': k = %lld is out of range (must be 1..=%lld = n_samples)", (long long)k,
                       (long long)n);
    if (!geom_ok(n, d, x_len) || d < 1) return shape_err("x", n, d, x_len);
    if (n > kU32Max) return shape_err("n", n, 0, kU32Max);
    if (d > kU32Max) return shape_err("d", d, 0, kU32Max);
    if (init_kind < 0 || init_kind > 2)
        return set_err(MLRS_ERR_UNSUPPORTED, "init", init_kind, 0, 0, 0, "init kind %d is not served", init_kind);
    if (init_kind == 0 && init_len != k * d) return shape_err("init", k, d, init_len);
    if (n_init < 1) return set_err(MLRS_ERR_INVALID_PARAM, "n_init", n_init, 0, 0, 0, "n_init must be >= 1");
    if (max_iter < 0) return set_err(MLRS_ERR_INVALID_PARAM, "max_iter", max_iter, 0, 0, 0, "max_iter must be >= 0");
    if (!(tol >= 0.0)) return set_err(MLRS_ERR_INVALID_PARAM, "tol", 0, 0, 0, 0, "tol must be >= 0");
    if (algorithm != MLRS_KMEANS_LLOYD && algorithm != MLRS_KMEANS_ELKAN)
        return set_err(MLRS_ERR_INVALID_PARAM, "algorithm", algorithm, 0, 0, 0,
                       "algorithm %d is neither lloyd (0) nor elkan (1)", algorithm);
    if (centers_len != k * d) return shape_err("centers", k, d, centers_len);
    if (labels_len != n) return shape_err("labels", n, 1, labels_len);
    if (!x || !out_centers || !out_labels || !out_inertia || !out_n_iter || (init_kind == 0 && !init))
        return set_err(MLRS_ERR_NULL_POINTER, "ptr", 0, 0, 0, 0, "a required pointer is NULL");
    hipStream_t s = (hipStream_t)stream;
    const int64_t kd = k * d;
    const int64_t runs = init_kind == 0 ? 1 : n_init;  // NInit::resolve: an explicit init runs once

    int64_t nb, rpb, nbv, rpbv, nbi, rpbi;
    km_layout(n, std::max<int64_t>(((int64_t)8 << 20) / kd, 64), &nb, &rpb);   // centroid_sums_dev
    km_layout(n, std::max<int64_t>(((int64_t)4 << 20) / d, 64), &nbv, &rpbv);  // feature_mean_var
    km_layout(n, 256, &nbi, &rpbi);                                            // sum_device

    const int64_t nsub = km_sub_blocks(nb, rpb, k);
    size_t bytes = 4 * aligned_bytes(sizeof(uint32_t) * (size_t)n) + 3 * aligned_bytes(sizeof(T) * (size_t)n) +
                   2 * aligned_bytes(sizeof(uint32_t) * (size_t)(nb * k)) +
                   aligned_bytes(sizeof(uint32_t) * (size_t)(nb * nsub * k)) + 2 * aligned_bytes(sizeof(uint32_t) * k) +
                   aligned_bytes(sizeof(T) * (size_t)(nb * kd)) + 3 * aligned_bytes(sizeof(T) * (size_t)kd) +
                   aligned_bytes(sizeof(T) * (size_t)std::max(nbi, nbv * d)) + aligned_bytes(sizeof(T) * d) +
                   aligned_bytes(sizeof(int64_t) * k) + 1024;
    // algorithm = 'elkan': the bound-pruned assignment (launch_km_elkan) for
    // k <= 4096 (its k x k half-distance tables), k > 1 and finite rows: per
    // row an f64 upper bound and a slot of the fused-search list; the k x k
    // tables (sorted rows); and dense buffers for up to prune_chunk rows (1 GB)
    // of one fused search of the rows it cannot settle itself.
    bool prune = algorithm == MLRS_KMEANS_ELKAN && k > 1 && k <= 4096;
    const int64_t prune_chunk =
        std::max<int64_t>(64, std::min<int64_t>(n, ((int64_t)1 << 30) / (d * (int64_t)sizeof(T))));
    const size_t psel = prune ? select_rows_scratch_bytes(k, (int)k, (int)sizeof(double)) : 0;
    if (prune)
        bytes += aligned_bytes(sizeof(double) * (size_t)n) + aligned_bytes(sizeof(uint32_t) * (size_t)n) +
                 2 * aligned_bytes(sizeof(double) * (size_t)(k * k)) + aligned_bytes(sizeof(uint32_t) * (size_t)(k * k)) +
                 2 * aligned_bytes(sizeof(double) * (size_t)k) + aligned_bytes(sizeof(uint32_t)) + aligned_bytes(psel) +
                 aligned_bytes(sizeof(T) * (size_t)(prune_chunk * d)) + 2 * aligned_bytes(sizeof(T) * (size_t)prune_chunk) +
                 aligned_bytes(sizeof(uint32_t) * (size_t)prune_chunk) + 1024;
    char* aux;
    int32_t rc = aux_workspace(bytes, s, &aux);
    if (rc) return rc;
    Carver cv(aux);
    uint32_t* lab[2] = {cv.take<uint32_t>(n), cv.take<uint32_t>(n)};
    uint32_t* perm = cv.take<uint32_t>(n);
    uint32_t* best_lab = cv.take<uint32_t>(n);
    T* dist = cv.take<T>(n);
    T* mind2 = cv.take<T>(n);
    KmScratch<T> w;
    w.pcount = cv.take<uint32_t>(nb * k);
    w.seg = cv.take<uint32_t>(nb * k);
    w.cursor = cv.take<uint32_t>(nb * nsub * k);
    w.counts = cv.take<uint32_t>(k);
    w.starts = cv.take<uint32_t>(k);
    w.perm = perm;
    w.psum = cv.take<T>(nb * kd);
    w.sums = cv.take<T>(kd);
    T* cdev = cv.take<T>(kd);
    T* cnext = cv.take<T>(kd);
    T* parts = cv.take<T>(std::max(nbi, nbv * d));
    T* means_dev = cv.take<T>(d);
    int64_t* idx_dev = cv.take<int64_t>(k);
    unsigned int* changed_dev = reinterpret_cast<unsigned int*>(cv.take<uint32_t>(1));
    // the rows' row_sumsq, which every assignment of this fit reads: computed once
    T* xsq = cv.take<T>(n);
    hipError_t e = launch_row_norms<T>(x, n, d, xsq, nullptr, nullptr, nullptr, s);
    if (e != hipSuccess) return hip_err(e, "kmeans row norms");
    KmPruneConsts pc{};
    double* pU = nullptr;
    uint32_t* pfb = nullptr;
    double *phcd = nullptr, *psv = nullptr, *pdnc = nullptr, *pdelta = nullptr;
    uint32_t* psi = nullptr;
    unsigned int* pfbn = nullptr;
    void* pscratch = nullptr;
    T *pxs = nullptr, *pxsq = nullptr, *pdist = nullptr;
    uint32_t* plab = nullptr;
    if (prune) {
        pU = cv.take<double>(n);
        pfb = cv.take<uint32_t>(n);
        phcd = cv.take<double>(k * k);
        psv = cv.take<double>(k * k);
        psi = cv.take<uint32_t>(k * k);
        pdnc = cv.take<double>(k);
        pdelta = cv.take<double>(k);
        pfbn = reinterpret_cast<unsigned int*>(cv.take<uint32_t>(1));
        pscratch = psel ? static_cast<void*>(cv.take<char>(psel)) : nullptr;
        pxs = cv.take<T>(prune_chunk * d);
        pxsq = cv.take<T>(prune_chunk);
        pdist = cv.take<T>(prune_chunk);
        plab = cv.take<uint32_t>(prune_chunk);
        // the computed squared distance sum (x_j - c_j)^2 (F, ascending j)
        // lies within gamma (relative) and eta (absolute, underflow) of the
        // true one
        const double uF = sizeof(T) == 4 ? std::ldexp(1.0, -24) : std::ldexp(1.0, -53);
        const double tinyF = sizeof(T) == 4 ? std::ldexp(1.0, -126) : std::ldexp(1.0, -1022);
        pc.gamma = 2.0 * (double)(d + 3) * uF;
        pc.eta = (double)(d + 3) * tinyF;
        pc.K = (1.0 + pc.gamma) / (1.0 - pc.gamma) * (1.0 + std::ldexp(1.0, -30));
        pc.umin = std::sqrt(std::ldexp(pc.eta, 30));
        pc.maxcand = 32;
        // finite rows only (the fused search's NaN rules stay its own)
        unsigned int bad = 0;
        e = launch_km_count_nonfinite<T>(xsq, n, pfbn, s);
        if (e != hipSuccess) return hip_err(e, "kmeans finite check");
        rc = km_d2h<T>(&bad, pfbn, sizeof(bad), s);
        if (rc) return rc;
        prune = bad == 0;
    }
    // Settles the assignment into lab_new from lab_old under the centres in
    // cdev, which moved by at most pdelta since lab_old's assignment: the
    // bound-pruned assignment plus fused searches of the rows it leaves
    // (all rows when they are most of them).  *fresh: every row's distance
    // was computed.
    auto prune_assign = [&](const uint32_t* lab_old, uint32_t* lab_new, bool* fresh) -> int32_t {
        hipError_t e2 = launch_km_half_dist<T>(cdev, k, d, phcd, pdnc, s);
        if (e2 == hipSuccess)
            e2 = launch_select_rows<double>(phcd, k, k, k, (int)k, EMIT_IDENTITY, psv, psi, pscratch, s);
        if (e2 == hipSuccess) e2 = launch_fill_u32(pfbn, 1, 0u, s);
        if (e2 == hipSuccess)
            e2 = launch_km_elkan<T>(x, n, d, cdev, k, w.perm, lab_old, lab_new, dist, pU, pdelta, pdnc, psv, psi, pc,
                                    pfb, pfbn, s);
        if (e2 != hipSuccess) return hip_err(e2, "kmeans pruned assignment");
        unsigned int m = 0;
        int32_t rc2 = km_d2h<T>(&m, pfbn, sizeof(m), s);
        if (rc2) return rc2;
        if ((int64_t)m * 5 > n * 3) {  // most rows left: one fused search of all of them
            rc2 = km_assign(x, n, cdev, k, d, lab_new, dist, s, xsq);
            if (rc2) return rc2;
            e2 = launch_km_bound_init<T>(dist, n, pc.gamma, pc.eta, pU, s);
            if (e2 != hipSuccess) return hip_err(e2, "kmeans bounds");
            *fresh = true;
            return MLRS_OK;
        }
        for (int64_t o = 0; o < (int64_t)m; o += prune_chunk) {
            const int64_t cm = std::min<int64_t>(prune_chunk, (int64_t)m - o);
            e2 = launch_km_gather_list<T>(x, xsq, pfb + o, cm, d, pxs, pxsq, s);
            if (e2 != hipSuccess) return hip_err(e2, "kmeans pruned gather");
            rc2 = km_assign(pxs, cm, cdev, k, d, plab, pdist, s, pxsq);
            if (rc2) return rc2;
            e2 = launch_km_scatter_list<T>(pfb + o, cm, plab, pdist, pc.gamma, pc.eta, lab_new, dist, pU, s);
            if (e2 != hipSuccess) return hip_err(e2, "kmeans pruned scatter");
        }
        *fresh = false;
        return MLRS_OK;
    };

    // ---- pipeline: every read-back lands in pinned memory and is waited for
    //      through an event, so the device keeps the next kernels queued while
    //      the host works.  Per iteration the host waits twice: for the
    //      counts (it decides on relocation before the assignment), and, with
    //      the next iteration's sums already queued, for the changed flag. ----
    const size_t st_bytes = aligned_bytes(sizeof(T) * (size_t)std::max(nbi, nbv * d)) +
                            2 * aligned_bytes(sizeof(T) * (size_t)kd) + aligned_bytes(sizeof(uint32_t) * (size_t)k) +
                            aligned_bytes(sizeof(int64_t) * (size_t)k) + aligned_bytes(sizeof(double) * (size_t)k) +
                            aligned_bytes(sizeof(T) * (size_t)d) + aligned_bytes(sizeof(unsigned int)) + 256;
    char* stage;
    rc = pinned_staging(st_bytes, &stage);
    if (rc) return rc;
    Carver sc(stage);
    T* h_parts = sc.take<T>((size_t)std::max(nbi, nbv * d));
    T* h_sums = sc.take<T>((size_t)kd);
    T* h_ct = sc.take<T>((size_t)kd);
    uint32_t* h_counts = sc.take<uint32_t>((size_t)k);
    int64_t* h_idx = sc.take<int64_t>((size_t)k);
    double* h_delta = sc.take<double>((size_t)k);
    T* h_means = sc.take<T>((size_t)d);
    unsigned int* h_changed = sc.take<unsigned int>(1);
    // the copies into pinned memory end before the call does, on every path
    struct Drain {
        hipStream_t s;
        bool on = false;
        hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
        ~Drain() {
            if (on) (void)hipStreamSynchronize(s);
            for (hipEvent_t x : ev)
                if (x) (void)hipEventDestroy(x);
        }
    } drain{s};
    for (hipEvent_t& x : drain.ev) {
        e = hipEventCreateWithFlags(&x, hipEventDisableTiming);
        if (e != hipSuccess) {
            x = nullptr;
            return hip_err(e, "hipEventCreateWithFlags");
        }
    }
    hipEvent_t evA = drain.ev[0], evB = drain.ev[1], evP = drain.ev[2];
    auto d2h_async = [&](void* dst, const void* src, size_t len) -> hipError_t {
        note_read_back();
        drain.on = true;
        return hipMemcpyAsync(dst, src, len, hipMemcpyDeviceToHost, s);
    };
    auto h2d_async = [&](void* dst, const void* src, size_t len) -> hipError_t {
        drain.on = true;
        return hipMemcpyAsync(dst, src, len, hipMemcpyHostToDevice, s);
    };
    auto wait_ev = [&](hipEvent_t ev, const char* what) -> int32_t {
        const hipError_t r = hipEventSynchronize(ev);
        return r == hipSuccess ? MLRS_OK : hip_err(r, what);
    };

    // ---- tol_scaled = tol * mean(var(X, axis=0)) (feature_mean_var).  The
    //      two passes' block partials come back asynchronously and the host
    //      sums them (f64, block order) while the first assignment runs. ----
    const double inv_n = 1.0 / (double)n;
    double tol_scaled = 0.0;
    int tol_stage = 0;  // 0: first pass queued; 1: second pass queued; 2: done
    e = launch_km_col_sums<T>(x, n, d, nbv, rpbv, nullptr, parts, s);
    if (e == hipSuccess) e = d2h_async(h_parts, parts, sizeof(T) * (size_t)(nbv * d));
    if (e == hipSuccess) e = hipEventRecord(evP, s);
    if (e != hipSuccess) return hip_err(e, "kmeans col sums");
    auto tol_step = [&]() -> int32_t {
        int32_t r = wait_ev(evP, "kmeans col sums");
        if (r) return r;
        if (tol_stage == 0) {
            std::vector<double> means((size_t)d, 0.0);
            for (int64_t b = 0; b < nbv; ++b)
                for (int64_t j = 0; j < d; ++j) means[j] += (double)h_parts[b * d + j];
            for (int64_t j = 0; j < d; ++j) {
                means[j] *= inv_n;
                h_means[j] = (T)means[j];
            }
            hipError_t e2 = h2d_async(means_dev, h_means, sizeof(T) * (size_t)d);
            if (e2 == hipSuccess) e2 = launch_km_col_sums<T>(x, n, d, nbv, rpbv, means_dev, parts, s);
            if (e2 == hipSuccess) e2 = d2h_async(h_parts, parts, sizeof(T) * (size_t)(nbv * d));
            if (e2 == hipSuccess) e2 = hipEventRecord(evP, s);
            if (e2 != hipSuccess) return hip_err(e2, "kmeans col sqdiff");
            tol_stage = 1;
        } else if (tol_stage == 1) {
            double var_sum = 0.0;
            for (int64_t q = 0; q < nbv * d; ++q) var_sum += (double)h_parts[q];
            tol_scaled = tol * ((var_sum * inv_n) / (double)d);
            tol_stage = 2;
        }
        return MLRS_OK;
    };

    // Two device centre buffers: the assignment reads one while the next
    // iteration's mean divide (queued before the loop knows whether it goes
    // on) writes the other.
    T* cbuf[2] = {cdev, cnext};
    int cb = 0;
    cdev = cbuf[cb];
    // This iteration's centroid sums under labv, the mean divide into cout,
    // the counts read back (the sums too where the host needs them before
    // the assignment: the pruned fit's centre moves); evA follows them.
    auto enqueue_sums = [&](const uint32_t* labv, T* cout) -> int32_t {
        hipError_t e2;
        {
            KernelTimer kt(s, "km_centroid_sums");
            e2 = launch_km_centroid_sums<T>(x, labv, n, d, k, nb, rpb, w, s);
        }
        if (e2 == hipSuccess) e2 = launch_km_mean<T>(w.sums, w.counts, k, d, cout, s);
        if (e2 == hipSuccess) e2 = d2h_async(h_counts, w.counts, sizeof(uint32_t) * (size_t)k);
        if (e2 == hipSuccess && prune) e2 = d2h_async(h_sums, w.sums, sizeof(T) * (size_t)kd);
        if (e2 == hipSuccess) e2 = hipEventRecord(evA, s);
        return e2 == hipSuccess ? MLRS_OK : hip_err(e2, "kmeans centroid sums");
    };

    std::vector<double> cen((size_t)kd), best_cen((size_t)kd), nc((size_t)kd);
    std::vector<T> ct((size_t)kd);
    std::vector<uint32_t> lab_h, best_lab_h;
    std::vector<T> dist_h;
    bool have = false;
    double best_inertia = 0.0;
    int64_t best_iter = 0;
    for (int64_t restart = 0; restart < runs; ++restart) {
        // ---- initial centres (init_centers, cluster/kmeans.rs:893-920) ----
        cb = 0;
        cdev = cbuf[cb];
        if (init_kind == 0) {
            e = hipMemcpyAsync(cdev, init, sizeof(T) * (size_t)kd, hipMemcpyDeviceToDevice, s);
            if (e != hipSuccess) return hip_err(e, "kmeans init");
        } else {
            KmRng rng{seed + (uint64_t)restart};
            std::vector<int64_t> chosen;
            chosen.reserve((size_t)k);
            if (init_kind == 2) {  // random_sample (prims/kmeans.rs:1769-1786)
                // the partial Fisher-Yates shuffle of 0..n over the positions
                // it touches only: a position absent from the map still holds
                // its own number (the same draws and swaps as a full array)
                std::unordered_map<int64_t, int64_t> ids;
                ids.reserve((size_t)(2 * k));
                auto at = [&](int64_t p) {
                    const auto it = ids.find(p);
                    return it == ids.end() ? p : it->second;
                };
                for (int64_t i = 0; i < k; ++i) {
                    const int64_t j = i + (int64_t)rng.next_below((uint64_t)(n - i));
                    const int64_t vi = at(i), vj = at(j);
                    ids[i] = vj;
                    ids[j] = vi;
                }
                chosen.resize((size_t)k);
                for (int64_t i = 0; i < k; ++i) chosen[i] = at(i);
            } else {  // kmeanspp_sample (prims/kmeans.rs:381-491)
                std::vector<char> is_chosen((size_t)n, 0);
                // the D^2 weights come back every draw: pinned host memory
                // (allocated here, freed on every exit) lets that copy run
                // as one DMA
                struct PinnedT {
                    T* p = nullptr;
                    ~PinnedT() {
                        if (p) (void)hipHostFree(p);
                    }
                } m2buf;
                e = hipHostMalloc((void**)&m2buf.p, sizeof(T) * (size_t)n, hipHostMallocDefault);
                if (e != hipSuccess) {
                    m2buf.p = nullptr;
                    return set_err(MLRS_ERR_ALLOC, "workspace", (int64_t)(sizeof(T) * (size_t)n), 0, 0, (int)e,
                                   "pinned host allocation of %zu bytes failed: %s", sizeof(T) * (size_t)n,
                                   hipGetErrorString(e));
                }
                T* const m2 = m2buf.p;
                // the weights' sequential f64 prefix, kept before every block
                // of kCk rows: the draw rescans one block, from the same
                // running sum, instead of every row before the pick
                constexpr int64_t kCk = 4096;
                std::vector<double> ck((size_t)((n + kCk - 1) / kCk + 1));
                int64_t cur = (int64_t)rng.next_below((uint64_t)n);
                chosen.push_back(cur);
                is_chosen[cur] = 1;
                for (int64_t m = 0; m + 1 < k; ++m) {
                    e = launch_km_mind2<T>(x, n, d, cur, m == 0 ? 1 : 0, mind2, s);
                    if (e != hipSuccess) return hip_err(e, "kmeans++ distances");
                    rc = km_d2h<T>(m2, mind2, sizeof(T) * (size_t)n, s);
                    if (rc) return rc;
                    double total = 0.0;
                    for (int64_t b0 = 0; b0 < n; b0 += kCk) {
                        ck[(size_t)(b0 / kCk)] = total;
                        const int64_t b1 = std::min<int64_t>(b0 + kCk, n);
                        for (int64_t i = b0; i < b1; ++i) total += (double)m2[i];
                    }
                    int64_t next = -1;
                    if (total <= 0.0) {
                        for (int64_t i = 0; i < n; ++i)
                            if (!is_chosen[i]) {
                                next = i;
                                break;
                            }
                        if (next < 0) return shape_err("k", 1, k, n);
                    } else {
                        const double target = rng.next_f64() * total;
                        // first row whose running sum reaches the target:
                        // the rows before the block whose starting sum is the
                        // last one below the target never reach it (the sums
                        // only grow), so the scan starts there with that sum.
                        // A non-finite total scans from the first row.
                        int64_t b = 0;
                        if (std::isfinite(total)) {
                            const int64_t nbk = (n + kCk - 1) / kCk;
                            int64_t lo = 0, hi = nbk;  // first block with start sum >= target
                            while (lo < hi) {
                                const int64_t mid = (lo + hi) / 2;
                                if (ck[(size_t)mid] < target)
                                    lo = mid + 1;
                                else
                                    hi = mid;
                            }
                            b = lo > 0 ? lo - 1 : 0;
                        }
                        double acc = ck[(size_t)b];
                        int64_t pick = n - 1;
                        for (int64_t i = b * kCk; i < n; ++i) {
                            acc += (double)m2[i];
                            if (acc >= target) {
                                pick = i;
                                break;
                            }
                        }
                        if ((double)m2[pick] <= 0.0)
                            for (int64_t i = n - 1; i >= 0; --i)
                                if ((double)m2[i] > 0.0) {
                                    pick = i;
                                    break;
                                }
                        if (is_chosen[pick])
                            for (int64_t i = 0; i < n; ++i)
                                if (!is_chosen[i]) {
                                    pick = i;
                                    break;
                                }
                        next = pick;
                    }
                    chosen.push_back(next);
                    is_chosen[next] = 1;
                    cur = next;
                }
            }
            for (int64_t i = 0; i < k; ++i) h_idx[i] = chosen[i];
            e = h2d_async(idx_dev, h_idx, sizeof(int64_t) * (size_t)k);
            if (e == hipSuccess) e = launch_km_gather<T>(x, idx_dev, k, d, cdev, s);
            if (e != hipSuccess) return hip_err(e, "kmeans init gather");
        }
        // the initial centres read back, waited for once the first assignment is queued
        e = d2h_async(h_ct, cdev, sizeof(T) * (size_t)kd);
        if (e == hipSuccess) e = hipEventRecord(evB, s);
        if (e != hipSuccess) return hip_err(e, "kmeans init read-back");

        // ---- single_run ----
        int cur = 0;
        rc = km_assign(x, n, cdev, k, d, lab[cur], dist, s, xsq);
        if (rc) return rc;
        bool dist_fresh = true;  // dist holds every row's distance to its centre
        if (prune) {
            e = launch_km_bound_init<T>(dist, n, pc.gamma, pc.eta, pU, s);
            if (e != hipSuccess) return hip_err(e, "kmeans bounds");
        }
        if (tol_stage == 0) {
            rc = tol_step();  // the means, summed while the assignment runs
            if (rc) return rc;
        }
        if (max_iter > 0) {
            rc = enqueue_sums(lab[cur], cbuf[cb ^ 1]);
            if (rc) return rc;
        }
        rc = wait_ev(evB, "kmeans init read-back");
        if (rc) return rc;
        for (int64_t q = 0; q < kd; ++q) {
            ct[q] = h_ct[q];
            cen[q] = (double)ct[q];
        }
        int64_t iters = 0;
        for (int64_t it = 0; it < max_iter; ++it) {
            ++iters;
            rc = wait_ev(evA, "kmeans centroid sums");
            if (rc) return rc;
            std::vector<int64_t> cnt((size_t)k);
            int64_t empties = 0;
            for (int64_t c = 0; c < k; ++c) {
                cnt[c] = h_counts[c];
                empties += cnt[c] == 0;
            }
            // The sums on the host: the pruned fit has them already (its
            // centre moves); a relocation needs them now; else they come back
            // with the changed flag, for the centre shift.
            bool have_sums = prune;
            if (empties && !have_sums) {
                e = d2h_async(h_sums, w.sums, sizeof(T) * (size_t)kd);
                if (e == hipSuccess) e = hipStreamSynchronize(s);
                if (e != hipSuccess) return hip_err(e, "kmeans centroid sums");
                have_sums = true;
            }
            if (have_sums)
                for (int64_t q = 0; q < kd; ++q) nc[q] = (double)h_sums[q];
            if (empties && !dist_fresh) {
                // the ranking reads every row's distance: the pruned
                // assignment left some untouched (same centres, same labels)
                rc = km_assign(x, n, cdev, k, d, lab[cur], dist, s, xsq);
                if (rc) return rc;
                e = launch_km_bound_init<T>(dist, n, pc.gamma, pc.eta, pU, s);
                if (e != hipSuccess) return hip_err(e, "kmeans bounds");
                dist_fresh = true;
            }
            if (empties) {
                // relocate_empty_clusters (prims/kmeans.rs:1323-1410): the
                // farthest rows by (distance desc, index asc) into the empty
                // clusters, never emptying their donor.  The walk records the
                // moves (target, row, donor) in its order; they are applied
                // afterwards in that order, so the sums see the same
                // operations as a walk that applies them as it goes.
                const int64_t m_top = std::min<int64_t>(8 * empties + 64, n);
                std::vector<int64_t> moves;  // (target, row, donor) triples
                std::vector<int64_t> cnt_w;
                // the walk over a ranked prefix: false when it runs past it
                auto walk = [&](int64_t len, const std::function<int64_t(int64_t)>& row_at,
                                const std::function<int64_t(int64_t)>& label_at) -> bool {
                    moves.clear();
                    cnt_w = cnt;
                    int64_t cursor = 0;
                    for (int64_t c = 0; c < k; ++c) {
                        if (cnt_w[c] != 0) continue;
                        bool ok_move = false;
                        while (cursor < len) {
                            const int64_t pos = cursor++;
                            const int64_t donor = label_at(pos);
                            if (cnt_w[donor] <= 1) continue;
                            moves.push_back(c);
                            moves.push_back(row_at(pos));
                            moves.push_back(donor);
                            ++cnt_w[c];
                            --cnt_w[donor];
                            ok_move = true;
                            break;
                        }
                        if (!ok_move) return false;
                    }
                    return true;
                };
                // (a) the top m_top rows ranked on the device: keys -distance
                //     selected by (key, index), the labels of those rows
                //     gathered; only they come back
                bool walked = false;
                if (m_top <= (int64_t)INT32_MAX) {
                    bool ranked = false;
                    std::vector<uint32_t> rows_r, labs_r;
                    rc = km_rank_device<T>(dist, lab[cur], n, m_top, rows_r, labs_r, &ranked, s);
                    if (rc) return rc;
                    if (ranked)
                        walked = walk(m_top, [&](int64_t p) { return (int64_t)rows_r[p]; },
                                      [&](int64_t p) { return (int64_t)labs_r[p]; });
                }
                // (b) the host ranking over every row: a NaN distance (ranked
                //     above every number, which the keys cannot express) or a
                //     walk past the device's prefix
                if (!walked) {
                    lab_h.resize((size_t)n);
                    dist_h.resize((size_t)n);
                    rc = km_d2h<T>(lab_h.data(), lab[cur], sizeof(uint32_t) * (size_t)n, s);
                    if (!rc) rc = km_d2h<T>(dist_h.data(), dist, sizeof(T) * (size_t)n, s);
                    if (rc) return rc;
                    std::vector<int64_t> order((size_t)n);
                    for (int64_t i = 0; i < n; ++i) order[i] = i;
                    // A total order (std::sort needs one): a NaN distance ranks
                    // above every number, NaNs and equal values by index.  On
                    // numbers it is the reference's (distance desc, index asc).
                    auto by_rank = [&](int64_t a, int64_t b) {
                        const double da = (double)dist_h[a], db = (double)dist_h[b];
                        const bool na = da != da, nb = db != db;
                        if (na != nb) return na;
                        if (!na) {
                            if (db < da) return true;
                            if (da < db) return false;
                        }
                        return a < b;
                    };
                    std::sort(order.begin(), order.end(), by_rank);
                    if (!walk(n, [&](int64_t p) { return order[p]; },
                              [&](int64_t p) { return (int64_t)lab_h[order[p]]; }))
                        return shape_err("labels", n, k, empties);
                }
                // the moved rows, gathered on the device and read back at once
                const int64_t nm = (int64_t)moves.size() / 3;
                std::vector<int64_t> mrow((size_t)nm);
                for (int64_t q = 0; q < nm; ++q) mrow[q] = moves[3 * q + 1];
                std::vector<T> rows_h((size_t)(nm * d));
                {
                    char* ws;
                    int cus;
                    rc = workspace(aligned_bytes(sizeof(T) * (size_t)(nm * d)) + 256, s, &ws, &cus);
                    if (rc) return rc;
                    T* rows_dev = reinterpret_cast<T*>(ws);
                    e = hipMemcpyAsync(idx_dev, mrow.data(), sizeof(int64_t) * (size_t)nm, hipMemcpyHostToDevice, s);
                    if (e == hipSuccess) e = launch_km_gather<T>(x, idx_dev, nm, d, rows_dev, s);
                    if (e != hipSuccess) return hip_err(e, "kmeans relocation rows");
                    rc = km_d2h<T>(rows_h.data(), rows_dev, sizeof(T) * (size_t)(nm * d), s);
                    if (rc) return rc;
                }
                for (int64_t q = 0; q < nm; ++q) {
                    const int64_t c = moves[3 * q], donor = moves[3 * q + 2];
                    for (int64_t j = 0; j < d; ++j) {
                        const double xij = (double)rows_h[q * d + j];
                        nc[c * d + j] += xij;
                        nc[donor * d + j] -= xij;
                    }
                }
                cnt = cnt_w;
            }
            // mean divide in f64 (single_run :1010-1030); the device's
            // km_mean_kernel made the same centres from the same operands, and
            // only a relocation changes them
            T* cnew = cbuf[cb ^ 1];
            auto mean_divide = [&]() {
                for (int64_t c = 0; c < k; ++c) {
                    const double inv = 1.0 / (double)cnt[c];
                    for (int64_t j = 0; j < d; ++j) nc[c * d + j] = nc[c * d + j] * inv;
                }
            };
            if (have_sums) {
                mean_divide();
                if (empties) {
                    for (int64_t q = 0; q < kd; ++q) h_ct[q] = (T)nc[q];
                    e = h2d_async(cnew, h_ct, sizeof(T) * (size_t)kd);
                    if (e != hipSuccess) return hip_err(e, "kmeans centres upload");
                }
                if (prune) {
                    // an upper bound of each centre's move (F centres, f64 sums)
                    for (int64_t c = 0; c < k; ++c) {
                        double acc = 0.0;
                        for (int64_t j = 0; j < d; ++j) {
                            const double diff = (double)(T)nc[c * d + j] - (double)ct[c * d + j];
                            acc += diff * diff;
                        }
                        h_delta[c] = std::sqrt(acc) * (1.0 + std::ldexp(1.0, -40));
                    }
                    e = h2d_async(pdelta, h_delta, sizeof(double) * (size_t)k);
                    if (e != hipSuccess) return hip_err(e, "kmeans centre moves upload");
                }
            }
            cb ^= 1;
            cdev = cnew;
            cur ^= 1;
            if (prune) {
                rc = prune_assign(lab[cur ^ 1], lab[cur], &dist_fresh);
            } else {
                rc = km_assign(x, n, cdev, k, d, lab[cur], dist, s, xsq);
                dist_fresh = true;
            }
            if (rc) return rc;
            e = launch_km_changed(lab[cur], lab[cur ^ 1], n, changed_dev, s);
            if (e == hipSuccess) e = d2h_async(h_changed, changed_dev, sizeof(unsigned int));
            if (e == hipSuccess && !have_sums) e = d2h_async(h_sums, w.sums, sizeof(T) * (size_t)kd);
            if (e == hipSuccess) e = hipEventRecord(evB, s);
            if (e != hipSuccess) return hip_err(e, "kmeans labels_changed");
            // the next iteration's sums, queued before this one's outcome is
            // known (unused when the loop stops here)
            if (it + 1 < max_iter) {
                rc = enqueue_sums(lab[cur], cbuf[cb ^ 1]);
                if (rc) return rc;
            }
            if (tol_stage == 1) {
                rc = tol_step();  // the variance, summed while the assignment runs
                if (rc) return rc;
            }
            rc = wait_ev(evB, "kmeans labels_changed");
            if (rc) return rc;
            if (!have_sums) {
                for (int64_t q = 0; q < kd; ++q) nc[q] = (double)h_sums[q];
                mean_divide();
            }
            double shift = 0.0;
            for (int64_t q = 0; q < kd; ++q) {
                const double diff = nc[q] - cen[q];
                shift += diff * diff;
            }
            cen.swap(nc);
            for (int64_t q = 0; q < kd; ++q) ct[q] = (T)cen[q];
            if (*h_changed == 0) break;    // strict convergence first
            if (shift <= tol_scaled) break;
        }
        // ---- inertia_ = sum of the per-row squared distances (inertia_rows +
        //      sum_device).  After a full assignment dist holds exactly those
        //      values (the assignment's exact value is inertia_rows' sum, in
        //      its order, under the final centres), so only the block sums run. ----
        if (dist_fresh)
            e = launch_km_block_sum<T>(dist, n, nbi, rpbi, parts, s);
        else
            e = launch_km_inertia<T>(x, cdev, lab[cur], n, d, dist, nbi, rpbi, parts, s);
        if (e != hipSuccess) return hip_err(e, "kmeans inertia");
        rc = km_d2h<T>(h_parts, parts, sizeof(T) * (size_t)nbi, s);
        if (rc) return rc;
        double inertia = 0.0;
        for (int64_t b = 0; b < nbi; ++b) inertia += (double)h_parts[b];
        // ---- keep the restart? strictly lower inertia on a different partition ----
        bool keep = !have;
        if (have && inertia < best_inertia) {
            lab_h.resize((size_t)n);
            rc = km_d2h<T>(lab_h.data(), lab[cur], sizeof(uint32_t) * (size_t)n, s);
            if (rc) return rc;
            std::vector<int64_t> map((size_t)k, -1);
            bool same = true;
            for (int64_t i = 0; i < n && same; ++i) {
                const uint32_t a = lab_h[i], b = best_lab_h[i];
                if (map[a] < 0)
                    map[a] = b;
                else if (map[a] != (int64_t)b)
                    same = false;
            }
            keep = !same;
        }
        if (keep) {
            have = true;
            best_inertia = inertia;
            best_iter = iters;
            best_cen = cen;
            e = hipMemcpyAsync(best_lab, lab[cur], sizeof(uint32_t) * (size_t)n, hipMemcpyDeviceToDevice, s);
            if (e != hipSuccess) return hip_err(e, "kmeans keep");
            if (runs > 1) {
                best_lab_h.resize((size_t)n);
                rc = km_d2h<T>(best_lab_h.data(), lab[cur], sizeof(uint32_t) * (size_t)n, s);
                if (rc) return rc;
            }
        }
    }
    for (int64_t q = 0; q < kd; ++q) ct[q] = (T)best_cen[q];
    e = hipMemcpyAsync(out_centers, ct.data(), sizeof(T) * (size_t)kd, hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(out_labels, best_lab, sizeof(uint32_t) * (size_t)n, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_err(e, "kmeans results");
    *out_inertia = best_inertia;
    *out_n_iter = best_iter;
    (void)perm;
    return ok();
}
}  // extern "C++"

int32_t mlrs_kmeans_fit_f32(const float* x, int64_t x_len, int64_t n, int64_t n_features, int64_t n_clusters,
                            int32_t init_kind, const float* init, int64_t init_len, uint64_t seed, int64_t n_init,
                            int64_t max_iter, double tol, int32_t algorithm, float* out_centers, int64_t centers_len,
                            uint32_t* out_labels, int64_t labels_len, double* out_inertia, int64_t* out_n_iter,
                            void* stream) {
    return kmeans_fit_impl<float>(x, x_len, n, n_features, n_clusters, init_kind, init, init_len, seed, n_init,
                                  max_iter, tol, algorithm, out_centers, centers_len, out_labels, labels_len, out_inertia,
                                  out_n_iter, stream);
}
int32_t mlrs_kmeans_fit_f64(const double* x, int64_t x_len, int64_t n, int64_t n_features, int64_t n_clusters,
                            int32_t init_kind, const double* init, int64_t init_len, uint64_t seed, int64_t n_init,
                            int64_t max_iter, double tol, int32_t algorithm, double* out_centers, int64_t centers_len,
                            uint32_t* out_labels, int64_t labels_len, double* out_inertia, int64_t* out_n_iter,
                            void* stream) {
    return kmeans_fit_impl<double>(x, x_len, n, n_features, n_clusters, init_kind, init, init_len, seed, n_init,
                                   max_iter, tol, algorithm, out_centers, centers_len, out_labels, labels_len, out_inertia,
                                   out_n_iter, stream);
}

int32_t mlrs_force_path(int32_t path) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (path < MLRS_PATH_AUTO || path > MLRS_PATH_GENERIC)
        return set_err(MLRS_ERR_UNSUPPORTED, "path", path, 0, 0, 0, "unknown kernel family %d", (int)path);
    g_force_path = path;
    return ok();
}

int32_t mlrs_timing_enable(int32_t on) {
    std::lock_guard<std::mutex> lk(g_mu);
    clear_timed();
    g_timing = on != 0;
    return MLRS_OK;
}

int32_t mlrs_timing_read(double* total_ms, int64_t* launches, char* kernel_name, int32_t name_len) {
    std::lock_guard<std::mutex> lk(g_mu);
    // per-name totals; the name with the largest summed time is reported
    std::vector<const char*> names;
    std::vector<double> tot;
    std::vector<int64_t> cnt;
    for (auto& t : g_timed) {
        hipError_t e = hipEventSynchronize(t.b);
        if (e != hipSuccess) return hip_err(e, "hipEventSynchronize");
        float ms = 0.0f;
        e = hipEventElapsedTime(&ms, t.a, t.b);
        if (e != hipSuccess) return hip_err(e, "hipEventElapsedTime");
        size_t i = 0;
        while (i < names.size() && std::strcmp(names[i], t.name) != 0) ++i;
        if (i == names.size()) {
            names.push_back(t.name);
            tot.push_back(0.0);
            cnt.push_back(0);
        }
        tot[i] += ms;
        ++cnt[i];
    }
    size_t best = 0;
    for (size_t i = 1; i < names.size(); ++i)
        if (tot[i] > tot[best]) best = i;
    const bool any = !names.empty();
    if (total_ms) *total_ms = any ? tot[best] : 0.0;
    if (launches) *launches = any ? cnt[best] : 0;
    if (kernel_name && name_len > 0) std::snprintf(kernel_name, (size_t)name_len, "%s", any ? names[best] : "");
    return MLRS_OK;
}

int32_t mlrs_probe_peak(int32_t kind, int32_t waves_per_simd, double* tflops, void* stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (kind < 0 || kind > 3) return set_err(MLRS_ERR_UNSUPPORTED, "kind", kind, 0, 0, 0, "probe kind %d", kind);
    if (waves_per_simd < 1 || waves_per_simd > 8)
        return set_err(MLRS_ERR_UNSUPPORTED, "waves_per_simd", waves_per_simd, 0, 0, 0,
                       "waves per SIMD must be 1..8, got %d", waves_per_simd);
    if (!tflops) return set_err(MLRS_ERR_NULL_POINTER, "tflops", 0, 0, 0, 0, "null pointer");
    int dev = 0, cus = 0;
    int32_t rc = current_device(&dev);
    if (rc) return rc;
    hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_err(e, "hipDeviceGetAttribute");
    // a workgroup is four waves, one per SIMD
    const int64_t blocks = (int64_t)cus * waves_per_simd;
    const int iters = kind <= 1 ? 4096 : 1024;
    hipStream_t s = (hipStream_t)stream;
    void* out = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    e = hipMalloc(&out, (size_t)blocks * 256 * 8);
    if (e == hipSuccess) e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    float ms = 0.0f;
    if (e == hipSuccess) e = launch_probe(kind, blocks, iters, out, s);  // warm-up
    if (e == hipSuccess) e = hipEventRecord(a, s);
    if (e == hipSuccess) e = launch_probe(kind, blocks, iters, out, s);
    if (e == hipSuccess) e = hipEventRecord(b, s);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (out) (void)hipFree(out);
    if (e != hipSuccess) return hip_err(e, "peak probe");
    *tflops = probe_flops(kind, blocks, iters) / ((double)ms * 1e-3) / 1e12;
    return MLRS_OK;
}

}  // extern "C"

namespace {
template <typename T>
int32_t device_copy_impl(const T* src, int64_t len, T* dst, int64_t dst_len, void* stream) {
    CallGuard cg;
    if (len < 0) return shape_err("src", len, 1, len);
    if (dst_len != len) return shape_err("dst", len, 1, dst_len);
    if (len == 0) return MLRS_OK;
    if (!src || !dst) return set_err(MLRS_ERR_NULL_POINTER, "src", 0, 0, 0, 0, "null pointer");
    const hipError_t e = launch_device_copy<T>(src, dst, len, (hipStream_t)stream);
    if (e != hipSuccess) return hip_err(e, "device_copy");
    return MLRS_OK;
}
}  // namespace

extern "C" {

int32_t mlrs_device_copy_f32(const float* src, int64_t len, float* dst, int64_t dst_len, void* stream) {
    return device_copy_impl<float>(src, len, dst, dst_len, stream);
}
int32_t mlrs_device_copy_f64(const double* src, int64_t len, double* dst, int64_t dst_len, void* stream) {
    return device_copy_impl<double>(src, len, dst, dst_len, stream);
}

int32_t mlrs_pool_stats_get(mlrs_pool_stats* out) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!out) return set_err(MLRS_ERR_NULL_POINTER, "out", 0, 0, 0, 0, "null pointer");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        std::memset(out, 0, sizeof(*out));
        return MLRS_OK;
    }
    *out = g_pool[dev];
    return MLRS_OK;
}

int32_t mlrs_pool_stats_reset(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MLRS_OK;
    mlrs_pool_stats& P = g_pool[dev];
    P.allocations = 0;
    P.reuses = 0;
    P.read_backs = 0;
    P.peak_bytes = P.live_bytes;
    return MLRS_OK;
}

int32_t mlrs_release_workspace(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MLRS_OK;
    Arena& A = g_arena[dev];
    Arena& X = g_aux[dev];
    RadiusPlan& P = g_rplan[dev];
    if (A.base || P.base || X.base) {
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) return hip_err(e, "hipDeviceSynchronize");
    }
    if (A.base) {
        buffer_free(&A.base, &A.pooled);
        pool_note_release(dev, A.cap);
        A.cap = 0;
    }
    if (X.base) {
        buffer_free(&X.base, &X.pooled);
        pool_note_release(dev, X.cap);
        X.cap = 0;
    }
    if (P.base) {
        buffer_free(&P.base, &P.pooled);
        pool_note_release(dev, P.cap);
        P.cap = 0;
        P.valid = false;
    }
    return MLRS_OK;
}

}  // extern "C"
