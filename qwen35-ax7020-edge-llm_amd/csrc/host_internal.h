// host_internal.h -- host-side state and helpers shared by the C-ABI
// translation units (qwen_kernels_api.cpp, qwen_runtime_api.cpp).  Not part
// of the public ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "bfp8_internal.h"
#include "qwen_kernels.h"

namespace qhost {

// ---- errors -----------------------------------------------------------------------
void set_error(const char* fmt, ...);
// Prints the last error and aborts: void entry points have no error channel
// and there is no CPU fallback.
[[noreturn]] void fatal(const char* where);

#define HIP_OK(expr)                                                                   \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess) {                                                        \
            set_error("%s: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__); \
            return BFP8_EHIP;                                                          \
        }                                                                              \
    } while (0)

// ---- profiler slots: 04/qwen_kernels_opt.c:71-82 ------------------------------------
enum {
    QP_GEMV = 0, QP_LMHEAD, QP_GDN, QP_CONV, QP_SWIGLU, QP_RMSNORM,
    QP_GATES, QP_QK, QP_GATED, QP_RESID, QP_EMBED, QP_PYCALLBACK,
    QP_LINEAR, QP_MLP, QP_TOTAL, QP_N
};
extern const char* const kProfNames[QP_N];
extern int g_prof_on;
extern double g_prof_ms[QP_N];
double now_ms();

struct ProfScope {
    int slot;
    double t0;
    explicit ProfScope(int s) : slot(s), t0(g_prof_on ? now_ms() : 0.0) {}
    ~ProfScope() {
        if (g_prof_on) g_prof_ms[slot] += now_ms() - t0;
    }
};

// ---- device buffers -------------------------------------------------------------------
// Bytes the library's DevBufs hold on the device, and a limit on them (0:
// none) that bfp8_debug_device_limit sets to rehearse a full device.
inline size_t g_dev_bytes = 0;
inline size_t g_dev_limit = 0;

struct DevBuf {
    void* p = nullptr;
    size_t n = 0;
    // BFP8_ENOMEM when the device cannot hold `bytes` more (the buffer is then
    // empty and HIP's last-error state clear, so that the next launch check
    // does not report this failure).
    int reserve(size_t bytes) {
        if (bytes <= n) return BFP8_OK;
        release();
        const size_t want = std::max<size_t>(bytes, 256);
        if (g_dev_limit && g_dev_bytes + want > g_dev_limit) {
            set_error("device memory: %zu more bytes exceed the limit of %zu", want, g_dev_limit);
            return BFP8_ENOMEM;
        }
        const hipError_t e = hipMalloc(&p, want);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            p = nullptr;
            set_error("hipMalloc(%zu): %s", want, hipGetErrorString(e));
            return e == hipErrorOutOfMemory ? BFP8_ENOMEM : BFP8_EHIP;
        }
        n = want;
        g_dev_bytes += n;
        return BFP8_OK;
    }
    void release() {
        if (p) {
            (void)hipFree(p);
            g_dev_bytes -= n;
        }
        p = nullptr;
        n = 0;
    }
    template <class T>
    T* as() const {
        return static_cast<T*>(p);
    }
};

// A cached bf16 table: row-major, or the 64-row tile layout of
// bf16_launch_tile_table (tiled) when the lm_head's tile kernel takes its width.
struct Bf16Table {
    DevBuf buf;
    int tiled = 0;
    uint64_t fp = 0;  // content fingerprint at conversion (content_fingerprint)
};

struct PinnedBuf {
    void* p = nullptr;
    size_t n = 0;
    int reserve(size_t bytes) {
        if (bytes <= n) return BFP8_OK;
        if (p) HIP_OK(hipHostFree(p));
        p = nullptr;
        n = 0;
        size_t want = std::max<size_t>(bytes, 4096);
        HIP_OK(hipHostMalloc(&p, want, hipHostMallocDefault));
        n = want;
        return BFP8_OK;
    }
};

struct CachedWeights {
    DevBuf mant, exps;
    uint64_t fp = 0;  // content fingerprint of both planes at conversion
};

// A cheap fingerprint of host memory [p, p+n): the first and last 64 bytes
// and 32 evenly spaced 8-byte words, hashed with the length.  A cached device
// copy is checked against it on every hit, so a buffer that was unmapped and
// replaced at the same address (a model reload) or rewritten is converted
// again instead of being served stale; changes that touch none of the sampled
// bytes still need bfp8_cache_clear().
uint64_t content_fingerprint(const void* p, size_t n);

using WeightKey = std::tuple<const void*, const void*, int, int>;

// Device scratch of the lm_head selections, one set per HIP stream: work on
// one stream is ordered, so calls on different streams never share partials.
struct StreamScratch {
    DevBuf partials;  // per-tile top-k lists
    DevBuf logits;    // scores of every row (general selection path)
    DevBuf keys;      // sort keys (k > BFP8_TOPK_MAX)
};

struct State {
    std::mutex mu;
    bool ready = false;
    bool gpu_checked = false, gpu_ok = false;  // bfp8_gpu_ready()'s verdict, once per process
    int device = 0;
    hipStream_t stream = nullptr;
    PinnedBuf h_in, h_out;
    DevBuf x, xq, xscale, xsplit, y;            // activation / output workspace
    DevBuf soa_m, soa_e, gpu_m, gpu_e;          // per-call weight upload
    DevBuf tk_out;                              // lm_head outputs of the host-pointer calls
    std::map<hipStream_t, StreamScratch> scratch;  // lm_head selection scratch per stream
    DevBuf bf16_ws;                             // per-call bf16 table upload
    DevBuf smp_in, smp_work, smp_out;           // sampler inputs / scratch / outputs
    PinnedBuf smp_h;
    DevBuf rt_dev;                              // runtime host-call arena (device)
    PinnedBuf rt_pin;                           // runtime host-call arena (pinned)
    std::map<WeightKey, CachedWeights> cache;
    std::map<WeightKey, Bf16Table> bf16_cache;  // read-only bf16 embedding tables
    size_t cache_bytes = 0;
    // ranges found writable by a /proc/self/maps scan: not scanned again
    // (such weights are uploaded per call either way)
    std::map<std::pair<const void*, size_t>, bool> writable;
};

extern State g;

int ensure_init_locked();
// Device-level entry points run on the caller's stream; NULL is the HIP
// default (null) stream, as everywhere in HIP.
inline hipStream_t pick_stream(void* s) { return static_cast<hipStream_t>(s); }
// Is every page of [p, p+n) mapped without write permission?
bool range_readonly(const void* p, size_t n);
// range_readonly, remembering a "writable" answer per (p, n) until
// bfp8_cache_clear(); g.mu held.
bool range_readonly_cached(const void* p, size_t n);
// The cached device copy of a bf16 table, if any (fingerprint checked).
bool bf16_table_lookup(const uint16_t* table, int vocab, int hidden, const uint16_t** out, int* tiled);

struct DevWeights {
    const uint8_t* mant;
    const uint8_t* exps;
};

// Device GPU-layout planes for host reference planes: cached when the planes
// are read-only (the engine's mmap), else converted into a per-call buffer.
int weights_for(const int8_t* mant, const uint8_t* exps, int M, int K, DevWeights* out);
// The same, cached whatever the memory's protection (force: the caller
// declares the planes immutable until bfp8_cache_clear()).
int weights_cached(const int8_t* mant, const uint8_t* exps, int M, int K, bool force, DevWeights* out);
// Device copy of a host bf16 table [vocab][hidden] (cached when read-only or
// forced; a cached copy is kept in the tile layout when bf16_tiled_ok(hidden),
// and *tiled says which layout *out has).
int bf16_table_for(const uint16_t* table, int vocab, int hidden, const uint16_t** out, int* tiled);
int bf16_table_cached(const uint16_t* table, int vocab, int hidden, bool force, const uint16_t** out, int* tiled);
// Pre-loads a float parameter the forward reads (host address, bytes); g.mu held.
int forward_preload_param(const void* p, size_t bytes);
// bf16 lm_head scores (+ fused top-k) on device buffers.
// tiled: the table is in the tile layout (then tail is moot: hidden % 8 == 0).
int bf16_lm_head_dev(int* ids, float* scores, int* count, int* argmax, float* logits, const float* h,
                     const uint16_t* table, int tiled, int vocab, int hidden, int k, int tail, hipStream_t s);
Bfp8GemvDesc plain_desc(float* y, const uint32_t* xsplit, const float* xscale, const uint8_t* m,
                        const uint8_t* e, int M, int K, int32_t* lanes);
// The lm_head selection scratch of stream s; g.mu held.
StreamScratch& scratch_for(hipStream_t s);
// The kk best rows of logits[0, n) by (score desc, id asc) among scores above
// -FLT_MAX into device outputs ids / scores [kk], count, argmax (the
// lm_head_argmax rule), on stream s: per-tile partials and the merge kernel
// for kk <= BFP8_TOPK_MAX, else a sort of all n keys.  g.mu held.
int select_topk_dev(const float* logits, int n, int kk, int* ids, float* scores, int* count, int* argmax,
                    hipStream_t s);

// One grouped launch: its tile table, either dealt over a persistent grid
// (wg_off per workgroup) or one tile per 16-wavefront workgroup (wide).
struct Launch {
    DevBuf tiles, wg_off;
    int nwg = 0;
    bool wide = false;
    int ntiles = 0, max_nb = 0;
    int rows[2] = {-1, -1};  // >= 0: one or two GEMVs sharing an activation, 16 rows per workgroup
};

// Drops the forward's device copies (qwen_runtime_api.cpp); g.mu held.
void forward_cache_clear();
// Forgets the preloaded tensors' names (qwen_weights.cpp); g.mu held.
void weights_index_clear();

// Deals the tiles of items[idx] over a launch (persistent or wide).
int deal_tiles(Launch& L, const std::vector<int>& idx, const bfp8_plan_item* items, int wg0_extra, bool allow_wide);

}  // namespace qhost
