// qwen_kernels_api.cpp -- host side of libqwen_kernels.so (C ABI in
// include/qwen_kernels.h).  Owns the device, a HIP stream, device
// workspaces, pinned staging buffers, the read-only weight cache and the
// grouped-GEMV plans.  All arithmetic runs in the HIP kernels of bfp8_ftz.hip
// and bfp8_ieee.hip; nothing here computes results on the CPU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <map>
#include <mutex>
#include <queue>
#include <string>
#include <tuple>
#include <vector>

#include "host_internal.h"
#include "runtime_internal.h"

namespace qhost {

// ---- errors ---------------------------------------------------------------------
std::mutex g_err_mu;
std::string g_err;

void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    std::lock_guard<std::mutex> lk(g_err_mu);
    g_err = buf;
}

[[noreturn]] void fatal(const char* where) {
    std::string msg;
    {
        std::lock_guard<std::mutex> lk(g_err_mu);
        msg = g_err;
    }
    fprintf(stderr, "libqwen_kernels: %s failed on the GPU: %s (no CPU fallback; aborting)\n", where,
            msg.c_str());
    fflush(stderr);
    abort();
}

// ---- profiler slots (names in the reference's order) -----------------------------
const char* const kProfNames[QP_N] = {
    "bfp8_gemv", "lm_head_argmax", "gdn_recurrent_step", "conv1d_silu", "swiglu", "rmsnorm",
    "gdn_gates", "qk_l2norm", "rmsnorm_gated", "add_residual", "embed_lookup", "py_full_attn",
    "forward_linear_layer", "forward_mlp", "forward_token_c"};
int g_prof_on = 0;
double g_prof_ms[QP_N];

double now_ms() {
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec * 1e3 + (double)ts.tv_nsec / 1e6;
}


State g;
constexpr size_t kCacheLimit = (size_t)200 << 30;

int ensure_init_locked() {
    if (g.ready) return BFP8_OK;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        set_error("no HIP device available (%s)", hipGetErrorString(e));
        return BFP8_EHIP;
    }
    HIP_OK(hipGetDevice(&g.device));
    HIP_OK(hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking));
    g.ready = true;
    return BFP8_OK;
}

bool range_readonly(const void* p, size_t n) {
    if (!p || n == 0) return false;
    FILE* f = fopen("/proc/self/maps", "r");
    if (!f) return false;
    uintptr_t cur = (uintptr_t)p, end = cur + n;
    char line[512];
    bool ok = false;
    while (fgets(line, sizeof line, f)) {
        unsigned long lo = 0, hi = 0;
        char perms[8] = {0};
        if (sscanf(line, "%lx-%lx %7s", &lo, &hi, perms) != 3) continue;
        if (hi <= cur) continue;
        if (lo > cur || perms[1] == 'w') break;  // gap or writable
        cur = hi;
        if (cur >= end) {
            ok = true;
            break;
        }
    }
    fclose(f);
    return ok;
}

bool range_readonly_cached(const void* p, size_t n) {
    const auto key = std::make_pair(p, n);
    if (g.writable.count(key)) return false;
    const bool ro = range_readonly(p, n);
    if (!ro) g.writable.emplace(key, true);
    return ro;
}

uint64_t content_fingerprint(const void* p, size_t n) {
    const unsigned char* b = static_cast<const unsigned char*>(p);
    uint64_t h = 0xcbf29ce484222325ull ^ (uint64_t)n;
    auto mix = [&h](const unsigned char* q, size_t len) {
        for (size_t i = 0; i < len; ++i) h = (h ^ q[i]) * 0x100000001b3ull;
    };
    if (!b || n == 0) return h;
    const size_t edge = std::min<size_t>(n, 64);
    mix(b, edge);
    mix(b + (n - edge), edge);
    if (n >= 8)
        for (size_t i = 0; i < 32; ++i) mix(b + (i * (n - 8)) / 31, 8);
    return h;
}

static uint64_t planes_fingerprint(const int8_t* mant, size_t mbytes, const uint8_t* exps, size_t ebytes) {
    return content_fingerprint(mant, mbytes) * 31 + content_fingerprint(exps, ebytes);
}

// Device GPU-layout planes for host reference planes.
int weights_cached(const int8_t* mant, const uint8_t* exps, int M, int K, bool force, DevWeights* out) {
    const int nb = bfp8_nblocks(K);
    const size_t mbytes = (size_t)M * (size_t)K, ebytes = (size_t)M * (size_t)nb;
    const WeightKey key{mant, exps, M, K};
    auto it = g.cache.find(key);
    if (it != g.cache.end()) {
        if (it->second.fp == planes_fingerprint(mant, mbytes, exps, ebytes)) {
            out->mant = it->second.mant.as<uint8_t>();
            out->exps = it->second.exps.as<uint8_t>();
            return BFP8_OK;
        }
        // the memory behind the cached address changed: convert again
        HIP_OK(hipStreamSynchronize(g.stream));
        g.cache_bytes -= it->second.mant.n + it->second.exps.n;
        it->second.mant.release();
        it->second.exps.release();
        g.cache.erase(it);
    }
    int rc;
    if ((rc = g.soa_m.reserve(mbytes)) || (rc = g.soa_e.reserve(ebytes))) return rc;
    HIP_OK(hipMemcpyAsync(g.soa_m.p, mant, mbytes, hipMemcpyHostToDevice, g.stream));
    HIP_OK(hipMemcpyAsync(g.soa_e.p, exps, ebytes, hipMemcpyHostToDevice, g.stream));
    const size_t gm = bfp8_gpu_mant_bytes(M, K), ge = bfp8_gpu_exps_bytes(M, K);
    bool cacheable = g.cache_bytes + gm + ge <= kCacheLimit &&
                     (force || (range_readonly_cached(mant, mbytes) && range_readonly_cached(exps, ebytes)));
    if (force && !cacheable) {
        set_error("device weight cache full (%zu bytes)", g.cache_bytes);
        return BFP8_EINVAL;
    }
    DevBuf* dm = &g.gpu_m;
    DevBuf* de = &g.gpu_e;
    CachedWeights cw;
    if (cacheable) {
        if ((rc = cw.mant.reserve(gm)) || (rc = cw.exps.reserve(ge))) {
            // the device holds no further cached copy: a preload fails, any
            // other call converts into the per-call buffers (recoverable)
            cw.mant.release();
            cw.exps.release();
            if (force) return rc;
            cacheable = false;
        } else {
            dm = &cw.mant;
            de = &cw.exps;
        }
    }
    if ((rc = dm->reserve(gm)) || (rc = de->reserve(ge))) return rc;
    HIP_OK(bfp8_launch_pack(dm->as<uint8_t>(), de->as<uint8_t>(), g.soa_m.as<int8_t>(),
                            g.soa_e.as<uint8_t>(), M, K, g.stream));
    out->mant = dm->as<uint8_t>();
    out->exps = de->as<uint8_t>();
    if (cacheable) {
        cw.fp = planes_fingerprint(mant, mbytes, exps, ebytes);
        g.cache_bytes += cw.mant.n + cw.exps.n;
        g.cache.emplace(key, cw);
    }
    return BFP8_OK;
}

int weights_for(const int8_t* mant, const uint8_t* exps, int M, int K, DevWeights* out) {
    return weights_cached(mant, exps, M, K, false, out);
}

int upload_x(const float* x, size_t nfloat);

// Device copy of a host bf16 table [vocab][hidden]: cached when it lives in
// read-only memory (the engine's mmap) or when forced, else uploaded per call.
// A cached table whose width the tile kernel takes is converted once, on the
// device, into the tile layout (the row-major upload goes through bf16_ws).
bool bf16_table_lookup(const uint16_t* table, int vocab, int hidden, const uint16_t** out, int* tiled) {
    const size_t bytes = (size_t)vocab * (size_t)hidden * 2;
    auto it = g.bf16_cache.find(WeightKey{table, nullptr, vocab, hidden});
    if (it == g.bf16_cache.end()) return false;
    if (it->second.fp != content_fingerprint(table, bytes)) {  // replaced or rewritten: convert again
        (void)hipStreamSynchronize(g.stream);
        g.cache_bytes -= it->second.buf.n;
        it->second.buf.release();
        g.bf16_cache.erase(it);
        return false;
    }
    *out = it->second.buf.as<uint16_t>();
    *tiled = it->second.tiled;
    return true;
}

int bf16_table_cached(const uint16_t* table, int vocab, int hidden, bool force, const uint16_t** out, int* tiled) {
    const size_t bytes = (size_t)vocab * (size_t)hidden * 2;
    const WeightKey key{table, nullptr, vocab, hidden};
    if (bf16_table_lookup(table, vocab, hidden, out, tiled)) return BFP8_OK;
    const bool tile = bf16_tiled_ok(hidden);
    const size_t kept = tile ? bf16_tiled_elems(vocab, hidden) * 2 : bytes;
    bool cacheable = g.cache_bytes + kept <= kCacheLimit && (force || range_readonly_cached(table, bytes));
    int rc;
    Bf16Table fresh;
    if (cacheable) {
        // (the tile layout is converted from a row-major upload in bf16_ws)
        if ((rc = fresh.buf.reserve(kept)) || (tile && (rc = g.bf16_ws.reserve(bytes)))) {
            fresh.buf.release();   // no room for another cached table: a preload
            if (force) return rc;  // fails, any other call uploads per call
            cacheable = false;
        }
    }
    if (!cacheable) {
        if ((rc = g.bf16_ws.reserve(bytes))) return rc;
        HIP_OK(hipMemcpyAsync(g.bf16_ws.p, table, bytes, hipMemcpyHostToDevice, g.stream));
        *out = g.bf16_ws.as<uint16_t>();
        *tiled = 0;
        return BFP8_OK;
    }
    if (tile) {
        HIP_OK(hipMemcpyAsync(g.bf16_ws.p, table, bytes, hipMemcpyHostToDevice, g.stream));
        HIP_OK(bf16_launch_tile_table(fresh.buf.as<uint16_t>(), g.bf16_ws.as<uint16_t>(), vocab, hidden, g.stream));
        fresh.tiled = 1;
    } else {
        HIP_OK(hipMemcpyAsync(fresh.buf.p, table, bytes, hipMemcpyHostToDevice, g.stream));
    }
    *out = fresh.buf.as<uint16_t>();
    *tiled = fresh.tiled;
    fresh.fp = content_fingerprint(table, bytes);
    g.cache_bytes += fresh.buf.n;
    g.bf16_cache.emplace(key, fresh);
    return BFP8_OK;
}

int bf16_table_for(const uint16_t* table, int vocab, int hidden, const uint16_t** out, int* tiled) {
    return bf16_table_cached(table, vocab, hidden, false, out, tiled);
}

StreamScratch& scratch_for(hipStream_t s) { return g.scratch[s]; }

// Selection with the caller's scratch: partials (bfp8_ntiles(n) * kk keys)
// when kk <= BFP8_TOPK_MAX, else keys (bfp8_select_scratch_bytes(n)).
// Allocates nothing.
int select_topk_raw(const float* logits, int n, int kk, int* ids, float* scores, int* count, int* argmax,
                    uint64_t* partials, uint64_t* keys, hipStream_t s) {
    if (kk <= BFP8_TOPK_MAX) {
        HIP_OK(bfp8_launch_select_partials(logits, n, kk, partials, s));
        Bfp8GemvDesc md{};
        md.M = n;
        md.topk = kk;
        md.partials = partials;
        md.out_ids = ids;
        md.out_scores = scores;
        md.out_count = count;
        md.out_argmax = argmax;
        HIP_OK(bfp8_launch_topk_merge(md, s));
        return BFP8_OK;
    }
    HIP_OK(bfp8_launch_select_sort(logits, n, kk, keys, ids, scores, count, argmax, s));
    return BFP8_OK;
}

int select_topk_bufs(const float* logits, int n, int kk, int* ids, float* scores, int* count, int* argmax,
                     DevBuf& partials, DevBuf& keys, hipStream_t s) {
    int rc;
    if (kk <= BFP8_TOPK_MAX) {
        if ((rc = partials.reserve((size_t)bfp8_ntiles(n) * kk * 8))) return rc;
    } else if ((rc = keys.reserve(bfp8_select_scratch_bytes(n)))) {
        return rc;
    }
    return select_topk_raw(logits, n, kk, ids, scores, count, argmax, partials.as<uint64_t>(), keys.as<uint64_t>(), s);
}

int select_topk_dev(const float* logits, int n, int kk, int* ids, float* scores, int* count, int* argmax,
                    hipStream_t s) {
    StreamScratch& ss = scratch_for(s);
    return select_topk_bufs(logits, n, kk, ids, scores, count, argmax, ss.partials, ss.keys, s);
}

// bf16 lm_head scores (+ top-k) on device buffers: k <= BFP8_TOPK_MAX fused
// into the scoring launch (per-tile lists, then the merge), larger k through
// the scores and a sort.
int bf16_lm_head_dev(int* ids, float* scores, int* count, int* argmax, float* logits, const float* h,
                     const uint16_t* table, int tiled, int vocab, int hidden, int k, int tail, hipStream_t s) {
    const int kk = k > 0 ? std::min(k, vocab) : 0;
    StreamScratch& ss = scratch_for(s);
    int rc;
    Bf16HeadDesc d{};
    d.table = table;
    d.h = h;
    d.logits = logits;
    d.vocab = vocab;
    d.hidden = hidden;
    d.tail = tail;
    d.tiled = tiled;
    if (kk > BFP8_TOPK_MAX) {
        if (!logits) {
            if ((rc = ss.logits.reserve((size_t)vocab * 4))) return rc;
            d.logits = ss.logits.as<float>();
        }
        HIP_OK(bf16_launch_lm_head(d, s));
        return select_topk_dev(d.logits, vocab, kk, ids, scores, count, argmax, s);
    }
    if (kk > 0 && (rc = ss.partials.reserve((size_t)bfp8_ntiles(vocab) * kk * 8))) return rc;
    d.partials = kk > 0 ? ss.partials.as<uint64_t>() : nullptr;
    d.topk = kk;
    HIP_OK(bf16_launch_lm_head(d, s));
    if (kk > 0) {
        Bfp8GemvDesc md{};
        md.M = vocab;
        md.topk = kk;
        md.partials = d.partials;
        md.out_ids = ids;
        md.out_scores = scores;
        md.out_count = count;
        md.out_argmax = argmax;
        HIP_OK(bfp8_launch_topk_merge(md, s));
    }
    return BFP8_OK;
}

// Host-pointer bf16 lm_head: returns the candidate count (fills ids/scores
// when given) and the argmax through *am.
int host_bf16_lm_head(const float* h, const uint16_t* table, int vocab, int hidden, int k, int tail,
                      int* out_ids, float* out_scores, int* am) {
    int rc;
    const uint16_t* tdev;
    int tiled = 0;
    if ((rc = bf16_table_for(table, vocab, hidden, &tdev, &tiled)) || (rc = upload_x(h, (size_t)hidden))) return rc;
    const int kk = std::min(k, vocab);
    const size_t outb = (size_t)(2 * kk + 2) * 4;
    if ((rc = g.tk_out.reserve(outb)) || (rc = g.h_out.reserve(outb))) return rc;
    int* d_ids = g.tk_out.as<int>();
    float* d_sc = reinterpret_cast<float*>(d_ids + kk);
    int* d_cnt = d_ids + 2 * kk;
    if ((rc = bf16_lm_head_dev(d_ids, d_sc, d_cnt, d_cnt + 1, nullptr, g.x.as<float>(), tdev, tiled, vocab, hidden,
                               kk, tail, g.stream)))
        return rc;
    HIP_OK(hipMemcpyAsync(g.h_out.p, g.tk_out.p, outb, hipMemcpyDeviceToHost, g.stream));
    HIP_OK(hipStreamSynchronize(g.stream));
    const int* hi = static_cast<const int*>(g.h_out.p);
    const int n = hi[2 * kk];
    if (am) *am = hi[2 * kk + 1];
    if (out_ids && n > 0) memcpy(out_ids, hi, (size_t)n * 4);
    if (out_scores && n > 0) memcpy(out_scores, hi + kk, (size_t)n * 4);
    return n;
}

int upload_x(const float* x, size_t nfloat) {
    int rc;
    if ((rc = g.h_in.reserve(nfloat * 4)) || (rc = g.x.reserve(nfloat * 4))) return rc;
    memcpy(g.h_in.p, x, nfloat * 4);
    HIP_OK(hipMemcpyAsync(g.x.p, g.h_in.p, nfloat * 4, hipMemcpyHostToDevice, g.stream));
    return BFP8_OK;
}

int quantize_ws(int K, int B) {
    int rc;
    const int nb = bfp8_nblocks(K);
    if ((rc = g.xq.reserve((size_t)B * nb * 64 * 2)) || (rc = g.xscale.reserve((size_t)B * nb * 4)) ||
        (rc = g.xsplit.reserve((size_t)B * bfp8_xsplit_bytes(K))))
        return rc;
    for (int b = 0; b < B; ++b) {
        Bfp8QuantDesc q{};
        q.x = g.x.as<float>() + (size_t)b * nb * 64;
        q.xq = g.xq.as<int16_t>() + (size_t)b * nb * 64;
        q.xscale = g.xscale.as<float>() + (size_t)b * nb;
        q.xsplit = g.xsplit.as<uint32_t>() + (size_t)b * nb * 32;
        q.K = K;
        HIP_OK(bfp8_launch_quantize1(q, g.stream));
    }
    return BFP8_OK;
}

Bfp8GemvDesc plain_desc(float* y, const uint32_t* xsplit, const float* xscale, const uint8_t* m,
                        const uint8_t* e, int M, int K, int32_t* lanes) {
    Bfp8GemvDesc d{};
    d.mant = m;
    d.exps = e;
    d.xsplit = xsplit;
    d.xscale = xscale;
    d.y = y;
    d.lanes = lanes;
    d.M = M;
    d.K = K;
    d.pair_rows = M & ~1;
    return d;
}

// Quantized GEMV on the device (K <= 4096): paired rows + odd last row.
int gemv_q(float* y, const uint32_t* xsplit, const float* xscale, const uint8_t* m, const uint8_t* e,
           int M, int K, int32_t* lanes, hipStream_t s) {
    HIP_OK(bfp8_launch_gemv(plain_desc(y, xsplit, xscale, m, e, M, K, lanes), s));
    HIP_OK(bfp8_launch_tail_row(y, xsplit, xscale, m, e, M, K, s));
    return BFP8_OK;
}

// A GEMV of at most BFP8_WIDE_MAX_TILES row tiles from float x on the device:
// the 16-row kernel quantizes x itself, leaving the records for the odd last
// row's kernel in xsplit_out / xscale_out (needed only for odd M).
int rows_gemv_float(float* y, const float* x, const uint8_t* m, const uint8_t* e, int M, int K,
                    uint32_t* xsplit_out, float* xscale_out, hipStream_t s) {
    RtRowsArgs a{};
    a.g[0].mant = m;
    a.g[0].exps = e;
    a.g[0].y = y;
    a.g[0].M = M;
    a.g[0].pair_rows = M & ~1;
    a.ngemv = 1;
    a.split = (M + 15) / 16;
    a.K = K;
    a.mode = RT_ROWS_FLOAT;
    a.x = x;
    if (M & 1) {
        a.xsplit_out = xsplit_out;
        a.xscale_out = xscale_out;
    }
    HIP_OK(rt_launch_rows(a, s));
    HIP_OK(bfp8_launch_tail_row(y, xsplit_out, xscale_out, m, e, M, K, s));
    return BFP8_OK;
}

// y_dev[M] = bfp8_gemv(x) for x already in g.x (K floats), on g.stream: the
// quantized path for K <= 4096 (whole blocks; an odd last row in the scalar
// order), the float path above; no whole block gives zeros.
int gemv_from_x(float* y_dev, const DevWeights& w, int M, int K) {
    const int nb = bfp8_nblocks(K);
    int rc;
    if (nb == 0) {
        HIP_OK(hipMemsetAsync(y_dev, 0, (size_t)M * 4, g.stream));
    } else if (K <= 4096 && bfp8_ntiles(M) <= BFP8_WIDE_MAX_TILES) {
        // one launch: the 16-row kernel quantizes x itself
        if ((rc = g.xscale.reserve((size_t)nb * 4)) || (rc = g.xsplit.reserve(bfp8_xsplit_bytes(K)))) return rc;
        if ((rc = rows_gemv_float(y_dev, g.x.as<float>(), w.mant, w.exps, M, K, g.xsplit.as<uint32_t>(),
                                  g.xscale.as<float>(), g.stream)))
            return rc;
    } else if (K <= 4096) {
        if ((rc = quantize_ws(K, 1))) return rc;
        if ((rc = gemv_q(y_dev, g.xsplit.as<uint32_t>(), g.xscale.as<float>(), w.mant, w.exps, M, K, nullptr,
                         g.stream)))
            return rc;
    } else {
        HIP_OK(bfp8_launch_gemv_float(y_dev, g.x.as<float>(), w.mant, w.exps, M, K, g.stream));
    }
    return BFP8_OK;
}

int host_gemv(float* y, const float* x, const int8_t* mant, const uint8_t* exps, int M, int K) {
    const int nb = bfp8_nblocks(K);
    if (nb == 0) {  // no whole block: the reference's accumulators stay 0
        memset(y, 0, (size_t)M * sizeof(float));
        return BFP8_OK;
    }
    int rc;
    DevWeights w;
    if ((rc = weights_for(mant, exps, M, K, &w))) return rc;
    if ((rc = upload_x(x, (size_t)(K <= 4096 ? nb * 64 : K)))) return rc;
    if ((rc = g.h_out.reserve((size_t)M * 4))) return rc;
    // the GEMV stores y straight into the pinned host buffer (no device
    // buffer and copy back: 19.5-20.1 against 21.2-22.3 us per call at the
    // engine callback's shapes); the stream synchronization makes the
    // stores visible to the host
    if ((rc = gemv_from_x(static_cast<float*>(g.h_out.p), w, M, K))) return rc;
    HIP_OK(hipStreamSynchronize(g.stream));
    memcpy(y, g.h_out.p, (size_t)M * 4);
    return BFP8_OK;
}

// The fused BFP8 lm_head launch takes: even vocab (every row in a pair),
// k <= BFP8_TOPK_MAX, a quantized activation (hidden 64 .. 4096).  Other
// arguments take the general path: the plain GEMV (odd last row included,
// the float path above 4096) into a scores buffer, then the selection.
bool lm_head_fused_ok(int vocab, int hidden, int kk) {
    return vocab > 0 && !(vocab & 1) && bfp8_ntiles(vocab) <= BFP8_TOPK_MAX_TILES && hidden >= 64 &&
           hidden <= 4096 && kk >= 1 && kk <= BFP8_TOPK_MAX;
}

bool lm_head_args_ok(int vocab, int hidden, int k) {
    return vocab > 0 && vocab <= BFP8_SELECT_MAX && hidden > 0 && k >= 1;
}

int lm_head_dev(int* ids, float* scores, int* count, int* argmax, const uint32_t* xsplit,
                const float* xscale, const uint8_t* m, const uint8_t* e, int vocab, int hidden, int k,
                hipStream_t s) {
    const int kk = std::min(k, vocab);
    StreamScratch& ss = scratch_for(s);
    int rc;
    if (!lm_head_fused_ok(vocab, hidden, kk)) {  // general path (hidden <= 4096: a quantized activation)
        if ((rc = ss.logits.reserve((size_t)vocab * 4))) return rc;
        float* lg = ss.logits.as<float>();
        if (bfp8_nblocks(hidden) == 0)
            HIP_OK(hipMemsetAsync(lg, 0, (size_t)vocab * 4, s));
        else if ((rc = gemv_q(lg, xsplit, xscale, m, e, vocab, hidden, nullptr, s)))
            return rc;
        return select_topk_dev(lg, vocab, kk, ids, scores, count, argmax, s);
    }
    if ((rc = ss.partials.reserve((size_t)bfp8_ntiles(vocab) * kk * 8))) return rc;
    Bfp8GemvDesc d = plain_desc(nullptr, xsplit, xscale, m, e, vocab, hidden, nullptr);
    d.topk = kk;
    d.partials = ss.partials.as<uint64_t>();
    d.out_ids = ids;
    d.out_scores = scores;
    d.out_count = count;
    d.out_argmax = argmax;
    HIP_OK(bfp8_launch_gemv(d, s));
    return BFP8_OK;
}

int host_lm_head(const float* h, const int8_t* mant, const uint8_t* exps, int vocab, int hidden, int k,
                 int* out_ids, float* out_scores, int* out_argmax) {
    int rc;
    DevWeights w;
    if ((rc = weights_for(mant, exps, vocab, hidden, &w))) return rc;
    const int nb = bfp8_nblocks(hidden);
    const int kk = std::min(k, vocab);
    const size_t outb = (size_t)(2 * kk + 2) * 4;
    if ((rc = g.tk_out.reserve(outb)) || (rc = g.h_out.reserve(outb))) return rc;
    int* d_ids = g.tk_out.as<int>();
    float* d_scores = reinterpret_cast<float*>(d_ids + kk);
    int* d_cnt = d_ids + 2 * kk;
    if ((rc = upload_x(h, (size_t)(hidden <= 4096 ? nb * 64 : hidden)))) return rc;
    if (lm_head_fused_ok(vocab, hidden, kk)) {
        if ((rc = quantize_ws(hidden, 1))) return rc;
        if ((rc = lm_head_dev(d_ids, d_scores, d_cnt, d_cnt + 1, g.xsplit.as<uint32_t>(), g.xscale.as<float>(),
                              w.mant, w.exps, vocab, hidden, kk, g.stream)))
            return rc;
    } else {  // the plain GEMV's scores, then the selection
        StreamScratch& ss = scratch_for(g.stream);
        if ((rc = ss.logits.reserve((size_t)vocab * 4))) return rc;
        if ((rc = gemv_from_x(ss.logits.as<float>(), w, vocab, hidden))) return rc;
        if ((rc = select_topk_dev(ss.logits.as<float>(), vocab, kk, d_ids, d_scores, d_cnt, d_cnt + 1, g.stream)))
            return rc;
    }
    HIP_OK(hipMemcpyAsync(g.h_out.p, g.tk_out.p, outb, hipMemcpyDeviceToHost, g.stream));
    HIP_OK(hipStreamSynchronize(g.stream));
    const int* hi = static_cast<const int*>(g.h_out.p);
    const int cnt = hi[2 * kk];
    if (out_ids) memcpy(out_ids, hi, (size_t)cnt * 4);
    if (out_scores) memcpy(out_scores, hi + kk, (size_t)cnt * 4);
    if (out_argmax) *out_argmax = hi[2 * kk + 1];
    return cnt;
}

// ---- synthetic inputs ----------------------------------------------------------------------
double unit53(uint64_t h) { return (double)(h >> 11) * (1.0 / 9007199254740992.0); }

double normal_at(uint64_t seed, uint64_t i) {
    const double u1 = unit53(bfp8_hash64(seed, 2 * i)) + (1.0 / 9007199254740992.0);  // (0, 1]
    const double u2 = unit53(bfp8_hash64(seed, 2 * i + 1));
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

}  // namespace qhost

using namespace qhost;

// =========================== C ABI ================================================
extern "C" {

// Whether the GPU path can run here: a HIP device, gfx950, this library's code
// object loaded on it, and the no-alloc scratch's address looked up.
// Records the reason in bfp8_last_error() otherwise.
static int gpu_ready_locked() {
    if (g.gpu_checked) return g.gpu_ok ? BFP8_OK : BFP8_EHIP;
    g.gpu_checked = true;
    if (ensure_init_locked() != BFP8_OK) return BFP8_EHIP;
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, g.device);
    if (e != hipSuccess) {
        set_error("hipGetDeviceProperties: %s", hipGetErrorString(e));
        return BFP8_EHIP;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error("device %d is %s; this library is built for gfx950 only", g.device, prop.gcnArchName);
        return BFP8_EHIP;
    }
    if ((e = bfp8_probe_code_object()) != hipSuccess) {
        set_error("the gfx950 code object does not load: %s", hipGetErrorString(e));
        return BFP8_EHIP;
    }
    void* scratch = nullptr;  // the no-alloc lm_head's device scratch: its address on this device
    if ((e = bfp8_noalloc_setup(&scratch)) != hipSuccess) {
        set_error("hipGetSymbolAddress of the no-alloc scratch: %s", hipGetErrorString(e));
        return BFP8_EHIP;
    }
    g.gpu_ok = true;
    return BFP8_OK;
}

// The reference's init_kernels cannot fail (04/qwen_kernels_opt.c:128-135),
// and the engine calls it inside the try block that picks the library
// (04/qwen_real_engine.py:663-671).  So it never aborts: without a usable GPU
// it leaves the reason in bfp8_last_error() and bfp8_gpu_ready() returns 0,
// which is what an engine checks to keep its own numpy path.
void init_kernels(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (gpu_ready_locked() != BFP8_OK) {
        std::string msg;
        {
            std::lock_guard<std::mutex> el(g_err_mu);
            msg = g_err;
        }
        fprintf(stderr, "libqwen_kernels: init_kernels: GPU path unavailable: %s\n", msg.c_str());
    }
}

int bfp8_gpu_ready(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    return gpu_ready_locked() == BFP8_OK ? 1 : 0;
}

void bfp8_gemv(float* y, const float* x, const int8_t* mantissas, const uint8_t* exps, int M, int K) {
    if (M <= 0) return;
    std::lock_guard<std::mutex> lk(g.mu);
    if (ensure_init_locked() != BFP8_OK || host_gemv(y, x, mantissas, exps, M, K) != BFP8_OK)
        fatal("bfp8_gemv");
}

void bfp8_gemv_batch(float* Y, const float* X, const int8_t* mantissas, const uint8_t* exps, int M, int K,
                     int B) {
    if (M <= 0 || B <= 0) return;
    std::lock_guard<std::mutex> lk(g.mu);
    if (ensure_init_locked() != BFP8_OK) fatal("bfp8_gemv_batch");
    const int nb = bfp8_nblocks(K);
    if (nb == 0 || K > 4096) {  // no batched kernel for these: per-vector calls
        for (int b = 0; b < B; ++b)
            if (host_gemv(Y + (size_t)b * M, X + (size_t)b * K, mantissas, exps, M, K) != BFP8_OK)
                fatal("bfp8_gemv_batch");
        return;
    }
    DevWeights w;
    int rc = weights_for(mantissas, exps, M, K, &w);
    // X rows have stride K; the quantizer reads the first nb*64 of each.
    if (!rc) rc = g.h_in.reserve((size_t)B * nb * 64 * 4);
    if (!rc) rc = g.x.reserve((size_t)B * nb * 64 * 4);
    if (!rc) {
        for (int b = 0; b < B; ++b)
            memcpy(static_cast<float*>(g.h_in.p) + (size_t)b * nb * 64, X + (size_t)b * K, (size_t)nb * 64 * 4);
        if (hipMemcpyAsync(g.x.p, g.h_in.p, (size_t)B * nb * 64 * 4, hipMemcpyHostToDevice, g.stream) !=
            hipSuccess) {
            set_error("hipMemcpyAsync of X failed");
            rc = BFP8_EHIP;
        }
    }
    if (!rc) rc = quantize_ws(K, B);
    if (!rc) rc = g.y.reserve((size_t)B * M * 4);
    if (!rc) rc = g.h_out.reserve((size_t)B * M * 4);
    for (int b0 = 0; !rc && b0 < B; b0 += 16) {
        const int bc = std::min(16, B - b0);
        hipError_t e = bfp8_launch_gemv_batch(g.y.as<float>() + (size_t)b0 * M,
                                              g.xsplit.as<uint32_t>() + (size_t)b0 * nb * 32,
                                              g.xscale.as<float>() + (size_t)b0 * nb, w.mant, w.exps, M, K, bc,
                                              g.stream);
        if (e != hipSuccess) {
            set_error("batched GEMV launch: %s", hipGetErrorString(e));
            rc = BFP8_EHIP;
        }
    }
    for (int b = 0; !rc && b < B && (M & 1); ++b) {
        hipError_t e = bfp8_launch_tail_row(g.y.as<float>() + (size_t)b * M, g.xsplit.as<uint32_t>() + (size_t)b * nb * 32,
                                            g.xscale.as<float>() + (size_t)b * nb, w.mant, w.exps, M, K, g.stream);
        if (e != hipSuccess) {
            set_error("tail row launch: %s", hipGetErrorString(e));
            rc = BFP8_EHIP;
        }
    }
    if (!rc) {
        if (hipMemcpyAsync(g.h_out.p, g.y.p, (size_t)B * M * 4, hipMemcpyDeviceToHost, g.stream) != hipSuccess ||
            hipStreamSynchronize(g.stream) != hipSuccess) {
            set_error("batched GEMV readback failed");
            rc = BFP8_EHIP;
        }
    }
    if (rc) fatal("bfp8_gemv_batch");
    memcpy(Y, g.h_out.p, (size_t)B * M * 4);
}

int bfp8_gemv_fallback(float* y, const float* x, const int8_t* mantissas, const uint8_t* exps, int M, int K,
                       int pairwise) {
    if (M < 0 || K < 0 || (K & 63) || bfp8_nblocks(K) > 16384 || (M > 0 && (!y || (K > 0 && (!x || !mantissas || !exps))))) {
        set_error("bfp8_gemv_fallback: invalid arguments (K must be a multiple of 64)");
        return BFP8_EINVAL;
    }
    if (M == 0) return BFP8_OK;
    std::lock_guard<std::mutex> lk(g.mu);
    int rc;
    if ((rc = ensure_init_locked())) return rc;
    if (K == 0) {  // np.sum over no block: +0.0
        memset(y, 0, (size_t)M * 4);
        return BFP8_OK;
    }
    DevWeights w;
    if ((rc = weights_for(mantissas, exps, M, K, &w)) || (rc = upload_x(x, (size_t)K))) return rc;
    if ((rc = g.y.reserve((size_t)M * 4)) || (rc = g.h_out.reserve((size_t)M * 4))) return rc;
    HIP_OK(bfp8_launch_gemv_fallback(g.y.as<float>(), g.x.as<float>(), w.mant, w.exps, M, K, pairwise ? 1 : 0,
                                     g.stream));
    HIP_OK(hipMemcpyAsync(g.h_out.p, g.y.p, (size_t)M * 4, hipMemcpyDeviceToHost, g.stream));
    HIP_OK(hipStreamSynchronize(g.stream));
    memcpy(y, g.h_out.p, (size_t)M * 4);
    return BFP8_OK;
}

int bfp8_lm_head_topk(const float* h, const int8_t* mantissas, const uint8_t* exps, int vocab, int hidden,
                      int k, int* out_ids, float* out_scores) {
    if (!h || !mantissas || !exps || !out_ids || !out_scores || !lm_head_args_ok(vocab, hidden, k)) return 0;
    std::lock_guard<std::mutex> lk(g.mu);
    if (ensure_init_locked() != BFP8_OK) return 0;
    const int n = host_lm_head(h, mantissas, exps, vocab, hidden, k, out_ids, out_scores, nullptr);
    return n < 0 ? 0 : n;
}

int bfp8_lm_head_argmax(const float* h, const int8_t* mantissas, const uint8_t* exps, int vocab, int hidden) {
    if (!h || !mantissas || !exps || !lm_head_args_ok(vocab, hidden, 1)) return -1;
    std::lock_guard<std::mutex> lk(g.mu);
    if (ensure_init_locked() != BFP8_OK) return -1;
    int am = -1;
    const int n = host_lm_head(h, mantissas, exps, vocab, hidden, 1, nullptr, nullptr, &am);
    return n < 0 ? -1 : am;
}

int lm_head_argmax(const float* h, const uint16_t* embed_table, int vocab_size, int hidden_dim) {
    if (!h || !embed_table || vocab_size <= 0 || hidden_dim <= 0) return 0;
    std::lock_guard<std::mutex> lk(g.mu);
    int am = 0;
    if (ensure_init_locked() != BFP8_OK ||
        host_bf16_lm_head(h, embed_table, vocab_size, hidden_dim, 1, 0, nullptr, nullptr, &am) < 0)
        fatal("lm_head_argmax");
    return am;
}

int qwen_lm_head_topk_bf16(const float* h, const uint16_t* embed_table, int vocab_size, int hidden_dim, int k,
                           int* out_ids, float* out_scores) {
    if (!h || !embed_table || !out_ids || !out_scores || vocab_size <= 0 || hidden_dim <= 0 || k <= 0) return 0;
    if (vocab_size > BFP8_SELECT_MAX) {
        set_error("lm_head_topk: vocab_size %d above %d", vocab_size, BFP8_SELECT_MAX);
        return 0;
    }
    std::lock_guard<std::mutex> lk(g.mu);
    if (ensure_init_locked() != BFP8_OK) return 0;
    const int n = host_bf16_lm_head(h, embed_table, vocab_size, hidden_dim, k, 1, out_ids, out_scores, nullptr);
    return n < 0 ? 0 : n;
}

int qwen_sample_from_topk(const int* ids, const float* scores, int n, float temperature, int top_k, float top_p,
                          unsigned int* rng_state) {
    if (!ids || !scores || n <= 0) return -1;
    if (!rng_state) return ids[0];
    if (n > BFP8_SELECT_MAX) {
        set_error("sample_from_topk: n = %d above %d candidates", n, BFP8_SELECT_MAX);
        return -1;
    }
    std::lock_guard<std::mutex> lk(g.mu);
    if (ensure_init_locked() != BFP8_OK) return -1;
    int rc;
    if ((rc = g.smp_in.reserve((size_t)n * 8 + 4)) || (rc = g.smp_work.reserve((size_t)n * 8)) ||
        (rc = g.smp_out.reserve(8)) || (rc = g.smp_h.reserve((size_t)n * 8 + 8)))
        return -1;
    char* hb = static_cast<char*>(g.smp_h.p);
    memcpy(hb, ids, (size_t)n * 4);
    memcpy(hb + (size_t)n * 4, scores, (size_t)n * 4);
    memcpy(hb + (size_t)n * 8, rng_state, 4);
    Bfp8SampleArgs a{};
    a.ids = g.smp_in.as<int>();
    a.scores = reinterpret_cast<const float*>(g.smp_in.as<char>() + (size_t)n * 4);
    a.rng = reinterpret_cast<uint32_t*>(g.smp_in.as<char>() + (size_t)n * 8);
    a.n = n;
    a.temperature = temperature;
    a.top_k = top_k;
    a.top_p = top_p;
    a.out = g.smp_out.as<int>();
    a.work = g.smp_work.p;
    if (hipMemcpyAsync(g.smp_in.p, hb, (size_t)n * 8 + 4, hipMemcpyHostToDevice, g.stream) != hipSuccess ||
        bfp8_launch_sample(a, g.stream) != hipSuccess ||
        hipMemcpyAsync(hb, g.smp_out.p, 4, hipMemcpyDeviceToHost, g.stream) != hipSuccess ||
        hipMemcpyAsync(hb + 4, a.rng, 4, hipMemcpyDeviceToHost, g.stream) != hipSuccess ||
        hipStreamSynchronize(g.stream) != hipSuccess) {
        set_error("sample_from_topk: the sampler launch failed on the GPU");
        return -1;
    }
    int out;
    memcpy(&out, hb, 4);
    memcpy(rng_state, hb + 4, 4);
    return out;
}

const char* bfp8_last_error(void) {
    static thread_local std::string copy;
    std::lock_guard<std::mutex> lk(g_err_mu);
    copy = g_err;
    return copy.c_str();
}

void bfp8_cache_clear(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (g.ready) (void)hipStreamSynchronize(g.stream);
    forward_cache_clear();
    weights_index_clear();
    for (auto& kv : g.bf16_cache) kv.second.buf.release();
    g.bf16_cache.clear();
    for (auto& kv : g.cache) {
        kv.second.mant.release();
        kv.second.exps.release();
    }
    g.cache.clear();
    g.cache_bytes = 0;
    g.writable.clear();
}

void bfp8_debug_device_limit(size_t bytes) {
    std::lock_guard<std::mutex> lk(g.mu);
    g_dev_limit = bytes;
}

size_t bfp8_device_bytes(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    return g_dev_bytes;
}

void qwen_prof_enable(int on) { g_prof_on = on; }
void qwen_prof_reset(void) {
    for (int i = 0; i < QP_N; i++) g_prof_ms[i] = 0.0;
}
int qwen_prof_count(void) { return QP_N; }
double qwen_prof_get(int i) { return (i >= 0 && i < QP_N) ? g_prof_ms[i] : 0.0; }
const char* qwen_prof_name(int i) { return (i >= 0 && i < QP_N) ? kProfNames[i] : "?"; }

// ---- device level ------------------------------------------------------------------------
size_t bfp8_dev_mant_bytes(int M, int K) { return bfp8_gpu_mant_bytes(M, K); }
size_t bfp8_dev_exps_bytes(int M, int K) { return bfp8_gpu_exps_bytes(M, K); }
size_t bfp8_dev_xsplit_bytes(int K) { return bfp8_xsplit_bytes(K); }

void* bfp8_stream(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (ensure_init_locked() != BFP8_OK) return nullptr;
    return g.stream;
}

#define DEV_PROLOGUE()                                                 \
    do {                                                               \
        std::lock_guard<std::mutex> lk_(g.mu);                         \
        if (ensure_init_locked() != BFP8_OK) return BFP8_EHIP;         \
    } while (0)

int bfp8_dev_pack(int8_t* mant_gpu, uint8_t* exps_gpu, const int8_t* mant_soa, const uint8_t* exps_soa, int M,
                  int K, void* stream) {
    if (M < 0 || K < 0 || (M > 0 && bfp8_nblocks(K) > 0 && (!mant_gpu || !exps_gpu || !mant_soa || !exps_soa)))
        return BFP8_EINVAL;
    DEV_PROLOGUE();
    HIP_OK(bfp8_launch_pack((uint8_t*)mant_gpu, exps_gpu, mant_soa, exps_soa, M, K, pick_stream(stream)));
    return BFP8_OK;
}

int bfp8_dev_unpack(int8_t* mant_soa, uint8_t* exps_soa, const int8_t* mant_gpu, const uint8_t* exps_gpu, int M,
                    int K, void* stream) {
    if (M < 0 || K < 0) return BFP8_EINVAL;
    DEV_PROLOGUE();
    HIP_OK(bfp8_launch_unpack(mant_soa, exps_soa, (const uint8_t*)mant_gpu, exps_gpu, M, K, pick_stream(stream)));
    return BFP8_OK;
}

int bfp8_dev_quantize(int16_t* xq, float* xscale, uint32_t* xsplit, const float* x, int K, void* stream) {
    if (K < 0 || K > 4096 || (bfp8_nblocks(K) > 0 && (!xscale || !xsplit || !x))) return BFP8_EINVAL;
    DEV_PROLOGUE();
    Bfp8QuantDesc q{};
    q.x = x;
    q.xq = xq;
    q.xscale = xscale;
    q.xsplit = xsplit;
    q.K = K;
    HIP_OK(bfp8_launch_quantize1(q, pick_stream(stream)));
    return BFP8_OK;
}

int bfp8_dev_gemv(float* y, const uint32_t* xsplit, const float* xscale, const int8_t* mant_gpu,
                  const uint8_t* exps_gpu, int M, int K, int32_t* lane_sums, void* stream) {
    if (M < 0 || K < 0 || K > 4096) return BFP8_EINVAL;
    if (M == 0) return BFP8_OK;
    if (!y || (bfp8_nblocks(K) > 0 && (!xsplit || !xscale || !mant_gpu || !exps_gpu))) return BFP8_EINVAL;
    DEV_PROLOGUE();
    hipStream_t s = pick_stream(stream);
    if (bfp8_nblocks(K) == 0) {
        HIP_OK(hipMemsetAsync(y, 0, (size_t)M * 4, s));
        return BFP8_OK;
    }
    return gemv_q(y, xsplit, xscale, (const uint8_t*)mant_gpu, exps_gpu, M, K, lane_sums, s);
}

int bfp8_dev_gemv_float(float* y, const float* x, const int8_t* mant_gpu, const uint8_t* exps_gpu, int M, int K,
                        void* stream) {
    if (M < 0 || K < 0 || bfp8_nblocks(K) > 16384) return BFP8_EINVAL;
    if (M == 0) return BFP8_OK;
    DEV_PROLOGUE();
    HIP_OK(bfp8_launch_gemv_float(y, x, (const uint8_t*)mant_gpu, exps_gpu, M, K, pick_stream(stream)));
    return BFP8_OK;
}

int bfp8_dev_gemv_fallback(float* y, const float* x, const int8_t* mant_gpu, const uint8_t* exps_gpu, int M, int K,
                           int pairwise, void* stream) {
    if (M < 0 || K < 0 || (K & 63) || bfp8_nblocks(K) > 16384 || (M > 0 && (!y || (K > 0 && (!x || !mant_gpu || !exps_gpu)))))
        return BFP8_EINVAL;
    if (M == 0) return BFP8_OK;
    DEV_PROLOGUE();
    HIP_OK(bfp8_launch_gemv_fallback(y, x, (const uint8_t*)mant_gpu, exps_gpu, M, K, pairwise ? 1 : 0,
                                     pick_stream(stream)));
    return BFP8_OK;
}

int bfp8_dev_gemv_batch(float* Y, const uint32_t* xsplit, const float* xscale, const int8_t* mant_gpu,
                        const uint8_t* exps_gpu, int M, int K, int B, void* stream) {
    if (M < 0 || K < 64 || K > 4096 || B < 1 || B > 16) return BFP8_EINVAL;
    if (M == 0) return BFP8_OK;
    DEV_PROLOGUE();
    hipStream_t s = pick_stream(stream);
    const int nb = bfp8_nblocks(K);
    HIP_OK(bfp8_launch_gemv_batch(Y, xsplit, xscale, (const uint8_t*)mant_gpu, exps_gpu, M, K, B, s));
    if (M & 1)
        for (int b = 0; b < B; ++b)
            HIP_OK(bfp8_launch_tail_row(Y + (size_t)b * M, xsplit + (size_t)b * nb * 32, xscale + (size_t)b * nb,
                                        (const uint8_t*)mant_gpu, exps_gpu, M, K, s));
    return BFP8_OK;
}

int bfp8_dev_lm_head_topk(int* out_ids, float* out_scores, int* out_count, int* out_argmax,
                          const uint32_t* xsplit, const float* xscale, const int8_t* mant_gpu,
                          const uint8_t* exps_gpu, int vocab, int hidden, int k, void* stream) {
    if (!lm_head_args_ok(vocab, hidden, k) || hidden > 4096 || !out_ids || !out_scores || !out_count ||
        !out_argmax || (bfp8_nblocks(hidden) > 0 && (!xsplit || !xscale || !mant_gpu || !exps_gpu)))
        return BFP8_EINVAL;
    std::lock_guard<std::mutex> lk(g.mu);
    if (ensure_init_locked() != BFP8_OK) return BFP8_EHIP;
    return lm_head_dev(out_ids, out_scores, out_count, out_argmax, xsplit, xscale, (const uint8_t*)mant_gpu,
                       exps_gpu, vocab, hidden, k, pick_stream(stream));
}

int bfp8_dev_lm_head_topk_noalloc(int* out_ids, float* out_scores, int* out_count, int* out_argmax,
                                  const uint32_t* xsplit, const float* xscale, const int8_t* mant_gpu,
                                  const uint8_t* exps_gpu, int vocab, int hidden, int k, void* stream) {
    if (vocab <= 0 || hidden < 64 || hidden > 4096 || k < 1 || !out_ids || !out_scores || !out_count ||
        !out_argmax || !xsplit || !xscale || !mant_gpu || !exps_gpu) {
        set_error("bfp8_dev_lm_head_topk_noalloc: invalid arguments");
        return BFP8_EINVAL;
    }
    if (vocab > BFP8_NOALLOC_MAX_VOCAB) {
        set_error("bfp8_dev_lm_head_topk_noalloc: vocab %d above the scratch's %d rows", vocab,
                  BFP8_NOALLOC_MAX_VOCAB);
        return BFP8_EINVAL;
    }
    std::lock_guard<std::mutex> lk(g.mu);
    void* base = nullptr;
    HIP_OK(bfp8_noalloc_setup(&base));
    uint64_t* partials = static_cast<uint64_t*>(base);
    float* logits = reinterpret_cast<float*>(static_cast<char*>(base) + BFP8_NOALLOC_PARTIALS_BYTES);
    uint64_t* keys = reinterpret_cast<uint64_t*>(static_cast<char*>(base) + BFP8_NOALLOC_PARTIALS_BYTES +
                                                 BFP8_NOALLOC_LOGITS_BYTES);
    hipStream_t s = pick_stream(stream);
    const uint8_t* m = (const uint8_t*)mant_gpu;
    const int kk = std::min(k, vocab);
    if (lm_head_fused_ok(vocab, hidden, kk)) {
        Bfp8GemvDesc d = plain_desc(nullptr, xsplit, xscale, m, exps_gpu, vocab, hidden, nullptr);
        d.topk = kk;
        d.partials = partials;
        d.out_ids = out_ids;
        d.out_scores = out_scores;
        d.out_count = out_count;
        d.out_argmax = out_argmax;
        HIP_OK(bfp8_launch_gemv(d, s));
        return BFP8_OK;
    }
    int rc = gemv_q(logits, xsplit, xscale, m, exps_gpu, vocab, hidden, nullptr, s);
    return rc ? rc : select_topk_raw(logits, vocab, kk, out_ids, out_scores, out_count, out_argmax, partials, keys, s);
}

int bfp8_dev_synth_planes(int8_t* mant_soa, uint8_t* exps_soa, int M, int K, uint64_t seed, int e_lo, int e_hi,
                          void* stream) {
    if (M < 0 || K < 0 || e_lo < 0 || e_hi > 255 || e_lo > e_hi) return BFP8_EINVAL;
    DEV_PROLOGUE();
    HIP_OK(bfp8_launch_synth_planes(mant_soa, exps_soa, M, K, seed, e_lo, e_hi, pick_stream(stream)));
    return BFP8_OK;
}

void bfp8_synth_planes_host(int8_t* mant_soa, uint8_t* exps_soa, int M, int K, uint64_t seed, int e_lo, int e_hi) {
    const size_t nm = (size_t)M * K, ne = (size_t)M * bfp8_nblocks(K);
    for (size_t i = 0; i < nm; ++i) mant_soa[i] = bfp8_synth_mant(seed, i);
    for (size_t i = 0; i < ne; ++i) exps_soa[i] = bfp8_synth_exp(seed, i, e_lo, e_hi);
}

void bfp8_synth_normal(float* out, int n, uint64_t seed) {
    for (int i = 0; i < n; ++i) out[i] = (float)normal_at(seed, (uint64_t)i);
}

void bfp8_synth_swiglu(float* out, int n, uint64_t seed, double outlier_frac, float mag) {
    for (int i = 0; i < n; ++i) {
        const double a = normal_at(seed, (uint64_t)i);
        const double b = normal_at(seed ^ 0x5DEECE66Dull, (uint64_t)i);
        double v = a / (1.0 + std::exp(-a)) * b;
        const uint64_t h = bfp8_hash64(seed ^ 0xA5A5A5A5A5A5A5A5ull, (uint64_t)i);
        if (unit53(h) < outlier_frac) v = (h & 1) ? (double)mag : -(double)mag;
        out[i] = (float)v;
    }
}

int bfp8_dev_read_probe(const void* buf, size_t bytes, uint32_t* out, void* stream) {
    DEV_PROLOGUE();
    HIP_OK(bfp8_launch_read_probe(buf, bytes, out, pick_stream(stream)));
    return BFP8_OK;
}

int bfp8_dev_copy_probe(void* dst, const void* src, size_t bytes, void* stream) {
    DEV_PROLOGUE();
    HIP_OK(bfp8_launch_copy_probe(dst, src, bytes, pick_stream(stream)));
    return BFP8_OK;
}

int bf16_dev_lm_head(int* out_ids, float* out_scores, int* out_count, int* out_argmax, float* logits,
                     const float* h, const uint16_t* table, int vocab, int hidden, int k, int tail, void* stream) {
    DEV_PROLOGUE();
    if (!h || !table || vocab <= 0 || vocab > BFP8_SELECT_MAX || hidden <= 0 || k < 0 ||
        (k > 0 && (!out_ids || !out_scores || !out_count || !out_argmax)) || (k == 0 && !logits)) {
        set_error("bf16_dev_lm_head: invalid arguments");
        return BFP8_EINVAL;
    }
    return bf16_lm_head_dev(out_ids, out_scores, out_count, out_argmax, logits, h, table, 0, vocab, hidden, k,
                            tail ? 1 : 0, pick_stream(stream));
}

size_t bf16_dev_tiles_bytes(int vocab, int hidden) {
    if (vocab <= 0 || !bf16_tiled_ok(hidden)) return 0;
    return bf16_tiled_elems(vocab, hidden) * 2;
}

int bf16_dev_tile_table(uint16_t* tiles, const uint16_t* table, int vocab, int hidden, void* stream) {
    DEV_PROLOGUE();
    if (!tiles || !table || vocab <= 0 || !bf16_tiled_ok(hidden)) {
        set_error("bf16_dev_tile_table: invalid arguments (hidden must be 1024)");
        return BFP8_EINVAL;
    }
    HIP_OK(bf16_launch_tile_table(tiles, table, vocab, hidden, pick_stream(stream)));
    return BFP8_OK;
}

int bf16_dev_lm_head_tiles(int* out_ids, float* out_scores, int* out_count, int* out_argmax, float* logits,
                           const float* h, const uint16_t* tiles, int vocab, int hidden, int k, void* stream) {
    DEV_PROLOGUE();
    if (!h || !tiles || vocab <= 0 || vocab > BFP8_SELECT_MAX || !bf16_tiled_ok(hidden) || k < 0 ||
        (k > 0 && (!out_ids || !out_scores || !out_count || !out_argmax)) || (k == 0 && !logits)) {
        set_error("bf16_dev_lm_head_tiles: invalid arguments");
        return BFP8_EINVAL;
    }
    return bf16_lm_head_dev(out_ids, out_scores, out_count, out_argmax, logits, h, tiles, 1, vocab, hidden, k, 0,
                            pick_stream(stream));
}

int bfp8_dev_sample_from_topk(int* out_id, const int* ids, const float* scores, const int* count, int n,
                              float temperature, int top_k, float top_p, uint32_t* rng_state, void* work,
                              void* stream) {
    DEV_PROLOGUE();
    if (!out_id || !ids || !scores || n <= 0 || n > BFP8_SELECT_MAX || !work) {
        set_error("bfp8_dev_sample_from_topk: invalid arguments");
        return BFP8_EINVAL;
    }
    Bfp8SampleArgs a{};
    a.ids = ids;
    a.scores = scores;
    a.count = count;
    a.n = n;
    a.temperature = temperature;
    a.top_k = top_k;
    a.top_p = top_p;
    a.rng = rng_state;
    a.out = out_id;
    a.work = work;
    HIP_OK(bfp8_launch_sample(a, pick_stream(stream)));
    return BFP8_OK;
}

}  // extern "C"

// =========================== plans ================================================
namespace qhost {

struct Plan {
    std::vector<bfp8_plan_item> items;
    std::vector<int> odd_items;    // items needing the odd-row kernel
    std::vector<int> float_items;  // K > 4096 items (float path, own launches)
    DevBuf descs, qdescs, xscale, xsplit, partials;
    DevBuf qtasks;                 // fused head: Bfp8HeadTask per block of the other activations
    Launch head, rest;             // lm_head tiles, then every other GEMV's
    int nq = 0, max_nb = 0, ntasks = 0;
    bool fused_head = false;       // the lm_head launch quantizes every activation
    bool rows_float = false;       // the 16-row launch quantizes its (shared) activation
    int topk_desc = -1;            // the lm_head item, if any
    // an lm_head item outside the fused launch's range (odd vocab, k > 64,
    // K > 4096) runs as a plain GEMV into `logits`, selected at the end
    int gen_head = -1;
    bfp8_plan_item gen_out{};      // its outputs and k
    DevBuf logits, gen_partials, gen_keys;
    std::vector<Bfp8GemvDesc> hdesc;
    // single launch (sweep.hip): the whole plan, a tile queue, activations quantized in LDS
    bool sweep = false;
    DevBuf s_gemvs, s_counters;
    int s_nwg = 0, s_ngemv = 0, s_nunits = 0;
    uint32_t s_launches = 0;       // of the single launch: its counter set is s_launches % 2
    uint32_t epoch = 0;            // of the last launch; the partials start zeroed (epoch 0)
};

// Sub-queues of a single launch on nwg workgroups: each is shared by the
// workgroups (w / 8) mod n = s, so that n divides nwg / 8 evenly (every
// sub-queue the same number of workgroups, from every XCD) -- at most
// BFP8_SWEEP_QUEUES, at least two groups of 8 per sub-queue.
int sweep_queues(int nwg) {
    const int groups = nwg / 8;
    int best = 1;
    for (int n = 1; n <= BFP8_SWEEP_QUEUES && 2 * n <= groups; ++n)
        if (groups % n == 0) best = n;
    return best;
}

// A unit of the single launch has an even number of 4-block chunks.
bool sweep_nb_ok(int K) {
    const int nb = bfp8_nblocks(K);
    return (K & 63) == 0 && nb >= BFP8_SWEEP_MIN_NB && nb <= 64 && nb % 8 == 0;
}

// The single launch (sweep.hip) for a plan whose every GEMV fits it: even M,
// whole units (sweep_nb_ok), 1 .. BFP8_SWEEP_MAX_GEMV GEMVs besides a fused
// lm_head.  Builds the queue table -- the GEMVs with the most blocks
// first, each GEMV's tiles consecutive -- and the zeroed ticket counters.
// Returns false (the plan keeps its launches) when the plan does not fit.
bool build_sweep(Plan* p, const bfp8_plan_item* items, int n) {
    const int head = p->topk_desc;
    if (!p->odd_items.empty() || !p->float_items.empty() || p->gen_head >= 0) return false;
    std::vector<int> rest;
    int total_tiles = 0;
    for (int i = 0; i < n; ++i) {
        if (!sweep_nb_ok(items[i].K) || (items[i].M & 1)) return false;
        total_tiles += bfp8_ntiles(items[i].M);
        if (i != head) rest.push_back(i);
    }
    // a lone lm_head takes the two launches (per-tile lists, then the merge
    // kernel): its scoring ends long before one workgroup's merge of every
    // list could
    if (rest.empty() || (int)rest.size() > BFP8_SWEEP_MAX_GEMV) return false;
    if (head < 0 && total_tiles <= BFP8_WIDE_MAX_TILES) return false;  // (small plans: one tile per workgroup)
    std::stable_sort(rest.begin(), rest.end(), [&](int a, int b) { return items[a].K > items[b].K; });
    std::vector<Bfp8SweepGemv> tab;
    int first = 0;
    for (int i : rest) {
        const bfp8_plan_item& it = items[i];
        Bfp8SweepGemv g{};
        g.mant = (const uint8_t*)it.mant_gpu;
        g.exps = it.exps_gpu;
        g.x = it.x;
        g.y = it.y;
        g.nb = bfp8_nblocks(it.K);
        g.pair_rows = it.M & ~1;
        g.first = first;
        g.ntiles = bfp8_ntiles(it.M);
        first += g.ntiles;
        tab.push_back(g);
    }
    const int grid = bfp8_sweep_grid(BFP8_SWEEP_WG_PER_CU);
    p->s_nwg = head >= 0 ? grid : std::min(grid, first);
    p->s_ngemv = (int)tab.size();
    p->s_nunits = first;

    if (p->s_gemvs.reserve(tab.size() * sizeof(Bfp8SweepGemv)) || p->s_counters.reserve(BFP8_SWEEP_CTR_BYTES))
        return false;
    if (hipMemcpy(p->s_gemvs.p, tab.data(), tab.size() * sizeof(Bfp8SweepGemv), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(p->s_counters.p, 0, BFP8_SWEEP_CTR_BYTES) != hipSuccess)
        return false;
    return true;
}

// Deals the tiles of `idx` (in that order) over at most bfp8_stream_grid()
// workgroups, longest first onto the least-loaded workgroup (bytes), and
// uploads the table.  `wg0_extra` blocks of load are pre-charged to
// workgroup 0 (a folded merge).
int deal_tiles(Launch& L, const std::vector<int>& idx, const bfp8_plan_item* items, int wg0_extra, bool allow_wide) {
    std::vector<Bfp8TileRef> order;
    for (int i : idx) {
        for (int t = 0; t < bfp8_ntiles(items[i].M); ++t) order.push_back(Bfp8TileRef{i, t});
        L.max_nb = std::max(L.max_nb, bfp8_nblocks(items[i].K));
    }
    if (order.empty()) return BFP8_OK;
    L.ntiles = (int)order.size();
    if (allow_wide && L.ntiles <= BFP8_WIDE_MAX_TILES) {
        L.wide = true;
        int rc;
        if ((rc = L.tiles.reserve(order.size() * sizeof(Bfp8TileRef)))) return rc;
        HIP_OK(hipMemcpy(L.tiles.p, order.data(), order.size() * sizeof(Bfp8TileRef), hipMemcpyHostToDevice));
        return BFP8_OK;
    }
    const int nwg = std::min<int>((int)order.size(), bfp8_stream_grid());
    std::vector<std::vector<Bfp8TileRef>> per(nwg);
    using Load = std::pair<long long, int>;
    std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
    for (int w = 0; w < nwg; ++w) heap.push({w == 0 ? (long long)wg0_extra * 4160 : 0LL, w});
    for (const Bfp8TileRef& tr : order) {
        Load l = heap.top();
        heap.pop();
        per[l.second].push_back(tr);
        l.first += (long long)bfp8_nblocks(items[tr.desc].K) * 4160;
        heap.push(l);
    }
    std::vector<Bfp8TileRef> tiles;
    std::vector<int> wg_off(1, 0);
    for (const auto& v : per) {
        tiles.insert(tiles.end(), v.begin(), v.end());
        wg_off.push_back((int)tiles.size());
    }
    int rc;
    if ((rc = L.tiles.reserve(tiles.size() * sizeof(Bfp8TileRef))) || (rc = L.wg_off.reserve(wg_off.size() * sizeof(int))))
        return rc;
    HIP_OK(hipMemcpy(L.tiles.p, tiles.data(), tiles.size() * sizeof(Bfp8TileRef), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(L.wg_off.p, wg_off.data(), wg_off.size() * sizeof(int), hipMemcpyHostToDevice));
    L.nwg = nwg;
    return BFP8_OK;
}

void release_plan(Plan* p) {
    p->descs.release(); p->qdescs.release(); p->xscale.release(); p->xsplit.release();
    p->partials.release(); p->qtasks.release();
    p->logits.release(); p->gen_partials.release(); p->gen_keys.release();
    p->s_gemvs.release(); p->s_counters.release();
    p->head.tiles.release(); p->head.wg_off.release(); p->rest.tiles.release(); p->rest.wg_off.release();
}

}  // namespace qhost

extern "C" {

void* bfp8_plan_create(const bfp8_plan_item* items, int n) {
    if (!items || n <= 0) {
        set_error("bfp8_plan_create: no items");
        return nullptr;
    }
    {
        std::lock_guard<std::mutex> lk(g.mu);
        if (ensure_init_locked() != BFP8_OK) return nullptr;
    }
    Plan* p = new Plan();
    p->items.assign(items, items + n);
    int ntopk = 0;
    size_t xs_words = 0, xsc_floats = 0;
    int rc = 0;
    for (int i = 0; i < n; ++i) {
        const bfp8_plan_item& it = items[i];
        if (it.M <= 0 || it.K < 64 || !it.x || !it.mant_gpu || !it.exps_gpu ||
            (it.topk > 0 && (!lm_head_args_ok(it.M, it.K, it.topk) || !it.out_ids || !it.out_scores ||
                             !it.out_count || !it.out_argmax)) ||
            (it.topk <= 0 && !it.y)) {
            set_error("bfp8_plan_create: invalid item %d", i);
            delete p;
            return nullptr;
        }
        ntopk += it.topk > 0;
        if (it.topk > 0 && !lm_head_fused_ok(it.M, it.K, std::min(it.topk, it.M))) {
            // the general path: a plain GEMV item into the plan's scores buffer
            const int kk = std::min(it.topk, it.M);
            p->gen_head = i;
            p->gen_out = it;
            p->gen_out.topk = kk;
            rc = rc ? rc : p->logits.reserve((size_t)it.M * 4);
            if (kk <= BFP8_TOPK_MAX)
                rc = rc ? rc : p->gen_partials.reserve((size_t)bfp8_ntiles(it.M) * kk * 8);
            else
                rc = rc ? rc : p->gen_keys.reserve(bfp8_select_scratch_bytes(it.M));
            p->items[i].topk = 0;
            p->items[i].y = p->logits.as<float>();
        }
        const int nb = bfp8_nblocks(it.K);
        if (it.K <= 4096) {
            xs_words += (size_t)nb * 32;
            xsc_floats += nb;
            p->max_nb = std::max(p->max_nb, nb);
        }
    }
    if (ntopk > 1 || rc) {
        set_error(rc ? "bfp8_plan_create: allocation failed" : "bfp8_plan_create: at most one lm_head item");
        release_plan(p);
        delete p;
        return nullptr;
    }
    items = p->items.data();  // the general lm_head, if any, is a plain item from here on
    rc = rc ? rc : p->xsplit.reserve(xs_words * 4);
    rc = rc ? rc : p->xscale.reserve(xsc_floats * 4);
    std::vector<Bfp8QuantDesc> hq;
    std::vector<int> hq_of_item(n, -1);
    size_t ow = 0, of = 0;
    for (int i = 0; i < n && !rc; ++i) {
        const bfp8_plan_item& it = items[i];
        Bfp8GemvDesc d{};
        if (it.K > 4096) {
            p->float_items.push_back(i);
            p->hdesc.push_back(d);
            continue;
        }
        const int nb = bfp8_nblocks(it.K);
        Bfp8QuantDesc q{};
        q.x = it.x;
        q.xq = nullptr;  // no plan kernel reads the int16 values (the tail rows read the split form)
        q.xscale = p->xscale.as<float>() + of;
        q.xsplit = p->xsplit.as<uint32_t>() + ow;
        q.K = it.K;
        hq_of_item[i] = (int)hq.size();
        hq.push_back(q);
        d = plain_desc(it.y, q.xsplit, q.xscale, (const uint8_t*)it.mant_gpu, it.exps_gpu, it.M, it.K, nullptr);
        if (it.topk > 0) {
            d.topk = std::min(it.topk, it.M);
            rc = rc ? rc : p->partials.reserve((size_t)bfp8_ntiles(it.M) * d.topk * 8);
            d.partials = p->partials.as<uint64_t>();
            d.out_ids = it.out_ids;
            d.out_scores = it.out_scores;
            d.out_count = it.out_count;
            d.out_argmax = it.out_argmax;
            p->topk_desc = (int)p->hdesc.size();
        }
        if ((it.M & 1) && it.topk <= 0) p->odd_items.push_back(i);
        p->hdesc.push_back(d);
        ow += (size_t)nb * 32;
        of += nb;
    }
    // Two persistent launches: the lm_head's tiles, then every other GEMV's
    // (larger K first).  Workgroup 0 of the second launch merges the lm_head's
    // top-k partials before its own tiles (the launch boundary makes them
    // visible); without other GEMVs the stand-alone merge kernel runs instead.
    std::vector<int> head_idx, rest_idx;
    for (int i = 0; i < n; ++i) {
        if (items[i].K > 4096) continue;
        (items[i].topk > 0 ? head_idx : rest_idx).push_back(i);
    }
    std::stable_sort(rest_idx.begin(), rest_idx.end(), [&](int a, int b) { return items[a].K > items[b].K; });
    const bool fold = p->topk_desc >= 0 && !rest_idx.empty();
    rc = rc ? rc : deal_tiles(p->head, head_idx, items, 0, false);
    // one GEMV, or two reading the same activation: 16 rows per workgroup
    const bool rows = !fold && !rest_idx.empty() && rest_idx.size() <= 2 &&
                      (rest_idx.size() == 1 || (items[rest_idx[0]].x == items[rest_idx[1]].x &&
                                                items[rest_idx[0]].K == items[rest_idx[1]].K));
    if (rows) {
        // the launch quantizes the shared x itself; its workgroup 0 leaves the
        // records in the first item's slots, which both items' tail rows read
        for (size_t i = 0; i < rest_idx.size(); ++i) p->rest.rows[i] = rest_idx[i];
        p->rows_float = true;
        for (size_t i = 1; i < rest_idx.size(); ++i) {
            p->hdesc[rest_idx[i]].xsplit = p->hdesc[rest_idx[0]].xsplit;
            p->hdesc[rest_idx[i]].xscale = p->hdesc[rest_idx[0]].xscale;
        }
    } else
        rc = rc ? rc : deal_tiles(p->rest, rest_idx, items, fold ? BFP8_MERGE_COST_BLOCKS : 0, !fold);
    p->nq = (int)hq.size();
    // An lm_head of K <= 1024 (whole blocks) quantizes in its own launch: its
    // own activation per workgroup, every other one block per wavefront task.
    if (p->topk_desc >= 0 && !rc) {
        const bfp8_plan_item& ht = items[p->topk_desc];
        if ((ht.K & 63) == 0 && (ht.K >> 6) <= BFP8_HEAD_MAX_NB && p->head.nwg > 0) {
            std::vector<Bfp8HeadTask> tasks;
            auto task = [&](int qi, int b) {
                Bfp8HeadTask t{};
                t.x = hq[qi].x + (size_t)b * 64;
                t.xq = hq[qi].xq;
                t.xscale = hq[qi].xscale;
                t.xsplit = hq[qi].xsplit;
                t.b = b;
                return t;
            };
            for (int qi = 0; qi < (int)hq.size(); ++qi) {
                if (qi == hq_of_item[p->topk_desc]) continue;  // quantized by every workgroup
                for (int b = 0; b < bfp8_nblocks(hq[qi].K); ++b) tasks.push_back(task(qi, b));
            }
            p->ntasks = (int)tasks.size();
            if (tasks.empty()) tasks.push_back(task(hq_of_item[p->topk_desc], 0));  // the kernel always reads one entry
            {
                rc = p->qtasks.reserve(tasks.size() * sizeof(Bfp8HeadTask));
                if (!rc && hipMemcpy(p->qtasks.p, tasks.data(), tasks.size() * sizeof(Bfp8HeadTask),
                                     hipMemcpyHostToDevice) != hipSuccess)
                    rc = BFP8_EHIP;
            }
            p->fused_head = !rc;
        }
    }
    // one launch for the whole plan when every GEMV fits it (build_sweep)
    if (!rc) {
        p->sweep = build_sweep(p, items, n);
        if (p->sweep && p->topk_desc >= 0 &&
            hipMemset(p->partials.p, 0, p->partials.n) != hipSuccess)  // epoch 0: never a run's
            rc = BFP8_EHIP;
    }
    rc = rc ? rc : p->descs.reserve(p->hdesc.size() * sizeof(Bfp8GemvDesc));
    rc = rc ? rc : p->qdescs.reserve(hq.size() * sizeof(Bfp8QuantDesc));
    if (!rc && (hipMemcpy(p->descs.p, p->hdesc.data(), p->hdesc.size() * sizeof(Bfp8GemvDesc), hipMemcpyHostToDevice) != hipSuccess ||
                (!hq.empty() && hipMemcpy(p->qdescs.p, hq.data(), hq.size() * sizeof(Bfp8QuantDesc), hipMemcpyHostToDevice) != hipSuccess)))
        rc = BFP8_EHIP;
    if (rc) {
        set_error("bfp8_plan_create: allocation or upload failed (%d)", rc);
        release_plan(p);
        delete p;
        return nullptr;
    }
    return p;
}

int bfp8_plan_quantize(void* plan, void* stream) {
    Plan* p = static_cast<Plan*>(plan);
    if (!p) return BFP8_EINVAL;
    HIP_OK(bfp8_launch_quantize(p->qdescs.as<Bfp8QuantDesc>(), p->nq, p->max_nb, pick_stream(stream)));
    return BFP8_OK;
}

int bfp8_plan_launch(void* plan, int stage, void* stream) {
    Plan* p = static_cast<Plan*>(plan);
    if (!p || stage < 0 || stage > 2) return BFP8_EINVAL;
    hipStream_t s = pick_stream(stream);
    const Bfp8GemvDesc* descs = p->descs.as<Bfp8GemvDesc>();
    const bool fold = p->topk_desc >= 0 && p->rest.nwg > 0;
    if (p->sweep) {  // everything in stage 0
        if (stage != 0) return BFP8_OK;
        Bfp8SweepArgs a{};
        a.gemvs = p->s_gemvs.as<Bfp8SweepGemv>();
        a.ngemv = p->s_ngemv;
        a.nunits = p->s_nunits;
        {
            uint32_t* sets = p->s_counters.as<uint32_t>();
            const int cur = (int)(p->s_launches & 1u);  // counted below once the launch is made
            a.counters = sets + cur * BFP8_SWEEP_QUEUES * BFP8_SWEEP_CTR_STRIDE;
            a.counters_next = sets + (1 - cur) * BFP8_SWEEP_QUEUES * BFP8_SWEEP_CTR_STRIDE;
        }
        a.nqueues = sweep_queues(p->s_nwg);
        if (p->topk_desc >= 0) {
            const Bfp8GemvDesc& hd = p->hdesc[p->topk_desc];
            const bfp8_plan_item& it = p->items[p->topk_desc];
            a.head_mant = hd.mant;
            a.head_exps = hd.exps;
            a.head_x = it.x;
            a.head_nb = bfp8_nblocks(hd.K);
            a.head_ntiles = bfp8_ntiles(hd.M);
            a.head_pair_rows = hd.pair_rows;
            a.topk = hd.topk;
            a.partials = hd.partials;
            a.out_ids = hd.out_ids;
            a.out_scores = hd.out_scores;
            a.out_count = hd.out_count;
            a.out_argmax = hd.out_argmax;
            a.ticket0 = 0;
        } else {
            a.ticket0 = p->s_nwg;  // queue units 0 .. nwg - 1 are the workgroups' first
        }
        p->epoch = p->epoch % 16383u + 1u;
        a.epoch = p->epoch;
        HIP_OK(bfp8_launch_sweep(a, p->s_nwg, s));
        ++p->s_launches;
        return BFP8_OK;
    }
    if (stage == 0) {
        if (p->fused_head) {
            const Bfp8GemvDesc& hd = p->hdesc[p->topk_desc];
            Bfp8HeadArgs a{};
            a.descs = descs;
            a.head = p->topk_desc;
            a.mant = hd.mant;
            a.exps = hd.exps;
            a.K = hd.K;
            a.ntiles = p->head.ntiles;
            a.hx = p->items[p->topk_desc].x;
            a.qtasks = p->qtasks.as<Bfp8HeadTask>();
            a.ntasks = p->ntasks;
            HIP_OK(bfp8_launch_gemv_head(a, p->head.nwg, s));
        } else
            HIP_OK(bfp8_launch_gemv_grouped(descs, p->head.tiles.as<Bfp8TileRef>(), p->head.wg_off.as<int>(),
                                            p->head.nwg, -1, s));
    } else if (stage == 1) {
        if (p->rest.rows[0] >= 0) {
            RtRowsArgs a{};
            for (int i = 0; i < 2 && p->rest.rows[i] >= 0; ++i) {
                const Bfp8GemvDesc& d = p->hdesc[p->rest.rows[i]];
                a.g[i].mant = d.mant;
                a.g[i].exps = d.exps;
                a.g[i].y = d.y;
                a.g[i].M = d.M;
                a.g[i].pair_rows = d.pair_rows;
                a.ngemv = i + 1;
            }
            const Bfp8GemvDesc& d0 = p->hdesc[p->rest.rows[0]];
            a.split = (d0.M + 15) / 16;
            a.K = d0.K;
            a.mode = RT_ROWS_FLOAT;
            a.x = p->items[p->rest.rows[0]].x;
            a.xsplit_out = const_cast<uint32_t*>(d0.xsplit);
            a.xscale_out = const_cast<float*>(d0.xscale);
            HIP_OK(rt_launch_rows(a, s));
        } else if (p->rest.wide)
            HIP_OK(bfp8_launch_gemv_wide_grouped(descs, p->rest.tiles.as<Bfp8TileRef>(), p->rest.ntiles,
                                                 p->rest.max_nb, s));
        else
            HIP_OK(bfp8_launch_gemv_grouped(descs, p->rest.tiles.as<Bfp8TileRef>(), p->rest.wg_off.as<int>(),
                                            p->rest.nwg, fold ? p->topk_desc : -1, s));
        if (p->topk_desc >= 0 && !fold) HIP_OK(bfp8_launch_topk_merge(p->hdesc[p->topk_desc], s));
    } else {
        for (int i : p->odd_items) {
            const Bfp8GemvDesc& d = p->hdesc[i];
            HIP_OK(bfp8_launch_tail_row(d.y, d.xsplit, d.xscale, d.mant, d.exps, d.M, d.K, s));
        }
        for (int i : p->float_items) {
            const bfp8_plan_item& it = p->items[i];
            HIP_OK(bfp8_launch_gemv_float(it.y, it.x, (const uint8_t*)it.mant_gpu, it.exps_gpu, it.M, it.K, s));
        }
        if (p->gen_head >= 0) {
            const bfp8_plan_item& o = p->gen_out;
            return select_topk_bufs(p->logits.as<float>(), o.M, o.topk, o.out_ids, o.out_scores, o.out_count,
                                    o.out_argmax, p->gen_partials, p->gen_keys, s);
        }
    }
    return BFP8_OK;
}

const char* bfp8_plan_kernel_name(void* plan, int stage) {
    const Plan* p = static_cast<const Plan*>(plan);
    if (!p) return "";
    if (p->sweep) return stage == 0 ? "bfp8_sweep_kernel" : "";
    const bool fold = p->topk_desc >= 0 && p->rest.nwg > 0;
    if (stage == 0) return p->head.nwg > 0 ? (p->fused_head ? "bfp8_gemv_head_kernel" : "bfp8_gemv_grouped_kernel") : "";
    if (stage == 1) {
        if (p->rest.rows[0] >= 0) return "rt_rows_gemv_kernel";
        if (p->rest.wide) return "bfp8_gemv_wide_grouped_kernel";
        if (fold) return "bfp8_gemv_grouped_merge_kernel";
        if (p->rest.nwg > 0) return "bfp8_gemv_grouped_kernel";
        return p->topk_desc >= 0 ? bfp8_topk_merge_kernel_name(p->hdesc[p->topk_desc].M) : "";
    }
    if (stage == 2) {
        if (!p->odd_items.empty()) return "bfp8_tail_row_kernel";
        if (!p->float_items.empty()) return "bfp8_gemv_float_kernel";
        if (p->gen_head >= 0)
            return p->gen_out.topk <= BFP8_TOPK_MAX ? "bfp8_select_partials_kernel" : "bfp8_select_sort_kernel";
        return "";
    }
    return "";
}

int bfp8_plan_run_gemv(void* plan, void* stream) {
    int rc = BFP8_OK;
    for (int stage = 0; stage < 3 && !rc; ++stage) rc = bfp8_plan_launch(plan, stage, stream);
    return rc;
}

int bfp8_plan_run(void* plan, void* stream) {
    const Plan* p = static_cast<const Plan*>(plan);
    // the single launch, a fused lm_head launch or a 16-row launch quantizes its activations itself
    int rc = (p && (p->sweep || p->fused_head || p->rows_float)) ? BFP8_OK : bfp8_plan_quantize(plan, stream);
    return rc ? rc : bfp8_plan_run_gemv(plan, stream);
}

void bfp8_plan_destroy(void* plan) {
    Plan* p = static_cast<Plan*>(plan);
    if (!p) return;
    {
        std::lock_guard<std::mutex> lk(g.mu);
        if (g.ready) (void)hipDeviceSynchronize();
    }
    release_plan(p);
    delete p;
}

}  // extern "C"
