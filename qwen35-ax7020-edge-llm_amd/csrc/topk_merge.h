// topk_merge.h -- the final top-k merge of per-tile partial lists, shared by
// the GEMV launches (bfp8_ftz.hip) and the single-launch sweep (sweep.hip).
//
// Partial lists: [ntiles][topk] keys per 64-row tile, each list sorted
// descending (score desc, id asc), "no candidate" entries last.  The merge
// selects the topk best keys of all lists and writes lm_head_topk's outputs
// (04/qwen_sampling.c:283-353) and lm_head_argmax's winner
// (04/qwen_kernels_opt.c:402-403, :483-490: lowest id among the maximal
// scores above -1e30, else 0).
//
// Two key formats, both ordering as unsigned 64-bit integers with the
// ordered score in the high word (0: no candidate):
//   PlainKeys  low word ~row.  Written by an earlier launch on the stream: the
//              launch boundary makes them visible.
//   EpochKeys  low word (epoch << 18) | (2^18 - 1 - row) (rows < 2^18).  Written
//              and merged within one launch: every key carries the run's
//              14-bit epoch, the writer stores it with one agent-scope atomic
//              store, and the merger re-reads (agent scope) any key whose epoch
//              is not yet the current one, a bounded number of times.  No
//              fence or counter orders anything; a key is either the old one
//              (wrong epoch) or the new one.
// Device code only; integer work, the same in flush-to-zero and IEEE units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bfp8_layout.h"
#include "wave_topk.h"

namespace {

constexpr int kTopkMaxK = 64;

// A key is read in two steps, so that a lane's reads all go out before any
// is waited for: peek() issues the read, settle() returns the final key.
struct PlainKeys {
    __device__ static int id(uint64_t k) { return (int)~(uint32_t)k; }
    __device__ uint64_t peek(const uint64_t* p) const { return __builtin_nontemporal_load(p); }
    __device__ uint64_t settle(uint64_t k, const uint64_t*, bool&) const { return k; }
};

constexpr uint32_t kEpochRowBits = 18;
constexpr uint32_t kEpochRowMask = (1u << kEpochRowBits) - 1u;
constexpr int kEpochSpin = 1 << 16;  // re-reads of one key before the merge gives up

struct EpochKeys {
    uint32_t epoch;  // 1 .. 2^14 - 1
    __device__ static int id(uint64_t k) { return (int)(kEpochRowMask - ((uint32_t)k & kEpochRowMask)); }
    // The key of a plain partial-list entry (0: no candidate) for `row`.
    __device__ uint64_t make(uint64_t plain, int row) const {
        const uint32_t lo = (epoch << kEpochRowBits) | (kEpochRowMask - (uint32_t)row);
        return (plain >> 32) ? ((plain & 0xffffffff00000000ull) | lo) : (uint64_t)lo;
    }
    __device__ uint64_t peek(const uint64_t* p) const {
        return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __device__ uint64_t settle(uint64_t k, const uint64_t* p, bool& stale) const {
        for (int i = 0; i < kEpochSpin; ++i) {
            if (((uint32_t)k >> kEpochRowBits) == epoch) return k;
            __builtin_amdgcn_s_sleep(2);
            k = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        stale = true;
        return 0;
    }
    __device__ void store(uint64_t* p, uint64_t k) const {
        __hip_atomic_store(p, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
};

__device__ __forceinline__ bool key_valid(uint64_t k) { return (k >> 32) != 0; }

// What the merge needs, by value so that non-inlined code never takes the
// address of a kernel argument.
struct TopkArgs {
    const uint64_t* partials;
    int* out_ids;
    float* out_scores;
    int* out_count;
    int* out_argmax;
    int topk, ntiles;
};

template <int W>
struct MergeLds {
    uint64_t xch[W][64];
    int list[kTopkMaxK];
    int stale;
};

// Tree-reduces the W wavefronts' descending lists into wavefront 0's (the
// partner's list is read reversed, i.e. ascending).  A wavefront writes its
// slot once, at the level where it drops out, and every slot is read at the
// level it is written, so one barrier per level suffices; the caller puts a
// barrier between two calls.
template <int W>
__device__ __forceinline__ uint64_t reduce_waves(uint64_t v, int w, int lane, MergeLds<W>& L) {
#pragma unroll
    for (int step = 1; step < W; step <<= 1) {
        if ((w & (2 * step - 1)) == step) L.xch[w][lane] = v;
        __syncthreads();
        if ((w & (2 * step - 1)) == 0) v = wave_merge<true>(v, L.xch[w + step][63 - lane], lane);
    }
    return v;
}

// Wavefront 0 writes the result: ids / scores of the kk best keys (lane's
// key v, lanes < kk), their count, and the argmax.  A merge that gave up on a
// stale key writes count = -1 and argmax = -1.
template <class KF>
__device__ __forceinline__ void topk_write(const TopkArgs& d, uint64_t v, int lane, bool stale) {
    const int kk = d.topk;
    const uint64_t t = lane < kk ? v : 0ull;
    const bool ok = key_valid(t);
    const int cnt = __popcll(__ballot(ok));
    if (lane < kk) {
        d.out_ids[lane] = ok ? KF::id(t) : -1;
        d.out_scores[lane] = ok ? key_score(t) : 0.0f;
    }
    if (lane == 0) {  // lane 0 holds the best key
        *d.out_count = stale ? -1 : cnt;
        *d.out_argmax = stale ? -1 : ((ok && key_score(t) > -1e30f) ? KF::id(t) : 0);
    }
}

__device__ __forceinline__ uint64_t wave_max_key(uint64_t v) {
#pragma unroll
    for (int j = 1; j < 64; j <<= 1) {
        const uint64_t o = xor_lane(v, j);
        v = o > v ? o : v;
    }
    return v;
}

// Final merge by one workgroup of W wavefronts, H list heads per lane per
// pass.  Keys are unique (they carry the row), so an entry at position i of a
// list whose head ranks h-th among all heads has at least h+i better keys:
// only the lists of the kk best heads, and in them only i < kk - h, can reach
// the top kk.
template <int W, int H, class KF>
__device__ __forceinline__ void topk_merge(const TopkArgs& d, const KF& kf, MergeLds<W>& L) {
    const int kk = d.topk;
    const int ntiles = d.ntiles;
    const uint64_t* parts = d.partials;
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    bool stale = false;
    if (threadIdx.x == 0) L.stale = 0;
    if (kk == 1) {  // the best key is the largest list head: a max-reduction, no list merge
        uint64_t m = 0;
        for (int i = w * 64 + lane; i < ntiles; i += W * 64) {
            const uint64_t h = kf.settle(kf.peek(&parts[i]), &parts[i], stale);
            m = h > m ? h : m;
        }
        m = wave_max_key(m);
        if (lane == 0) L.xch[0][w] = m;
        __syncthreads();
        if (stale) L.stale = 1;
        __syncthreads();
        if (w == 0) {
            m = wave_max_key(lane < W ? L.xch[0][lane] : 0ull);
            topk_write<KF>(d, m, lane, L.stale != 0);
        }
        return;
    }
    // 1. the 64 best list heads
    uint64_t v = 0;
    for (int base = w * 64 * H; base < ntiles; base += W * 64 * H) {
        uint64_t h[H];
        bool desc[H];
#pragma unroll
        for (int u = 0; u < H; ++u) {
            const int i = base + u * 64 + lane;
            h[u] = i < ntiles ? kf.peek(&parts[(size_t)i * kk]) : 0ull;
            desc[u] = (H > 1) && (u % 2 == 0);  // the last tree level must come out ascending
        }
#pragma unroll
        for (int u = 0; u < H; ++u) {
            const int i = base + u * 64 + lane;
            if (i < ntiles) h[u] = kf.settle(h[u], &parts[(size_t)i * kk], stale);
        }
        wave_sort<H>(h, desc, lane);
#pragma unroll
        for (int s = 1; s < H; s <<= 1) {
#pragma unroll
            for (int i = 0; i < H; i += 2 * s) {
                if ((i / (2 * s)) % 2 == 0 && 2 * s < H)
                    h[i] = wave_merge<true>(h[i], h[i + s], lane);
                else
                    h[i] = wave_merge<false>(h[i], h[i + s], lane);
            }
        }
        v = wave_merge<true>(v, h[0], lane);
    }
    v = reduce_waves<W>(v, w, lane, L);
    if (w == 0 && lane < kk) L.list[lane] = key_valid(v) ? KF::id(v) / BFP8_TILE_ROWS : -1;
    __syncthreads();
    // 2. wavefront w merges lists h = w, w + W, ... (list h cut after kk - h
    // entries); odd slots are loaded reversed (ascending) for the tree.
    constexpr int kSlots = kTopkMaxK / W;
    uint64_t e[kSlots];
    int at[kSlots];
#pragma unroll
    for (int sl = 0; sl < kSlots; ++sl) {
        const int hh = w + sl * W;
        const int list = hh < kk ? L.list[hh] : -1;
        const int idx = (sl & 1) ? 63 - lane : lane;
        at[sl] = (list >= 0 && idx < kk - hh) ? list * kk + idx : -1;
        e[sl] = at[sl] >= 0 ? kf.peek(&parts[at[sl]]) : 0ull;
    }
#pragma unroll
    for (int sl = 0; sl < kSlots; ++sl)
        if (at[sl] >= 0) e[sl] = kf.settle(e[sl], &parts[at[sl]], stale);
    if (kSlots > 1)
        v = wave_merge_tree<kSlots>(e, lane);
    else
        v = e[0];
    v = reduce_waves<W>(v, w, lane, L);
    if (stale) L.stale = 1;
    __syncthreads();
    if (w == 0) topk_write<KF>(d, v, lane, L.stale != 0);
}

}  // namespace
