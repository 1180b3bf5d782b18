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
typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));

struct PlainKeys {
    __device__ static int id(uint64_t k) { return (int)~(uint32_t)k; }
    __device__ uint64_t peek(const uint64_t* p) const { return __builtin_nontemporal_load(p); }
    __device__ uint64_t settle(uint64_t k, const uint64_t*, bool&) const { return k; }
    // every key current (nothing to wait for)
    template <int NT>
    __device__ void verify_all(const uint64_t*, int, bool&) const {}
    __device__ PlainKeys verified() const { return *this; }
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
        if (stale) return 0;  // already given up: the result is reported invalid anyway
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
    // Waits (bounded) until each of the n keys carries the run's epoch; the
    // merge's NT threads (threadIdx.x < NT) share the keys.  After it (and a
    // barrier) every key can be read as verified(): no waiting per read.
    template <int NT>
    __device__ void verify_all(const uint64_t* p, int n, bool& stale) const {
        constexpr int nt = NT;
        for (int i0 = threadIdx.x; i0 < n; i0 += 8 * nt) {  // eight reads in flight
            uint64_t k[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) k[u] = i0 + u * nt < n ? peek(p + i0 + u * nt) : 0ull;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (i0 + u * nt < n) (void)settle(k[u], p + i0 + u * nt, stale);
        }
    }
    struct Current {  // keys already seen with the run's epoch
        __device__ static int id(uint64_t k) { return EpochKeys::id(k); }
        __device__ uint64_t peek(const uint64_t* p) const {
            return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __device__ uint64_t settle(uint64_t k, const uint64_t*, bool&) const { return k; }
    };
    __device__ Current verified() const { return Current{}; }
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

// Threshold selection (topk_select below): at most kSelCap candidates are
// ranked.
constexpr int kSelCap = 256;
constexpr int kSelPad = kSelCap + 16;  // zero-padded: the ranking reads sixteen keys at a time

template <int W>
struct MergeLds {
    uint64_t xch[W][64];
    uint64_t cand[kSelPad];
    uint32_t tw[W];
    uint64_t best;
    int list[kTopkMaxK];
    int ncand;
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

// Largest high word (ordered score) of the wavefront's keys, wave-uniform:
// DPP within each row of 16 lanes, then the four row maxima by v_readlane.
__device__ __forceinline__ uint32_t wave_max_score(uint32_t v) {
#pragma unroll
    for (int j = 1; j < 16; j <<= 1) {
        const uint32_t o = xor_lane32(v, j);
        v = o > v ? o : v;
    }
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
    const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    const uint32_t ab = a > b ? a : b, cd = c > d ? c : d;
    return ab > cd ? ab : cd;
}

// The c-th largest distinct score among the lanes' representatives (0 when
// there are fewer than c): at least c keys have a score >= it.
__device__ __forceinline__ uint32_t wave_cth_score(uint64_t rep, int c) {
    uint32_t r = (uint32_t)(rep >> 32), m = 0;
    for (int it = 0; it < c; ++it) {
        m = wave_max_score(r);
        if (r == m) r = 0;
    }
    return m;
}

// Ranks the n <= kSelCap candidates of L.cand (zero-padded) and writes the
// result: candidate j's position is the number of candidates above it (keys
// are unique).  Eight lanes count for one candidate, each over keys
// 16m + 2 part, 16m + 2 part + 1; wavefronts without a candidate skip.
template <int W, class KF>
__device__ __forceinline__ void select_rank_write(const TopkArgs& d, MergeLds<W>& L, int n, bool stale) {
    constexpr int NT = W * 64, NJ = NT / 8;
    const int tid = threadIdx.x, w = tid >> 6, kk = d.topk;
    const int part = tid & 7;
    const u64x2* c2 = reinterpret_cast<const u64x2*>(L.cand) + part;
    for (int j0 = 0; j0 < n; j0 += NJ) {
        if (j0 + w * 8 >= n) break;  // wave-uniform
        const int j = j0 + (tid >> 3);
        const uint64_t key = L.cand[j < kSelCap ? j : 0];
        int rank = 0;
        int m = 0;
        for (; m + 64 <= n; m += 64) {
            u64x2 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = c2[(m >> 1) + 8 * u];
#pragma unroll
            for (int u = 0; u < 4; ++u) rank += (v[u].x > key ? 1 : 0) + (v[u].y > key ? 1 : 0);
        }
        for (; m < n; m += 16) {
            const u64x2 v = c2[m >> 1];
            rank += (v.x > key ? 1 : 0) + (v.y > key ? 1 : 0);
        }
        rank += (int)xor_lane32((uint32_t)rank, 1);
        rank += (int)xor_lane32((uint32_t)rank, 2);
        rank += (int)xor_lane32((uint32_t)rank, 4);
        if (part == 0 && j < n) {
            if (rank < kk) {
                d.out_ids[rank] = KF::id(key);
                d.out_scores[rank] = key_score(key);
            }
            if (rank == 0) L.best = key;
        }
    }
    for (int j = n + tid; j < kk; j += NT) {
        d.out_ids[j] = -1;
        d.out_scores[j] = 0.0f;
    }
    if (stale) L.stale = 1;
    __syncthreads();
    if (tid == 0) {
        const uint64_t b = L.best;
        const bool st = L.stale != 0;
        *d.out_count = st ? -1 : (n < kk ? n : kk);
        *d.out_argmax = st ? -1 : ((key_valid(b) && key_score(b) > -1e30f) ? KF::id(b) : 0);
    }
}

// Gathers the rest of a list above T from entry j0 on (rare), in batches
// of eight: each batch is read, its prefix above T counted, given slots by
// one LDS atomic and stored.
template <int W, class KF>
__device__ __forceinline__ void list_offer(const KF& kf, const uint64_t* list, int j0, int kk, uint64_t T,
                                           bool& stale, MergeLds<W>& L) {
    for (; j0 < kk; j0 += 8) {
        uint64_t k8[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) k8[u] = j0 + u < kk ? kf.peek(list + j0 + u) : 0ull;
        int cnt = 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (j0 + u < kk) k8[u] = kf.settle(k8[u], list + j0 + u, stale);
            cnt += (cnt == u && key_valid(k8[u]) && k8[u] >= T) ? 1 : 0;
        }
        if (cnt) {
            const int off = atomicAdd(&L.ncand, cnt);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (u < cnt && off + u < kSelCap) L.cand[off + u] = k8[u];
        }
        if (cnt < 8) break;
    }
}

// Selection by threshold, the fast path of topk_merge for 2 <= kk <= 64.
// A lane's representative is the best key it read; wavefront w takes the
// c-th best distinct score t_w among its representatives (c = ceil(kk / W);
// 0 when it has fewer than c), and T is the lowest key with the score
// min_w t_w.  Each wavefront with t_w != 0 holds at least c distinct keys
// >= T, so at least kk keys are >= T when every t_w is valid, and T = 0 admits
// every valid key otherwise: the kk best keys are always among the keys
// >= T.  Lists are sorted descending, so a list's candidates are a prefix.
// The candidates are gathered in LDS (one LDS atomic per wavefront for its
// slots) and ranked (select_rank_write).
// Returns false (uniformly) when there are more than kSelCap candidates or
// more lists than the form covers; the caller then runs the tree merge.
// Random scores give ~100 candidates at kk = 40 over 1,024 lists; tables of
// equal scores overflow and take the tree.
//
// KEEP (latency form, the stand-alone merge): lane quad t >> 2 reads the
// first four entries of lists (t >> 2) + (NT / 4) p, p < PASSES, one entry
// per lane (one wavefront load touches 16 lists' 32-byte heads), and keeps
// them; only a list whose fourth entry is >= T is read on.
// Otherwise (few registers, the merge folded into a streaming launch): lane t
// reads the heads of lists t + NT p, p < PASSES, then reads on only through
// the lists whose head is >= T, one batch of eight entries at a time.
template <int W, int PASSES, bool KEEP, class KF>
__device__ __forceinline__ bool topk_select(const TopkArgs& d, const KF& kf, MergeLds<W>& L, bool& stale) {
    constexpr int NT = W * 64, NQ = NT / 4;
    const int kk = d.topk, ntiles = d.ntiles;
    if (ntiles > PASSES * (KEEP ? NQ : NT)) return false;
    const uint64_t* parts = d.partials;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ent = KEEP ? (tid & 3) : 0, q = KEEP ? (tid >> 2) : tid;
    auto list_of = [&](int p) { return q + p * (KEEP ? NQ : NT); };
    auto at = [&](int p) -> const uint64_t* { return &parts[(size_t)list_of(p) * kk + ent]; };
    auto mine = [&](int p) { return list_of(p) < ntiles && ent < kk; };
    uint64_t e[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) e[p] = mine(p) ? kf.peek(at(p)) : 0ull;
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
        if (mine(p)) e[p] = kf.settle(e[p], at(p), stale);
    uint64_t rep = 0;  // any distinct keys serve: the lane's best entry
#pragma unroll
    for (int p = 0; p < PASSES; ++p) rep = e[p] > rep ? e[p] : rep;
    const uint32_t tw = wave_cth_score(rep, (kk + W - 1) / W);
    if (lane == 0) L.tw[w] = tw;
    for (int j = tid; j < kSelPad; j += NT) L.cand[j] = 0;
    if (tid == 0) {
        L.ncand = 0;
        L.best = 0;
    }
    __syncthreads();
    uint32_t ts = ~0u;
#pragma unroll
    for (int v = 0; v < W; ++v) ts = L.tw[v] < ts ? L.tw[v] : ts;
    const uint64_t T = (uint64_t)ts << 32;
    auto above = [&](uint64_t k) { return key_valid(k) && k >= T; };
    // slots: one LDS atomic per wavefront; within it, pass p's candidates
    // after those of passes < p, in lane order (ballots and lane counts; a
    // per-lane atomic was serialized lane by lane)
    int slot[PASSES];
    int wtotal = 0;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const uint64_t mk = __builtin_amdgcn_ballot_w64(above(e[p]));
        slot[p] = wtotal + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u));
        wtotal += (int)__popcll(mk);
    }
    int wbase = 0;
    if (lane == 0 && wtotal > 0) wbase = atomicAdd(&L.ncand, wtotal);
    wbase = __builtin_amdgcn_readfirstlane(wbase);
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
        if (above(e[p]) && wbase + slot[p] < kSelCap) L.cand[wbase + slot[p]] = e[p];
    if (KEEP) {  // lane 3 of a quad holds entry 3: the list goes on above T (rare)
#pragma unroll
        for (int p = 0; p < PASSES; ++p)
            if (above(e[p]) && ent == 3 && kk > 4) list_offer(kf, at(p) - 3, 4, kk, T, stale, L);
    } else {
#pragma unroll
        for (int p = 0; p < PASSES; ++p)
            if (above(e[p]) && kk > 1) list_offer(kf, at(p), 1, kk, T, stale, L);
    }
    __syncthreads();
    const int n = L.ncand;
    if (n > kSelCap) return false;
    select_rank_write<W, KF>(d, L, n, stale);
    return true;
}

// The bitonic tree merge (lists of every length, any key distribution).
template <int W, int H, class KF>
__device__ __forceinline__ void topk_tree(const TopkArgs& d, const KF& kf, MergeLds<W>& L, bool& stale) {
    const int kk = d.topk;
    const int ntiles = d.ntiles;
    const uint64_t* parts = d.partials;
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
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


// Final merge by one workgroup of W wavefronts, H list heads per lane per
// pass.  Keys are unique (they carry the row), so an entry at position i of a
// list whose head ranks h-th among all heads has at least h+i better keys:
// only the lists of the kk best heads, and in them only i < kk - h, can reach
// the top kk.
template <int W, int H, int PASSES, bool KEEP, class KF>
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
    if (topk_select<W, PASSES, KEEP>(d, kf, L, stale)) return;
    // more candidates than the selection ranks: the bitonic tree, over keys
    // first waited for all at once (its reads then wait for nothing)
    kf.template verify_all<W * 64>(parts, ntiles * kk, stale);
    __syncthreads();
    topk_tree<W, H>(d, kf.verified(), L, stale);
}

}  // namespace
