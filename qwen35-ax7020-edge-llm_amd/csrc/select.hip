// select.hip -- selection over a vector of scores on the device, for the
// argument ranges the fused lm_head launches do not cover, and the sampler.
//
//   * per-tile top-k partials of a logits vector (k <= 64), merged by the
//     stand-alone merge kernel of bfp8_ftz.hip: odd vocabularies, hidden
//     sizes the fused launches do not take;
//   * for k > 64 (04/qwen_sampling.c:283-353 returns min(k, vocab) entries
//     for any k) the (score desc, id asc) keys sorted in 2048-key blocks in
//     LDS and registers, one workgroup each, then each block's first
//     min(k, 2048) keys ranked against every block's (one bisection in LDS per
//     candidate and block; keys are unique, so a key's rank is the count of
//     keys above it).  At 65536 keys: 13.8 us of block sorts, then 5.5 us
//     (k = 65) to 49 us (all keys) of ranking.  Beyond 2^20 keys one workgroup
//     sorts them all in global memory (about 2 ms at 65536 keys);
//   * sample_from_topk (04/qwen_sampling.c:384-529) for any candidate count.
//
// Compiled with IEEE f32 subnormals and -ffp-contract=off: the sampler
// restates scalar C (glibc expf, double sums); everything else here is
// integer work on 64-bit keys.
#include <float.h>
#include <hip/hip_runtime.h>

#include "bfp8_internal.h"
#include "wave_topk.h"

namespace {

constexpr int kSortThreads = 1024;
constexpr int kSelBlock = BFP8_SELECT_BLOCK;  // keys per LDS-sorted block
constexpr int kSelLog = __builtin_ctz(kSelBlock);
constexpr int kBlkThreads = 1024;                        // block sort: threads
constexpr int kBlkKeys = kSelBlock / kBlkThreads;        // keys per thread (key r * 1024 + thread)
constexpr int kBlkPairs = (kSelBlock / 2 + kBlkThreads - 1) / kBlkThreads;  // LDS compare-exchanges per thread, step
constexpr int kRankParts = (kSelBlock + 1023) / 1024;  // rank kernel: workgroups (1024 candidates) per block
constexpr int kRankTab = 8192;                         // keys of the rank kernel's LDS tables per batch
static_assert(kSelBlock == 1 << kSelLog && kSelBlock >= 1024 && kSelBlock <= 8192, "block size");

// In-place sort of keys[0, n) into descending order by one workgroup.  The
// bitonic network in its one-direction form: at every stage of size s, element
// i of each s-block is compared with its mirror (block end - 1 - i), then with
// i + s/4, i + s/8, ... (half-cleaners); the larger key always goes to the
// lower index.  Padding the array to a power of two with keys below every
// real key would never move a padding element, so the compare-exchanges whose
// upper index reaches n are simply skipped.  Pairs of one step are disjoint:
// four are loaded before any is stored.
__device__ void block_sort_desc(uint64_t* keys, int n) {
    if (n < 2) return;
    int P = 1;
    while (P < n) P <<= 1;
    const int half_p = P >> 1;
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int size = 2; size <= P; size <<= 1) {
        for (int j = size >> 1; j >= 1; j >>= 1) {
            const bool flip = j == (size >> 1);
            for (int i0 = tid; i0 < half_p; i0 += 4 * nt) {
                int a[4], b[4];
                uint64_t ka[4], kb[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int i = i0 + u * nt;
                    if (flip) {  // mirror within the size-block
                        const int blk = i / j, off = i % j;
                        a[u] = blk * size + off;
                        b[u] = blk * size + size - 1 - off;
                    } else {
                        a[u] = (i / j) * 2 * j + i % j;
                        b[u] = a[u] + j;
                    }
                    const bool ok = i < half_p && b[u] < n;
                    if (!ok) b[u] = -1;
                    ka[u] = ok ? keys[a[u]] : 0ull;
                    kb[u] = ok ? keys[b[u]] : 0ull;
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (b[u] >= 0 && kb[u] > ka[u]) {
                        keys[a[u]] = kb[u];
                        keys[b[u]] = ka[u];
                    }
                }
            }
            __syncthreads();
        }
    }
}

// The kSelBlock keys v (thread t holds keys r * 1024 + t) sorted descending
// into LDS by the workgroup's 1024 threads: the one-direction bitonic network
// of block_sort_desc.  A step whose partner (key index ^ mask) is in the same
// wavefront runs in registers (a lane exchange, the larger key to the lower
// index); the others run on LDS, one pair or more per thread and step.  Of
// the 66 steps of 2048 keys, 15 go through LDS.
__device__ void block_sort_regs(uint64_t (&v)[kBlkKeys], uint64_t* lds) {
    const int tid = threadIdx.x;
    bool in_lds = false;
#pragma unroll
    for (int ls = 1; ls <= kSelLog; ++ls) {
#pragma unroll
        for (int lj = ls - 1; lj >= 0; --lj) {
            const int j = 1 << lj, size = 1 << ls;
            const bool mirror = lj == ls - 1;
            const int mask = mirror ? size - 1 : j;  // partner = index ^ mask
            if (mask < 64) {
                if (in_lds) {
                    __syncthreads();
#pragma unroll
                    for (int r = 0; r < kBlkKeys; ++r) v[r] = lds[r * kBlkThreads + tid];
                    in_lds = false;
                }
                const bool lower = (tid & (mirror ? size >> 1 : j)) == 0;  // index below its partner's
#pragma unroll
                for (int r = 0; r < kBlkKeys; ++r) {
                    const uint64_t o = xor_lane(v[r], mask);
                    v[r] = ((o > v[r]) == lower) ? o : v[r];
                }
            } else {
                if (!in_lds) {
#pragma unroll
                    for (int r = 0; r < kBlkKeys; ++r) lds[r * kBlkThreads + tid] = v[r];
                    in_lds = true;
                }
                __syncthreads();
#pragma unroll
                for (int r = 0; r < kBlkPairs; ++r) {
                    const int i = tid + r * kBlkThreads;  // pair 0 .. kSelBlock / 2 - 1
                    const int blk = i >> lj, off = i & (j - 1);
                    const int a = mirror ? blk * size + off : blk * 2 * j + off;
                    const int b = mirror ? blk * size + size - 1 - off : a + j;
                    if (i >= kSelBlock / 2) continue;
                    const uint64_t ka = lds[a], kb = lds[b];
                    if (kb > ka) {
                        lds[a] = kb;
                        lds[b] = ka;
                    }
                }
            }
        }
    }
    if (!in_lds) {
#pragma unroll
        for (int r = 0; r < kBlkKeys; ++r) lds[r * kBlkThreads + tid] = v[r];
    }
    __syncthreads();
}

}  // namespace

// ---- top-k over a logits vector ------------------------------------------------------------
// Block b of the keys of logits[0, n) (kSelBlock rows; the last one
// shorter) sorted descending in LDS and stored over keys[kSelBlock b, ...
// + len); its count of candidates (nonzero keys) into valid[b].
extern "C" __global__ __launch_bounds__(kBlkThreads) void bfp8_select_block_sort_kernel(
    const float* __restrict__ logits, int n, uint64_t* __restrict__ keys, uint32_t* __restrict__ valid) {
    __shared__ uint64_t s[kSelBlock];
    __shared__ uint32_t nv;
    const int base = blockIdx.x * kSelBlock, len = min(kSelBlock, n - base);
    const int tid = threadIdx.x;
    if (tid == 0) nv = 0;
    uint32_t mine = 0;  // the wavefront's valid keys (ballots; one LDS atomic per wavefront)
    uint64_t v[kBlkKeys];
#pragma unroll
    for (int r = 0; r < kBlkKeys; ++r) {
        const int i = tid + r * kBlkThreads;
        v[r] = i < len ? topk_key(logits[base + i], base + i) : 0ull;
        mine += (uint32_t)__popcll(__builtin_amdgcn_ballot_w64(v[r] != 0));
    }
    __syncthreads();
    if ((tid & 63) == 0 && mine) atomicAdd(&nv, mine);
    block_sort_regs(v, s);
    for (int i = tid; i < len; i += kBlkThreads) keys[base + i] = s[i];
    if (tid == 0) valid[blockIdx.x] = nv;
}

// The kk best keys by rank: workgroup (b, part) takes positions part*1024 +
// t of sorted block b below min(kk, len_b) as candidates; a candidate's rank
// is the number of keys above it in every block's first min(kk, len) keys
// (the blocks' prefixes go through LDS in batches of whole tables; every
// (candidate, table) pair is one bisection; a key with kk or more keys above
// it in one prefix is out whatever the rest).  Rank < kk: written at its rank.  Workgroup 0
// writes the count (min(kk, candidates)), fills the places past it with
// -1 / 0, and the argmax when there is no candidate; the rank-0 key writes
// it otherwise (04/qwen_kernels_opt.c:402-403, :483-490).
extern "C" __global__ __launch_bounds__(kSortThreads) void bfp8_select_rank_kernel(
    const uint64_t* __restrict__ keys, const uint32_t* __restrict__ valid, int n, int kk, int* __restrict__ ids,
    float* __restrict__ scores, int* __restrict__ count, int* __restrict__ argmax) {
    __shared__ uint64_t tab[kRankTab];
    __shared__ uint64_t cand[kSortThreads];
    __shared__ int crank[kSortThreads];
    __shared__ uint32_t red[kSortThreads / 64];
    const int nblk = (n + kSelBlock - 1) >> kSelLog;
    const int b = blockIdx.x / kRankParts, part = blockIdx.x % kRankParts;
    const int tid = threadIdx.x;
    const int m = min(kk, kSelBlock);  // prefix length of a whole block
    if (blockIdx.x == 0) {
        uint32_t v = 0;
        for (int i = tid; i < nblk; i += kSortThreads) v += valid[i];
        for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
        if ((tid & 63) == 0) red[tid >> 6] = v;
        __syncthreads();
        v = 0;
#pragma unroll
        for (int w = 0; w < kSortThreads / 64; ++w) v += red[w];
        const int cnt = (int)min((uint32_t)kk, v);
        for (int i = cnt + tid; i < kk; i += kSortThreads) {
            ids[i] = -1;
            scores[i] = 0.0f;
        }
        if (tid == 0) {
            *count = cnt;
            if (v == 0) *argmax = 0;
        }
    }
    const int len_b = min(kSelBlock, n - (b << kSelLog));
    const int ncand = min(m, len_b) - part * kSortThreads;  // this workgroup's candidates
    if (ncand <= 0) return;
    const int nc = min(ncand, kSortThreads);
    const int pos = part * kSortThreads + tid;
    const uint64_t key = tid < nc ? keys[(size_t)(b << kSelLog) + pos] : 0ull;
    if (tid < nc) {
        cand[tid] = key;
        crank[tid] = 0;
    }
    const int per_batch = kRankTab / m;
    int top = 1;  // the largest power of two <= m
    while (2 * top <= m) top *= 2;
    for (int b0 = 0; b0 < nblk; b0 += per_batch) {
        const int nt = min(per_batch, nblk - b0);
        // every load of the batch goes out before any is stored
        uint64_t v[kRankTab / kSortThreads];
#pragma unroll
        for (int r = 0; r < kRankTab / kSortThreads; ++r) {
            const int i = tid + r * kSortThreads;
            const int t = i / m, e = i - t * m, b2 = b0 + t;
            v[r] = i < nt * m && e < n - (b2 << kSelLog) ? keys[(size_t)(b2 << kSelLog) + e] : 0ull;  // past the block: 0
        }
        __syncthreads();  // the previous batch's searches are done
#pragma unroll
        for (int r = 0; r < kRankTab / kSortThreads; ++r) {
            const int i = tid + r * kSortThreads;
            if (i < nt * m) tab[i] = v[r];
        }
        __syncthreads();
        // one (candidate, table) pair per thread at a time: the keys above the
        // candidate in the table (descending, unique; 0s last) by a
        // bisection of fixed steps, added to the candidate's rank in LDS
        for (int w = tid; w < nc * nt; w += kSortThreads) {
            const int t = w / nc, c = w - t * nc;
            const uint64_t ck = cand[c];
            if (!ck) continue;
            const uint64_t* T = tab + t * m;
            int at = 0;
            for (int step = top; step > 0; step >>= 1) {
                const int q = at + step;  // T[q - 1] > key: at least q keys above
                if (q <= m && T[q - 1] > ck) at = q;
            }
            if (at) atomicAdd(&crank[c], at);
        }
    }
    __syncthreads();
    if (key) {
        const int rank = crank[tid];
        if (rank < kk) {
            ids[rank] = key_id(key);
            scores[rank] = key_score(key);
            if (rank == 0) *argmax = key_score(key) > -1e30f ? key_id(key) : 0;
        }
    }
}
// keys[i] = the (score desc, id asc) key of logits[i] (0: not a candidate).
extern "C" __global__ __launch_bounds__(256) void bfp8_select_keys_kernel(const float* __restrict__ logits, int n,
                                                                          uint64_t* __restrict__ keys) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) keys[i] = topk_key(logits[i], i);
}

// One wavefront per 64-row tile: its `topk` best keys, sorted, as the tile's
// partial list ([ntiles][topk], 0-padded), which the merge kernel reads.
extern "C" __global__ __launch_bounds__(256) void bfp8_select_partials_kernel(const float* __restrict__ logits, int n,
                                                                              int topk, uint64_t* __restrict__ partials) {
    const int lane = threadIdx.x & 63;
    const int ntiles = (n + 63) >> 6;
    for (int t = blockIdx.x * 4 + (threadIdx.x >> 6); t < ntiles; t += gridDim.x * 4) {
        const int row = t * 64 + lane;
        uint64_t key[1] = {row < n ? topk_key(logits[row], row) : 0ull};
        const bool desc[1] = {true};
        wave_sort<1>(key, desc, lane);
        if (lane < topk) partials[(size_t)t * topk + lane] = key[0];
    }
}

// All n keys sorted in place (one workgroup), then the first kk as the
// lm_head_topk result: ids / scores of the candidates among them, their count,
// and the lm_head_argmax winner (lowest id among the maximal scores above
// -1e30, else 0: 04/qwen_kernels_opt.c:402-403, :483-490).
extern "C" __global__ __launch_bounds__(kSortThreads) void bfp8_select_sort_kernel(uint64_t* __restrict__ keys, int n,
                                                                                   int kk, int* __restrict__ ids,
                                                                                   float* __restrict__ scores,
                                                                                   int* __restrict__ count,
                                                                                   int* __restrict__ argmax) {
    block_sort_desc(keys, n);
    __shared__ int cnt;
    if (threadIdx.x == 0) cnt = 0;
    __syncthreads();
    int mine = 0;  // the wavefront's valid keys (ballots; one LDS atomic per wavefront)
    for (int i0 = threadIdx.x & ~63; i0 < kk; i0 += blockDim.x) {  // wavefront-uniform trip count
        const int i = i0 + (int)(threadIdx.x & 63);
        const uint64_t k = i < kk ? keys[i] : 0ull;
        if (i < kk) {
            ids[i] = k ? key_id(k) : -1;
            scores[i] = k ? key_score(k) : 0.0f;
        }
        mine += (int)__popcll(__builtin_amdgcn_ballot_w64(k != 0));
    }
    if ((threadIdx.x & 63) == 0 && mine) atomicAdd(&cnt, mine);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint64_t k = keys[0];
        *count = cnt;
        *argmax = (k && key_score(k) > -1e30f) ? key_id(k) : 0;
    }
}

// ---- sampler, 04/qwen_sampling.c:358-529 ------------------------------------------------------
namespace {

// expf as the float rounding of the double exponential (glibc's expf is
// correctly rounded but for results within about 2^-29 ulp of a rounding
// boundary).
__device__ __forceinline__ float sample_expf(float x) { return (float)exp((double)x); }

// Sort key of a candidate for sample_pair_cmp's order (score desc, then id
// asc, 04/qwen_sampling.c:411-420): the score's bits mapped to an unsigned
// order (-0 read as +0, which the comparator does not tell apart), then the
// id with its sign flipped and complemented.  A NaN score sorts above +inf
// or below -inf by its sign bit (the comparator gives no order for it).
__device__ __forceinline__ uint64_t sample_key(float s, int id) {
    uint32_t b = __float_as_uint(s);
    if ((b & 0x7fffffffu) == 0u) b = 0u;
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)~((uint32_t)id ^ 0x80000000u);
}
__device__ __forceinline__ float sample_key_score(uint64_t k) {
    const uint32_t o = (uint32_t)(k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
__device__ __forceinline__ int sample_key_id(uint64_t k) { return (int)(~(uint32_t)k ^ 0x80000000u); }

// work[i] after the ordering step: the candidate's score bits (later its
// exponential's) in the high word, its id in the low word.
__device__ __forceinline__ uint64_t pack_pair(float s, int id) {
    return ((uint64_t)__float_as_uint(s) << 32) | (uint32_t)id;
}
__device__ __forceinline__ float pair_val(uint64_t w) { return __uint_as_float((uint32_t)(w >> 32)); }
__device__ __forceinline__ int pair_id(uint64_t w) { return (int)(uint32_t)w; }

}  // namespace

// One workgroup: the ordering and the exponentials in parallel, the sums and
// the draw in one thread in the reference's order (double accumulation, i
// ascending).  work: 8 * a.n bytes.
extern "C" __global__ __launch_bounds__(kSortThreads) void bfp8_sample_kernel(Bfp8SampleArgs a) {
    __shared__ int unsorted;
    __shared__ float red[kSortThreads / 64];
    const int tid = threadIdx.x, nt = blockDim.x;
    int n = a.n;
    if (a.count) {
        const int c = *a.count;
        n = c < 0 ? 0 : (c < a.n ? c : a.n);
    }
    if (n <= 0) {
        if (tid == 0) *a.out = -1;
        return;
    }
    if (!a.rng) {  // 04/qwen_sampling.c:405: no state, the first candidate as given
        if (tid == 0) *a.out = a.ids[0];
        return;
    }
    uint64_t* w = reinterpret_cast<uint64_t*>(a.work);
    if (tid == 0) unsorted = 0;
    __syncthreads();
    int mine = 0;
    for (int i = tid + 1; i < n; i += nt) mine |= a.scores[i] > a.scores[i - 1];
    if (mine) unsorted = 1;
    __syncthreads();
    if (unsorted) {  // :408-422, sorted on a copy
        for (int i = tid; i < n; i += nt) w[i] = sample_key(a.scores[i], a.ids[i]);
        __syncthreads();
        block_sort_desc(w, n);
        for (int i = tid; i < n; i += nt) {
            const uint64_t k = w[i];
            w[i] = pack_pair(sample_key_score(k), sample_key_id(k));
        }
    } else {
        for (int i = tid; i < n; i += nt) w[i] = pack_pair(a.scores[i], a.ids[i]);
    }
    __syncthreads();
    if (!(a.temperature >= 1e-6f)) {  // :424-429, greedy
        if (tid == 0) *a.out = pair_id(w[0]);
        return;
    }
    const int m = (a.top_k > 0 && a.top_k < n) ? a.top_k : n;
    // :431-436: maxf = s0, raised by every later s > maxf, i.e. s0 when s0 is
    // NaN, else the largest non-NaN score (the sign of a zero maximum never
    // reaches a result: s - (+-0) and exp(+-0) agree)
    float mx = -INFINITY;
    for (int i = tid; i < m; i += nt) mx = fmaxf(mx, pair_val(w[i]));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
    for (int i = 1; i < nt / 64; ++i) mx = fmaxf(mx, red[i]);
    const float s0 = pair_val(w[0]);
    if (s0 != s0) mx = s0;
    const float inv_t = 1.0f / a.temperature;
    __syncthreads();  // every thread has read w[0] before it is rewritten
    for (int i = tid; i < m; i += nt) {
        const uint64_t v = w[i];
        w[i] = pack_pair(sample_expf((pair_val(v) - mx) * inv_t), pair_id(v));
    }
    __syncthreads();
    if (tid != 0) return;
    int out = pair_id(w[0]);
    double all = 0.0;  // :441-444
#pragma unroll 8
    for (int i = 0; i < m; ++i) all += (double)pair_val(w[i]);
    if (all > 0.0) {
        float p = a.top_p;  // :452-454
        if (!(p > 0.0f)) p = 0.0f;
        if (p > 1.0f) p = 1.0f;
        int keep = m;  // :456-463
        double cum = 0.0;
        for (int i = 0; i < m; ++i) {
            cum += (double)pair_val(w[i]) / all;
            if (cum > (double)p) {
                keep = i + 1;
                break;
            }
        }
        double kept = 0.0;  // :467-471
#pragma unroll 8
        for (int i = 0; i < keep; ++i) kept += (double)pair_val(w[i]);
        if (kept > 0.0) {  // :478-489
            uint32_t x = *a.rng;
            if (x == 0u) x = 0x9E3779B9u;
            x ^= x << 13;
            x ^= x >> 17;
            x ^= x << 5;
            *a.rng = x;
            const double r = (double)((float)(x >> 8) * (1.0f / 16777216.0f)) * kept;
            int pick = keep - 1;
            cum = 0.0;
            for (int i = 0; i < keep; ++i) {
                cum += (double)pair_val(w[i]);
                if (r < cum) {
                    pick = i;
                    break;
                }
            }
            out = pair_id(w[pick]);
        }
    }
    *a.out = out;
}

// ---- launchers ------------------------------------------------------------------------------
static int select_grid(long long work, int per_block) {
    long long g = (work + per_block - 1) / per_block;
    if (g > 4096) g = 4096;
    return g < 1 ? 1 : (int)g;
}

hipError_t bfp8_launch_select_partials(const float* logits, int n, int topk, uint64_t* partials, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (topk < 1 || topk > BFP8_TOPK_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(bfp8_select_partials_kernel, dim3(select_grid(bfp8_ntiles(n), 4)), dim3(256), 0, s, logits, n,
                       topk, partials);
    return hipGetLastError();
}

hipError_t bfp8_launch_select_sort(const float* logits, int n, int kk, uint64_t* keys, int* ids, float* scores,
                                   int* count, int* argmax, hipStream_t s) {
    if (n <= 0 || kk < 1 || kk > n || n > BFP8_SELECT_MAX) return hipErrorInvalidValue;
    if (n <= BFP8_SELECT_RANK_MAX) {
        const int nblk = (n + kSelBlock - 1) / kSelBlock;
        uint32_t* valid = reinterpret_cast<uint32_t*>(keys + n);
        hipLaunchKernelGGL(bfp8_select_block_sort_kernel, dim3(nblk), dim3(kBlkThreads), 0, s, logits, n, keys,
                           valid);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(bfp8_select_rank_kernel, dim3(nblk * kRankParts), dim3(kSortThreads), 0, s, keys, valid,
                           n, kk, ids, scores, count, argmax);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(bfp8_select_keys_kernel, dim3(select_grid(n, 256)), dim3(256), 0, s, logits, n, keys);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(bfp8_select_sort_kernel, dim3(1), dim3(kSortThreads), 0, s, keys, n, kk, ids, scores, count,
                       argmax);
    return hipGetLastError();
}

hipError_t bfp8_launch_sample(const Bfp8SampleArgs& a, hipStream_t s) {
    if (a.n < 1 || a.n > BFP8_SELECT_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(bfp8_sample_kernel, dim3(1), dim3(kSortThreads), 0, s, a);
    return hipGetLastError();
}
