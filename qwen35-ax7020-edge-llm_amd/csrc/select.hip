// select.hip -- selection over a vector of scores on the device, for the
// argument ranges the fused lm_head launches do not cover, and the sampler.
//
//   * per-tile top-k partials of a logits vector (k <= 64), merged by the
//     stand-alone merge kernel of bfp8_ftz.hip: odd vocabularies, hidden
//     sizes the fused launches do not take;
//   * a full sort of the (score desc, id asc) keys for k > 64
//     (04/qwen_sampling.c:283-353 returns min(k, vocab) entries for any k);
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

}  // namespace

// ---- top-k over a logits vector ------------------------------------------------------------
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
    int mine = 0;
    for (int i = threadIdx.x; i < kk; i += blockDim.x) {
        const uint64_t k = keys[i];
        ids[i] = k ? key_id(k) : -1;
        scores[i] = k ? key_score(k) : 0.0f;
        mine += k != 0;
    }
    if (mine) atomicAdd(&cnt, mine);
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
