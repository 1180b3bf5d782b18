// bfp8_ftz.hip -- BFP8 W8A16 GEMV kernels for gfx950 (MI355X).
//
// Compiled with -fgpu-flush-denormals-to-zero -ffp-contract=off: every f32
// operation here flushes subnormal operands and results to signed zero and
// rounds once, which is how the reference's Advanced SIMD code computes
// (ARMv7 NEON is always flush-to-zero; vmlaq_n_f32 on Cortex-A9 rounds the
// product and then the sum).
//
// Reference semantics restated (04/qwen_kernels_opt.c:207-278, row pairs):
//   for every row and block b:  S_j = sum_{k = j mod 4} w[k] * xq[k]   (int32)
//     fs_j = fs_j + ((float(S_j) * EXP_SCALE[e]) * xscale[b])         (j = 0..3)
//   y = (fs_0 + fs_2) + (fs_1 + fs_3)
// with EXP_SCALE[e] = 2^(e-134), read as zero when subnormal (e < 8).
//
// Work mapping: a workgroup of 4 wavefronts owns a tile of 64 rows; wavefront
// q computes residue lane q of all 64 rows (lane = row), streaming one 1 KiB
// contiguous dwordx4 load per block.  The residue's activation dwords are
// wave-uniform and live in SGPRs (scalar loads), so the inner loop is
// 8 x v_dot4_i32_i8 + 1 shift per 16 weight bytes per lane, no LDS traffic.
// The per-block float epilogue runs in block order inside each lane, which is
// exactly the reference's per-lane accumulation order.  No MFMA: batch-1 is a
// bandwidth-bound matrix-vector product.
#include <float.h>
#include <hip/hip_runtime.h>

#include "bfp8_internal.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(4))) uint32_t* sgpr_u32_ptr;
typedef const __attribute__((address_space(4))) float* sgpr_f32_ptr;

constexpr int kChunk = 8;              // blocks per load batch (8 KiB per wave)
constexpr int kBufDword3 = 0x00020000;  // gfx9 raw buffer descriptor word 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             kBufDword3);
}

__device__ __forceinline__ u32x4 load_w(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0));
}

__device__ __forceinline__ uint32_t load_e(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, 0);
}

// Exact S_q of one (row, block, residue): xq = 256*xh + xl.
__device__ __forceinline__ int residue_sum(u32x4 w, sgpr_u32_ptr xb) {
    int acc = __builtin_amdgcn_sdot4((int)w.x, (int)xb[0], 0, false);
    acc = __builtin_amdgcn_sdot4((int)w.y, (int)xb[1], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.z, (int)xb[2], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w, (int)xb[3], acc, false);
    acc = (int)((uint32_t)acc << 8);
    acc = __builtin_amdgcn_sdot4((int)w.x, (int)xb[4], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.y, (int)xb[5], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.z, (int)xb[6], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w, (int)xb[7], acc, false);
    return acc;
}

// EXP_SCALE[e] under flush-to-zero: 2^(e-134) for e >= 8, else +0.
__device__ __forceinline__ float exp_scale_ftz(uint32_t e) {
    return __uint_as_float((max(e, 7u) - 7u) << 23);
}

// fs += (float(S) * EXP_SCALE[e]) * xscale   (three roundings, flush-to-zero)
__device__ __forceinline__ float epilogue(float fs, int S, uint32_t e, float xs) {
    float t1 = (float)S * exp_scale_ftz(e);
    float t2 = t1 * xs;
    return fs + t2;
}

// ---- top-k keys ------------------------------------------------------------
// Order (score desc, id asc) as one unsigned 64-bit key, larger = better.
// Candidates are the scores the reference would ever offer: > -FLT_MAX, not
// NaN (04/qwen_sampling.c:243-248 with thr = -FLT_MAX).  -0 equals +0 there,
// so it is keyed as +0.  0 is "no candidate".
__device__ __forceinline__ uint64_t topk_key(float y, int row) {
    if (!(y > -FLT_MAX)) return 0;
    uint32_t b = __float_as_uint(y == 0.0f ? 0.0f : y);
    uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)~(uint32_t)row;
}
__device__ __forceinline__ float key_score(uint64_t k) {
    uint32_t o = (uint32_t)(k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
__device__ __forceinline__ int key_id(uint64_t k) { return (int)~(uint32_t)k; }

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    int lo = __shfl_xor((int)(uint32_t)v, m, 64);
    int hi = __shfl_xor((int)(uint32_t)(v >> 32), m, 64);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// Bitonic sort of one key per lane, descending by lane (wave64).
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t key, int lane) {
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            uint64_t o = shfl_xor64(key, j);
            bool take_max = ((lane & j) == 0) == ((lane & k) == 0);
            uint64_t mx = key > o ? key : o;
            uint64_t mn = key > o ? o : key;
            key = take_max ? mx : mn;
        }
    }
    return key;
}

// Bitonic sort of n (power of two) keys in LDS, descending; whole workgroup.
__device__ void lds_sort_desc(uint64_t* s, int n) {
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < (n >> 1); i += blockDim.x) {
                int a = 2 * i - (i & (j - 1));
                int c = a + j;
                uint64_t x = s[a], y = s[c];
                bool desc = (a & k) == 0;
                if (desc ? (x < y) : (x > y)) {
                    s[a] = y;
                    s[c] = x;
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ int pow2_ceil(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

// Final merge of the per-tile top-k lists, run by the last workgroup.
// Keys are unique (they carry the row), so an entry at position i of a list
// whose head ranks h-th among all heads has at least h+i better keys: only
// i < kk - h can reach the top kk, at most kk(kk+1)/2 candidates.
__device__ void topk_merge(const Bfp8GemvDesc& d, int ntiles, uint64_t* s) {
    const int kk = d.topk;
    __shared__ int s_list[BFP8_TOPK_MAX];
    const int np = pow2_ceil(ntiles);
    for (int i = threadIdx.x; i < np; i += blockDim.x)
        s[i] = (i < ntiles) ? __builtin_nontemporal_load(&d.partials[(size_t)i * kk]) : 0ull;
    __syncthreads();
    lds_sort_desc(s, np);
    if ((int)threadIdx.x < kk) {
        uint64_t h = ((int)threadIdx.x < np) ? s[threadIdx.x] : 0ull;
        s_list[threadIdx.x] = h ? (key_id(h) / BFP8_TILE_ROWS) : -1;
    }
    __syncthreads();
    const int ncand = kk * (kk + 1) / 2;
    const int nc = pow2_ceil(ncand);
    for (int i = threadIdx.x; i < nc; i += blockDim.x) {
        uint64_t v = 0;
        if (i < ncand) {
            int h = 0, off = 0;
            while (off + (kk - h) <= i) {
                off += kk - h;
                ++h;
            }
            int list = s_list[h];
            if (list >= 0) v = __builtin_nontemporal_load(&d.partials[(size_t)list * kk + (i - off)]);
        }
        s[i] = v;
    }
    __syncthreads();
    lds_sort_desc(s, nc);
    if (threadIdx.x < 64) {
        int lane = threadIdx.x;
        uint64_t v = (lane < kk) ? s[lane] : 0ull;
        unsigned long long valid = __ballot(v != 0);
        int cnt = __popcll(valid);
        if (lane < kk) {
            d.out_ids[lane] = v ? key_id(v) : -1;
            d.out_scores[lane] = v ? key_score(v) : 0.0f;
        }
        if (lane == 0) {
            *d.out_count = cnt;
            // lm_head_argmax: lowest id among maxima above -1e30, else 0
            // (04/qwen_kernels_opt.c:402-403, :483-490)
            *d.out_argmax = (v && key_score(v) > -1e30f) ? key_id(v) : 0;
        }
    }
}

// ---- one 64-row tile --------------------------------------------------------
// Returns y of row 64t+lane in wavefront 0 (unspecified in the others).
__device__ __forceinline__ float gemv_tile(const Bfp8GemvDesc& d, int t, float* red) {
    const int q = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = threadIdx.x & 63;
    const int nb = d.K >> 6;
    const int nb4 = (nb + 3) >> 2;
    const uint8_t* mtile = d.mant + (size_t)t * nb * 4096u;
    const uint8_t* etile = d.exps + (size_t)t * nb4 * 256u;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(mtile, (uint32_t)nb * 4096u);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(etile, (uint32_t)nb4 * 256u);
    const int wv = q * 1024 + r * 16;
    const int ev = r * 4;
    const sgpr_u32_ptr xs = (sgpr_u32_ptr)(d.xsplit) + q * 8;
    const sgpr_f32_ptr xsc = (sgpr_f32_ptr)(d.xscale);
    const int row = t * BFP8_TILE_ROWS + r;
    int32_t* lanes = d.lanes;

    float fs = 0.0f;
    int b = 0;
    const int nfull = nb & ~(kChunk - 1);
    if (nfull > 0) {
        u32x4 wa[kChunk], wb[kChunk];
        uint32_t ea0, ea1, eb0, eb1;
#pragma unroll
        for (int u = 0; u < kChunk; ++u) wa[u] = load_w(wrs, wv, u * 4096);
        ea0 = load_e(ers, ev, 0);
        ea1 = load_e(ers, ev, 256);
        for (;;) {
            const bool more_a = b + kChunk < nfull;
            if (more_a) {
#pragma unroll
                for (int u = 0; u < kChunk; ++u) wb[u] = load_w(wrs, wv, (b + kChunk + u) * 4096);
                eb0 = load_e(ers, ev, ((b + kChunk) >> 2) * 256);
                eb1 = load_e(ers, ev, ((b + kChunk) >> 2) * 256 + 256);
            }
#pragma unroll
            for (int u = 0; u < kChunk; ++u) {
                int S = residue_sum(wa[u], xs + (b + u) * 32);
                uint32_t e = ((u < 4 ? ea0 : ea1) >> (8 * (u & 3))) & 0xffu;
                fs = epilogue(fs, S, e, xsc[b + u]);
                if (lanes && row < d.M) lanes[((size_t)row * nb + b + u) * 4 + q] = S;
            }
            b += kChunk;
            if (!more_a) break;
            const bool more_b = b + kChunk < nfull;
            if (more_b) {
#pragma unroll
                for (int u = 0; u < kChunk; ++u) wa[u] = load_w(wrs, wv, (b + kChunk + u) * 4096);
                ea0 = load_e(ers, ev, ((b + kChunk) >> 2) * 256);
                ea1 = load_e(ers, ev, ((b + kChunk) >> 2) * 256 + 256);
            }
#pragma unroll
            for (int u = 0; u < kChunk; ++u) {
                int S = residue_sum(wb[u], xs + (b + u) * 32);
                uint32_t e = ((u < 4 ? eb0 : eb1) >> (8 * (u & 3))) & 0xffu;
                fs = epilogue(fs, S, e, xsc[b + u]);
                if (lanes && row < d.M) lanes[((size_t)row * nb + b + u) * 4 + q] = S;
            }
            b += kChunk;
            if (!more_b) break;
        }
    }
    for (; b < nb; ++b) {  // remainder blocks (K/64 not a multiple of 8)
        u32x4 w = load_w(wrs, wv, b * 4096);
        uint32_t e = (load_e(ers, ev, (b >> 2) * 256) >> (8 * (b & 3))) & 0xffu;
        int S = residue_sum(w, xs + b * 32);
        fs = epilogue(fs, S, e, xsc[b]);
        if (lanes && row < d.M) lanes[((size_t)row * nb + b) * 4 + q] = S;
    }

    red[q * 64 + r] = fs;
    __syncthreads();
    float y = 0.0f;
    if (q == 0) {
        // vadd_f32(low, high) then vpadd_f32: (fs0 + fs2) + (fs1 + fs3)
        y = (red[r] + red[128 + r]) + (red[64 + r] + red[192 + r]);
        if (d.y && row < d.pair_rows) d.y[row] = y;
    }
    return y;
}

__device__ __forceinline__ void run_tile(const Bfp8GemvDesc& d, int t, float* red, uint64_t* sbuf) {
    const float y = gemv_tile(d, t, red);
    if (d.topk <= 0) return;
    const int ntiles = (d.M + BFP8_TILE_ROWS - 1) / BFP8_TILE_ROWS;
    const int lane = threadIdx.x & 63;
    if (threadIdx.x < 64) {
        const int row = t * BFP8_TILE_ROWS + lane;
        uint64_t key = (row < d.pair_rows) ? topk_key(y, row) : 0ull;
        key = wave_sort_desc(key, lane);
        if (lane < d.topk) d.partials[(size_t)t * d.topk + lane] = key;
    }
    __threadfence();
    __syncthreads();
    __shared__ int s_last;
    if (threadIdx.x == 0) {
        unsigned prev = atomicAdd(d.counter, 1u);
        s_last = (prev == (unsigned)(ntiles - 1));
    }
    __syncthreads();
    if (s_last) {
        __threadfence();
        topk_merge(d, ntiles, sbuf);
        if (threadIdx.x == 0) atomicExch(d.counter, 0u);
    }
}

}  // namespace

// Single GEMV: grid = ntiles(M) workgroups of 256.
extern "C" __global__ __launch_bounds__(256) void bfp8_gemv_kernel(Bfp8GemvDesc d) {
    __shared__ float red[256];
    extern __shared__ uint64_t sbuf[];
    run_tile(d, blockIdx.x, red, sbuf);
}

// Grouped GEMV: one workgroup per (GEMV, tile) entry of the tile table.
extern "C" __global__ __launch_bounds__(256) void bfp8_gemv_grouped_kernel(
    const Bfp8GemvDesc* __restrict__ descs, const Bfp8TileRef* __restrict__ tiles) {
    __shared__ float red[256];
    extern __shared__ uint64_t sbuf[];
    const Bfp8TileRef tr = tiles[blockIdx.x];
    const Bfp8GemvDesc d = descs[tr.desc];
    run_tile(d, tr.tile, red, sbuf);
}

// Batched GEMV: B activation vectors against one weight matrix, weights read
// once.  Activations of a chunk of 8 blocks for all B vectors are staged in
// LDS (wave-uniform broadcast reads); each lane keeps B residue accumulators.
template <int B>
__global__ __launch_bounds__(256) void bfp8_gemv_batch_kernel(float* __restrict__ Y,
                                                              const uint32_t* __restrict__ xsplit,
                                                              const float* __restrict__ xscale,
                                                              const uint8_t* __restrict__ mant,
                                                              const uint8_t* __restrict__ exps, int M,
                                                              int K) {
    __shared__ uint32_t xl[B * kChunk * 32];
    __shared__ float red[4 * 64 * B];
    const int q = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = threadIdx.x & 63;
    const int t = blockIdx.x;
    const int nb = K >> 6;
    const int nb4 = (nb + 3) >> 2;
    const uint8_t* mtile = mant + (size_t)t * nb * 4096u;
    const uint8_t* etile = exps + (size_t)t * nb4 * 256u;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(mtile, (uint32_t)nb * 4096u);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(etile, (uint32_t)nb4 * 256u);
    const int wv = q * 1024 + r * 16;
    const int xwords = nb * 32;
    float fs[B];
#pragma unroll
    for (int v = 0; v < B; ++v) fs[v] = 0.0f;

    for (int b0 = 0; b0 < nb; b0 += kChunk) {
        const int nbc = min(kChunk, nb - b0);
        u32x4 w[kChunk];
        uint32_t ew[2] = {0u, 0u};
#pragma unroll
        for (int u = 0; u < kChunk; ++u)
            if (u < nbc) w[u] = load_w(wrs, wv, (b0 + u) * 4096);
        ew[0] = load_e(ers, r * 4, (b0 >> 2) * 256);
        if (nbc > 4) ew[1] = load_e(ers, r * 4, (b0 >> 2) * 256 + 256);
        __syncthreads();  // previous chunk's LDS reads are done
        for (int i = threadIdx.x; i < B * nbc * 32; i += 256) {
            int v = i / (nbc * 32), o = i - v * nbc * 32;
            xl[v * kChunk * 32 + o] = xsplit[(size_t)v * xwords + b0 * 32 + o];
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            if (u >= nbc) break;
            const uint32_t e = (ew[u >> 2] >> (8 * (u & 3))) & 0xffu;
            const float sc = exp_scale_ftz(e);
#pragma unroll
            for (int v = 0; v < B; ++v) {
                const uint32_t* xb = xl + (v * kChunk + u) * 32 + q * 8;
                const uint4 h = *reinterpret_cast<const uint4*>(xb);
                const uint4 l = *reinterpret_cast<const uint4*>(xb + 4);
                int acc = __builtin_amdgcn_sdot4((int)w[u].x, (int)h.x, 0, false);
                acc = __builtin_amdgcn_sdot4((int)w[u].y, (int)h.y, acc, false);
                acc = __builtin_amdgcn_sdot4((int)w[u].z, (int)h.z, acc, false);
                acc = __builtin_amdgcn_sdot4((int)w[u].w, (int)h.w, acc, false);
                acc = (int)((uint32_t)acc << 8);
                acc = __builtin_amdgcn_sdot4((int)w[u].x, (int)l.x, acc, false);
                acc = __builtin_amdgcn_sdot4((int)w[u].y, (int)l.y, acc, false);
                acc = __builtin_amdgcn_sdot4((int)w[u].z, (int)l.z, acc, false);
                acc = __builtin_amdgcn_sdot4((int)w[u].w, (int)l.w, acc, false);
                float t1 = (float)acc * sc;
                float t2 = t1 * xscale[(size_t)v * nb + b0 + u];
                fs[v] = fs[v] + t2;
            }
        }
    }
#pragma unroll
    for (int v = 0; v < B; ++v) red[(v * 4 + q) * 64 + r] = fs[v];
    __syncthreads();
    const int pair_rows = M & ~1;
    for (int i = threadIdx.x; i < B * 64; i += 256) {
        int v = i >> 6, rr = i & 63;
        int row = t * 64 + rr;
        const float* p = red + v * 256;
        float y = (p[rr] + p[128 + rr]) + (p[64 + rr] + p[192 + rr]);
        if (row < pair_rows) Y[(size_t)v * M + row] = y;
    }
}

// ---- launchers ---------------------------------------------------------------
hipError_t bfp8_launch_gemv(const Bfp8GemvDesc& d, hipStream_t s) {
    const int nt = bfp8_ntiles(d.M);
    if (nt == 0) return hipSuccess;
    const size_t lds = d.topk > 0 ? BFP8_TOPK_LDS_BYTES : 0;
    hipLaunchKernelGGL(bfp8_gemv_kernel, dim3(nt), dim3(256), lds, s, d);
    return hipGetLastError();
}

hipError_t bfp8_launch_gemv_grouped(const Bfp8GemvDesc* descs_dev, const Bfp8TileRef* tiles_dev,
                                    int ntiles, bool any_topk, hipStream_t s) {
    if (ntiles <= 0) return hipSuccess;
    const size_t lds = any_topk ? BFP8_TOPK_LDS_BYTES : 0;
    hipLaunchKernelGGL(bfp8_gemv_grouped_kernel, dim3(ntiles), dim3(256), lds, s, descs_dev,
                       tiles_dev);
    return hipGetLastError();
}

template <int B>
static hipError_t launch_batch_t(float* Y, const uint32_t* xsplit, const float* xscale,
                                 const uint8_t* mant, const uint8_t* exps, int M, int K,
                                 hipStream_t s) {
    hipLaunchKernelGGL(bfp8_gemv_batch_kernel<B>, dim3(bfp8_ntiles(M)), dim3(256), 0, s, Y, xsplit,
                       xscale, mant, exps, M, K);
    return hipGetLastError();
}

hipError_t bfp8_launch_gemv_batch(float* Y, const uint32_t* xsplit, const float* xscale,
                                  const uint8_t* mant, const uint8_t* exps, int M, int K, int B,
                                  hipStream_t s) {
    if (bfp8_ntiles(M) == 0) return hipSuccess;
    switch (B) {
        case 1: return launch_batch_t<1>(Y, xsplit, xscale, mant, exps, M, K, s);
        case 2: return launch_batch_t<2>(Y, xsplit, xscale, mant, exps, M, K, s);
        case 4: return launch_batch_t<4>(Y, xsplit, xscale, mant, exps, M, K, s);
        case 8: return launch_batch_t<8>(Y, xsplit, xscale, mant, exps, M, K, s);
        case 16: return launch_batch_t<16>(Y, xsplit, xscale, mant, exps, M, K, s);
        default: return hipErrorInvalidValue;
    }
}
