// fused_gemv.hip -- the forward's GEMVs over 16-row sub-tiles, each workgroup
// also producing the GEMV's activation itself.
//
// A decode layer is a chain of small dependent GEMVs (1024 to 8192 rows):
// per launch there are too few 64-row tiles to keep the chip busy, and the
// rmsnorm / swiglu that produce each GEMV's input were launches of their own.
// Here a workgroup of 16 wavefronts owns 16 rows of one GEMV (four times the
// workgroups of a 64-row tile), issues all of its weight loads first, and
// while they are in flight computes the activation the reference computes
// before that GEMV -- rmsnorm(h + residual) (04/qwen_kernels_opt.c:140-175,
// :386-393) or swiglu(gate, up) (:363-384) -- and quantizes it
// (:182-205) into LDS.  Every workgroup computes the same vector with the
// same operations, so every one quantizes it identically; workgroup 0 also
// writes the float results the rest of the layer reads.
//
// Per lane: rows 16g + (lane & 15) of the tile, residue q = lane >> 4; the
// four 256-byte row slices of a block's residue chunks form one wavefront
// load.  Per block the exact int32 residue sum (8 v_dot4 + a shift), then
// t2 = (float(S) * 2^(e-134)) * xscale, the reference's per-block term; the
// terms go to LDS and one thread per (row, q) adds them in block order, then
// y = (fs0 + fs2) + (fs1 + fs3): the same arithmetic as bfp8_gemv.
//
// Compiled with f32 flush-to-zero and -ffp-contract=off, like the other GEMV
// and runtime kernels.
#include <hip/hip_runtime.h>

#include "bfp8_internal.h"
#include "gemv_dev.h"
#include "quant_block.h"
#include "runtime_dev.h"
#include "runtime_internal.h"

namespace {

constexpr int kWaves = 16;                    // wavefronts per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kMaxNb = RT_ROWS_MAX_K / 64;    // blocks per row

struct RowsLds {
    __attribute__((aligned(16))) uint32_t xs[kMaxNb * 32];  // split activation records
    float xsc[kMaxNb];                                       // block scales
    float terms[kMaxNb][128];                                // t2 per block and (sub-tile, lane)
    __attribute__((aligned(16))) float sq[4][kChunk / 4 + 4];  // rmsnorm's squares, one row per residue
    float gp[RT_HEADS][4][36];  // the gated norm's per-head products (16-byte rows)
    float gr[RT_HEADS];         // ... and per-head scales
    float scale;
};

// kPer = blocks per wavefront = activation elements per thread = ceil(K / 1024)
// (1, 2 or 4): every load is issued unconditionally (indices clamped), so
// the compiler can count them and wait for exactly the ones it needs.

// The prologue's inputs, loaded before the weights: a wavefront's loads
// complete in order, so waiting for these must not wait for the weights.
// Element e = tid + kThreads * k of the activation.
template <int kE>
struct PrologueIn {
    float a[kE], b[kE], c[kE];  // norm: h, res, w; swiglu: gate, up; quantized: record words, scales
};

template <int kMode, int kE>
__device__ __forceinline__ void load_prologue(const RtRowsArgs& a, PrologueIn<kE>& in) {
    // Indices are clamped rather than predicated: a branch around a load
    // joined with another write of its register would force a wait for it.
    const int tid = threadIdx.x, n = a.K;
    if constexpr (kMode == RT_ROWS_NORM) {
        const float* res = a.res ? a.res : a.h;  // no residual: the add below is skipped
#pragma unroll
        for (int k = 0; k < kE; ++k) {
            const int e = min(tid + kThreads * k, n - 1);
            in.a[k] = a.h[e];
            in.b[k] = res[e];
            in.c[k] = a.w[e];
        }
    } else if constexpr (kMode == RT_ROWS_SWIGLU) {
#pragma unroll
        for (int k = 0; k < kE; ++k) {
            const int e = min(tid + kThreads * k, n - 1);
            in.a[k] = a.gate[e];
            in.b[k] = a.up[e];
        }
    } else if constexpr (kMode == RT_ROWS_GATED) {
#pragma unroll
        for (int k = 0; k < kE; ++k) {
            const int e = min(tid + kThreads * k, n - 1);
            in.a[k] = a.attn[e];
            in.b[k] = a.zsilu[e];
            in.c[k] = a.w[e & (RT_HEAD_DIM - 1)];
        }
    } else if constexpr (kMode == RT_ROWS_FLOAT) {
#pragma unroll
        for (int k = 0; k < kE; ++k) in.a[k] = a.x[min(tid + kThreads * k, n - 1)];
    } else {
        const int nb = n >> 6;
#pragma unroll
        for (int k = 0; k < kE; ++k) {
            const int e = tid + kThreads * k;
            in.a[k] = __uint_as_float(a.xsplit[min(e, nb * 32 - 1)]);
            in.b[k] = a.xscale[min(e, nb - 1)];
        }
    }
}

// rmsnorm of x = h (+ res) into the LDS activation (n = K, a multiple of 64).
template <int kE>
__device__ __forceinline__ void norm_prologue(const RtRowsArgs& a, const PrologueIn<kE>& in, RowsLds& L) {
    const int tid = threadIdx.x, n = a.K, nb = n >> 6, lane = lane_id();
    const bool w0 = tid < 64;
    float x[kE];
#pragma unroll
    for (int k = 0; k < kE; ++k) x[k] = a.res ? in.a[k] + in.b[k] : in.a[k];  // add_residual's vector add
    // sum of squares in the 4-lane order (element e = 4m + j feeds lane j, m
    // ascending), kChunk elements per pass; lanes 0-3 of wavefront 0 keep the
    // four sums
    float s = 0.0f;
    for (int base = 0; base < n; base += kChunk) {
#pragma unroll
        for (int k = 0; k < kE; ++k) {
            const int e = tid + kThreads * k;
            if (e >= base && e < base + kChunk && e < n) L.sq[e & 3][(e - base) >> 2] = x[k] * x[k];
        }
        __syncthreads();
        if (tid < 4) {
            const int cnt = min(kChunk, n - base) >> 2;
            s = (cnt == kChunk / 4) ? chain_add256(s, &L.sq[tid][0]) : chain_add(s, &L.sq[tid][0], cnt);
        }
        if (base + kChunk < n) __syncthreads();
    }
    if (w0) {
        const float r = (readlane_f(s, 0) + readlane_f(s, 2)) + (readlane_f(s, 1) + readlane_f(s, 3));
        if (lane == 0) L.scale = rms_scale(r, n, a.eps);
    }
    __syncthreads();
    const float r = L.scale;
    const bool first = blockIdx.x == 0;
#pragma unroll
    for (int k = 0; k < kE; ++k) {
        const int e = tid + kThreads * k;
        float y = 0.0f;
        if (e < n) {
            y = x[k] * (r * (1.0f + in.c[k]));
            if (first) {
                if (a.h_out) a.h_out[e] = x[k];
                if (a.y_norm) a.y_norm[e] = y;
            }
        }
        const int b = e >> 6;  // one block per wavefront
        if (b < nb) bfp8_quant_block_lds(y, lane, &L.xsc[b], &L.xs[b * 32]);
    }
}

// rmsnorm_gated(attn, z) over heads of 128 (04/qwen_kernels_opt.c:818-847)
// into the LDS activation (n = 16 * 128).  Per head: the 4-lane sum of
// squares (one lane per head and residue, all 64 lanes of wavefront 0), the
// scalar scale, then ((x * r) * w) * silu(z) per element in IEEE arithmetic
// (silu(z) computed once by the attention kernel).
template <int kE>
__device__ __forceinline__ void gated_prologue(const RtRowsArgs& a, const PrologueIn<kE>& in, RowsLds& L) {
    const int tid = threadIdx.x, n = a.K, nb = n >> 6;
#pragma unroll
    for (int k = 0; k < kE; ++k) {
        const int e = tid + kThreads * k;
        if (e < n) {
            const int i = e & (RT_HEAD_DIM - 1);
            L.gp[e / RT_HEAD_DIM][i & 3][i >> 2] = in.a[k] * in.a[k];
        }
    }
    __syncthreads();
    if (tid < 64) {
        float s = 0.0f;
#pragma unroll
        for (int m = 0; m < RT_HEAD_DIM / 4; m += 4) {
            const float4 v = *reinterpret_cast<const float4*>(&L.gp[tid >> 2][tid & 3][m]);
            s = s + v.x;
            s = s + v.y;
            s = s + v.z;
            s = s + v.w;
        }
        const float r = lanes4_combine(s);
        if ((tid & 3) == 0) L.gr[tid >> 2] = rms_scale(r, RT_HEAD_DIM, a.eps);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kE; ++k) {
        const int e = tid + kThreads * k;
        float y = 0.0f;
        if (e < n) y = gated_mul(in.a[k], L.gr[e / RT_HEAD_DIM], in.c[k], in.b[k]);
        const int b = e >> 6;
        if (b < nb) bfp8_quant_block_lds(y, lane_id(), &L.xsc[b], &L.xs[b * 32]);
    }
}

// swiglu(gate, up) into the LDS activation.
template <int kE>
__device__ __forceinline__ void swiglu_prologue(const RtRowsArgs& a, const PrologueIn<kE>& in, RowsLds& L) {
    const int tid = threadIdx.x, n = a.K, nb = n >> 6;
#pragma unroll
    for (int k = 0; k < kE; ++k) {
        const int e = tid + kThreads * k;
        float y = 0.0f;
        if (e < n) y = swiglu_elem(in.a[k], in.b[k], true);  // n % 4 == 0: all vector part
        const int b = e >> 6;
        if (b < nb) bfp8_quant_block_lds(y, lane_id(), &L.xsc[b], &L.xs[b * 32]);
    }
}

// x as given (quant_x_blocks, 04/qwen_kernels_opt.c:182-205) into the LDS
// activation: the K / 64 whole blocks.
template <int kE>
__device__ __forceinline__ void float_prologue(const RtRowsArgs& a, const PrologueIn<kE>& in, RowsLds& L) {
    const int tid = threadIdx.x, nb = a.K >> 6;
#pragma unroll
    for (int k = 0; k < kE; ++k) {
        const int b = (tid + kThreads * k) >> 6;
        if (b < nb) bfp8_quant_block_lds(in.a[k], lane_id(), &L.xsc[b], &L.xs[b * 32]);
    }
}

}  // namespace

// kSub 16-row sub-tiles per workgroup (1, or 2 when a launch would otherwise
// put more than one workgroup on a CU): the sub-tiles share the prologue.
template <int kMode, int kPer, int kSub>
__global__ __launch_bounds__(kThreads) void rt_rows_gemv_kernel(RtRowsArgs a) {
    __shared__ RowsLds L;
    const int w = __builtin_amdgcn_readfirstlane(wave_id());
    const int lane = lane_id();
    const bool second = a.ngemv > 1 && (int)blockIdx.x >= a.split;
    const RtRowsGemv G = second ? a.g[1] : a.g[0];
    const int s0 = ((int)blockIdx.x - (second ? a.split : 0)) * kSub;  // first sub-tile (one 64-row tile holds all)
    const int t = s0 >> 2, g0 = s0 & 3;
    const int nb = a.K >> 6, nb4 = (nb + 3) >> 2;
    const int q = lane >> 4;

    // 0. the activation's inputs, then 1. this wavefront's weight blocks
    // b = w, w + kWaves, ... of every sub-tile, all in flight
    PrologueIn<kPer> in;
    load_prologue<kMode, kPer>(a, in);
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(G.mant + (size_t)t * nb * 4096u, (uint32_t)nb * 4096u);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(G.exps + (size_t)t * nb4 * 256u, (uint32_t)nb4 * 256u);
    u32x4 wv[kSub][kPer];
    uint32_t ev[kSub][kPer];
#pragma unroll
    for (int j = 0; j < kSub; ++j) {
        const int r = (g0 + j) * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int b = min(w + kWaves * i, nb - 1);
            wv[j][i] = load_w(wrs, q * 1024 + r * 16, b * 4096);
            ev[j][i] = load_e(ers, r * 4, (b >> 2) * 256);
        }
    }

    // 2. the activation, quantized, into LDS
    if constexpr (kMode == RT_ROWS_NORM) {
        norm_prologue(a, in, L);
    } else if constexpr (kMode == RT_ROWS_SWIGLU) {
        swiglu_prologue(a, in, L);
    } else if constexpr (kMode == RT_ROWS_GATED) {
        gated_prologue(a, in, L);
    } else if constexpr (kMode == RT_ROWS_FLOAT) {
        float_prologue(a, in, L);
    } else {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int e = threadIdx.x + kThreads * k;
            if (e < nb * 32) L.xs[e] = __float_as_uint(in.a[k]);
            if (e < nb) L.xsc[e] = in.b[k];
        }
    }
    __syncthreads();
    if constexpr (kMode == RT_ROWS_FLOAT) {
        if (blockIdx.x == 0 && a.xsplit_out) {
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int e = threadIdx.x + kThreads * k;
                if (e < nb * 32) a.xsplit_out[e] = L.xs[e];
                if (e < nb) a.xscale_out[e] = L.xsc[e];
            }
        }
    }

    // 3. per-block terms
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int b = w + kWaves * i;
        if (b < nb) {
            const uint4 xh = *reinterpret_cast<const uint4*>(&L.xs[(b * 4 + q) * 8]);
            const uint4 xl = *reinterpret_cast<const uint4*>(&L.xs[(b * 4 + q) * 8 + 4]);
            const float xsb = L.xsc[b];
#pragma unroll
            for (int j = 0; j < kSub; ++j) {
                const u32x4 wq = wv[j][i];
                int S = __builtin_amdgcn_sdot4((int)wq.x, (int)xh.x, 0, false);
                S = __builtin_amdgcn_sdot4((int)wq.y, (int)xh.y, S, false);
                S = __builtin_amdgcn_sdot4((int)wq.z, (int)xh.z, S, false);
                S = __builtin_amdgcn_sdot4((int)wq.w, (int)xh.w, S, false);
                S = (int)((uint32_t)S << 8);
                S = __builtin_amdgcn_sdot4((int)wq.x, (int)xl.x, S, false);
                S = __builtin_amdgcn_sdot4((int)wq.y, (int)xl.y, S, false);
                S = __builtin_amdgcn_sdot4((int)wq.z, (int)xl.z, S, false);
                S = __builtin_amdgcn_sdot4((int)wq.w, (int)xl.w, S, false);
                const uint32_t e = (ev[j][i] >> (8 * (b & 3))) & 0xffu;
                const float t1 = (float)S * exp_scale_ftz(e);
                L.terms[b][j * 64 + lane] = t1 * xsb;
            }
        }
    }
    __syncthreads();

    // 4. block-order sums per (row, q) -- wavefront j for sub-tile j -- then
    // the reference's lane combination
    if (w < kSub) {
        float fs = 0.0f;
        int b = 0;
        const int c = w * 64 + lane;
        for (; b + 8 <= nb; b += 8) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = L.terms[b + k][c];
#pragma unroll
            for (int k = 0; k < 8; ++k) fs = fs + v[k];
        }
        for (; b < nb; ++b) fs = fs + L.terms[b][c];
        const int rr = lane & 15;
        const float f0 = __shfl(fs, rr, 64), f1 = __shfl(fs, 16 + rr, 64);
        const float f2 = __shfl(fs, 32 + rr, 64), f3 = __shfl(fs, 48 + rr, 64);
        const int row = t * 64 + (g0 + w) * 16 + lane;
        if (lane < 16 && row < G.pair_rows) G.y[row] = (f0 + f2) + (f1 + f3);
    }
}

hipError_t rt_launch_rows(const RtRowsArgs& a, hipStream_t s) {
    // a given or float activation uses the K / 64 whole blocks (as the
    // reference does); one computed from other inputs covers exactly K elements
    if (a.K < 64 || a.K > RT_ROWS_MAX_K || ((a.K & 63) && a.mode != RT_ROWS_QUANTIZED && a.mode != RT_ROWS_FLOAT) ||
        a.ngemv < 1 || a.ngemv > 2 || (a.mode == RT_ROWS_FLOAT && a.xsplit_out && !a.xscale_out))
        return hipErrorInvalidValue;
    if (a.mode == RT_ROWS_GATED && a.K != RT_HEADS * RT_HEAD_DIM) return hipErrorInvalidValue;
    const int n0 = (a.g[0].M + 15) / 16, n1 = a.ngemv > 1 ? (a.g[1].M + 15) / 16 : 0;
    if (a.ngemv > 1 && a.split != n0) return hipErrorInvalidValue;
    // more 16-row workgroups than CUs: two sub-tiles per workgroup, one
    // workgroup per CU (a second one per CU finishes later)
    const int sub = (n0 + n1 > bfp8_stream_grid() / 4) ? 2 : 1;
    RtRowsArgs b = a;
    b.split = (a.g[0].M + 16 * sub - 1) / (16 * sub);
    const int n1s = a.ngemv > 1 ? (a.g[1].M + 16 * sub - 1) / (16 * sub) : 0;
    const dim3 grid((unsigned)(b.split + n1s)), block(kThreads);
    const int per = (a.K + 1023) / 1024;
#define RT_ROWS_CASE(MODE, PER)                                                                                \
    if (a.mode == MODE && per == PER && sub == 1)                                                              \
        hipLaunchKernelGGL((rt_rows_gemv_kernel<MODE, PER, 1>), grid, block, 0, s, b);                         \
    else if (a.mode == MODE && per == PER && sub == 2)                                                         \
        hipLaunchKernelGGL((rt_rows_gemv_kernel<MODE, PER, 2>), grid, block, 0, s, b)
    RT_ROWS_CASE(RT_ROWS_NORM, 1);
    else RT_ROWS_CASE(RT_ROWS_NORM, 2);
    else RT_ROWS_CASE(RT_ROWS_NORM, 3);
    else RT_ROWS_CASE(RT_ROWS_NORM, 4);
    else RT_ROWS_CASE(RT_ROWS_SWIGLU, 1);
    else RT_ROWS_CASE(RT_ROWS_SWIGLU, 2);
    else RT_ROWS_CASE(RT_ROWS_SWIGLU, 3);
    else RT_ROWS_CASE(RT_ROWS_SWIGLU, 4);
    else RT_ROWS_CASE(RT_ROWS_QUANTIZED, 1);
    else RT_ROWS_CASE(RT_ROWS_QUANTIZED, 2);
    else RT_ROWS_CASE(RT_ROWS_QUANTIZED, 3);
    else RT_ROWS_CASE(RT_ROWS_QUANTIZED, 4);
    else RT_ROWS_CASE(RT_ROWS_GATED, 2);
    else RT_ROWS_CASE(RT_ROWS_FLOAT, 1);
    else RT_ROWS_CASE(RT_ROWS_FLOAT, 2);
    else RT_ROWS_CASE(RT_ROWS_FLOAT, 3);
    else RT_ROWS_CASE(RT_ROWS_FLOAT, 4);
    else return hipErrorInvalidValue;
#undef RT_ROWS_CASE
    return hipGetLastError();
}
