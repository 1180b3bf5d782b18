// fused_gemv.hip -- the forward's GEMVs over 16-row sub-tiles, each workgroup
// also producing the GEMV's activation itself.
//
// A decode layer is a chain of small dependent GEMVs (1024 to 8192 rows):
// per launch there are too few 64-row tiles to keep the chip busy, and the
// rmsnorm / swiglu that produce each GEMV's input were launches of their own.
// Here a workgroup of 16 wavefronts owns 16 rows of one GEMV (four times the
// workgroups of a 64-row tile; 4 or 8 rows, or 32, where that puts one
// workgroup on each CU), issues all of its weight loads first, and
// while they are in flight computes the activation the reference computes
// before that GEMV -- rmsnorm(h + residual) (04/qwen_kernels_opt.c:140-175,
// :386-393) or swiglu(gate, up) (:363-384) -- and quantizes it
// (:182-205) into LDS.  Every workgroup computes the same vector with the
// same operations, so every one quantizes it identically; workgroup 0 also
// writes the float results the rest of the layer reads.
//
// Per lane (sub-tiles of R = 16, 8 or 4 rows): row lane % R of the
// sub-tile, residue q = (lane / R) % 4, block lane / (4R) of the wavefront's
// 16 / R; the R * 16-byte row slices of the residue chunks form one wavefront
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
constexpr int kTermPitch = kMaxNb + 4;        // floats per (row, residue) chain of terms (16-byte rows)
static_assert(4 * kThreads >= RT_ROWS_MAX_K, "four activation elements per thread cover K");

struct RowsLds {
    __attribute__((aligned(16))) uint32_t xs[kMaxNb * 32];  // split activation records
    float xsc[kMaxNb];                                       // block scales
    // t2 per chain (sub-tile, residue, row) and block; -0.0 past the last block
    __attribute__((aligned(16))) float terms[128][kTermPitch];
    __attribute__((aligned(16))) float sq[4][kChunk / 4 + 4];  // rmsnorm's squares, one row per residue
    float gp[RT_HEADS][4][36];  // the gated norm's per-head products (16-byte rows)
    float gr[RT_HEADS];         // ... and per-head scales
    float scale;
};

// The activation: thread tid holds elements e = 4 tid + j (j < 4), so a row
// of 16 lanes holds one 64-element block (block tid / 16, element 4 (tid %
// 16) + j) and quantizes it with one row-wide maximum.  Elements past the
// whole blocks are clamped reads, never stored.

// The prologue's inputs, loaded before the weights: a wavefront's loads
// complete in order, so waiting for these must not wait for the weights.
struct PrologueIn {
    float a[4], b[4], c[4];  // norm: h, res, w; swiglu: gate, up; gated: attn, silu(z), w; float: x
};

// First element of this thread's four, clamped to the whole blocks.
__device__ __forceinline__ int prologue_base(int nb) { return min(4 * (int)threadIdx.x, nb * 64 - 4); }

template <int kMode>
__device__ __forceinline__ void load_prologue(const RtRowsArgs& a, PrologueIn& in) {
    // Indices are clamped rather than predicated: a branch around a load
    // joined with another write of its register would force a wait for it.
    const int e0 = prologue_base(a.K >> 6);
    if constexpr (kMode == RT_ROWS_NORM) {
        const float* res = a.res ? a.res : a.h;  // no residual: the add below is skipped
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            in.a[j] = a.h[e0 + j];
            in.b[j] = res[e0 + j];
            in.c[j] = a.w[e0 + j];
        }
    } else if constexpr (kMode == RT_ROWS_SWIGLU) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            in.a[j] = a.gate[e0 + j];
            in.b[j] = a.up[e0 + j];
        }
    } else if constexpr (kMode == RT_ROWS_GATED) {  // two elements per thread: e = 2 tid + j
        const int g0 = min(2 * (int)threadIdx.x, a.K - 2);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            in.a[j] = a.attn[g0 + j];
            in.b[j] = a.zsilu[g0 + j];
            in.c[j] = a.w[(g0 + j) & (RT_HEAD_DIM - 1)];
        }
    } else if constexpr (kMode == RT_ROWS_FLOAT) {
#pragma unroll
        for (int j = 0; j < 4; ++j) in.a[j] = a.x[e0 + j];
    } else {  // the records as given: words tid, tid + kThreads; scales tid
        const int nb = a.K >> 6, tid = threadIdx.x;
        in.a[0] = __uint_as_float(a.xsplit[min(tid, nb * 32 - 1)]);
        in.a[1] = __uint_as_float(a.xsplit[min(tid + kThreads, nb * 32 - 1)]);
        in.b[0] = a.xscale[min(tid, nb - 1)];
    }
}

// Quantizes this row's block (y: the thread's four elements) into the LDS
// activation when the block is one of the nb whole blocks.
__device__ __forceinline__ void quant_row_lds(const float (&y)[4], int nb, RowsLds& L) {
    const int tid = threadIdx.x, b = tid >> 4;
    bfp8_quant4_store_lds(y, tid & 15, &L.xsc[min(b, nb - 1)], &L.xs[min(b, nb - 1) * 32], b < nb);
}

// rmsnorm of x = h (+ res) into the LDS activation (n = K, a multiple of 64).
__device__ __forceinline__ void norm_prologue(const RtRowsArgs& a, const PrologueIn& in, RowsLds& L) {
    const int tid = threadIdx.x, n = a.K, nb = n >> 6, lane = lane_id();
    const bool w0 = tid < 64, mine = 4 * tid < n;
    float x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = a.res ? in.a[j] + in.b[j] : in.a[j];  // add_residual's vector add
    // sum of squares in the 4-lane order (element e = 4m + j feeds lane j, m
    // ascending), kChunk elements per pass; lanes 0-3 of wavefront 0 keep the
    // four sums
    float s = 0.0f;
    for (int base = 0; base < n; base += kChunk) {
        const int m = tid - base / 4;  // this thread's position in the pass
        if (mine && m >= 0 && m < kChunk / 4) {
#pragma unroll
            for (int j = 0; j < 4; ++j) L.sq[j][m] = x[j] * x[j];
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
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) y[j] = x[j] * (r * (1.0f + in.c[j]));
    if (first && mine) {
        const int e0 = 4 * tid;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (a.h_out) a.h_out[e0 + j] = x[j];
            if (a.y_norm) a.y_norm[e0 + j] = y[j];
        }
    }
    quant_row_lds(y, nb, L);
}

// rmsnorm_gated(attn, z) over heads of 128 (04/qwen_kernels_opt.c:818-847)
// into the LDS activation (n = 16 * 128).  Per head: the 4-lane sum of
// squares (one lane per head and residue, all 64 lanes of wavefront 0), the
// scalar scale, then ((x * r) * w) * silu(z) per element in IEEE arithmetic
// (silu(z) computed once by the attention kernel) -- two elements per thread
// (e = 2 tid + j), staged in LDS for the four-element rows of the quantizer.
__device__ __forceinline__ void gated_prologue(const RtRowsArgs& a, const PrologueIn& in, RowsLds& L) {
    const int tid = threadIdx.x, n = a.K, nb = n >> 6;
    const bool mine = 2 * tid < n;
    const int head = min(2 * tid / RT_HEAD_DIM, RT_HEADS - 1);
    if (mine) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int i = (2 * tid + j) & (RT_HEAD_DIM - 1);
            L.gp[head][i & 3][i >> 2] = in.a[j] * in.a[j];
        }
    }
    __syncthreads();
    if (tid < 64) {
        float s = 0.0f;
#pragma unroll
        for (int mm = 0; mm < RT_HEAD_DIM / 4; mm += 4) {
            const float4 v = *reinterpret_cast<const float4*>(&L.gp[tid >> 2][tid & 3][mm]);
            s = s + v.x;
            s = s + v.y;
            s = s + v.z;
            s = s + v.w;
        }
        const float r = lanes4_combine(s);
        if ((tid & 3) == 0) L.gr[tid >> 2] = rms_scale(r, RT_HEAD_DIM, a.eps);
    }
    __syncthreads();
    // the products staged where the terms go later (written after the
    // barrier that ends the prologue)
    float* ys = &L.terms[0][0];
    const float gr = L.gr[head];
    if (mine) {
#pragma unroll
        for (int j = 0; j < 2; ++j) ys[2 * tid + j] = gated_mul(in.a[j], gr, in.c[j], in.b[j]);
    }
    __syncthreads();
    const float4 v = *reinterpret_cast<const float4*>(&ys[prologue_base(nb)]);
    const float y[4] = {v.x, v.y, v.z, v.w};
    quant_row_lds(y, nb, L);
}

// swiglu(gate, up) into the LDS activation.
__device__ __forceinline__ void swiglu_prologue(const RtRowsArgs& a, const PrologueIn& in, RowsLds& L) {
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) y[j] = swiglu_elem(in.a[j], in.b[j], true);  // n % 4 == 0: all vector part
    quant_row_lds(y, a.K >> 6, L);
}

// x as given (quant_x_blocks, 04/qwen_kernels_opt.c:182-205) into the LDS
// activation: the K / 64 whole blocks.
__device__ __forceinline__ void float_prologue(const RtRowsArgs& a, const PrologueIn& in, RowsLds& L) {
    quant_row_lds(in.a, a.K >> 6, L);
}

}  // namespace

// Sub-tiles of kR rows (16, 8 or 4) per workgroup, kSub of them (2 only with
// kR = 16, when a launch would otherwise put more than one workgroup on a CU):
// the sub-tiles share the prologue.  Fewer rows per workgroup spread a small
// GEMV over more CUs, with fewer weight loads per lane before the terms (a
// long-K GEMV such as 1024 x 3584 has one instead of four); a wavefront load
// then covers 16 / kR blocks of kR rows.
//
// With kR = 4 a row slice run is 64 bytes, half a 128-byte line whose other
// half belongs to the neighbouring sub-tile.  Workgroups are dealt to the 8
// XCDs round-robin by id, so the two sub-tiles of a line go to workgroup ids
// 16p + x and 16p + x + 8 (one XCD, one L2) when the grid allows it.  (All of
// a tile's workgroups on one XCD would also share its exponent lines: 4 %
// less traffic at 1024 x 3584, but 0.2 us slower.)
template <int kR>
__device__ __forceinline__ int rows_group(int grid) {
    const int x = (int)blockIdx.x;
    if (kR != 4 || (grid & 15)) return x;
    return 2 * ((x >> 4) * 8 + (x & 7)) + ((x >> 3) & 1);
}

// kPer = ceil(K / kThreads) >= nb / kWaves sizes the weight loads (kLd per
// wavefront and sub-tile, each issued unconditionally with a clamped index,
// so the compiler can count them and wait for exactly the ones it needs) and
// the sums (kNb terms per chain).
template <int kMode, int kPer, int kSub, int kR>
__global__ __launch_bounds__(kThreads) void rt_rows_gemv_kernel(RtRowsArgs a) {
    static_assert(kR == 16 || kR == 8 || kR == 4, "sub-tile rows");
    static_assert(kSub == 1 || kR == 16, "two sub-tiles only of 16 rows");
    constexpr int kBpl = 16 / kR;                   // blocks per wavefront load
    constexpr int kLd = (kPer + kBpl - 1) / kBpl;   // loads per wavefront and sub-tile
    constexpr int kChains = kSub * 4 * kR;          // (row, residue) sums of the workgroup
    __shared__ RowsLds L;
    const int w = __builtin_amdgcn_readfirstlane(wave_id());
    const int lane = lane_id();
    const int grp = rows_group<kR>((int)gridDim.x);
    const bool second = a.ngemv > 1 && grp >= a.split;
    const RtRowsGemv G = second ? a.g[1] : a.g[0];
    const int s0 = (grp - (second ? a.split : 0)) * kSub;  // first sub-tile
    const int t = (s0 * kR) >> 6, rin = (s0 * kR) & 63;   // its 64-row tile and first row there
    const int nb = a.K >> 6, nb4 = (nb + 3) >> 2;
    const int r = lane % kR, q = (lane / kR) & 3, blk = lane / (4 * kR);

    // 0. the activation's inputs, then 1. this wavefront's weight blocks
    // (w + kWaves * i) * kBpl + blk of every sub-tile, all in flight
    PrologueIn in;
    load_prologue<kMode>(a, in);
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(G.mant + (size_t)t * nb * 4096u, (uint32_t)nb * 4096u);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(G.exps + (size_t)t * nb4 * 256u, (uint32_t)nb4 * 256u);
    u32x4 wv[kSub][kLd];
    uint32_t ev[kSub][kLd];
#pragma unroll
    for (int j = 0; j < kSub; ++j) {
        const int row = rin + j * kR + r;
#pragma unroll
        for (int i = 0; i < kLd; ++i) {
            const int b = min((w + kWaves * i) * kBpl + blk, nb - 1);
            wv[j][i] = load_w(wrs, b * 4096 + q * 1024 + row * 16, 0);
            ev[j][i] = load_e(ers, (b >> 2) * 256 + row * 4, 0);
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
        const int tid = threadIdx.x;
        if (tid < nb * 32) L.xs[tid] = __float_as_uint(in.a[0]);
        if (tid + kThreads < nb * 32) L.xs[tid + kThreads] = __float_as_uint(in.a[1]);
        if (tid < nb) L.xsc[tid] = in.b[0];
    }
    __syncthreads();
    if constexpr (kMode == RT_ROWS_FLOAT) {
        if (blockIdx.x == 0 && a.xsplit_out) {
            const int tid = threadIdx.x;
            if (tid < nb * 32) a.xsplit_out[tid] = L.xs[tid];
            if (tid + kThreads < nb * 32) a.xsplit_out[tid + kThreads] = L.xs[tid + kThreads];
            if (tid < nb) a.xscale_out[tid] = L.xsc[tid];
        }
    }

    // 3. per-block terms, and -0.0 for the blocks from nb to kNb (they cover
    // them: kWaves * kBpl * kLd >= kNb), which leaves the sums unchanged
    constexpr int kNb = kPer * kWaves;  // nb <= kWaves * ceil(K / kThreads)
    const int chain = lane % (4 * kR);
#pragma unroll
    for (int i = 0; i < kLd; ++i) {
        const int b = (w + kWaves * i) * kBpl + blk;
        if (b >= nb && b < kNb) {
#pragma unroll
            for (int j = 0; j < kSub; ++j) L.terms[j * 4 * kR + chain][b] = -0.0f;
        }
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
                L.terms[j * 4 * kR + chain][b] = t1 * xsb;
            }
        }
    }
    __syncthreads();

    // 4. block-order sums per (row, q): chain c = q * kR + r of sub-tile j at
    // j * 4 * kR + c, one lane each -- then the reference's lane combination
    if (w * 64 < kChains) {
        const int c = w * 64 + lane;
        float fs = 0.0f;
        if (c < kChains) {
            // every term read first (16-byte reads, one LDS wait), then the
            // dependent adds in block order; the -0.0 past nb change nothing
            float4 v[kNb / 4];
#pragma unroll
            for (int i = 0; i < kNb / 4; ++i) v[i] = *reinterpret_cast<const float4*>(&L.terms[c][4 * i]);
#pragma unroll
            for (int i = 0; i < kNb / 4; ++i) {
                fs = fs + v[i].x;
                fs = fs + v[i].y;
                fs = fs + v[i].z;
                fs = fs + v[i].w;
            }
        }
        // wavefront w holds sub-tile w (kR = 16) or the whole workgroup (w = 0)
        const int rr = lane % kR;
        const float f0 = __shfl(fs, rr, 64), f1 = __shfl(fs, kR + rr, 64);
        const float f2 = __shfl(fs, 2 * kR + rr, 64), f3 = __shfl(fs, 3 * kR + rr, 64);
        const int row = t * 64 + rin + w * kR + lane;
        if (lane < kR && row < G.pair_rows) G.y[row] = (f0 + f2) + (f1 + f3);
    }
}

namespace {

template <int kMode, int kPer>
hipError_t launch_rows(const RtRowsArgs& b, int rows, int sub, dim3 grid, hipStream_t s) {
    const dim3 block(kThreads);
    if (sub == 2)
        hipLaunchKernelGGL((rt_rows_gemv_kernel<kMode, kPer, 2, 16>), grid, block, 0, s, b);
    else if (rows == 16)
        hipLaunchKernelGGL((rt_rows_gemv_kernel<kMode, kPer, 1, 16>), grid, block, 0, s, b);
    else if (rows == 8)
        hipLaunchKernelGGL((rt_rows_gemv_kernel<kMode, kPer, 1, 8>), grid, block, 0, s, b);
    else
        hipLaunchKernelGGL((rt_rows_gemv_kernel<kMode, kPer, 1, 4>), grid, block, 0, s, b);
    return hipGetLastError();
}

// kPer = ceil(K / kThreads) from 1 to RT_ROWS_MAX_K / kThreads
template <int kMode, int kPer = 1>
hipError_t launch_rows_per(const RtRowsArgs& b, int per, int rows, int sub, dim3 grid, hipStream_t s) {
    if (per == kPer) return launch_rows<kMode, kPer>(b, rows, sub, grid, s);
    if constexpr (kPer < RT_ROWS_MAX_K / kThreads)
        return launch_rows_per<kMode, kPer + 1>(b, per, rows, sub, grid, s);
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t rt_launch_rows(const RtRowsArgs& a, hipStream_t s) {
    // a given or float activation uses the K / 64 whole blocks (as the
    // reference does); one computed from other inputs covers exactly K elements
    if (a.K < 64 || a.K > RT_ROWS_MAX_K || ((a.K & 63) && a.mode != RT_ROWS_QUANTIZED && a.mode != RT_ROWS_FLOAT) ||
        a.ngemv < 1 || a.ngemv > 2 || (a.mode == RT_ROWS_FLOAT && a.xsplit_out && !a.xscale_out))
        return hipErrorInvalidValue;
    if (a.mode == RT_ROWS_GATED && a.K != RT_HEADS * RT_HEAD_DIM) return hipErrorInvalidValue;
    const int n0 = (a.g[0].M + 15) / 16, n1 = a.ngemv > 1 ? (a.g[1].M + 15) / 16 : 0;
    if (a.ngemv > 1 && a.split != n0) return hipErrorInvalidValue;
    // workgroups of R rows for the GEMVs: one per CU at most (a second one
    // per CU finishes later) -- the fewest rows that fit, else two 16-row
    // sub-tiles per workgroup
    const int cus = bfp8_stream_grid() / 4;
    auto groups = [&](int R) { return (a.g[0].M + R - 1) / R + (a.ngemv > 1 ? (a.g[1].M + R - 1) / R : 0); };
    int rows = 16, sub = 1;
    if (n0 + n1 > cus)
        sub = 2;
    else if (groups(4) <= cus)
        rows = 4;
    else if (groups(8) <= cus)
        rows = 8;
    RtRowsArgs b = a;
    const int R = rows * sub;
    b.split = (a.g[0].M + R - 1) / R;
    const int n1s = a.ngemv > 1 ? (a.g[1].M + R - 1) / R : 0;
    const dim3 grid((unsigned)(b.split + n1s));
    const int per = (a.K + kThreads - 1) / kThreads;
    switch (a.mode) {
        case RT_ROWS_NORM: return launch_rows_per<RT_ROWS_NORM>(b, per, rows, sub, grid, s);
        case RT_ROWS_SWIGLU: return launch_rows_per<RT_ROWS_SWIGLU>(b, per, rows, sub, grid, s);
        case RT_ROWS_QUANTIZED: return launch_rows_per<RT_ROWS_QUANTIZED>(b, per, rows, sub, grid, s);
        case RT_ROWS_FLOAT: return launch_rows_per<RT_ROWS_FLOAT>(b, per, rows, sub, grid, s);
        case RT_ROWS_GATED: {  // K = 16 * 128 only
            constexpr int kGatedPer = (RT_HEADS * RT_HEAD_DIM + kThreads - 1) / kThreads;
            return per == kGatedPer ? launch_rows<RT_ROWS_GATED, kGatedPer>(b, rows, sub, grid, s)
                                    : hipErrorInvalidValue;
        }
        default: return hipErrorInvalidValue;
    }
}
