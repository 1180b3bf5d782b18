// runtime_ftz.hip -- the decode runtime around the GEMV
// (04/qwen_kernels_opt.c:140-175, :328-398, :511-860): rmsnorm, swiglu,
// causal conv1d + SiLU, q/k L2 norm, GDN gates, GDN recurrent step, gated
// RMSNorm, residual add, and the fused per-layer kernels of the
// device-resident forward.
//
// Compiled with f32 flush-to-zero and -ffp-contract=off: a plain float
// operation here is one Advanced SIMD operation of the reference (vmulq,
// vaddq, vsubq; vmlaq = product rounded, then sum rounded).  The reference's
// scalar VFP steps keep IEEE subnormals; they go through ieee_*() below,
// which compute in double and round once to float by hand, so they do not
// depend on the f32 denormal mode.  expf / log1pf of the reference's libm are
// taken as exp / log1p in double rounded to float.
//
// Reductions follow the reference's 4-lane accumulators: lane j adds the
// products of elements 4m + j in ascending m (one rounding per add), and the
// lanes combine as (l0 + l2) + (l1 + l3) (vadd of the halves, then vpadd).
#include <hip/hip_runtime.h>

#include "quant_block.h"
#include "runtime_internal.h"

namespace {

// ---- exact scalar IEEE steps inside a flush-to-zero unit ----------------------------
// float -> double, subnormals included (bit-built, so no conversion flushes them)
__device__ __forceinline__ double widen(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7f800000u) == 0u) {
        const double m = (double)(u & 0x007fffffu) * 0x1p-149;
        return (u >> 31) ? -m : m;
    }
    return (double)x;
}

// double -> float, round to nearest even, subnormal results built by hand.
// The operations below round twice (to double, then to float); with 53 >=
// 2*24 + 2 bits that never changes a product, sum, quotient or square root of
// floats.
__device__ __forceinline__ float narrow(double r) {
    const double a = __builtin_fabs(r);
    if (!(a < 0x1p-126)) return (float)r;  // normal, inf, NaN
    const uint32_t m = (uint32_t)__builtin_rint(a * 0x1p149);  // <= 2^23 (2^23 = FLT_MIN)
    return __uint_as_float(m | (__builtin_signbit(r) ? 0x80000000u : 0u));
}

__device__ __forceinline__ float ieee_mul(float a, float b) { return narrow(widen(a) * widen(b)); }
__device__ __forceinline__ float ieee_add(float a, float b) { return narrow(widen(a) + widen(b)); }
__device__ __forceinline__ float ieee_div(float a, float b) { return narrow(widen(a) / widen(b)); }
__device__ __forceinline__ float ieee_sqrt(float a) { return narrow(__builtin_sqrt(widen(a))); }
__device__ __forceinline__ float libm_expf(float x) { return narrow(exp(widen(x))); }
__device__ __forceinline__ float libm_log1pf(float x) { return narrow(log1p(widen(x))); }

// ---- exp_neon, 04/qwen_kernels_opt.c:332-352 --------------------------------------
// Clamp to [-87, 88] (a NaN stays NaN), n = round(x*log2 e) by adding and
// subtracting 1.5*2^23, f = x*log2 e - n, degree-6 Horner polynomial in f,
// times 2^n built from the exponent bits (vcvtq_s32_f32 of NaN is 0).  The
// constants are the reference's: the polynomial is part of the result.
__device__ __forceinline__ float exp_neon(float x) {
    x = (x < -87.0f) ? -87.0f : x;
    x = (x > 88.0f) ? 88.0f : x;
    const float fx = x * 1.44269504088896341f;
    const float t = fx + 12582912.0f;
    const float n = t - 12582912.0f;
    const float f = fx - n;
    float p = 1.5403530393381608e-4f;
    p = 1.3333558146428443e-3f + p * f;
    p = 9.6181291076284770e-3f + p * f;
    p = 5.5504108664821580e-2f + p * f;
    p = 2.4022650695910070e-1f + p * f;
    p = 6.9314718055994530e-1f + p * f;
    p = 1.0f + p * f;
    const int e = (n == n) ? (int)n : 0;
    return p * __int_as_float((e + 127) << 23);
}

// ---- 4-lane residue sums -------------------------------------------------------------
constexpr int kChunk = 1024;              // elements staged per pass
constexpr int kPitch = kChunk / 4 + 4;    // floats per residue row (16-byte rows, 4-bank offset)

struct ResidueLds {
    float p[2][4][kPitch];
    float out[2];
};

__device__ __forceinline__ float chain_add(float s, const float* p, int cnt) {
    int m = 0;
#pragma unroll 4
    for (; m + 4 <= cnt; m += 4) {
        const float4 v = *reinterpret_cast<const float4*>(p + m);
        s = s + v.x;
        s = s + v.y;
        s = s + v.z;
        s = s + v.w;
    }
    for (; m < cnt; ++m) s = s + p[m];
    return s;
}

// Sums over the vector part [0, 4*(n/4)) of one or two product sequences,
// prod0(e) and prod1(e), in the 4-lane order; every thread of the block calls
// it (same n) and gets (sum0, sum1).  Staging hands element e to thread
// e % blockDim.x of each chunk.
template <class F0, class F1>
__device__ float2 residue_sums(int n, bool two, F0 prod0, F1 prod1, ResidueLds& L) {
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int nv = n & ~3;
    const int seq = tid >> 2, j = tid & 3;
    const bool chains = tid < (two ? 8 : 4);
    float s = 0.0f;
    for (int base = 0; base < nv; base += kChunk) {
        const int cnt = min(kChunk, nv - base);
        for (int e = tid; e < cnt; e += nthr) {
            L.p[0][e & 3][e >> 2] = prod0(base + e);
            if (two) L.p[1][e & 3][e >> 2] = prod1(base + e);
        }
        __syncthreads();
        if (chains) s = chain_add(s, &L.p[seq][j][0], cnt >> 2);
        __syncthreads();
    }
    if (tid < 64) {
        const int g = tid & ~3;
        const float l0 = __shfl(s, g + 0, 64), l1 = __shfl(s, g + 1, 64);
        const float l2 = __shfl(s, g + 2, 64), l3 = __shfl(s, g + 3, 64);
        const float r = (l0 + l2) + (l1 + l3);
        if (tid == 0) L.out[0] = r;
        if (tid == 4) L.out[1] = r;
    }
    __syncthreads();
    const float2 r = make_float2(L.out[0], L.out[1]);
    __syncthreads();
    return r;
}

// ---- per-element pieces --------------------------------------------------------------
// swiglu element: vector part s = g / (1 + exp_neon(-g)) (scalar division of
// div_neon), y = s * up; scalar tail with expf.
__device__ __forceinline__ float swiglu_elem(float g, float u, bool vec) {
    if (vec) return ieee_div(g, 1.0f + exp_neon(-g)) * u;
    return ieee_mul(ieee_div(g, ieee_add(1.0f, libm_expf(-g))), u);
}

// conv1d + SiLU of one channel; shifts the three taps.
__device__ __forceinline__ float conv_elem(float xc, float* s0, float* s1, float* s2, const float* w, bool vec) {
    const float t0 = *s0, t1 = *s1, t2 = *s2;
    float y;
    if (vec) {
        float d = w[0] * t0;
        d = d + w[1] * t1;
        d = d + w[2] * t2;
        d = d + w[3] * xc;
        y = ieee_div(d, 1.0f + exp_neon(-d));
    } else {
        float dot = ieee_add(ieee_mul(w[0], t0), ieee_mul(w[1], t1));
        dot = ieee_add(dot, ieee_mul(w[2], t2));
        dot = ieee_add(dot, ieee_mul(w[3], xc));
        y = ieee_div(dot, ieee_add(1.0f, libm_expf(-dot)));
    }
    *s0 = t1;
    *s1 = t2;
    *s2 = xc;
    return y;
}

// 1 / sqrtf(ss / n + eps), scalar
__device__ __forceinline__ float rms_scale(float ss, int n, float eps) {
    return ieee_div(1.0f, ieee_sqrt(ieee_add(ieee_div(ss, (float)n), eps)));
}

// gated RMSNorm element: ((x * r) * w) * (z / (1 + expf(-z))), scalar
__device__ __forceinline__ float gated_elem(float x, float r, float w, float z) {
    const float silu = ieee_div(z, ieee_add(1.0f, libm_expf(-z)));
    return ieee_mul(ieee_mul(ieee_mul(x, r), w), silu);
}

// gdn gates of one head from the two dot products: beta = 1/(1 + expf(-bv)),
// alpha = expf(nea * log1pf(expf(av + dt))).
__device__ __forceinline__ void gates_scalar(float av, float bv, float nea, float dt, float* alpha, float* beta) {
    *beta = ieee_div(1.0f, ieee_add(1.0f, libm_expf(-bv)));
    const float z = ieee_add(av, dt);
    *alpha = libm_expf(ieee_mul(nea, libm_log1pf(libm_expf(z))));
}

// One state column j of one head, both passes of the reference's blocked
// kernel: kv = sum_i k[i] S[i][j], qs = sum_i q[i] S[i][j] (ascending i),
// d = (v - kv*a) * b, out = qs*a + qk*d, then S[i][j] = S[i][j]*a + d*k[i].
// S = the head's blocked state; qh, kh = the head's q and k (LDS).  kNG > 0:
// ng == kNG and the column stays in registers between the passes.
template <int kNG>
__device__ __forceinline__ float gdn_column(float* S, int ng, int j, const float* qh, const float* kh, float vj,
                                            float a, float b, float qk) {
    float* col = S + ((size_t)(j >> 2) * ng * 4 + (j & 3)) * 4;
    float kv = 0.0f, qs = 0.0f;
    if constexpr (kNG > 0) {
        float4 s[kNG];
#pragma unroll
        for (int ig = 0; ig < kNG; ++ig) s[ig] = *reinterpret_cast<const float4*>(col + ig * 16);
#pragma unroll
        for (int ig = 0; ig < kNG; ++ig) {
            const float4 k4 = *reinterpret_cast<const float4*>(kh + 4 * ig);
            const float4 q4 = *reinterpret_cast<const float4*>(qh + 4 * ig);
            kv = kv + s[ig].x * k4.x;
            qs = qs + s[ig].x * q4.x;
            kv = kv + s[ig].y * k4.y;
            qs = qs + s[ig].y * q4.y;
            kv = kv + s[ig].z * k4.z;
            qs = qs + s[ig].z * q4.z;
            kv = kv + s[ig].w * k4.w;
            qs = qs + s[ig].w * q4.w;
        }
        const float d = (vj - kv * a) * b;
        const float out = qs * a + qk * d;
#pragma unroll
        for (int ig = 0; ig < kNG; ++ig) {
            const float4 k4 = *reinterpret_cast<const float4*>(kh + 4 * ig);
            float4 nv;
            nv.x = s[ig].x * a + d * k4.x;
            nv.y = s[ig].y * a + d * k4.y;
            nv.z = s[ig].z * a + d * k4.z;
            nv.w = s[ig].w * a + d * k4.w;
            *reinterpret_cast<float4*>(col + ig * 16) = nv;
        }
        return out;
    } else {
        for (int ig = 0; ig < ng; ++ig) {
            const float4 s4 = *reinterpret_cast<const float4*>(col + ig * 16);
            const float4 k4 = *reinterpret_cast<const float4*>(kh + 4 * ig);
            const float4 q4 = *reinterpret_cast<const float4*>(qh + 4 * ig);
            kv = kv + s4.x * k4.x;
            qs = qs + s4.x * q4.x;
            kv = kv + s4.y * k4.y;
            qs = qs + s4.y * q4.y;
            kv = kv + s4.z * k4.z;
            qs = qs + s4.z * q4.z;
            kv = kv + s4.w * k4.w;
            qs = qs + s4.w * q4.w;
        }
        const float d = (vj - kv * a) * b;
        const float out = qs * a + qk * d;
        for (int ig = 0; ig < ng; ++ig) {
            const float4 s4 = *reinterpret_cast<const float4*>(col + ig * 16);
            const float4 k4 = *reinterpret_cast<const float4*>(kh + 4 * ig);
            float4 nv;
            nv.x = s4.x * a + d * k4.x;
            nv.y = s4.y * a + d * k4.y;
            nv.z = s4.z * a + d * k4.z;
            nv.w = s4.w * a + d * k4.w;
            *reinterpret_cast<float4*>(col + ig * 16) = nv;
        }
        return out;
    }
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

}  // namespace

// ---- rmsnorm (+ residual, + quantize): one workgroup of 256 ----------------------------
extern "C" __global__ __launch_bounds__(256) void rt_rmsnorm_kernel(RtNormArgs a) {
    __shared__ ResidueLds L;
    __shared__ uint32_t rec[4][32];
    __shared__ float rs;
    const int tid = threadIdx.x, n = a.n, nv = n & ~3;
    if (a.res) {  // add_residual: vector part vaddq, tail scalar
        for (int e = tid; e < n; e += 256) {
            const float x = a.h[e], r = a.res[e];
            a.h[e] = (e < nv) ? x + r : ieee_add(x, r);
        }
        __syncthreads();
    }
    const float* h = a.h;
    const float ss_vec = residue_sums(n, false, [&](int e) { const float x = h[e]; return x * x; },
                                      [](int) { return 0.0f; }, L).x;
    if (tid == 0) {
        float ss = ss_vec;
        for (int e = nv; e < n; ++e) ss = ieee_add(ss, ieee_mul(h[e], h[e]));
        rs = rms_scale(ss, n, a.eps);
    }
    __syncthreads();
    const float r = rs;
    const int nb = n >> 6;
    for (int base = 0; base < n; base += 256) {
        const int e = base + tid;
        float y = 0.0f;
        if (e < n) {
            const float x = h[e], w = a.w[e];
            y = (e < nv) ? x * (r * (1.0f + w)) : ieee_mul(ieee_mul(x, r), ieee_add(1.0f, w));
            if (a.y) a.y[e] = y;
        }
        const int b = e >> 6;  // the same for the whole wavefront
        if (a.xsplit && b < nb) bfp8_quant_block_wave(y, lane_id(), nullptr, a.xscale + b, a.xsplit + (size_t)b * 32,
                                                      rec[wave_id()]);
    }
}

// ---- swiglu (+ quantize) ---------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void rt_swiglu_kernel(RtSwigluArgs a) {
    __shared__ uint32_t rec[4][32];
    const int e = blockIdx.x * 256 + threadIdx.x;
    float y = 0.0f;
    if (e < a.n) {
        y = swiglu_elem(a.gate[e], a.up[e], e < (a.n & ~3));
        a.y[e] = y;
    }
    const int b = e >> 6;
    if (a.xsplit && b < (a.n >> 6))
        bfp8_quant_block_wave(y, lane_id(), nullptr, a.xscale + b, a.xsplit + (size_t)b * 32, rec[wave_id()]);
}

// ---- causal conv1d + SiLU --------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void rt_conv1d_kernel(RtConvArgs a) {
    const int c = blockIdx.x * 256 + threadIdx.x, C = a.channels;
    if (c >= C) return;
    a.y[c] = conv_elem(a.x[c], a.state + c, a.state + C + c, a.state + 2 * C + c, a.w + (size_t)c * 4,
                       c < (C & ~3));
}

// ---- q/k L2 norm: one workgroup per head ----------------------------------------------
extern "C" __global__ __launch_bounds__(256) void rt_qk_l2norm_kernel(float* q, float* k, int D) {
    __shared__ ResidueLds L;
    __shared__ float sc[2];
    float* qh = q + (size_t)blockIdx.x * D;
    float* kh = k + (size_t)blockIdx.x * D;
    const int nv = D & ~3;
    const float2 sq = residue_sums(D, true, [&](int e) { const float x = kh[e]; return x * x; },
                                   [&](int e) { const float x = qh[e]; return x * x; }, L);
    if (threadIdx.x == 0) {
        float k_sq = sq.x, q_sq = sq.y;
        for (int e = nv; e < D; ++e) {
            k_sq = ieee_add(k_sq, ieee_mul(kh[e], kh[e]));
            q_sq = ieee_add(q_sq, ieee_mul(qh[e], qh[e]));
        }
        const float q_scale = ieee_div(1.0f, ieee_sqrt((float)D));
        sc[0] = ieee_div(1.0f, ieee_sqrt(ieee_add(k_sq, 1e-6f)));
        sc[1] = ieee_div(q_scale, ieee_sqrt(ieee_add(q_sq, 1e-6f)));
    }
    __syncthreads();
    const float kr = sc[0], qr = sc[1];
    for (int e = threadIdx.x; e < nv; e += 256) {  // the board leaves a D % 4 tail unscaled
        kh[e] = kh[e] * kr;
        qh[e] = qh[e] * qr;
    }
}

// ---- gdn gates: one workgroup per head ------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void rt_gates_kernel(RtGatesArgs a) {
    __shared__ ResidueLds L;
    const int h = blockIdx.x, K = a.K, nv = K & ~3;
    const float* ra = a.wa + (size_t)h * K;
    const float* rb = a.wb + (size_t)h * K;
    const float* x = a.x;
    const float2 ab = residue_sums(K, true, [&](int e) { return ra[e] * x[e]; },
                                   [&](int e) { return rb[e] * x[e]; }, L);
    if (threadIdx.x == 0) {
        float av = ab.x, bv = ab.y;
        for (int e = nv; e < K; ++e) {
            av = ieee_add(av, ieee_mul(ra[e], x[e]));
            bv = ieee_add(bv, ieee_mul(rb[e], x[e]));
        }
        gates_scalar(av, bv, a.nea[h], a.dt[h], a.alpha + h, a.beta + h);
    }
}

// ---- gdn recurrent step: workgroups of 64 columns of one head --------------------------
template <int kNG>
__global__ __launch_bounds__(64) void rt_gdn_step_kernel(RtGdnArgs a) {
    __shared__ ResidueLds L;
    __shared__ __attribute__((aligned(16))) float qs[RT_MAX_HEAD_DIM];
    __shared__ __attribute__((aligned(16))) float ks[RT_MAX_HEAD_DIM];
    const int h = blockIdx.y, D = a.D, ng = D >> 2;
    const float* qh = a.q + (size_t)h * D;
    const float* kh = a.k + (size_t)h * D;
    for (int e = threadIdx.x; e < D; e += 64) {
        qs[e] = qh[e];
        ks[e] = kh[e];
    }
    __syncthreads();
    const float qk = residue_sums(D, false, [&](int e) { return qs[e] * ks[e]; }, [](int) { return 0.0f; }, L).x;
    const int j = blockIdx.x * 64 + threadIdx.x;
    if (j >= D) return;
    float* S = a.state + (size_t)h * D * D;
    a.out[(size_t)h * D + j] =
        gdn_column<kNG>(S, ng, j, qs, ks, a.v[(size_t)h * D + j], a.alpha[h], a.beta[h], qk);
}

// ---- gated RMSNorm (+ quantize): one workgroup per head ------------------------------------
extern "C" __global__ __launch_bounds__(256) void rt_gated_kernel(RtGatedArgs a) {
    __shared__ ResidueLds L;
    __shared__ uint32_t rec[4][32];
    __shared__ float rs;
    const int h = blockIdx.x, D = a.D, nv = D & ~3;
    const float* xh = a.x + (size_t)h * D;
    const float* zh = a.z + (size_t)h * D;
    float* yh = a.y + (size_t)h * D;
    const float ss_vec = residue_sums(D, false, [&](int e) { const float x = xh[e]; return x * x; },
                                      [](int) { return 0.0f; }, L).x;
    if (threadIdx.x == 0) {
        float ss = ss_vec;
        for (int e = nv; e < D; ++e) ss = ieee_add(ss, ieee_mul(xh[e], xh[e]));
        rs = rms_scale(ss, D, a.eps);
    }
    __syncthreads();
    const float r = rs;
    const bool quant = a.xsplit && (D & 63) == 0;
    for (int base = 0; base < D; base += 256) {
        const int e = base + threadIdx.x;
        float y = 0.0f;
        if (e < D) {
            y = gated_elem(xh[e], r, a.w[e], zh[e]);
            yh[e] = y;
        }
        const int bb = e >> 6;
        if (quant && bb < (D >> 6)) {
            const size_t b = (size_t)h * (D >> 6) + bb;
            bfp8_quant_block_wave(y, lane_id(), nullptr, a.xscale + b, a.xsplit + b * 32, rec[wave_id()]);
        }
    }
}

// ---- add_residual -----------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void rt_add_residual_kernel(float* x, const float* res, int n) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= n) return;
    x[e] = (e < (n & ~3)) ? x[e] + res[e] : ieee_add(x[e], res[e]);
}

// ---- embedding row (bf16 -> f32) --------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void rt_embed_kernel(float* h, const uint16_t* table, int row,
                                                                  int hidden) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e < hidden) h[e] = __uint_as_float((uint32_t)table[(size_t)row * hidden + e] << 16);
}

// ---- the model's linear-attention block, one workgroup per head ---------------------------
extern "C" __global__ __launch_bounds__(256) void rt_linear_attn_kernel(RtLinearAttnArgs a) {
    constexpr int D = RT_HEAD_DIM, C = RT_CONV_CH, HD = RT_HEADS * RT_HEAD_DIM;
    __shared__ ResidueLds L;
    __shared__ uint32_t rec[4][32];
    __shared__ __attribute__((aligned(16))) float qv[D];
    __shared__ __attribute__((aligned(16))) float kv[D];
    __shared__ float vv[D];
    __shared__ float ov[D];
    __shared__ float sc[4];
    const int h = blockIdx.x, tid = threadIdx.x;

    // conv1d + SiLU over this head's q, k and v channels (all in the vector part)
    for (int i = tid; i < 3 * D; i += 256) {
        const int part = i / D, jj = i - part * D;
        const int c = part * HD + h * D + jj;
        const float y = conv_elem(a.qkv[c], a.conv_s + c, a.conv_s + C + c, a.conv_s + 2 * C + c,
                                  a.conv_w + (size_t)c * 4, c < (C & ~3));
        (part == 0 ? qv : part == 1 ? kv : vv)[jj] = y;
        if (part == 2 && a.mixed) a.mixed[c] = y;
    }
    __syncthreads();

    // gates from the input-norm output
    const float* ra = a.wa + (size_t)h * RT_HIDDEN;
    const float* rb = a.wb + (size_t)h * RT_HIDDEN;
    const float* x = a.normed;
    const float2 ab = residue_sums(RT_HIDDEN, true, [&](int e) { return ra[e] * x[e]; },
                                   [&](int e) { return rb[e] * x[e]; }, L);
    // q/k L2 norm sums
    const float2 sq = residue_sums(D, true, [&](int e) { return kv[e] * kv[e]; },
                                   [&](int e) { return qv[e] * qv[e]; }, L);
    if (tid == 0) {
        gates_scalar(ab.x, ab.y, a.nea[h], a.dt[h], &sc[0], &sc[1]);
        const float q_scale = ieee_div(1.0f, ieee_sqrt((float)D));
        sc[2] = ieee_div(1.0f, ieee_sqrt(ieee_add(sq.x, 1e-6f)));
        sc[3] = ieee_div(q_scale, ieee_sqrt(ieee_add(sq.y, 1e-6f)));
        if (a.alpha_beta) {
            a.alpha_beta[h] = sc[0];
            a.alpha_beta[RT_HEADS + h] = sc[1];
        }
    }
    __syncthreads();
    const float alpha = sc[0], beta = sc[1];
    if (tid < D) {
        kv[tid] = kv[tid] * sc[2];
        qv[tid] = qv[tid] * sc[3];
        if (a.mixed) {
            a.mixed[h * D + tid] = qv[tid];
            a.mixed[HD + h * D + tid] = kv[tid];
        }
    }
    __syncthreads();

    // recurrent step
    const float qk = residue_sums(D, false, [&](int e) { return qv[e] * kv[e]; }, [](int) { return 0.0f; }, L).x;
    if (tid < D) {
        const float o = gdn_column<D / 4>(a.state + (size_t)h * D * D, D / 4, tid, qv, kv, vv[tid], alpha, beta, qk);
        ov[tid] = o;
        if (a.attn) a.attn[h * D + tid] = o;
    }
    __syncthreads();

    // gated RMSNorm + quantizer of the o GEMV's input (two blocks per head)
    const float ss = residue_sums(D, false, [&](int e) { return ov[e] * ov[e]; }, [](int) { return 0.0f; }, L).x;
    if (tid == 0) sc[0] = rms_scale(ss, D, 1e-6f);
    __syncthreads();
    if (tid < D) {
        const float y = gated_elem(ov[tid], sc[0], a.norm_w[tid], a.zbuf[h * D + tid]);
        if (a.gated) a.gated[h * D + tid] = y;
        const int b = h * (D / 64) + wave_id();
        bfp8_quant_block_wave(y, lane_id(), nullptr, a.xscale + b, a.xsplit + (size_t)b * 32, rec[wave_id()]);
    }
}

// ---- launchers ------------------------------------------------------------------------------
static unsigned blocks_for(int n) { return (unsigned)((n + 255) / 256); }

hipError_t rt_launch_rmsnorm(const RtNormArgs& a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    hipLaunchKernelGGL(rt_rmsnorm_kernel, dim3(1), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t rt_launch_swiglu(const RtSwigluArgs& a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    hipLaunchKernelGGL(rt_swiglu_kernel, dim3(blocks_for(a.n)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t rt_launch_conv1d(const RtConvArgs& a, hipStream_t s) {
    if (a.channels <= 0) return hipSuccess;
    hipLaunchKernelGGL(rt_conv1d_kernel, dim3(blocks_for(a.channels)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t rt_launch_qk_l2norm(float* q, float* k, int H, int D, hipStream_t s) {
    if (H <= 0 || D <= 0) return hipSuccess;
    hipLaunchKernelGGL(rt_qk_l2norm_kernel, dim3(H), dim3(256), 0, s, q, k, D);
    return hipGetLastError();
}

hipError_t rt_launch_gates(const RtGatesArgs& a, hipStream_t s) {
    if (a.H <= 0) return hipSuccess;
    hipLaunchKernelGGL(rt_gates_kernel, dim3(a.H), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t rt_launch_gdn_step(const RtGdnArgs& a, hipStream_t s) {
    if (a.H <= 0 || a.D <= 0) return hipSuccess;
    if ((a.D & 3) || a.D > RT_MAX_HEAD_DIM) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.D + 63) / 64), (unsigned)a.H);
    if (a.D == 128)
        hipLaunchKernelGGL(rt_gdn_step_kernel<32>, grid, dim3(64), 0, s, a);
    else if (a.D == 64)
        hipLaunchKernelGGL(rt_gdn_step_kernel<16>, grid, dim3(64), 0, s, a);
    else
        hipLaunchKernelGGL(rt_gdn_step_kernel<0>, grid, dim3(64), 0, s, a);
    return hipGetLastError();
}

hipError_t rt_launch_gated(const RtGatedArgs& a, hipStream_t s) {
    if (a.H <= 0 || a.D <= 0) return hipSuccess;
    hipLaunchKernelGGL(rt_gated_kernel, dim3(a.H), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t rt_launch_add_residual(float* x, const float* res, int n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(rt_add_residual_kernel, dim3(blocks_for(n)), dim3(256), 0, s, x, res, n);
    return hipGetLastError();
}

hipError_t rt_launch_linear_attn(const RtLinearAttnArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(rt_linear_attn_kernel, dim3(RT_HEADS), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t rt_launch_embed(float* h, const uint16_t* table, int row, int hidden, hipStream_t s) {
    if (hidden <= 0) return hipSuccess;
    hipLaunchKernelGGL(rt_embed_kernel, dim3(blocks_for(hidden)), dim3(256), 0, s, h, table, row, hidden);
    return hipGetLastError();
}
