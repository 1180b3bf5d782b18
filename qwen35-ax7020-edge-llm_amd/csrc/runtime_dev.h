// runtime_dev.h -- device helpers of the decode runtime shared by the
// flush-to-zero translation units (runtime_ftz.hip, fused_gemv.hip): the
// reference's Advanced SIMD steps in f32 flush-to-zero arithmetic, its scalar
// VFP steps through exact double-based helpers, and the 4-lane reductions.
// Include only from a unit compiled with -fgpu-flush-denormals-to-zero
// -ffp-contract=off.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ieee_dev.h"

namespace {

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

// s + p[0] + p[1] + ... + p[cnt-1], one rounding per add, in this order.
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

// s + p[0] + ... + p[255] (LDS, 16-byte aligned), one rounding per add, in
// this order.  A wavefront issues LDS reads and adds in order and a 16-byte
// read holds its issue for about as long as four adds, so the reads are
// spread evenly: one after every four adds, kAhead reads ahead of their use
// (an empty asm statement that takes s and clobbers memory pins each step).
__device__ __forceinline__ float chain_add256(float s, const float* p) {
    constexpr int kAhead = 8;
    const float4* p4 = reinterpret_cast<const float4*>(p);
    float4 buf[64];
#pragma unroll
    for (int i = 0; i < kAhead; ++i) buf[i] = p4[i];
#pragma unroll
    for (int i = 0; i < 64; ++i) {
        if (i + kAhead < 64) buf[i + kAhead] = p4[i + kAhead];
        s = s + buf[i].x;
        s = s + buf[i].y;
        s = s + buf[i].z;
        s = s + buf[i].w;
        asm volatile("" : "+v"(s)::"memory");
    }
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
        if (chains) s = (cnt == kChunk) ? chain_add256(s, &L.p[seq][j][0]) : chain_add(s, &L.p[seq][j][0], cnt >> 2);
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
// Each step is one IEEE operation.  The float instructions answer when every
// operand and intermediate is normal (one combined test, no branch per step;
// the square root of a normal positive float is normal), else the exact
// helpers do; a power-of-two n divides exactly as a product with 1/n.
__device__ __forceinline__ float rms_scale(float ss, int n, float eps) {
    const float fn = (float)n;
    const float m = ((n & (n - 1)) == 0) ? ss * (1.0f / fn) : __fdiv_rn(ss, fn);
    const float t = m + eps;
    const float q = (float)__builtin_sqrt((double)t);
    const float r = __fdiv_rn(1.0f, q);
    if (normal_u(ss) & normal_u(fn) & normal_u(m) & normal_u(eps) & normal_u(t) & normal_u(r)) return r;
    return ieee_div(1.0f, ieee_sqrt(ieee_add(ieee_div(ss, fn), eps)));
}

// num / sqrtf(x + eps), scalar, with one combined normality test as in rms_scale
__device__ __forceinline__ float div_sqrt_add(float num, float x, float eps) {
    const float t = x + eps;
    const float q = (float)__builtin_sqrt((double)t);
    const float r = __fdiv_rn(num, q);
    if (normal_u(num) & normal_u(x) & normal_u(eps) & normal_u(t) & normal_u(r)) return r;
    return ieee_div(num, ieee_sqrt(ieee_add(x, eps)));
}

// silu(z) = z / (1 + expf(-z)), scalar.  For a normal argument whose result
// is normal, expf is the double exp rounded once (libm_expf without its
// subnormal handling); one combined test as in rms_scale.
__device__ __forceinline__ float silu_scalar(float z) {
    const float e = (float)exp(-(double)z);
    const float d = 1.0f + e;
    const float r = __fdiv_rn(z, d);
    if (normal_u(z) & normal_u(e) & normal_u(d) & normal_u(r)) return r;
    return ieee_div(z, ieee_add(1.0f, libm_expf(-z)));
}

// gated RMSNorm element: ((x * r) * w) * silu(z), scalar
__device__ __forceinline__ float gated_mul(float x, float r, float w, float silu) {
    const float a = x * r, b = a * w, c = b * silu;  // one combined normality test, as in rms_scale
    if (normal_u(x) & normal_u(r) & normal_u(a) & normal_u(w) & normal_u(b) & normal_u(silu) & normal_u(c)) return c;
    return ieee_mul(ieee_mul(ieee_mul(x, r), w), silu);
}
__device__ __forceinline__ float gated_elem(float x, float r, float w, float z) {
    return gated_mul(x, r, w, silu_scalar(z));
}

// gdn gates of one head from the two dot products: beta = 1/(1 + expf(-bv)),
// alpha = expf(nea * log1pf(expf(av + dt))).
// Every step is one IEEE operation or one libm call (the double function
// rounded once); one combined normality test as in silu_scalar.
__device__ __forceinline__ void gates_scalar(float av, float bv, float nea, float dt, float* alpha, float* beta) {
    const float e1 = (float)exp(-(double)bv);
    const float d1 = 1.0f + e1;
    const float b = __fdiv_rn(1.0f, d1);
    const float z = av + dt;
    const float e2 = (float)exp((double)z);
    const float l = (float)log1p((double)e2);
    const float m = nea * l;
    const float al = (float)exp((double)m);
    if (normal_u(bv) & normal_u(e1) & normal_u(d1) & normal_u(b) & normal_u(av) & normal_u(dt) & normal_u(z) &
        normal_u(e2) & normal_u(l) & normal_u(nea) & normal_u(m) & normal_u(al)) {
        *beta = b;
        *alpha = al;
        return;
    }
    *beta = ieee_div(1.0f, ieee_add(1.0f, libm_expf(-bv)));
    const float ze = ieee_add(av, dt);
    *alpha = libm_expf(ieee_mul(nea, libm_log1pf(libm_expf(ze))));
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

// (l0 + l2) + (l1 + l3) over the four lanes 4g..4g+3 that hold the calling
// lane's group (vadd of the halves, then vpadd); every lane of the
// wavefront calls it.
__device__ __forceinline__ float lanes4_combine(float s) {
    // quad_perm [j,j,j,j] hands lane j of the quad to all four (every lane active)
    const int x = __float_as_int(s);
    const float l0 = __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x00, 0xF, 0xF, false));
    const float l1 = __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x55, 0xF, 0xF, false));
    const float l2 = __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xAA, 0xF, 0xF, false));
    const float l3 = __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xFF, 0xF, 0xF, false));
    return (l0 + l2) + (l1 + l3);
}

// A long 4-lane chain with its operands in registers: row j of a wavefront
// (lanes 16j .. 16j+15) holds residue j's products, product m = 16r + i in
// v[r] of lane 16j + i, and lane 16j adds products 0 .. 16*nr - 1 to s in
// ascending m, one rounding per add.  Lane 16j reads lane 16j + i through a
// DPP row shift (row_shl:i), so no add waits on memory.  nr (<= 16) is
// uniform; the other lanes' results are meaningless.
#define RT_ROW_ADD(k) s = s + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x100 + (k), 0xF, 0xF, true))
__device__ __forceinline__ float row_chain(float s, const float (&v)[16], int nr) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        if (r < nr) {
            const float x = v[r];
            s = s + x;
            RT_ROW_ADD(1);
            RT_ROW_ADD(2);
            RT_ROW_ADD(3);
            RT_ROW_ADD(4);
            RT_ROW_ADD(5);
            RT_ROW_ADD(6);
            RT_ROW_ADD(7);
            RT_ROW_ADD(8);
            RT_ROW_ADD(9);
            RT_ROW_ADD(10);
            RT_ROW_ADD(11);
            RT_ROW_ADD(12);
            RT_ROW_ADD(13);
            RT_ROW_ADD(14);
            RT_ROW_ADD(15);
        }
    }
    return s;
}
#undef RT_ROW_ADD
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

}  // namespace
