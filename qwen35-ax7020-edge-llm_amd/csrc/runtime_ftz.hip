// runtime_ftz.hip -- the decode runtime around the GEMV
// (04/qwen_kernels_opt.c:140-175, :328-398, :511-860): rmsnorm, swiglu,
// causal conv1d + SiLU, q/k L2 norm, GDN gates, GDN recurrent step, gated
// RMSNorm, residual add, and the fused per-layer kernels of the
// device-resident forward.
//
// Compiled with f32 flush-to-zero and -ffp-contract=off: a plain float
// operation here is one Advanced SIMD operation of the reference (vmulq,
// vaddq, vsubq; vmlaq = product rounded, then sum rounded).  The reference's
// scalar VFP steps keep IEEE subnormals; they go through ieee_*() of
// runtime_dev.h, which compute in double and round once to float by hand, so
// they do not depend on the f32 denormal mode.  expf / log1pf of the reference's libm are
// taken as exp / log1p in double rounded to float.
//
// Reductions follow the reference's 4-lane accumulators: lane j adds the
// products of elements 4m + j in ascending m (one rounding per add), and the
// lanes combine as (l0 + l2) + (l1 + l3) (vadd of the halves, then vpadd).
#include <hip/hip_runtime.h>

#include "quant_block.h"
#include "runtime_dev.h"
#include "runtime_internal.h"

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
// ntiles == 0: row-major, element e of the row at row * hidden + e.  Else
// the lm_head's tile layout over ntiles 64-row tiles (nT = 4 * ntiles groups
// of 16 rows): element e = 8c + j of row 16T + r, c = 4q + cc, q = 2p + s,
// j = 4 hi + g, in 16-byte slot ((p * nT + T) * 2 + s) * 64 + 4r + g, word
// cc, half hi.
extern "C" __global__ __launch_bounds__(256) void rt_embed_kernel(float* h, const uint16_t* table, int ntiles, int row,
                                                                  int hidden) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= hidden) return;
    size_t at = (size_t)row * hidden + e;
    if (ntiles) {
        const int c = e >> 3, j = e & 7;
        const int q = c >> 2;
        const size_t slot =
            (((size_t)(q >> 1) * (size_t)(4 * ntiles) + (size_t)(row >> 4)) * 2 + (q & 1)) * 64 + 4 * (row & 15) + (j & 3);
        at = slot * 8 + 2 * (c & 3) + (j >> 2);
    }
    h[e] = __uint_as_float((uint32_t)table[at] << 16);
}

// ---- the model's linear-attention block ----------------------------------------------------
// RT_ATTN_SPLIT workgroups per head; workgroup (h, part) owns state columns
// [part*32, part*32 + 32).  Independent work overlaps: wavefront 3 owns the
// columns (two lanes per column: one sums k.S, the other q.S) and issues its
// state loads first; wavefront 0 forms the gates (two 256-step sums over the
// input-norm output, then the scalar part); wavefronts 1-2 run the conv over
// the head's q, k, v channels with every load issued before any use.  Every
// workgroup of a head computes the same conv, norms and gates.
template <int N>
__device__ __forceinline__ float chain_add_n(float s, const float* p) {
    // N % 4 == 0 and p 16-byte aligned; fully unrolled so the LDS reads run ahead of the adds
#pragma unroll
    for (int m = 0; m < N; m += 4) {
        const float4 v = *reinterpret_cast<const float4*>(p + m);
        s = s + v.x;
        s = s + v.y;
        s = s + v.z;
        s = s + v.w;
    }
    return s;
}

extern "C" __global__ __launch_bounds__(256) void rt_linear_attn_kernel(RtLinearAttnArgs a) {
    constexpr int D = RT_HEAD_DIM, NG = D / 4, C = RT_CONV_CH, HD = RT_HEADS * RT_HEAD_DIM, KG = RT_HIDDEN;
    constexpr int COLS = D / RT_ATTN_SPLIT;
    static_assert(D == 128 && COLS == 32 && KG / 4 <= kPitch, "sized for 16 heads of 128 and a 1024 gate input");
    __shared__ ResidueLds L;
    __shared__ __attribute__((aligned(16))) float kq[2][D];  // k, q: one array, so a lane's vector is one address
    float* const kv = kq[0];
    float* const qv = kq[1];
    __shared__ float vv[D];
    __shared__ float sc[5];
    const int h = blockIdx.x / RT_ATTN_SPLIT, part = blockIdx.x % RT_ATTN_SPLIT;
    const int tid = threadIdx.x, w = wave_id(), lane = lane_id();

    // wavefront 3: lane = (role, column): role 0 sums k[i] S[i][j], role 1 q[i] S[i][j]
    const int cj = part * COLS + (lane & 31), role = lane >> 5;
    float* col = a.state + (size_t)h * D * D + ((size_t)(cj >> 2) * NG * 4 + (cj & 3)) * 4;
    float4 st[NG];
    if (w == 3) {
        // silu(z) of this workgroup's columns, for the gated norm in the o GEMV
        // (z loaded ahead of the state, so its wait does not wait for the state)
        const int ez = h * D + cj;
        const float zv = a.z[ez];
#pragma unroll
        for (int ig = 0; ig < NG; ++ig) st[ig] = *reinterpret_cast<const float4*>(col + ig * 16);
        if (lane < COLS) a.zsilu[ez] = silu_scalar(zv);
    } else if (w == 0) {
        // gates' products wa[h] * x, wb[h] * x (all loads first)
        const float* ra = a.wa + (size_t)h * KG;
        const float* rb = a.wb + (size_t)h * KG;
        float xs[KG / 64], pa[KG / 64], pb[KG / 64];
#pragma unroll
        for (int k = 0; k < KG / 64; ++k) {
            const int e = lane + 64 * k;
            xs[k] = a.normed[e];
            pa[k] = ra[e];
            pb[k] = rb[e];
        }
#pragma unroll
        for (int k = 0; k < KG / 64; ++k) {
            const int e = lane + 64 * k;
            L.p[0][e & 3][e >> 2] = pa[k] * xs[k];
            L.p[1][e & 3][e >> 2] = pb[k] * xs[k];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float s = 0.0f;
        if (lane < 8) s = chain_add256(0.0f, &L.p[lane >> 2][lane & 3][0]);
        const float r = lanes4_combine(s);
        const float bv = readlane_f(r, 4);
        if (lane == 0) gates_scalar(r, bv, a.nea[h], a.dt[h], &sc[0], &sc[1]);
    } else {
        // conv1d + SiLU over the head's q, k and v channels (all in the vector
        // part): 128 lanes x 3 channels, loads first
        const int t = tid - 64;
        float xc[3], t0[3], t1[3], t2[3];
        float4 wt[3];
        int cc[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int i = t + 128 * k;  // channel i of the head's 384: part i / 128 of q, k, v
            const int c = (i >> 7) * HD + h * D + (i & 127);
            cc[k] = c;
            xc[k] = a.qkv[c];
            t0[k] = a.conv_in[c];
            t1[k] = a.conv_in[C + c];
            t2[k] = a.conv_in[2 * C + c];
            wt[k] = *reinterpret_cast<const float4*>(a.conv_w + (size_t)c * 4);
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            float d = wt[k].x * t0[k];
            d = d + wt[k].y * t1[k];
            d = d + wt[k].z * t2[k];
            d = d + wt[k].w * xc[k];
            const float y = ieee_div(d, 1.0f + exp_neon(-d));
            const int i = t + 128 * k, jj = i & 127;
            (k == 0 ? qv : k == 1 ? kv : vv)[jj] = y;
            if (part == 0) {  // one writer for the shifted taps
                const int c = cc[k];
                a.conv_out[c] = t1[k];
                a.conv_out[C + c] = t2[k];
                a.conv_out[2 * C + c] = xc[k];
                if (k == 2 && a.mixed) a.mixed[c] = y;
            }
        }
    }
    __syncthreads();

    // q/k L2 norm
    if (tid < D) {
        const int e = tid;
        L.p[0][e & 3][e >> 2] = kv[e] * kv[e];
        L.p[1][e & 3][e >> 2] = qv[e] * qv[e];
    }
    __syncthreads();
    if (w == 1) {  // wavefront 0 may still be in the gates' scalar part
        float s = 0.0f;
        if (lane < 8) s = chain_add_n<NG>(0.0f, &L.p[lane >> 2][lane & 3][0]);
        const float r = lanes4_combine(s);
        const float q_sq = readlane_f(r, 4);
        if (lane == 0) {
            // 1 / sqrtf(D): both steps of normal constants, so the instructions are exact
            const float q_scale = __fdiv_rn(1.0f, (float)__builtin_sqrt((double)D));
            sc[2] = div_sqrt_add(1.0f, r, 1e-6f);
            sc[3] = div_sqrt_add(q_scale, q_sq, 1e-6f);
        }
    }
    __syncthreads();
    if (tid < D) {
        const float k = kv[tid] * sc[2], q = qv[tid] * sc[3];
        kv[tid] = k;
        qv[tid] = q;
        L.p[0][tid & 3][tid >> 2] = q * k;  // the q.k sum's products
        if (a.mixed && part == 0) {
            a.mixed[h * D + tid] = q;
            a.mixed[HD + h * D + tid] = k;
        }
    }
    __syncthreads();
    if (w == 1) {
        float s = 0.0f;
        if (lane < 4) s = chain_add_n<NG>(0.0f, &L.p[0][lane][0]);
        const float r = lanes4_combine(s);
        if (lane == 0) sc[4] = r;
    }
    __syncthreads();
    if (w == 0 && lane == 0 && a.alpha_beta && part == 0) {
        a.alpha_beta[h] = sc[0];
        a.alpha_beta[RT_HEADS + h] = sc[1];
    }

    // recurrent step on the columns held in registers
    if (w == 3) {
        const float alpha = sc[0], beta = sc[1], qk = sc[4];
        // kv (role 0) or qs (role 1), ascending i; the vector's 16-byte groups
        // are read a few steps ahead (an empty asm statement pins each step,
        // so the reads do not all land in registers at once)
        const float4* vec = reinterpret_cast<const float4*>(&kq[role][0]);
        constexpr int kAhead = 4;
        float4 vr[NG];
#pragma unroll
        for (int ig = 0; ig < kAhead; ++ig) vr[ig] = vec[ig];
        float acc = 0.0f;
#pragma unroll
        for (int ig = 0; ig < NG; ++ig) {
            if (ig + kAhead < NG) vr[ig + kAhead] = vec[ig + kAhead];
            acc = acc + st[ig].x * vr[ig].x;
            acc = acc + st[ig].y * vr[ig].y;
            acc = acc + st[ig].z * vr[ig].z;
            acc = acc + st[ig].w * vr[ig].w;
            asm volatile("" : "+v"(acc)::"memory");
        }
        const int c = lane & 31;
        const float kvs = __shfl(acc, c, 64), qss = __shfl(acc, 32 + c, 64);
        const float d = (vv[cj] - kvs * alpha) * beta;
        const float o = qss * alpha + qk * d;
        // S[i][j] = S[i][j] * a + d * k[i]: role 0 the first 16 row groups, role 1
        // the rest, in the same instructions (the lane's half chosen by select)
        const float4* k4v = reinterpret_cast<const float4*>(kv) + role * (NG / 2);
        float* colr = col + role * (NG / 2) * 16;
#pragma unroll
        for (int g = 0; g < NG / 2; ++g) {
            const float4 s4 = role ? st[g + NG / 2] : st[g];
            const float4 k4 = k4v[g];
            float4 nv;
            nv.x = s4.x * alpha + d * k4.x;
            nv.y = s4.y * alpha + d * k4.y;
            nv.z = s4.z * alpha + d * k4.z;
            nv.w = s4.w * alpha + d * k4.w;
            *reinterpret_cast<float4*>(colr + g * 16) = nv;
        }
        if (role == 0) a.attn[h * D + cj] = o;
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
    if (a.conv_in == a.conv_out) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rt_linear_attn_kernel, dim3(RT_HEADS * RT_ATTN_SPLIT), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t rt_launch_embed(float* h, const uint16_t* table, int ntiles, int row, int hidden, hipStream_t s) {
    if (hidden <= 0) return hipSuccess;
    if (ntiles && ((hidden & 31) || row >= ntiles * 64)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rt_embed_kernel, dim3(blocks_for(hidden)), dim3(256), 0, s, h, table, ntiles, row, hidden);
    return hipGetLastError();
}
