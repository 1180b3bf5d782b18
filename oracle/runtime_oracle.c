/*
 * runtime_oracle.c -- CPU restatement of the reference's decode runtime
 * kernels (04/qwen_kernels_opt.c:140-175, :328-398, :511-866) and of its
 * compiled forward loop (:866-1049), board build (Advanced SIMD).
 *
 * TEST INFRASTRUCTURE ONLY, like bfp8_oracle.c: only tests/ loads the
 * library built from it; the HIP library never links or calls it.
 *
 * Vector arithmetic uses orc_neon_mul / orc_neon_add (flush-to-zero, one
 * rounding each); vmlaq_f32(a, b, c) is a + b*c with the product rounded
 * first.  Scalar code (VFP: IEEE subnormals) is plain C compiled with
 * -ffp-contract=off; sqrtf is the host C library's, expf / log1pf see
 * o_expf below.
 *
 * Pinning (tests/test_oracle.py):
 *   orc_exp_neon        relative error bound against exp over [-87, 88],
 *                       exact points (0 -> 1, the clamps), NaN / inf
 *   reductions (rmsnorm, qk_l2norm, gdn_gates, rmsnorm_gated, gdn step)
 *                       integer inputs whose sums are exact (any order
 *                       agrees, so the reference's own host build pins them),
 *                       lane-order inputs that fail every other order
 *   orc_gdn_step        bit-exact vs the reference's own host build of
 *                       gdn_recurrent_step (same operation order, blocked
 *                       state layout converted) on normal data
 *   orc_swiglu / orc_conv1d_silu  per-element formula with exp_neon, vs a
 *                       float64 bound; tails vs the reference host build
 *   o_expf / o_log1pf   host libm by default; correctly rounded in
 *                       orc_set_cr_libm(1) mode (checked against float64)
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float orc_neon_mul(float a, float b);
float orc_neon_add(float a, float b);
void orc_gemv_neon(float* y, const float* x, const int8_t* mant, const uint8_t* exps, int M, int K, int16_t* xq_out,
                   float* xscale_out, int32_t* lanes_out);
float orc_bf16_dot(const float* h, const uint16_t* row, int hidden, int tail);
int orc_argmax(const float* logits, int n);

static float nsub(float a, float b) { return orc_neon_add(a, -b); }

/* The reference's scalar code calls libm expf / log1pf.  By default the
 * oracle uses the host C library's; orc_set_cr_libm(1) switches to exp /
 * log1p in double rounded once to float (correctly rounded except within
 * 2^-29 of a rounding boundary), the definition the GPU implements, so that
 * whole-layer comparisons can be bit for bit. */
static int g_cr_libm = 0;
void orc_set_cr_libm(int on) { g_cr_libm = on; }
static float o_expf(float x) { return g_cr_libm ? (float)exp((double)x) : expf(x); }
static float o_log1pf(float x) { return g_cr_libm ? (float)log1p((double)x) : log1pf(x); }

/* Advanced SIMD vmaxq/vminq: a NaN operand gives the default NaN. */
static float nmax(float a, float b) { return (isnan(a) || isnan(b)) ? NAN : (a > b ? a : b); }
static float nmin(float a, float b) { return (isnan(a) || isnan(b)) ? NAN : (a < b ? a : b); }

/* 4-lane reduction result: vpadd(vadd(low, high)) lane 0. */
static float lanes4(const float* s) {
    return orc_neon_add(orc_neon_add(s[0], s[2]), orc_neon_add(s[1], s[3]));
}

/* ---- exp_neon, 04/qwen_kernels_opt.c:332-352 --------------------------------
 * Clamp to [-87, 88], n = round(x*log2(e)) by the 1.5*2^23 trick,
 * f = x*log2(e) - n, degree-6 Horner polynomial in f (vmlaq), times 2^n built
 * from the exponent bits (vcvtq_s32_f32 truncates; NaN converts to 0). */
float orc_exp_neon(float x) {
    x = nmax(x, -87.0f);
    x = nmin(x, 88.0f);
    const float fx = orc_neon_mul(x, 1.44269504088896341f);
    const float t = orc_neon_add(fx, 12582912.0f);
    const float n = nsub(t, 12582912.0f);
    const float f = nsub(fx, n);
    float p = 1.5403530393381608e-4f;
    p = orc_neon_add(1.3333558146428443e-3f, orc_neon_mul(p, f));
    p = orc_neon_add(9.6181291076284770e-3f, orc_neon_mul(p, f));
    p = orc_neon_add(5.5504108664821580e-2f, orc_neon_mul(p, f));
    p = orc_neon_add(2.4022650695910070e-1f, orc_neon_mul(p, f));
    p = orc_neon_add(6.9314718055994530e-1f, orc_neon_mul(p, f));
    p = orc_neon_add(1.0f, orc_neon_mul(p, f));
    int32_t e = isnan(n) ? 0 : (int32_t)n;
    e += 127;
    uint32_t bits = (uint32_t)e << 23;
    float sc;
    memcpy(&sc, &bits, 4);
    return orc_neon_mul(p, sc);
}

/* ---- swiglu, 04/qwen_kernels_opt.c:363-384 ----------------------------------
 * Vector part: s = g / (1 + exp_neon(-g)) with a scalar IEEE division
 * (div_neon), y = s * up; the n % 4 tail in scalar arithmetic with expf. */
void orc_swiglu(float* y, const float* gate, const float* up, int n) {
    int i = 0;
    for (; i < (n & ~3); i++) {
        const float g = gate[i];
        const float e = orc_exp_neon(-g);
        const float s = g / orc_neon_add(1.0f, e);
        y[i] = orc_neon_mul(s, up[i]);
    }
    for (; i < n; i++) {
        const float g = gate[i];
        y[i] = (g / (1.0f + o_expf(-g))) * up[i];
    }
}

/* ---- add_residual, 04/qwen_kernels_opt.c:386-393 ---------------------------- */
void orc_add_residual(float* x, const float* res, int n) {
    int i = 0;
    for (; i < (n & ~3); i++) x[i] = orc_neon_add(x[i], res[i]);
    for (; i < n; i++) x[i] += res[i];
}

/* ---- rmsnorm, 04/qwen_kernels_opt.c:140-175 ---------------------------------
 * Sum of squares in 4 lanes (vmlaq, elements i = j mod 4) over the vector
 * part, combined (s0+s2)+(s1+s3), then the scalar tail; r = 1/sqrtf(ss/n +
 * eps); vector part y = x * (r * (1 + w)), tail y = (x * r) * (1 + w). */
void orc_rmsnorm(float* y, const float* x, const float* w, int n, float eps) {
    float s[4] = {0, 0, 0, 0};
    int i = 0;
    for (; i < (n & ~3); i++) s[i & 3] = orc_neon_add(s[i & 3], orc_neon_mul(x[i], x[i]));
    float ss = lanes4(s);
    for (; i < n; i++) ss += x[i] * x[i];
    const float r = 1.0f / sqrtf((ss / (float)n) + eps);
    for (i = 0; i < (n & ~3); i++) y[i] = orc_neon_mul(x[i], orc_neon_mul(r, orc_neon_add(1.0f, w[i])));
    for (; i < n; i++) y[i] = x[i] * r * (1.0f + w[i]);
}

/* ---- causal_conv1d_update_silu, 04/qwen_kernels_opt.c:511-542 ---------------
 * conv_state = [3][channels] taps (oldest first), weight = [channels][4].
 * Vector part: d = w0*t0, then += w1*t1, w2*t2, w3*x (vmlaq); y = d / (1 +
 * exp_neon(-d)) (scalar division); the taps shift.  Tail: scalar with expf. */
void orc_conv1d_silu(float* y, const float* x, float* st, const float* wt, int C) {
    float* s0 = st;
    float* s1 = st + C;
    float* s2 = st + 2 * C;
    int c = 0;
    for (; c < (C & ~3); c++) {
        const float xc = x[c];
        float d = orc_neon_mul(wt[c * 4 + 0], s0[c]);
        d = orc_neon_add(d, orc_neon_mul(wt[c * 4 + 1], s1[c]));
        d = orc_neon_add(d, orc_neon_mul(wt[c * 4 + 2], s2[c]));
        d = orc_neon_add(d, orc_neon_mul(wt[c * 4 + 3], xc));
        const float e = orc_exp_neon(-d);
        y[c] = d / orc_neon_add(1.0f, e);
        s0[c] = s1[c];
        s1[c] = s2[c];
        s2[c] = xc;
    }
    for (; c < C; c++) {
        const float xc = x[c];
        const float dot = wt[c * 4] * s0[c] + wt[c * 4 + 1] * s1[c] + wt[c * 4 + 2] * s2[c] + wt[c * 4 + 3] * xc;
        y[c] = dot / (1.0f + o_expf(-dot));
        s0[c] = s1[c];
        s1[c] = s2[c];
        s2[c] = xc;
    }
}

/* ---- qk_l2norm, 04/qwen_kernels_opt.c:547-588 -------------------------------
 * Per head: sums of squares in 4 lanes + scalar tail; k *= 1/sqrtf(k_sq +
 * 1e-6), q *= (1/sqrtf(head_dim)) / sqrtf(q_sq + 1e-6), vector part only (the
 * board build leaves a head_dim % 4 tail unscaled). */
void orc_qk_l2norm(float* q, float* k, int H, int D) {
    const float q_scale = 1.0f / sqrtf((float)D);
    const float eps = 1e-6f;
    for (int h = 0; h < H; h++) {
        float* kh = k + h * D;
        float* qh = q + h * D;
        float a[4] = {0, 0, 0, 0}, b[4] = {0, 0, 0, 0};
        int i = 0;
        for (; i < (D & ~3); i++) {
            a[i & 3] = orc_neon_add(a[i & 3], orc_neon_mul(kh[i], kh[i]));
            b[i & 3] = orc_neon_add(b[i & 3], orc_neon_mul(qh[i], qh[i]));
        }
        float k_sq = lanes4(a), q_sq = lanes4(b);
        for (; i < D; i++) {
            k_sq += kh[i] * kh[i];
            q_sq += qh[i] * qh[i];
        }
        const float kr = 1.0f / sqrtf(k_sq + eps);
        const float qr = q_scale / sqrtf(q_sq + eps);
        for (i = 0; i < (D & ~3); i++) {
            kh[i] = orc_neon_mul(kh[i], kr);
            qh[i] = orc_neon_mul(qh[i], qr);
        }
    }
}

/* ---- gdn_gates, 04/qwen_kernels_opt.c:593-620 -------------------------------
 * Per head: av = wa[h].x, bv = wb[h].x (4 lanes + scalar tail);
 * beta = 1/(1 + expf(-bv)); alpha = expf(nea[h] * log1pf(expf(av + dt[h]))). */
void orc_gdn_gates(float* alpha, float* beta, const float* x, const float* wa, const float* wb, const float* nea,
                   const float* dt, int H, int K) {
    for (int h = 0; h < H; h++) {
        const float* ra = wa + (size_t)h * K;
        const float* rb = wb + (size_t)h * K;
        float a[4] = {0, 0, 0, 0}, b[4] = {0, 0, 0, 0};
        int i = 0;
        for (; i < (K & ~3); i++) {
            a[i & 3] = orc_neon_add(a[i & 3], orc_neon_mul(ra[i], x[i]));
            b[i & 3] = orc_neon_add(b[i & 3], orc_neon_mul(rb[i], x[i]));
        }
        float av = lanes4(a), bv = lanes4(b);
        for (; i < K; i++) {
            av += ra[i] * x[i];
            bv += rb[i] * x[i];
        }
        beta[h] = 1.0f / (1.0f + o_expf(-bv));
        const float z = av + dt[h];
        alpha[h] = o_expf(nea[h] * o_log1pf(o_expf(z)));
    }
}

/* ---- gdn_recurrent_step, 04/qwen_kernels_opt.c:659-813 (board path) ---------
 * State S[h][i][j] kept logically (row i = input index, column j = output);
 * the reference's blocked layout is internal to it.  Per head: qk = q.k in 4
 * lanes over j (combined (l0+l2)+(l1+l3)); per column j: kv = sum_i k[i] *
 * S[i][j] and qs = sum_i q[i] * S[i][j] in ascending i; d = (v[j] - kv*a) *
 * b; out[j] = qs*a + qk*d; then S[i][j] = S[i][j]*a + d*k[i]. */
void orc_gdn_step(float* out, float* S, const float* q, const float* k, const float* v, const float* alpha,
                  const float* beta, int H, int D) {
    for (int h = 0; h < H; h++) {
        const float* qh = q + h * D;
        const float* kh = k + h * D;
        const float* vh = v + h * D;
        float* Sh = S + (size_t)h * D * D;
        const float a = alpha[h], b = beta[h];
        float acc[4] = {0, 0, 0, 0};
        for (int j = 0; j < D; j++) acc[j & 3] = orc_neon_add(acc[j & 3], orc_neon_mul(qh[j], kh[j]));
        const float qk = lanes4(acc);
        for (int j = 0; j < D; j++) {
            float kv = 0.0f, qs = 0.0f;
            for (int i = 0; i < D; i++) {
                const float s = Sh[(size_t)i * D + j];
                kv = orc_neon_add(kv, orc_neon_mul(s, kh[i]));
                qs = orc_neon_add(qs, orc_neon_mul(s, qh[i]));
            }
            const float d = orc_neon_mul(nsub(vh[j], orc_neon_mul(kv, a)), b);
            out[h * D + j] = orc_neon_add(orc_neon_mul(qs, a), orc_neon_mul(qk, d));
            for (int i = 0; i < D; i++) {
                float* s = &Sh[(size_t)i * D + j];
                *s = orc_neon_add(orc_neon_mul(*s, a), orc_neon_mul(d, kh[i]));
            }
        }
    }
}

/* ---- rmsnorm_gated, 04/qwen_kernels_opt.c:818-847 ---------------------------
 * Per head: sum of squares in 4 lanes + tail; r = 1/sqrtf(ss/head_dim + eps);
 * y = ((x * r) * w) * (z / (1 + expf(-z))) in scalar arithmetic. */
void orc_rmsnorm_gated(float* y, const float* x, const float* z, const float* w, int H, int D, float eps) {
    for (int h = 0; h < H; h++) {
        const float* xh = x + h * D;
        const float* zh = z + h * D;
        float* yh = y + h * D;
        float s[4] = {0, 0, 0, 0};
        int i = 0;
        for (; i < (D & ~3); i++) s[i & 3] = orc_neon_add(s[i & 3], orc_neon_mul(xh[i], xh[i]));
        float ss = lanes4(s);
        for (; i < D; i++) ss += xh[i] * xh[i];
        const float r = 1.0f / sqrtf((ss / (float)D) + eps);
        for (i = 0; i < D; i++) {
            const float zi = zh[i];
            yh[i] = xh[i] * r * w[i] * (zi / (1.0f + o_expf(-zi)));
        }
    }
}

/* ---- the compiled forward loop, 04/qwen_kernels_opt.c:866-1049 -------------
 * Plans mirror the reference's LinearLayerPlan / MlpPlan (host pointers to
 * the SoA planes and float parameters); GEMVs are the board-build bfp8_gemv
 * (orc_gemv_neon). */
typedef struct {
    const float* in_ln_w;
    const int8_t* mant_qkv; const uint8_t* exp_qkv; int M_qkv; int K_qkv;
    const float* conv_w; float* conv_s;
    const float* wa; const float* wb; const float* nea; const float* dt;
    float* state;
    const int8_t* mant_z; const uint8_t* exp_z; int M_z; int K_z;
    const float* norm_w;
    const int8_t* mant_o; const uint8_t* exp_o; int M_o; int K_o;
    const float* post_ln_w;
    const int8_t* mant_gate; const uint8_t* exp_gate; int M_gate; int K_gate;
    const int8_t* mant_up; const uint8_t* exp_up; int M_up; int K_up;
    const int8_t* mant_down; const uint8_t* exp_down; int M_down; int K_down;
} orc_linear_plan;

typedef struct {
    const float* post_ln_w;
    const int8_t* mant_gate; const uint8_t* exp_gate; int M_gate; int K_gate;
    const int8_t* mant_up; const uint8_t* exp_up; int M_up; int K_up;
    const int8_t* mant_down; const uint8_t* exp_down; int M_down; int K_down;
} orc_mlp_plan;

static void gemv(float* y, const float* x, const int8_t* m, const uint8_t* e, int M, int K) {
    orc_gemv_neon(y, x, m, e, M, K, NULL, NULL, NULL);
}

/* forward_mlp, 04/qwen_kernels_opt.c:994-1004 (h updated in place). */
void orc_forward_mlp(const orc_mlp_plan* p, float* h) {
    float normed[1024], gate[3584], up[3584], inter[3584], down[1024];
    orc_rmsnorm(normed, h, p->post_ln_w, 1024, 1e-6f);
    gemv(gate, normed, p->mant_gate, p->exp_gate, p->M_gate, p->K_gate);
    gemv(up, normed, p->mant_up, p->exp_up, p->M_up, p->K_up);
    orc_swiglu(inter, gate, up, 3584);
    gemv(down, inter, p->mant_down, p->exp_down, p->M_down, p->K_down);
    orc_add_residual(h, down, 1024);
}

/* forward_linear_layer, 04/qwen_kernels_opt.c:938-992 (h updated in place). */
void orc_forward_linear_layer(const orc_linear_plan* p, float* h) {
    static float normed[1024], qkv[6144], mixed[6144], alpha[16], beta[16], attn[2048], zb[2048], gated[2048],
        o[1024], post[1024], gate[3584], up[3584], inter[3584], down[1024];
    orc_rmsnorm(normed, h, p->in_ln_w, 1024, 1e-6f);
    gemv(qkv, normed, p->mant_qkv, p->exp_qkv, p->M_qkv, p->K_qkv);
    orc_conv1d_silu(mixed, qkv, p->conv_s, p->conv_w, 6144);
    orc_qk_l2norm(mixed, mixed + 2048, 16, 128);
    orc_gdn_gates(alpha, beta, normed, p->wa, p->wb, p->nea, p->dt, 16, 1024);
    orc_gdn_step(attn, p->state, mixed, mixed + 2048, mixed + 4096, alpha, beta, 16, 128);
    gemv(zb, normed, p->mant_z, p->exp_z, p->M_z, p->K_z);
    orc_rmsnorm_gated(gated, attn, zb, p->norm_w, 16, 128, 1e-6f);
    gemv(o, gated, p->mant_o, p->exp_o, p->M_o, p->K_o);
    orc_add_residual(h, o, 1024);
    orc_rmsnorm(post, h, p->post_ln_w, 1024, 1e-6f);
    gemv(gate, post, p->mant_gate, p->exp_gate, p->M_gate, p->K_gate);
    gemv(up, post, p->mant_up, p->exp_up, p->M_up, p->K_up);
    orc_swiglu(inter, gate, up, 3584);
    gemv(down, inter, p->mant_down, p->exp_down, p->M_down, p->K_down);
    orc_add_residual(h, down, 1024);
}

/* forward_token_c, 04/qwen_kernels_opt.c:1008-1049: embedding row (bf16,
 * token_id % 65536), 24 layers (full-attention layers: the callback, then the
 * MLP), final rmsnorm, bf16 lm_head argmax (tail dropped). */
typedef void (*orc_attn_cb)(int layer, float* h, void* ctx);

int orc_forward_token(int token_id, float* h, const orc_linear_plan* lin, const orc_mlp_plan* mlp,
                      const int* is_full, const float* final_norm_w, const uint16_t* embed, orc_attn_cb cb,
                      void* ctx, int vocab) {
    const uint16_t* row = embed + (size_t)(token_id % 65536) * 1024;
    for (int i = 0; i < 1024; i++) {
        uint32_t u = (uint32_t)row[i] << 16;
        memcpy(h + i, &u, 4);
    }
    int li = 0;
    for (int l = 0; l < 24; l++) {
        if (is_full[l]) {
            if (cb) cb(l, h, ctx);
            orc_forward_mlp(&mlp[l], h);
        } else {
            orc_forward_linear_layer(&lin[li++], h);
        }
    }
    static float normed[1024];
    orc_rmsnorm(normed, h, final_norm_w, 1024, 1e-6f);
    float* logits = (float*)malloc((size_t)vocab * sizeof(float));
    if (!logits) return -1;
    for (int t = 0; t < vocab; t++) logits[t] = orc_bf16_dot(normed, embed + (size_t)t * 1024, 1024, 0);
    const int best = orc_argmax(logits, vocab);
    free(logits);
    return best;
}
