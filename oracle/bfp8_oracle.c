/*
 * bfp8_oracle.c -- CPU restatement of the reference's W8A16 BFP8 GEMV path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the oracle, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load the library built from it.  The HIP library never links or calls it.
 *
 * Every function restates the reference's algorithm from its source text
 * (citations are relative to the reference root; `04/` is the on-board tools
 * directory, `02/` the RTL directory).  The reference's NEON path cannot be
 * compiled here (no ARM toolchain), so its arithmetic is restated scalar:
 *
 *   - Advanced SIMD on ARMv7 always runs flush-to-zero with round-to-nearest:
 *     subnormal operands are read as signed zero and results that are tiny
 *     before rounding are written as signed zero.  neon_mul / neon_add model
 *     that exactly (products and sums are formed exactly in double, whose 53
 *     bits make the final float rounding innocuous: 53 >= 2*24+2).
 *   - vmlaq_n_f32 on Cortex-A9 is the chained (unfused) multiply-accumulate:
 *     the product is rounded, then the sum is rounded.
 *   - Scalar code (quant_x_blocks, the odd-M tail, the float path) runs on
 *     VFP with IEEE subnormals; this file is compiled with
 *     -ffp-contract=off so C float expressions round after every operation.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   orc_lane_sums       brute-force integer sums; 279616 known answer;
 *                       tb_gemv_core LCG legacy cases (02/tb_gemv_core.v)
 *   orc_quant_x         closed-form cases (amax element -> +-16384, zero and
 *                       tiny blocks, half-way ties, NaN/inf), brute force
 *   orc_gemv_neon       exact-arithmetic cases whose float sums cannot round,
 *                       lane-order cases that fail every other summation
 *                       order, flush-to-zero cases, float64 bound vs the
 *                       tb_gemv_core golden model
 *   orc_gemv_float      bit-exact vs the reference's own host build (oracle/_ref)
 *   orc_gemv_fallback   pairwise: bit-exact vs numpy's own np.sum on the
 *                       engine's expression (the numpy of this image, 2.2.6);
 *                       sequential: vs np.cumsum's last element (add.accumulate
 *                       adds left to right in every numpy)
 *   orc_argmax/orc_topk bit-exact vs the reference's own host build of
 *                       lm_head_argmax / lm_head_topk (oracle/_ref), and a
 *                       brute-force (score desc, id asc) sort
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- EXP_SCALE, 04/qwen_kernels_opt.c:104, :126-135 -------------------- */
float orc_exp_scale(int e) { return ldexpf(1.0f, e - 134); }

/* ---- Advanced SIMD float model (flush-to-zero, unfused) ----------------- */
static float ftz_in(float v) {
    return (fabsf(v) < FLT_MIN) ? copysignf(0.0f, v) : v; /* NaN passes through */
}
static float ftz_out(double exact) {
    if (exact != 0.0 && fabs(exact) < (double)FLT_MIN) return copysignf(0.0f, (float)exact);
    return (float)exact;
}
float orc_neon_mul(float a, float b) {
    a = ftz_in(a);
    b = ftz_in(b);
    return ftz_out((double)a * (double)b); /* 24x24 bits: exact in double */
}
float orc_neon_add(float a, float b) {
    a = ftz_in(a);
    b = ftz_in(b);
    return ftz_out((double)a + (double)b);
}

/* ---- quant_x_blocks, 04/qwen_kernels_opt.c:182-205 ----------------------
 * Per 64-block: amax = max |x| (a NaN never wins `v > amax`); if amax > 1e-20
 * then q = 16384/amax, xscale = amax/16384, xq = (int16)lrintf(x*q); else the
 * block is zero.  The reference skips the work when called again with the
 * same (x pointer, K); that cache is not restated: results are identical
 * whenever the contents are unchanged. */
void orc_quant_x(const float* x, int K, int16_t* xq, float* xscale) {
    int nb = K / 64;
    for (int b = 0; b < nb; b++) {
        const float* xb = x + (size_t)b * 64;
        float amax = 0.0f;
        for (int i = 0; i < 64; i++) {
            float v = fabsf(xb[i]);
            if (v > amax) amax = v;
        }
        if (amax > 1e-20f) {
            float q = 16384.0f / amax;
            xscale[b] = amax / 16384.0f;
            for (int i = 0; i < 64; i++) {
                float p = xb[i] * q;
                /* lrintf: round half to even; NaN converts to 0 on the board
                 * (VFP vcvt) and, truncated to int16, on x86 as well. */
                long r = isnan(p) ? 0 : lrintf(p);
                xq[b * 64 + i] = (int16_t)r;
            }
        } else {
            xscale[b] = 0.0f;
            memset(xq + (size_t)b * 64, 0, 64 * sizeof(int16_t));
        }
    }
}

/* ---- per-lane int32 block sums, 04/qwen_kernels_opt.c:226-257 ------------
 * vmlal_s16 over (w, xq) slices at i, i+4, i+8, i+12 leaves lane j of a0+a1
 * holding S_j = sum over k = j (mod 4) of w[k]*xq[k].  Exact integers, so the
 * order of the brute force below is free.  lanes: [M][K/64][4]. */
void orc_lane_sums(const int8_t* mant, const int16_t* xq, int M, int K, int32_t* lanes) {
    int nb = K / 64;
    for (int m = 0; m < M; m++) {
        const int8_t* row = mant + (size_t)m * K; /* row stride is K, 04/...:220 */
        for (int b = 0; b < nb; b++) {
            int32_t s[4] = {0, 0, 0, 0};
            for (int k = 0; k < 64; k++)
                s[k & 3] += (int32_t)row[b * 64 + k] * (int32_t)xq[b * 64 + k];
            for (int j = 0; j < 4; j++) lanes[((size_t)m * nb + b) * 4 + j] = s[j];
        }
    }
}

/* ---- the engine's numpy fallback, 04/qwen_real_engine.py:1230-1238 -------
 *   scales = 2 ** (exps - 134)          float32, exact powers of two
 *   dots   = np.sum(m * x, axis=-1)     per block, float32 products
 *   y      = np.sum(dots * scales, axis=-1)
 * in numpy's float32 summation order: pairwise (numpy >= 1.9: +0.0 plus
 * pairwise_sum, which adds n < 8 elements one by one from -0.0, keeps eight
 * accumulators up to 128 elements, splits larger n at n/2 rounded down to a
 * multiple of 8) or sequential (numpy 1.8.2, the board's: a[0] + a[1] + ...).
 * K % 64 == 0 (the engine's reshape requires it). */
static float orc_np_pairwise(const float* a, int n) {
    if (n < 8) {
        float r = -0.0f;
        for (int i = 0; i < n; i++) r += a[i];
        return r;
    }
    if (n <= 128) {
        float r[8];
        int i;
        for (int j = 0; j < 8; j++) r[j] = a[j];
        for (i = 8; i < n - (n % 8); i += 8)
            for (int j = 0; j < 8; j++) r[j] += a[i + j];
        float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < n; i++) res += a[i];
        return res;
    }
    int n2 = n / 2;
    n2 -= n2 % 8;
    return orc_np_pairwise(a, n2) + orc_np_pairwise(a + n2, n - n2);
}

static float orc_np_sum(const float* a, int n, int pairwise) {
    if (pairwise) return 0.0f + orc_np_pairwise(a, n);
    if (n == 0) return 0.0f;
    float r = a[0];
    for (int i = 1; i < n; i++) r += a[i];
    return r;
}

void orc_gemv_fallback(float* y, const float* x, const int8_t* mant, const uint8_t* exps, int M, int K,
                       int pairwise) {
    int nb = K / 64;
    float* terms = (float*)malloc(sizeof(float) * (size_t)(nb > 0 ? nb : 1));
    float p[64];
    for (int m = 0; m < M; m++) {
        for (int b = 0; b < nb; b++) {
            const int8_t* blk = mant + (size_t)m * K + (size_t)b * 64;
            for (int k = 0; k < 64; k++) p[k] = (float)blk[k] * x[b * 64 + k];
            terms[b] = orc_np_sum(p, 64, pairwise) * ldexpf(1.0f, (int)exps[(size_t)m * nb + b] - 134);
        }
        y[m] = orc_np_sum(terms, nb, pairwise);
    }
    free(terms);
}

/* ---- host float path, 04/qwen_kernels_opt.c:311-325 ----------------------
 * Unquantized float x, sequential float dot per block, then sum += dot*scale.
 * Used by the NEON build when K > 4096 and by any non-NEON build. */
void orc_gemv_float(float* y, const float* x, const int8_t* mant, const uint8_t* exps,
                    int M, int K) {
    int nb = K / 64;
    for (int m = 0; m < M; m++) {
        const int8_t* row_m = mant + (size_t)m * K;
        const uint8_t* row_e = exps + (size_t)m * nb;
        float sum = 0.0f;
        for (int b = 0; b < nb; b++) {
            float scale = orc_exp_scale(row_e[b]);
            const int8_t* blk_m = row_m + b * 64;
            const float* blk_x = x + b * 64;
            float block_dot = 0.0f;
            for (int i = 0; i < 64; i++) block_dot += (float)(int)blk_m[i] * blk_x[i];
            sum += block_dot * scale;
        }
        y[m] = sum;
    }
}

/* ---- bfp8_gemv as built for the board, 04/qwen_kernels_opt.c:207-308 -----
 * K <= 4096: quantize x, then
 *   row pairs (m < M&~1), per block b and lane j (NEON, flush-to-zero):
 *       fs_j = fs_j + ((float(S_j) * EXP_SCALE[e]) * xscale[b])
 *     y = (fs_0 + fs_2) + (fs_1 + fs_3)                       (:258-277)
 *   odd last row (IEEE scalar, one int32 per block):
 *       sum = sum + ((float(S) * EXP_SCALE[e]) * xscale[b])    (:279-306)
 * K > 4096: the float path above.
 * Optional outputs (may be NULL): xq[K], xscale[K/64], lanes[M][K/64][4]. */
void orc_gemv_neon(float* y, const float* x, const int8_t* mant, const uint8_t* exps,
                   int M, int K, int16_t* xq_out, float* xscale_out, int32_t* lanes_out) {
    if (K > 4096) {
        orc_gemv_float(y, x, mant, exps, M, K);
        return;
    }
    int nb = K / 64;
    int16_t xq[4096];
    float xscale[64];
    orc_quant_x(x, K, xq, xscale);
    if (xq_out) memcpy(xq_out, xq, (size_t)nb * 64 * sizeof(int16_t));
    if (xscale_out) memcpy(xscale_out, xscale, (size_t)nb * sizeof(float));

    for (int m = 0; m < M; m++) {
        const int8_t* row = mant + (size_t)m * K;
        const uint8_t* re = exps + (size_t)m * nb;
        int paired = m < (M & ~1);
        float fs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        float sum = 0.0f;
        for (int b = 0; b < nb; b++) {
            int32_t s[4] = {0, 0, 0, 0};
            for (int k = 0; k < 64; k++)
                s[k & 3] += (int32_t)row[b * 64 + k] * (int32_t)xq[b * 64 + k];
            if (lanes_out)
                for (int j = 0; j < 4; j++) lanes_out[((size_t)m * nb + b) * 4 + j] = s[j];
            float es = orc_exp_scale(re[b]);
            if (paired) {
                for (int j = 0; j < 4; j++) {
                    float fA = (float)s[j];
                    float t = orc_neon_mul(fA, es);
                    float u = orc_neon_mul(t, xscale[b]);
                    fs[j] = orc_neon_add(fs[j], u);
                }
            } else {
                int32_t tot = s[0] + s[1] + s[2] + s[3];
                sum += (float)tot * es * xscale[b];
            }
        }
        y[m] = paired ? orc_neon_add(orc_neon_add(fs[0], fs[2]), orc_neon_add(fs[1], fs[3]))
                      : sum;
    }
}

/* ---- lm_head_argmax selection, 04/qwen_kernels_opt.c:401-506 -------------
 * Two halves (chunk = n/2, the second takes the remainder); each keeps the
 * first strict maximum above -1e30 (starting id = half start); the halves
 * merge with `>=`, so the first half wins ties.  Restated over a logits
 * array (the reference computes bf16 dot products on the fly). */
int orc_argmax(const float* logits, int n) {
    float bs[2] = {-1e30f, -1e30f};
    int bi[2] = {0, 0};
    int chunk = n / 2;
    for (int tid = 0; tid < 2; tid++) {
        int start = tid * chunk, end = tid ? n : start + chunk;
        float my = -1e30f;
        int id = start;
        for (int t = start; t < end; t++)
            if (logits[t] > my) { my = logits[t]; id = t; }
        bs[tid] = my;
        bi[tid] = id;
    }
    return (bs[0] >= bs[1]) ? bi[0] : bi[1];
}

/* ---- lm_head_topk selection, 04/qwen_sampling.c:110-155, :283-353 --------
 * Streaming insertion tables (strict `<` shifting, eviction only on strict
 * `>` past a full table, offers only above -FLT_MAX) over two halves of the
 * vocabulary, then the second table merged into the first.  Returns the
 * entry count; 0 on invalid arguments. */
typedef struct { int cap, count; int* ids; float* scores; } orc_tk;

static void orc_tk_offer(orc_tk* t, int id, float score) {
    int pos;
    if (t->count < t->cap) {
        pos = t->count;
        while (pos > 0 && t->scores[pos - 1] < score) {
            t->scores[pos] = t->scores[pos - 1];
            t->ids[pos] = t->ids[pos - 1];
            --pos;
        }
        t->scores[pos] = score;
        t->ids[pos] = id;
        t->count++;
    } else if (t->cap > 0 && score > t->scores[t->cap - 1]) {
        pos = t->cap - 1;
        while (pos > 0 && t->scores[pos - 1] < score) {
            t->scores[pos] = t->scores[pos - 1];
            t->ids[pos] = t->ids[pos - 1];
            --pos;
        }
        t->scores[pos] = score;
        t->ids[pos] = id;
    }
}

int orc_topk(const float* logits, int n, int k, int* out_ids, float* out_scores) {
    if (!logits || !out_ids || !out_scores || n <= 0 || k <= 0) return 0;
    int kk = k < n ? k : n;
    int* ib = (int*)malloc((size_t)kk * 2 * sizeof(int));
    float* sb = (float*)malloc((size_t)kk * 2 * sizeof(float));
    if (!ib || !sb) { free(ib); free(sb); return 0; }
    orc_tk tabs[2];
    for (int i = 0; i < 2; i++) {
        tabs[i].cap = kk;
        tabs[i].count = 0;
        tabs[i].ids = ib + (size_t)i * kk;
        tabs[i].scores = sb + (size_t)i * kk;
    }
    int chunk = n / 2;
    for (int tid = 0; tid < 2; tid++) {
        int start = tid * chunk, end = tid ? n : start + chunk;
        float thr = -FLT_MAX;
        for (int t = start; t < end; t++) {
            if (logits[t] > thr) {
                orc_tk_offer(&tabs[tid], t, logits[t]);
                thr = (tabs[tid].count < tabs[tid].cap) ? -FLT_MAX
                                                        : tabs[tid].scores[tabs[tid].cap - 1];
            }
        }
    }
    for (int i = 0; i < tabs[1].count; i++) orc_tk_offer(&tabs[0], tabs[1].ids[i], tabs[1].scores[i]);
    int cnt = tabs[0].count;
    memcpy(out_ids, tabs[0].ids, (size_t)cnt * sizeof(int));
    memcpy(out_scores, tabs[0].scores, (size_t)cnt * sizeof(float));
    free(ib);
    free(sb);
    return cnt;
}

/* ---- block-sum / dequant golden model of 02/tb_gemv_core.v:150-170 --------
 * y[m] = sum_b (double)dots[m][b] * 2^(e-134) * xscale[b], in double: the
 * testbench's independent model, used as a float64 bound on orc_gemv_neon. */
void orc_gemv_f64(double* y, const int8_t* mant, const uint8_t* exps, const int16_t* xq,
                  const float* xscale, int M, int K) {
    int nb = K / 64;
    for (int m = 0; m < M; m++) {
        double acc = 0.0;
        for (int b = 0; b < nb; b++) {
            int64_t s = 0;
            for (int k = 0; k < 64; k++)
                s += (int64_t)mant[(size_t)m * K + b * 64 + k] * xq[b * 64 + k];
            acc += (double)s * ldexp(1.0, exps[(size_t)m * nb + b] - 134) * (double)xscale[b];
        }
        y[m] = acc;
    }
}
