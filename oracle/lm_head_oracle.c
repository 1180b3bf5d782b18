/*
 * lm_head_oracle.c -- CPU restatement of the reference's bf16 tied-embedding
 * lm_head (argmax / streaming top-k) and of its sampler.
 *
 * TEST INFRASTRUCTURE ONLY, like bfp8_oracle.c: only tests/,
 * __graft_entry__.smoke() and bench.py's CPU-baseline leg load the library
 * built from it; the HIP library never links or calls it.
 *
 * Pinning (tests/test_oracle.py):
 *   orc_bf16_dot        exact-arithmetic rows, lane-order rows whose result
 *                       fails every other summation order, flush-to-zero rows,
 *                       the tail rule of each entry point, float64 bound
 *   orc_sample_from_topk  bit-exact vs the reference's own host build of
 *                       sample_from_topk (oracle/_ref/libref_qwen_sampling.so)
 *                       over random candidate lists and arguments
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float orc_neon_mul(float a, float b);
float orc_neon_add(float a, float b);

/* bf16 -> f32: the table holds the high half of the float bits
 * (04/qwen_sampling.c:96-101). */
static float orc_bf16(uint16_t u) {
    uint32_t b = (uint32_t)u << 16;
    float f;
    memcpy(&f, &b, sizeof f);
    return f;
}

/* ---- bf16 row dot product, board build -------------------------------------
 * 04/qwen_kernels_opt.c:417-457 (lm_head_argmax) and 04/qwen_sampling.c:161-245
 * (scan_range_neon): per 8-element chunk, accumulator a0 lane j takes element
 * 8c+j and a1 lane j element 8c+4+j, each by vmlaq_f32 (product rounded, then
 * sum rounded, Advanced SIMD flush-to-zero).  The row's score is
 * ((a0+a1)[0] + (a0+a1)[2]) + ((a0+a1)[1] + (a0+a1)[3]) (vaddq, vadd of the
 * halves, vpadd).  The hidden % 8 trailing elements are dropped by
 * lm_head_argmax (tail = 0) and added one by one in scalar VFP arithmetic by
 * lm_head_topk (tail = 1, 04/qwen_sampling.c:204-207). */
float orc_bf16_dot(const float* h, const uint16_t* row, int hidden, int tail) {
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= hidden; i += 8)
        for (int j = 0; j < 8; j++) a[j] = orc_neon_add(a[j], orc_neon_mul(orc_bf16(row[i + j]), h[i + j]));
    float acc[4];
    for (int j = 0; j < 4; j++) acc[j] = orc_neon_add(a[j], a[4 + j]);
    float s = orc_neon_add(orc_neon_add(acc[0], acc[2]), orc_neon_add(acc[1], acc[3]));
    if (tail)
        for (; i < hidden; i++) s += h[i] * orc_bf16(row[i]);
    return s;
}

/* All vocab scores of the table (rows of `hidden` bf16 values). */
void orc_bf16_logits(const float* h, const uint16_t* table, int vocab, int hidden, int tail, float* out) {
    for (int t = 0; t < vocab; t++) out[t] = orc_bf16_dot(h, table + (size_t)t * hidden, hidden, tail);
}

/* ---- sampler, 04/qwen_sampling.c:358-529 ------------------------------------
 * xorshift32 (a zero state restarts from 0x9E3779B9), uniform = (x >> 8) / 2^24.
 * Candidates are used in (score desc, id asc) order (re-sorted when the list
 * is not non-increasing; an unsorted list holding NaN scores is outside what
 * this restates: the reference's qsort order is then unspecified).  Greedy
 * when !(temperature >= 1e-6); otherwise the first min(top_k, n) candidates
 * (top_k > 0), softmax weights
 * expf((s - max) * (1/T)) summed in double, the top-p prefix (first
 * cumulative probability > clamp(top_p, 0, 1)), one draw r = u * sum_keep
 * against the running sum.  Returns the chosen id, -1 on invalid input,
 * ids[0] without a state. */
static uint32_t orc_xorshift32(uint32_t* s) {
    uint32_t x = *s;
    if (x == 0u) x = 0x9E3779B9u;
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    *s = x;
    return x;
}

int orc_sample_from_topk(const int* ids, const float* scores, int n, float temperature, int top_k, float top_p,
                         uint32_t* rng) {
    if (!ids || !scores || n <= 0) return -1;
    if (!rng) return ids[0];
    int* id = (int*)malloc((size_t)n * sizeof(int));
    float* sc = (float*)malloc((size_t)n * sizeof(float));
    if (!id || !sc) {
        free(id);
        free(sc);
        return ids[0];
    }
    memcpy(id, ids, (size_t)n * sizeof(int));
    memcpy(sc, scores, (size_t)n * sizeof(float));
    int sorted = 1;
    for (int i = 1; i < n && sorted; i++)
        if (sc[i] > sc[i - 1]) sorted = 0;
    if (!sorted) { /* insertion sort by (score desc, id asc) */
        for (int i = 1; i < n; i++) {
            int ci = id[i];
            float cs = sc[i];
            int j = i - 1;
            while (j >= 0 && (sc[j] < cs || (!(sc[j] > cs) && id[j] > ci))) {
                id[j + 1] = id[j];
                sc[j + 1] = sc[j];
                j--;
            }
            id[j + 1] = ci;
            sc[j + 1] = cs;
        }
    }
    int out = id[0];
    if (temperature >= 1e-6f) {
        int m = (top_k > 0 && top_k < n) ? top_k : n;
        float mx = sc[0];
        for (int i = 1; i < m; i++)
            if (sc[i] > mx) mx = sc[i];
        const float inv_t = 1.0f / temperature;
        double all = 0.0;
        for (int i = 0; i < m; i++) all += (double)expf((sc[i] - mx) * inv_t);
        if (all > 0.0) {
            float p = top_p;
            if (!(p > 0.0f)) p = 0.0f;
            if (p > 1.0f) p = 1.0f;
            int keep = m;
            double cum = 0.0;
            for (int i = 0; i < m; i++) {
                cum += (double)expf((sc[i] - mx) * inv_t) / all;
                if (cum > (double)p) {
                    keep = i + 1;
                    break;
                }
            }
            double kept = 0.0;
            for (int i = 0; i < keep; i++) kept += (double)expf((sc[i] - mx) * inv_t);
            if (kept > 0.0) {
                const double u = (double)((float)(orc_xorshift32(rng) >> 8) * (1.0f / 16777216.0f));
                const double r = u * kept;
                int pick = keep - 1;
                cum = 0.0;
                for (int i = 0; i < keep; i++) {
                    cum += (double)expf((sc[i] - mx) * inv_t);
                    if (r < cum) {
                        pick = i;
                        break;
                    }
                }
                out = id[pick];
            }
        }
    }
    free(id);
    free(sc);
    return out;
}
