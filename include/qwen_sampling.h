/*
 * qwen_sampling.h -- C ABI of libqwen_sampling.so, the MI355X drop-in for the
 * reference's sampling library (04/qwen_sampling.c; loaded by ctypes in
 * 04/chat_v3.py:145-159).  It forwards to libqwen_kernels.so (found next to
 * it), so the embedding table's device copy is shared with lm_head_argmax.
 */
#ifndef QWEN_SAMPLING_H
#define QWEN_SAMPLING_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

/* Replaces lm_head_topk(), 04/qwen_sampling.c:283-353: streaming top-k of the
 * bf16 lm_head (board-build dot products; hidden % 8 trailing elements
 * added), sorted by (score desc, id asc) among scores above -FLT_MAX.
 * Returns min(k, vocab_size) candidates or fewer; 0 on invalid arguments
 * (here also a vocabulary above 2^28 rows).  k <= 64 runs fused into the
 * scoring launch, larger k through the scores and a multi-workgroup
 * selection of their keys (include/qwen_kernels.h). */
int lm_head_topk(const float* h, const uint16_t* embed_table, int vocab_size, int hidden_dim, int k, int* out_ids,
                 float* out_scores);

/* Replaces sample_from_topk(), 04/qwen_sampling.c:384-529: temperature /
 * top-k / top-p sampling with the xorshift32 state *rng_state.  Returns the
 * chosen id, -1 on invalid arguments (here also above 2^28 candidates). */
int sample_from_topk(const int* ids, const float* scores, int n, float temperature, int top_k, float top_p,
                     unsigned int* rng_state);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif
