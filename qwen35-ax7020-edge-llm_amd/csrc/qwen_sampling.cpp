// qwen_sampling.cpp -- libqwen_sampling.so: the reference sampling library's
// two entry points (04/qwen_sampling.c:283-353, :384-529), forwarding to
// libqwen_kernels.so so that both libraries share one GPU context and one
// device copy of the embedding table.
#include "qwen_kernels.h"
#include "qwen_sampling.h"

extern "C" int lm_head_topk(const float* h, const uint16_t* embed_table, int vocab_size, int hidden_dim, int k,
                            int* out_ids, float* out_scores) {
    return qwen_lm_head_topk_bf16(h, embed_table, vocab_size, hidden_dim, k, out_ids, out_scores);
}

extern "C" int sample_from_topk(const int* ids, const float* scores, int n, float temperature, int top_k,
                                float top_p, unsigned int* rng_state) {
    return qwen_sample_from_topk(ids, scores, n, temperature, top_k, top_p, rng_state);
}
