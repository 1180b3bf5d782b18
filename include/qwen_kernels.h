/*
 * qwen_kernels.h -- C ABI of libqwen_kernels.so, the MI355X (gfx950) drop-in
 * for the reference's BFP8 GEMV operator library.
 *
 * Three groups of entry points:
 *
 *  1. Reference symbols, same names, signatures and meaning as the
 *     reference's libqwen_kernels.so (bound by ctypes in
 *     04/qwen_real_engine.py:656-725, :848-866).  Host pointers, synchronous:
 *     y is fully written when the call returns.  The GPU does the work.
 *
 *  2. New host-pointer symbols for paths the reference has no entry for
 *     (fused BFP8 lm_head with argmax / top-k, batched GEMV).  Conventions
 *     follow 04/qwen_sampling.c:283-285: return a count, 0 on invalid
 *     arguments.
 *
 *  3. Device-level symbols (prefix bfp8_dev_ / bfp8_plan_): device pointers,
 *     an explicit HIP stream (hipStream_t passed as void*; NULL is the HIP
 *     default stream, bfp8_stream() the library's own), asynchronous; return 0 on success or a negative
 *     BFP8_E* code.  These keep weights and activations resident in HBM.
 *
 * Failure behaviour: the reference's bfp8_gemv has no error channel
 * (04/qwen_kernels_opt.c:207, void).  init_kernels() never aborts; without a
 * usable GPU it prints why and bfp8_gpu_ready() returns 0, so an engine can
 * keep its own numpy path (the reference engine's behaviour when the library
 * does not load, 04/qwen_real_engine.py:663-671).  A void compute entry point
 * called without a usable GPU prints the HIP error to stderr and aborts the
 * process: there is no silent CPU fallback.  Int-returning entry points
 * return their error value instead; bfp8_last_error() gives the message.
 *
 * Numerics: identical to the reference's board build (-DUSE_NEON):
 *   - K <= 4096: x quantized per 64-block to int16 (04/qwen_kernels_opt.c:182-205),
 *     int32 residue-lane block sums, flush-to-zero float epilogue in the
 *     reference's lane order (:226-277); an odd last row uses the scalar
 *     order (:279-306).
 *   - K > 4096: the reference's float path (:311-325).
 */
#ifndef QWEN_KERNELS_H
#define QWEN_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

/* ---- 1. reference symbols -------------------------------------------------- */

/* Replaces init_kernels(), 04/qwen_kernels_opt.c:128-135.  Also selects the
 * GPU (current HIP device) and creates the library's stream.  Idempotent.
 * Does not fail: without a usable GPU it prints the reason to stderr and
 * bfp8_gpu_ready() returns 0. */
void init_kernels(void);

/* 1 when the GPU path can run: a HIP device that is gfx950, this library's
 * code object loaded on it.  0 otherwise, with bfp8_last_error() set.  No
 * counterpart in the reference (whose CPU library is always usable); it is
 * what an engine checks after init_kernels() to fall back to its own numpy
 * path instead of calling entry points that would abort. */
int bfp8_gpu_ready(void);

/* Replaces bfp8_gemv(), 04/qwen_kernels_opt.c:207-326.
 * y[M] = BFP8 W[M][K] (mantissas int8 [M][K], row stride K; exps uint8
 * [M][K/64]) times x[K].  Host pointers.  Weights that live in read-only
 * memory (the engine's PROT_READ mmap, 04/qwen_real_engine.py:745-751) are
 * converted to the GPU layout once and cached by (mantissas, exps, M, K);
 * writable weight buffers are re-uploaded on every call. */
void bfp8_gemv(float* y, const float* x, const int8_t* mantissas, const uint8_t* exps, int M, int K);

/* Replaces lm_head_argmax(), 04/qwen_kernels_opt.c:401-506: the bf16 tied-
 * embedding lm_head (embed_table uint16 [vocab][hidden], the high halves of
 * floats) dotted with h[hidden] in the board build's order (two float32x4
 * accumulators over 8-element chunks, flush-to-zero; hidden % 8 trailing
 * elements dropped), then the lowest id among the maximal scores above -1e30,
 * else 0.  Any hidden.  Host pointers; a read-only table is kept on the
 * device after the first call. */
int lm_head_argmax(const float* h, const uint16_t* embed_table, int vocab_size, int hidden_dim);

/* Replace the stage profiler, 04/qwen_kernels_opt.c:63-101 (same 15 slots,
 * names and order).  As in the reference, only forward_linear_layer,
 * forward_mlp and forward_token_c accumulate into the slots: wall
 * milliseconds per step, each step synchronised while profiling is on.  The
 * forward's fused linear-attention kernel (conv1d, q/k norm, gates, recurrent
 * step, gated norm) is booked to gdn_recurrent_step; the norms, residual adds
 * and swiglu computed inside the GEMV launches to bfp8_gemv; the final norm
 * to rmsnorm. */
void qwen_prof_enable(int on);
void qwen_prof_reset(void);
int qwen_prof_count(void);
double qwen_prof_get(int i);
const char* qwen_prof_name(int i);

/* The decode runtime around the GEMV (04/qwen_kernels_opt.c), host pointers,
 * synchronous, same arguments and results as the board build: Advanced SIMD
 * steps in flush-to-zero float arithmetic in the reference's lane order,
 * scalar steps in IEEE arithmetic; expf / log1pf are computed as exp / log1p
 * in double rounded to float (the board's libm is within an ulp of that). */
void rmsnorm(float* y, const float* x, const float* w, int n, float eps);             /* :140-175 */
void swiglu(float* y, const float* gate, const float* up, int n);                      /* :365-384 */
void add_residual(float* x, const float* res, int n);                                  /* :388-395 */
void causal_conv1d_update_silu(float* y, const float* x, float* conv_state, const float* weight,
                               int channels);                                          /* :511-542 */
void qk_l2norm(float* q, float* k, int num_heads, int head_dim);                      /* :548-588 */
void gdn_gates(float* alpha, float* beta, const float* x, const float* wa, const float* wb,
               const float* neg_exp_alog, const float* dt, int H, int K);             /* :593-620 */
/* state: the reference's blocked layout (:637-650), num_heads x head_dim^2
 * floats; head_dim must be a multiple of 4 and at most 4096 (the board's
 * vector path assumes the former). */
void gdn_recurrent_step(float* attn_out, float* state, const float* q, const float* k, const float* v,
                        const float* alpha, const float* beta, int num_heads, int head_dim);  /* :664-813 */
void rmsnorm_gated(float* y, const float* x, const float* z, const float* norm_w, int num_heads,
                   int head_dim, float eps);                                           /* :832-847 */

/* The compiled forward loop, 04/qwen_kernels_opt.c:866-1049.  The plan
 * structs have the reference's fields, order and layout (the engine's ctypes
 * mirrors, 04/qwen_real_engine.py:20-74).  Shapes are the model's: hidden
 * 1024, 16 linear-attention heads of 128, conv channels 6144, MLP 3584,
 * vocabulary 65536; a plan with other GEMV shapes aborts.  Weights and
 * parameters are converted to device copies on first use and treated as
 * immutable afterwards (bfp8_cache_clear() drops them); the conv and
 * recurrent states follow qwen_forward_state_resident(). */
typedef struct LinearLayerPlan {
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
} LinearLayerPlan;

typedef struct MlpPlan {
    const float* post_ln_w;
    const int8_t* mant_gate; const uint8_t* exp_gate; int M_gate; int K_gate;
    const int8_t* mant_up; const uint8_t* exp_up; int M_up; int K_up;
    const int8_t* mant_down; const uint8_t* exp_down; int M_down; int K_down;
} MlpPlan;

/* 04/qwen_kernels_opt.c:1006; called with the library unlocked, so it may
 * call back into this library (the engine's attention runs bfp8_gemv). */
typedef void (*FullAttnCallback)(int layer_idx, float* h, void* py_context);

void forward_linear_layer(const LinearLayerPlan* p, float* h);                        /* :938-992 */
void forward_mlp(const MlpPlan* p, float* h);                                         /* :994-1004 */
/* :1008-1049: embedding row token_id % 65536 (a negative remainder wraps),
 * 24 layers (full-attention layers: the callback on h, then the MLP), final
 * rmsnorm, lm_head_argmax over 65536 x 1024; h ends as the last hidden state. */
int forward_token_c(int token_id, float* h, const LinearLayerPlan* linear_plans, const MlpPlan* mlp_plans,
                    const int* layer_is_full, const float* final_norm_w, const uint16_t* embed_table,
                    FullAttnCallback full_attn_cb, void* py_context);

/* ---- 2. new host-pointer symbols ------------------------------------------- */

/* BFP8 lm_head: logits = bfp8_gemv(h) over vocab rows (04/qwen_kernels_opt.c:
 * 207-326: an odd last row in the scalar order, the float path for
 * hidden > 4096), then the top k by (score desc, id asc) among logits above
 * -FLT_MAX, exactly the selection of lm_head_topk (04/qwen_sampling.c:283-353).
 * Even vocab, k <= 64 and hidden in [64, 4096] run fused (the logits are
 * never materialised); other arguments go through the scores and a selection
 * kernel.  Returns min(k, #candidates); 0 on invalid arguments (k < 1,
 * vocab < 1 or above 2^28, hidden < 1). */
int bfp8_lm_head_topk(const float* h, const int8_t* mantissas, const uint8_t* exps, int vocab,
                      int hidden, int k, int* out_ids, float* out_scores);

/* Fused BFP8 lm_head argmax with the rule of lm_head_argmax
 * (04/qwen_kernels_opt.c:401-506): lowest id among the maximal logits above
 * -1e30, else 0.  Returns -1 on invalid arguments (as bfp8_lm_head_topk). */
int bfp8_lm_head_argmax(const float* h, const int8_t* mantissas, const uint8_t* exps, int vocab,
                        int hidden);

/* Y[b][M] = bfp8_gemv(X[b][K]) for b < B, weights read once per batch.  The
 * reference's equivalent is B separate bfp8_gemv calls (it has no batched
 * entry, 01/FINAL_REPORT.md:361); results are bit-identical to those. */
void bfp8_gemv_batch(float* Y, const float* X, const int8_t* mantissas, const uint8_t* exps, int M,
                     int K, int B);

/* Replaces the engine's numpy fallback QwenRealEngine.gemv_bfp8
 * (04/qwen_real_engine.py:1230-1238, the path it takes when the operator
 * library lacks bfp8_gemv): y[m] = sum_b (sum_k float(w) * x) * 2^(e-134) with
 * unquantized x, float32 products and numpy's float32 summation order --
 * pairwise != 0: numpy >= 1.9 (pairwise_sum: eight accumulators per 128
 * elements, +0.0 start), pairwise == 0: numpy 1.8.2, the board's (left to
 * right); 04/qwen_real_engine.py:323-329 names both.  Host pointers,
 * synchronous; K a multiple of 64 (the engine's reshape requires it).
 * Returns 0, or a BFP8_E* code (bfp8_last_error says why). */
int bfp8_gemv_fallback(float* y, const float* x, const int8_t* mantissas, const uint8_t* exps, int M, int K,
                       int pairwise);

/* The implementations behind libqwen_sampling.so (include/qwen_sampling.h):
 * lm_head_topk over the bf16 table (04/qwen_sampling.c:283-353; any k and
 * hidden: k <= 64 fused into the scoring launch, larger k through the scores
 * and the selection kernels) and sample_from_topk (04/qwen_sampling.c:384-529;
 * any n up to 2^28 candidates, whose unsorted lists one workgroup sorts).  GPU
 * failures return 0 / -1 with bfp8_last_error set.
 *
 * The selection for k > 64 (every lm_head entry point): the keys sorted in
 * 2048-key blocks, one workgroup each, then each block's first min(k, 2048)
 * keys ranked against every block's; at 65,536 rows about 20 us for k = 65
 * and 60 us for k >= vocab after the scores.  Above 2^20 rows one workgroup
 * sorts every key instead (about 2 ms at 65,536 keys, growing as n log^2 n). */
int qwen_lm_head_topk_bf16(const float* h, const uint16_t* embed_table, int vocab_size, int hidden_dim, int k,
                           int* out_ids, float* out_scores);
int qwen_sample_from_topk(const int* ids, const float* scores, int n, float temperature, int top_k, float top_p,
                          unsigned int* rng_state);

/* Where the forward keeps the layers' conv and recurrent states.
 * 0 (default): in the caller's buffers, as the reference does: every
 * forward call copies them to the device and back.  1: on the device, after
 * one copy from the caller's buffers when a layer is first seen; the caller's
 * buffers are then neither read nor written, qwen_forward_reset_state()
 * zeroes the device states (what the engine's reset_state does to its
 * buffers, 04/qwen_real_engine.py:808-813) and qwen_forward_sync_state()
 * copies them back.  Switching to 0 copies them back first.  Returns the
 * previous mode. */
int qwen_forward_state_resident(int on);
void qwen_forward_reset_state(void);
void qwen_forward_sync_state(void);

/* The weight image the exporter writes (05/export_qwen35_weights_bfp8_64k.py:
 * 64-80, :159-174) and its JSON manifest (06/qwen35_weights_64k_manifest.json:
 * per tensor type, shape, file_offset, byte_size, and for "block64_bfp8"
 * mantissa_bytes / exponent_bytes).
 *
 * qwen_weights_scan parses and checks the manifest against an image of
 * image_bytes: 64-byte aligned offsets inside the image, a BFP8 tensor [M, K]
 * with K % 64 == 0 holding M*K mantissa bytes then ceil8(M*K/64) exponent
 * bytes (05/bfp8_packer.py:53-86), raw tensors of 4 (fp32) or 2 (bf16) bytes
 * per element.  Returns the number of tensors and fills the per-type counts
 * and the BFP8 byte total; a negative BFP8_E* code on the first bad entry
 * (bfp8_last_error names it).  No GPU is touched.
 *
 * qwen_weights_preload does the same checks on the mapped image (host
 * memory), then converts every BFP8 tensor to the GPU layout once and keeps
 * it under the host addresses the engine's slicing produces (mant = raw[:M*K],
 * exps = raw[M*K:], 04/qwen_real_engine.py:834-846), so that bfp8_gemv and
 * the forward find it resident; the bf16 table and the fp32 tensors are
 * copied to the device too.  The image is treated as immutable until
 * bfp8_cache_clear().  Returns the number of BFP8 tensors converted. */
int qwen_weights_scan(const char* manifest_json, size_t image_bytes, int* n_bfp8, int* n_f32, int* n_bf16,
                      uint64_t* bfp8_bytes);
int qwen_weights_preload(const void* image, size_t image_bytes, const char* manifest_json);

/* Message of the most recent failure of this library ("" if none). */
const char* bfp8_last_error(void);

/* Drops every cached device copy of weights and forward parameters (and
 * the forward's device states, resident ones included). */
void bfp8_cache_clear(void);
/* Device bytes the library holds (caches, workspaces, per-stream scratch). */
size_t bfp8_device_bytes(void);
/* No counterpart in the reference; a testing aid for callers that must rehearse
 * a full device: the library's device allocations beyond `bytes` in total then
 * fail as a full device's would (0 lifts the limit).  A weight or bf16 table
 * that would be cached is then uploaded per call instead (the result is the
 * same); an entry point that still cannot allocate returns its error code, or,
 * without an error channel (bfp8_gemv and the other void entry points),
 * aborts. */
void bfp8_debug_device_limit(size_t bytes);

/* ---- 3. device-level symbols ------------------------------------------------ */

#define BFP8_OK 0
#define BFP8_EINVAL (-1)
#define BFP8_EHIP (-2)
#define BFP8_ENOMEM (-3)

/* Bytes of the GPU planes of an M x K BFP8 matrix (bfp8_layout.h). */
size_t bfp8_dev_mant_bytes(int M, int K);
size_t bfp8_dev_exps_bytes(int M, int K);
/* Bytes of the split activation of a K vector (K/64 * 128). */
size_t bfp8_dev_xsplit_bytes(int K);

/* Converter: the packer's SoA planes (05/bfp8_packer.py:53-86 as sliced by
 * 04/qwen_real_engine.py:834-846: mantissas [M][K], exps [M][K/64]) to the
 * GPU planes, and back.  All pointers on the device. */
int bfp8_dev_pack(int8_t* mant_gpu, uint8_t* exps_gpu, const int8_t* mant_soa,
                  const uint8_t* exps_soa, int M, int K, void* stream);
int bfp8_dev_unpack(int8_t* mant_soa, uint8_t* exps_soa, const int8_t* mant_gpu,
                    const uint8_t* exps_gpu, int M, int K, void* stream);

/* Activation quantizer (04/qwen_kernels_opt.c:182-205) on the device:
 * x[K] -> xq[K] (may be NULL), xscale[K/64], xsplit (bfp8_dev_xsplit_bytes). */
int bfp8_dev_quantize(int16_t* xq, float* xscale, uint32_t* xsplit, const float* x, int K,
                      void* stream);

/* GEMV on quantized activations, K <= 4096.  y[M]; lane_sums (may be NULL)
 * receives the int32 residue-lane block sums [M][K/64][4] (lane j of block b
 * = sum over k = j mod 4 of w*xq, the reference's NEON accumulator lanes). */
int bfp8_dev_gemv(float* y, const uint32_t* xsplit, const float* xscale, const int8_t* mant_gpu,
                  const uint8_t* exps_gpu, int M, int K, int32_t* lane_sums, void* stream);

/* The reference's float path (04/qwen_kernels_opt.c:311-325) on the device,
 * unquantized x; the path bfp8_gemv takes for K > 4096. */
int bfp8_dev_gemv_float(float* y, const float* x, const int8_t* mant_gpu, const uint8_t* exps_gpu,
                        int M, int K, void* stream);

/* bfp8_gemv_fallback on device buffers (x: K floats, unquantized). */
int bfp8_dev_gemv_fallback(float* y, const float* x, const int8_t* mant_gpu, const uint8_t* exps_gpu, int M, int K,
                           int pairwise, void* stream);

/* Batched GEMV: Y[B][M]; xsplit is B consecutive split vectors
 * (bfp8_dev_xsplit_bytes(K) each), xscale B x K/64.  B in 1..16. */
int bfp8_dev_gemv_batch(float* Y, const uint32_t* xsplit, const float* xscale,
                        const int8_t* mant_gpu, const uint8_t* exps_gpu, int M, int K, int B,
                        void* stream);

/* The BFP8 lm_head on quantized activations (hidden <= 4096): outputs on the
 * device (ids[min(k, vocab)], scores[min(k, vocab)], count, argmax), any
 * vocab and k as bfp8_lm_head_topk.  Uses library-owned device scratch kept
 * per stream: calls on one stream are ordered, calls on different streams
 * use different scratch. */
int bfp8_dev_lm_head_topk(int* out_ids, float* out_scores, int* out_count, int* out_argmax,
                          const uint32_t* xsplit, const float* xscale, const int8_t* mant_gpu,
                          const uint8_t* exps_gpu, int vocab, int hidden, int k, void* stream);

/* No counterpart in the reference: bfp8_dev_lm_head_topk for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results; it
 * allocates nothing: its partial lists, scores and sort keys live in one
 * fixed device array of the library (5 MiB per GPU, held until the process
 * ends; its address is looked up by init_kernels or the first call on a
 * device).  Limits: vocab <= 262144, hidden in [64, 4096]; larger sizes
 * return BFP8_EINVAL with bfp8_last_error set.  Every call on one GPU shares
 * that array: calls that overlap on one GPU (other streams, other threads)
 * race and must be ordered by the caller. */
int bfp8_dev_lm_head_topk_noalloc(int* out_ids, float* out_scores, int* out_count, int* out_argmax,
                                  const uint32_t* xsplit, const float* xscale, const int8_t* mant_gpu,
                                  const uint8_t* exps_gpu, int vocab, int hidden, int k, void* stream);

/* bf16 tied-embedding lm_head on device buffers: scores of every row in the
 * board build's order (tail = 0: hidden % 8 trailing elements dropped, as
 * lm_head_argmax; tail = 1: added in IEEE arithmetic, as lm_head_topk),
 * written to logits[vocab] when logits is not NULL; with k > 0 also the top
 * k (ids[min(k, vocab)], scores, count, argmax by the lm_head_argmax rule;
 * k <= 64 fused into the scoring launch).  k = 0 needs logits.  Any hidden
 * (above 4096 h is read from global memory instead of an LDS copy).
 * Scratch per stream, as bfp8_dev_lm_head_topk. */
int bf16_dev_lm_head(int* out_ids, float* out_scores, int* out_count, int* out_argmax, float* logits,
                     const float* h, const uint16_t* embed_table, int vocab, int hidden, int k, int tail,
                     void* stream);

/* The same lm_head over the table in its tile layout, which the library's
 * own cached tables use (lm_head_argmax, lm_head_topk, forward_token_c,
 * qwen_weights_preload) and which streams the table with one contiguous
 * 2 KiB run per wavefront step and 16 rows per wavefront: rows in groups of
 * 16, nT = 4 * ceil(vocab / 64) groups (rows past vocab zero); element
 * e = 8c + j of row 16T + r, with c = 4q + cc, q = 2p + s and j = 4 hi + g,
 * at uint16 offset (((p * nT + T) * 2 + s) * 64 + 4r + g) * 8 + 2 cc + hi.
 * The model's width only: hidden == 1024.  No counterpart in the reference (its table is
 * row-major in host memory).
 * bf16_dev_tiles_bytes: bytes of the layout (0: width not supported);
 * bf16_dev_tile_table: row-major device table -> tile layout (distinct
 * buffers); bf16_dev_lm_head_tiles: bf16_dev_lm_head's results (no tail:
 * hidden % 8 == 0) from the tile layout. */
size_t bf16_dev_tiles_bytes(int vocab, int hidden);
int bf16_dev_tile_table(uint16_t* tiles, const uint16_t* embed_table, int vocab, int hidden, void* stream);
int bf16_dev_lm_head_tiles(int* out_ids, float* out_scores, int* out_count, int* out_argmax, float* logits,
                           const float* h, const uint16_t* tiles, int vocab, int hidden, int k, void* stream);

/* sample_from_topk (04/qwen_sampling.c:384-529) on the device: candidates
 * ids[]/scores[] (count from *count when count is not NULL, clamped to
 * [0, n], else n; n is the capacity, at most 2^28; no candidate gives -1),
 * xorshift32 state *rng_state updated in place (NULL: ids[0]), chosen id to
 * *out_id.  work: 8*n bytes of device scratch.  One workgroup: the ordering
 * and the exponentials in parallel, the double sums and the draw in the
 * reference's order. */
int bfp8_dev_sample_from_topk(int* out_id, const int* ids, const float* scores, const int* count, int n,
                              float temperature, int top_k, float top_p, uint32_t* rng_state, void* work,
                              void* stream);

/* GPU planes of a tensor qwen_weights_preload converted, by manifest name. */
int qwen_weights_find(const char* name, const int8_t** mant_gpu, const uint8_t** exps_gpu, int* M, int* K);

/* GPU planes from the PL GEMV core's per-row stream (device memory): for each
 * row, its K/64 exponent bytes, then its K mantissas (02/gemv_core.v:23-24,
 * 02/tb_gemv_core.v:281-297).  K % 64 == 0. */
int bfp8_dev_pack_rows(int8_t* mant_gpu, uint8_t* exps_gpu, const uint8_t* row_stream, int M, int K, void* stream);

/* A sweep plan: many independent GEMVs (and at most one fused lm_head).
 * Item i reads x (device, K floats) and writes y (device, M floats), or, for
 * the lm_head item (topk > 0), the four top-k outputs.
 *
 * A plan whose every item has an even M and K a multiple of 512 up to 4096,
 * with 1..128 GEMVs besides the lm_head (and, without an lm_head, more than
 * 384 row tiles in all) runs as ONE launch (bfp8_sweep_kernel): workgroups
 * take 64-row tiles from a device tile queue, quantize each tile's
 * activation in LDS, and the grid's last workgroup merges the lm_head's
 * per-tile top-k lists as they are published.  That merge waits for each
 * list a bounded time (milliseconds); a list that never comes -- possible
 * only if the launch's workgroups are not all resident at once -- makes the
 * run write *out_count = -1 and *out_argmax = -1 (the top-k outputs are then
 * invalid; the caller must treat the run as failed).
 *
 * Other plans run as streaming launches: the lm_head's tiles, then every
 * other GEMV's (larger K first), whose workgroup 0 first merges the lm_head's
 * per-tile top-k partials (without other GEMVs: the stand-alone merge
 * kernel).  When the lm_head's K is a multiple of 64 and at most 1024 its
 * launch also quantizes every activation of the plan (else, and without an
 * lm_head, a quantize launch comes first).  A plan without an lm_head runs
 * one GEMV, or two reading the same x, 16 rows per workgroup, and other
 * plans of few row tiles one tile per 16-wavefront workgroup.
 *
 * Runs of one plan must not overlap in time (queue them on one stream, or
 * order them): the plan's workspaces, ticket counters and partial lists are
 * its own. */
typedef struct bfp8_plan_item {
    const float* x;
    float* y;
    const int8_t* mant_gpu;
    const uint8_t* exps_gpu;
    int M;
    int K;
    int topk;
    int* out_ids;
    float* out_scores;
    int* out_count;
    int* out_argmax;
} bfp8_plan_item;

void* bfp8_plan_create(const bfp8_plan_item* items, int n);
int bfp8_plan_run(void* plan, void* stream);
/* Only the GEMV launches (activations already quantized by a previous
 * bfp8_plan_run or bfp8_plan_quantize; a plan whose lm_head launch quantizes
 * does so here too). */
int bfp8_plan_run_gemv(void* plan, void* stream);
/* One stage of bfp8_plan_run_gemv, for timing each launch on its own:
 * 0 = the single launch, or the lm_head's tiles; 1 = the other GEMVs' tiles
 * with the top-k merge (or the stand-alone merge kernel when the plan has no
 * other GEMV); 2 = odd-row tails and K > 4096 items.  Stages must run in this
 * order; a single-launch plan's stages 1 and 2 are empty. */
int bfp8_plan_launch(void* plan, int stage, void* stream);
/* Name of the (main) kernel a stage launches, "" if the stage is empty. */
const char* bfp8_plan_kernel_name(void* plan, int stage);
int bfp8_plan_quantize(void* plan, void* stream);
void bfp8_plan_destroy(void* plan);

/* Synthetic reference-format planes on the device: mantissas uniform in
 * [-127, 127], exponents uniform in [e_lo, e_hi], from a counter-based hash
 * of (seed, index) -- bfp8_synth_planes_host gives the same bytes. */
int bfp8_dev_synth_planes(int8_t* mant_soa, uint8_t* exps_soa, int M, int K, uint64_t seed,
                          int e_lo, int e_hi, void* stream);
void bfp8_synth_planes_host(int8_t* mant_soa, uint8_t* exps_soa, int M, int K, uint64_t seed,
                            int e_lo, int e_hi);
/* x ~ N(0,1) (Box-Muller over the same hash), float32. */
void bfp8_synth_normal(float* out, int n, uint64_t seed);
/* silu(a)*b with a, b ~ N(0,1), then a fraction of positions set to +-mag. */
void bfp8_synth_swiglu(float* out, int n, uint64_t seed, double outlier_frac, float mag);

/* Bandwidth probes for the roofline: a read-only sweep of `bytes` (2 KiB runs
 * per wavefront, interleaved, one in flight: the fastest read pattern measured)
 * and a device-to-device copy (used to calibrate hardware byte counters). */
int bfp8_dev_read_probe(const void* buf, size_t bytes, uint32_t* out, void* stream);
int bfp8_dev_copy_probe(void* dst, const void* src, size_t bytes, void* stream);

/* The library's HIP stream (hipStream_t as void*). */
void* bfp8_stream(void);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* QWEN_KERNELS_H */
