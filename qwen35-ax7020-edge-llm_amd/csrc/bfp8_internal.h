// bfp8_internal.h -- kernel descriptors and launchers shared by the two kernel
// translation units and the C-ABI host code.  Not part of the public ABI.
//
//   bfp8_ftz.hip   kernels whose float arithmetic restates the reference's
//                  Advanced SIMD code: compiled with f32 flush-to-zero, no
//                  contraction (GEMV, grouped GEMV + fused lm_head top-k,
//                  batched GEMV).
//   bfp8_ieee.hip  kernels whose float arithmetic restates the reference's
//                  scalar VFP code: IEEE subnormals, no contraction
//                  (activation quantizer, odd-M last row, K > 4096 float
//                  path), plus integer-only kernels (layout conversion,
//                  synthetic planes, bandwidth probes).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bfp8_layout.h"

// One GEMV of a grouped launch (or the only one of a single launch).
struct Bfp8GemvDesc {
    const uint8_t* mant;     // GPU mantissa plane (bfp8_layout.h)
    const uint8_t* exps;     // GPU exponent plane
    const uint32_t* xsplit;  // split activation, NB*32 words
    const float* xscale;     // NB per-block activation scales
    float* y;                // M outputs (rows < pair_rows are written), may be null
    int32_t* lanes;          // optional [M][NB][4] residue-lane sums (debug), may be null
    int M, K;
    int pair_rows;           // rows computed with the paired (NEON) epilogue: M & ~1
    int topk;                // 0: plain GEMV; 1..64: fused lm_head top-k over the rows
    uint64_t* partials;      // [ntiles][topk] per-tile sorted keys (topk > 0)
    int* out_ids;            // [topk]
    float* out_scores;       // [topk]
    int* out_count;          // number of valid entries
    int* out_argmax;         // lm_head_argmax-rule winner
};

// One activation vector to quantize.
struct Bfp8QuantDesc {
    const float* x;
    int16_t* xq;       // K (may be null)
    float* xscale;     // K/64
    uint32_t* xsplit;  // K/64 * 32 words
    int K;
    int pad_;
};

// The bf16 tied-embedding lm_head (bf16_head.hip).
struct Bf16HeadDesc {
    const uint16_t* table;  // [vocab][hidden] bf16 (high halves of floats)
    const float* h;         // [hidden]
    float* logits;          // optional [vocab] scores, may be null
    uint64_t* partials;     // [ntiles][topk] per-tile sorted keys (topk > 0)
    int vocab, hidden;
    int topk;               // 0: scores only
    int tail;               // 1: add the hidden % 8 trailing elements (lm_head_topk)
    int tiled;              // 1: table in the 64-row tile layout (bf16_launch_tile_table)
};

// The sampler over a candidate list (select.hip).
struct Bfp8SampleArgs {
    const int* ids;
    const float* scores;
    const int* count;       // device candidate count (clamped to [0, n]), or null to use n
    int n;                  // capacity of ids / scores / work
    float temperature;
    int top_k;
    float top_p;
    uint32_t* rng;          // xorshift32 state, updated in place (null: ids[0])
    int* out;               // chosen id
    void* work;             // 8 * n bytes of scratch
};

// Grouped-launch work item: which descriptor and which row tile.
struct Bfp8TileRef {
    int desc;
    int tile;
};

#define BFP8_TOPK_MAX 64
#define BFP8_TOPK_MAX_TILES 4096
#define BFP8_SELECT_MAX (1 << 28)  // entries the sort-based selection and the sampler take
#define BFP8_SELECT_BLOCK 2048       // keys per LDS-sorted block of the selection
#define BFP8_SELECT_RANK_MAX (1 << 20)  // entries the block-sort + rank selection takes
// Scratch of bfp8_launch_select_sort: the n keys, then a count per block.
constexpr size_t bfp8_select_scratch_bytes(long long n) {
    return ((size_t)n * 8 + (size_t)((n + BFP8_SELECT_BLOCK - 1) / BFP8_SELECT_BLOCK) * 4 + 255) & ~(size_t)255;
}
#define BF16_HEAD_MAX_HIDDEN 4096  // hidden size of the bf16 lm_head (LDS copy of h)
#define BFP8_STREAM_WG_PER_CU 4
// Row tiles up to which a GEMV (or a plan's GEMVs) runs one tile per
// 16-wavefront workgroup instead of the persistent streaming kernel.
#ifndef BFP8_WIDE_MAX_TILES
#define BFP8_WIDE_MAX_TILES 384
#endif

// ---- bfp8_ftz.hip --------------------------------------------------------
// Single GEMV: up to BFP8_WIDE_MAX_TILES row tiles 16 rows per workgroup
// (fused_gemv.hip; one tile per 16-wavefront workgroup when per-lane sums are
// asked for), else the persistent streaming kernel (for topk > 0 always, then
// followed by the stand-alone merge kernel).
hipError_t bfp8_launch_gemv(const Bfp8GemvDesc& d, hipStream_t s);
// One tile per 16-wavefront workgroup over a tile table (small plans);
// max_nb = the largest K/64 among the table's GEMVs.
hipError_t bfp8_launch_gemv_wide_grouped(const Bfp8GemvDesc* descs_dev, const Bfp8TileRef* tiles_dev, int ntiles,
                                         int max_nb, hipStream_t s);
// Stand-alone final top-k merge of partials an earlier launch wrote.
hipError_t bfp8_launch_topk_merge(const Bfp8GemvDesc& d, hipStream_t s);
// Name of the stand-alone merge kernel bfp8_launch_topk_merge runs for an M-row lm_head.
const char* bfp8_topk_merge_kernel_name(int M);
// Persistent grouped launch: workgroup w walks tiles_dev[wg_off_dev[w] ..
// wg_off_dev[w+1]); nwg <= bfp8_stream_grid().  merge_desc >= 0: workgroup 0
// first merges the top-k partials of descs_dev[merge_desc] (written by an
// earlier launch on the stream).
hipError_t bfp8_launch_gemv_grouped(const Bfp8GemvDesc* descs_dev, const Bfp8TileRef* tiles_dev,
                                    const int* wg_off_dev, int nwg, int merge_desc, hipStream_t s);
// The lm_head's persistent launch with the plan's quantization folded in:
// every workgroup quantizes the lm_head activation hx (K <= 64 *
// BFP8_HEAD_MAX_NB, K % 64 == 0) itself, and wavefront task j quantizes block
// qtasks[2j+1] of qdescs_dev[qtasks[2j]] into that descriptor's records.
#define BFP8_HEAD_MAX_NB 16
// The fused lm_head launch: everything its weight loads need is an argument
// (no table lookups ahead of them); workgroup w takes tiles w, w + nwg, ...
// One 64-element block of another activation, quantized by one wavefront of
// the lm_head launch: everything the wavefront needs in one record, so that
// it is read with the lm_head activation, before any weight load.
struct Bfp8HeadTask {
    const float* x;    // the block's 64 floats
    int16_t* xq;       // the activation's outputs (bfp8_quantize's), block b of each
    float* xscale;
    uint32_t* xsplit;
    int b;
    int pad_[3];
};
struct Bfp8HeadArgs {
    const Bfp8GemvDesc* descs;    // descs[head]: the outputs (y, partials, topk, pair_rows)
    int head;
    const uint8_t* mant;          // the lm_head's device planes and width
    const uint8_t* exps;
    int K, ntiles;
    const float* hx;              // the lm_head's activation
    const Bfp8HeadTask* qtasks;   // the other activations' blocks; at least one entry even when ntasks == 0
    int ntasks;
};
hipError_t bfp8_launch_gemv_head(const Bfp8HeadArgs& a, int nwg, hipStream_t s);
// Extra load, in blocks of the byte-balanced dealing, that a folded merge
// puts on workgroup 0 of a grouped launch (the threshold selection of the
// 24-layer sweep's 1024 lm_head lists, ~7 us in one workgroup, about 11 blocks
// at a workgroup's streaming rate; the layer launch measured the same with 8,
// 16 and 32).
#define BFP8_MERGE_COST_BLOCKS 16
// Number of workgroups the persistent GEMV kernels keep resident.
int bfp8_stream_grid();
// hipSuccess when this library's gfx950 code object loads on the current
// device (an attribute query of one of its kernels).
hipError_t bfp8_probe_code_object();

// ---- sweep.hip: a whole plan in one persistent launch -----------------------
// One GEMV of the launch's queue: its row tiles are queue units first ..
// first + ntiles - 1 (the table is ordered by first unit).  48 bytes.
struct Bfp8SweepGemv {
    const uint8_t* mant;  // GPU planes
    const uint8_t* exps;
    const float* x;       // activation, nb * 64 floats
    float* y;             // outputs, rows < pair_rows written
    int nb, pair_rows;
    int first, ntiles;
};
struct Bfp8SweepArgs {
    const Bfp8SweepGemv* gemvs;
    int ngemv, nunits;
    int ticket0;           // the queue unit the first ticket of sub-queue 0 stands for
    int nqueues;           // sub-queues (1, or up to BFP8_SWEEP_QUEUES with 8 nqueues <= the grid): sub-queue
                           // s holds units ticket0 + s + nqueues t, taken by workgroups (w / 8) mod nqueues = s
    uint32_t* counters;    // this launch's BFP8_SWEEP_QUEUES tickets-taken counters (BFP8_SWEEP_CTR_STRIDE
                           // words apart), zero when it starts
    uint32_t* counters_next;  // the other set (the previous launch's): zeroed by this launch for the next
    // the lm_head (head_ntiles > 0): workgroup w < grid - 1 takes its tiles w, w + grid - 1, ...
    // first; the last workgroup merges their top-k lists
    const uint8_t* head_mant;
    const uint8_t* head_exps;
    const float* head_x;
    int head_nb, head_ntiles, head_pair_rows, topk;
    uint64_t* partials;    // [head_ntiles][topk] epoch keys
    int* out_ids;
    float* out_scores;
    int* out_count;
    int* out_argmax;
    uint32_t epoch;        // 1 .. 2^14 - 1, different from the previous launch's
};
#define BFP8_SWEEP_MAX_GEMV 128
// Workgroups per CU of the single launch (5 wavefronts each) with queue
// units; a lone lm_head takes one tile per workgroup (up to what is resident).
#define BFP8_SWEEP_WG_PER_CU 3
#define BFP8_SWEEP_QUEUES 64
#define BFP8_SWEEP_CTR_STRIDE 1024  // words (4 KiB apart: counters in different memory channels)
// Two counter sets: launches of a plan take them in turn.
#define BFP8_SWEEP_CTR_BYTES (2 * BFP8_SWEEP_QUEUES * BFP8_SWEEP_CTR_STRIDE * 4)
// Units of a sweep launch have an even number of 4-block chunks (nb % 8 == 0,
// 8 <= nb <= 64): their chunks alternate between two register buffers.
#define BFP8_SWEEP_MIN_NB 8
// Resident workgroups of the single launch with at most per_cu per CU (every
// workgroup of a launch must be resident: the merging one waits for the
// others' lists).
int bfp8_sweep_grid(int per_cu);
hipError_t bfp8_launch_sweep(const Bfp8SweepArgs& a, int nwg, hipStream_t s);
// Y[v][M] for v < B (1..16): B split activations (rows of nb*32 words) and
// scales (rows of nb floats); pair rows only (the odd last row is the tail
// kernel's).  8..16 vectors run on the matrix cores (batch_mfma.hip), fewer
// on the dot-product kernel, in power-of-two steps.
hipError_t bfp8_launch_gemv_batch(float* Y, const uint32_t* xsplit, const float* xscale,
                                  const uint8_t* mant, const uint8_t* exps, int M, int K, int B,
                                  hipStream_t s);

// ---- batch_mfma.hip -------------------------------------------------------
hipError_t bfp8_launch_gemv_batch_mfma(float* Y, const uint32_t* xsplit, const float* xscale, const uint8_t* mant,
                                       const uint8_t* exps, int M, int K, int B, hipStream_t s);

// ---- bf16_head.hip --------------------------------------------------------
hipError_t bf16_launch_lm_head(const Bf16HeadDesc& d, hipStream_t s);
// The lm_head's tile layout of a bf16 table [vocab][hidden] (bf16_tiled_ok:
// the model's hidden 1024): rows in groups of 16, nT = 4 * ceil(vocab / 64)
// groups (rows past vocab zero); element e = 8c + j of row 16T + r, with
// c = 4q + cc, q = 2p + s and j = 4 hi + g, at uint16 offset
// (((p * nT + T) * 2 + s) * 64 + 4r + g) * 8 + 2 cc + hi.
bool bf16_tiled_ok(int hidden);
size_t bf16_tiled_elems(int vocab, int hidden);
hipError_t bf16_launch_tile_table(uint16_t* dst, const uint16_t* src, int vocab, int hidden, hipStream_t s);

// ---- noalloc.hip ---------------------------------------------------------
// The fixed device scratch of bfp8_dev_lm_head_topk_noalloc: vocabularies up
// to BFP8_NOALLOC_MAX_VOCAB rows.
#define BFP8_NOALLOC_MAX_VOCAB 262144
#define BFP8_NOALLOC_PARTIALS_BYTES ((size_t)(BFP8_NOALLOC_MAX_VOCAB / 64) * BFP8_TOPK_MAX * 8)
#define BFP8_NOALLOC_LOGITS_BYTES ((size_t)BFP8_NOALLOC_MAX_VOCAB * 4)
#define BFP8_NOALLOC_KEYS_BYTES bfp8_select_scratch_bytes(BFP8_NOALLOC_MAX_VOCAB)
// Device address of the scratch on the current device (looked up once per
// device with hipGetSymbolAddress, then cached).
hipError_t bfp8_noalloc_setup(void** out);

// ---- select.hip ----------------------------------------------------------
// Per-tile top-`topk` partials ([ntiles(n)][topk] keys) of logits[0, n), for
// bfp8_launch_topk_merge (topk <= BFP8_TOPK_MAX).
hipError_t bfp8_launch_select_partials(const float* logits, int n, int topk, uint64_t* partials, hipStream_t s);
// The kk best of logits[0, n) (kk > BFP8_TOPK_MAX): 4096-key blocks sorted
// in LDS, then ranked (n <= BFP8_SELECT_RANK_MAX), else all n keys sorted by
// one workgroup; keys: bfp8_select_scratch_bytes(n) of scratch.  ids /
// scores [kk], count, argmax as the merge writes them.
hipError_t bfp8_launch_select_sort(const float* logits, int n, int kk, uint64_t* keys, int* ids, float* scores,
                                   int* count, int* argmax, hipStream_t s);
hipError_t bfp8_launch_sample(const Bfp8SampleArgs& a, hipStream_t s);

// ---- bfp8_ieee.hip -------------------------------------------------------
hipError_t bfp8_launch_quantize(const Bfp8QuantDesc* descs_dev, int ndesc, int max_nb, hipStream_t s);
hipError_t bfp8_launch_quantize1(const Bfp8QuantDesc& d, hipStream_t s);
hipError_t bfp8_launch_tail_row(float* y, const uint32_t* xsplit, const float* xscale,
                                const uint8_t* mant, const uint8_t* exps, int M, int K, hipStream_t s);
hipError_t bfp8_launch_gemv_float(float* y, const float* x, const uint8_t* mant, const uint8_t* exps,
                                  int M, int K, hipStream_t s);
// The engine's numpy fallback (04/qwen_real_engine.py:1230-1238): unquantized
// x, float32 products, numpy's summation order (pairwise: numpy >= 1.9;
// else sequential: numpy 1.8.2).  K % 64 == 0.
hipError_t bfp8_launch_gemv_fallback(float* y, const float* x, const uint8_t* mant, const uint8_t* exps, int M,
                                     int K, int pairwise, hipStream_t s);
hipError_t bfp8_launch_pack(uint8_t* mant_gpu, uint8_t* exps_gpu, const int8_t* mant_soa,
                            const uint8_t* exps_soa, int M, int K, hipStream_t s);
// Row r's mantissas at mant_src + r*mant_stride, its exponents at
// exps_src + r*exps_stride (SoA planes: K and K/64; the per-row stream of
// exponents-then-mantissas: K/64 + K for both).
hipError_t bfp8_launch_pack_strided(uint8_t* mant_gpu, uint8_t* exps_gpu, const int8_t* mant_src, size_t mant_stride,
                                    const uint8_t* exps_src, size_t exps_stride, int M, int K, hipStream_t s);
hipError_t bfp8_launch_unpack(int8_t* mant_soa, uint8_t* exps_soa, const uint8_t* mant_gpu,
                              const uint8_t* exps_gpu, int M, int K, hipStream_t s);
hipError_t bfp8_launch_synth_planes(int8_t* mant_soa, uint8_t* exps_soa, int M, int K, uint64_t seed,
                                    int e_lo, int e_hi, hipStream_t s);
hipError_t bfp8_launch_read_probe(const void* buf, size_t bytes, uint32_t* out, hipStream_t s);
hipError_t bfp8_launch_copy_probe(void* dst, const void* src, size_t bytes, hipStream_t s);

// ---- synthetic inputs (shared host/device integer hash) -------------------
// splitmix64 finaliser over (seed, index): the same integers on host and GPU.
BFP8_HD static inline uint64_t bfp8_hash64(uint64_t seed, uint64_t idx) {
    uint64_t z = seed + (idx + 1u) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
// Mantissa of element i: uniform in [-127, 127].
BFP8_HD static inline int8_t bfp8_synth_mant(uint64_t seed, uint64_t i) {
    return (int8_t)((int)((bfp8_hash64(seed, i) >> 32) % 255u) - 127);
}
// Exponent of block i: uniform in [lo, hi].
BFP8_HD static inline uint8_t bfp8_synth_exp(uint64_t seed, uint64_t i, int lo, int hi) {
    uint64_t h = bfp8_hash64(seed ^ 0xE7E7E7E7E7E7E7E7ull, i);
    return (uint8_t)(lo + (int)((h >> 32) % (uint64_t)(hi - lo + 1)));
}
