// runtime_internal.h -- descriptors and launchers of the decode-runtime
// kernels (runtime_ftz.hip) shared with the C-ABI host code.  Not part of the
// public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// rmsnorm (04/qwen_kernels_opt.c:140-175), optionally preceded by
// add_residual into h (:386-393) and followed by the activation quantizer of
// the next GEMV (:182-205).
struct RtNormArgs {
    float* h;             // x; with res, h = h + res is written back first
    const float* res;     // residual, or null
    const float* w;       // norm weight (applied as 1 + w)
    float* y;             // normalised output, or null
    float* xscale;        // non-null: quantize y (n / 64 blocks) ...
    uint32_t* xsplit;     // ... into these GEMV activation records
    int n;
    float eps;
};

// swiglu (:363-384), optionally followed by the quantizer (n % 64 == 0).
struct RtSwigluArgs {
    float* y;
    const float* gate;
    const float* up;
    float* xscale;
    uint32_t* xsplit;
    int n;
};

// causal_conv1d_update_silu (:511-542).
struct RtConvArgs {
    float* y;
    const float* x;
    float* state;  // [3][channels], oldest tap first
    const float* w;  // [channels][4]
    int channels;
};

// gdn_gates (:593-620).
struct RtGatesArgs {
    float* alpha;
    float* beta;
    const float* x;
    const float* wa;
    const float* wb;
    const float* nea;
    const float* dt;
    int H, K;
};

// gdn_recurrent_step (:659-813); the state uses the reference's blocked
// layout state[h][((jg*ng + ig)*4 + l)*4 + t] = S[h][4ig+t][4jg+l].
struct RtGdnArgs {
    float* out;
    float* state;
    const float* q;
    const float* k;
    const float* v;
    const float* alpha;
    const float* beta;
    int H, D;
};

// rmsnorm_gated (:818-847), optionally followed by the quantizer of its
// output (D % 64 == 0).
struct RtGatedArgs {
    float* y;
    const float* x;
    const float* z;
    const float* w;
    float* xscale;
    uint32_t* xsplit;
    int H, D;
    float eps;
};

// The model's linear-attention block between the qkv/z GEMVs and the o GEMV
// (04/qwen_kernels_opt.c:943-967, steps 3-6) for 16 heads of 128: conv1d +
// SiLU over the head's q/k/v channels, q/k L2 norm, gates and the recurrent
// step; RT_ATTN_SPLIT workgroups per head, each owning 128 / RT_ATTN_SPLIT
// state columns (and computing the head's conv, norms and gates itself).
// The conv taps are read from conv_in and the shifted taps written to
// conv_out (a different buffer: every workgroup of a head reads the taps).
// The gated RMSNorm that follows is the o GEMV's prologue (RT_ROWS_GATED);
// each workgroup writes silu(z) of its columns for it.
#define RT_HEADS 16
#define RT_HEAD_DIM 128
#define RT_CONV_CH 6144
#define RT_HIDDEN 1024
#define RT_ATTN_SPLIT 4
struct RtLinearAttnArgs {
    const float* qkv;      // [6144] qkv GEMV output
    const float* normed;   // [1024] input-norm output (gate input)
    const float* conv_in;  // [3][6144] taps, oldest first
    float* conv_out;       // [3][6144] shifted taps
    const float* conv_w;   // [6144][4]
    const float* wa;       // [16][1024]
    const float* wb;       // [16][1024]
    const float* nea;      // [16]
    const float* dt;       // [16]
    float* state;          // [16][128*128], blocked
    float* attn;           // [2048] recurrent-step output
    const float* z;        // [2048] z GEMV output ...
    float* zsilu;          // ... and silu(z), for the gated norm
    float* mixed;          // optional [6144]: q, k after L2 norm, v
    float* alpha_beta;     // optional [32]: alpha[16], beta[16]
};

// The forward's GEMVs (fused_gemv.hip): one or two GEMVs sharing one
// activation, 16 rows per workgroup; the activation is given quantized or is
// computed by every workgroup from its inputs.
#define RT_ROWS_QUANTIZED 0  // xsplit / xscale given
#define RT_ROWS_NORM 1       // rmsnorm(h + res) with weight w, eps
#define RT_ROWS_SWIGLU 2     // swiglu(gate, up)
#define RT_ROWS_GATED 3      // rmsnorm_gated(attn, z) over 16 heads of 128 with weight w, eps (silu(z) given)
#define RT_ROWS_FLOAT 4      // x given as floats, quantized here (K / 64 whole blocks)
#define RT_ROWS_MAX_K 4096
struct RtRowsGemv {
    const uint8_t* mant;  // GPU planes (bfp8_layout.h)
    const uint8_t* exps;
    float* y;
    int M;
    int pair_rows;        // rows written: M & ~1 (an odd last row takes the tail kernel)
};
struct RtRowsArgs {
    RtRowsGemv g[2];
    int ngemv;            // 1 or 2
    int split;            // workgroups of g[0]: ceil(g[0].M / 16)
    int K;
    int mode;
    const uint32_t* xsplit;  // RT_ROWS_QUANTIZED
    const float* xscale;
    const float* h;          // RT_ROWS_NORM: x = h (+ res)
    const float* res;
    const float* w;
    float eps;
    float* h_out;            // optional: workgroup 0 writes x (must not alias h)
    float* y_norm;           // optional: workgroup 0 writes the normalised vector
    const float* gate;       // RT_ROWS_SWIGLU
    const float* up;
    const float* attn;       // RT_ROWS_GATED (with w, eps)
    const float* zsilu;      // silu(z), elementwise
    const float* x;          // RT_ROWS_FLOAT
    uint32_t* xsplit_out;    // optional (RT_ROWS_FLOAT): workgroup 0 also writes the
    float* xscale_out;       // activation's records here, for a later tail-row launch
};
hipError_t rt_launch_rows(const RtRowsArgs& a, hipStream_t s);

hipError_t rt_launch_rmsnorm(const RtNormArgs& a, hipStream_t s);
hipError_t rt_launch_swiglu(const RtSwigluArgs& a, hipStream_t s);
hipError_t rt_launch_conv1d(const RtConvArgs& a, hipStream_t s);
hipError_t rt_launch_qk_l2norm(float* q, float* k, int H, int D, hipStream_t s);
hipError_t rt_launch_gates(const RtGatesArgs& a, hipStream_t s);
hipError_t rt_launch_gdn_step(const RtGdnArgs& a, hipStream_t s);
hipError_t rt_launch_gated(const RtGatedArgs& a, hipStream_t s);
hipError_t rt_launch_add_residual(float* x, const float* res, int n, hipStream_t s);
hipError_t rt_launch_linear_attn(const RtLinearAttnArgs& a, hipStream_t s);
// h[i] = the float whose high half is table[row*hidden + i]
// ntiles > 0: the table is in the 64-row tile layout over ntiles tiles
// (bf16_launch_tile_table); 0: row-major.
hipError_t rt_launch_embed(float* h, const uint16_t* table, int ntiles, int row, int hidden, hipStream_t s);

// Largest head_dim / gate input the per-head kernels stage in LDS.
#define RT_MAX_HEAD_DIM 4096
