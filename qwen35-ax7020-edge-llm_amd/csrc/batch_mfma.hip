// batch_mfma.hip -- the batched BFP8 GEMV (8..16 activation vectors against
// one weight matrix, weights read once) on the matrix cores, f32 flush-to-zero
// like the reference's Advanced SIMD epilogue.
//
// The reference has no batched GEMV: a batch is B calls of bfp8_gemv
// (04/qwen_kernels_opt.c:207-278), each keeping four int32 residue lanes per
// row and block (elements k = q mod 4), S_q = sum of mantissa * xq, and a
// float epilogue per block  fs_q += (float(S_q) * 2^(e-134)) * xscale,
// y = (fs_0 + fs_2) + (fs_1 + fs_3).
//
// Integer part on v_mfma_i32_32x32x16_i8, whose K of 16 is exactly the 16
// elements of one residue of one block.  With xq = 256*xh + xl (xh, xl int8,
// bfp8_layout.h) one MFMA computes, for 32 weight rows and residue q,
//   D[(v, p)][row] = sum over the residue's 16 elements of x_p[v] * m[row]
// for the 16 vectors v and both parts p (h, l) as its 32 rows: the A operand
// is the batch's split activations, the B operand the weight plane's
// residue-q slice.  A lane of D holds column `row` and rows 8(i/4) + 4(l/32)
// + i%4 (i < 16), so its registers i and i + 8 are the h and l sums of the same
// vector: S_q = 256 * D[i] + D[i + 8] exactly, in the lane, for 8 vectors.
// Integer sums are exact in any order.
//
// Float part, per (row, vector, block, residue), in the reference's order:
// float(S_q) * es * xs with es = 2^(e-134) a power of two.  float(S_q) * es is
// exact whenever it is a normal float (e in 8..236: |S_q| <= 2^25), so the two
// products round once, on S_q * es * xs.  When c = es * xs is itself a normal
// float it is exact too, and float(S_q) * c rounds the same real number: one
// product instead of two.  Each block checks that c is normal for every
// vector of the batch (a range of e computed from the batch's block scales)
// and takes the two products otherwise; e < 8 (es = 0) and zero, infinite or
// NaN scales give the same result either way.
//
// Work split: wavefront (s, g) takes a 64-row tile's 32-row half s and the
// residues of group g (kRes residues per wavefront), keeping fs_q of its
// residues; the wavefronts of a half combine their fs_q into y at the end
// through LDS.  GEMVs with many tiles and K <= 1024: a workgroup per four
// tiles, all 4 residues per wavefront (bfp8_gemv_batch_cu_kernel); with
// larger K, a workgroup per tile, 2 residues per wavefront.  GEMVs with few
// tiles: a workgroup per half, 1 residue per wavefront, every weight load of
// a chunk in flight at once, and (more than 8 vectors) a workgroup per half
// of the vectors too, so that more wavefronts, each with a shorter epilogue
// chain, run on more CUs; with K <= 1024 each residue's blocks are split
// over four wavefronts besides (bfp8_gemv_batch_split_kernel).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bfp8_internal.h"
#include "bfp8_layout.h"
#include "gemv_dev.h"

namespace {

typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kMfVec = 16;   // vectors (the MFMA's rows are vector x part)
constexpr int kMfGroup = 2;  // blocks per weight-load group

// CH: blocks of split activations staged in LDS at a time (16: the whole K of
// the configured shapes in one staging; 8: half the LDS and the staging
// registers, for the kernel whose occupancy they limit).
template <int CH>
struct MfLds {
    // A operands: [block][residue][k half][part][vector], 8 bytes each: the
    // 64 lanes of one (block, residue) read 512 contiguous bytes
    uint64_t xa[CH][4][64];
    float xs[CH][kMfVec];      // [block][vector] block scales
    int lo[CH], hi[CH];        // per block: e range of the one-product epilogue
    // the end's exchange: 3 residue groups x 2 halves x 8 values x 64 lanes at most
    static_assert(CH * 4 * 64 * sizeof(uint64_t) >= 3 * 2 * 8 * 64 * sizeof(float),
                  "the fs exchange fits in the staging area");
};

// Staging of blocks c0 .. c0+nbc-1 of the B split activations and scales
// (vectors >= B and blocks >= nbc as zeros) into LDS, with each block's
// exponent range [lo, hi] inside which es * xs is a normal float for every
// normal scale xs of the batch: biased exponent of es * xs = e - 134 + E(xs),
// normal for 1..254, and e <= 236 keeps float(S) * es finite.  In two halves
// so that a caller can issue other loads between them: mf_stage_load issues
// every load of the NT threads (one round trip to L2 for all of them),
// mf_stage_store waits for them, writes LDS and synchronizes the workgroup.
template <int NT, int CH>
struct MfStaged {
    static constexpr int kItems = CH * 4 * 2 * kMfVec;  // 16-byte pieces of split activations
    static constexpr int kScales = CH * kMfVec;
    static_assert(kItems % NT == 0, "whole staging rounds");
    static constexpr int kScaleRounds = (kScales + NT - 1) / NT;
    u32x4 val[kItems / NT];
    float xs[kScaleRounds];
};

// 16 bytes of xsplit = one part of one residue (both k halves): item
// ((u * 4 + q) * 2 + p) * 16 + v, vectors fastest, so the LDS stores of
// consecutive threads are consecutive
// kVH: -1 every vector, else only vectors 8 kVH .. 8 kVH + 7 (the others
// staged as zeros: their MFMA rows are computed and not used).
template <int NT, int kVH, int CH>
__device__ __forceinline__ void mf_stage_load(MfStaged<NT, CH>& S, const uint32_t* __restrict__ xsplit,
                                              const float* __restrict__ xscale, int nb, int B, int c0, int nbc) {
#pragma unroll
    for (int j = 0; j < MfStaged<NT, CH>::kItems / NT; ++j) {
        const int i = threadIdx.x + j * NT;
        const int v = i % kMfVec, p = (i / kMfVec) % 2, q = (i / (2 * kMfVec)) % 4, u = i / (8 * kMfVec);
        S.val[j] = u32x4{0u, 0u, 0u, 0u};
        if (v < B && (kVH < 0 || (v >> 3) == kVH) && u < nbc)
            S.val[j] = *reinterpret_cast<const u32x4*>(
                xsplit + ((size_t)v * nb + c0 + u) * BFP8_XSPLIT_WORDS_PER_BLOCK + q * 8 + p * 4);
    }
#pragma unroll
    for (int j = 0; j < MfStaged<NT, CH>::kScaleRounds; ++j) {
        const int i = threadIdx.x + j * NT, v = i % kMfVec, u = i / kMfVec;
        S.xs[j] = (i < MfStaged<NT, CH>::kScales && v < B && (kVH < 0 || (v >> 3) == kVH) && u < nbc) ? xscale[(size_t)v * nb + c0 + u]
                                                                                        : 0.0f;
    }
}

template <int NT, int CH, bool kSync = true>
__device__ __forceinline__ void mf_stage_store(MfLds<CH>& L, const MfStaged<NT, CH>& S) {
#pragma unroll
    for (int j = 0; j < MfStaged<NT, CH>::kItems / NT; ++j) {
        const int i = threadIdx.x + j * NT;
        const int v = i % kMfVec, p = (i / kMfVec) % 2, q = (i / (2 * kMfVec)) % 4, u = i / (8 * kMfVec);
        L.xa[u][q][p * 16 + v] = ((uint64_t)S.val[j].y << 32) | S.val[j].x;       // k half 0: bytes 0..7
        L.xa[u][q][32 + p * 16 + v] = ((uint64_t)S.val[j].w << 32) | S.val[j].z;  // k half 1: bytes 8..15
    }
#pragma unroll
    for (int j = 0; j < MfStaged<NT, CH>::kScaleRounds; ++j) {
        const int i = threadIdx.x + j * NT;
        if (i < MfStaged<NT, CH>::kScales) {  // whole wavefronts (a multiple of 64)
            const int v = i % kMfVec, u = i / kMfVec;
            const float xs = S.xs[j];
            L.xs[u][v] = xs;
            const int E = (int)((__float_as_uint(xs) >> 23) & 0xffu);
            const bool normal = E >= 1 && E <= 254;
            int emin = normal ? E : 255, emax = normal ? E : 0;
#pragma unroll
            for (int m = 1; m < kMfVec; m <<= 1) {  // over the 16 lanes of block u
                emin = min(emin, __shfl_xor(emin, m, 64));
                emax = max(emax, __shfl_xor(emax, m, 64));
            }
            if (v == 0) {
                L.lo[u] = 135 - emin;
                L.hi[u] = min(236, 388 - emax);
            }
        }
    }
    if (kSync) __syncthreads();
}

// A lane's result slots: register i of the MFMA result (and i + 8, the low
// parts) is vector 8(i/4) + 4*kh + i%4 of the lane's row; every vector: slots
// i = 0..7; vector half kVH: slots i = 4 kVH .. 4 kVH + 3.
template <int kVH>
struct MfSlots {
    static constexpr int n = kVH < 0 ? 8 : 4;
    static constexpr int i0 = kVH < 0 ? 0 : 4 * kVH;
};

template <int kRes, int kVH>
struct MfState {
    float fs[kRes][MfSlots<kVH>::n];  // [residue of the group][slot]
};

template <int kRes>
struct MfLoads {
    uint64_t w[kMfGroup][kRes];  // [block][residue of the group]
    uint32_t e;
};

// One block: an MFMA per residue of the group and the epilogue.
template <int kRes, int kVH, int CH>
__device__ __forceinline__ void mf_block(MfState<kRes, kVH>& st, const MfLds<CH>& L, const uint64_t (&w)[kRes], uint32_t e,
                                         int u, int q0, int lane) {
    constexpr int NS = MfSlots<kVH>::n, I0 = MfSlots<kVH>::i0;
    i32x16 d[kRes];
    const i32x16 zero = {};
#pragma unroll
    for (int r = 0; r < kRes; ++r)
        d[r] = __builtin_amdgcn_mfma_i32_32x32x16_i8((long)L.xa[u][q0 + r][lane], (long)w[r], zero, 0, 0, 0);
    const int kh = lane >> 5;
    float xs[NS];
#pragma unroll
    for (int h = 0; h < NS / 4; ++h) {  // slots 4h..4h+3: vectors 8 (I0 / 4 + h) + 4 kh ..
        const f32x4 x4 = *reinterpret_cast<const f32x4*>(&L.xs[u][8 * (I0 / 4 + h) + 4 * kh]);
#pragma unroll
        for (int m = 0; m < 4; ++m) xs[4 * h + m] = x4[m];
    }
    const float es = exp_scale_ftz(e);
    const int lo = L.lo[u], hi = L.hi[u];
    const bool one_product = (e < 8u) | ((uint32_t)((int)e - lo) <= (uint32_t)(hi - lo));
    if (__builtin_amdgcn_ballot_w64(!one_product) == 0) {
        float c[NS];
#pragma unroll
        for (int k = 0; k < NS; ++k) c[k] = es * xs[k];
#pragma unroll
        for (int r = 0; r < kRes; ++r)
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                const int S = (int)((uint32_t)d[r][I0 + k] << 8) + d[r][I0 + k + 8];
                st.fs[r][k] = st.fs[r][k] + (float)S * c[k];
            }
    } else {
#pragma unroll
        for (int r = 0; r < kRes; ++r)
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                const int S = (int)((uint32_t)d[r][I0 + k] << 8) + d[r][I0 + k + 8];
                const float t1 = (float)S * es;
                st.fs[r][k] = st.fs[r][k] + t1 * xs[k];
            }
    }
}

// Weights of group gi (blocks kMfGroup*gi ..) for the lane's row, k half and
// the group's residues, and the row's exponent dword holding them (4 blocks
// per dword).  The whole offset goes in the per-lane offset, which the buffer
// range check covers: groups past the tile read zeros without touching memory.
static_assert(4 % kMfGroup == 0, "a group's exponents share one dword");
template <int kRes>
__device__ __forceinline__ void mf_issue(MfLoads<kRes>& ld, __amdgpu_buffer_rsrc_t wrs, __amdgpu_buffer_rsrc_t ers, int wv,
                                         int ev, int gi) {
#pragma unroll
    for (int uu = 0; uu < kMfGroup; ++uu)
#pragma unroll
        for (int r = 0; r < kRes; ++r) {
            const u32x2 v = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(wrs, wv + (gi * kMfGroup + uu) * 4096 + r * 1024, 0,
                                                            kNonTemporal));
            ld.w[uu][r] = ((uint64_t)v.y << 32) | v.x;
        }
    ld.e = load_e(ers, ev + (gi * kMfGroup / 4) * 256, 0);
}

template <int kRes, int NT, int kVH, int CH>
__device__ __forceinline__ void mf_group(MfState<kRes, kVH>& st, MfLds<CH>& L, const MfLoads<kRes>& ld, int gi, int nb,
                                         const uint32_t* __restrict__ xsplit, const float* __restrict__ xscale, int B,
                                         int q0, int lane) {
    const int b0 = gi * kMfGroup;
    if (b0 % CH == 0 && b0 > 0) {  // the first chunk is staged before the loop
        __syncthreads();  // every wavefront is done with the previous chunk
        MfStaged<NT, CH> S;
        mf_stage_load<NT, kVH, CH>(S, xsplit, xscale, nb, B, b0, min(CH, nb - b0));
        mf_stage_store<NT, CH>(L, S);
    }
#pragma unroll
    for (int uu = 0; uu < kMfGroup; ++uu) {
        if (b0 + uu >= nb) break;
        mf_block<kRes, kVH, CH>(st, L, ld.w[uu], (ld.e >> (8 * ((b0 + uu) & 3))) & 0xffu, (b0 + uu) % CH, q0, lane);
    }
}

// The work of one workgroup: tile t, its 32-row half s (kHalves == 1) or both
// (kHalves == 2, wavefront w takes half w & 1), the residues of group grp,
// the vectors of kVH (every vector, or one half of them).
// kDepth: weight-load groups in flight per wavefront (2: one group computed
// while the next loads; CH / kMfGroup: a chunk's every weight load issued at
// once, for GEMVs with too few tiles to fill the memory system otherwise).
template <int kRes, int kHalves, int kDepth, int kVH, int CH>
__device__ __forceinline__ void mf_body(MfLds<CH>& L, float* __restrict__ Y, const uint32_t* __restrict__ xsplit,
                                        const float* __restrict__ xscale, const uint8_t* __restrict__ mant,
                                        const uint8_t* __restrict__ exps, int M, int K, int B, int t, int s, int grp) {
    constexpr int NS = MfSlots<kVH>::n, I0 = MfSlots<kVH>::i0;
    const int lane = threadIdx.x & 63;
    const int q0 = grp * kRes;
    const int col = lane & 31, kh = lane >> 5;
    const int nb = K >> 6, nb4 = (nb + 3) >> 2;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(mant + (size_t)t * nb * 4096u, (uint32_t)nb * 4096u);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(exps + (size_t)t * nb4 * 256u, (uint32_t)nb4 * 256u);
    const int wv = q0 * 1024 + (32 * s + col) * 16 + kh * 8;
    const int ev = (32 * s + col) * 4;
    MfState<kRes, kVH> st;
#pragma unroll
    for (int r = 0; r < kRes; ++r)
#pragma unroll
        for (int k = 0; k < NS; ++k) st.fs[r][k] = 0.0f;
    const int ng = (nb + kMfGroup - 1) / kMfGroup;
    // the first chunk's activation loads go out first, then the first
    // weight groups: the staging then waits for its own loads only (a
    // wavefront's loads complete in the order issued)
    constexpr int NT = 64 * kHalves * (4 / kRes);
    MfStaged<NT, CH> S0;
    mf_stage_load<NT, kVH, CH>(S0, xsplit, xscale, nb, B, 0, min(CH, nb));
    MfLoads<kRes> ld[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) mf_issue<kRes>(ld[d], wrs, ers, wv, ev, d);
    mf_stage_store<NT, CH>(L, S0);
    for (int gi = 0; gi < ng; gi += kDepth) {
        // kDepth load sets in turn: set d holds group gi + d, then gi + d + kDepth
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            if (gi + d < ng) mf_group<kRes, NT, kVH, CH>(st, L, ld[d], gi + d, nb, xsplit, xscale, B, q0, lane);
            mf_issue<kRes>(ld[d], wrs, ers, wv, ev, gi + d + kDepth);
        }
    }
    float (&fs)[kRes][NS] = st.fs;

    // y = (fs_0 + fs_2) + (fs_1 + fs_3): the other residue groups of the half
    // hand their sums to group 0 through the (no longer needed) staging area
    __syncthreads();
    float* xch = reinterpret_cast<float*>(&L.xa[0][0][0]);  // [group - 1][half][residue][slot][lane]
    if (grp > 0) {
#pragma unroll
        for (int r = 0; r < kRes; ++r)
#pragma unroll
            for (int k = 0; k < NS; ++k) xch[((((grp - 1) * 2 + s) * kRes + r) * NS + k) * 64 + lane] = fs[r][k];
    }
    __syncthreads();
    if (grp == 0) {
        const int row = t * 64 + 32 * s + col;
        const int pair_rows = M & ~1;
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            float f[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int gq = q / kRes, rq = q % kRes;
                f[q] = gq == 0 ? fs[rq][k] : xch[((((gq - 1) * 2 + s) * kRes + rq) * NS + k) * 64 + lane];
            }
            const int i = I0 + k;
            const int v = 8 * (i / 4) + 4 * kh + (i % 4);
            const float y = (f[0] + f[2]) + (f[1] + f[3]);
            if (v < B && row < pair_rows) Y[(size_t)v * M + row] = y;
        }
    }
}

// ---- many tiles, K <= 1024: a workgroup per CU's four tiles ------------------
// Eight wavefronts, two per SIMD; wavefront w takes tile 4 * blockIdx + w / 2,
// its 32-row half w % 2, and all four residues, so that the per-block work
// (exponent, one-product check, the eight scale products) is shared by 32
// values per lane.  Its weights are 8 VGPRs per block (four residue slices,
// 8 bytes per lane), loaded kAhead blocks ahead.  The batch's split
// activations and scales of every block are staged into LDS once, by the
// eight wavefronts together.  The staging's loads go out first, then the row
// exponents, then the first blocks' weights: a wavefront's vector loads
// complete in issue order, so the L2-resident staging never waits behind the
// HBM round trip, and the weights are in flight during the LDS stores.
// The two wavefronts of a SIMD run different tiles; the one issued first
// would win every issue slot and leave the other to finish alone, so each
// wavefront lowers its priority as it progresses (s_setprio 3 .. 0 over the
// blocks): the one behind is served first.
constexpr int kCuWaves = 8;
constexpr int kCuMaxNb = 16;

struct CuOps {
    uint64_t a[4];  // MFMA A operands (split activations) per residue
    f32x4 x0, x1;   // block scales of the lane's slots 0..3 and 4..7
    int lo, hi;     // the block's one-product exponent range
};

// The epilogue of one block for the four residues (as mf_block's)
__device__ __forceinline__ void cu_epilogue(float (&fs)[4][8], const i32x16 (&d)[4], const CuOps& o, uint32_t e) {
    float xs[8];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        xs[m] = o.x0[m];
        xs[4 + m] = o.x1[m];
    }
    const float es = exp_scale_ftz(e);
    const bool one_product = (e < 8u) | ((uint32_t)((int)e - o.lo) <= (uint32_t)(o.hi - o.lo));
    if (__builtin_amdgcn_ballot_w64(!one_product) == 0) {
        float c[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) c[k] = es * xs[k];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int S = (int)((uint32_t)d[r][k] << 8) + d[r][k + 8];
                fs[r][k] = fs[r][k] + (float)S * c[k];
            }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int S = (int)((uint32_t)d[r][k] << 8) + d[r][k + 8];
                const float t1 = (float)S * es;
                fs[r][k] = fs[r][k] + t1 * xs[k];
            }
    }
}

// s_setprio takes an immediate: level 3 for blocks 0..4, 2 for 5..9, 1 for
// 10..14, 0 after
__device__ __forceinline__ void cu_priority(int u) {
    const int level = u / 5;
    if (level == 0)
        __builtin_amdgcn_s_setprio(3);
    else if (level == 1)
        __builtin_amdgcn_s_setprio(2);
    else if (level == 2)
        __builtin_amdgcn_s_setprio(1);
    else
        __builtin_amdgcn_s_setprio(0);
}

template <int kAhead>
__global__ __launch_bounds__(64 * kCuWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void
bfp8_gemv_batch_cu_kernel(float* __restrict__ Y, const uint32_t* __restrict__ xsplit, const float* __restrict__ xscale,
                          const uint8_t* __restrict__ mant, const uint8_t* __restrict__ exps, int M, int K, int B) {
    static_assert(kAhead >= 1 && kAhead <= kCuMaxNb, "blocks in flight");
    __shared__ MfLds<kCuMaxNb> L;
    constexpr int NT = 64 * kCuWaves;
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, col = lane & 31, kh = lane >> 5;
    const int nb = K >> 6, nb4 = (nb + 3) >> 2;  // nb <= kCuMaxNb (host-checked)
    const int t = (int)blockIdx.x * (kCuWaves / 2) + (w >> 1), s = w & 1;
    const bool live = t < bfp8_ntiles(M);  // the last workgroup may hold fewer tiles
    const int tt = live ? t : 0;
    // the staging's loads first (from L2), then the row's exponents and the
    // weights (from HBM): a wavefront's loads complete in issue order, so the
    // staging then waits for its own round trip only
    MfStaged<NT, kCuMaxNb> S0;
    mf_stage_load<NT, -1, kCuMaxNb>(S0, xsplit, xscale, nb, B, 0, nb);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(exps + (size_t)tt * nb4 * 256u, (uint32_t)nb4 * 256u);
    uint32_t ev[kCuMaxNb / 4];
#pragma unroll
    for (int g = 0; g < kCuMaxNb / 4; ++g) ev[g] = load_e(ers, (32 * s + col) * 4 + g * 256, 0);
    // residue q of block b for the lane's row and k half, through a buffer
    // range starting at the block (the lane offset stays fixed); blocks past
    // the tile, and wavefronts without a tile, have an empty range and read
    // zeros without touching memory
    const int wv = (32 * s + col) * 16 + kh * 8;
    uint64_t wq[kCuMaxNb][4];
    auto issue = [&](int b) {
        const __amdgpu_buffer_rsrc_t rs =
            make_rsrc(mant + ((size_t)tt * nb + b) * 4096u, live && b < nb ? (uint32_t)(nb - b) * 4096u : 0u);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x2 v =
                __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, wv + q * 1024, 0, kNonTemporal));
            wq[b][q] = ((uint64_t)v.y << 32) | v.x;
        }
    };
#pragma unroll
    for (int b = 0; b < kAhead; ++b) issue(b);
    mf_stage_store<NT, kCuMaxNb, false>(L, S0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the staging is in LDS; the weight loads stay in flight
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (!live) return;

    float fs[4][8];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int k = 0; k < 8; ++k) fs[r][k] = 0.0f;
    const i32x16 zero = {};
    // block u's LDS operands are read behind block u - 1's MFMAs
    auto ops = [&](CuOps& o, int u) {
#pragma unroll
        for (int q = 0; q < 4; ++q) o.a[q] = L.xa[u][q][lane];
        o.x0 = *reinterpret_cast<const f32x4*>(&L.xs[u][4 * kh]);
        o.x1 = *reinterpret_cast<const f32x4*>(&L.xs[u][8 + 4 * kh]);
        o.lo = L.lo[u];
        o.hi = L.hi[u];
    };
    CuOps o[2];
    ops(o[0], 0);
#pragma unroll
    for (int u = 0; u < kCuMaxNb; ++u) {
        if (u + kAhead < kCuMaxNb) issue(u + kAhead);
        if (u >= nb) continue;  // (uniform; the loads above read nothing past the tile)
        cu_priority(u);
        i32x16 d[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            d[r] = __builtin_amdgcn_mfma_i32_32x32x16_i8((long)o[u & 1].a[r], (long)wq[u][r], zero, 0, 0, 0);
        if (u + 1 < kCuMaxNb && u + 1 < nb) ops(o[(u + 1) & 1], u + 1);
        __builtin_amdgcn_sched_barrier(0);
        cu_epilogue(fs, d, o[u & 1], (ev[u >> 2] >> (8 * (u & 3))) & 0xffu);
    }

    // non-temporal stores: every wavefront writes its 2 KiB at its end, and
    // these leave the launch's last write burst sooner
    const int row = t * 64 + 32 * s + col;
    const int pair_rows = M & ~1;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int v = 8 * (k / 4) + 4 * kh + (k % 4);
        const float y = (fs[0][k] + fs[2][k]) + (fs[1][k] + fs[3][k]);
        if (v < B && row < pair_rows) __builtin_nontemporal_store(y, Y + (size_t)v * M + row);
    }
}

// The block's terms float(S) * es * xs of the lane's four result slots of
// vector half kVH (one product where es * xs is normal for the batch, as
// mf_block's)
template <int kVH>
__device__ __forceinline__ void half_terms(float (&tv)[4], const i32x16& d, f32x4 x4, int lo, int hi, uint32_t e) {
    constexpr int I0 = 4 * kVH;
    const float es = exp_scale_ftz(e);
    const bool one_product = (e < 8u) | ((uint32_t)((int)e - lo) <= (uint32_t)(hi - lo));
    if (__builtin_amdgcn_ballot_w64(!one_product) == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float c = es * x4[k];
            const int S = (int)((uint32_t)d[I0 + k] << 8) + d[I0 + k + 8];
            tv[k] = (float)S * c;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int S = (int)((uint32_t)d[I0 + k] << 8) + d[I0 + k + 8];
            const float t1 = (float)S * es;
            tv[k] = t1 * x4[k];
        }
    }
}
// ---- few tiles, K <= 1024: a workgroup per 32-row half and half of the vectors,
// the blocks split over four wavefronts per residue ---------------------------
// Few tiles leave about one wavefront per SIMD with a workgroup of four
// (one per residue), so a wavefront's chain of sixteen blocks (LDS read, MFMA,
// epilogue, each waiting for the last) set the time.  Here wavefront (q, j)
// computes residue q's terms float(S) * es * xs of blocks 4j .. 4j + 3 only,
// each block's MFMA issued before the previous block's terms; the terms of
// blocks 4 .. 15 go through LDS to wavefront (q, 0), which adds all sixteen in
// block order (the reference's chain, unchanged).  All blocks run, also past
// nb (K < 1024): their weights, activations and scales read as zeros, so each
// adds an exact +0 to a sum that is never -0.
constexpr int kSplitParts = 4;
struct SplitLds {
    MfLds<kCuMaxNb> a;
    f32x4 t[kSplitParts - 1][4][4][64];     // [group - 1][residue][block of the group][lane]: the 4 slots
    float xch[3][4][64];                     // residues 1..3: [residue - 1][slot][lane]
};

template <int kVH>
__device__ __forceinline__ void split_body(SplitLds& L, float* __restrict__ Y, const uint32_t* __restrict__ xsplit,
                                           const float* __restrict__ xscale, const uint8_t* __restrict__ mant,
                                           const uint8_t* __restrict__ exps, int M, int K, int B, int t, int s, int q,
                                           int j) {
    constexpr int NT = 64 * 4 * kSplitParts;
    const int lane = threadIdx.x & 63, col = lane & 31, kh = lane >> 5;
    const int nb = K >> 6, nb4 = (nb + 3) >> 2;  // nb <= kCuMaxNb (host-checked)
    // the staging of the half's split activations and scales (the workgroup's
    // sixteen wavefronts together), its loads issued before the exponents'
    // and the weights' so that the staging waits for them alone (loads
    // complete in issue order)
    MfStaged<NT, kCuMaxNb> S0;
    mf_stage_load<NT, kVH, kCuMaxNb>(S0, xsplit, xscale, nb, B, 0, nb);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(exps + (size_t)t * nb4 * 256u, (uint32_t)nb4 * 256u);
    const uint32_t ev = load_e(ers, (32 * s + col) * 4 + j * 256, 0);  // blocks 4j .. 4j + 3
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(mant + (size_t)t * nb * 4096u, (uint32_t)nb * 4096u);
    const int wv = q * 1024 + (32 * s + col) * 16 + kh * 8;
    uint64_t wq[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x2 v = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(wrs, wv + (4 * j + i) * 4096, 0, kNonTemporal));
        wq[i] = ((uint64_t)v.y << 32) | v.x;
    }
    mf_stage_store<NT, kCuMaxNb, false>(L.a, S0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the staging is in LDS; the weight loads stay in flight
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    uint64_t a[4];
    f32x4 x4[4];
    int lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = 4 * j + i;
        a[i] = L.a.xa[b][q][lane];
        x4[i] = *reinterpret_cast<const f32x4*>(&L.a.xs[b][8 * kVH + 4 * kh]);
        lo[i] = L.a.lo[b];
        hi[i] = L.a.hi[b];
    }
    const i32x16 zero = {};
    float tv[4][4];
    i32x16 d = __builtin_amdgcn_mfma_i32_32x32x16_i8((long)a[0], (long)wq[0], zero, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        i32x16 dn = zero;
        if (i + 1 < 4) dn = __builtin_amdgcn_mfma_i32_32x32x16_i8((long)a[i + 1], (long)wq[i + 1], zero, 0, 0, 0);
        half_terms<kVH>(tv[i], d, x4[i], lo[i], hi[i], (ev >> (8 * i)) & 0xffu);
        d = dn;
    }
    if (j > 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) L.t[j - 1][q][i][lane] = f32x4{tv[i][0], tv[i][1], tv[i][2], tv[i][3]};
    }
    __syncthreads();
    float fs[4];
    if (j == 0) {
        f32x4 tg[kSplitParts - 1][4];  // every read out first, then the chain
#pragma unroll
        for (int g = 0; g < kSplitParts - 1; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) tg[g][i] = L.t[g][q][i][lane];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float f = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) f = f + tv[i][k];
#pragma unroll
            for (int g = 0; g < kSplitParts - 1; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i) f = f + tg[g][i][k];
            fs[k] = f;
        }
        if (q > 0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) L.xch[q - 1][k][lane] = fs[k];
        }
    }
    __syncthreads();
    if (j == 0 && q == 0) {
        const int row = t * 64 + 32 * s + col;
        const int pair_rows = M & ~1;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float y = (fs[k] + L.xch[1][k][lane]) + (L.xch[0][k][lane] + L.xch[2][k][lane]);
            const int v = 8 * kVH + 4 * kh + k;
            if (v < B && row < pair_rows) __builtin_nontemporal_store(y, Y + (size_t)v * M + row);  // as the cu kernel's
        }
    }
}

// Blocks 16a + x and 16a + 8 + x (x < 8, the same XCD, so the second reads
// the weights from its L2) take unit 8a + x's two vector halves; unit =
// (tile, 32-row half); blocks past the last unit exit.
__global__ __launch_bounds__(64 * 4 * kSplitParts) void bfp8_gemv_batch_split_kernel(
    float* __restrict__ Y, const uint32_t* __restrict__ xsplit, const float* __restrict__ xscale,
    const uint8_t* __restrict__ mant, const uint8_t* __restrict__ exps, int M, int K, int B) {
    __shared__ SplitLds L;
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int b = (int)blockIdx.x;
    const int unit = 8 * (b >> 4) + (b & 7);
    if (unit >= 2 * bfp8_ntiles(M)) return;  // the whole workgroup: no barrier is left waiting
    if (((b >> 3) & 1) == 0)
        split_body<0>(L, Y, xsplit, xscale, mant, exps, M, K, B, unit >> 1, unit & 1, w & 3, w >> 2);
    else
        split_body<1>(L, Y, xsplit, xscale, mant, exps, M, K, B, unit >> 1, unit & 1, w & 3, w >> 2);
}

// kHalves: halves of a tile per workgroup (2: both, workgroup per tile; 1:
// workgroup per 32-row half, twice the workgroups for GEMVs with few tiles).
// kSplit: 1, every vector in each workgroup; 2, a workgroup per half of the
// vectors, each wavefront then finishing 4 of the 8 result slots of its
// lanes -- half the epilogue per wavefront, on twice the wavefronts, for
// GEMVs whose wavefronts are too few to hide the epilogue's latencies.  The
// two workgroups of a unit are blocks 16a + x and 16a + 8 + x (x < 8), which
// go to the same XCD (blocks are dealt to the 8 XCDs in turn), so the second
// reads the unit's weights from that XCD's L2; unit 8a + x, blocks past the
// last unit exit at once.
template <int kRes, int kHalves, int kDepth, int kSplit, int CH>
__global__ __launch_bounds__(64 * kHalves * (4 / kRes)) __attribute__((amdgpu_waves_per_eu(kSplit == 2 ? 2 : 4))) void
bfp8_gemv_batch_mfma_kernel(float* __restrict__ Y, const uint32_t* __restrict__ xsplit,
                            const float* __restrict__ xscale, const uint8_t* __restrict__ mant,
                            const uint8_t* __restrict__ exps, int M, int K, int B) {
    __shared__ MfLds<CH> L;
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int b = (int)blockIdx.x;
    const int bid = kSplit == 2 ? 8 * (b >> 4) + (b & 7) : b;
    const int nunits = kHalves == 2 ? bfp8_ntiles(M) : 2 * bfp8_ntiles(M);
    if (kSplit == 2 && bid >= nunits) return;  // the grid's last 16 blocks may hold fewer units
    // 32-row half, residue group, tile
    const int s = kHalves == 2 ? (w & 1) : (bid & 1), grp = kHalves == 2 ? (w >> 1) : w;
    const int t = kHalves == 2 ? bid : (bid >> 1);
    if (kSplit == 1)
        mf_body<kRes, kHalves, kDepth, -1, CH>(L, Y, xsplit, xscale, mant, exps, M, K, B, t, s, grp);
    else if (((b >> 3) & 1) == 0)
        mf_body<kRes, kHalves, kDepth, 0, CH>(L, Y, xsplit, xscale, mant, exps, M, K, B, t, s, grp);
    else
        mf_body<kRes, kHalves, kDepth, 1, CH>(L, Y, xsplit, xscale, mant, exps, M, K, B, t, s, grp);
}

}  // namespace

hipError_t bfp8_launch_gemv_batch_mfma(float* Y, const uint32_t* xsplit, const float* xscale, const uint8_t* mant,
                                       const uint8_t* exps, int M, int K, int B, hipStream_t s) {
    const int nt = bfp8_ntiles(M);
    if (nt == 0) return hipSuccess;
    // a ragged K drops its last K % 64 elements, as every other GEMV path does
    // (nb = K / 64 blocks; the split activation's stride is nb blocks)
    if (B < 1 || B > kMfVec || K < 64) return hipErrorInvalidValue;
    // few tiles: a workgroup per 32-row half (and, above 8 vectors, per half
    // of the vectors) so that more run; with K <= 1024 and above 8 vectors
    // the blocks are split over four wavefronts per residue (3584 x 1024,
    // B = 16: 5.5-5.7 us against 6.5-6.8 on one box), else one residue per
    // wavefront, 16-block staging, all of a chunk's weight loads in flight.  Many tiles: a
    // workgroup per four tiles, four residues per wavefront (K <= 1024; at
    // 65536 x 1024, B = 16: 14.9-15.0 us against 18.4 for a workgroup per
    // tile, on one box); beyond that, a workgroup per tile with 8-block staging.
    if (nt < 512 && B > 8 && (K >> 6) <= kCuMaxNb)  // four wavefronts per residue, a workgroup per half of the vectors
        hipLaunchKernelGGL(bfp8_gemv_batch_split_kernel, dim3(16 * ((2 * nt + 7) / 8)), dim3(64 * 4 * kSplitParts), 0, s,
                           Y, xsplit, xscale, mant, exps, M, K, B);
    else if (nt < 512 && B > 8)  // and a workgroup per half of the vectors: 2 nt units, 16 blocks per 8
        hipLaunchKernelGGL((bfp8_gemv_batch_mfma_kernel<1, 1, 16 / kMfGroup, 2, 16>), dim3(16 * ((2 * nt + 7) / 8)),
                           dim3(256), 0, s, Y, xsplit, xscale, mant, exps, M, K, B);
    else if (nt < 512)
        hipLaunchKernelGGL((bfp8_gemv_batch_mfma_kernel<1, 1, 16 / kMfGroup, 1, 16>), dim3(2 * nt), dim3(256), 0, s,
                           Y, xsplit, xscale, mant, exps, M, K, B);
    else if ((K >> 6) <= kCuMaxNb)  // many tiles, K <= 1024: a workgroup per four tiles, two blocks ahead
        hipLaunchKernelGGL((bfp8_gemv_batch_cu_kernel<2>), dim3((nt + kCuWaves / 2 - 1) / (kCuWaves / 2)),
                           dim3(64 * kCuWaves), 0, s, Y, xsplit, xscale, mant, exps, M, K, B);
    else
        hipLaunchKernelGGL((bfp8_gemv_batch_mfma_kernel<2, 2, 2, 1, 8>), dim3(nt), dim3(256), 0, s, Y, xsplit, xscale,
                           mant, exps, M, K, B);
    return hipGetLastError();
}
