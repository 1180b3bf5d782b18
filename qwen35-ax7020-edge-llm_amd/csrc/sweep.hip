// sweep.hip -- a whole sweep plan (many independent BFP8 GEMVs and at most
// one fused lm_head with its top-k) in ONE persistent launch on gfx950.
//
// Compiled with -fgpu-flush-denormals-to-zero -ffp-contract=off, like
// bfp8_ftz.hip: the per-block epilogue is the reference's Advanced SIMD one,
//   fs_q = fs_q + ((float(S_q) * 2^(e-134)) * xscale_b)   (block order),
//   y    = (fs_0 + fs_2) + (fs_1 + fs_3)                  (04/qwen_kernels_opt.c:226-277).
//
// Work mapping (as the streaming GEMV kernels): a workgroup of 4 wavefronts
// owns a 64-row tile at a time, wavefront q computes residue lane q of its 64
// rows (lane = row), streaming one 1 KiB non-temporal dwordx4 per block and
// keeping the next 4-block chunk in flight across tile boundaries.
//
// What makes one launch possible:
//   * Activations are quantized by the workgroup that reads them, into LDS,
//     all of them before the stream starts: their x loads go out before the
//     first weights (loads return in order per wavefront), the first weights
//     are in flight while they are quantized, 16 lanes per block.  Workgroup
//     w's work list is its lm_head tiles (w, w + grid, ...) then a host-built
//     list of layer tiles, dealt GEMV by GEMV so that a workgroup reads few
//     activations.
//   * The lm_head's tiles publish their top-k lists as epoch-tagged keys
//     (topk_merge.h: one agent-scope atomic store per key) and one workgroup,
//     after its own tiles, merges them, re-reading any key of an older epoch
//     (bounded).  No grid barrier, fence or counter.
#include <float.h>
#include <hip/hip_runtime.h>

#include "bfp8_internal.h"
#include "gemv_dev.h"
#include "quant_block.h"
#include "topk_merge.h"
#include "wave_topk.h"

namespace {

// Tables are read through the constant address space: scalar loads, which
// count on the scalar counter only.  A vector load of a table entry would
// have to be waited for with the vector counter, which also drains the weight
// chunk in flight.
template <class T>
using cptr = const __attribute__((address_space(4))) T*;
template <class T>
__device__ __forceinline__ cptr<T> cp(const T* p) {
    return (cptr<T>)p;
}

constexpr int kWaves = 4;
constexpr int kChunk = 4;          // blocks per streamed chunk (4 KiB per wavefront)

__device__ __forceinline__ float epilogue(float fs, int S, uint32_t e, float xs) {
    const float t1 = (float)S * exp_scale_ftz(e);
    const float t2 = t1 * xs;
    return fs + t2;
}

struct SweepLds {
    float red[2][256];       // cross-wave reduction, double-buffered by tile parity
    uint64_t keys[64];       // the lm_head tile's rank keys
    MergeLds<kWaves> merge;  // the in-launch top-k merge (one workgroup)
};

struct WBuf {
    u32x4 w[kChunk];
    uint32_t e;
};

struct Tile {  // wave-uniform
    const uint8_t* mant;
    const uint8_t* exps;
    int nb, desc, tile, xoff, slot;
};

// The workgroup's activations, all quantized into their LDS slots before the
// stream starts.  Block g of the workgroup (the slots' blocks in order) goes
// to a row of 16 lanes in passes of 16 blocks: in pass u, row k of wavefront q
// takes block 16u + 4q + k, each lane four consecutive elements.  Every x load of a group of passes is issued
// before the first weights and waited for before the weights are: loads
// return in order per wavefront, and x loads issued behind weight loads came
// back microseconds later.
constexpr int kMaxSlots = BFP8_SWEEP_MAX_SLOTS;
constexpr int kPasses = 4;  // passes whose loads are in flight together (64 blocks)

struct SlotTable {
    const float* x[kMaxSlots];
    int pre[kMaxSlots + 1];  // first block of each slot; pre[n] = all blocks
    int xoff[kMaxSlots], nb[kMaxSlots];
    int n;
};

__device__ __forceinline__ void slot_table(cptr<Bfp8SweepAct> act, int n, SlotTable& S) {
    S.n = n < kMaxSlots ? n : kMaxSlots;  // (the host deals at most kMaxSlots)
    int acc = 0;
#pragma unroll
    for (int k = 0; k < kMaxSlots; ++k) {
        const bool in = k < S.n;
        S.x[k] = in ? act[k].x : nullptr;
        S.nb[k] = in ? act[k].K >> 6 : 0;
        S.xoff[k] = in ? act[k].xoff : 0;
        S.pre[k] = acc;
        acc += S.nb[k];
    }
    S.pre[kMaxSlots] = acc;
}

struct SlotBlock {
    const float* x;  // the block's 64 floats
    int rec, scl;    // LDS word offsets of its record and its scale
};

__device__ __forceinline__ SlotBlock slot_block(const SlotTable& S, int g) {
    SlotBlock r{S.x[0], S.xoff[0], S.xoff[0] + S.nb[0] * 32};
#pragma unroll
    for (int k = 0; k < kMaxSlots; ++k) {
        if (k < S.n && g >= S.pre[k]) {
            const int b = g - S.pre[k];
            r.x = S.x[k] + (size_t)b * 64;
            r.rec = S.xoff[k] + b * 32;
            r.scl = S.xoff[k] + S.nb[k] * 32 + b;
        }
    }
    return r;
}

// Blocks g0 .. g0 + 16 kPasses - 1 of the workgroup: every x load, then
// `between` (the first weights, for the first group), then the quantization.
template <class F>
__device__ __forceinline__ void quantize_slots(const SlotTable& S, int g0, int q, int r, uint32_t* xact,
                                               F between) {
    const int row = r >> 4, ii = r & 15, total = S.pre[kMaxSlots];
    float xv[kPasses][4];
    SlotBlock sb[kPasses];
#pragma unroll
    for (int u = 0; u < kPasses; ++u) {
        const int g = g0 + 16 * u + 4 * q + row;
        sb[u] = slot_block(S, g < total ? g : 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) xv[u][j] = sb[u].x[4 * ii + j];
    }
    __builtin_amdgcn_sched_barrier(0);  // the x loads go out first
    between();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kPasses; ++u) {
        const int g = g0 + 16 * u + 4 * q + row;
        bfp8_quant4_store_lds(xv[u], ii, reinterpret_cast<float*>(xact + sb[u].scl), xact + sb[u].rec, g < total);
    }
}

__device__ __forceinline__ void issue(WBuf& B, const Tile& T, int c, int voff, int eoff) {
    const int b0 = c * kChunk;
    const int cn = min(kChunk, T.nb - b0);
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(T.mant, (uint32_t)T.nb * 4096u);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(T.exps, (uint32_t)((T.nb + 3) >> 2) * 256u);
    // every load is issued (past the tile's blocks the buffer range returns 0):
    // a fixed count per step lets the compiler wait for each chunk alone
    (void)cn;
#pragma unroll
    for (int u = 0; u < kChunk; ++u) B.w[u] = load_w(wrs, voff + u * 4096, b0 * 4096);
    B.e = load_e(ers, eoff, (b0 >> 2) * 256);
}

__device__ __forceinline__ float reduce_chunk(float fs, const WBuf& B, const Tile& T, int c, int q,
                                              const uint32_t* xact) {
    const int b0 = c * kChunk;
    const int cn = min(kChunk, T.nb - b0);
    const uint32_t* xs = xact + T.xoff;
    const float* scl = reinterpret_cast<const float*>(xs + T.nb * 32);
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
        if (u < cn) {
            const int b = b0 + u;
            const uint4 h = *reinterpret_cast<const uint4*>(xs + (b * 4 + q) * 8);
            const uint4 l = *reinterpret_cast<const uint4*>(xs + (b * 4 + q) * 8 + 4);
            const u32x4 w = B.w[u];
            int S = __builtin_amdgcn_sdot4((int)w.x, (int)h.x, 0, false);
            S = __builtin_amdgcn_sdot4((int)w.y, (int)h.y, S, false);
            S = __builtin_amdgcn_sdot4((int)w.z, (int)h.z, S, false);
            S = __builtin_amdgcn_sdot4((int)w.w, (int)h.w, S, false);
            S = (int)((uint32_t)S << 8);
            S = __builtin_amdgcn_sdot4((int)w.x, (int)l.x, S, false);
            S = __builtin_amdgcn_sdot4((int)w.y, (int)l.y, S, false);
            S = __builtin_amdgcn_sdot4((int)w.z, (int)l.z, S, false);
            S = __builtin_amdgcn_sdot4((int)w.w, (int)l.w, S, false);
            fs = epilogue(fs, S, (B.e >> (8 * u)) & 0xffu, scl[b]);
        }
    }
    return fs;
}

// A finished tile: y = (fs0 + fs2) + (fs1 + fs3); the lm_head's tile ranks
// its 64 keys and publishes its top-k list as epoch keys.
__device__ __forceinline__ void finish_tile(cptr<Bfp8GemvDesc> descs, const Tile& T, float fs, int q, int r,
                                            int parity, bool head, const EpochKeys& kf, SweepLds& L) {
    const cptr<Bfp8GemvDesc> dp = descs + T.desc;
    float* red = L.red[parity];
    red[q * 64 + r] = fs;
    __syncthreads();
    if (!head) {
        if (q == 0) {
            const float y = (red[r] + red[128 + r]) + (red[64 + r] + red[192 + r]);
            const int row = T.tile * BFP8_TILE_ROWS + r;
            if (row < dp->pair_rows) dp->y[row] = y;
        }
        return;
    }
    const int pair_rows = dp->pair_rows, topk = dp->topk;
    uint64_t* partials = dp->partials;
    // wavefront q, lane (rr, qq): row 16q + rr of the tile (each quad forms its row's y)
    const int tr = 16 * q + (r >> 2);
    const float y = (red[tr] + red[128 + tr]) + (red[64 + tr] + red[192 + tr]);
    const int row = T.tile * BFP8_TILE_ROWS + tr;
    if ((r & 3) == 0) L.keys[tr] = tile_rank_key(y, row, row < pair_rows);
    __syncthreads();
    const int rr = r >> 2, qq = r & 3;
    const uint64_t mine = L.keys[16 * q + rr];
    const uint64_t* quarter = L.keys + 16 * qq;
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) cnt += quarter[i] > mine ? 1 : 0;
    cnt += __builtin_amdgcn_update_dpp(0, cnt, 0xB1, 0xF, 0xF, false);  // + quad lane ^ 1
    cnt += __builtin_amdgcn_update_dpp(0, cnt, 0x4E, 0xF, 0xF, false);  // + quad lane ^ 2
    if (qq == 0 && cnt < topk)
        kf.store(partials + (size_t)T.tile * topk + cnt, kf.make(tile_partial_key(mine), (int)~(uint32_t)mine));
}

}  // namespace

// ---- the kernel -------------------------------------------------------------------------------
namespace {

// Everything a step needs that is the same for the whole workgroup.
struct Ctx {
    cptr<Bfp8GemvDesc> descs;
    cptr<Bfp8SweepTile> tiles;  // this workgroup's table tiles
    const uint8_t* head_mant;
    const uint8_t* head_exps;
    int head, head_K;
    int nh, ntot;               // lm_head tiles, all tiles of this workgroup
    int wg, nwg, q, r, voff, eoff;
    EpochKeys kf;

    __device__ void tile_at(int i, Tile& T) const {
        if (i < nh) {
            const int nb = head_K >> 6, nb4 = (nb + 3) >> 2;
            T.tile = wg + i * nwg;
            T.desc = head;
            T.mant = head_mant + (size_t)T.tile * nb * 4096u;
            T.exps = head_exps + (size_t)T.tile * nb4 * 256u;
            T.nb = nb;
            T.xoff = 0;
            T.slot = 0;
        } else {
            const cptr<Bfp8SweepTile> st = tiles + (i - nh);
            const cptr<Bfp8GemvDesc> d = descs + st->desc;
            const int nb = d->K >> 6, nb4 = (nb + 3) >> 2;
            T.tile = st->tile;
            T.desc = st->desc;
            T.mant = d->mant + (size_t)T.tile * nb * 4096u;
            T.exps = d->exps + (size_t)T.tile * nb4 * 256u;
            T.nb = nb;
            T.xoff = st->xoff;
            T.slot = st->slot;
        }
    }
};

struct Pos {
    int i, c, parity;
    float fs;
};

// One chunk step: the next chunk (of this tile, or the next tile's first)
// goes out into `nxt`, then chunk `cur` is reduced.  Called with the buffers'
// roles alternating, so that no register a pending load targets is ever
// copied.  Returns false after the last chunk.
__device__ __forceinline__ bool sweep_step(const Ctx& C, Pos& P, WBuf& cur, WBuf& nxt, Tile& Tc, Tile& Tn,
                                           const uint32_t* xact, SweepLds& L) {
    int ni = P.i, nc = P.c + 1;
    bool more = true;
    if (nc * kChunk >= Tc.nb) {
        ni = P.i + 1;
        nc = 0;
        more = ni < C.ntot;
        if (more) C.tile_at(ni, Tn);
    } else {
        Tn = Tc;
    }
    // issued in every step (after the last chunk into an empty buffer range:
    // no memory is read), so that the wait for `cur` never has to assume the
    // next chunk's loads are missing
    if (!more) Tn.nb = 0;
    issue(nxt, Tn, nc, C.voff, C.eoff);
    P.fs = reduce_chunk(P.fs, cur, Tc, P.c, C.q, xact);
    if (nc == 0 || !more) {
        finish_tile(C.descs, Tc, P.fs, C.q, C.r, P.parity, P.i < C.nh, C.kf, L);
        P.fs = 0.0f;
        P.parity ^= 1;
    }
    P.i = ni;
    P.c = nc;
    return more;
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void bfp8_sweep_kernel(Bfp8SweepArgs a) {
    extern __shared__ __align__(16) uint32_t xact[];  // the workgroup's activation slots
    __shared__ SweepLds L;
    Ctx C;
    C.q = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    C.r = threadIdx.x & 63;
    C.voff = C.q * 1024 + C.r * 16;
    C.eoff = C.r * 4;
    C.kf = EpochKeys{a.epoch};
    C.wg = (int)blockIdx.x;
    C.nwg = (int)gridDim.x;
    C.head = a.head;
    C.head_K = a.head_K;
    C.head_mant = a.head_mant;
    C.head_exps = a.head_exps;
    C.descs = cp(a.descs);
    C.nh = (a.head >= 0 && C.wg < a.head_ntiles) ? (a.head_ntiles - C.wg + C.nwg - 1) / C.nwg : 0;
    // work list: this workgroup's lm_head tiles (computed), then its table tiles
    Tile TA, TB;
    WBuf A, B;
    const int tbeg = cp(a.wg_off)[C.wg];
    C.ntot = C.nh + cp(a.wg_off)[C.wg + 1] - tbeg;
    C.tiles = cp(a.tiles) + tbeg;
    if (C.ntot == 0) return;  // uniform per workgroup
    C.tile_at(0, TA);
    // the activations: every x load of a group of passes, then (the first
    // group only) the first weights, then the quantization into LDS
    SlotTable S;
    slot_table(cp(a.acts) + cp(a.act_off)[C.wg], cp(a.act_off)[C.wg + 1] - cp(a.act_off)[C.wg], S);
    if (S.pre[kMaxSlots] > 0)  // (always: every tile reads a slot) straight-line, so it waits for x only
        quantize_slots(S, 0, C.q, C.r, xact, [&] { issue(A, TA, 0, C.voff, C.eoff); });
    else
        issue(A, TA, 0, C.voff, C.eoff);
    for (int g0 = 16 * kPasses; g0 < S.pre[kMaxSlots]; g0 += 16 * kPasses)
        quantize_slots(S, g0, C.q, C.r, xact, [] {});
    __syncthreads();
    Pos P{0, 0, 0, 0.0f};
    for (;;) {
        if (!sweep_step(C, P, A, B, TA, TB, xact, L)) break;
        if (!sweep_step(C, P, B, A, TB, TA, xact, L)) break;
    }
    // the lm_head's top-k: one workgroup, after its own tiles
    if (a.head >= 0 && C.wg == a.merger) {
        const cptr<Bfp8GemvDesc> d = C.descs + a.head;
        const TopkArgs ta{d->partials, d->out_ids, d->out_scores, d->out_count, d->out_argmax, d->topk,
                          a.head_ntiles};
        __syncthreads();
        topk_merge<kWaves, 4, 4, false>(ta, C.kf, L.merge);
    }
}

// ---- launcher -----------------------------------------------------------------------------
int bfp8_sweep_grid() {
    static const int g = [] {
        int dev = 0, cus = 256, occ = 0;
        hipDeviceProp_t p;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess)
            cus = p.multiProcessorCount;
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(bfp8_sweep_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, BFP8_SWEEP_LDS_WORDS * 4);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(bfp8_sweep_kernel), 256,
                                                         BFP8_SWEEP_LDS_WORDS * 4) != hipSuccess ||
            occ <= 0)
            occ = 1;
        return cus * (occ < BFP8_STREAM_WG_PER_CU ? occ : BFP8_STREAM_WG_PER_CU);
    }();
    return g;
}

hipError_t bfp8_launch_sweep(const Bfp8SweepArgs& a, int nwg, int lds_words, hipStream_t s) {
    if (nwg <= 0) return hipSuccess;
    if (lds_words > BFP8_SWEEP_LDS_WORDS || nwg > bfp8_sweep_grid()) return hipErrorInvalidValue;
    hipLaunchKernelGGL(bfp8_sweep_kernel, dim3(nwg), dim3(256), (size_t)(lds_words > 0 ? lds_words : 1) * 4, s, a);
    return hipGetLastError();
}
