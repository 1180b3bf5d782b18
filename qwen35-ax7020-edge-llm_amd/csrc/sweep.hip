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
//   * Activations are quantized by the workgroup that reads them, into LDS.
//     Workgroup w's work list is its lm_head tiles (w, w + grid, ...: no
//     table lookup stands before their weights) then a host-built list of
//     layer tiles, dealt GEMV by GEMV so that a workgroup reads few
//     activations.  The first tile's activation is quantized while the first
//     weights are in flight; every other slot at the end of the tile before
//     its first use, while the next chunk is in flight.
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

// The workgroup's activation slots and their background quantization.
struct Slots {
    cptr<Bfp8SweepAct> act;   // this workgroup's slots (slot 0 first)
    int n;                    // number of slots
    int tasks;                // total blocks to quantize
    int next;                 // first block not yet started
};

// Slot of background task t (blocks of slot 0, then slot 1, ...), and its block.
__device__ __forceinline__ void task_of(const Slots& S, int t, int& slot, int& b) {
    slot = 0;
    b = t;
    while (slot + 1 < S.n && b >= (S.act[slot].K >> 6)) {
        b -= S.act[slot].K >> 6;
        ++slot;
    }
}

__device__ __forceinline__ int slot_end(const Slots& S, int slot) {
    int e = 0;
    for (int i = 0; i <= slot; ++i) e += S.act[i].K >> 6;
    return e;
}

// x of task t for this lane; past the last task the last task's x is read
// (and never used), so that every step issues the same loads.
__device__ __forceinline__ float task_x(const Slots& S, int t, int lane) {
    int sl, b;
    task_of(S, min(t, S.tasks - 1), sl, b);
    return S.act[sl].x[(size_t)b * 64 + lane];
}

__device__ __forceinline__ void task_run(const Slots& S, int t, float xv, int lane, uint32_t* xact) {
    if (t >= S.tasks) return;
    int sl, b;
    task_of(S, t, sl, b);
    const int nb = S.act[sl].K >> 6, xoff = S.act[sl].xoff;
    bfp8_quant_block_lds(xv, lane, reinterpret_cast<float*>(xact + xoff + nb * 32 + b), xact + xoff + b * 32);
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

// Quantizes blocks [S.next, upto) into their slots now: wavefront q takes
// blocks S.next + q, + 4, ..., up to 16 of them with all their x loads issued
// before the first is used (one memory round trip per 64 blocks).
constexpr int kBatch = 16;
__device__ __forceinline__ void run_tasks_now(Slots& S, int upto, int q, int r, uint32_t* xact) {
    while (S.next < upto) {
        float xv[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) xv[u] = task_x(S, S.next + q + kWaves * u, r);
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (S.next + q + kWaves * u < upto) task_run(S, S.next + q + kWaves * u, xv[u], r, xact);
        S.next = min(S.next + kWaves * kBatch, upto);
    }
}

// One chunk step: the next chunk (of this tile, or the next tile's first)
// goes out into `nxt`, then chunk `cur` is reduced.  Called with the buffers'
// roles alternating, so that no register a pending load targets is ever
// copied.  At a tile's end, a slot the next tile needs is quantized (its x
// loads wait behind the chunk in flight, which is needed next anyway).
// Returns false after the last chunk.
__device__ __forceinline__ bool sweep_step(const Ctx& C, Pos& P, WBuf& cur, WBuf& nxt, Tile& Tc, Tile& Tn, Slots& S,
                                           uint32_t* xact, SweepLds& L) {
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
        if (more && slot_end(S, Tn.slot) > S.next) {  // the next tile's slot
            run_tasks_now(S, slot_end(S, Tn.slot), C.q, C.r, xact);
            __syncthreads();
        }
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
    if (C.nh > 0) {  // the lm_head tile's weights before anything else
        C.tile_at(0, TA);
        issue(A, TA, 0, C.voff, C.eoff);
    }
    const int tbeg = cp(a.wg_off)[C.wg];
    C.ntot = C.nh + cp(a.wg_off)[C.wg + 1] - tbeg;
    C.tiles = cp(a.tiles) + tbeg;
    if (C.ntot == 0) return;  // uniform per workgroup
    if (C.nh == 0) {
        C.tile_at(0, TA);
        issue(A, TA, 0, C.voff, C.eoff);
    }
    Slots S;
    S.act = cp(a.acts) + cp(a.act_off)[C.wg];
    S.n = cp(a.act_off)[C.wg + 1] - cp(a.act_off)[C.wg];
    S.tasks = slot_end(S, S.n - 1);
    S.next = 0;
    // the first tile's slot now, while its weights are in flight
    run_tasks_now(S, slot_end(S, TA.slot), C.q, C.r, xact);
    __syncthreads();
    Pos P{0, 0, 0, 0.0f};
    for (;;) {
        if (!sweep_step(C, P, A, B, TA, TB, S, xact, L)) break;
        if (!sweep_step(C, P, B, A, TB, TA, S, xact, L)) break;
    }
    // the lm_head's top-k: one workgroup, after its own tiles
    if (a.head >= 0 && C.wg == a.merger) {
        const cptr<Bfp8GemvDesc> d = C.descs + a.head;
        const TopkArgs ta{d->partials, d->out_ids, d->out_scores, d->out_count, d->out_argmax, d->topk,
                          a.head_ntiles};
        __syncthreads();
        topk_merge<kWaves, 4>(ta, C.kf, L.merge);
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
