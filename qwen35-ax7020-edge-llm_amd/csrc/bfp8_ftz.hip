// bfp8_ftz.hip -- BFP8 W8A16 GEMV kernels for gfx950 (MI355X).
//
// Compiled with -fgpu-flush-denormals-to-zero -ffp-contract=off: every f32
// operation here flushes subnormal operands and results to signed zero and
// rounds once, which is how the reference's Advanced SIMD code computes
// (ARMv7 NEON is always flush-to-zero; vmlaq_n_f32 on Cortex-A9 rounds the
// product and then the sum).
//
// Reference semantics restated (04/qwen_kernels_opt.c:207-278, row pairs):
//   for every row and block b:  S_j = sum_{k = j mod 4} w[k] * xq[k]   (int32)
//     fs_j = fs_j + ((float(S_j) * EXP_SCALE[e]) * xscale[b])         (j = 0..3)
//   y = (fs_0 + fs_2) + (fs_1 + fs_3)
// with EXP_SCALE[e] = 2^(e-134), read as zero when subnormal (e < 8).
//
// Work mapping: a workgroup of 4 wavefronts owns a tile of 64 rows; wavefront
// q computes residue lane q of all 64 rows (lane = row), streaming one 1 KiB
// contiguous non-temporal dwordx4 load per block (the four wavefronts together
// read 4 KiB contiguous per block step).  The split activation (xq = 256*xh +
// xl, four bytes per dword) is read with scalar loads straight into SGPRs, so
// the inner loop is 8 x v_dot4_i32_i8 with SGPR operands + 1 shift per 16
// weight bytes per lane.  The GEMV kernels are persistent: a resident grid of
// workgroups streams a list of tiles each with the next chunk always in
// flight.  The per-block float epilogue runs in block order inside each lane,
// which is exactly the reference's per-lane accumulation order.  No MFMA:
// batch-1 is a bandwidth-bound matrix-vector product.
#include <float.h>
#include <hip/hip_runtime.h>

#include "bfp8_internal.h"
#include "gemv_dev.h"
#include "quant_block.h"
#include "runtime_internal.h"
#include "topk_merge.h"
#include "wave_topk.h"

namespace {

typedef const __attribute__((address_space(4))) uint32_t* sgpr_u32_ptr;
typedef const __attribute__((address_space(4))) float* sgpr_f32_ptr;

constexpr int kChunk = 4;       // streamed blocks per load batch (4 KiB per wavefront)
constexpr int kBatchChunk = 8;  // blocks per LDS-staged step of the batched kernel
static_assert(kChunk == 4 || kChunk == 8, "a chunk spans one or two exponent words");
// fs += (float(S) * EXP_SCALE[e]) * xscale   (three roundings, flush-to-zero)
__device__ __forceinline__ float epilogue(float fs, int S, uint32_t e, float xs) {
    float t1 = (float)S * exp_scale_ftz(e);
    float t2 = t1 * xs;
    return fs + t2;
}

// ---- top-k final merge (topk_merge.h) --------------------------------------------
// The per-tile partials ([ntiles][topk] sorted keys) are written by one
// streaming launch and merged by a later launch on the same stream: the
// kernel boundary makes them visible, so no cross-workgroup fence or atomic
// is needed.  The merge runs as its own 16-wavefront kernel, or folded into
// workgroup 0 of the next grouped launch (4 wavefronts).
__device__ __forceinline__ TopkArgs topk_args(const Bfp8GemvDesc& d) {
    return TopkArgs{d.partials, d.out_ids, d.out_scores, d.out_count, d.out_argmax, d.topk, bfp8_ntiles(d.M)};
}

constexpr int kWaves = 4;        // wavefronts per GEMV workgroup
constexpr int kMergeWaves = 16;  // wavefronts of the stand-alone merge kernel

// Folded merge for workgroup 0 of a grouped launch.
__device__ __noinline__ void topk_merge_folded(TopkArgs d, MergeLds<kWaves>& L) {
    topk_merge<kWaves, 4, 4, false>(d, PlainKeys{}, L);
    __syncthreads();  // L is reused by the streaming code
}

// Per-tile top-k partial: the tile's keys sorted in wavefront 0, the best
// `topk` stored.  Plain stores: the merge runs in a later launch.
__device__ __noinline__ void topk_partial(uint64_t* partials, int topk, int pair_rows, int t, float y) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const int row = t * BFP8_TILE_ROWS + lane;
        uint64_t key[1] = {(row < pair_rows) ? topk_key(y, row) : 0ull};
        const bool desc[1] = {true};
        wave_sort<1>(key, desc, lane);
        if (lane < topk) partials[(size_t)t * topk + lane] = key[0];
    }
}

// ---- persistent streaming GEMV ------------------------------------------------
// A workgroup of 4 wavefronts owns one 64-row tile at a time; wavefront q
// computes residue lane q of the tile's rows (lane = row).  Each workgroup
// walks a list of tiles -- a host-built, byte-balanced slice of a tile table
// (plans) or every gridDim-th tile of one GEMV -- and streams their weights as
// chunks of kChunk blocks (1 KiB per block per wavefront).  The next chunk, including the
// first chunk of the next tile, is always in flight while the current chunk is
// reduced, so no workgroup stalls on a cold start between tiles.

struct WBuf {  // one chunk: kChunk residue slices of 16 B and its exponent word(s)
    u32x4 w[kChunk];
    uint32_t e0, e1;
};

struct Tile {  // the tile being streamed; every field is wave-uniform
    const uint8_t* mant;  // this tile's mantissas (nb * 4 KiB)
    const uint8_t* exps;  // this tile's exponent words (nb4 * 256 B)
    const uint32_t* xsplit;
    const float* xscale;
    int nb, desc, tile;
};

struct StreamLds {
    float red[2][256];        // cross-wave reduction, double-buffered by tile parity
    MergeLds<kWaves> merge;   // folded top-k merge (workgroup 0 only)
};

__device__ __forceinline__ int nchunks(const Tile& T) { return (T.nb + kChunk - 1) / kChunk; }

__device__ __forceinline__ void open_tile(Tile& T, const Bfp8GemvDesc& d, int desc, int t) {
    const int nb = d.K >> 6, nb4 = (nb + 3) >> 2;
    T.mant = d.mant + (size_t)t * nb * 4096u;
    T.exps = d.exps + (size_t)t * nb4 * 256u;
    T.xsplit = d.xsplit;
    T.xscale = d.xscale;
    T.nb = nb;
    T.desc = desc;
    T.tile = t;
}

// wv[u]: this lane's byte offset of block u of a chunk (q*1 KiB + lane*16 +
// u*4 KiB); the chunk itself is one scalar offset.
__device__ __forceinline__ void issue(WBuf& B, const Tile& T, int c, const int* wv, int ev) {
    const int b0 = c * kChunk;
    const int cn = min(kChunk, T.nb - b0);
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(T.mant, (uint32_t)T.nb * 4096u);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(T.exps, (uint32_t)((T.nb + 3) >> 2) * 256u);
    if (cn == kChunk) {
#pragma unroll
        for (int u = 0; u < kChunk; ++u) B.w[u] = load_w(wrs, wv[u], b0 * 4096);
    } else {
#pragma unroll
        for (int u = 0; u < kChunk; ++u)
            if (u < cn) B.w[u] = load_w(wrs, wv[u], b0 * 4096);
    }
    B.e0 = load_e(ers, ev, (b0 >> 2) * 256);
    B.e1 = (kChunk > 4 && cn > 4) ? load_e(ers, ev, ((b0 >> 2) + 1) * 256) : 0u;
}

// Exact S_q of one (row, block, residue) from the scalar-loaded split activation.
__device__ __forceinline__ int residue_sum(u32x4 w, sgpr_u32_ptr xb) {
    int acc = __builtin_amdgcn_sdot4((int)w.x, (int)xb[0], 0, false);
    acc = __builtin_amdgcn_sdot4((int)w.y, (int)xb[1], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.z, (int)xb[2], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w, (int)xb[3], acc, false);
    acc = (int)((uint32_t)acc << 8);
    acc = __builtin_amdgcn_sdot4((int)w.x, (int)xb[4], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.y, (int)xb[5], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.z, (int)xb[6], acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w, (int)xb[7], acc, false);
    return acc;
}

// lanes_row: this lane's row of the optional [M][nb][4] residue-lane output.
template <bool kLanes>
__device__ __forceinline__ float reduce_block(float fs, const WBuf& B, int u, const Tile& T, int b, int q,
                                              int32_t* lanes_row) {
    const int S = residue_sum(B.w[u], (sgpr_u32_ptr)T.xsplit + (b * 4 + q) * 8);
    const uint32_t e = ((u < 4 ? B.e0 : B.e1) >> (8 * (u & 3))) & 0xffu;
    if (kLanes && lanes_row) lanes_row[b * 4 + q] = S;
    return epilogue(fs, S, e, ((sgpr_f32_ptr)T.xscale)[b]);
}

template <bool kLanes>
__device__ __forceinline__ float reduce_chunk(float fs, const WBuf& B, const Tile& T, int c, int q,
                                              int32_t* lanes_row) {
    const int b0 = c * kChunk;
    const int cn = min(kChunk, T.nb - b0);
    if (cn == kChunk) {
#pragma unroll
        for (int u = 0; u < kChunk; ++u) fs = reduce_block<kLanes>(fs, B, u, T, b0 + u, q, lanes_row);
    } else {
#pragma unroll
        for (int u = 0; u < kChunk; ++u)
            if (u < cn) fs = reduce_block<kLanes>(fs, B, u, T, b0 + u, q, lanes_row);
    }
    return fs;
}

// Cross-wave combine of a finished tile: vadd_f32(low, high) then vpadd_f32,
// i.e. y = (fs0 + fs2) + (fs1 + fs3).
__device__ __forceinline__ void finish_tile(const Bfp8GemvDesc& d, const Tile& T, float fs, int q, int r,
                                            int parity, StreamLds& L) {
    float* red = L.red[parity];
    red[q * 64 + r] = fs;
    __syncthreads();
    float y = 0.0f;
    if (q == 0) {
        y = (red[r] + red[128 + r]) + (red[64 + r] + red[192 + r]);
        const int row = T.tile * BFP8_TILE_ROWS + r;
        if (d.y && row < d.pair_rows) d.y[row] = y;
    }
    if (d.topk > 0) topk_partial(d.partials, d.topk, d.pair_rows, T.tile, y);
}

// Tile lists: a slice of a tile table, or a strided walk over one GEMV.
struct TableTiles {
    const Bfp8GemvDesc* descs;
    const Bfp8TileRef* tiles;
    int beg, cnt;
    __device__ int count() const { return cnt; }
    __device__ void get(int i, int& desc, int& tile) const {
        const Bfp8TileRef tr = tiles[beg + i];
        desc = tr.desc;
        tile = tr.tile;
    }
    __device__ const Bfp8GemvDesc& desc(int i) const { return descs[i]; }
};

struct StridedTiles {
    const Bfp8GemvDesc* d;
    int ntiles;
    __device__ int count() const {
        return (int)blockIdx.x < ntiles ? (ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;
    }
    __device__ void get(int i, int& desc, int& tile) const {
        desc = 0;
        tile = (int)blockIdx.x + i * (int)gridDim.x;
    }
    __device__ const Bfp8GemvDesc& desc(int) const { return *d; }
};

// One half of the double-buffered stream: reduce `cur` (chunk `c` of tile
// `Tc`) while the following chunk goes out into `nxt` / `Tn`.  Returns false
// after the last chunk of the list.
template <bool kLanes, class Src>
__device__ __forceinline__ bool stream_step(const Src& src, WBuf& cur, WBuf& nxt, Tile& Tc, Tile& Tn, int& i,
                                            int& c, float& fs, int& parity, int q, int r, const int* wv,
                                            int ev, StreamLds& L) {
    const int n = src.count();
    int ni = i, nc = c + 1;
    bool more = true;
    if (nc == nchunks(Tc)) {
        ni = i + 1;
        nc = 0;
        more = ni < n;
        if (more) {
            int di, ti;
            src.get(ni, di, ti);
            open_tile(Tn, src.desc(di), di, ti);
        }
    } else {
        Tn = Tc;
    }
    if (more) issue(nxt, Tn, nc, wv, ev);
    int32_t* lanes_row = nullptr;
    if (kLanes) {
        const Bfp8GemvDesc& dc = src.desc(Tc.desc);
        const int row = Tc.tile * BFP8_TILE_ROWS + r;
        if (dc.lanes && row < dc.M) lanes_row = dc.lanes + (size_t)row * Tc.nb * 4;
    }
    fs = reduce_chunk<kLanes>(fs, cur, Tc, c, q, lanes_row);
    if (nc == 0 || !more) {
        finish_tile(src.desc(Tc.desc), Tc, fs, q, r, parity, L);
        fs = 0.0f;
        parity ^= 1;
    }
    i = ni;
    c = nc;
    return more;
}

template <bool kLanes, class Src>
__device__ __forceinline__ void stream_tiles(const Src& src, StreamLds& L) {
    const int n = src.count();
    if (n <= 0) return;
    const int q = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = threadIdx.x & 63;
    int wv[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u) wv[u] = q * 1024 + r * 16 + u * 4096;
    const int ev = r * 4;
    Tile TA, TB;
    WBuf A, B;
    {
        int di, ti;
        src.get(0, di, ti);
        open_tile(TA, src.desc(di), di, ti);
    }
    issue(A, TA, 0, wv, ev);
    int i = 0, c = 0, parity = 0;
    float fs = 0.0f;
    for (;;) {
        if (!stream_step<kLanes>(src, A, B, TA, TB, i, c, fs, parity, q, r, wv, ev, L)) break;
        if (!stream_step<kLanes>(src, B, A, TB, TA, i, c, fs, parity, q, r, wv, ev, L)) break;
    }
}

// ---- one tile per workgroup, K split across wavefronts (small M) ------------------
// A lone GEMV of a few thousand rows has too few 64-row tiles to keep the chip
// busy with one 4-wavefront workgroup per tile.  Here 16 wavefronts own a
// tile: wavefront (q, s) computes residue q of the 64 rows over block slice s
// and issues all of that slice's loads before any arithmetic, so the whole
// tile is in flight at once.  The per-block term t2 = (float(S) * 2^(e-134))
// * xscale is formed independently per block (the same two roundings as the
// streaming kernel); the reference's order is kept by adding the terms per
// (row, q) in block order: slice 0 adds its own as it forms them, slices 1..3
// leave theirs in LDS.
constexpr int kWideWaves = 16;
constexpr int kWideSlices = kWideWaves / 4;
constexpr int kWideMaxPer = 16;  // blocks per slice (K <= 4096)

__host__ __device__ __forceinline__ int wide_per(int nb) { return (nb + kWideSlices - 1) / kWideSlices; }

template <bool kLanes>
__device__ __forceinline__ void wide_tile(const Bfp8GemvDesc& d, int t, float* terms, float (*red)[64]) {
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = threadIdx.x & 63;
    const int q = w & 3, sl = w >> 2;
    const int nb = d.K >> 6, nb4 = (nb + 3) >> 2;
    const int per = wide_per(nb);
    const int b0 = sl * per;
    const int cnt = max(0, min(per, nb - b0));
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(d.mant + (size_t)t * nb * 4096u, (uint32_t)nb * 4096u);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(d.exps + (size_t)t * nb4 * 256u, (uint32_t)nb4 * 256u);
    const int voff = q * 1024 + r * 16;
    u32x4 wv[kWideMaxPer];
    uint32_t ev[kWideMaxPer];
#pragma unroll
    for (int u = 0; u < kWideMaxPer; ++u) {
        if (u < cnt) {
            const int b = b0 + u;
            wv[u] = load_w(wrs, voff, b * 4096);
            ev[u] = load_e(ers, r * 4, (b >> 2) * 256);
        }
    }
    // The slice's split activation and scales, fetched with the weights by
    // vector loads (a cold scalar cache would serialise one round trip per
    // block): lane l holds word (l & 7) of block b0 + (l >> 3) (+ 8 in xb) and
    // the scale of block b0 + l; v_readlane broadcasts them as SGPR operands.
    const int xj = r >> 3, xw = r & 7;
    const uint32_t xa = xj < cnt ? d.xsplit[((b0 + xj) * 4 + q) * 8 + xw] : 0u;
    const uint32_t xb = xj + 8 < cnt ? d.xsplit[((b0 + xj + 8) * 4 + q) * 8 + xw] : 0u;
    const float xsv = r < cnt ? d.xscale[b0 + r] : 0.0f;
    const int row = t * BFP8_TILE_ROWS + r;
    int32_t* lanes_row = (kLanes && d.lanes && row < d.M) ? d.lanes + (size_t)row * nb * 4 : nullptr;
    float fs = 0.0f;
#pragma unroll
    for (int u = 0; u < kWideMaxPer; ++u) {
        if (u < cnt) {
            const int b = b0 + u;
            const uint32_t src = u < 8 ? xa : xb;
            uint32_t x[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) x[k] = __builtin_amdgcn_readlane(src, (u & 7) * 8 + k);
            const u32x4 w = wv[u];
            int S = __builtin_amdgcn_sdot4((int)w.x, (int)x[0], 0, false);
            S = __builtin_amdgcn_sdot4((int)w.y, (int)x[1], S, false);
            S = __builtin_amdgcn_sdot4((int)w.z, (int)x[2], S, false);
            S = __builtin_amdgcn_sdot4((int)w.w, (int)x[3], S, false);
            S = (int)((uint32_t)S << 8);
            S = __builtin_amdgcn_sdot4((int)w.x, (int)x[4], S, false);
            S = __builtin_amdgcn_sdot4((int)w.y, (int)x[5], S, false);
            S = __builtin_amdgcn_sdot4((int)w.z, (int)x[6], S, false);
            S = __builtin_amdgcn_sdot4((int)w.w, (int)x[7], S, false);
            if (kLanes && lanes_row) lanes_row[b * 4 + q] = S;
            const uint32_t e = (ev[u] >> (8 * (b & 3))) & 0xffu;
            const float t1 = (float)S * exp_scale_ftz(e);
            const float t2 = t1 * __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(uint32_t, xsv), u));
            if (sl == 0)
                fs = fs + t2;
            else
                terms[((b - per) * 4 + q) * 64 + r] = t2;
        }
    }
    __syncthreads();
    if (sl == 0) {
        for (int b = per; b < nb; ++b) fs = fs + terms[((b - per) * 4 + q) * 64 + r];
        red[q][r] = fs;
    }
    __syncthreads();
    if (w == 0) {
        // vadd_f32(low, high) then vpadd_f32: y = (fs0 + fs2) + (fs1 + fs3)
        const float y = (red[0][r] + red[2][r]) + (red[1][r] + red[3][r]);
        if (d.y && row < d.pair_rows) d.y[row] = y;
    }
}

// ---- the lm_head launch with the plan's activation quantization folded in ------------
// A plan step was a quantize launch (every activation) and then the lm_head's
// streaming launch.  Here one launch does both: every workgroup quantizes the
// lm_head's activation (K <= 1024) into LDS while its tile's weights are in
// flight, and each wavefront one 64-element block of the plan's other
// activations (a task) into the records the next launch reads -- the launch
// boundary publishes them.  Tiles are reduced as in the streaming kernel:
// wavefront q computes residue q of the tile's 64 rows (lane = row), fs_q in
// block order, y = (fs0 + fs2) + (fs1 + fs3), with the split activation words
// broadcast from registers by v_readlane.
struct HeadLds {
    __attribute__((aligned(16))) uint32_t xs[BFP8_HEAD_MAX_NB * 32];
    float xsc[BFP8_HEAD_MAX_NB];
    uint32_t rec[kWaves][32];
    float red[256];
    uint64_t keys[BFP8_TILE_ROWS];
};

// bfp8_quant_block_wave with the records written through global-address-space
// pointers (flat stores would also count on the LDS counter).
typedef __attribute__((address_space(1))) uint32_t* g_u32_ptr;
typedef __attribute__((address_space(1))) float* g_f32_ptr;
typedef __attribute__((address_space(1))) int16_t* g_i16_ptr;
__device__ __forceinline__ void quantize_task(const Bfp8HeadTask& d, float xv, int lane, uint32_t* rec) {
    const int b = d.b;
    const Bfp8QuantLane r = bfp8_quant_lane(xv);
    if (d.xq) ((g_i16_ptr)d.xq)[(size_t)b * 64 + lane] = (int16_t)r.xq;
    if (lane == 0) ((g_f32_ptr)d.xscale)[b] = r.xs;
    const int xl = (int)(int8_t)(r.xq & 0xff);
    const int xh = (r.xq - xl) >> 8;
    const int pos = bfp8_split_pos(lane);
    uint8_t* rb = reinterpret_cast<uint8_t*>(rec);
    rb[pos] = (uint8_t)xh;
    rb[pos + 16] = (uint8_t)xl;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < 32) ((g_u32_ptr)d.xsplit)[(size_t)b * 32 + lane] = rec[lane];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace

// Every load is unconditional (indices clamped): the compiler can then count
// them and wait for each block's weights alone.  A tile's blocks are issued
// kHeadDepth ahead of the block being reduced: with 4096 wavefronts streaming,
// 4 KiB in flight per wavefront beat the whole tile at once (13.1 against
// 15.1 us for the 65536 x 1024 lm_head launch; 2 KiB: 13.2-13.9 us).
constexpr int kHeadDepth = 4;
struct HeadTile {
    u32x4 w[BFP8_HEAD_MAX_NB];
    uint32_t e[BFP8_HEAD_MAX_NB / 4];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_wrs(const Bfp8HeadArgs& a, int t, int nb) {
    return make_rsrc(a.mant + (size_t)t * nb * 4096u, (uint32_t)nb * 4096u);
}

__device__ __forceinline__ void head_issue(HeadTile& T, const Bfp8HeadArgs& a, int t, int nb, int q, int lane) {
    const int nb4 = (nb + 3) >> 2;
    const __amdgpu_buffer_rsrc_t wrs = head_wrs(a, t, nb);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(a.exps + (size_t)t * nb4 * 256u, (uint32_t)nb4 * 256u);
#pragma unroll
    for (int u = 0; u < kHeadDepth; ++u) T.w[u] = load_w(wrs, q * 1024 + lane * 16, min(u, nb - 1) * 4096);
#pragma unroll
    for (int m = 0; m < BFP8_HEAD_MAX_NB / 4; ++m) T.e[m] = load_e(ers, lane * 4, min(m, nb4 - 1) * 256);
}

// fs_q of one tile (blocks in order), then y = (fs0 + fs2) + (fs1 + fs3) and
// the tile's top-k partial
__device__ __forceinline__ void head_reduce(HeadTile& T, const Bfp8HeadArgs& a, int t, int nb, int q, int lane,
                                            uint32_t xr0, uint32_t xr1, uint32_t xsv, HeadLds& L) {
    const __amdgpu_buffer_rsrc_t wrs = head_wrs(a, t, nb);
    float fs = 0.0f;
#pragma unroll
    for (int b = 0; b < BFP8_HEAD_MAX_NB; ++b) {
        if (b + kHeadDepth < BFP8_HEAD_MAX_NB)
            T.w[b + kHeadDepth] = load_w(wrs, q * 1024 + lane * 16, min(b + kHeadDepth, nb - 1) * 4096);
        if (b < nb) {
            const uint32_t src = b < 8 ? xr0 : xr1;
            uint32_t x[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) x[k] = __builtin_amdgcn_readlane(src, (b & 7) * 8 + k);
            const u32x4 w = T.w[b];
            int S = __builtin_amdgcn_sdot4((int)w.x, (int)x[0], 0, false);
            S = __builtin_amdgcn_sdot4((int)w.y, (int)x[1], S, false);
            S = __builtin_amdgcn_sdot4((int)w.z, (int)x[2], S, false);
            S = __builtin_amdgcn_sdot4((int)w.w, (int)x[3], S, false);
            S = (int)((uint32_t)S << 8);
            S = __builtin_amdgcn_sdot4((int)w.x, (int)x[4], S, false);
            S = __builtin_amdgcn_sdot4((int)w.y, (int)x[5], S, false);
            S = __builtin_amdgcn_sdot4((int)w.z, (int)x[6], S, false);
            S = __builtin_amdgcn_sdot4((int)w.w, (int)x[7], S, false);
            const uint32_t e = (T.e[b >> 2] >> (8 * (b & 3))) & 0xffu;
            fs = epilogue(fs, S, e, __uint_as_float(__builtin_amdgcn_readlane(xsv, b)));
        }
    }
    // (constant address space: scalar loads, not waited for with the weights)
    const __attribute__((address_space(4))) Bfp8GemvDesc* dp =
        (const __attribute__((address_space(4))) Bfp8GemvDesc*)a.descs + a.head;
    float* const dy = dp->y;
    uint64_t* const partials = dp->partials;
    const int pair_rows = dp->pair_rows, topk = dp->topk;
    L.red[q * 64 + lane] = fs;
    __syncthreads();
    // wavefront q, lane (r, qq): row 16q + r of the tile (each quad computes
    // its row's y; vadd_f32(low, high) then vpadd_f32: (fs0 + fs2) + (fs1 + fs3))
    const int tr = 16 * q + (lane >> 2);
    const float y = (L.red[tr] + L.red[128 + tr]) + (L.red[64 + tr] + L.red[192 + tr]);
    const int row = t * BFP8_TILE_ROWS + tr;
    if ((lane & 3) == 0) {
        if (dy && row < pair_rows) dy[row] = y;
        L.keys[tr] = tile_rank_key(y, row, row < pair_rows);
    }
    if (topk > 0) {
        __syncthreads();
        tile_topk_rank(L.keys, partials, t, topk, q, lane);
    }
    __syncthreads();  // L.red and L.keys are reused by the next tile
}

// The tile's first kHeadDepth blocks of weights go out first, with nothing
// but the arguments before them; then the lm_head activation and this
// wavefront's quantization task (a record and its 64 floats), which are
// waited for (with those weights: a wavefront's loads complete in issue
// order) before the activation is quantized.  The weights cannot be reduced
// before the activation is in either way; issued first, they stream during
// the activation's round trip instead of after it (13.08-13.22 -> 12.94-13.02
// us for the 65536 x 1024 launch, three interleaved pairs on one box).  The
// record comes in by a vector load (one 8-byte word per lane) and readlanes,
// not by scalar loads: those count on the counter that the LDS barrier below
// waits for, and under the weight streams they returned late.
extern "C" __global__ __launch_bounds__(256) void bfp8_gemv_head_kernel(Bfp8HeadArgs a) {
    __shared__ HeadLds L;
    const int q = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int nb = a.K >> 6;  // 1 .. BFP8_HEAD_MAX_NB (host-checked)
    const int wid = (int)blockIdx.x * kWaves + q, nw = (int)gridDim.x * kWaves;

    // 0. the first weights (the tile's exponents and kHeadDepth blocks)
    HeadTile T;
    int t = blockIdx.x;
    head_issue(T, a, t, nb, q, lane);
    __builtin_amdgcn_sched_barrier(0);

    // the lm_head activation: block 4q + lane / 16, elements 4 (lane % 16)
    // + j (blocks past nb read block nb - 1 and are never stored); this
    // wavefront's task record, one 8-byte word per lane 0..5; then its element
    static_assert(BFP8_HEAD_MAX_NB == 4 * kWaves, "one block per row of 16 lanes");
    static_assert(sizeof(Bfp8HeadTask) == 48, "six 8-byte words");
    const int hb = 4 * q + (lane >> 4), hi = lane & 15;
    float hv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) hv[j] = a.hx[min(hb, nb - 1) * 64 + 4 * hi + j];
    const int ti = min(wid, max(a.ntasks - 1, 0));
    typedef const __attribute__((address_space(1))) uint64_t* g_u64_ptr;
    const uint64_t tw = ((g_u64_ptr)(a.qtasks + ti))[min(lane, 5)];
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the activation and the record are in (the first weights too)
    __builtin_amdgcn_sched_barrier(0);
    Bfp8HeadTask task;
    {
        const uint32_t lo[6] = {(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)tw, 0),
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)tw, 1),
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)tw, 2),
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)tw, 3),
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)tw, 4),
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)tw, 5)};
        const uint32_t hw[6] = {(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(tw >> 32), 0),
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(tw >> 32), 1),
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(tw >> 32), 2),
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(tw >> 32), 3),
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(tw >> 32), 4),
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(tw >> 32), 5)};
        uint64_t wd[6];
#pragma unroll
        for (int k = 0; k < 6; ++k) wd[k] = ((uint64_t)hw[k] << 32) | lo[k];
        __builtin_memcpy(&task, wd, sizeof(task));
    }
    // (a global-address-space pointer: a flat load would count on both counters)
    const float tv = ((const __attribute__((address_space(1))) float*)task.x)[lane];

    // 1. the lm_head activation, quantized into LDS: one block per row of 16
    // lanes, four blocks per wavefront
    // (hb passed through an opaque move: left visible, the compiler derived the
    // scale's address from the record's with a 64-bit multiply-add whose
    // unused high half sat in a register a weight load targets, which made the
    // quantization wait for the weights)
    int hbs;
    asm("v_mov_b32 %0, %1" : "=v"(hbs) : "v"(hb));
    bfp8_quant4_store_lds(hv, hi, &L.xsc[hbs], &L.xs[hb * 32], hb < nb);
    // this wavefront's quantization task now too (its element is the one load
    // issued after the wait), so that its stores go out before the tile
    if (wid < a.ntasks) quantize_task(task, tv, lane, L.rec[q]);
    __syncthreads();

    // 2. residue q's split words in registers: lane l holds word l & 7 of
    // block l >> 3 (xr0) and of block 8 + (l >> 3) (xr1), and the scale of block l
    const int xbk = lane >> 3, xw = lane & 7;
    const uint32_t xr0 = xbk < nb ? L.xs[(xbk * 4 + q) * 8 + xw] : 0u;
    const uint32_t xr1 = xbk + 8 < nb ? L.xs[((xbk + 8) * 4 + q) * 8 + xw] : 0u;
    const uint32_t xsv = lane < nb ? __float_as_uint(L.xsc[lane]) : 0u;

    // 3. the tiles
    head_reduce(T, a, t, nb, q, lane, xr0, xr1, xsv, L);
    for (t += gridDim.x; t < a.ntiles; t += gridDim.x) {
        head_issue(T, a, t, nb, q, lane);
        head_reduce(T, a, t, nb, q, lane, xr0, xr1, xsv, L);
    }
    // 4. the quantization tasks beyond one per wavefront (more tasks than
    // wavefronts)
    for (int j = wid + nw; j < a.ntasks; j += nw) {
        const Bfp8HeadTask tj = a.qtasks[j];
        quantize_task(tj, tj.x[lane], lane, L.rec[q]);
    }
}

// Single GEMV, persistent: workgroup w takes tiles w, w + gridDim, ...
// kLanes also writes the int32 residue-lane block sums.
template <bool kLanes>
__global__ __launch_bounds__(256) void bfp8_gemv_kernel(Bfp8GemvDesc d) {
    __shared__ StreamLds L;
    StridedTiles src{&d, (d.M + BFP8_TILE_ROWS - 1) / BFP8_TILE_ROWS};
    stream_tiles<kLanes>(src, L);
}

// Grouped GEMV, persistent: workgroup w walks tiles[wg_off[w] .. wg_off[w+1]).
extern "C" __global__ __launch_bounds__(256) void bfp8_gemv_grouped_kernel(
    const Bfp8GemvDesc* __restrict__ descs, const Bfp8TileRef* __restrict__ tiles,
    const int* __restrict__ wg_off) {
    __shared__ StreamLds L;
    const int beg = wg_off[blockIdx.x];
    TableTiles src{descs, tiles, beg, wg_off[blockIdx.x + 1] - beg};
    stream_tiles<false>(src, L);
}

// The same, with workgroup 0 first merging descs[merge_desc]'s top-k
// partials, written by an earlier launch on the stream.
extern "C" __global__ __launch_bounds__(256) void bfp8_gemv_grouped_merge_kernel(
    const Bfp8GemvDesc* __restrict__ descs, const Bfp8TileRef* __restrict__ tiles,
    const int* __restrict__ wg_off, int merge_desc) {
    __shared__ StreamLds L;
    if (blockIdx.x == 0) topk_merge_folded(topk_args(descs[merge_desc]), L.merge);
    const int beg = wg_off[blockIdx.x];
    TableTiles src{descs, tiles, beg, wg_off[blockIdx.x + 1] - beg};
    stream_tiles<false>(src, L);
}

// Small-M GEMV: one tile per workgroup of 16 wavefronts (dynamic LDS: the
// terms of blocks wide_per(nb) .. nb-1).
template <bool kLanes>
__global__ __launch_bounds__(kWideWaves * 64) void bfp8_gemv_wide_kernel(Bfp8GemvDesc d) {
    extern __shared__ float wide_terms[];
    __shared__ float red[4][64];
    wide_tile<kLanes>(d, blockIdx.x, wide_terms, red);
}

// The same over a tile table spanning several GEMVs (small plans).
extern "C" __global__ __launch_bounds__(kWideWaves * 64) void bfp8_gemv_wide_grouped_kernel(
    const Bfp8GemvDesc* __restrict__ descs, const Bfp8TileRef* __restrict__ tiles) {
    extern __shared__ float wide_terms[];
    __shared__ float red[4][64];
    const Bfp8TileRef tr = tiles[blockIdx.x];
    wide_tile<false>(descs[tr.desc], tr.tile, wide_terms, red);
}

// Stand-alone final top-k merge (one workgroup of 16 wavefronts).  Its
// selection reads the lists' first keys in passes of 256 lists: 4 passes for
// up to kMergeLists lists (a 65,536-row vocabulary), 8 in the wide form (more
// lists take the tree merge).  The shorter form's code is about half as long,
// and the one-workgroup launch runs 0.3-0.4 us faster with it.
constexpr int kMergeLists = 4 * kMergeWaves * 64 / 4;
extern "C" __global__ __launch_bounds__(kMergeWaves * 64) void bfp8_topk_merge_kernel(Bfp8GemvDesc d) {
    __shared__ MergeLds<kMergeWaves> L;
    topk_merge<kMergeWaves, 1, 4, true>(topk_args(d), PlainKeys{}, L);
}
extern "C" __global__ __launch_bounds__(kMergeWaves * 64) void bfp8_topk_merge_wide_kernel(Bfp8GemvDesc d) {
    __shared__ MergeLds<kMergeWaves> L;
    topk_merge<kMergeWaves, 1, 8, true>(topk_args(d), PlainKeys{}, L);
}

// Batched GEMV: B activation vectors against one weight matrix, weights read
// once.  Activations of a chunk of 8 blocks for all B vectors are staged in
// LDS (wave-uniform broadcast reads); each lane keeps B residue accumulators.
template <int B>
__global__ __launch_bounds__(256) void bfp8_gemv_batch_kernel(float* __restrict__ Y,
                                                              const uint32_t* __restrict__ xsplit,
                                                              const float* __restrict__ xscale,
                                                              const uint8_t* __restrict__ mant,
                                                              const uint8_t* __restrict__ exps, int M,
                                                              int K) {
    __shared__ uint32_t xl[B * kBatchChunk * 32];
    __shared__ float xsl[B * kBatchChunk];  // the chunk's block scales (LDS, like the split words: no scalar loads,
                                            // whose out-of-order returns would make every LDS wait a full wait)
    float* red = reinterpret_cast<float*>(xl);  // the cross-wave sums reuse the staging space (4 * 64 * B floats)
    static_assert(kBatchChunk * 32 >= 4 * 64, "red fits in xl");
    const int q = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = threadIdx.x & 63;
    const int t = blockIdx.x;
    const int nb = K >> 6;
    // blockIdx.y: which B vectors of the call (a GEMV with fewer tiles than
    // CUs spreads its vectors over several workgroups per tile)
    Y += (size_t)blockIdx.y * B * M;
    xsplit += (size_t)blockIdx.y * B * nb * 32;
    xscale += (size_t)blockIdx.y * B * nb;
    const int nb4 = (nb + 3) >> 2;
    const uint8_t* mtile = mant + (size_t)t * nb * 4096u;
    const uint8_t* etile = exps + (size_t)t * nb4 * 256u;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(mtile, (uint32_t)nb * 4096u);
    const __amdgpu_buffer_rsrc_t ers = make_rsrc(etile, (uint32_t)nb4 * 256u);
    const int wv = q * 1024 + r * 16;
    const int xwords = nb * 32;
    float fs[B];
#pragma unroll
    for (int v = 0; v < B; ++v) fs[v] = 0.0f;

    for (int b0 = 0; b0 < nb; b0 += kBatchChunk) {
        const int nbc = min(kBatchChunk, nb - b0);
        u32x4 w[kBatchChunk];
        uint32_t ew[kBatchChunk / 4] = {};
#pragma unroll
        for (int u = 0; u < kBatchChunk; ++u)
            if (u < nbc) w[u] = load_w(wrs, wv, (b0 + u) * 4096);
#pragma unroll
        for (int m = 0; m < kBatchChunk / 4; ++m)
            if (4 * m < nbc) ew[m] = load_e(ers, r * 4, ((b0 >> 2) + m) * 256);
        __syncthreads();  // previous chunk's LDS reads are done
        for (int i = threadIdx.x; i < B * nbc * 32; i += 256) {
            int v = i / (nbc * 32), o = i - v * nbc * 32;
            xl[v * kBatchChunk * 32 + o] = xsplit[(size_t)v * xwords + b0 * 32 + o];
        }
        for (int i = threadIdx.x; i < B * nbc; i += 256) {
            const int v = i / nbc, u = i - v * nbc;
            xsl[v * kBatchChunk + u] = xscale[(size_t)v * nb + b0 + u];
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kBatchChunk; ++u) {
            if (u >= nbc) break;
            const uint32_t e = (ew[u >> 2] >> (8 * (u & 3))) & 0xffu;
            const float sc = exp_scale_ftz(e);
            // vectors in groups of four: the group's LDS reads go out together,
            // then its four dot-product chains interleave
            constexpr int kG = B < 4 ? B : 4;
#pragma unroll
            for (int v0 = 0; v0 < B; v0 += kG) {
                uint4 h[kG], l[kG];
                float xs[kG];
#pragma unroll
                for (int j = 0; j < kG; ++j) {
                    const uint32_t* xb = xl + ((v0 + j) * kBatchChunk + u) * 32 + q * 8;
                    h[j] = *reinterpret_cast<const uint4*>(xb);
                    l[j] = *reinterpret_cast<const uint4*>(xb + 4);
                    xs[j] = xsl[(v0 + j) * kBatchChunk + u];
                }
                int acc[kG];
#pragma unroll
                for (int j = 0; j < kG; ++j) acc[j] = __builtin_amdgcn_sdot4((int)w[u].x, (int)h[j].x, 0, false);
#pragma unroll
                for (int j = 0; j < kG; ++j) acc[j] = __builtin_amdgcn_sdot4((int)w[u].y, (int)h[j].y, acc[j], false);
#pragma unroll
                for (int j = 0; j < kG; ++j) acc[j] = __builtin_amdgcn_sdot4((int)w[u].z, (int)h[j].z, acc[j], false);
#pragma unroll
                for (int j = 0; j < kG; ++j) acc[j] = __builtin_amdgcn_sdot4((int)w[u].w, (int)h[j].w, acc[j], false);
#pragma unroll
                for (int j = 0; j < kG; ++j) {
                    acc[j] = (int)((uint32_t)acc[j] << 8);
                    acc[j] = __builtin_amdgcn_sdot4((int)w[u].x, (int)l[j].x, acc[j], false);
                }
#pragma unroll
                for (int j = 0; j < kG; ++j) acc[j] = __builtin_amdgcn_sdot4((int)w[u].y, (int)l[j].y, acc[j], false);
#pragma unroll
                for (int j = 0; j < kG; ++j) acc[j] = __builtin_amdgcn_sdot4((int)w[u].z, (int)l[j].z, acc[j], false);
#pragma unroll
                for (int j = 0; j < kG; ++j) acc[j] = __builtin_amdgcn_sdot4((int)w[u].w, (int)l[j].w, acc[j], false);
#pragma unroll
                for (int j = 0; j < kG; ++j) {
                    const float t1 = (float)acc[j] * sc;
                    const float t2 = t1 * xs[j];
                    fs[v0 + j] = fs[v0 + j] + t2;
                }
            }
        }
    }
    __syncthreads();  // every wavefront is done with the staged activations
#pragma unroll
    for (int v = 0; v < B; ++v) red[(v * 4 + q) * 64 + r] = fs[v];
    __syncthreads();
    const int pair_rows = M & ~1;
    for (int i = threadIdx.x; i < B * 64; i += 256) {
        int v = i >> 6, rr = i & 63;
        int row = t * 64 + rr;
        const float* p = red + v * 256;
        float y = (p[rr] + p[128 + rr]) + (p[64 + rr] + p[192 + rr]);
        if (row < pair_rows) Y[(size_t)v * M + row] = y;
    }
}

// ---- launchers ---------------------------------------------------------------
// Workgroups a persistent kernel keeps resident: all CUs times the kernel's
// occupancy (capped at BFP8_STREAM_WG_PER_CU), queried once per kernel.
static int resident_grid(const void* kernel) {
    int dev = 0, cus = 256, occ = 0;
    if (hipGetDevice(&dev) == hipSuccess) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) == hipSuccess) cus = p.multiProcessorCount;
    }
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, 256, 0) != hipSuccess || occ <= 0) occ = 1;
    return cus * (occ < BFP8_STREAM_WG_PER_CU ? occ : BFP8_STREAM_WG_PER_CU);
}

hipError_t bfp8_probe_code_object() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(bfp8_gemv_grouped_kernel));
}

int bfp8_stream_grid() {
    static const int a = resident_grid(reinterpret_cast<const void*>(bfp8_gemv_grouped_kernel));
    static const int b = resident_grid(reinterpret_cast<const void*>(bfp8_gemv_grouped_merge_kernel));
    return a < b ? a : b;
}

static size_t wide_lds_bytes(int max_nb) {
    const int rest = max_nb - wide_per(max_nb);
    return (size_t)(rest > 0 ? rest : 1) * 4 * 64 * sizeof(float);
}

hipError_t bfp8_launch_gemv(const Bfp8GemvDesc& d, hipStream_t s) {
    const int nt = bfp8_ntiles(d.M);
    if (nt == 0) return hipSuccess;
    if (d.topk <= 0 && nt <= BFP8_WIDE_MAX_TILES && !d.lanes && d.K <= RT_ROWS_MAX_K) {
        // few row tiles: 16 rows per workgroup (fused_gemv.hip)
        RtRowsArgs a{};
        a.g[0].mant = d.mant;
        a.g[0].exps = d.exps;
        a.g[0].y = d.y;
        a.g[0].M = d.M;
        a.g[0].pair_rows = d.pair_rows;
        a.ngemv = 1;
        a.split = (d.M + 15) / 16;
        a.K = d.K;
        a.mode = RT_ROWS_QUANTIZED;
        a.xsplit = d.xsplit;
        a.xscale = d.xscale;
        return rt_launch_rows(a, s);
    }
    if (d.topk <= 0 && nt <= BFP8_WIDE_MAX_TILES) {
        const size_t lds = wide_lds_bytes(d.K >> 6);
        if (d.lanes)
            hipLaunchKernelGGL(bfp8_gemv_wide_kernel<true>, dim3(nt), dim3(kWideWaves * 64), lds, s, d);
        else
            hipLaunchKernelGGL(bfp8_gemv_wide_kernel<false>, dim3(nt), dim3(kWideWaves * 64), lds, s, d);
        return hipGetLastError();
    }
    static const int g_plain = resident_grid(reinterpret_cast<const void*>(bfp8_gemv_kernel<false>));
    static const int g_lanes = resident_grid(reinterpret_cast<const void*>(bfp8_gemv_kernel<true>));
    const int cap = d.lanes ? g_lanes : g_plain;
    const int grid = nt < cap ? nt : cap;
    if (d.lanes)
        hipLaunchKernelGGL(bfp8_gemv_kernel<true>, dim3(grid), dim3(256), 0, s, d);
    else
        hipLaunchKernelGGL(bfp8_gemv_kernel<false>, dim3(grid), dim3(256), 0, s, d);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || d.topk <= 0) return e;
    return bfp8_launch_topk_merge(d, s);
}

const char* bfp8_topk_merge_kernel_name(int M) {
    return bfp8_ntiles(M) <= kMergeLists ? "bfp8_topk_merge_kernel" : "bfp8_topk_merge_wide_kernel";
}

hipError_t bfp8_launch_topk_merge(const Bfp8GemvDesc& d, hipStream_t s) {
    if (bfp8_ntiles(d.M) <= kMergeLists)
        hipLaunchKernelGGL(bfp8_topk_merge_kernel, dim3(1), dim3(kMergeWaves * 64), 0, s, d);
    else
        hipLaunchKernelGGL(bfp8_topk_merge_wide_kernel, dim3(1), dim3(kMergeWaves * 64), 0, s, d);
    return hipGetLastError();
}

hipError_t bfp8_launch_gemv_grouped(const Bfp8GemvDesc* descs_dev, const Bfp8TileRef* tiles_dev,
                                    const int* wg_off_dev, int nwg, int merge_desc, hipStream_t s) {
    if (nwg <= 0) return hipSuccess;
    if (merge_desc >= 0)
        hipLaunchKernelGGL(bfp8_gemv_grouped_merge_kernel, dim3(nwg), dim3(256), 0, s, descs_dev, tiles_dev,
                           wg_off_dev, merge_desc);
    else
        hipLaunchKernelGGL(bfp8_gemv_grouped_kernel, dim3(nwg), dim3(256), 0, s, descs_dev, tiles_dev,
                           wg_off_dev);
    return hipGetLastError();
}

hipError_t bfp8_launch_gemv_head(const Bfp8HeadArgs& a, int nwg, hipStream_t s) {
    if (nwg <= 0 || a.ntiles < nwg) return nwg <= 0 ? hipSuccess : hipErrorInvalidValue;
    hipLaunchKernelGGL(bfp8_gemv_head_kernel, dim3(nwg), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t bfp8_launch_gemv_wide_grouped(const Bfp8GemvDesc* descs_dev, const Bfp8TileRef* tiles_dev, int ntiles,
                                         int max_nb, hipStream_t s) {
    if (ntiles <= 0) return hipSuccess;
    hipLaunchKernelGGL(bfp8_gemv_wide_grouped_kernel, dim3(ntiles), dim3(kWideWaves * 64), wide_lds_bytes(max_nb), s,
                       descs_dev, tiles_dev);
    return hipGetLastError();
}

template <int B>
static hipError_t launch_batch_t(float* Y, const uint32_t* xsplit, const float* xscale,
                                 const uint8_t* mant, const uint8_t* exps, int M, int K, int groups,
                                 hipStream_t s) {
    hipLaunchKernelGGL(bfp8_gemv_batch_kernel<B>, dim3(bfp8_ntiles(M), groups), dim3(256), 0, s, Y, xsplit,
                       xscale, mant, exps, M, K);
    return hipGetLastError();
}

static int cu_count() {
    static const int n = [] {
        int dev = 0, cus = 256;
        hipDeviceProp_t p;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess) cus = p.multiProcessorCount;
        return cus;
    }();
    return n;
}

// One launch of the dot-product kernel for B in {1, 2, 4}.
static hipError_t launch_batch_pow2(float* Y, const uint32_t* xsplit, const float* xscale, const uint8_t* mant,
                                    const uint8_t* exps, int M, int K, int B, hipStream_t s) {
    const int nt = bfp8_ntiles(M);
    // while the tiles leave CUs idle, split the vectors over more workgroups
    // (each re-reads its tile's weights, from L2 / MALL for such small GEMVs)
    int groups = 1;
    while (groups * 2 <= B && nt * groups * 2 <= cu_count()) groups *= 2;
    switch (B / groups) {
        case 1: return launch_batch_t<1>(Y, xsplit, xscale, mant, exps, M, K, groups, s);
        case 2: return launch_batch_t<2>(Y, xsplit, xscale, mant, exps, M, K, groups, s);
        default: return launch_batch_t<4>(Y, xsplit, xscale, mant, exps, M, K, groups, s);
    }
}

hipError_t bfp8_launch_gemv_batch(float* Y, const uint32_t* xsplit, const float* xscale,
                                  const uint8_t* mant, const uint8_t* exps, int M, int K, int B,
                                  hipStream_t s) {
    if (bfp8_ntiles(M) == 0) return hipSuccess;
    if (B < 1 || B > 16) return hipErrorInvalidValue;
    // from 8 vectors on, the matrix cores: their epilogue costs the same for
    // 8 and for 16 vectors, the dot-product kernel's grows with B
    if (B >= 8) return bfp8_launch_gemv_batch_mfma(Y, xsplit, xscale, mant, exps, M, K, B, s);
    const int nb = K >> 6;
    int done = 0;
    while (done < B) {
        int step = 4;
        while (step > B - done) step >>= 1;
        const hipError_t e = launch_batch_pow2(Y + (size_t)done * M, xsplit + (size_t)done * nb * 32,
                                               xscale + (size_t)done * nb, mant, exps, M, K, step, s);
        if (e != hipSuccess) return e;
        done += step;
    }
    return hipSuccess;
}
