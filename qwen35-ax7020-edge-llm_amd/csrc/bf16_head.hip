// bf16_head.hip -- the reference's tied-embedding lm_head on gfx950: every row
// of the bf16 embedding table dotted with the final hidden state, fused with
// the greedy argmax / streaming top-k selection.
//
// Compiled with -fgpu-flush-denormals-to-zero -ffp-contract=off, like
// bfp8_ftz.hip: the reference's board build computes the dot products with
// Advanced SIMD (flush-to-zero, vmlaq_f32 = rounded product then rounded sum).
//
// Reference arithmetic restated per row (04/qwen_kernels_opt.c:417-457,
// 04/qwen_sampling.c:161-245):
//   for each 8-element chunk c:  a[j] = a[j] + bf16(w[8c+j]) * h[8c+j]  (j = 0..7;
//                                 a[0..3] is accumulator a0, a[4..7] is a1)
//   acc[j] = a[j] + a[4+j];  score = (acc[0] + acc[2]) + (acc[1] + acc[3])
//   hidden % 8 trailing elements: dropped by lm_head_argmax, added one by one
//   by lm_head_topk (its scalar VFP tail: IEEE subnormals, product rounded
//   then sum rounded, 04/qwen_sampling.c:201-204).
//
// Work mapping: a persistent workgroup of 4 wavefronts walks 64-row tiles;
// wavefront w owns rows 16w..16w+15 of each tile.  A tile is streamed in
// slices of up to 32 chunks (512 B) per row by direct-to-LDS loads (one
// half-wavefront load per row slice, so every LDS row gets a padded,
// conflict-free pitch) into four LDS buffers, three slices in flight while
// the fourth is reduced.  A wavefront only reads the rows it loaded itself,
// so it waits on its own load counter and the stream needs no workgroup
// barrier.  Lane (row r, group g) keeps accumulators a[g] and a[g+4] of its
// row: every chain still adds its chunks in order, a[g] + a[g+4] is formed
// in the lane, and the two cross-lane steps of the final combine are quad
// DPP exchanges.  The hidden state sits in LDS as pairs (h[8c+g], h[8c+4+g])
// per group.  Each tile's 64 keys are sorted in wavefront 0 and its best
// `topk` published as the tile's partial list; the stand-alone merge kernel
// of bfp8_ftz.hip selects the final top-k and the argmax from those lists.
#include <hip/hip_runtime.h>

#include "bfp8_internal.h"
#include "ieee_dev.h"
#include "wave_topk.h"

namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kSlice = 32;                   // 16-byte chunks per row slice (512 B)
constexpr int kPitch = kSlice * 16 + 16;     // LDS row pitch: 16 rows of a wave hit distinct banks
constexpr int kRows = BFP8_TILE_ROWS;        // rows per tile
constexpr int kWaveRows = kRows / 4;         // rows per wavefront
constexpr int kThreads = 256;
constexpr int kBufs = 4;                     // LDS slice buffers (3 in flight + 1 reduced)
constexpr int kBufBytes = kRows * kPitch;
constexpr int kMaxHidden = BF16_HEAD_MAX_HIDDEN;

// Dynamic LDS: kBufs slice buffers, the 64 tile scores, then the hidden-state
// pairs hpair[g][c] = (h[8c+g], h[8c+4+g]) (4 * hidden bytes * 2).
constexpr int kScoreOff = kBufs * kBufBytes;
constexpr int kPairOff = kScoreOff + kRows * 4;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

struct Unit {
    int tile, slice;
};

__device__ __forceinline__ void next_unit(Unit& u, int nslices) {
    if (++u.slice == nslices) {
        u.slice = 0;
        u.tile += gridDim.x;
    }
}

// This wavefront's 16 row slices of unit u into LDS buffer `buf`: one
// half-wavefront load per row (lanes 0..31 carry 16 B each, lanes below the
// slice's chunk count).  Rows past the vocabulary re-load the tile's last
// row so that every unit issues exactly kWaveRows loads per wavefront (the
// wait below counts them).
__device__ __forceinline__ void issue(uint8_t* buf, const Bf16HeadDesc& d, Unit u, int nch, int w, int lane) {
    const int row0 = u.tile * kRows;
    const int rows = min(kRows, d.vocab - row0);
    const uint32_t rowbytes = (uint32_t)d.hidden * 2u;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(d.table + (size_t)row0 * d.hidden, (uint32_t)rows * rowbytes);
    const int c0 = u.slice * kSlice;
    const int sc = min(kSlice, nch - c0);
#pragma unroll
    for (int rr = 0; rr < kWaveRows; ++rr) {
        const int row = kWaveRows * w + rr;
        const int src = row < rows ? row : rows - 1;
        if (lane < sc)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(buf + row * kPitch),
                                                     16, (int)(src * rowbytes) + (c0 + lane) * 16, 0, 0, 0);
    }
}

// Workgroup barrier for the tile's score array: this wavefront's LDS stores
// complete first (lgkmcnt 0), but direct-to-LDS loads still in flight are
// not waited for (a __syncthreads() fence would drain them: they count as
// LDS writes); they target slots that only their own wavefront reads.  The
// signal fences keep the compiler from moving memory accesses across.
__device__ __forceinline__ void score_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Wait until at most `later` units' loads of this wavefront are pending.
__device__ __forceinline__ void wait_units(int later) {
    switch (later) {  // vmcnt = later * kWaveRows (gfx9 encoding, expcnt/lgkmcnt left alone)
        case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
        case 1: __builtin_amdgcn_s_waitcnt(0x0F70 | (16 & 15) | ((16 >> 4) << 14)); break;
        case 2: __builtin_amdgcn_s_waitcnt(0x0F70 | (32 & 15) | ((32 >> 4) << 14)); break;
        default: __builtin_amdgcn_s_waitcnt(0x0F70 | (48 & 15) | ((48 >> 4) << 14)); break;
    }
}

}  // namespace

// Persistent: workgroup b takes tiles b, b + gridDim, ...; kTail adds the
// hidden % 8 trailing elements (lm_head_topk's scalar tail).  kHGlobal: h is
// read from global memory at every chunk instead of an LDS copy of its pairs
// (hidden sizes whose copy would not fit beside the slice buffers).
template <bool kTail, bool kHGlobal>
__global__ __launch_bounds__(kThreads) void bf16_lm_head_kernel(Bf16HeadDesc d) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    float* score = reinterpret_cast<float*>(lds_raw + kScoreOff);
    u32x2* hpair = reinterpret_cast<u32x2*>(lds_raw + kPairOff);
    const int ntiles = (d.vocab + kRows - 1) / kRows;
    const int nch = d.hidden >> 3;
    const int nslices = nch > 0 ? (nch + kSlice - 1) / kSlice : 1;
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r = lane >> 2, g = lane & 3;
    const int trow = kWaveRows * w + r;  // this lane's row within the tile
    if (!kHGlobal) {
        for (int i = threadIdx.x; i < 4 * nch; i += kThreads) {
            const int gg = i / nch, c = i % nch;
            u32x2 v;
            v.x = __float_as_uint(d.h[8 * c + gg]);
            v.y = __float_as_uint(d.h[8 * c + 4 + gg]);
            hpair[gg * nch + c] = v;
        }
    }
    __syncthreads();
    if ((int)blockIdx.x >= ntiles) return;  // uniform per workgroup
    const int units = ((ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x) * nslices;
    const int sh = (g & 1) ? 0 : 16;  // element g of a dword: high half when g is odd
    const int dw = g >> 1;            // dword of element g (element g + 4: dword 2 + g/2)
    const u32x2* hp_g = hpair + g * nch;
    Unit u{(int)blockIdx.x, 0}, ahead = u;
    int issued = 0;
    for (; issued < kBufs - 1 && issued < units; ++issued) {
        issue(lds_raw + (issued % kBufs) * kBufBytes, d, ahead, nch, w, lane);
        next_unit(ahead, nslices);
    }
    float a0 = 0.0f, a1 = 0.0f;  // a[g], a[g+4]
    for (int n = 0; n < units; ++n) {
        if (issued < units) {  // refill the buffer reduced in the previous step
            issue(lds_raw + (issued % kBufs) * kBufBytes, d, ahead, nch, w, lane);
            next_unit(ahead, nslices);
            ++issued;
        }
        wait_units(issued - n - 1);
        const uint8_t* rowp = lds_raw + (n % kBufs) * kBufBytes + trow * kPitch;
        const int c0 = u.slice * kSlice;
        const int sc = min(kSlice, nch - c0);
        for (int ch = 0; ch < sc; ++ch) {
            const uint32_t lo = *reinterpret_cast<const uint32_t*>(rowp + ch * 16 + dw * 4);
            const uint32_t hi = *reinterpret_cast<const uint32_t*>(rowp + ch * 16 + 8 + dw * 4);
            u32x2 hp;
            if (kHGlobal) {
                hp.x = __float_as_uint(d.h[8 * (c0 + ch) + g]);
                hp.y = __float_as_uint(d.h[8 * (c0 + ch) + 4 + g]);
            } else {
                hp = hp_g[c0 + ch];
            }
            a0 = a0 + __uint_as_float((lo << sh) & 0xFFFF0000u) * __uint_as_float(hp.x);
            a1 = a1 + __uint_as_float((hi << sh) & 0xFFFF0000u) * __uint_as_float(hp.y);
        }
        if (u.slice == nslices - 1) {  // tile done: combine, select, publish
            const int row0 = u.tile * kRows;
            const int rows = min(kRows, d.vocab - row0);
            const float acc = a0 + a1;  // acc[g]
            const float x = acc + __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(
                                      0, (int)__float_as_uint(acc), 0x4E, 0xF, 0xF, false));  // + acc[g^2]
            float sc_row = x + __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(
                                   0, (int)__float_as_uint(x), 0xB1, 0xF, 0xF, false));  // (acc0+acc2)+(acc1+acc3)
            if (kTail && g == 0 && trow < rows) {
                const uint16_t* wr = d.table + (size_t)(row0 + trow) * d.hidden;
                for (int i = nch * 8; i < d.hidden; ++i)
                    sc_row = ieee_add(sc_row, ieee_mul(d.h[i], __uint_as_float((uint32_t)wr[i] << 16)));
            }
            if (g == 0) {
                score[trow] = sc_row;
                if (d.logits && trow < rows) d.logits[row0 + trow] = sc_row;
            }
            a0 = a1 = 0.0f;
            if (d.topk > 0) {
                score_barrier();
                if (w == 0) {
                    uint64_t key[1] = {lane < rows ? topk_key(score[lane], row0 + lane) : 0ull};
                    const bool desc[1] = {true};
                    wave_sort<1>(key, desc, lane);
                    if (lane < d.topk) d.partials[(size_t)u.tile * d.topk + lane] = key[0];
                }
                score_barrier();  // score[] is rewritten by the next tile
            }
        }
        next_unit(u, nslices);
    }
}

// ---- the tile layout (hidden == 1024) ---------------------------------------------------
// Rows in groups of 16 (group T = rows 16T .. 16T+15, groups padded with zero
// rows to whole 64-row tiles: nT = 4 * ceil(vocab / 64)).  For row 16T + r and
// element e = 8c + j (chunk c = 4q + cc, quad q = 2p + s, j = 4 hi + g):
// 16-byte slot ((p * nT + T) * 2 + s) * 64 + 4r + g, 4-byte word cc, bf16
// half hi.  So lane 4r + g of the wavefront that owns group T reads one
// contiguous 2 KiB run per quad pair p (two 1 KiB loads) and finds in each
// word the two elements of its accumulator chains a[g] (hi 0) and a[g+4]
// (hi 1) for chunk 4q + cc; and pair p of all groups is one contiguous
// 2 nT KiB run, so the wavefronts, which advance through the pairs
// together, read one dense region at a time.
//
// Each wavefront keeps only one pair (2 KiB) in flight and four wavefronts
// share a SIMD: sweeps over loads per batch (1-16), batches in flight (1-8),
// run length (1-8 quads) and the non-temporal hint settled on this point
// (20.7 us for 65536 x 1024, against 27.8 us with 16 KiB per wavefront in
// flight): fewer outstanding requests, each from a denser region, keep the
// HBM stream closer to sequential.
constexpr int kGrpRows = 16;    // rows per wavefront
constexpr int kQuadLoads = 2;   // 16-byte loads per lane per batch
constexpr int kBatchBufs = 1;   // batches in flight per wavefront
constexpr int kQuads = 1024 / 32;
constexpr int kRunLog2 = 1;     // 2^kRunLog2 consecutive quads of a group are adjacent
constexpr int kBatches = kQuads / kQuadLoads;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The batch's loads (quads q0 .. q0 + kQuadLoads - 1), issued in order by
// inline assembly so that no compiler pass moves or merges them; non-temporal
// (the table is streamed once).
template <int Q0, int K>
__device__ __forceinline__ void grp_issue(u32x4 (&v)[kQuadLoads], uint64_t base, uint64_t rstride, uint32_t vo) {
    if constexpr (K < kQuadLoads) {
        constexpr int q = Q0 + K;
        asm volatile("global_load_dwordx4 %0, %1, %2 nt"
                     : "=v"(v[K])
                     : "v"(vo), "s"(base + (uint64_t)(q >> kRunLog2) * rstride + (uint64_t)((q & ((1 << kRunLog2) - 1)) * 1024))
                     : "memory");
        grp_issue<Q0, K + 1>(v, base, rstride, vo);
    }
}

// Reduce a batch whose loads were followed by kLater other loads: quad k
// waits until at most kLater + kQuadLoads - 1 - k loads are pending (loads
// complete in issue order).  The wait takes the quad's register and both
// accumulators as in/out operands, so the quad's products are formed after
// its wait and before the next one.  hq: this lane's h pairs, 8 floats per
// quad (h[8c + g], h[8c + 4 + g]) for c = 4q .. 4q + 3.
template <int kLater, int K>
__device__ __forceinline__ void grp_reduce(float& a0, float& a1, u32x4 (&v)[kQuadLoads], const float4* hq, int q0) {
    if constexpr (K < kQuadLoads) {
        asm volatile("s_waitcnt vmcnt(%3)" : "+v"(v[K]), "+v"(a0), "+v"(a1) : "n"(kLater + kQuadLoads - 1 - K));
        const float4 p0 = hq[(q0 + K) * 8];
        const float4 p1 = hq[(q0 + K) * 8 + 1];
        const uint32_t wd[4] = {v[K].x, v[K].y, v[K].z, v[K].w};
        const float hl[4] = {p0.x, p0.z, p1.x, p1.z}, hh[4] = {p0.y, p0.w, p1.y, p1.w};
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            a0 = a0 + __uint_as_float(wd[cc] << 16) * hl[cc];
            a1 = a1 + __uint_as_float(wd[cc] & 0xFFFF0000u) * hh[cc];
        }
        grp_reduce<kLater, K + 1>(a0, a1, v, hq, q0);
    }
}

template <int b>
__device__ __forceinline__ void grp_first(u32x4 (&V)[kBatchBufs][kQuadLoads], uint64_t base, uint64_t rstride,
                                          uint32_t vo) {
    if constexpr (b < kBatchBufs) {
        grp_issue<b * kQuadLoads, 0>(V[b], base, rstride, vo);
        grp_first<b + 1>(V, base, rstride, vo);
    }
}

// Batch b (in buffer b % kBatchBufs) is reduced while the batches after it,
// up to kBatchBufs - 1 of them, are in flight; then the buffer is refilled
// with batch b + kBatchBufs.
template <int b>
__device__ __forceinline__ void grp_pipe(float& a0, float& a1, u32x4 (&V)[kBatchBufs][kQuadLoads], const float4* hq,
                                         uint64_t base, uint64_t rstride, uint32_t vo) {
    if constexpr (b < kBatches) {
        constexpr int last = b + kBatchBufs - 1 < kBatches - 1 ? b + kBatchBufs - 1 : kBatches - 1;
        grp_reduce<kQuadLoads * (last - b), 0>(a0, a1, V[b % kBatchBufs], hq, b * kQuadLoads);
        if constexpr (b + kBatchBufs < kBatches)
            grp_issue<(b + kBatchBufs) * kQuadLoads, 0>(V[b % kBatchBufs], base, rstride, vo);
        grp_pipe<b + 1>(a0, a1, V, hq, base, rstride, vo);
    }
}

// One 64-row tile per workgroup, wavefront w owns group 4 * tile + w.
__global__ __launch_bounds__(kThreads) void bf16_lm_head_tiles_kernel(Bf16HeadDesc d) {
    __shared__ __align__(16) float hqs[kQuads * 4 * 8];  // [q][g][cc][hi]
    __shared__ float score[kRows];
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int tile = blockIdx.x;
    const int nT = 4 * (int)gridDim.x;
    const uint64_t rstride = (uint64_t)nT * (1024u << kRunLog2);  // bytes from one run of quads to the next
    const uint32_t vo = (uint32_t)(4 * tile + w) * (1024u << kRunLog2) + (uint32_t)lane * 16u;
    const uint64_t base = (uint64_t)d.table;
    // h (4 KiB) first: thread i loads h[4i .. 4i + 3]; then the first batches
    u32x4 hv;
    asm volatile("global_load_dwordx4 %0, %1, %2 nt" : "=v"(hv) : "v"((uint32_t)threadIdx.x * 16u), "s"((uint64_t)d.h)
                 : "memory");
    u32x4 V[kBatchBufs][kQuadLoads];
    grp_first<0>(V, base, rstride, vo);
    asm volatile("s_waitcnt vmcnt(%1)" : "+v"(hv) : "n"(kBatchBufs * kQuadLoads));
    {   // elements 4i .. 4i+3 = chunk i/2, half i%2, g = 0..3
        const int c = threadIdx.x >> 1, hi = threadIdx.x & 1;
        float* dst = hqs + (((c >> 2) * 4) * 4 + (c & 3)) * 2 + hi;
        dst[0] = __uint_as_float(hv.x);
        dst[8] = __uint_as_float(hv.y);
        dst[16] = __uint_as_float(hv.z);
        dst[24] = __uint_as_float(hv.w);
    }
    score_barrier();
    const float4* hq = reinterpret_cast<const float4*>(hqs) + (lane & 3) * 2;
    float a0 = 0.0f, a1 = 0.0f;  // a[g], a[g + 4]
    grp_pipe<0>(a0, a1, V, hq, base, rstride, vo);
    // acc[g] = a[g] + a[g+4]; score = (acc0 + acc2) + (acc1 + acc3) by quad DPP
    const float acc = a0 + a1;
    const float x = acc + __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(acc), 0x4E, 0xF,
                                                                                  0xF, false));
    const float sc_row = x + __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(x), 0xB1, 0xF,
                                                                                     0xF, false));
    const int row0 = tile * kRows;
    const int rows = min(kRows, d.vocab - row0);
    const int trow = kGrpRows * w + (lane >> 2);
    if ((lane & 3) == 0) {
        score[trow] = sc_row;
        if (d.logits && trow < rows) d.logits[row0 + trow] = sc_row;
    }
    if (d.topk > 0) {
        score_barrier();
        if (w == 0) {
            uint64_t key[1] = {lane < rows ? topk_key(score[lane], row0 + lane) : 0ull};
            const bool desc[1] = {true};
            wave_sort<1>(key, desc, lane);
            if (lane < d.topk) d.partials[(size_t)tile * d.topk + lane] = key[0];
        }
    }
}

// Row-major [vocab][hidden] -> the tile layout: one thread per 16-byte slot.
__global__ __launch_bounds__(256) void bf16_tile_table_kernel(u32x4* __restrict__ dst, const uint16_t* __restrict__ src,
                                                              int vocab, int hidden) {
    const size_t nT = (size_t)4 * ((vocab + kRows - 1) / kRows);
    const size_t total = nT * (size_t)(hidden / 32) * 64;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        // slot i = (((q >> kRunLog2) * nT + T) << kRunLog2 | q % 2^kRunLog2) * 64 + 4r + g
        const int g = (int)(i & 3), r = (int)((i >> 2) & 15);
        const size_t run = i >> 6;
        const size_t pT = run >> kRunLog2;
        const int q = (int)((pT / nT) << kRunLog2) + (int)(run & ((1u << kRunLog2) - 1));
        const int row = (int)(pT % nT) * kGrpRows + r;
        uint32_t wd[4] = {0u, 0u, 0u, 0u};
        if (row < vocab) {
            const uint16_t* sp = src + (size_t)row * hidden + 32 * q + g;
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) wd[cc] = (uint32_t)sp[8 * cc] | ((uint32_t)sp[8 * cc + 4] << 16);
        }
        dst[i] = u32x4{wd[0], wd[1], wd[2], wd[3]};
    }
}

// One resident workgroup per CU (the LDS copy takes most of a CU's LDS).
static size_t head_lds_bytes(int hidden) {
    return (size_t)kPairOff + (hidden > kMaxHidden ? (size_t)0 : (size_t)4 * (hidden >> 3) * 8);
}

static int head_grid(const void* kernel) {
    const int most = (int)head_lds_bytes(kMaxHidden);
    static const bool attr_ok =
        hipFuncSetAttribute(reinterpret_cast<const void*>(bf16_lm_head_kernel<false, false>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, most) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(bf16_lm_head_kernel<true, false>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, most) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(bf16_lm_head_kernel<false, true>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, most) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(bf16_lm_head_kernel<true, true>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, most) == hipSuccess;
    (void)kernel;
    if (!attr_ok) return 0;
    int dev = 0, cus = 256;
    hipDeviceProp_t p;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess) cus = p.multiProcessorCount;
    return cus;
}

hipError_t bf16_launch_lm_head(const Bf16HeadDesc& d, hipStream_t s) {
    const int ntiles = (d.vocab + kRows - 1) / kRows;
    if (ntiles <= 0) return hipSuccess;
    static const int cap = head_grid(nullptr);
    if (cap <= 0) return hipErrorInvalidConfiguration;
    if (d.tiled) {  // one 64-row tile per workgroup
        if (!bf16_tiled_ok(d.hidden)) return hipErrorInvalidValue;
        hipLaunchKernelGGL(bf16_lm_head_tiles_kernel, dim3(ntiles), dim3(kThreads), 0, s, d);
        return hipGetLastError();
    }
    const int grid = ntiles < cap ? ntiles : cap;
    const size_t lds = head_lds_bytes(d.hidden);
    const bool tail = d.tail && (d.hidden & 7), hg = d.hidden > kMaxHidden;
    if (tail && hg)
        hipLaunchKernelGGL((bf16_lm_head_kernel<true, true>), dim3(grid), dim3(kThreads), lds, s, d);
    else if (tail)
        hipLaunchKernelGGL((bf16_lm_head_kernel<true, false>), dim3(grid), dim3(kThreads), lds, s, d);
    else if (hg)
        hipLaunchKernelGGL((bf16_lm_head_kernel<false, true>), dim3(grid), dim3(kThreads), lds, s, d);
    else
        hipLaunchKernelGGL((bf16_lm_head_kernel<false, false>), dim3(grid), dim3(kThreads), lds, s, d);
    return hipGetLastError();
}

bool bf16_tiled_ok(int hidden) { return hidden == 32 * kQuads; }

size_t bf16_tiled_elems(int vocab, int hidden) {
    return (size_t)((vocab + kRows - 1) / kRows) * (size_t)kRows * (size_t)hidden;
}

hipError_t bf16_launch_tile_table(uint16_t* dst, const uint16_t* src, int vocab, int hidden, hipStream_t s) {
    if (vocab <= 0 || hidden <= 0) return hipSuccess;
    if (!bf16_tiled_ok(hidden)) return hipErrorInvalidValue;
    const size_t chunks = bf16_tiled_elems(vocab, hidden) / 8;
    const unsigned blocks = (unsigned)std::min<size_t>((chunks + 255) / 256, 65536);
    hipLaunchKernelGGL(bf16_tile_table_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<u32x4*>(dst), src,
                       vocab, hidden);
    return hipGetLastError();
}
