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
//   by lm_head_topk (its scalar tail; here in flush-to-zero arithmetic).
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
// hidden % 8 trailing elements (lm_head_topk's scalar tail).
template <bool kTail>
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
    for (int i = threadIdx.x; i < 4 * nch; i += kThreads) {
        const int gg = i / nch, c = i % nch;
        u32x2 v;
        v.x = __float_as_uint(d.h[8 * c + gg]);
        v.y = __float_as_uint(d.h[8 * c + 4 + gg]);
        hpair[gg * nch + c] = v;
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
            const u32x2 hp = hp_g[c0 + ch];
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
                for (int i = nch * 8; i < d.hidden; ++i) sc_row = sc_row + d.h[i] * __uint_as_float((uint32_t)wr[i] << 16);
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

// One resident workgroup per CU (the LDS copy takes most of a CU's LDS).
static size_t head_lds_bytes(int hidden) { return (size_t)kPairOff + (size_t)4 * (hidden >> 3) * 8; }

static int head_grid(const void* kernel) {
    const int most = (int)head_lds_bytes(kMaxHidden);
    static const bool attr_ok =
        hipFuncSetAttribute(reinterpret_cast<const void*>(bf16_lm_head_kernel<false>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, most) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(bf16_lm_head_kernel<true>),
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
    if (d.hidden > kMaxHidden) return hipErrorInvalidValue;
    static const int cap = head_grid(nullptr);
    if (cap <= 0) return hipErrorInvalidConfiguration;
    const int grid = ntiles < cap ? ntiles : cap;
    const size_t lds = head_lds_bytes(d.hidden);
    if (d.tail && (d.hidden & 7))
        hipLaunchKernelGGL(bf16_lm_head_kernel<true>, dim3(grid), dim3(kThreads), lds, s, d);
    else
        hipLaunchKernelGGL(bf16_lm_head_kernel<false>, dim3(grid), dim3(kThreads), lds, s, d);
    return hipGetLastError();
}
