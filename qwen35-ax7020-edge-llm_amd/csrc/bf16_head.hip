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
// Work mapping: one wavefront owns a tile of 64 rows, lane = row, so each
// lane keeps the eight sequential accumulators of its row in registers (the
// reference's chain order needs no cross-lane step).  A lane streams its row
// as 16-byte chunks, eight chunks per load group, double-buffered; the hidden
// state is read with scalar loads (wave-uniform).  The tile's 64 keys are
// sorted in the wavefront and its best `topk` published as the tile's partial
// list; the stand-alone merge kernel of bfp8_ftz.hip selects the final top-k
// and the argmax from those lists.
#include <hip/hip_runtime.h>

#include "bfp8_internal.h"
#include "wave_topk.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(4))) float* sgpr_f32_ptr;

constexpr int kGroup = 8;  // 16-byte chunks per load group (128 B per lane)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// The table is streamed once: non-temporal loads.
__device__ __forceinline__ u32x4 load_chunk(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 2));
}

// bf16 -> f32: the bf16 bits are the float's high half (little-endian: the
// element at the lower address is the dword's low half).
__device__ __forceinline__ float bf_lo(uint32_t d) { return __uint_as_float(d << 16); }
__device__ __forceinline__ float bf_hi(uint32_t d) { return __uint_as_float(d & 0xFFFF0000u); }

// One chunk into the eight accumulators (product rounded, then sum rounded).
__device__ __forceinline__ void accumulate(float (&a)[8], u32x4 v, sgpr_f32_ptr hc) {
    a[0] = a[0] + bf_lo(v.x) * hc[0];
    a[1] = a[1] + bf_hi(v.x) * hc[1];
    a[2] = a[2] + bf_lo(v.y) * hc[2];
    a[3] = a[3] + bf_hi(v.y) * hc[3];
    a[4] = a[4] + bf_lo(v.z) * hc[4];
    a[5] = a[5] + bf_hi(v.z) * hc[5];
    a[6] = a[6] + bf_lo(v.w) * hc[6];
    a[7] = a[7] + bf_hi(v.w) * hc[7];
}

__device__ __forceinline__ void issue(u32x4 (&buf)[kGroup], __amdgpu_buffer_rsrc_t rs, int voff, int c0, int nch) {
    if (c0 + kGroup <= nch) {
#pragma unroll
        for (int u = 0; u < kGroup; ++u) buf[u] = load_chunk(rs, voff, (c0 + u) * 16);
    } else {
#pragma unroll
        for (int u = 0; u < kGroup; ++u)
            if (c0 + u < nch) buf[u] = load_chunk(rs, voff, (c0 + u) * 16);
    }
}

__device__ __forceinline__ void consume(float (&a)[8], const u32x4 (&buf)[kGroup], const float* h, int c0, int nch) {
    if (c0 + kGroup <= nch) {
#pragma unroll
        for (int u = 0; u < kGroup; ++u) accumulate(a, buf[u], (sgpr_f32_ptr)h + (c0 + u) * 8);
    } else {
#pragma unroll
        for (int u = 0; u < kGroup; ++u)
            if (c0 + u < nch) accumulate(a, buf[u], (sgpr_f32_ptr)h + (c0 + u) * 8);
    }
}

}  // namespace

// One wavefront per 64-row tile; kTail adds the hidden % 8 trailing elements.
template <bool kTail>
__global__ __launch_bounds__(256) void bf16_lm_head_kernel(Bf16HeadDesc d) {
    const int tile = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int ntiles = (d.vocab + BFP8_TILE_ROWS - 1) / BFP8_TILE_ROWS;
    if (tile >= ntiles) return;  // no workgroup barrier follows
    const int row0 = tile * BFP8_TILE_ROWS;
    const int rows = min(BFP8_TILE_ROWS, d.vocab - row0);
    const uint32_t rowbytes = (uint32_t)d.hidden * 2u;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(d.table + (size_t)row0 * d.hidden, (uint32_t)rows * rowbytes);
    const int voff = lane * (int)rowbytes;
    const int nch = d.hidden >> 3;
    float a[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 A[kGroup], B[kGroup];
    issue(A, rs, voff, 0, nch);
    for (int c = 0; c < nch; c += 2 * kGroup) {
        if (c + kGroup < nch) issue(B, rs, voff, c + kGroup, nch);
        consume(a, A, d.h, c, nch);
        if (c + kGroup >= nch) break;
        if (c + 2 * kGroup < nch) issue(A, rs, voff, c + 2 * kGroup, nch);
        consume(a, B, d.h, c + kGroup, nch);
    }
    float acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = a[j] + a[4 + j];
    float s = (acc[0] + acc[2]) + (acc[1] + acc[3]);
    const int row = row0 + lane;
    if (kTail && lane < rows) {
        const uint16_t* w = d.table + (size_t)row * d.hidden;
        for (int i = nch * 8; i < d.hidden; ++i) s = s + d.h[i] * __uint_as_float((uint32_t)w[i] << 16);
    }
    if (d.logits && lane < rows) d.logits[row] = s;
    if (d.topk > 0) {
        uint64_t key[1] = {lane < rows ? topk_key(s, row) : 0ull};
        const bool desc[1] = {true};
        wave_sort<1>(key, desc, lane);
        if (lane < d.topk) d.partials[(size_t)tile * d.topk + lane] = key[0];
    }
}

hipError_t bf16_launch_lm_head(const Bf16HeadDesc& d, hipStream_t s) {
    const int ntiles = (d.vocab + BFP8_TILE_ROWS - 1) / BFP8_TILE_ROWS;
    if (ntiles <= 0) return hipSuccess;
    const int grid = (ntiles + 3) / 4;
    if (d.tail && (d.hidden & 7))
        hipLaunchKernelGGL(bf16_lm_head_kernel<true>, dim3(grid), dim3(256), 0, s, d);
    else
        hipLaunchKernelGGL(bf16_lm_head_kernel<false>, dim3(grid), dim3(256), 0, s, d);
    return hipGetLastError();
}
