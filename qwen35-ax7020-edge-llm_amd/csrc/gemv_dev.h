// gemv_dev.h -- device helpers shared by the GEMV kernels (bfp8_ftz.hip,
// fused_gemv.hip): buffer resources for the GPU weight planes
// (bfp8_layout.h), non-temporal weight loads, and EXP_SCALE under
// flush-to-zero.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBufDword3 = 0x00020000;  // gfx9 raw buffer descriptor word 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             kBufDword3);
}

// Weights are streamed once: non-temporal loads (cache policy bit nt).
constexpr int kNonTemporal = 2;
__device__ __forceinline__ u32x4 load_w(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, kNonTemporal));
}

__device__ __forceinline__ uint32_t load_e(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, 0);
}

// EXP_SCALE[e] under flush-to-zero: 2^(e-134) for e >= 8, else +0.
__device__ __forceinline__ float exp_scale_ftz(uint32_t e) {
    return __uint_as_float((max(e, 7u) - 7u) << 23);
}

}  // namespace
