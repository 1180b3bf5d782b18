// quant_block.h -- one wavefront quantizes one 64-element activation block
// (04/qwen_kernels_opt.c:182-205):
//   amax = max |x| over the block (a NaN never wins `v > amax`)
//   amax > 1e-20:  q = 16384/amax, xscale = amax/16384, xq = (int16)lrintf(x*q)
//   otherwise:     xscale = 0, xq = 0
// and writes the split record xq = 256*xh + xl in the residue-major order the
// GEMV kernels read (bfp8_layout.h).
//
// The result is the same in an IEEE and in a flush-to-zero translation unit:
// q and xscale are quotients of a normal amax (> 1e-20) and a power of two,
// and a subnormal x gives |x*q| < 2^-13, which rounds to 0 either way.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// lane = this thread's element (0..63) of the block, xv its value; rec = 32
// dwords of LDS owned by the calling wavefront.  Every lane of the wavefront
// calls this.
__device__ __forceinline__ void bfp8_quant_block_wave(float xv, int lane, int16_t* xq_b, float* xscale_b,
                                                      uint32_t* xsplit_b, uint32_t* rec) {
    const float v = fabsf(xv);
    float amax = (v > 0.0f) ? v : 0.0f;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float o = __shfl_xor(amax, m, 64);
        amax = (o > amax) ? o : amax;
    }
    int xq = 0;
    float xs = 0.0f;
    if (amax > 1e-20f) {
        const float q = __fdiv_rn(16384.0f, amax);
        xs = __fdiv_rn(amax, 16384.0f);
        const float p = __fmul_rn(xv, q);
        // lrintf rounds half to even; a NaN product (x NaN, or inf*0) gives 0.
        xq = (p == p) ? (int)__builtin_rintf(p) : 0;
    }
    if (xq_b) xq_b[lane] = (int16_t)xq;
    if (lane == 0) *xscale_b = xs;
    const int xl = (int)(int8_t)(xq & 0xff);
    const int xh = (xq - xl) >> 8;
    const int res = lane & 3, ii = lane >> 2;
    const int pos = res * 32 + (ii >> 2) * 4 + (ii & 3);
    uint8_t* rb = reinterpret_cast<uint8_t*>(rec);
    rb[pos] = (uint8_t)xh;
    rb[pos + 16] = (uint8_t)xl;
    // the record's bytes come from other lanes of this wavefront
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < 32) xsplit_b[lane] = rec[lane];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
