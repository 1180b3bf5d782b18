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

// Maximum over the wavefront of a float that is neither negative nor NaN, in
// every lane (such floats order as their bit patterns): DPP exchanges within
// each row of 16 lanes (quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror), then the four row maxima.  Every lane of the
// wavefront must be active.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    int x = __float_as_int(v);
    x = max(x, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false));
    const int r0 = __builtin_amdgcn_readlane(x, 0), r1 = __builtin_amdgcn_readlane(x, 16);
    const int r2 = __builtin_amdgcn_readlane(x, 32), r3 = __builtin_amdgcn_readlane(x, 48);
    return __int_as_float(max(max(r0, r1), max(r2, r3)));
}

// The block's scale and this lane's int16 value.
struct Bfp8QuantLane {
    float xs;
    int xq;
};
// Branch-free (selects, not a branch on amax), so that the quantizations of
// several blocks by one wavefront can overlap.
__device__ __forceinline__ Bfp8QuantLane bfp8_quant_lane(float xv) {
    const float v = fabsf(xv);
    const float amax = wave_max_nonneg((v > 0.0f) ? v : 0.0f);  // a NaN never wins `v > amax`
    const bool live = amax > 1e-20f;
    const float q = __fdiv_rn(16384.0f, live ? amax : 1.0f);
    const float p = __fmul_rn(xv, q);
    // lrintf rounds half to even; a NaN product (x NaN, or inf*0) gives 0.
    const float pr = (live && p == p) ? p : 0.0f;
    Bfp8QuantLane r;
    r.xs = live ? amax * 0x1p-14f : 0.0f;  // = amax / 16384 exactly: the quotient of amax > 1e-20 by 2^14 is normal
    r.xq = (int)__builtin_rintf(pr);
    return r;
}

// Byte offset of lane's high byte in the block's 128-byte split record (its
// low byte is 16 further on).
__device__ __forceinline__ int bfp8_split_pos(int lane) {
    const int res = lane & 3, ii = lane >> 2;
    return res * 32 + (ii >> 2) * 4 + (ii & 3);
}

// Stores a quantized block into LDS: the record's bytes and the scale go
// straight into xsplit_b / xscale_b (__shared__), and the caller's next
// barrier publishes them.  bfp8_quant_block_lds quantizes and stores; every
// lane of the wavefront calls either.
__device__ __forceinline__ void bfp8_store_lds(const Bfp8QuantLane& r, int lane, float* xscale_b, uint32_t* xsplit_b) {
    if (lane == 0) *xscale_b = r.xs;
    const int xl = (int)(int8_t)(r.xq & 0xff);
    const int xh = (r.xq - xl) >> 8;
    uint8_t* rb = reinterpret_cast<uint8_t*>(xsplit_b);
    const int pos = bfp8_split_pos(lane);
    rb[pos] = (uint8_t)xh;
    rb[pos + 16] = (uint8_t)xl;
}

__device__ __forceinline__ void bfp8_quant_block_lds(float xv, int lane, float* xscale_b, uint32_t* xsplit_b) {
    bfp8_store_lds(bfp8_quant_lane(xv), lane, xscale_b, xsplit_b);
}

// Maximum over each row of 16 lanes of a float that is neither negative nor
// NaN, in every lane of the row (the first four steps of wave_max_nonneg).
__device__ __forceinline__ float row_max_nonneg(float v) {
    int x = __float_as_int(v);
    x = max(x, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false));
    return __int_as_float(x);
}

// One block quantized by a row of 16 lanes, four consecutive elements per
// lane: lane ii (0..15 in the row) holds elements 4 ii + j in x[j].  The
// split record puts element 4 ii + j's high byte at byte j * 32 + ii and its
// low byte 16 further on (bfp8_split_pos), so with `store` the lane writes
// those eight bytes and lane 0 of the row the scale, into LDS (the caller's
// next barrier publishes them).  Every lane of the wavefront calls this.
__device__ __forceinline__ void bfp8_quant4_store_lds(const float (&x)[4], int ii, float* xscale_b,
                                                      uint32_t* xsplit_b, bool store) {
    float v = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float aj = fabsf(x[j]);
        v = fmaxf(v, (aj > 0.0f) ? aj : 0.0f);  // a NaN never wins `v > amax`
    }
    const float amax = row_max_nonneg(v);
    const bool live = amax > 1e-20f;
    const float q = __fdiv_rn(16384.0f, live ? amax : 1.0f);
    // LDS pointers (32-bit offsets), not generic ones
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    typedef __attribute__((address_space(3))) float lds_f32;
    lds_u8* rb = (lds_u8*)xsplit_b;
    if (store && ii == 0) *(lds_f32*)xscale_b = live ? amax * 0x1p-14f : 0.0f;  // = amax / 16384 exactly (normal)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float p = __fmul_rn(x[j], q);
        // lrintf rounds half to even; a NaN product (x NaN, or inf*0) gives 0.
        const int xq = (int)__builtin_rintf((live && p == p) ? p : 0.0f);
        const int xl = (int)(int8_t)(xq & 0xff);
        const int xh = (xq - xl) >> 8;
        if (store) {
            rb[j * 32 + ii] = (uint8_t)xh;
            rb[j * 32 + 16 + ii] = (uint8_t)xl;
        }
    }
}

// lane = this thread's element (0..63) of the block, xv its value; rec = 32
// dwords of LDS owned by the calling wavefront (the record is assembled there
// and stored to xsplit_b, which may be global memory, as 32 dwords).  Every
// lane of the wavefront calls this.
__device__ __forceinline__ void bfp8_quant_block_wave(float xv, int lane, int16_t* xq_b, float* xscale_b,
                                                      uint32_t* xsplit_b, uint32_t* rec) {
    const Bfp8QuantLane r = bfp8_quant_lane(xv);
    if (xq_b) xq_b[lane] = (int16_t)r.xq;
    if (lane == 0) *xscale_b = r.xs;
    const int xl = (int)(int8_t)(r.xq & 0xff);
    const int xh = (r.xq - xl) >> 8;
    const int pos = bfp8_split_pos(lane);
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
