// ieee_dev.h -- the reference's scalar (VFP) float steps, IEEE subnormals
// included, inside a translation unit compiled with
// -fgpu-flush-denormals-to-zero: each operation widens its operands to double
// from their bit patterns, computes there, and rounds once to float by hand.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

// ---- exact scalar IEEE steps inside a flush-to-zero unit ----------------------------
// float -> double, subnormals included (bit-built, so no conversion flushes them)
__device__ __forceinline__ double widen(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7f800000u) == 0u) {
        const double m = (double)(u & 0x007fffffu) * 0x1p-149;
        return (u >> 31) ? -m : m;
    }
    return (double)x;
}

// double -> float, round to nearest even, subnormal results built by hand.
// The operations below round twice (to double, then to float); with 53 >=
// 2*24 + 2 bits that never changes a product, sum, quotient or square root of
// floats.
__device__ __forceinline__ float narrow(double r) {
    const double a = __builtin_fabs(r);
    if (!(a < 0x1p-126)) return (float)r;  // normal, inf, NaN
    const uint32_t m = (uint32_t)__builtin_rint(a * 0x1p149);  // <= 2^23 (2^23 = FLT_MIN)
    return __uint_as_float(m | (__builtin_signbit(r) ? 0x80000000u : 0u));
}

// Normal: neither zero, subnormal, infinite nor NaN.  When both operands and
// the flush-to-zero result of an operation are normal, that result is the
// IEEE one (flushing only touches subnormal operands and results), so the
// float instruction answers; every other case takes the double path.
__device__ __forceinline__ bool normal_f(float x) {
    const uint32_t e = (__float_as_uint(x) >> 23) & 0xffu;
    return e != 0u && e != 0xffu;
}
// The same test as 0 / 1, for conjunctions of many tests with a bitwise `&`
// (no branch per test).
__device__ __forceinline__ uint32_t normal_u(float x) { return normal_f(x) ? 1u : 0u; }
__device__ __forceinline__ float ieee_mul(float a, float b) {
    const float r = __fmul_rn(a, b);
    return (normal_f(a) && normal_f(b) && normal_f(r)) ? r : narrow(widen(a) * widen(b));
}
__device__ __forceinline__ float ieee_add(float a, float b) {
    const float r = __fadd_rn(a, b);
    return (normal_f(a) && normal_f(b) && normal_f(r)) ? r : narrow(widen(a) + widen(b));
}
__device__ __forceinline__ float ieee_div(float a, float b) {
    const float r = __fdiv_rn(a, b);
    return (normal_f(a) && normal_f(b) && normal_f(r)) ? r : narrow(widen(a) / widen(b));
}
// The f32 square-root instruction is not correctly rounded on gfx950 (about
// one result in seven is an ulp off), so the square root always goes through
// double, whose square root is.
__device__ __forceinline__ float ieee_sqrt(float a) { return narrow(__builtin_sqrt(widen(a))); }
__device__ __forceinline__ float libm_expf(float x) { return narrow(exp(widen(x))); }
__device__ __forceinline__ float libm_log1pf(float x) { return narrow(log1p(widen(x))); }

}  // namespace
