// fp32 helpers of the update kernels whose results must equal another, slower form bit
// for bit: the bf16 conversion of the stored moments and copies, and the quotient by a
// per-step constant in the fused=True chain (positive divisor) and in the capturable chain
// (negative divisor).  Kept in a header so that the check program
// tests/c/fp32_math_check.hip runs this very code against the forms it replaces.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> two bf16 (a in the low half), round to nearest even; every NaN becomes
// 0x7FC0 (the value torch's Tensor.to(torch.bfloat16) produces).  The conversion is
// gfx950's v_cvt_pk_bf16_f32, which rounds every non-NaN input as the integer form
// u + 0x7fff + ((u >> 16) & 1) does (denormals and overflow to inf included) but
// keeps a NaN's sign and payload bits; a NaN input is therefore replaced by the
// canonical quiet NaN first.  Five instructions per pair instead of eleven.
__device__ __forceinline__ uint32_t bf16x2_bits(float a, float b) {
    a = (a == a) ? a : __builtin_nanf("");
    b = (b == b) ? b : __builtin_nanf("");
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}
__device__ __forceinline__ uint32_t bf16_bits(float x) { return bf16x2_bits(x, 0.0f) & 0xffffu; }

// s / b, correctly rounded, given r = 1.0f / b (correctly rounded), for the quotients of
// the fused=True chain when bc2_sqrt comes from the host or from the per-row launch:
// s = sqrtf(v) (+-0, inf, NaN, or in [2^-74.5, 2^64]) and b = bc2_sqrt (in [2^-26.5, 1]
// for every step count >= 1 and float64 beta2 in [0, 1)).  q0 = s * r is within one ulp of s / b, so e = s - q0 * b is exactly
// representable (a multiple of 2^(i-47) below 2^(i-23), i the exponent of s, normal or
// subnormal alike at these ranges) and one fma gives it; q0 + e * r, rounded once, is the
// correctly rounded quotient (Markstein's correction).  The rounding of that last fma is
// scale-invariant at these ranges, so the check of every pair of significands in [1, 2)
// (tests/c/fp32_math_check.hip) covers every s and b above.
// e is formed as -(q0 * b - s) so that s = -0 gives e = -0 and the quotient -0.  e is NaN
// only when q0 is +-inf or NaN; fmaxf then gives -FLT_MAX, a finite correction that the
// exact fma adds to an infinite or NaN q0 without changing it.  Four instructions (the
// negations are operand modifiers) instead of the division's ten.
__device__ __forceinline__ float div_by_recip(float s, float b, float r) {
    const float q0 = s * r;
    const float e = -__builtin_fmaf(q0, b, -s);
    return __builtin_fmaf(__builtin_fmaxf(e, -3.40282347e38f), r, q0);
}

// s / b, correctly rounded, for a negative b given r = 1.0f / b (correctly rounded): the
// capturable chain's sqrtf(v) / (sqrt(bc2) * -step_size), with s as above (+-0, inf, NaN,
// or in [2^-74.5, 2^64]) and |b| in [2^-62, 2^50], where q0, e and the quotient stay
// normal (the caller divides outside that range).  Every nonzero result is the exact
// negation of div_by_recip's for |b| (round-to-nearest-even is symmetric), which the
// significand check covers; e is formed as s - q0 * b here, the form that gives a zero
// quotient the sign of s / b when b < 0 (the other form does when b > 0).  e is NaN only
// when q0 is +-inf or NaN, and fmaxf then leaves q0 as it is, as above.
__device__ __forceinline__ float div_by_neg_recip(float s, float b, float r) {
    const float q0 = s * r;
    const float e = __builtin_fmaf(-q0, b, s);
    return __builtin_fmaf(__builtin_fmaxf(e, -3.40282347e38f), r, q0);
}

// The range of |b| in which div_by_neg_recip gives the division's bits.
__device__ __forceinline__ bool neg_recip_in_range(float b) {
    const float a = __builtin_fabsf(b);
    return a >= 0x1p-62f && a <= 0x1p50f;
}
