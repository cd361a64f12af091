// Elementwise fp32 math whose bits the CPU restatement reproduces operation for operation
// (oracle/jit_oracle.c runs the same sequences with contraction off), and the exact fixed-point
// helpers of the sampler's sums.
#pragma once

#include "common.hpp"

namespace fmath {

// e^x for x <= 0: Cody-Waite reduction x = n ln2 + r with fdlibm's two-part ln2,
// degree-7 Taylor polynomial of e^r in Horner form (|r| <= ln2/2), scaling by 2^n
// through the exponent field; x <= -64 (and NaN) gives 0 so no subnormal is ever formed.
__device__ __forceinline__ float exp_neg(float x) {
#pragma clang fp contract(off)
  if (!(x > -64.0f)) return 0.0f;
  const float t = x * 1.44269504088896341f;
  const float n = __builtin_rintf(t);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.42860682030941723e-6f, r);
  float p = 1.98412698412698413e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int e = (int)n;
  const float sc = __uint_as_float((uint32_t)(e + 127) << 23);
  return p * sc;
}

// ln s for 1 <= s < 2^64: s = 2^k f with f in [sqrt(1/2), sqrt(2)], ln f = 2 atanh(z) with
// z = (f - 1) / (f + 1) (|z| <= 0.1716, correctly rounded division) by its odd series through
// z^11 in Horner form on z^2, then k ln2 + ln f with one fused multiply-add.
__device__ __forceinline__ float log_ge1(float s) {
#pragma clang fp contract(off)
  const uint32_t u = __float_as_uint(s);
  int k = (int)((u >> 23) & 0xffu) - 127;
  float f = __uint_as_float((u & 0x007fffffu) | 0x3f800000u);
  if (f > 1.41421356f) {
    f = f * 0.5f;
    k += 1;
  }
  const float z = (f - 1.0f) / (f + 1.0f);
  const float z2 = z * z;
  float p = 9.09090909090909091e-2f;
  p = __builtin_fmaf(p, z2, 1.11111111111111111e-1f);
  p = __builtin_fmaf(p, z2, 1.42857142857142857e-1f);
  p = __builtin_fmaf(p, z2, 2.0e-1f);
  p = __builtin_fmaf(p, z2, 3.33333333333333333e-1f);
  p = __builtin_fmaf(p, z2, 1.0f);
  const float lf = (z + z) * p;
  return __builtin_fmaf((float)k, 0.693147182464599609375f, lf);
}

// floor(w 2^42) for 0 <= w <= 1 (the scaling is exact, the conversion truncates)
__device__ __forceinline__ uint64_t fix42(float w) { return (uint64_t)(w * 0x1p42f); }

// c rounded to nearest even at `bits` significant bits, as a float times 2^scale_exp
__device__ __forceinline__ float u64_round(uint64_t c, int bits, int scale_exp) {
  if (c == 0) return 0.0f;
  const int e = 63 - __builtin_clzll(c);
  int sh = e - (bits - 1);
  uint64_t m = c;
  if (sh > 0) {
    const uint64_t rem = c & ((1ull << sh) - 1), half = 1ull << (sh - 1);
    m = c >> sh;
    if (rem > half || (rem == half && (m & 1))) m++;
  } else {
    sh = 0;
  }
  return __builtin_ldexpf((float)m, sh + scale_exp);
}

// c 2^-42 rounded once to fp32 (24 bits) and to bf16 (8 bits)
__device__ __forceinline__ float fix42_to_f32(uint64_t c) { return u64_round(c, 24, -42); }
__device__ __forceinline__ float fix42_to_bf16(uint64_t c) { return u64_round(c, 8, -42); }

// floor(u T 2^-32) for A = u 2^32 < 2^32 and T < 2^64, exactly
__device__ __forceinline__ uint64_t mul_u32_u64_hi(uint64_t A, uint64_t T) {
  return A * (T >> 32) + ((A * (T & 0xffffffffull)) >> 32);
}

}  // namespace fmath
