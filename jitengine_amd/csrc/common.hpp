// Shared device helpers for the gfx950 kernels: bf16 conversion, MFMA operand
// types, wave-level exchange, and the error plumbing of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "jit_moe.h"

// ------------------------------------------------------------------ types
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef float f32x4 __attribute__((ext_vector_type(4)));

union Frag8 {  // 8 bf16 = one MFMA 16x16x32 operand fragment of one lane
  bf16x8_t v;
  uint32_t u[4];
  uint4 q;
};

// ------------------------------------------------------------------ streaming loads
// Bytes a launch reads exactly once (packed expert weights, KV pages) are loaded with the
// nontemporal hint: the measured streaming-read rate of contiguous per-workgroup runs on MI355X
// rises from ~6.2 to ~7.0 TB/s with it (bench.py --probe).  JIT_NT_LOADS=0 builds plain loads.
#ifndef JIT_NT_LOADS
#define JIT_NT_LOADS 1
#endif
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 ld_stream16(const void *p) {
#if JIT_NT_LOADS
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
#else
  return *(const uint4 *)p;
#endif
}

__device__ __forceinline__ uint2 ld_stream8(const void *p) {
#if JIT_NT_LOADS
  const u32x2_t v = __builtin_nontemporal_load((const u32x2_t *)p);
  return make_uint2(v.x, v.y);
#else
  return *(const uint2 *)p;
#endif
}

// ------------------------------------------------------------------ bf16
__device__ __forceinline__ float bf2f(uint32_t h16) { return __uint_as_float(h16 << 16); }
__device__ __forceinline__ float bf2f_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 round-to-nearest-even (NaN kept quiet: its top 16 bits with the quiet bit set),
// the rounding of MLX's bf16 type.  Numbers take the hardware conversion (v_cvt_pk_bf16_f32,
// the same rounding); only the NaN payload is formed by hand.
__device__ __forceinline__ uint32_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t h = __builtin_bit_cast(unsigned short, (__bf16)f);
  return (u & 0x7fffffffu) > 0x7f800000u ? (((u >> 16) | 0x40u) & 0xffffu) : h;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f2bf(lo) | (f2bf(hi) << 16);
}

// The same rounding in one instruction (v_cvt_pk_bf16_f32, round-to-nearest-even), for finite
// values: NaN payloads may differ from f2bf's.
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Round two floats to bf16 (the hardware rounding above) and widen them back: the bf16 values
// as floats, in three instructions for the pair.
__device__ __forceinline__ void round_bf2(float &a, float &b) {
  const uint32_t p = pack_bf16x2_rne(a, b);
  a = __uint_as_float(p << 16);
  b = __uint_as_float(p & 0xffff0000u);
}

// Split two floats into bf16 high parts and bf16 residuals: hi = bf16(a), lo = bf16(a - hi) (the
// subtraction is exact).  hi + lo carries a to 16 significant bits (relative error <= 2^-17), so a
// P.V product issued as two bf16 MFMAs, V.hi + V.lo, keeps the probabilities at nearly fp32
// precision where one bf16 P would round each of them by up to 2^-9.
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t &hi, uint32_t &lo) {
  hi = pack_bf16x2_rne(a, b);
  lo = pack_bf16x2_rne(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
}

// ------------------------------------------------------------------ wave
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63u); }

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ float shfl_f(float v, int src) { return __shfl(v, src, 64); }

// The butterfly over lane offsets 32, 16, 8, 4, 2, 1 (in that order; after step o every lane
// holds the combination of its own value and lane l ^ o's), in VALU lane exchanges instead of LDS
// permutes: the permlane swaps for 32 and 16, a row rotation by 8 (lane l ^ 8 within its 16-lane
// row), two bank-masked row shifts for 4, quad permutes for 2 and 1.  Each step pairs the same
// lanes as a shuffle by l ^ o would, and the combination is commutative, so the results are the
// shuffle butterfly's bit for bit.
template <bool MAX>
__device__ __forceinline__ float wave_butterfly(float v) {
  auto op = [](float a, float b) { return MAX ? (b > a ? b : a) : a + b; };
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const int vi = __float_as_int(v);
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(vi, vi, 0x128, 0xF, 0xF, false)));  // row_ror:8
  int x4 = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x104, 0xF, 0x5, false);  // row_shl:4, banks 0, 2
  x4 = __builtin_amdgcn_update_dpp(x4, __float_as_int(v), 0x114, 0xF, 0xA, false);               // row_shr:4, banks 1, 3
  v = op(v, __int_as_float(x4));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  return op(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0xB1, 0xF, 0xF, false)));
}

__device__ __forceinline__ f32x4 mfma16x16x32(const Frag8 &a, const Frag8 &b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, c, 0, 0, 0);
}

// ------------------------------------------------------------------ paged KV layout
// Element offset of (slot, d) inside the K block of one (page, kv head): chunk-major
// [4 d-chunks of 32][16 slots][32 dims], so one MFMA fragment's 16 slots x 32 dims
// are 1 KB contiguous.  (The V block is dim-major: offset d * 16 + slot.)
__device__ __forceinline__ int k_page_offset(int slot, int d) {
  return (d >> 5) * (JIT_PAGE_TOKENS * 32) + slot * 32 + (d & 31);
}

// ------------------------------------------------------------------ q/k norm + RoPE of one head
// One head of one token, on the 64 lanes of a wave (lane l: dims l and l + 64, RoPE's pairs):
// RMSNorm over the head's 128 dims with the norm weight (w1, w2 = dims l, l + 64), each step
// rounded to bf16 as the reference's bf16 arithmetic does, then the rotation by ang = pos *
// inv_freq[l] (Q36/model/attention.py:99-119).  Every kernel that norms and rotates a head calls
// this, so their bits agree; the expression is fixed (no contraction).
__device__ __forceinline__ void qk_head_norm_rope(float x1, float x2, float w1, float w2, float eps, float ang,
                                                  uint32_t &o1, uint32_t &o2) {
#pragma clang fp contract(off)
  float ss = __builtin_fmaf(x1, x1, x2 * x2);
  ss = wave_butterfly<false>(ss);  // (the pairs of a shuffle butterfly over offsets 32..1)
  const float r = rsqrtf(ss / 128.0f + eps);
  x1 = bf2f(f2bf(w1 * bf2f(f2bf(x1 * r))));
  x2 = bf2f(f2bf(w2 * bf2f(f2bf(x2 * r))));
  float sn, cs;
  sincosf(ang, &sn, &cs);
  o1 = f2bf(x1 * cs - x2 * sn);
  o2 = f2bf(x1 * sn + x2 * cs);
}

// ------------------------------------------------------------------ host error plumbing
namespace jit {
void set_error(const char *fmt, ...);
int fail(int code, const char *fmt, ...);
int check_launch(const char *what);
// Compute units of the current device (queried once per device, at most 64 devices).
int cu_count();
}  // namespace jit
