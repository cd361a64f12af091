// The build's packed 4-bit tile layout and the per-wave MFMA step over it, shared by
// the quantized projection kernels.
//
// Packed layout (jit_q4_prepack): per (expert, 16-row block) a block of GP = K / 128
// group pairs -- first GP nibble tiles of 1 KB, 64 lanes x 16 B in MFMA fragment order
// (lane 16*lg + lr holds words 2lg, 2lg+1 of the pair's first group and 2lg, 2lg+1 of
// the second, row lr), then GP scale tiles of 128 B, 16 rows x (scale pair, bias
// pair) bf16.  A wave reads a nibble tile with one fully coalesced 1 KB load, and the
// scales of up to 4 consecutive pairs with one 512 B load (lane 16*p + lr: pair p, row
// lr) whose pieces it then passes to the lanes of row lr.
//
// MFMA tile: v_mfma_f32_16x16x32_bf16 computes C[16 tokens x 16 weight rows], tokens
// on the M side (A operand = activations), weight rows on the N side (B operand =
// nibbles).  Every MFMA sees k values of a single quant group, so the group's scale
// and bias apply to the MFMA result:
//   sum_k x_k (s q_k + b) = s * sum_k x_k (q_k + 128) + (b - 128 s) * sum_k x_k,
// with q + 128 formed as a bf16 by one AND-OR and sum_k x_k from an MFMA against ones.
#pragma once

#include "common.hpp"

namespace qtile {

constexpr int kNibbleBytes = 1024, kScaleBytes = 128;
constexpr int kTileBytes = kNibbleBytes + kScaleBytes;  // per (16-row block, group pair)

// Nibble order inside a packed-layout word: the MLX word holds q0..q7 at bits 4i;
// the packed word holds q0, q2, q4, q6 at nibble positions 0-3 and q1, q3, q5, q7 at
// 4-7, so that unpacking yields the k values in natural order and the activations
// need no shuffle.  jit_q4_prepack applies this once; the MLX-layout kernels apply it
// in registers, so both feed the matrix cores the same operands.
__device__ __forceinline__ uint32_t nibbles_natural(uint32_t w) {
  uint32_t e = w & 0x0F0F0F0Fu, o = (w >> 4) & 0x0F0F0F0Fu;
  e = (e | (e >> 4)) & 0x00FF00FFu;
  o = (o | (o >> 4)) & 0x00FF00FFu;
  e = (e | (e >> 8)) & 0x0000FFFFu;
  o = (o | (o >> 8)) & 0x0000FFFFu;
  return e | (o << 16);
}

// bf16 fragment of the 8 nibbles of a packed-order word: (q0, ..., q7) + 128, each
// output one shift and one v_and_or_b32 (m = 0x000F000F and c = 0x43004300 are
// passed in registers: the instruction takes no literal operands).
__device__ __forceinline__ Frag8 unpack_nibbles(uint32_t w, uint32_t m, uint32_t c) {
  Frag8 f;
  f.u[0] = (w & m) | c;
  f.u[1] = ((w >> 4) & m) | c;
  f.u[2] = ((w >> 8) & m) | c;
  f.u[3] = ((w >> 12) & m) | c;
  return f;
}

// Both words of a lane's group (w0, w1) at once: the shifts by 4, 8 and 12 are 64-bit shifts of
// the pair (one v_lshrrev_b64 each instead of one shift a word; written out, as the compiler
// splits a 64-bit shift into two 32-bit ones).  The low word of (w1:w0) >> s takes w1's low bits
// into its bits 32 - s .. 31, which the mask (bits 0-3 and 16-19) never keeps.
__device__ __forceinline__ void unpack_nibbles2(uint32_t w0, uint32_t w1, uint32_t m, uint32_t c, Frag8 &b0,
                                                Frag8 &b1) {
  const uint64_t w = ((uint64_t)w1 << 32) | w0;
  b0.u[0] = (w0 & m) | c;
  b1.u[0] = (w1 & m) | c;
#pragma unroll
  for (int j = 1; j < 4; j++) {
    uint64_t t;
    asm("v_lshrrev_b64 %0, %1, %2" : "=v"(t) : "n"(4 * j), "v"(w));
    b0.u[j] = ((uint32_t)t & m) | c;
    b1.u[j] = ((uint32_t)(t >> 32) & m) | c;
  }
}

// The unpack masks as register values the compiler cannot fold back into literals.
#define QTILE_UNPACK_CONSTANTS(m, c)         \
  uint32_t m = 0x000F000Fu, c = 0x43004300u; \
  asm volatile("" : "+v"(m), "+v"(c))

// Loads of one wave's slice of a packed 16-row block: GPW consecutive groups from
// group g0 (GPW even, at most 8).  wv[g] are the nibble words the lane feeds into
// group g's two MFMAs; sv[j] / bv[j] the (scale, bias) bf16 pairs of groups 2j, 2j+1
// of the lane's row.
template <int GPW>
__device__ __forceinline__ void load_packed_slice(const uint8_t *blk, int K, int g0, int l, uint2 (&wv)[GPW],
                                                  uint32_t (&sv)[GPW / 2], uint32_t (&bv)[GPW / 2]) {
  static_assert(GPW % 2 == 0 && GPW / 2 <= 4, "packed tiles hold pairs of groups; one scale load covers 4");
  const int GP = K >> 7, lr = l & 15, lg = l >> 4;
  const uint8_t *nb = blk + (g0 >> 1) * kNibbleBytes;
  // lane group lg fetches pair min(lg, GPW/2 - 1) (lanes past the slice re-read its last pair)
  const uint2 sbl = *(const uint2 *)(blk + (long long)GP * kNibbleBytes +
                                     ((g0 >> 1) + min(lg, GPW / 2 - 1)) * kScaleBytes + 8 * lr);
#pragma unroll
  for (int j = 0; j < GPW / 2; j++) {
    const uint4 q = *(const uint4 *)(nb + j * kNibbleBytes + 16 * l);
    wv[2 * j] = make_uint2(q.x, q.y);
    wv[2 * j + 1] = make_uint2(q.z, q.w);
  }
#pragma unroll
  for (int j = 0; j < GPW / 2; j++) {
    sv[j] = (uint32_t)__shfl((int)sbl.x, 16 * j + lr, 64);
    bv[j] = (uint32_t)__shfl((int)sbl.y, 16 * j + lr, 64);
  }
}

// One quant group of one 16-row block against one token tile: acc (lane l: tokens
// 4 * (l / 16) + i, row l % 16) += s * C + (b - 128 s) * X, where C = x . (q + 128)
// over the group's 64 k (two MFMAs) and X = sum of the tile's x over the group (from
// the caller, one MFMA pair against ones per tile and group).
__device__ __forceinline__ void group_step(const Frag8 (&xa)[2], const f32x4 &X, uint32_t w0, uint32_t w1,
                                           uint32_t spair, uint32_t bpair, int odd, uint32_t um, uint32_t uc,
                                           f32x4 &acc) {
  const Frag8 B0 = unpack_nibbles(w0, um, uc), B1 = unpack_nibbles(w1, um, uc);
  const float sc = odd ? bf2f_hi(spair) : bf2f(spair & 0xffffu);
  const float bi = odd ? bf2f_hi(bpair) : bf2f(bpair & 0xffffu);
  const float bq = fmaf(-128.0f, sc, bi);
  f32x4 C = mfma16x16x32(xa[0], B0, f32x4{0.f, 0.f, 0.f, 0.f});
  C = mfma16x16x32(xa[1], B1, C);
#pragma unroll
  for (int i = 0; i < 4; i++) acc[i] = fmaf(bq, X[i], fmaf(sc, C[i], acc[i]));
}

__device__ __forceinline__ f32x4 group_xsum(const Frag8 (&xa)[2]) {
  Frag8 ones;
#pragma unroll
  for (int i = 0; i < 4; i++) ones.u[i] = 0x3F803F80u;
  f32x4 X = mfma16x16x32(xa[0], ones, f32x4{0.f, 0.f, 0.f, 0.f});
  return mfma16x16x32(xa[1], ones, X);
}

// e^x for 0 <= x: Cody-Waite reduction x = n ln2 + r with fdlibm's two-part ln2, degree-7
// Taylor polynomial of e^r in Horner form with fused multiply-adds, scaled by 2^(n-1) and then 2
// (n = 128 stays finite); x > 89 or NaN gives x * inf.  The CPU restatement (jo_exp_pos) runs
// the identical operation sequence, so the sigmoid below rounds the same fp32 value to bf16.
__device__ __forceinline__ float exp_pos(float x) {
#pragma clang fp contract(off)
  // (no branch: the polynomial runs for every x, and x > 89 or NaN selects x * inf at the end)
  const float x0 = x;
  const bool big = !(x <= 89.0f);
  x = big ? 0.0f : x;
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
  const float sc = __uint_as_float((uint32_t)(e - 1 + 127) << 23);
  const float y = (p * sc) * 2.0f;
  return big ? x0 * __builtin_inff() : y;
}

// bf16 round trip of a float (round to nearest even, v_cvt_pk_bf16_f32): exact for every
// number; NaN payloads are not kept (the final outputs below still go through f2bf).
__device__ __forceinline__ float rne_bf16(float x) { return static_cast<float>(static_cast<__bf16>(x)); }

// SigmoidX on a bf16 value g (MLX's Sigmoid on bf16, Q36/kernels/expert_solo.py:56-62): every
// step is an fp32 operation on bf16 operands rounded to bf16 -- e = bf16(exp|g|),
// d = bf16(1 + e), y = bf16(1 / d), g < 0 ? y : bf16(1 - y) -- the bits of the CPU restatement
// (which divides correctly rounded).  1 / d: the reciprocal of any bf16 value lies at least 192
// fp32 ulps from every bf16 rounding tie, so the 1-ulp hardware reciprocal rounds to the same bf16;
// from d = 2^126 on (|g| > 87.3) the reciprocal is subnormal and is formed as rcp(d / 4) / 4.
__device__ __forceinline__ float sigmoid_bf16(float g) {
#pragma clang fp contract(off)
  const float e = rne_bf16(exp_pos(fabsf(g)));
  const float d = rne_bf16(1.0f + e);
  const float sc = d < 0x1p126f ? 1.0f : 0.25f;
  const float y = rne_bf16(__builtin_amdgcn_rcpf(d * sc) * sc);
  return g < 0.0f ? y : rne_bf16(1.0f - y);
}

// SwiGLU with the reference's bf16 rounding points (Q36/kernels/expert_solo.py:106-115): g, u
// rounded; sigmoid(g) by the bf16 steps above; sl = bf16(g * sigmoid); h = bf16(sl * u).
__device__ __forceinline__ uint32_t swiglu_bf16(float gacc, float uacc) {
#pragma clang fp contract(off)
  const float g = rne_bf16(gacc), u = rne_bf16(uacc);
  const float sl = rne_bf16(g * sigmoid_bf16(g));
  return f2bf(sl * u);
}

// sigmoid_bf16 as a table over the bf16 bits of g, for kernels with many SwiGLU outputs per lane
// (the segment GEMM's epilogue: ~40 a lane, each ~45 instructions by the steps above).  The
// function is constant outside 2^-8 <= |g| < 2^7: below, bf16(e^|g|) = 1 (e^|g| < 1 + 2^-8, the
// rounding midpoint), so d = 2 and the result is 0.5 on both sides; from 2^7 on, e^|g| overflows
// (exp_pos(x > 89) = inf), y = 0 and the result is 0 for g < 0 and 1 otherwise (a NaN g lands here
// too and keeps a NaN product below).  Entry 2 i + s: sign s and magnitude index i -- 0 for the
// small ones, 1 + (bits - 0x3B80) for the 1,920 bf16 magnitudes of the middle, 1,921 for the large
// ones -- as bf16 bits; the table is exhaustively equal to sigmoid_bf16.
constexpr int kSigLo = 0x3B80, kSigMid = 0x4300 - 0x3B80;
constexpr int kSigEntries = 2 * (kSigMid + 2);
__device__ __forceinline__ uint16_t sigmoid_entry(int e) {
  const int i = e >> 1, sgn = e & 1;
  if (i == 0) return 0x3F00;                     // 0.5
  if (i == kSigMid + 1) return sgn ? 0 : 0x3F80;  // 0 or 1
  const float g = __uint_as_float((uint32_t)((sgn << 15) | (kSigLo + i - 1)) << 16);
  return (uint16_t)(__float_as_uint(sigmoid_bf16(g)) >> 16);
}
__device__ __forceinline__ uint32_t swiglu_bf16_tab(float gacc, float uacc, const uint16_t *tab) {
#pragma clang fp contract(off)
  const float g = rne_bf16(gacc), u = rne_bf16(uacc);
  const uint32_t b = __float_as_uint(g) >> 16;
  const int i = min(max((int)(b & 0x7fffu) - kSigLo, -1), kSigMid) + 1;
  const float sig = __uint_as_float((uint32_t)tab[2 * i + (int)(b >> 15)] << 16);
  const float sl = rne_bf16(g * sig);
  return f2bf(sl * u);
}

}  // namespace qtile
