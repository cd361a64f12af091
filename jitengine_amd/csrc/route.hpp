// The router's top-k of one token row on one wave, shared by the router kernels (router.hip) and
// by the expert GEMV that routes a one-token step itself (qmm.hip): the softmax gates as
// (value, index) keys and the rank rule's slots.  Every floating-point step is one IEEE operation
// in a fixed order (no contraction), so each caller gets the CPU restatement's bits.
#pragma once

#include "common.hpp"
#include "fmath.hpp"

namespace route {

using fmath::exp_neg;

// Key of a bf16 value in the ascending (value, index) order of the rank rule: the
// value's bits made monotonic as an unsigned integer (-0 ties +0, as the float
// comparison does) above a 16-bit index.  Gates must not be NaN.
__device__ __forceinline__ uint32_t order_key(uint32_t b, int i) {
  b = b == 0x8000u ? 0u : b;
  const uint32_t o = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
  return (o << 16) | (uint32_t)i;
}
__device__ __forceinline__ uint32_t key_bf16(uint32_t key) {
  const uint32_t o = key >> 16;
  return (o & 0x8000u) ? (o & 0x7fffu) : (~o & 0xffffu);
}

// Wave maximum with no LDS round trip: DPP quad permutes (lane ^ 1, lane ^ 2), row
// half-mirror and row mirror (every lane of a 16-lane row then holds the row's
// maximum), then the permlane swaps across rows.  A maximum needs no fixed pairing,
// so the mirrors serve where an xor butterfly would.
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v, int ctrl) {
  uint32_t y;
  switch (ctrl) {  // the DPP control is an immediate
    case 0: y = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false); break;   // [1,0,3,2]
    case 1: y = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false); break;   // [2,3,0,1]
    case 2: y = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false); break;  // half mirror
    default: y = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false); break; // mirror
  }
  return y > v ? y : v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = dpp_max_u32(v, 0);
  v = dpp_max_u32(v, 1);
  v = dpp_max_u32(v, 2);
  v = dpp_max_u32(v, 3);
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = r[0] > r[1] ? r[0] : r[1];
  r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return r[0] > r[1] ? r[0] : r[1];
}

// The keys of one row on one wave: lane l holds experts l, l + 64, ... (NPL of them).  Unless
// FROM_GATES, the softmax: lane l sums its experts' exps in that order, the wave adds the 64 partial
// sums by a butterfly over offsets 32..1 (every lane ends with the same total), then every gate is
// e_i * (1 / total) rounded to bf16 (also written to gates_out when given).  Invalid lanes get key 0.
template <int NPL, bool FROM_GATES>
__device__ __forceinline__ void row_keys(const uint16_t *__restrict__ lg, int row, int N, int l, uint32_t (&key)[NPL],
                                         uint16_t *__restrict__ gates_out) {
#pragma clang fp contract(off)
  if (FROM_GATES) {
    uint32_t raw[NPL];
#pragma unroll
    for (int j = 0; j < NPL; j++) raw[j] = lg[min(l + 64 * j, N - 1)];
#pragma unroll
    for (int j = 0; j < NPL; j++) {
      const int i = l + 64 * j;
      key[j] = i < N ? order_key(raw[j], i) : 0u;
    }
  } else {
    float v[NPL], e[NPL];
    float mx = -INFINITY;
    uint32_t raw[NPL];
#pragma unroll
    for (int j = 0; j < NPL; j++) raw[j] = lg[min(l + 64 * j, N - 1)];  // (every load issued before any is used)
#pragma unroll
    for (int j = 0; j < NPL; j++) {
      const int i = l + 64 * j;
      v[j] = i < N ? bf2f(raw[j]) : -INFINITY;
      mx = v[j] > mx ? v[j] : mx;
    }
    mx = wave_butterfly<true>(mx);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NPL; j++) {
      const int i = l + 64 * j;
      e[j] = (i < N) ? exp_neg(v[j] - mx) : 0.0f;
      s = s + e[j];
    }
    s = wave_butterfly<false>(s);
    const float inv = 1.0f / s;
#pragma unroll
    for (int j = 0; j < NPL; j++) {
      const int i = l + 64 * j;
      const uint32_t g = f2bf(e[j] * inv);
      key[j] = i < N ? order_key(g, i) : 0u;
      if (gates_out && i < N) gates_out[(size_t)row * N + i] = (uint16_t)g;
    }
  }
}

// The top-k slots of a row on one wave, for k <= 64: the rank rule of the reference (the rank of
// gate i counts the gates below it, ties broken by index, and ranks >= N - k fill slots
// rank - (N - k) in ascending (value, index) order), found as k rounds of a wave maximum over the
// keys, round t filling slot k - 1 - t.  Lane j < k returns slot j's key, the other lanes 0.
template <int NPL>
__device__ __forceinline__ uint32_t topk_slot_key(const uint16_t *__restrict__ lg, int N, int k, int l) {
  uint32_t key[NPL];
  row_keys<NPL, false>(lg, 0, N, l, key, nullptr);
  uint32_t mine = 0;
  for (int t = 0; t < k; t++) {  // (every valid key is > 0; a taken key becomes 0)
    uint32_t m = key[0];
#pragma unroll
    for (int j = 1; j < NPL; j++) m = key[j] > m ? key[j] : m;
    m = wave_max_u32(m);
#pragma unroll
    for (int j = 0; j < NPL; j++) key[j] = key[j] == m ? 0u : key[j];
    mine = l == k - 1 - t ? m : mine;
  }
  return mine;
}

// The renormalising total of the k slots' gates, added in slot order with each sum rounded to bf16
// (as the reference's bf16 sum does); `slot` is the key of slot j in lane j.
__device__ __forceinline__ float slots_total(uint32_t slot, int k) {
#pragma clang fp contract(off)
  float tot = 0.0f;
  for (int j = 0; j < k; j++) tot = bf2f(f2bf(tot + bf2f(key_bf16((uint32_t)__builtin_amdgcn_readlane((int)slot, j)))));
  return tot;
}

}  // namespace route
