// Row operations of the decoder block shared by its kernels (block.hip) and by the dense projection
// that builds its one input row itself (qmm.hip): one row of D <= 2048 on 256 threads, thread t
// owning the 8 consecutive elements 8t .. 8t + 7 -- the layout and summation order every caller
// shares, so a row built anywhere has the same bits.
#pragma once

#include "common.hpp"

namespace rowops {

// Eight floats to eight bf16 (round-to-nearest-even), packed.
__device__ __forceinline__ uint4 pack8(const float (&v)[8]) {
  uint4 o;
  o.x = pack_bf16x2_rne(v[0], v[1]);
  o.y = pack_bf16x2_rne(v[2], v[3]);
  o.z = pack_bf16x2_rne(v[4], v[5]);
  o.w = pack_bf16x2_rne(v[6], v[7]);
  return o;
}

// The sum of v over the first 256 threads of the workgroup (a wave butterfly, then the four wave
// totals in a fixed order); every thread of the workgroup must call it (two workgroup barriers),
// threads past 256 passing anything; in a workgroup of fewer than 256 threads the missing waves
// count as zero totals (as waves whose threads all pass 0).  red: 8 floats of LDS.
__device__ __forceinline__ float block_sum_256(float v, float *red) {
  v = wave_butterfly<false>(v);  // (the pairs of a shuffle butterfly over offsets 32..1)
  const int w = threadIdx.x >> 6;
  if (lane_id() == 0 && w < 4) red[w] = v;
  if (threadIdx.x < 4 && blockDim.x <= 64 * threadIdx.x) red[threadIdx.x] = 0.0f;
  __syncthreads();
  const float s = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return s;
}

// Weighted combine of one row's 8 consecutive outputs n..n+7 (slot order, each
// product and each partial sum rounded to bf16; a dropped pair, inv < 0,
// contributes nothing), plus the residual when given.  Every slot's loads are
// issued before any is used.
__device__ __forceinline__ void combine8(const uint16_t *__restrict__ r, const int32_t *__restrict__ inv,
                                         const uint16_t *__restrict__ scores, int k, int D,
                                         const uint16_t *__restrict__ resid, long long bt, int n, float (&acc)[8]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = 0.0f;
  const uint4 res = resid ? *(const uint4 *)(resid + bt * D + n) : make_uint4(0u, 0u, 0u, 0u);
  for (int j0 = 0; j0 < k; j0 += 8) {
    uint4 rv[8];
    float sc[8];
    bool use[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      const int j = min(j0 + jj, k - 1);
      const int p = inv[bt * k + j];
      use[jj] = j0 + jj < k && p >= 0;
      sc[jj] = bf2f(scores[bt * k + j]);
      rv[jj] = *(const uint4 *)(r + (long long)(p < 0 ? 0 : p) * D + n);
    }
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      if (!use[jj]) continue;
      const uint32_t wds[4] = {rv[jj].x, rv[jj].y, rv[jj].z, rv[jj].w};
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float p0 = bf2f(wds[i >> 1] & 0xffffu) * sc[jj], p1 = bf2f_hi(wds[i >> 1]) * sc[jj];
        round_bf2(p0, p1);
        float a0 = acc[i] + p0, a1 = acc[i + 1] + p1;
        round_bf2(a0, a1);
        acc[i] = a0;
        acc[i + 1] = a1;
      }
    }
  }
  if (resid) {
    const uint32_t wds[4] = {res.x, res.y, res.z, res.w};
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      float a0 = bf2f(wds[i >> 1] & 0xffffu) + acc[i], a1 = bf2f_hi(wds[i >> 1]) + acc[i + 1];
      round_bf2(a0, a1);
      acc[i] = a0;
      acc[i + 1] = a1;
    }
  }
}


// RMSNorm's output for the 8 elements v of a row whose mean-square reciprocal root is rs:
// bf16(w * bf16(v * rs)), w the 8 norm weights (packed bf16 pairs).
__device__ __forceinline__ void norm8(const float (&v)[8], float rs, const uint4 wq, float (&o)[8]) {
  const uint32_t ww[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    float n0 = v[i] * rs, n1 = v[i + 1] * rs;
    round_bf2(n0, n1);
    o[i] = bf2f(ww[i >> 1] & 0xffffu) * n0;
    o[i + 1] = bf2f_hi(ww[i >> 1]) * n1;
  }
}

}  // namespace rowops
