// 4-bit affine (MLX layout, group 64) quantized projections on gfx950 matrix
// cores, for dense projections and for expert segments of packed pairs.
//
// Tile: one wave computes C[16 tokens x 16 weight rows] per row block with
// v_mfma_f32_16x16x32_bf16, tokens on the M side (A operand = activations) and
// weight rows on the N side (B operand = nibbles).  Each lane therefore owns one
// weight row (l % 16) and, per quant group of 64 k, loads the two 32-bit words
// (16 nibbles) its lane group (l / 16) feeds into the two MFMAs of that group --
// every MFMA sees k values of a single group, so the group's scale and bias are
// applied to the MFMA result, not per weight:
//   sum_k x_k (s q_k + b) = s * sum_k x_k (q_k + 128) + (b - 128 s) * sum_k x_k.
// A nibble q becomes the bf16 value 128 + q with one AND-OR (0x43pq bit pattern),
// and sum_k x_k comes out of one more MFMA against an all-ones B operand, so the
// per-weight vector work is 7 integer ops per 8 nibbles.  The two bf16 halves of
// an unpacked word hold nibbles (i, i + 4), so the activation fragment is loaded
// in the matching k order with byte permutes.
#include "common.hpp"

namespace {

struct QmmArgs {
  const uint16_t *x;          // activations, row stride K (bf16)
  const int32_t *row_index;   // x row of each sorted position (null: the position itself)
  const int32_t *cnt;         // pairs per expert (null: dense, T tokens)
  const int32_t *off;         // first sorted position per expert
  const uint32_t *w;          // weight stack [E, rows_w, K / 8]
  const uint16_t *s, *b;      // scales, biases [E, rows_w, K / 64]
  uint16_t *out;              // [positions, N] bf16
  int K, N, T;
  long long w_estride, g_estride;
};

// bf16 fragment of 8 nibbles: elements (q0, q4, q1, q5, q2, q6, q3, q7) + 128.
__device__ __forceinline__ Frag8 unpack_nibbles(uint32_t w) {
  Frag8 f;
  f.u[0] = (w & 0x000F000Fu) | 0x43004300u;
  f.u[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  f.u[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  f.u[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return f;
}

// 8 consecutive bf16 x0..x7 -> the fragment order (x0, x4, x1, x5, x2, x6, x3, x7).
__device__ __forceinline__ Frag8 permute_x(uint4 d) {
  Frag8 f;
  f.u[0] = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);
  f.u[1] = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);
  f.u[2] = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);
  f.u[3] = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);
  return f;
}

__device__ __forceinline__ float sel_bf16(uint2 v, int i) {
  const uint32_t w = (i < 2) ? v.x : v.y;
  return (i & 1) ? bf2f_hi(w) : bf2f(w & 0xffffu);
}

// SwiGLU with the reference's bf16 rounding points: g, u rounded; sigmoid(g)
// rounded; bf16(g * sigmoid) * u rounded.
__device__ __forceinline__ uint32_t swiglu_bf16(float gacc, float uacc) {
  const float g = bf2f(f2bf(gacc)), u = bf2f(f2bf(uacc));
  const float y = 1.0f / (1.0f + __expf(fabsf(g)));
  const float sg = bf2f(f2bf(g < 0.0f ? y : 1.0f - y));
  const float sl = bf2f(f2bf(g * sg));
  return f2bf(sl * u);
}

// NB output row blocks of 16 per wave, 4 waves per workgroup.  With SWIGLU each
// output block reads a gate block (rows n) and an up block (rows N + n) of the
// fused stack.
template <int NB, bool SWIGLU>
__global__ __launch_bounds__(256) void qmm_kernel(const QmmArgs a) {
  constexpr int NBW = SWIGLU ? 2 * NB : NB;
  const int wave = threadIdx.x >> 6, l = lane_id();
  const int lr = l & 15, lg = l >> 4;
  const int e = blockIdx.y;
  int cnt, off;
  if (a.cnt) {
    cnt = a.cnt[e];
    off = a.off[e];
  } else {
    cnt = a.T;
    off = 0;
  }
  if (cnt <= 0) return;
  const int n0 = (blockIdx.x * 4 + wave) * (16 * NB);
  if (n0 >= a.N) return;
  const int G = a.K >> 6, KW = a.K >> 3;
  const uint32_t *wb = a.w + (long long)e * a.w_estride;
  const uint16_t *sb = a.s + (long long)e * a.g_estride;
  const uint16_t *bb = a.b + (long long)e * a.g_estride;

  const uint32_t *wrow[NBW];
  const uint16_t *srow[NBW], *brow[NBW];
  bool live[NBW];
#pragma unroll
  for (int rb = 0; rb < NBW; rb++) {
    const int ob = SWIGLU ? (rb % NB) : rb;
    const int rowo = n0 + 16 * ob;
    live[rb] = rowo < a.N;
    const int row = (SWIGLU && rb >= NB ? a.N : 0) + (live[rb] ? rowo : n0) + lr;
    wrow[rb] = wb + (long long)row * KW + 2 * lg;
    srow[rb] = sb + (long long)row * G;
    brow[rb] = bb + (long long)row * G;
  }
  Frag8 ones;
#pragma unroll
  for (int i = 0; i < 4; i++) ones.u[i] = 0x3F803F80u;

  for (int t0 = 0; t0 < cnt; t0 += 16) {
    const int tok = t0 + lr;
    const bool tv = tok < cnt;
    const uint16_t *xr = a.x;
    if (tv) {
      const int pos = off + tok;
      const int xrow = a.row_index ? a.row_index[pos] : pos;
      xr = a.x + (long long)xrow * a.K + 16 * lg;
    }
    f32x4 acc[NBW];
#pragma unroll
    for (int rb = 0; rb < NBW; rb++) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int g = 0; g < G; g += 4) {
      uint2 s4[NBW], b4[NBW], wv[4][NBW];
      uint4 xa[4][2];
#pragma unroll
      for (int rb = 0; rb < NBW; rb++) {
        s4[rb] = *(const uint2 *)(srow[rb] + g);
        b4[rb] = *(const uint2 *)(brow[rb] + g);
      }
#pragma unroll
      for (int gg = 0; gg < 4; gg++) {
#pragma unroll
        for (int rb = 0; rb < NBW; rb++) wv[gg][rb] = *(const uint2 *)(wrow[rb] + 8 * (g + gg));
        if (tv) {
          xa[gg][0] = *(const uint4 *)(xr + 64 * (g + gg));
          xa[gg][1] = *(const uint4 *)(xr + 64 * (g + gg) + 8);
        } else {
          xa[gg][0] = make_uint4(0, 0, 0, 0);
          xa[gg][1] = make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int gg = 0; gg < 4; gg++) {
        const Frag8 A0 = permute_x(xa[gg][0]), A1 = permute_x(xa[gg][1]);
        f32x4 X = mfma16x16x32(A0, ones, f32x4{0.f, 0.f, 0.f, 0.f});
        X = mfma16x16x32(A1, ones, X);
#pragma unroll
        for (int rb = 0; rb < NBW; rb++) {
          if (!live[rb]) continue;
          const Frag8 B0 = unpack_nibbles(wv[gg][rb].x), B1 = unpack_nibbles(wv[gg][rb].y);
          f32x4 C = mfma16x16x32(A0, B0, f32x4{0.f, 0.f, 0.f, 0.f});
          C = mfma16x16x32(A1, B1, C);
          const float sc = sel_bf16(s4[rb], gg), bi = sel_bf16(b4[rb], gg);
          const float bp = fmaf(-128.0f, sc, bi);
#pragma unroll
          for (int i = 0; i < 4; i++) acc[rb][i] = fmaf(bp, X[i], fmaf(sc, C[i], acc[rb][i]));
        }
      }
    }
    // lane l holds C[token 4*lg + i][row lr] of each block
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int t = t0 + 4 * lg + i;
      if (t >= cnt) continue;
      uint16_t *orow = a.out + (long long)(off + t) * a.N + n0 + lr;
#pragma unroll
      for (int ob = 0; ob < NB; ob++) {
        if (!live[ob]) continue;
        if (SWIGLU)
          orow[16 * ob] = (uint16_t)swiglu_bf16(acc[ob][i], acc[NB + ob][i]);
        else
          orow[16 * ob] = (uint16_t)f2bf(acc[ob][i]);
      }
    }
  }
}

template <int NB, bool SWIGLU>
int launch_qmm(const QmmArgs &a, int E, hipStream_t st, const char *what) {
  const int rows_per_wg = 4 * 16 * NB;
  const dim3 grid((a.N + rows_per_wg - 1) / rows_per_wg, E), block(256);
  qmm_kernel<NB, SWIGLU><<<grid, block, 0, st>>>(a);
  return jit::check_launch(what);
}

// Weighted combine: one workgroup per token row, 8 outputs per thread; each
// product and each partial sum is rounded to bf16, slots in ascending order.
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t *__restrict__ r,
                                                      const int32_t *__restrict__ inv,
                                                      const uint16_t *__restrict__ scores, int k,
                                                      int D, const uint16_t *__restrict__ resid,
                                                      uint16_t *__restrict__ y) {
#pragma clang fp contract(off)
  const int bt = blockIdx.x;
  for (int n = threadIdx.x * 8; n < D; n += blockDim.x * 8) {
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = 0.0f;
    for (int j = 0; j < k; j++) {
      const int p = inv[bt * k + j];
      if (p < 0) continue;  // a dropped pair (expert id >= E) contributes nothing
      const float sc = bf2f(scores[bt * k + j]);
      const uint4 rv = *(const uint4 *)(r + (long long)p * D + n);
      const uint32_t wds[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float rr = (i & 1) ? bf2f_hi(wds[i >> 1]) : bf2f(wds[i >> 1] & 0xffffu);
        const float pr = bf2f(f2bf(rr * sc));
        acc[i] = bf2f(f2bf(acc[i] + pr));
      }
    }
    if (resid) {
      const uint4 rv = *(const uint4 *)(resid + (long long)bt * D + n);
      const uint32_t wds[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float rr = (i & 1) ? bf2f_hi(wds[i >> 1]) : bf2f(wds[i >> 1] & 0xffffu);
        acc[i] = bf2f(f2bf(rr + acc[i]));
      }
    }
    uint4 o;
    o.x = f2bf(acc[0]) | (f2bf(acc[1]) << 16);
    o.y = f2bf(acc[2]) | (f2bf(acc[3]) << 16);
    o.z = f2bf(acc[4]) | (f2bf(acc[5]) << 16);
    o.w = f2bf(acc[6]) | (f2bf(acc[7]) << 16);
    *(uint4 *)(y + (long long)bt * D + n) = o;
  }
}

}  // namespace

extern "C" int jit_qmm(const uint16_t *x, int T, int K, const uint32_t *w, const uint16_t *scales,
                       const uint16_t *biases, int N, uint16_t *y, void *stream) {
  if (T < 0 || K <= 0 || N <= 0) return jit::fail(JIT_EINVAL, "qmm: bad dims T=%d K=%d N=%d", T, K, N);
  if (K % 256 != 0 || N % 16 != 0)
    return jit::fail(JIT_EUNSUPPORTED, "qmm covers K %% 256 == 0 and N %% 16 == 0, got K=%d N=%d", K, N);
  if (T == 0) return JIT_OK;
  if (!x || !w || !scales || !biases || !y) return jit::fail(JIT_EINVAL, "qmm: null pointer");
  QmmArgs a{x, nullptr, nullptr, nullptr, w, scales, biases, y, K, N, T, 0, 0};
  return launch_qmm<1, false>(a, 1, (hipStream_t)stream, "jit_qmm");
}

extern "C" int jit_moe_gate_up_swiglu(const uint16_t *x, int K, const int32_t *pair_row,
                                      const int32_t *expert_cnt, const int32_t *expert_off, int E,
                                      const uint32_t *w, const uint16_t *scales,
                                      const uint16_t *biases, int I, int P, uint16_t *h,
                                      void *stream) {
  if (K <= 0 || I <= 0 || E <= 0 || P < 0)
    return jit::fail(JIT_EINVAL, "moe_gate_up: bad dims K=%d I=%d E=%d P=%d", K, I, E, P);
  if (K % 256 != 0 || I % 16 != 0)
    return jit::fail(JIT_EUNSUPPORTED, "moe_gate_up covers K %% 256 == 0 and I %% 16 == 0, got K=%d I=%d", K, I);
  if (P == 0) return JIT_OK;
  if (!x || !pair_row || !expert_cnt || !expert_off || !w || !scales || !biases || !h)
    return jit::fail(JIT_EINVAL, "moe_gate_up: null pointer");
  QmmArgs a{x, pair_row, expert_cnt, expert_off, w, scales, biases, h, K, I, 0,
            (long long)2 * I * (K / 8), (long long)2 * I * (K / 64)};
  return launch_qmm<1, true>(a, E, (hipStream_t)stream, "jit_moe_gate_up_swiglu");
}

extern "C" int jit_moe_down(const uint16_t *h, int I, const int32_t *expert_cnt,
                            const int32_t *expert_off, int E, const uint32_t *w,
                            const uint16_t *scales, const uint16_t *biases, int D, int P, uint16_t *r,
                            void *stream) {
  if (I <= 0 || D <= 0 || E <= 0 || P < 0)
    return jit::fail(JIT_EINVAL, "moe_down: bad dims I=%d D=%d E=%d P=%d", I, D, E, P);
  if (I % 256 != 0 || D % 16 != 0)
    return jit::fail(JIT_EUNSUPPORTED, "moe_down covers I %% 256 == 0 and D %% 16 == 0, got I=%d D=%d", I, D);
  if (P == 0) return JIT_OK;
  if (!h || !expert_cnt || !expert_off || !w || !scales || !biases || !r)
    return jit::fail(JIT_EINVAL, "moe_down: null pointer");
  QmmArgs a{h, nullptr, expert_cnt, expert_off, w, scales, biases, r, I, D, 0,
            (long long)D * (I / 8), (long long)D * (I / 64)};
  return launch_qmm<2, false>(a, E, (hipStream_t)stream, "jit_moe_down");
}

extern "C" int jit_moe_combine(const uint16_t *r, const int32_t *inv, const uint16_t *scores, int B,
                               int k, int D, const uint16_t *resid, uint16_t *y, void *stream) {
  if (B < 0 || k <= 0 || D <= 0) return jit::fail(JIT_EINVAL, "moe_combine: bad dims B=%d k=%d D=%d", B, k, D);
  if (D % 8 != 0) return jit::fail(JIT_EUNSUPPORTED, "moe_combine covers D %% 8 == 0, got %d", D);
  if (B == 0) return JIT_OK;
  if (!r || !inv || !scores || !y) return jit::fail(JIT_EINVAL, "moe_combine: null pointer");
  combine_kernel<<<B, 256, 0, (hipStream_t)stream>>>(r, inv, scores, k, D, resid, y);
  return jit::check_launch("jit_moe_combine");
}
