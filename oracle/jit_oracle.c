/*
 * jit_oracle.c -- CPU restatement of JITEngine's ragged-batch MoE decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP path is compared
 * against; it is linked by tests/, by __graft_entry__.smoke() and by bench.py's
 * cpu_baseline leg, and by nothing the product ships.  Each function cites the
 * reference lines it restates (paths relative to the reference repository;
 * Q36 = engines/qwen3.6-35b-a3b-m4pro/src/jitengine_qwen3_6_35b_a3b_m4pro,
 * FN  = engines/qwen3.8-flash-next-m4pro/src/jitengine_qwen3_8_flash_next_m4pro,
 * FL  = engines/flint-m4pro/src/jitengine_flint_m4pro).
 *
 * Number formats: bf16 is carried as uint16_t bit patterns; every rounding to
 * bf16 is round-to-nearest-even from fp32 (jo_f2bf), the conversion MLX's bf16
 * type performs.  Dot products of the quantized projections and attention are
 * accumulated in float64 ("exact" relative to the fp32 arithmetic of both the
 * reference and the GPU) and then rounded at the points where the reference
 * rounds.  Integer work (top-k ranks, pair packing, page addressing) is exact.
 *
 * Build: oracle/build.py (gcc -O2 -fopenmp -ffp-contract=off -shared).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define JO_OK 0
#define JO_EINVAL -1
#define JO_ENOMEM -2

/* ------------------------------------------------------------------ bf16 */
static inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float jo_bf2f(uint16_t h) { return bf2f(h); }
uint16_t jo_f2bf(float f) { return f2bf(f); }

/* ------------------------------------------------------- exp for x <= 0
 * The router softmax needs the same fp32 bits on CPU and GPU (the expert
 * indices are compared bit for bit), so the build pins its own exp rather than
 * a platform libm or MLX's fast::exp (Q36/kernels/router_topk.py:116).
 * Method: Cody-Waite range reduction x = n ln2 + r with the two-part ln2 split
 * of fdlibm's expf, then the degree-7 Taylor polynomial of e^r on |r| <= ln2/2
 * in Horner form with fused multiply-adds, then scaling by 2^n through the
 * exponent field.  Inputs below -64 return 0 (e^-64 < 2^-92, far below the
 * resolution of a sum that contains e^0 = 1), so no subnormal is ever formed.
 * The HIP kernel (router_topk.hip) executes the identical operation sequence.
 */
float jo_exp_neg(float x) {
  if (!(x > -64.0f)) return 0.0f;
  const float t = x * 1.44269504088896341f;
  const float n = rintf(t);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.42860682030941723e-6f, r);
  float p = 1.98412698412698413e-4f;
  p = fmaf(p, r, 1.38888888888888889e-3f);
  p = fmaf(p, r, 8.33333333333333333e-3f);
  p = fmaf(p, r, 4.16666666666666667e-2f);
  p = fmaf(p, r, 1.66666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int e = (int)n;
  const uint32_t bits = (uint32_t)(e + 127) << 23;
  float sc;
  memcpy(&sc, &bits, 4);
  return p * sc;
}

/* ------------------------------------------------------------ a2 router
 * Softmax of one row of bf16 logits, stored as bf16 gates.  Restates the
 * precise softmax of Q36/kernels/router_topk.py:86-133: fp32 max, exp(x - max),
 * fp32 sum, one reciprocal, multiply, round to bf16.  The reduction order is
 * the build's (MLX's simd_sum order is a hardware detail): 64 lanes, lane l
 * holds indices l, l+64, ... and sums them in that order, then a butterfly over
 * lane offsets 32, 16, 8, 4, 2, 1.
 */
static void softmax_row(const uint16_t *lg, int N, float *e, uint16_t *g) {
  float mx = -INFINITY;
  for (int i = 0; i < N; i++) {
    const float v = bf2f(lg[i]);
    mx = v > mx ? v : mx;
  }
  float part[64];
  for (int l = 0; l < 64; l++) {
    float s = 0.0f;
    for (int i = l; i < N; i += 64) {
      e[i] = jo_exp_neg(bf2f(lg[i]) - mx);
      s = s + e[i];
    }
    part[l] = s;
  }
  for (int o = 32; o >= 1; o >>= 1) {
    float nxt[64];
    for (int l = 0; l < 64; l++) nxt[l] = part[l] + part[l ^ o];
    memcpy(part, nxt, sizeof part);
  }
  const float inv = 1.0f / part[0];
  for (int i = 0; i < N; i++) g[i] = f2bf(e[i] * inv);
}

/* Exact top-k by rank (Q36/kernels/router_topk.py:14-28,135-145): the rank of
 * gate i is #{j : g_j < g_i or (g_j == g_i and j < i)}; gates of rank >= N-k
 * are selected and stored at slot rank-(N-k), i.e. ascending (value, index)
 * order, slot k-1 holding the largest gate, a boundary tie going to the higher
 * index -- the order mx.argpartition(g, kth=-k)[..., -k:] returns on Metal. */
static void topk_rank_row(const uint16_t *g, int N, int k, uint32_t *inds) {
  for (int i = 0; i < N; i++) {
    const float v = bf2f(g[i]);
    int rank = 0;
    for (int j = 0; j < N; j++) {
      const float u = bf2f(g[j]);
      rank += (u < v) || (u == v && j < i);
    }
    if (rank >= N - k) inds[rank - (N - k)] = (uint32_t)i;
  }
}

int jo_topk_from_gates(const uint16_t *gates, int rows, int N, int k, uint32_t *inds) {
  if (rows < 0 || N <= 0 || k <= 0 || k > N) return JO_EINVAL;
  for (int r = 0; r < rows; r++) topk_rank_row(gates + (size_t)r * N, N, k, inds + (size_t)r * k);
  return JO_OK;
}

int jo_softmax_bf16(const uint16_t *logits, int rows, int N, uint16_t *gates) {
  if (rows < 0 || N <= 0) return JO_EINVAL;
  float *e = (float *)malloc(sizeof(float) * (size_t)N);
  if (!e) return JO_ENOMEM;
  for (int r = 0; r < rows; r++) softmax_row(logits + (size_t)r * N, N, e, gates + (size_t)r * N);
  free(e);
  return JO_OK;
}

/* The fused router (Q36/kernels/router_topk.py:72-192; stock chain
 * Q36/model/moe.py:304-315): softmax, rank top-k, gather the k gates and, with
 * norm, divide them by their sum accumulated sequentially in bf16 in slot order
 * (router_topk.py:147-157). */
int jo_router_topk(const uint16_t *logits, int rows, int N, int k, int norm, uint32_t *inds,
                   uint16_t *scores, uint16_t *gates_out) {
  if (rows < 0 || N <= 0 || k <= 0 || k > N) return JO_EINVAL;
  float *e = (float *)malloc(sizeof(float) * (size_t)N);
  uint16_t *g = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)N);
  if (!e || !g) {
    free(e);
    free(g);
    return JO_ENOMEM;
  }
  for (int r = 0; r < rows; r++) {
    softmax_row(logits + (size_t)r * N, N, e, g);
    if (gates_out) memcpy(gates_out + (size_t)r * N, g, sizeof(uint16_t) * (size_t)N);
    uint32_t *ind = inds + (size_t)r * k;
    uint16_t *sc = scores + (size_t)r * k;
    topk_rank_row(g, N, k, ind);
    uint16_t tot = 0;
    for (int j = 0; j < k; j++) {
      sc[j] = g[ind[j]];
      tot = f2bf(bf2f(tot) + bf2f(sc[j]));
    }
    if (norm)
      for (int j = 0; j < k; j++) sc[j] = f2bf(bf2f(sc[j]) / bf2f(tot));
  }
  free(e);
  free(g);
  return JO_OK;
}

/* ------------------------------------------------------------ a3 packing
 * Token-to-expert packing.  Canonical order = stable sort of the flat (row,
 * slot) pairs by expert id (Q36/model/moe.py:151-159 argsort / argsort;
 * FN/model/moe/expert_mlp.py:39-49,147-163 stable argsort, np.unique ->
 * seg_slot, seg_start, seg_cnt, pair_row = pos // k).  Outputs:
 *   order[p]      flat pair index at sorted position p
 *   pair_row[p]   = order[p] / k, the activation row of sorted position p
 *   inv[f]        sorted position of flat pair f (inv[order[p]] = p)
 *   expert_cnt[e], expert_off[e]  pairs per expert and their first position
 *   seg_expert/seg_start/seg_cnt[u], u < n_seg: the non-empty experts ascending
 *   meta[0] = n_seg, meta[1] = max_cnt
 */
int jo_moe_pack(const uint32_t *inds, int P, int k, int E, int32_t *order, int32_t *pair_row,
                int32_t *inv, int32_t *expert_cnt, int32_t *expert_off, int32_t *seg_expert,
                int32_t *seg_start, int32_t *seg_cnt, int32_t *meta) {
  if (P < 0 || k <= 0 || E <= 0 || (P % k) != 0) return JO_EINVAL;
  for (int p = 0; p < P; p++)
    if (inds[p] >= (uint32_t)E) return JO_EINVAL;
  for (int e = 0; e < E; e++) expert_cnt[e] = 0;
  for (int p = 0; p < P; p++) expert_cnt[inds[p]]++;
  int run = 0, u = 0, mc = 0;
  for (int e = 0; e < E; e++) {
    expert_off[e] = run;
    if (expert_cnt[e] > 0) {
      seg_expert[u] = e;
      seg_start[u] = run;
      seg_cnt[u] = expert_cnt[e];
      u++;
    }
    if (expert_cnt[e] > mc) mc = expert_cnt[e];
    run += expert_cnt[e];
  }
  int32_t *next = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
  if (!next) return JO_ENOMEM;
  memcpy(next, expert_off, sizeof(int32_t) * (size_t)E);
  for (int p = 0; p < P; p++) {
    const int pos = next[inds[p]]++;
    order[pos] = p;
    pair_row[pos] = p / k;
    inv[p] = pos;
  }
  free(next);
  meta[0] = u;
  meta[1] = mc;
  return JO_OK;
}

/* ------------------------------------------------- a10 MLX 4-bit affine
 * Layout (Q36/linear.py:101-128, FN/kernels/qmv_row_blocked.py:23-33): a
 * matrix [N, K] is weight uint32 [N, K/8] (element j of row n = nibble j%8 of
 * word j/8, low nibble first), scales and biases bf16 [N, K/64], and
 * w = scale * q + bias.  Dequantize one row into float64. */
static void dequant_row(const uint32_t *w, const uint16_t *s, const uint16_t *b, int K, double *out) {
  for (int j = 0; j < K; j++) {
    const uint32_t q = (w[j >> 3] >> (4 * (j & 7))) & 0xfu;
    out[j] = (double)bf2f(s[j >> 6]) * (double)q + (double)bf2f(b[j >> 6]);
  }
}

/* The segment GEMM's weights (a9, Q36/kernels/gather_qmm_prefill.py:1-257, whose
 * MLX quantized block loader dequantizes into the activation type before the
 * tile MMA): w = bf16(s * q + b), formed as one fp32 fused multiply-add rounded
 * to bf16.  bf16w selects these weights over the exact ones of dequant_row. */
static void dequant_row_w(const uint32_t *w, const uint16_t *s, const uint16_t *b, int K, int bf16w,
                          double *out) {
  if (!bf16w) {
    dequant_row(w, s, b, K, out);
    return;
  }
  for (int j = 0; j < K; j++) {
    const uint32_t q = (w[j >> 3] >> (4 * (j & 7))) & 0xfu;
    out[j] = (double)bf2f(f2bf(fmaf(bf2f(s[j >> 6]), (float)q, bf2f(b[j >> 6]))));
  }
}

int jo_dequant4(const uint32_t *w, const uint16_t *s, const uint16_t *b, int N, int K, int bf16w, double *out) {
  if (N < 0 || K <= 0 || (K % 64) != 0) return JO_EINVAL;
  for (int n = 0; n < N; n++)
    dequant_row_w(w + (size_t)n * (K / 8), s + (size_t)n * (K / 64), b + (size_t)n * (K / 64), K, bf16w,
                  out + (size_t)n * K);
  return JO_OK;
}

/* Quantized projection y[t, n] = sum_j x[t, j] * w(n, j) for T rows, exact
 * (float64) accumulation; out_f64 gets the sums, out_bf16 (if given) their
 * bf16 rounding -- the value QLinear's quantized_matmul returns
 * (Q36/linear.py:146-157). */
int jo_qmm(const uint16_t *x, int T, const uint32_t *w, const uint16_t *s, const uint16_t *b, int N,
           int K, double *out_f64, uint16_t *out_bf16) {
  if (T < 0 || N < 0 || K <= 0 || (K % 64) != 0) return JO_EINVAL;
#pragma omp parallel
  {
    double *row = (double *)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(static)
    for (int n = 0; n < N; n++) {
      dequant_row(w + (size_t)n * (K / 8), s + (size_t)n * (K / 64), b + (size_t)n * (K / 64), K, row);
      for (int t = 0; t < T; t++) {
        const uint16_t *xr = x + (size_t)t * K;
        double acc = 0.0;
        for (int j = 0; j < K; j++) acc += (double)bf2f(xr[j]) * row[j];
        if (out_f64) out_f64[(size_t)t * N + n] = acc;
        if (out_bf16) out_bf16[(size_t)t * N + n] = f2bf((float)acc);
      }
    }
    free(row);
  }
  return JO_OK;
}

/* MLX qmv_fast's per-lane fp32 arithmetic for 4-bit group-64 weights, the
 * reference's "stock" numerics (Q36/kernels/qmv_mrow.py:52-59 load_vector,
 * :103-122 qdot, :140-160 and :179-207 the k-block loop): 32 lanes, lane l
 * covers values [16l, 16l+16) of each 512-wide block; x is pre-scaled by 1,
 * 1/16, 1/256, 1/4096 and summed; the nibbles are masked in place; each block
 * adds scale*accum + sum*bias to the lane's result; the 32 lane results are
 * summed by a butterfly (the simd_sum order is the hardware's, unpinned).
 * Used only as the error yardstick of the no-worse-than-stock criterion
 * (FN/kernels/selfcheck.py:313-331). */
int jo_qmv_mlx_f32(const uint16_t *x, int T, const uint32_t *w, const uint16_t *s,
                   const uint16_t *b, int N, int K, float *out) {
  /* K % 512 is qmv_fast's case; a K with a partial last block (K % 64 == 0, e.g. the
   * 768-wide down projection) leaves the lanes past K out of that block (MLX's plain qmv
   * tail; its lane bits there are not pinned) */
  if (T < 0 || N < 0 || K <= 0 || (K % 64) != 0) return JO_EINVAL;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++) {
    const uint8_t *wb = (const uint8_t *)(w + (size_t)n * (K / 8));
    const uint16_t *sr = s + (size_t)n * (K / 64), *br = b + (size_t)n * (K / 64);
    for (int t = 0; t < T; t++) {
      const uint16_t *xr = x + (size_t)t * K;
      float lane[32];
      for (int l = 0; l < 32; l++) {
        float res = 0.0f;
        for (int kb = 0; kb < K; kb += 512) {
          const int k0 = kb + 16 * l;
          if (k0 >= K) continue;
          float xt[16], sum = 0.0f;
          for (int i = 0; i < 16; i += 4) {
            const float a0 = bf2f(xr[k0 + i]), a1 = bf2f(xr[k0 + i + 1]);
            const float a2 = bf2f(xr[k0 + i + 2]), a3 = bf2f(xr[k0 + i + 3]);
            sum += ((a0 + a1) + a2) + a3;
            xt[i] = a0;
            xt[i + 1] = a1 / 16.0f;
            xt[i + 2] = a2 / 256.0f;
            xt[i + 3] = a3 / 4096.0f;
          }
          float accum = 0.0f;
          for (int i = 0; i < 4; i++) {
            const uint32_t ws = (uint32_t)wb[k0 / 2 + 2 * i] | ((uint32_t)wb[k0 / 2 + 2 * i + 1] << 8);
            accum += (((xt[4 * i] * (float)(ws & 0x000fu)) + xt[4 * i + 1] * (float)(ws & 0x00f0u)) +
                      xt[4 * i + 2] * (float)(ws & 0x0f00u)) +
                     xt[4 * i + 3] * (float)(ws & 0xf000u);
          }
          const float sc = bf2f(sr[k0 / 64]), bi = bf2f(br[k0 / 64]);
          res += sc * accum + sum * bi;
        }
        lane[l] = res;
      }
      for (int o = 16; o >= 1; o >>= 1) {
        float nxt[32];
        for (int l = 0; l < 32; l++) nxt[l] = lane[l] + lane[l ^ o];
        memcpy(lane, nxt, sizeof lane);
      }
      out[(size_t)t * N + n] = lane[0];
    }
  }
  return JO_OK;
}

/* ------------------------------------------------ a4 gate||up + SwiGLU
 * e^x for 0 <= x (the sigmoid's exp(|g|)): the method of jo_exp_neg (Cody-Waite
 * reduction with fdlibm's two-part ln2, degree-7 Taylor polynomial in Horner form
 * with fused multiply-adds), scaled by 2^(n-1) then 2 so that n = 128 (x up to
 * 88.72) stays finite; x > 89 (or NaN) gives x * inf.  The GPU's SwiGLU epilogue
 * (qtile.hpp) executes the identical operation sequence, so both round the same
 * fp32 value to bf16. */
float jo_exp_pos(float x) {
  if (!(x <= 89.0f)) return x * INFINITY;
  const float t = x * 1.44269504088896341f;
  const float n = rintf(t);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.42860682030941723e-6f, r);
  float p = 1.98412698412698413e-4f;
  p = fmaf(p, r, 1.38888888888888889e-3f);
  p = fmaf(p, r, 8.33333333333333333e-3f);
  p = fmaf(p, r, 4.16666666666666667e-2f);
  p = fmaf(p, r, 1.66666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int e = (int)n;
  const uint32_t bits = (uint32_t)(e - 1 + 127) << 23;
  float sc;
  memcpy(&sc, &bits, 4);
  return (p * sc) * 2.0f;
}

/* One pair p (sorted position) against expert e's fused gate||up stack
 * [2I, D]: g, u = x . dequant(W)^T, rounded to bf16; then the exact kernel's
 * bf16 chain (Q36/kernels/expert_solo.py:106-115): sg = SigmoidX(g), sl =
 * bf16(g * sg), h = bf16(sl * u).  SigmoidX (MLX's Sigmoid on bf16,
 * Q36/kernels/expert_solo.py:56-62: y = 1 / (1 + exp(|g|)), g < 0 ? y : 1 - y)
 * evaluates each step in fp32 from bf16 operands and rounds it to bf16, as MLX's
 * bf16 type does for bf16-with-integer arithmetic and its bf16 exp overload:
 *   e = bf16(exp(|g|)); d = bf16(1 + e); y = bf16(1 / d); sg = g < 0 ? y : bf16(1 - y).
 * exp is jo_exp_pos (Metal's exp bits are not reproducible here; the bf16
 * rounding of e hides its last fp32 bits except within 2^-16 of a tie) and the
 * division is the correctly rounded one. */
static inline uint16_t sigmoid_bf16(uint16_t gt) {
  const float ag = fabsf(bf2f(gt));
  const float e = bf2f(f2bf(jo_exp_pos(ag)));
  const float d = bf2f(f2bf(1.0f + e));
  const float y = bf2f(f2bf(1.0f / d));
  return bf2f(gt) < 0.0f ? f2bf(y) : f2bf(1.0f - y);
}

static inline uint16_t swiglu_bf16(uint16_t gt, uint16_t ut) {
  const uint16_t sg = sigmoid_bf16(gt);
  const uint16_t sl = f2bf(bf2f(gt) * bf2f(sg));
  return f2bf(bf2f(sl) * bf2f(ut));
}

int jo_sigmoid_bf16_n(const uint16_t *g, int n, uint16_t *out) {
  if (n < 0) return JO_EINVAL;
  for (int i = 0; i < n; i++) out[i] = sigmoid_bf16(g[i]);
  return JO_OK;
}
uint16_t jo_swiglu_bf16(uint16_t g, uint16_t u) { return swiglu_bf16(g, u); }

/* h[p, :] for every sorted pair p; x [B, D] bf16; stacks [E, 2I, D/8] u32 and
 * [E, 2I, D/64] bf16; pair_row/order from jo_moe_pack; inds the flat expert ids;
 * bf16w: the segment GEMM's bf16 weights (dequant_row_w). */
int jo_moe_gate_up(const uint16_t *x, int B, int D, const uint32_t *inds, int P, const int32_t *order,
                   const int32_t *pair_row, const uint32_t *w, const uint16_t *s, const uint16_t *b,
                   int E, int I, int bf16w, uint16_t *h) {
  if (B < 0 || P < 0 || D <= 0 || (D % 64) != 0 || I <= 0) return JO_EINVAL;
  const size_t ws = (size_t)2 * I * (D / 8), gs = (size_t)2 * I * (D / 64);
#pragma omp parallel
  {
    double *gr = (double *)malloc(sizeof(double) * (size_t)D);
    double *ur = (double *)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic, 4)
    for (int n = 0; n < I; n++) {
      int last_e = -1;
      for (int p = 0; p < P; p++) {
        const int e = (int)inds[order[p]];
        if (e < 0 || e >= E) continue;
        if (e != last_e) {
          dequant_row_w(w + e * ws + (size_t)n * (D / 8), s + e * gs + (size_t)n * (D / 64),
                        b + e * gs + (size_t)n * (D / 64), D, bf16w, gr);
          dequant_row_w(w + e * ws + (size_t)(I + n) * (D / 8), s + e * gs + (size_t)(I + n) * (D / 64),
                        b + e * gs + (size_t)(I + n) * (D / 64), D, bf16w, ur);
          last_e = e;
        }
        const uint16_t *xr = x + (size_t)pair_row[p] * D;
        double ga = 0.0, ua = 0.0;
        for (int j = 0; j < D; j++) {
          const double xv = (double)bf2f(xr[j]);
          ga += xv * gr[j];
          ua += xv * ur[j];
        }
        h[(size_t)p * I + n] = swiglu_bf16(f2bf((float)ga), f2bf((float)ua));
      }
    }
    free(gr);
    free(ur);
  }
  return JO_OK;
}

/* ---------------------------------------------------- a5 down + combine
 * r[p, :] = bf16(h[p] . dequant(Wd_e)^T) for every sorted pair (the down
 * gather's bf16 output, Q36/model/moe.py:193); bf16w as in jo_moe_gate_up. */
int jo_moe_down(const uint16_t *h, int P, int I, const uint32_t *inds, const int32_t *order,
                const uint32_t *w, const uint16_t *s, const uint16_t *b, int E, int D, int bf16w, uint16_t *r) {
  if (P < 0 || I <= 0 || (I % 64) != 0 || D <= 0) return JO_EINVAL;
  const size_t ws = (size_t)D * (I / 8), gs = (size_t)D * (I / 64);
#pragma omp parallel
  {
    double *row = (double *)malloc(sizeof(double) * (size_t)I);
#pragma omp for schedule(dynamic, 16)
    for (int n = 0; n < D; n++) {
      int last_e = -1;
      for (int p = 0; p < P; p++) {
        const int e = (int)inds[order[p]];
        if (e < 0 || e >= E) continue;
        if (e != last_e) {
          dequant_row_w(w + e * ws + (size_t)n * (I / 8), s + e * gs + (size_t)n * (I / 64),
                        b + e * gs + (size_t)n * (I / 64), I, bf16w, row);
          last_e = e;
        }
        const uint16_t *hr = h + (size_t)p * I;
        double acc = 0.0;
        for (int j = 0; j < I; j++) acc += (double)bf2f(hr[j]) * row[j];
        r[(size_t)p * D + n] = f2bf((float)acc);
      }
    }
    free(row);
  }
  return JO_OK;
}

/* y[b, n] = sum over slots j = 0..k-1 of bf16(r_j * score_j), each product
 * rounded to bf16 and the sum accumulated sequentially in bf16 in slot order
 * (Q36/kernels/expert_solo.py:1-6,155-163,307-315; the stock
 * (e * scores[..., None]).sum(-2) of Q36/model/moe.py:286). */
int jo_moe_combine(const uint16_t *r, const int32_t *inv, const uint16_t *scores, int B, int k, int D,
                   uint16_t *y) {
  if (B < 0 || k <= 0 || D <= 0) return JO_EINVAL;
#pragma omp parallel for schedule(static)
  for (int t = 0; t < B; t++) {
    for (int n = 0; n < D; n++) {
      uint16_t acc = 0;
      for (int j = 0; j < k; j++) {
        const uint16_t rv = r[(size_t)inv[t * k + j] * D + n];
        const uint16_t pr = f2bf(bf2f(rv) * bf2f(scores[t * k + j]));
        acc = f2bf(bf2f(acc) + bf2f(pr));
      }
      y[(size_t)t * D + n] = acc;
    }
  }
  return JO_OK;
}

/* ----------------------------------------------------- a6/a7 paged KV
 * Paged pool layout (the build's design; the reference keeps one contiguous
 * [1, Hkv, cap, Dh] buffer per request, Q36/kvcache/kv_cache.py:27-85):
 * pool [num_pages, Hkv, 2, 16 * Dh] bf16; for each kv head part 0 of a page is
 * K chunk-major ([d / 32][slot][d % 32]), part 1 is V dim-major ([d][slot]).
 * Token t of sequence b lives in page page_table[b * max_pages + t / 16], slot
 * t % 16. */
#define JO_PAGE 16

static inline size_t k_index(int page, int Hkv, int Dh, int h, int slot, int d) {
  /* chunk-major K block: [Dh / 32 chunks][16 slots][32 dims] */
  return (((size_t)page * Hkv + h) * 2 + 0) * (size_t)(JO_PAGE * Dh) + (size_t)(d / 32) * (JO_PAGE * 32) +
         (size_t)slot * 32 + (d % 32);
}
static inline size_t v_index(int page, int Hkv, int Dh, int h, int slot, int d) {
  return (((size_t)page * Hkv + h) * 2 + 1) * (size_t)(JO_PAGE * Dh) + (size_t)d * JO_PAGE + slot;
}

/* KVSlot.append restated for pages (Q36/kvcache/kv_cache.py:76-85): the k, v
 * of row b ([B, Hkv, Dh]) go to position pos[b]. */
int jo_kv_append_paged(const uint16_t *k, const uint16_t *v, int B, int Hkv, int Dh,
                       const int32_t *pos, const int32_t *page_table, int max_pages, int num_pages,
                       uint16_t *pool) {
  if (B < 0 || Hkv <= 0 || Dh <= 0) return JO_EINVAL;
  for (int b = 0; b < B; b++) {
    if (pos[b] < 0 || pos[b] / JO_PAGE >= max_pages) return JO_EINVAL;
    const int page = page_table[(size_t)b * max_pages + pos[b] / JO_PAGE];
    if (page < 0 || page >= num_pages) return JO_EINVAL;
    const int slot = pos[b] % JO_PAGE;
    for (int h = 0; h < Hkv; h++)
      for (int d = 0; d < Dh; d++) {
        pool[k_index(page, Hkv, Dh, h, slot, d)] = k[((size_t)b * Hkv + h) * Dh + d];
        pool[v_index(page, Hkv, Dh, h, slot, d)] = v[((size_t)b * Hkv + h) * Dh + d];
      }
  }
  return JO_OK;
}

/* Gather the first n tokens of sequence b into contiguous [Hkv, n, Dh] K and V
 * (the reference's KVSlot layout, the parity contract of the paged pool). */
int jo_kv_gather(const uint16_t *pool, int Hkv, int Dh, const int32_t *page_row, int n, uint16_t *kc,
                 uint16_t *vc) {
  for (int h = 0; h < Hkv; h++)
    for (int t = 0; t < n; t++) {
      const int page = page_row[t / JO_PAGE], slot = t % JO_PAGE;
      for (int d = 0; d < Dh; d++) {
        kc[((size_t)h * n + t) * Dh + d] = pool[k_index(page, Hkv, Dh, h, slot, d)];
        vc[((size_t)h * n + t) * Dh + d] = pool[v_index(page, Hkv, Dh, h, slot, d)];
      }
    }
  return JO_OK;
}

/* Decode attention, one query per row, GQA (q head h reads kv head h / G), over
 * the first lens[b] tokens: softmax(scale * q . K^T) . V, the result of
 * sdpa_decode / mx.fast.scaled_dot_product_attention with mask=None
 * (Q36/kernels/sdpa_decode.py:16-74,448-476; Q36/model/attention.py:70-74),
 * evaluated in float64 and rounded to bf16 once.  q [B, H, Dh], out [B, H, Dh];
 * out64 (may be NULL) receives the float64 values before that rounding. */
int jo_paged_decode_attn(const uint16_t *q, const uint16_t *pool, const int32_t *page_table,
                         int max_pages, const int32_t *lens, int B, int H, int Hkv, int Dh, float scale,
                         uint16_t *out, double *out64) {
  if (B < 0 || H <= 0 || Hkv <= 0 || (H % Hkv) != 0 || Dh <= 0) return JO_EINVAL;
  for (int b = 0; b < B; b++)
    if (lens[b] < 1 || (lens[b] + JO_PAGE - 1) / JO_PAGE > max_pages) return JO_EINVAL;
  const int G = H / Hkv;
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
  for (int b = 0; b < B; b++) {
    for (int h = 0; h < H; h++) {
      const int n = lens[b], kvh = h / G;
      const int32_t *prow = page_table + (size_t)b * max_pages;
      double *sc = (double *)malloc(sizeof(double) * (size_t)n);
      double *acc = (double *)calloc((size_t)Dh, sizeof(double));
      const uint16_t *qh = q + ((size_t)b * H + h) * Dh;
      double mx = -INFINITY;
      for (int t = 0; t < n; t++) {
        const int page = prow[t / JO_PAGE], slot = t % JO_PAGE;
        double dot = 0.0;
        for (int d = 0; d < Dh; d++)
          dot += (double)bf2f(qh[d]) * (double)bf2f(pool[k_index(page, Hkv, Dh, kvh, slot, d)]);
        sc[t] = dot * (double)scale;
        if (sc[t] > mx) mx = sc[t];
      }
      double den = 0.0;
      for (int t = 0; t < n; t++) {
        sc[t] = exp(sc[t] - mx);
        den += sc[t];
      }
      for (int t = 0; t < n; t++) {
        const int page = prow[t / JO_PAGE], slot = t % JO_PAGE;
        for (int d = 0; d < Dh; d++)
          acc[d] += sc[t] * (double)bf2f(pool[v_index(page, Hkv, Dh, kvh, slot, d)]);
      }
      uint16_t *o = out + ((size_t)b * H + h) * Dh;
      for (int d = 0; d < Dh; d++) o[d] = f2bf((float)(acc[d] / den));
      if (out64)
        for (int d = 0; d < Dh; d++) out64[((size_t)b * H + h) * Dh + d] = acc[d] / den;
      free(sc);
      free(acc);
    }
  }
  return JO_OK;
}

/* MLX's decode attention in its own fp32 arithmetic, the reference's "stock"
 * numerics for one query over n keys (the error yardstick of the attention
 * parity tests, as jo_qmv_mlx_f32 is for the projections).  Restated from the
 * reference's transcriptions of MLX's kernels:
 *  - one pass, sdpa_vector (Q36/kernels/sdpa_decode.py:16-74): q pre-scaled in
 *    fp32; 32 simdgroups, simdgroup s taking keys s, s + 32, ...; per key the 32
 *    lanes' 4-element partial dots are simd-summed; online softmax with
 *    max = -FLT_MAX initially, factor = exp(max - new_max), o = o * factor +
 *    exp_score * v; then the 32 simdgroups' (max, sum, o) merge by simd_max /
 *    simd_sum of o * factor, o / sum, cast to bf16;
 *  - two passes, sdpa_vector_2pass_1/_2 (:217-315): `blocks` strided key sets,
 *    each pass-1 block runs the same online softmax and stores its unnormalised o
 *    AS BF16 with fp32 (sum, max); pass 2 takes the max over blocks, sums
 *    exp(m_b - max) * s_b, adds exp(m_b - max) * o_b over blocks j = lane + 32 i
 *    per lane, simd-sums the 32 lanes and divides.
 * Routing (:318-350) is that of the reference's M4 Pro ('s' architecture):
 * two passes when n >= 1024 (or n >= 4096 with GQA), blocks = 64, or for n >
 * 1024 with more than 4 q heads per kv head 128 / 256 / 512 / 1024 up to 8192 /
 * 32768 / 65536 / beyond keys.  Unpinned here: Metal's fast::exp (exp2f(x *
 * log2 e) in fp32 stands in) and simd_sum's order (an xor butterfly).
 * out_f32 [B, H, Dh] receives the fp32 values before the final bf16 cast. */
static float simd_sum32(float *v) {
  float t[32];
  memcpy(t, v, sizeof t);
  for (int o = 16; o >= 1; o >>= 1) {
    float nx[32];
    for (int l = 0; l < 32; l++) nx[l] = t[l] + t[l ^ o];
    memcpy(t, nx, sizeof t);
  }
  return t[0];
}

static inline float mlx_exp(float x) { return exp2f(x * 1.44269504088896341f); }

static int mlx_blocks(int n, int gqa) {
  int blocks = 64;
  if (n > 1024 && gqa > 4) blocks = n <= 8192 ? 128 : n <= 32768 ? 256 : n <= 65536 ? 512 : 1024;
  return blocks;
}

/* one online-softmax run over keys first, first + stride, ... < n of one (q head, kv head):
 * returns (max, sum) and o[Dh] (fp32), the per-simdgroup loop of both kernels */
static void mlx_run(const float *qs, const uint16_t *pool, const int32_t *prow, int Hkv, int Dh, int kvh, int first,
                    int stride, int n, float *m_out, float *s_out, float *o) {
  const int per = Dh / 32;
  float max_score = -3.40282347e38f, sum = 0.0f;
  for (int d = 0; d < Dh; d++) o[d] = 0.0f;
  for (int t = first; t < n; t += stride) {
    const int page = prow[t / JO_PAGE], slot = t % JO_PAGE;
    float lane[32];
    for (int l = 0; l < 32; l++) {
      float sc = 0.0f;
      for (int j = 0; j < per; j++)
        sc += qs[l * per + j] * bf2f(pool[k_index(page, Hkv, Dh, kvh, slot, l * per + j)]);
      lane[l] = sc;
    }
    const float score = simd_sum32(lane);
    const float new_max = fmaxf(max_score, score);
    const float factor = mlx_exp(max_score - new_max);
    const float es = mlx_exp(score - new_max);
    max_score = new_max;
    sum = sum * factor + es;
    for (int d = 0; d < Dh; d++) o[d] = o[d] * factor + es * bf2f(pool[v_index(page, Hkv, Dh, kvh, slot, d)]);
  }
  *m_out = max_score;
  *s_out = sum;
}

int jo_sdpa_mlx_f32(const uint16_t *q, const uint16_t *pool, const int32_t *page_table, int max_pages,
                    const int32_t *lens, int B, int H, int Hkv, int Dh, float scale, uint16_t *out,
                    float *out_f32) {
  if (B < 0 || H <= 0 || Hkv <= 0 || (H % Hkv) != 0 || Dh <= 0 || (Dh % 32) != 0) return JO_EINVAL;
  for (int b = 0; b < B; b++)
    if (lens[b] < 1 || (lens[b] + JO_PAGE - 1) / JO_PAGE > max_pages) return JO_EINVAL;
  const int G = H / Hkv;
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
  for (int b = 0; b < B; b++) {
    for (int h = 0; h < H; h++) {
      const int n = lens[b], kvh = h / G;
      const int32_t *prow = page_table + (size_t)b * max_pages;
      const uint16_t *qh = q + ((size_t)b * H + h) * Dh;
      float *qs = (float *)malloc(sizeof(float) * (size_t)Dh);
      float *res = (float *)malloc(sizeof(float) * (size_t)Dh);
      for (int d = 0; d < Dh; d++) qs[d] = scale * bf2f(qh[d]);
      const int two_pass = n >= 1024 || (Hkv < H && n >= 4096);
      const int nb = two_pass ? mlx_blocks(n, G) : 32;
      float *ms = (float *)malloc(sizeof(float) * (size_t)nb);
      float *ss = (float *)malloc(sizeof(float) * (size_t)nb);
      float *os = (float *)malloc(sizeof(float) * (size_t)nb * Dh);
      for (int blk = 0; blk < nb; blk++) {
        mlx_run(qs, pool, prow, Hkv, Dh, kvh, blk, nb, n, &ms[blk], &ss[blk], os + (size_t)blk * Dh);
        if (two_pass)  /* pass 1 stores o as bf16 */
          for (int d = 0; d < Dh; d++) os[(size_t)blk * Dh + d] = bf2f(f2bf(os[(size_t)blk * Dh + d]));
      }
      if (!two_pass) {  /* sdpa_vector's merge of its 32 simdgroups */
        float new_max = ms[0];
        for (int j = 1; j < 32; j++) new_max = fmaxf(new_max, ms[j]);
        float v[32];
        for (int j = 0; j < 32; j++) v[j] = ss[j] * mlx_exp(ms[j] - new_max);
        const float total = simd_sum32(v);
        for (int d = 0; d < Dh; d++) {
          for (int j = 0; j < 32; j++) v[j] = os[(size_t)j * Dh + d] * mlx_exp(ms[j] - new_max);
          const float od = simd_sum32(v);
          res[d] = total == 0.0f ? od : od / total;
        }
      } else {  /* sdpa_vector_2pass_2: lane l holds blocks l, l + 32, ... */
        float mx = -3.40282347e38f;
        float lanev[32];
        for (int l = 0; l < 32; l++) {
          float m = -3.40282347e38f;
          for (int i = 0; i < nb / 32; i++) m = fmaxf(m, ms[l + 32 * i]);
          lanev[l] = m;
        }
        for (int l = 0; l < 32; l++) mx = fmaxf(mx, lanev[l]);
        for (int l = 0; l < 32; l++) {
          float acc = 0.0f;
          for (int i = 0; i < nb / 32; i++) acc += mlx_exp(ms[l + 32 * i] - mx) * ss[l + 32 * i];
          lanev[l] = acc;
        }
        const float total = simd_sum32(lanev);
        for (int d = 0; d < Dh; d++) {
          for (int l = 0; l < 32; l++) {
            float acc = 0.0f;
            for (int i = 0; i < nb / 32; i++)
              acc += mlx_exp(ms[l + 32 * i] - mx) * os[(size_t)(l + 32 * i) * Dh + d];
            lanev[l] = acc;
          }
          const float od = simd_sum32(lanev);
          res[d] = total == 0.0f ? od : od / total;
        }
      }
      for (int d = 0; d < Dh; d++) {
        out[((size_t)b * H + h) * Dh + d] = f2bf(res[d]);
        if (out_f32) out_f32[((size_t)b * H + h) * Dh + d] = res[d];
      }
      free(qs);
      free(res);
      free(ms);
      free(ss);
      free(os);
    }
  }
  return JO_OK;
}

int jo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void jo_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------- decoder block glue
 * RMSNorm as mx.fast.rms_norm computes it for the decoder layer
 * (Q36/model/model.py:65-80, Q36/model/attention.py:59-60): r = 1/sqrt(mean(x^2)
 * + eps) (float64 here), y = bf16(w * bf16(x * r)).  With resid, the normed row
 * is h = bf16(x + resid) (written to h_out if given). */
int jo_rmsnorm(const uint16_t *x, const uint16_t *resid, int rows, int D, const uint16_t *w, float eps,
               uint16_t *h_out, uint16_t *y) {
  if (rows < 0 || D <= 0) return JO_EINVAL;
  float *v = (float *)malloc(sizeof(float) * (size_t)D);
  if (!v) return JO_ENOMEM;
  for (int r = 0; r < rows; r++) {
    double ss = 0.0;
    for (int i = 0; i < D; i++) {
      float a = bf2f(x[(size_t)r * D + i]);
      if (resid) a = bf2f(f2bf(a + bf2f(resid[(size_t)r * D + i])));
      if (resid && h_out) h_out[(size_t)r * D + i] = f2bf(a);
      v[i] = a;
      ss += (double)a * (double)a;
    }
    const double rr = 1.0 / sqrt(ss / D + (double)eps);
    for (int i = 0; i < D; i++)
      y[(size_t)r * D + i] = f2bf(bf2f(w[i]) * bf2f(f2bf((float)((double)v[i] * rr))));
  }
  free(v);
  return JO_OK;
}

/* q/k RMSNorm + RoPE + KV append (Qwen3_5MoeAttention.step without the output
 * gate, Q36/model/attention.py:99-119): per head of 128 dims, RMSNorm with the
 * q or k norm weight, then RoPE with traditional = False (mx.fast.rope): pairs
 * (i, i + 64) rotated by angle = fp32(pos) * inv_freq[i] -- the fp32 product
 * MLX forms -- with cos/sin and the rotation in float64, rounded to bf16 once.
 * q -> q_out [B, H, 128]; k and v -> the pool at pos[b] (jo_kv_append_paged's
 * layout). */
int jo_qk_norm_rope_append(const uint16_t *qkv, int B, int H, int Hkv, const uint16_t *qn,
                           const uint16_t *kn, float eps, const float *inv_freq, const int32_t *pos,
                           const int32_t *page_table, int max_pages, int num_pages, uint16_t *pool,
                           uint16_t *q_out) {
  if (B < 0 || H <= 0 || Hkv <= 0) return JO_EINVAL;
  const int Dh = 128, nh = H + 2 * Hkv;
  for (int b = 0; b < B; b++) {
    if (pos[b] < 0 || pos[b] / JO_PAGE >= max_pages) return JO_EINVAL;
    const int page = page_table[(size_t)b * max_pages + pos[b] / JO_PAGE];
    if (page < 0 || page >= num_pages) return JO_EINVAL;
    const int slot = pos[b] % JO_PAGE;
    for (int hd = 0; hd < nh; hd++) {
      const uint16_t *src = qkv + ((size_t)b * nh + hd) * Dh;
      if (hd >= H + Hkv) {
        const int h = hd - H - Hkv;
        for (int d = 0; d < Dh; d++) pool[v_index(page, Hkv, Dh, h, slot, d)] = src[d];
        continue;
      }
      const uint16_t *nw = hd < H ? qn : kn;
      double ss = 0.0;
      for (int d = 0; d < Dh; d++) ss += (double)bf2f(src[d]) * (double)bf2f(src[d]);
      const double rr = 1.0 / sqrt(ss / Dh + (double)eps);
      float xn[128];
      for (int d = 0; d < Dh; d++) xn[d] = bf2f(f2bf(bf2f(nw[d]) * bf2f(f2bf((float)((double)bf2f(src[d]) * rr)))));
      uint16_t out[128];
      for (int i = 0; i < 64; i++) {
        const float ang = (float)pos[b] * inv_freq[i];
        const double c = cos((double)ang), s = sin((double)ang);
        out[i] = f2bf((float)(xn[i] * c - xn[i + 64] * s));
        out[i + 64] = f2bf((float)(xn[i] * s + xn[i + 64] * c));
      }
      if (hd < H) {
        memcpy(q_out + ((size_t)b * H + hd) * Dh, out, sizeof out);
      } else {
        for (int d = 0; d < Dh; d++) pool[k_index(page, Hkv, Dh, hd - H, slot, d)] = out[d];
      }
    }
  }
  return JO_OK;
}

/* ------------------------------------------------- packed tile layout
 * The build's MI355X layout of a quantized stack [E, N, K] (no counterpart in
 * the reference): per (expert, block of 16 rows) a block of GP = K / 128 group
 * pairs, GP * 1152 bytes: first GP nibble tiles of 1024 bytes -- tile gp holds,
 * for lane l = 16 j + r (j = l / 16, r = l % 16), words 2j, 2j+1 of group 2gp
 * and words 2j, 2j+1 of group 2gp+1 of row 16 rb + r (word w of group g = word
 * 8g + w of the row), each with its nibbles reordered as below -- then GP scale
 * tiles of 128 bytes: tile gp holds, for row r, (scale[2gp], scale[2gp+1],
 * bias[2gp], bias[2gp+1]) bf16. */
/* Nibble order of a packed-layout word: q0, q2, q4, q6 at nibble positions 0-3 and
 * q1, q3, q5, q7 at 4-7 (the MLX word holds q_i at position i). */
static uint32_t nibbles_natural(uint32_t w) {
  uint32_t r = 0;
  for (int i = 0; i < 8; i++) {
    const uint32_t q = (w >> (4 * i)) & 0xFu;
    const int pos = (i % 2 == 0) ? i / 2 : 4 + i / 2;
    r |= q << (4 * pos);
  }
  return r;
}

int jo_q4_prepack(const uint32_t *w, const uint16_t *s, const uint16_t *b, int E, int N, int K,
                  uint8_t *out) {
  if (E <= 0 || N <= 0 || K <= 0 || (N % 16) != 0 || (K % 128) != 0) return JO_EINVAL;
  const int GP = K / 128, NRB = N / 16, G = K / 64, KW = K / 8;
  for (int e = 0; e < E; e++)
    for (int rb = 0; rb < NRB; rb++)
      for (int gp = 0; gp < GP; gp++) {
        uint8_t *blk = out + ((size_t)e * NRB + rb) * GP * 1152; /* GP nibble tiles, then GP scale tiles */
        uint8_t *t = blk + (size_t)gp * 1024;
        for (int l = 0; l < 64; l++) {
          const int j = l / 16, r = l % 16;
          const uint32_t *wr = w + ((size_t)e * N + rb * 16 + r) * KW;
          const uint32_t words[4] = {nibbles_natural(wr[8 * (2 * gp) + 2 * j]),
                                     nibbles_natural(wr[8 * (2 * gp) + 2 * j + 1]),
                                     nibbles_natural(wr[8 * (2 * gp + 1) + 2 * j]),
                                     nibbles_natural(wr[8 * (2 * gp + 1) + 2 * j + 1])};
          memcpy(t + 16 * l, words, 16);
        }
        for (int r = 0; r < 16; r++) {
          const size_t row = (size_t)e * N + rb * 16 + r;
          const uint16_t v[4] = {s[row * G + 2 * gp], s[row * G + 2 * gp + 1], b[row * G + 2 * gp],
                                 b[row * G + 2 * gp + 1]};
          memcpy(blk + (size_t)GP * 1024 + (size_t)gp * 128 + 8 * r, v, 8);
        }
      }
  return JO_OK;
}

/* ---------------------------------------------------------- f.4 sampler
 * Token sampling in mlx_lm's order (Q36/sampler.py): logprobs_from_logits
 * (:295-297), the greedy draw (Sampler.__call__, :371-374) and
 * _sample_exact_full (:451-476), which is bit for bit the stock chain
 * (apply_top_p :300-312, apply_top_k :315-318, categorical), restated with
 * the reference's own steps: one stable ascending argsort, the top-p mask on
 * the cumulative mass, the top-k cut v = sv[n-k] / above / first /
 * cut = first + (k - above), x = bf16(sv * bf16(1/T)), w = exp(x - max),
 * exclusive cumulative weights in vocabulary order and count(cdf <= u sum) - 1.
 * The fp32 reductions whose association MLX fixes inside its kernels
 * (logsumexp's sum, the cumsums, sum(w)) are exact integer sums of 2^42-scaled
 * terms here (the GPU path adds in another order and must reach the same
 * bits); exp is jo_exp_neg and ln is jo_log_ge1 (Metal's bits are not
 * reproducible here).  Where no position survives top_p the greedy token is
 * drawn (the reference's windowed and full chains disagree there).
 */

/* ln s for 1 <= s: s = 2^k f, f in [sqrt(1/2), sqrt(2)], ln f = 2 atanh(z),
 * z = (f - 1) / (f + 1), by the odd series through z^11 (Horner on z^2), then
 * k ln2 + ln f with one fused multiply-add. */
float jo_log_ge1(float s) {
  uint32_t u;
  memcpy(&u, &s, 4);
  int k = (int)((u >> 23) & 0xffu) - 127;
  const uint32_t fu = (u & 0x007fffffu) | 0x3f800000u;
  float f;
  memcpy(&f, &fu, 4);
  if (f > 1.41421356f) {
    f = f * 0.5f;
    k += 1;
  }
  const float z = (f - 1.0f) / (f + 1.0f);
  const float z2 = z * z;
  float p = 9.09090909090909091e-2f;
  p = fmaf(p, z2, 1.11111111111111111e-1f);
  p = fmaf(p, z2, 1.42857142857142857e-1f);
  p = fmaf(p, z2, 2.0e-1f);
  p = fmaf(p, z2, 3.33333333333333333e-1f);
  p = fmaf(p, z2, 1.0f);
  const float lf = (z + z) * p;
  return fmaf((float)k, 0.693147182464599609375f, lf);
}

static inline uint64_t fix42(float w) { return (uint64_t)(w * 0x1p42f); }

/* c rounded to nearest even at `bits` significant bits, times 2^scale_exp */
static float u64_round(uint64_t c, int bits, int scale_exp) {
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
  return ldexpf((float)m, sh + scale_exp);
}

float jo_fix42_to_bf16(uint64_t c) { return u64_round(c, 8, -42); }

/* lse of one row: bf16(m0 + ln(S 2^-42 rounded to fp32)), S = sum floor(e^(x - m0) 2^42) */
static float row_lse(const uint16_t *x, int V) {
  float m0 = -INFINITY;
  for (int i = 0; i < V; i++) m0 = fmaxf(m0, bf2f(x[i]));
  uint64_t S = 0;
  for (int i = 0; i < V; i++) S += fix42(jo_exp_neg(bf2f(x[i]) - m0));
  return bf2f(f2bf(m0 + jo_log_ge1(u64_round(S, 24, -42))));
}

int jo_logprobs_rows(const uint16_t *x, int B, int V, uint16_t *lp) {
  if (B < 0 || V <= 0) return JO_EINVAL;
  for (int b = 0; b < B; b++) {
    const uint16_t *r = x + (size_t)b * V;
    const float lse = row_lse(r, V);
    for (int i = 0; i < V; i++) lp[(size_t)b * V + i] = f2bf(bf2f(r[i]) - lse);
  }
  return JO_OK;
}

typedef struct {
  float v;
  int i;
} jo_vi;

static int cmp_vi(const void *a, const void *b) {
  const jo_vi *p = (const jo_vi *)a, *q = (const jo_vi *)b;
  if (p->v < q->v) return -1;
  if (p->v > q->v) return 1;
  return (p->i > q->i) - (p->i < q->i);
}

/* the first index of the largest value; NaN never wins, a row without a number gives 0 */
static int first_max(const float *lp, int V) {
  int best = -1;
  for (int i = 0; i < V; i++)
    if (lp[i] == lp[i] && (best < 0 || lp[i] > lp[best])) best = i;
  return best < 0 ? 0 : best;
}

/* temperature <= 0: greedy.  u: [B] uniforms (clamped to [0, 1 - 2^-24]).
 * w_out (optional, [B, V]): each row's integer weights W in vocabulary order
 * (all 0 for a greedy or degenerate row). */
int jo_sample_rows(const uint16_t *x, int B, int V, double temperature, double top_p, int top_k,
                   const float *u, int32_t *tok, uint64_t *w_out) {
  if (B < 0 || V <= 0 || top_k < 0) return JO_EINVAL;
  const int greedy = !(temperature > 0.0);
  const float inv_t = greedy ? 0.0f : bf2f(f2bf((float)(1.0 / temperature)));
  const int topp = top_p > 0.0 && top_p < 1.0;
  const float thr = topp ? bf2f(f2bf((float)(1.0 - top_p))) : 0.0f;
  const int k = top_k >= V ? 0 : top_k;
  float *lp = (float *)malloc(sizeof(float) * V), *sv = (float *)malloc(sizeof(float) * V);
  jo_vi *s = (jo_vi *)malloc(sizeof(jo_vi) * V);
  uint64_t *W = (uint64_t *)malloc(sizeof(uint64_t) * V);
  if (!lp || !sv || !s || !W) {
    free(lp); free(sv); free(s); free(W);
    return JO_ENOMEM;
  }
  for (int b = 0; b < B; b++) {
    const uint16_t *r = x + (size_t)b * V;
    const float lse = row_lse(r, V);
    for (int i = 0; i < V; i++) lp[i] = bf2f(f2bf(bf2f(r[i]) - lse));
    if (w_out) memset(w_out + (size_t)b * V, 0, sizeof(uint64_t) * V);
    if (greedy) {
      tok[b] = first_max(lp, V);
      continue;
    }
    /* idx = argsort(lp) (stable, ascending), sv = lp[idx] */
    for (int i = 0; i < V; i++) {
      s[i].v = lp[i];
      s[i].i = i;
    }
    qsort(s, V, sizeof(jo_vi), cmp_vi);
    for (int p = 0; p < V; p++) sv[p] = s[p].v;
    /* top-p: cum = cumsum(exp(sv)) over bf16 exponentials; sv = where(cum > thr, sv, -inf) */
    if (topp) {
      uint64_t cum = 0;
      for (int p = 0; p < V; p++) {
        cum += fix42(bf2f(f2bf(jo_exp_neg(sv[p]))));
        if (!(u64_round(cum, 8, -42) > thr)) sv[p] = -INFINITY;
      }
    }
    if (!(sv[V - 1] > -INFINITY)) {  /* nothing survived top-p */
      tok[b] = first_max(lp, V);
      continue;
    }
    /* top-k: v = sv[n-k]; keep sv > v, or sv == v at positions < first + (k - above) */
    if (k > 0) {
      const float v = sv[V - k];
      int above = 0, first = 0;
      for (int p = 0; p < V; p++) {
        above += sv[p] > v;
        first += sv[p] < v;
      }
      const int cut = first + (k - above);
      for (int p = 0; p < V; p++)
        if (!(sv[p] > v || (sv[p] == v && p < cut))) sv[p] = -INFINITY;
    }
    /* x = put_along_axis(zeros, idx, sv) * inv_t in bf16, then fp32; w = exp(x - max x) */
    float m = -INFINITY;
    for (int p = 0; p < V; p++) {
      sv[p] = bf2f(f2bf(sv[p] * inv_t));
      m = fmaxf(m, sv[p]);
    }
    for (int p = 0; p < V; p++) W[s[p].i] = fix42(jo_exp_neg(sv[p] - m));
    /* cdf = exclusive cumsum in vocabulary order; token = count(cdf <= u * sum) - 1 */
    uint64_t T = 0;
    for (int i = 0; i < V; i++) T += W[i];
    if (w_out) memcpy(w_out + (size_t)b * V, W, sizeof(uint64_t) * V);
    float uu = u[b];
    uu = fminf(fmaxf(uu, 0.0f), 0x1.fffffep-1f);
    const uint64_t A = (uint64_t)(uu * 4294967296.0f);
    const uint64_t U = A * (T >> 32) + ((A * (T & 0xffffffffull)) >> 32);
    uint64_t C = 0;
    int count = 0;
    for (int i = 0; i < V; i++) {
      count += C <= U;
      C += W[i];
    }
    tok[b] = count - 1;
  }
  free(lp); free(sv); free(s); free(W);
  return JO_OK;
}

/* Threefry-2x32 with 20 rounds (Salmon, Moraes, Dror, Shaw, "Parallel random
 * numbers: as easy as 1, 2, 3", SC'11; the Random123 library): rotation
 * constants 13 15 26 6 17 29 16 24, key-schedule parity 0x1BD11BDA, a key
 * injection after every 4 rounds.  MLX's random bits use it (the reference's
 * replay, Q36/sampler.py:160-177). */
void jo_threefry2x32(const uint32_t *key, const uint32_t *ctr, uint32_t *out) {
  static const int rot[8] = {13, 15, 26, 6, 17, 29, 16, 24};
  const uint32_t ks[3] = {key[0], key[1], key[0] ^ key[1] ^ 0x1BD11BDAu};
  uint32_t x0 = ctr[0] + ks[0], x1 = ctr[1] + ks[1];
  for (int i = 0; i < 5; i++) {
    for (int q = 0; q < 4; q++) {
      const int r = rot[(i & 1) * 4 + q];
      x0 += x1;
      x1 = (x1 << r) | (x1 >> (32 - r));
      x1 ^= x0;
    }
    x0 += ks[(i + 1) % 3];
    x1 += ks[(i + 2) % 3] + (uint32_t)(i + 1);
  }
  out[0] = x0;
  out[1] = x1;
}

/* u[b] = min(fp32(y0) / 2^32, 1 - 2^-24), y = threefry(keys[b], (0, 0)):
 * mx.random.uniform(shape=(1,), key) (Sampler.uniform, Q36/sampler.py:367-369). */
void jo_threefry_uniform(const uint32_t *keys, int B, float *u) {
  const uint32_t zero[2] = {0u, 0u};
  for (int b = 0; b < B; b++) {
    uint32_t y[2];
    jo_threefry2x32(keys + 2 * b, zero, y);
    u[b] = fminf((float)y[0] / 4294967296.0f, 0x1.fffffep-1f);
  }
}
