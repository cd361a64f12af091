// Token sampling over rows of bf16 logits for gfx950: log-probabilities, the greedy draw, and
// temperature / top-p / top-k draws in mlx_lm's order (Q36/sampler.py:320-383), one 1024-thread
// workgroup per row.
//
// Definitions (shared with the CPU restatement, oracle/jit_oracle.c):
//   lse  = bf16(m0 + ln s), m0 = the row's largest logit, s = S 2^-42 rounded to fp32, where
//          S = sum_i floor(e^(x_i - m0) 2^42) (an integer, so the order of the additions is free)
//   lp_i = bf16(x_i - lse)                                   (logprobs_from_logits, :295-297)
//   greedy: the first index of the largest lp                (mx.argmax, :373-374)
//   sort order: ascending (lp, index), -0 tying +0           (the stable argsort, :458-459)
//   top-p: cum_r = sum over sorted positions <= r of floor(bf16(e^lp) 2^42), survivor iff
//          bf16(cum_r 2^-42) > bf16(1 - top_p)                (:460-462; apply_top_p :300-312)
//   top-k: of the survivors, the k largest by (value desc, index asc)   (:463-469)
//   x_i  = bf16(lp_i * bf16(1 / T)) over the kept, m = max x, W_i = floor(e^(x_i - m) 2^42)
//   draw: C_i = sum_{j < i} W_j in vocabulary order, U = floor(u sum(W)), token = the last i
//         with C_i <= U                                         (:470-476)
// Every sum is an exact integer sum, so the histogram selection below reaches the bits of the
// restatement's sort-based chain.  Where no token survives top-p (bf16 mass below 1 - top_p,
// only for top_p under about 0.03) the greedy token is drawn.
//
// Selection without a sort: the bf16 log-probabilities are <= 0, so their magnitudes index a
// 32,768-bin count histogram in LDS (128 KB); the cut points of top-p and top-k are found by
// scans over the bins (the mass of a bin is its count times the bin value's weight).  Only the
// tie group at the top-k / top-p cut needs the vocabulary order: its members' ranks come from a
// counting pass.
#include <cstring>
#include <mutex>

#include "common.hpp"
#include "fmath.hpp"

namespace {

using namespace fmath;

constexpr int kThreads = 1024, kWaves = 16;
constexpr int kStep = 512;        // values a wave covers per step: 64 lanes x 8
constexpr int kKeys = 32768;      // histogram bins: the magnitudes of values <= 0
constexpr int kBinsPerThread = kKeys / kThreads;
constexpr int kHistSlots = kKeys + kKeys / kBinsPerThread;  // the LDS histogram with its pad words
static_assert(kKeys % (4 * kThreads) == 0, "the histogram copy takes whole 16-byte words a thread");
constexpr int kMaxV = 1 << 19;    // (2^42-scaled sums of at most 2^20 terms stay below 2^62)
constexpr int kMaxSteps = (kMaxV / (kWaves * 8) * 8 + kStep - 1) / kStep;  // steps of a wave's range

enum Mode { kLogprobs = 0, kGreedy = 1, kSample = 2 };

struct SplitScratch;  // the split launches' partials (below)

struct SampleArgs {
  const uint16_t *logits;
  int V;
  float inv_t, thr;  // bf16 values; thr > 0 turns top-p on
  int k;             // 0: no top-k
  const float *u;
  int32_t *tok;
  uint16_t *lp;
  int ns;    // > 0: the row's max and integer sum come as ns slice partials from the split launches
  int hist;  // (ns > 0) the row's histogram comes from split_hist_kernel
  SplitScratch *sp;  // the partials of the split launches (a caller's workspace or the library's array)
};

// ascending-order key of a log-probability (a bf16 value <= 0): 0x7fff - magnitude, so that
// +0 and -0 tie at the top and -inf sits at 0x7f
__device__ __forceinline__ int key_of(float lp) { return 0x7fff - (int)((__float_as_uint(lp) >> 16) & 0x7fffu); }
__device__ __forceinline__ float value_of(int key) { return __uint_as_float((0x8000u | (uint32_t)(0x7fff - key)) << 16); }

__device__ __forceinline__ float bf16r(float x) { return bf2f(f2bf(x)); }

// the LDS slot of histogram bin k (one pad word after every kBinsPerThread bins)
__device__ __forceinline__ int hslot(int k) { return k + k / kBinsPerThread; }

// ---- workgroup reductions and scans (every thread of the workgroup calls them) ----
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// inclusive prefix over the wave's lanes
template <typename T>
__device__ __forceinline__ T wave_incl(T v) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const T n = __shfl_up(v, o, 64);
    if (l >= o) v += n;
  }
  return v;
}

struct Shared {
  float f[kWaves];
  uint64_t q[kWaves];
  uint64_t qx[kWaves];
  int cut[8];
};

__device__ __forceinline__ float wg_max(float v, Shared &sh) {
  v = wave_max(v);
  __syncthreads();
  if (lane_id() == 0) sh.f[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = sh.f[0];
#pragma unroll
  for (int w = 1; w < kWaves; w++) m = fmaxf(m, sh.f[w]);
  return m;
}

__device__ __forceinline__ uint64_t wg_sum(uint64_t v, Shared &sh) {
  v = wave_sum(v);
  __syncthreads();
  if (lane_id() == 0) sh.q[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t s = 0;
#pragma unroll
  for (int w = 0; w < kWaves; w++) s += sh.q[w];
  return s;
}

// exclusive prefix over the workgroup's threads in thread order (rev: in reverse thread order)
template <bool kRev>
__device__ __forceinline__ uint64_t wg_excl(uint64_t v, Shared &sh) {
  const int t = kRev ? kThreads - 1 - (int)threadIdx.x : (int)threadIdx.x;
  // kRev: lanes and waves are walked from the top, so the wave scan runs over the mirrored lane
  // (a shuffle of lane 63 - l) and the wave totals are combined from the last wave down
  uint64_t x = kRev ? __shfl(v, 63 - lane_id(), 64) : v;
  const uint64_t inc = wave_incl(x);
  __syncthreads();
  if (lane_id() == 63) sh.qx[t >> 6] = inc;
  __syncthreads();
  uint64_t base = 0;
  for (int w = 0; w < (t >> 6); w++) base += sh.qx[w];
  const uint64_t ex = base + inc - x;
  return kRev ? __shfl(ex, 63 - lane_id(), 64) : ex;
}

// ---- the row, a wave's contiguous range of it at a time ----
// wave w covers [w R, min(V, (w + 1) R)), R a multiple of 8; step s of the wave covers 512
// values, lane l the 8 consecutive ones from s + 8 l (kVec: one 16-byte load)
struct Range {
  int lo, hi;
};

__device__ __forceinline__ Range wave_range(int V) {
  const int R = ((V + kWaves * 8 - 1) / (kWaves * 8)) * 8;
  const int w = threadIdx.x >> 6;
  return Range{min(V, w * R), min(V, (w + 1) * R)};
}

// the lane's 8 values of a step from i0 (kVec: one 16-byte load; else element loads, -inf past hi)
struct Raw8 {
  uint32_t w[4];
};

template <bool kVec>
__device__ __forceinline__ Raw8 load8(const uint16_t *row, int i0, int hi) {
  Raw8 r;
  if (kVec) {
    const uint4 q = i0 < hi ? *(const uint4 *)(row + i0) : make_uint4(0u, 0u, 0u, 0u);
    r.w[0] = q.x, r.w[1] = q.y, r.w[2] = q.z, r.w[3] = q.w;
  } else {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t lo = i0 + 2 * j < hi ? row[i0 + 2 * j] : 0xff80u;
      const uint32_t hi16 = i0 + 2 * j + 1 < hi ? row[i0 + 2 * j + 1] : 0xff80u;
      r.w[j] = lo | (hi16 << 16);
    }
  }
  return r;
}

__device__ __forceinline__ float val(const Raw8 &r, int j) {
  return (j & 1) ? bf2f_hi(r.w[j >> 1]) : bf2f(r.w[j >> 1] & 0xffffu);
}

constexpr int kAhead = 8;  // steps whose loads a wave issues before it uses the first

// f(i0, raw, n) for every step of the wave's range in order (n = the lane's values in range);
// the loads of kAhead steps are in flight together.  The step condition is uniform over the
// wave, so f may use cross-lane operations.
template <bool kVec, typename F>
__device__ __forceinline__ void for_steps(const uint16_t *row, int V, F &&f) {
  const Range r = wave_range(V);
  const int l8 = 8 * lane_id();
  for (int s = r.lo; s < r.hi; s += kStep * kAhead) {
    Raw8 q[kAhead];
#pragma unroll
    for (int u = 0; u < kAhead; u++) q[u] = load8<kVec>(row, s + u * kStep + l8, r.hi);
#pragma unroll
    for (int u = 0; u < kAhead; u++)
      if (s + u * kStep < r.hi) f(s + u * kStep + l8, q[u], max(0, min(8, r.hi - (s + u * kStep + l8))));
  }
}

template <bool kVec, typename F>
__device__ __forceinline__ void for_each(const uint16_t *row, int V, F &&f) {
  for_steps<kVec>(row, V, [&](int i0, const Raw8 &q, int n) {
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (j < n) f(i0 + j, val(q, j));
  });
}

__global__ __launch_bounds__(kThreads) void threefry_uniform_kernel(const uint32_t *__restrict__ keys, int B,
                                                                    float *__restrict__ u) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  // Threefry-2x32 with 20 rounds (Salmon et al., SC'11; Random123): counter (0, 0) under the
  // row's key; the draw's uniform is the first output word / 2^32, clamped below 1
  const uint32_t k0 = keys[2 * b], k1 = keys[2 * b + 1];
  const uint32_t ks[3] = {k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
  const int rot[8] = {13, 15, 26, 6, 17, 29, 16, 24};
  uint32_t x0 = ks[0], x1 = ks[1];
#pragma unroll
  for (int i = 0; i < 5; i++) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int r = rot[(i & 1) * 4 + q];
      x0 += x1;
      x1 = (x1 << r) | (x1 >> (32 - r));
      x1 ^= x0;
    }
    x0 += ks[(i + 1) % 3];
    x1 += ks[(i + 2) % 3] + (uint32_t)(i + 1);
  }
  u[b] = fminf((float)x0 / 4294967296.0f, 0x1.fffffep-1f);
}

constexpr int kSplitThreads = 256, kSplitWaves = kSplitThreads / 64;
constexpr int kSplitRows = 64, kSplitMax = 64;  // rows, slices per row
constexpr int kSplitMin = 2048;                  // values a slice holds at least

// a draw's cut, from sample_rows_kernel to the slice launches (done: the token is written)
struct SplitCut {
  int key_t, r_lo, r_hi, partial, done;
  float lse, m;
};

struct SplitScratch {
  float max[kSplitRows][kSplitMax];
  unsigned long long sum[kSplitRows][kSplitMax];
  int idx[kSplitRows][kSplitMax];             // greedy: first index; draws: members of key_t
  unsigned long long wsum[kSplitRows][kSplitMax];  // draws: the slice's total weight
  SplitCut cut[kSplitRows];
  uint32_t hist[kSplitRows][kKeys];  // draws with a cut: the row's histogram of lp keys
};
// The library's own partials, for the entry points without a workspace: every device holds its copy
// until the process ends.  On the host `g_split` names a stand-in, never device memory: host code
// only passes the per-device address hipGetSymbolAddress returns (split_scratch_of_current_device).
__device__ __align__(16) SplitScratch g_split;

template <int kMode, bool kVec>
__global__ __launch_bounds__(kThreads) void sample_rows_kernel(const SampleArgs a) {
  __shared__ Shared sh;
  const int b = blockIdx.x, t = threadIdx.x, l = lane_id();
  const int V = a.V;
  const uint16_t *row = a.logits + (long long)b * V;

  // log-sum-exp: the largest logit, then the exact integer sum of the 2^42-scaled exponentials
  // (a.ns > 0: combined from the slice partials of split_max_kernel / split_sum_kernel)
  float m0 = -INFINITY;
  uint64_t S = 0;
  if (a.ns > 0) {
    m0 = wg_max(t < a.ns ? a.sp->max[b][t] : -INFINITY, sh);
    S = wg_sum(t < a.ns ? a.sp->sum[b][t] : 0ull, sh);
  } else {
    for_each<kVec>(row, V, [&](int, float x) { m0 = fmaxf(m0, x); });
    m0 = wg_max(m0, sh);
    for_each<kVec>(row, V, [&](int, float x) { S += fix42(exp_neg(x - m0)); });
    S = wg_sum(S, sh);
  }
  const float lse = bf16r(m0 + log_ge1(fix42_to_f32(S)));
  const float lpmax = bf16r(m0 - lse);

  if constexpr (kMode == kLogprobs) {
    uint16_t *out = a.lp + (long long)b * V;
    for_steps<kVec>(row, V, [&](int i0, const Raw8 &q, int n) {
      uint32_t h[8];
#pragma unroll
      for (int j = 0; j < 8; j++) h[j] = f2bf(val(q, j) - lse);
      if (kVec) {
        if (n == 8)
          *(uint4 *)(out + i0) = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                                            h[6] | (h[7] << 16));
      } else {
#pragma unroll
        for (int j = 0; j < 8; j++)
          if (j < n) out[i0 + j] = (uint16_t)h[j];
      }
    });
    return;
  }

  // the first index of the largest log-probability (lp is monotone in x: the indices with
  // lp == lpmax are the x whose difference rounds to it)
  auto first_max = [&]() {
    uint64_t best = (uint64_t)V;
    for_each<kVec>(row, V, [&](int i, float x) {
      if (bf16r(x - lse) == lpmax && (uint64_t)i < best) best = (uint64_t)i;
    });
    // workgroup minimum through the sum slots (min of non-negative values)
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint64_t n = __shfl_xor(best, o, 64);
      best = n < best ? n : best;
    }
    __syncthreads();
    if (l == 0) sh.q[t >> 6] = best;
    __syncthreads();
    uint64_t m = sh.q[0];
    for (int w = 1; w < kWaves; w++) m = sh.q[w] < m ? sh.q[w] : m;
    return m < (uint64_t)V ? (int)m : 0;  // (a row without a number: 0)
  };

  if constexpr (kMode == kGreedy) {
    const int i = first_max();
    if (t == 0) a.tok[b] = i;
    return;
  }

  if constexpr (kMode == kSample) {
    // bin k sits in slot hslot(k): a pad word after every 32 bins, so that the 32 bins of thread
    // t start at word 33 t and the lanes' element reads of them fall in distinct banks
    __shared__ uint32_t hist[kHistSlots];
    if (a.hist) {  // the row's histogram from split_hist_kernel (all loads issued before the stores)
      constexpr int kCopy = kKeys / 4 / kThreads;
      uint4 q[kCopy];
#pragma unroll
      for (int i = 0; i < kCopy; i++) q[i] = ((const uint4 *)a.sp->hist[b])[t + i * kThreads];
#pragma unroll
      for (int i = 0; i < kCopy; i++) {
        uint32_t *d = hist + hslot(4 * (t + i * kThreads));  // (4 j .. 4 j + 3 lie in one run of 32)
        d[0] = q[i].x, d[1] = q[i].y, d[2] = q[i].z, d[3] = q[i].w;
      }
    } else {
      for (int j = t; j < kHistSlots; j += kThreads) hist[j] = 0u;
      __syncthreads();
      for_each<kVec>(row, V, [&](int, float x) { atomicAdd(&hist[hslot(key_of(bf16r(x - lse)))], 1u); });
    }
    __syncthreads();

    // The row's values sit in a narrow range of keys (a few hundred bins for logits of any
    // spread), so the scans below give each thread a contiguous share of the range of non-empty
    // keys [kl, kh], in key order, rather than of all 32,768: the prefixes are the same (the
    // empty bins add nothing), and the exp and roundings of the bins run in all 16 waves rather
    // than in the one whose 32-bin stretches cover them.
    int kl = kKeys, kh = -1;
    {
      const uint32_t *own = hist + hslot(t * kBinsPerThread);  // (slots from 33 t: distinct banks)
      for (int j = 0; j < kBinsPerThread; j++)
        if (own[j]) kl = min(kl, t * kBinsPerThread + j), kh = max(kh, t * kBinsPerThread + j);
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        kl = min(kl, __shfl_xor(kl, o, 64));
        kh = max(kh, __shfl_xor(kh, o, 64));
      }
      __shared__ int shk[2][kWaves];
      if (l == 0) shk[0][t >> 6] = kl, shk[1][t >> 6] = kh;
      __syncthreads();
#pragma unroll
      for (int w = 0; w < kWaves; w++) kl = min(kl, shk[0][w]), kh = max(kh, shk[1][w]);
    }
    const int span = kh >= kl ? kh - kl + 1 : 0;
    const int per = (span + kThreads - 1) / kThreads;  // keys a thread scans (1 for most rows)
    const int kb = min(kl + t * per, kh + 1), ke = min(kb + per, kh + 1);  // the thread's keys [kb, ke)
    auto bin = [&](int key) { return hist[hslot(key)]; };
    auto mass_of = [&](int key) { return fix42(bf16r(exp_neg(value_of(key)))); };

    // top-p: the boundary bin key_p and the number j0 of its (lowest-index) members cut
    const bool topp = a.thr > 0.0f;
    if (t == 0) {
      sh.cut[0] = topp ? -1 : 0;  // key_p (no top-p: every bin survives, from key 0)
      sh.cut[1] = 0;              // j0
    }
    if (topp) {
      uint64_t mass = 0;
      for (int k = kb; k < ke; k++)
        if (const uint32_t c = bin(k)) mass += (uint64_t)c * mass_of(k);
      uint64_t cb = wg_excl<false>(mass, sh);  // (its barriers order the writes above)
      int kc = -1;                             // the thread's bin where the kept mass starts
      uint64_t cbc = 0;
      for (int k = kb; k < ke; k++) {
        const uint32_t c = bin(k);
        if (!c) continue;
        const uint64_t ce = cb + (uint64_t)c * mass_of(k);
        if (fix42_to_bf16(cb) <= a.thr && fix42_to_bf16(ce) > a.thr) kc = k, cbc = cb;
        cb = ce;
      }
      if (kc >= 0) {
        // the smallest j0 whose member (rank j0, cum cbc + (j0 + 1) Fc) survives
        const uint64_t Fc = mass_of(kc);
        uint32_t lo = 0, hi = bin(kc) - 1;
        while (lo < hi) {
          const uint32_t mid = (lo + hi) >> 1;
          if (fix42_to_bf16(cbc + (uint64_t)(mid + 1) * Fc) > a.thr) hi = mid;
          else lo = mid + 1;
        }
        sh.cut[0] = kc;
        sh.cut[1] = (int)lo;
      }
    }
    __syncthreads();
    const int key_p = sh.cut[0], j0 = sh.cut[1];
    if (key_p < 0) {  // nothing survives top-p: the greedy token
      const int i = first_max();
      if (t == 0) {
        a.tok[b] = i;
        if (a.ns > 0) a.sp->cut[b] = SplitCut{0, 0, 0, 0, 1, 0.0f, 0.0f};
      }
      return;
    }
    auto surv = [&](int key, uint32_t c) -> uint32_t {
      return key > key_p ? c : (key == key_p ? c - (uint32_t)j0 : 0u);
    };

    // the kept set: keys above key_t, and the members of key_t's group of rank [r_lo, r_hi)
    uint64_t nt = 0;
    for (int k = kb; k < ke; k++) nt += surv(k, bin(k));
    const uint64_t n_surv = wg_sum(nt, sh);
    if (t == 0) {
      sh.cut[2] = key_p;                    // key_t
      sh.cut[3] = j0;                       // r_lo
      sh.cut[4] = (int)hist[hslot(key_p)];  // r_hi
    }
    if (a.k > 0 && n_surv > (uint64_t)a.k) {
      uint64_t above = wg_excl<true>(nt, sh);  // survivors in the bins of the threads above
      for (int k = ke - 1; k >= kb; k--) {
        const uint32_t s = surv(k, bin(k));
        if (above < (uint64_t)a.k && (uint64_t)a.k <= above + s) {
          const int lo = (k == key_p) ? j0 : 0;
          sh.cut[2] = k;
          sh.cut[3] = lo;
          sh.cut[4] = lo + (a.k - (int)above);
        }
        above += s;
      }
    }
    __syncthreads();
    const int key_t = sh.cut[2], r_lo = sh.cut[3], r_hi = sh.cut[4];
    const bool partial = r_lo > 0 || r_hi < (int)hist[hslot(key_t)];
    const float m = bf16r(lpmax * a.inv_t);
    if (a.ns > 0) {  // the ranks, weights and the draw run over the row's slices
      if (t == 0) a.sp->cut[b] = SplitCut{key_t, r_lo, r_hi, (int)partial, 0, lse, m};
      return;
    }

    // ranks of key_t's members: the members in the waves below
    uint32_t tie_base = 0;
    if (partial) {
      uint64_t n = 0;
      for_each<kVec>(row, V, [&](int, float x) { n += key_of(bf16r(x - lse)) == key_t; });
      n = wave_sum(n);
      __syncthreads();
      if (l == 0) sh.q[t >> 6] = n;
      __syncthreads();
      for (int w = 0; w < (t >> 6); w++) tie_base += (uint32_t)sh.q[w];
    }

    // the weights of one step of the wave's range: W[j] of the lane's values; the rank of key_t's
    // members runs on from `carry` (the members in earlier waves and in the wave's earlier steps);
    // returns the step's members
    auto step_weights = [&](const Raw8 &q, int n, uint32_t carry, uint64_t W[8]) -> uint32_t {
      int key[8];
      uint32_t ties = 0;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        key[j] = j < n ? key_of(bf16r(val(q, j) - lse)) : -1;
        ties += key[j] == key_t;
      }
      const uint32_t tincl = partial ? wave_incl(ties) : 0u;
      uint32_t rank = carry + tincl - ties;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        bool kept = key[j] > key_t;
        if (key[j] == key_t) {
          kept = !partial || ((int)rank >= r_lo && (int)rank < r_hi);
          rank++;
        }
        W[j] = kept ? fix42(exp_neg(bf16r(bf16r(val(q, j) - lse) * a.inv_t) - m)) : 0ull;
      }
      return partial ? __shfl(tincl, 63, 64) : 0u;
    };

    // each step's total weight and starting rank, recorded for the draw below
    __shared__ uint64_t step_tot[kWaves][kMaxSteps];
    __shared__ uint32_t step_carry[kWaves][kMaxSteps];
    const int w = t >> 6;
    uint64_t tw = 0;
    uint32_t carry = tie_base;
    int js = 0;
    for_steps<kVec>(row, V, [&](int, const Raw8 &q, int n) {
      uint64_t W[8];
      const uint32_t c0 = carry;
      carry += step_weights(q, n, c0, W);
      uint64_t lt = 0;
#pragma unroll
      for (int j = 0; j < 8; j++) lt += W[j];
      const uint64_t st = wave_sum(lt);
      if (l == 0) {
        step_tot[w][js] = st;
        step_carry[w][js] = c0;
      }
      tw += st;
      js++;
    });
    __syncthreads();
    if (l == 0) sh.q[w] = tw;
    __syncthreads();
    uint64_t base = 0, total = 0;
    for (int v = 0; v < kWaves; v++) {
      if (v < w) base += sh.q[v];
      total += sh.q[v];
    }
    float u = a.u[b];
    u = fminf(fmaxf(u, 0.0f), 0x1.fffffep-1f);  // (NaN -> 0)
    const uint64_t U = mul_u32_u64_hi((uint64_t)(u * 4294967296.0f), total);

    // the number of i with C_i <= U, wave by wave: a wave whose values all lie at or below U
    // counts its range, one above U none; in the one wave that holds U, the steps before the
    // step that holds it count whole, and that step is reloaded and walked
    const Range r = wave_range(V);
    uint64_t cnt = 0;
    if (base + tw <= U) {
      cnt = l == 0 ? (uint64_t)(r.hi - r.lo) : 0ull;
    } else if (base <= U) {
      uint64_t run = base;
      int j = 0;
      while (run + step_tot[w][j] <= U) run += step_tot[w][j++];
      const int i0 = r.lo + j * kStep + 8 * l;
      const Raw8 q = load8<kVec>(row, i0, r.hi);
      const int n = max(0, min(8, r.hi - i0));
      uint64_t W[8];
      step_weights(q, n, step_carry[w][j], W);
      uint64_t lt = 0;
#pragma unroll
      for (int jj = 0; jj < 8; jj++) lt += W[jj];
      uint64_t c = run + wave_incl(lt) - lt;  // C of the lane's first value
#pragma unroll
      for (int jj = 0; jj < 8; jj++) {
        if (jj < n && c <= U) cnt++;
        c += W[jj];
      }
      if (l == 0) cnt += (uint64_t)j * kStep;
    }
    const uint64_t count = wg_sum(cnt, sh);
    if (t == 0) a.tok[b] = (int32_t)(count - 1);
  }
}

// ---- log-probabilities and the greedy draw of a few rows, each row split over workgroups ----
// One workgroup walks a whole row in the kernel above, so a batch of a few rows leaves most CUs
// idle (a 248,320-entry row: ~80 us on one CU).  For up to kSplitRows rows each row is cut into
// slices of whole 8-value steps, one workgroup each, and the row's reductions become launches:
//   slice maxima -> the row max m0 and the slices' exact integer sums S -> lse, lpmax, and the
//   slices' log-probabilities or first indices of lpmax -> (greedy) the smallest of those.
// The partials pass between launches through plain stores to a static buffer and are combined in
// slice order; max, the integer sum and min do not depend on the order, so every result has the
// bits of the one-workgroup kernel.  Calls that overlap on one device share the buffer and race.
struct SplitArgs {
  const uint16_t *logits;
  int V, ns, len;  // slices per row, values per slice (a multiple of 8)
  int32_t *tok;
  uint16_t *lp;
  int hist;  // draws with a cut: split_sum_kernel clears the row's histogram, split_hist_kernel fills it
  int hg;    // slices a split_hist_kernel workgroup counts
  SplitScratch *sp;
};

template <bool kVec, typename F>
__device__ __forceinline__ void slice_steps(const uint16_t *row, int lo, int hi, F &&f) {
  for (int i0 = lo + 8 * (int)threadIdx.x; i0 < hi; i0 += 8 * kSplitThreads)
    f(i0, load8<kVec>(row, i0, hi), min(8, hi - i0));
}

template <bool kVec, typename F>
__device__ __forceinline__ void slice_each(const uint16_t *row, int lo, int hi, F &&f) {
  slice_steps<kVec>(row, lo, hi, [&](int i0, const Raw8 &q, int n) {
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (j < n) f(i0 + j, val(q, j));
  });
}

__device__ __forceinline__ float split_max(float v, float *sh) {
  v = wave_max(v);
  __syncthreads();
  if (lane_id() == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = sh[0];
#pragma unroll
  for (int w = 1; w < kSplitWaves; w++) m = fmaxf(m, sh[w]);
  return m;
}

__device__ __forceinline__ unsigned long long split_sum(unsigned long long v, unsigned long long *sh) {
  v = wave_sum(v);
  __syncthreads();
  if (lane_id() == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  unsigned long long t = 0;
#pragma unroll
  for (int w = 0; w < kSplitWaves; w++) t += sh[w];
  return t;
}

__device__ __forceinline__ int split_min(int v, int *sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if (lane_id() == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  int m = sh[0];
#pragma unroll
  for (int w = 1; w < kSplitWaves; w++) m = min(m, sh[w]);
  return m;
}

// the row max from the slice maxima (thread t < ns reads slice t's)
__device__ __forceinline__ float split_row_max(const SplitScratch *sp, int b, int ns, float *sh) {
  return split_max((int)threadIdx.x < ns ? sp->max[b][threadIdx.x] : -INFINITY, sh);
}

template <bool kVec>
__global__ __launch_bounds__(kSplitThreads) void split_max_kernel(const SplitArgs a) {
  __shared__ float sh[kSplitWaves];
  const int s = blockIdx.x, b = blockIdx.y;
  const uint16_t *row = a.logits + (long long)b * a.V;
  const int lo = s * a.len, hi = min(a.V, lo + a.len);
  float m = -INFINITY;
  slice_each<kVec>(row, lo, hi, [&](int, float x) { m = fmaxf(m, x); });
  m = split_max(m, sh);
  if (threadIdx.x == 0) a.sp->max[b][s] = m;
}

template <bool kVec>
__global__ __launch_bounds__(kSplitThreads) void split_sum_kernel(const SplitArgs a) {
  __shared__ float shf[kSplitWaves];
  __shared__ unsigned long long shq[kSplitWaves];
  const int s = blockIdx.x, b = blockIdx.y;
  const uint16_t *row = a.logits + (long long)b * a.V;
  const int lo = s * a.len, hi = min(a.V, lo + a.len);
  const float m0 = split_row_max(a.sp, b, a.ns, shf);
  uint64_t S = 0;
  slice_each<kVec>(row, lo, hi, [&](int, float x) { S += fix42(exp_neg(x - m0)); });
  S = split_sum(S, shq);
  if (threadIdx.x == 0) a.sp->sum[b][s] = S;
  if (a.hist) {  // the row's slices clear its histogram for split_hist_kernel
    uint4 *h = (uint4 *)a.sp->hist[b];
    for (int i = s * kSplitThreads + threadIdx.x; i < kKeys / 4; i += a.ns * kSplitThreads)
      h[i] = make_uint4(0u, 0u, 0u, 0u);
  }
}

// The row's histogram of lp keys (sample_rows_kernel's, which then only copies it): each workgroup
// counts the values of hg consecutive slices in LDS and adds its non-empty bins to the row's.  The adds are system-scope
// atomics (performed past the XCDs' L2s, so slices on different XCDs add to one copy); integer
// adds, so the counts do not depend on their order.
template <bool kVec>
__global__ __launch_bounds__(kSplitThreads) void split_hist_kernel(const SplitArgs a) {
  __shared__ __align__(16) uint32_t hist[kKeys];
  __shared__ float shf[kSplitWaves];
  __shared__ unsigned long long shq[kSplitWaves];
  const int s = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const uint16_t *row = a.logits + (long long)b * a.V;
  const int lo = s * a.hg * a.len, hi = min(a.V, lo + a.hg * a.len);
  for (int i = t; i < kKeys / 4; i += kSplitThreads) ((uint4 *)hist)[i] = make_uint4(0u, 0u, 0u, 0u);
  const float m0 = split_row_max(a.sp, b, a.ns, shf);
  const uint64_t S = split_sum(t < a.ns ? a.sp->sum[b][t] : 0ull, shq);
  const float lse = bf16r(m0 + log_ge1(fix42_to_f32(S)));
  __syncthreads();
  slice_each<kVec>(row, lo, hi, [&](int, float x) { atomicAdd(&hist[key_of(bf16r(x - lse))], 1u); });
  __syncthreads();
  for (int k = t; k < kKeys; k += kSplitThreads) {
    const uint32_t c = hist[k];
    if (c) __hip_atomic_fetch_add(&a.sp->hist[b][k], c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

template <int kMode, bool kVec>
__global__ __launch_bounds__(kSplitThreads) void split_final_kernel(const SplitArgs a) {
  __shared__ float shf[kSplitWaves];
  __shared__ unsigned long long shq[kSplitWaves];
  __shared__ int shi[kSplitWaves];
  const int s = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const uint16_t *row = a.logits + (long long)b * a.V;
  const int lo = s * a.len, hi = min(a.V, lo + a.len);
  const float m0 = split_row_max(a.sp, b, a.ns, shf);
  const uint64_t S = split_sum(t < a.ns ? a.sp->sum[b][t] : 0ull, shq);
  const float lse = bf16r(m0 + log_ge1(fix42_to_f32(S)));
  if constexpr (kMode == kLogprobs) {
    uint16_t *out = a.lp + (long long)b * a.V;
    slice_steps<kVec>(row, lo, hi, [&](int i0, const Raw8 &q, int n) {
      uint32_t h[8];
#pragma unroll
      for (int j = 0; j < 8; j++) h[j] = f2bf(val(q, j) - lse);
      if (kVec) {
        if (n == 8)
          *(uint4 *)(out + i0) = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                                            h[6] | (h[7] << 16));
      } else {
#pragma unroll
        for (int j = 0; j < 8; j++)
          if (j < n) out[i0 + j] = (uint16_t)h[j];
      }
    });
  } else {
    const float lpmax = bf16r(m0 - lse);
    int best = a.V;
    slice_each<kVec>(row, lo, hi, [&](int i, float x) {
      if (bf16r(x - lse) == lpmax && i < best) best = i;
    });
    best = split_min(best, shi);
    if (t == 0) a.sp->idx[b][s] = best;
  }
}

__global__ __launch_bounds__(64) void split_argmin_kernel(const SplitScratch *sp, int ns, int V,
                                                                    int32_t *__restrict__ tok) {
  const int b = blockIdx.x;
  int m = (int)threadIdx.x < ns ? sp->idx[b][threadIdx.x] : V;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = min(m, __shfl_xor(m, o, 64));
  if (threadIdx.x == 0) tok[b] = m < V ? m : 0;  // (a row without a number: 0)
}

// ---- a draw's weights and walk over the slices (after sample_rows_kernel has set the cut) ----
struct DrawArgs {
  const uint16_t *logits;
  int V, ns, len;
  float inv_t;
  const float *u;
  int32_t *tok;
  int nocut;  // no top-p and no top-k: every value is kept, and no histogram or cut ran
  SplitScratch *sp;
};

// The row's cut: sample_rows_kernel's, or without top-p and top-k the one that keeps every value
// (key_t 0, no partial tie group) with lse and m from the slice partials.
__device__ __forceinline__ SplitCut split_cut(const DrawArgs &a, int b, float *shf, unsigned long long *shq) {
  if (!a.nocut) return a.sp->cut[b];
  const int t = threadIdx.x;
  const float m0 = split_max(t < a.ns ? a.sp->max[b][t] : -INFINITY, shf);
  const uint64_t S = split_sum(t < a.ns ? a.sp->sum[b][t] : 0ull, shq);
  const float lse = bf16r(m0 + log_ge1(fix42_to_f32(S)));
  return SplitCut{0, 0, 0, 0, 0, lse, bf16r(bf16r(m0 - lse) * a.inv_t)};
}

// exclusive prefix over the workgroup's threads in thread order, and the workgroup's total
template <typename T>
__device__ __forceinline__ T split_excl(T v, T *sh, T &total) {
  const T inc = wave_incl(v);
  __syncthreads();
  if (lane_id() == 63) sh[threadIdx.x >> 6] = inc;
  __syncthreads();
  T base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kSplitWaves; w++) {
    if (w < (int)(threadIdx.x >> 6)) base += sh[w];
    tot += sh[w];
  }
  total = tot;
  return base + inc - v;
}

// the members of key_t in slice s (partial cuts only)
template <bool kVec>
__global__ __launch_bounds__(kSplitThreads) void split_ties_kernel(const DrawArgs a) {
  __shared__ unsigned long long sh[kSplitWaves];
  const int s = blockIdx.x, b = blockIdx.y;
  const SplitCut c = a.sp->cut[b];
  if (c.done || !c.partial) return;
  const uint16_t *row = a.logits + (long long)b * a.V;
  const int lo = s * a.len, hi = min(a.V, lo + a.len);
  unsigned long long n = 0;
  slice_each<kVec>(row, lo, hi, [&](int, float x) { n += key_of(bf16r(x - c.lse)) == c.key_t; });
  n = split_sum(n, sh);
  if (threadIdx.x == 0) a.sp->idx[b][s] = (int)n;
}

// The weights of one 2048-value step of a slice from i0s (thread t: the 8 values from i0s + 8 t),
// the ranks of key_t's members running on from `rank0` in vocabulary order; returns the step's
// members.  W and the kept rule are sample_rows_kernel's.
template <bool kVec>
__device__ __forceinline__ uint32_t split_step_weights(const uint16_t *row, int i0s, int hi, const SplitCut &c,
                                                       float inv_t, uint32_t rank0, uint32_t *shu, uint64_t W[8],
                                                       int &n) {
  const int i0 = i0s + 8 * (int)threadIdx.x;
  const Raw8 q = load8<kVec>(row, i0, hi);
  n = max(0, min(8, hi - i0));
  int key[8];
  uint32_t ties = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    key[j] = j < n ? key_of(bf16r(val(q, j) - c.lse)) : -1;
    ties += key[j] == c.key_t;
  }
  uint32_t total = 0;
  uint32_t rank = c.partial ? rank0 + split_excl(ties, shu, total) : 0u;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    bool kept = key[j] > c.key_t;
    if (key[j] == c.key_t) {
      kept = !c.partial || ((int)rank >= c.r_lo && (int)rank < c.r_hi);
      rank++;
    }
    W[j] = kept ? fix42(exp_neg(bf16r(bf16r(val(q, j) - c.lse) * inv_t) - c.m)) : 0ull;
  }
  return total;
}

// the members of key_t in the slices before s (partial cuts only)
__device__ __forceinline__ uint32_t split_tie_base(const SplitScratch *sp, int b, int s, const SplitCut &c,
                                                   unsigned long long *sh) {
  if (!c.partial) return 0u;
  const int t = threadIdx.x;
  return (uint32_t)split_sum(t < s ? (unsigned long long)sp->idx[b][t] : 0ull, sh);
}

// the slice's total weight
template <bool kVec>
__global__ __launch_bounds__(kSplitThreads) void split_weights_kernel(const DrawArgs a) {
  __shared__ float shf[kSplitWaves];
  __shared__ unsigned long long shq[kSplitWaves];
  __shared__ uint32_t shu[kSplitWaves];
  const int s = blockIdx.x, b = blockIdx.y;
  const SplitCut c = split_cut(a, b, shf, shq);
  if (c.done) return;
  const uint16_t *row = a.logits + (long long)b * a.V;
  const int lo = s * a.len, hi = min(a.V, lo + a.len);
  uint32_t rank = split_tie_base(a.sp, b, s, c, shq);
  unsigned long long tw = 0;
  for (int i0s = lo; i0s < hi; i0s += 8 * kSplitThreads) {
    uint64_t W[8];
    int n;
    rank += split_step_weights<kVec>(row, i0s, hi, c, a.inv_t, rank, shu, W, n);
#pragma unroll
    for (int j = 0; j < 8; j++) tw += W[j];
  }
  tw = split_sum(tw, shq);
  if (threadIdx.x == 0) a.sp->wsum[b][s] = tw;
}

// The draw: U = floor(u * total weight); the token is the number of i with C_i = sum_{j<i} W_j
// <= U, less one.  The slices before the first slice whose prefix passes U count whole, the
// slices after it none, and that slice is walked.
template <bool kVec>
__global__ __launch_bounds__(kSplitThreads) void split_draw_kernel(const DrawArgs a) {
  __shared__ float shf[kSplitWaves];
  __shared__ unsigned long long shq[kSplitWaves];
  __shared__ uint32_t shu[kSplitWaves];
  __shared__ unsigned long long pick[2];
  const int b = blockIdx.x, t = threadIdx.x;
  const SplitCut c = split_cut(a, b, shf, shq);
  if (c.done) return;
  const unsigned long long T = t < a.ns ? a.sp->wsum[b][t] : 0ull;
  unsigned long long total;
  const unsigned long long P = split_excl(T, shq, total);
  float u = a.u[b];
  u = fminf(fmaxf(u, 0.0f), 0x1.fffffep-1f);  // (NaN -> 0)
  const uint64_t U = mul_u32_u64_hi((uint64_t)(u * 4294967296.0f), total);
  if (t == 0) pick[0] = (unsigned long long)a.ns;
  __syncthreads();
  // the first slice whose prefix with it passes U (the prefixes grow with the slice)
  if (t < a.ns && P <= U && U < P + T) pick[0] = t, pick[1] = P;
  __syncthreads();
  const int s = (int)pick[0];
  if (s >= a.ns) {  // (a total of 0: every C_i is 0)
    if (t == 0) a.tok[b] = a.V - 1;
    return;
  }
  const uint16_t *row = a.logits + (long long)b * a.V;
  const int lo = s * a.len, hi = min(a.V, lo + a.len);
  uint32_t rank = split_tie_base(a.sp, b, s, c, shq);
  unsigned long long run = pick[1], cnt = 0;
  for (int i0s = lo; i0s < hi; i0s += 8 * kSplitThreads) {
    uint64_t W[8];
    int n;
    rank += split_step_weights<kVec>(row, i0s, hi, c, a.inv_t, rank, shu, W, n);
    unsigned long long lt = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) lt += W[j];
    unsigned long long st;
    unsigned long long cc = run + split_excl(lt, shq, st);  // C of the thread's first value
#pragma unroll
    for (int j = 0; j < 8; j++) {
      if (j < n && cc <= U) cnt++;
      cc += W[j];
    }
    run += st;
  }
  cnt = split_sum(cnt, shq);
  if (t == 0) a.tok[b] = (int32_t)((unsigned long long)lo + cnt - 1);
}

// The split launches of B <= kSplitRows rows: log-probabilities (kLogprobs), the greedy draw
// (kGreedy), or only the slice maxima and sums that sample_rows_kernel then combines (kSample).
template <int kMode, bool kVec>
int launch_split_vec(const SplitArgs &a, int B, hipStream_t st) {
  const dim3 grid(a.ns, B);
  split_max_kernel<kVec><<<grid, kSplitThreads, 0, st>>>(a);
  split_sum_kernel<kVec><<<grid, kSplitThreads, 0, st>>>(a);
  if constexpr (kMode == kSample)
    if (a.hist) split_hist_kernel<kVec><<<dim3((a.ns + a.hg - 1) / a.hg, B), kSplitThreads, 0, st>>>(a);
  if constexpr (kMode != kSample) split_final_kernel<kMode, kVec><<<grid, kSplitThreads, 0, st>>>(a);
  if constexpr (kMode == kGreedy) split_argmin_kernel<<<B, 64, 0, st>>>(a.sp, a.ns, a.V, a.tok);
  return jit::check_launch(kMode == kGreedy ? "jit_argmax_rows" : kMode == kLogprobs ? "jit_logprobs_rows"
                                                                                       : "jit_sample_rows");
}

// The slices of a row: about 1024 workgroups in all, at most kSplitMax a row, at least kSplitMin
// values each, whole 8-value steps.
SplitArgs split_args(const uint16_t *logits, int B, int V, int32_t *tok, uint16_t *lp, SplitScratch *sp) {
  int ns = min(kSplitMax, max(1, 1024 / B));
  ns = min(ns, (V + kSplitMin - 1) / kSplitMin);
  const int len = ((V + ns - 1) / ns + 7) / 8 * 8;
  ns = (V + len - 1) / len;
  return SplitArgs{logits, V, ns, len, tok, lp, 0, 0, sp};
}

template <int kMode>
int launch_split(const SplitArgs &a, int B, void *stream) {
  if ((a.V & 7) == 0 && ((uintptr_t)a.logits & 15) == 0)
    return launch_split_vec<kMode, true>(a, B, (hipStream_t)stream);
  return launch_split_vec<kMode, false>(a, B, (hipStream_t)stream);
}

int check_rows(const char *what, const void *logits, int B, int V, const void *out) {
  if (B < 0 || V <= 0) return jit::fail(JIT_EINVAL, "%s: bad dims B=%d V=%d", what, B, V);
  if (V > kMaxV) return jit::fail(JIT_EUNSUPPORTED, "%s covers V <= %d, got %d", what, kMaxV, V);
  if (B > 0 && (!logits || !out)) return jit::fail(JIT_EINVAL, "%s: null pointer", what);
  return JIT_OK;
}

template <int kMode>
int launch(const SampleArgs &a, int B, void *stream) {
  if ((a.V & 7) == 0 && ((uintptr_t)a.logits & 15) == 0)
    sample_rows_kernel<kMode, true><<<B, kThreads, 0, (hipStream_t)stream>>>(a);
  else
    sample_rows_kernel<kMode, false><<<B, kThreads, 0, (hipStream_t)stream>>>(a);
  return jit::check_launch("jit_sample_rows");
}

// bf16 round trip of a float on the host (round to nearest even)
float host_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return f;
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

// The current device's address of g_split (looked up on the first call on that device).
constexpr int kMaxDevices = 64;
std::mutex g_split_mu;
SplitScratch *g_split_dev[kMaxDevices];

int split_scratch_of_current_device(SplitScratch **sp, const char *what) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return jit::fail(JIT_ELAUNCH, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return jit::fail(JIT_EUNSUPPORTED, "%s: device %d is past the %d devices the scratch table covers", what, dev,
                     kMaxDevices);
  std::lock_guard<std::mutex> lock(g_split_mu);
  if (!g_split_dev[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_split));
    if (e != hipSuccess || !p)
      return jit::fail(JIT_ELAUNCH, "%s: hipGetSymbolAddress(g_split) failed on device %d: %s", what, dev,
                       hipGetErrorString(e));
    g_split_dev[dev] = (SplitScratch *)p;
  }
  *sp = g_split_dev[dev];
  return JIT_OK;
}

}  // namespace

static int logprobs_rows(const uint16_t *logits, int B, int V, uint16_t *lp, SplitScratch *sp, void *stream) {
  if (B <= kSplitRows) return launch_split<kLogprobs>(split_args(logits, B, V, nullptr, lp, sp), B, stream);
  SampleArgs a{logits, V, 0.0f, 0.0f, 0, nullptr, nullptr, lp};
  return launch<kLogprobs>(a, B, stream);
}

static int argmax_rows(const uint16_t *logits, int B, int V, int32_t *out, SplitScratch *sp, void *stream) {
  if (B <= kSplitRows) return launch_split<kGreedy>(split_args(logits, B, V, out, nullptr, sp), B, stream);
  SampleArgs a{logits, V, 0.0f, 0.0f, 0, nullptr, out, nullptr};
  return launch<kGreedy>(a, B, stream);
}

static int sample_rows(const uint16_t *logits, int B, int V, double temperature, double top_p, int top_k,
                       const float *u, int32_t *tokens, SplitScratch *sp, void *stream) {
  if (temperature <= 0.0) {
    if (B <= kSplitRows) return launch_split<kGreedy>(split_args(logits, B, V, tokens, nullptr, sp), B, stream);
    SampleArgs a{logits, V, 0.0f, 0.0f, 0, nullptr, tokens, nullptr};
    return launch<kGreedy>(a, B, stream);
  }
  if (!u) return jit::fail(JIT_EINVAL, "sample_rows: null uniforms");
  // the settings as the reference's scalars reach its bf16 arrays: a Python float, then fp32,
  // then bf16 (Q36/sampler.py:381, 462, 470)
  const float inv_t = host_bf16((float)(1.0 / temperature));
  const float thr = (top_p > 0.0 && top_p < 1.0) ? host_bf16((float)(1.0 - top_p)) : 0.0f;
  if (!(inv_t > 0.0f) || !(inv_t < INFINITY))
    return jit::fail(JIT_EUNSUPPORTED, "sample_rows: 1 / T = %g is not a finite positive bf16", 1.0 / temperature);
  const int k = top_k >= V ? 0 : top_k;
  SampleArgs a{logits, V, inv_t, thr, k, u, tokens, nullptr, 0, 0, sp};
  if (B > kSplitRows) return launch<kSample>(a, B, stream);
  // the row's log-sum-exp over slices, the histogram and the cut in one workgroup a row, then the
  // ranks, weights and the draw over slices again
  // (without top-p and top-k every value is kept: no histogram, no cut)
  const int nocut = thr == 0.0f && k == 0;
  SplitArgs sa = split_args(logits, B, V, nullptr, nullptr, sp);
  // the histogram over runs of slices, about 256 workgroups in all (each clears and scans 128 KB
  // of LDS, so more of them with fewer values each cost more than they save)
  sa.hist = !nocut;
  sa.hg = max(1, (sa.ns * B + 255) / 256);
  if (int rc = launch_split<kSample>(sa, B, stream)) return rc;
  a.ns = sa.ns;
  a.hist = sa.hist;
  if (!nocut)
    if (int rc = launch<kSample>(a, B, stream)) return rc;
  const DrawArgs da{logits, V, sa.ns, sa.len, inv_t, u, tokens, nocut, sp};
  const dim3 grid(sa.ns, B);
  const hipStream_t st = (hipStream_t)stream;
  if ((V & 7) == 0 && ((uintptr_t)logits & 15) == 0) {
    if (!nocut) split_ties_kernel<true><<<grid, kSplitThreads, 0, st>>>(da);
    split_weights_kernel<true><<<grid, kSplitThreads, 0, st>>>(da);
    split_draw_kernel<true><<<B, kSplitThreads, 0, st>>>(da);
  } else {
    if (!nocut) split_ties_kernel<false><<<grid, kSplitThreads, 0, st>>>(da);
    split_weights_kernel<false><<<grid, kSplitThreads, 0, st>>>(da);
    split_draw_kernel<false><<<B, kSplitThreads, 0, st>>>(da);
  }
  return jit::check_launch("jit_sample_rows");
}

// The split launches' partials: the library's own array (the entry points without a workspace) or a
// caller's workspace of jit_sampler_workspace_bytes() bytes.
static int scratch_arg(void *workspace, long long bytes, const char *what, SplitScratch **sp) {
  if (workspace) {
    if (bytes < (long long)sizeof(SplitScratch) || ((uintptr_t)workspace & 15))
      return jit::fail(JIT_EINVAL, "%s: workspace of %lld bytes at %p; %lld bytes, 16-byte aligned, needed", what,
                       bytes, workspace, (long long)sizeof(SplitScratch));
    *sp = (SplitScratch *)workspace;
    return JIT_OK;
  }
  return split_scratch_of_current_device(sp, what);
}

extern "C" long long jit_sampler_workspace_bytes(void) { return (long long)sizeof(SplitScratch); }

extern "C" int jit_logprobs_rows_ws(const uint16_t *logits, int B, int V, uint16_t *lp, void *workspace,
                                    long long workspace_bytes, void *stream) {
  if (int rc = check_rows("logprobs_rows", logits, B, V, lp)) return rc;
  if (B == 0) return JIT_OK;
  SplitScratch *sp = nullptr;
  if (int rc = scratch_arg(workspace, workspace_bytes, "logprobs_rows", &sp)) return rc;
  return logprobs_rows(logits, B, V, lp, sp, stream);
}

extern "C" int jit_logprobs_rows(const uint16_t *logits, int B, int V, uint16_t *lp, void *stream) {
  return jit_logprobs_rows_ws(logits, B, V, lp, nullptr, 0, stream);
}

extern "C" int jit_argmax_rows_ws(const uint16_t *logits, int B, int V, int32_t *out, void *workspace,
                                  long long workspace_bytes, void *stream) {
  if (int rc = check_rows("argmax_rows", logits, B, V, out)) return rc;
  if (B == 0) return JIT_OK;
  SplitScratch *sp = nullptr;
  if (int rc = scratch_arg(workspace, workspace_bytes, "argmax_rows", &sp)) return rc;
  return argmax_rows(logits, B, V, out, sp, stream);
}

extern "C" int jit_argmax_rows(const uint16_t *logits, int B, int V, int32_t *out, void *stream) {
  return jit_argmax_rows_ws(logits, B, V, out, nullptr, 0, stream);
}

extern "C" int jit_sample_rows_ws(const uint16_t *logits, int B, int V, double temperature, double top_p, int top_k,
                                  const float *u, int32_t *tokens, void *workspace, long long workspace_bytes,
                                  void *stream) {
  if (int rc = check_rows("sample_rows", logits, B, V, tokens)) return rc;
  if (!(temperature == temperature) || !(top_p == top_p) || top_k < 0)
    return jit::fail(JIT_EINVAL, "sample_rows: bad settings T=%g top_p=%g top_k=%d", temperature, top_p, top_k);
  if (B == 0) return JIT_OK;
  if (temperature > 0.0) {  // (the draw's own contract, before the workspace is looked up)
    if (!u) return jit::fail(JIT_EINVAL, "sample_rows: null uniforms");
    const float inv_t = host_bf16((float)(1.0 / temperature));
    if (!(inv_t > 0.0f) || !(inv_t < INFINITY))
      return jit::fail(JIT_EUNSUPPORTED, "sample_rows: 1 / T = %g is not a finite positive bf16", 1.0 / temperature);
  }
  SplitScratch *sp = nullptr;
  if (int rc = scratch_arg(workspace, workspace_bytes, "sample_rows", &sp)) return rc;
  return sample_rows(logits, B, V, temperature, top_p, top_k, u, tokens, sp, stream);
}

extern "C" int jit_sample_rows(const uint16_t *logits, int B, int V, double temperature, double top_p, int top_k,
                               const float *u, int32_t *tokens, void *stream) {
  return jit_sample_rows_ws(logits, B, V, temperature, top_p, top_k, u, tokens, nullptr, 0, stream);
}

extern "C" int jit_threefry_uniform(const uint32_t *keys, int B, float *u, void *stream) {
  if (B < 0) return jit::fail(JIT_EINVAL, "threefry_uniform: B=%d", B);
  if (B == 0) return JIT_OK;
  if (!keys || !u) return jit::fail(JIT_EINVAL, "threefry_uniform: null pointer");
  threefry_uniform_kernel<<<(B + 255) / 256, 256, 0, (hipStream_t)stream>>>(keys, B, u);
  return jit::check_launch("jit_threefry_uniform");
}
