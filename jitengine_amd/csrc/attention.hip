// Paged KV pool append and split-K paged GQA decode attention for gfx950.
//
// Pool page (one layer): [Hkv][2][16 * 128] bf16 -- per kv head its K part, then
// its V part, so what one wave reads of a page (its kv head) is 8 KiB contiguous.
// The K part is chunk-major -- [4 d-chunks][16 slots][32 dims], so the 16 slots x
// 32 dims one MFMA A fragment covers are 1 KB contiguous -- and the V part is
// dim-major -- [128 dims][16 slots], so a fragment's 16 dims x 4 slots per lane
// group are 512 B contiguous.
//
// Attention work item: one workgroup per chunk (1536 keys; longer for sequences past
// 196,608 keys) of one sequence and 2 kv heads, 4 waves per kv head, each wave streaming
// a quarter of the chunk (384 keys) two 16-key
// pages (32 keys) per step; the 4 waves' states meet in LDS:
//   S^T[16 keys x 16 q heads] = K_page . Q^T      (4 MFMA 16x16x32 per page)
//   online softmax in the exp2 domain (fp32 running max / sum per q head)
//   O^T[128 d x 16 q heads] += V^T . P^T           (16 MFMA 16x16x32, all 32 keys: P as a
//                                                   bf16 high part plus a bf16 residual)
// Every lane owns one q head (lane % 16) in the scores, the softmax state and the
// output tile alike, so the rescale needs no lane exchange; the cross-lane max and
// sum use the gfx950 permlane swaps.  Each K/V byte is read once for all
// G = H / Hkv query heads of its kv head (G <= 16; tile columns G..15 are
// padding).  A step's K registers are refilled for the next step as soon as its
// scores are formed and its V registers as soon as P.V is issued, so the next
// step's loads are in flight during the softmax and the MFMAs; the chunk's page
// ids are fetched once up front.  A sequence of one chunk writes its output
// directly, longer ones write fp32 (max, sum, o[128]) partials that
// attn_merge_kernel combines in chunk order.
#include "common.hpp"

#include <mutex>

namespace {

constexpr int kD = JIT_HEAD_DIM;      // 128
constexpr int kPage = JIT_PAGE_TOKENS;  // 16
constexpr int kPageHead = kPage * kD;   // bf16 elements of one (page, kv head, part)
#ifndef JIT_ATTN_CHUNK
#define JIT_ATTN_CHUNK 1536
#endif
// keys per work item: fewer, longer chunks write fewer partials for the merge, and the
// waves that split a chunk keep the parallelism of short ones (config 2 on MI355X:
// kernel + merge 73.4 us with 384-key chunks of one wave per kv head, 68.3 us here)
constexpr int kChunk = JIT_ATTN_CHUNK;
#ifndef JIT_ATTN_SPLITS
#define JIT_ATTN_SPLITS 4
#endif
constexpr int kAttnSplits = JIT_ATTN_SPLITS;  // waves per kv head and chunk
#ifndef JIT_ATTN_HB
#define JIT_ATTN_HB (8 / JIT_ATTN_SPLITS)
#endif
constexpr int kAttnHeadsPerBlock = JIT_ATTN_HB;  // kv heads per workgroup
// A sequence longer than kLongChunks chunks of kChunk keys is cut into about kLongChunks
// chunks instead (two workgroups each: one per CU of MI355X's 256), so that a lone long
// sequence still fills the chip in one even wave of workgroups (262,144 keys: 128 chunks of
// 2048, 100 us a layer against 116 us for 171 chunks of 1536).  A wave's run stays at most
// 64 pages (one page id per lane), hence the cap.
#ifndef JIT_ATTN_LONG_CHUNKS
#define JIT_ATTN_LONG_CHUNKS 128
#endif
constexpr int kLongChunks = JIT_ATTN_LONG_CHUNKS;
constexpr int kChunkMax = 64 * kPage * kAttnSplits;
static_assert(kChunk % (32 * kAttnSplits) == 0 && kChunk <= kChunkMax, "a wave's run is whole 32-key steps");

__host__ __device__ __forceinline__ int chunk_tokens(int len) {
  if (len <= kChunk * kLongChunks) return kChunk;
  constexpr int kStep = 32 * kAttnSplits;
  const int c = ((len + kLongChunks - 1) / kLongChunks + kStep - 1) / kStep * kStep;
  return c < kChunkMax ? c : kChunkMax;
}

__device__ __forceinline__ int k_off(int slot, int d) { return k_page_offset(slot, d); }

}  // namespace

// Chunk length rule: a pure function of the sequence's own length (so results do
// not depend on the batch).
extern "C" int jit_attn_chunk_tokens(int len) { return chunk_tokens(len); }

namespace {

// ---------------------------------------------------------------- append
__global__ void kv_append_kernel(const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
                                 int Hkv, const int32_t *__restrict__ pos,
                                 const int32_t *__restrict__ page_table, int max_pages,
                                 uint16_t *__restrict__ pool) {
  const int b = blockIdx.x;
  const int p = pos[b];
  const int page = page_table[(long long)b * max_pages + p / kPage];
  const int slot = p % kPage;
  for (int t = threadIdx.x; t < Hkv * kD; t += blockDim.x) {
    const int h = t / kD, d = t % kD;
    const long long src = ((long long)b * Hkv + h) * kD + d;
    uint16_t *hp = pool + ((long long)page * Hkv + h) * 2 * kPageHead;
    hp[k_off(slot, d)] = k[src];
    hp[kPageHead + d * kPage + slot] = v[src];
  }
}

struct AttnArgs {
  const uint16_t *q;
  const uint16_t *pool;
  const int32_t *page_table;
  const int32_t *lens;
  const int32_t *chunk_start;
  const int32_t *chunk_seq;
  float *part_o;   // [total_chunks][H][128]
  float *part_ml;  // [total_chunks][H][2]
  uint16_t *out;
  int max_pages, H, Hkv, G;
  float qk_scale;  // scale * log2(e)
  int hb;          // kv heads per workgroup (a kernel argument: blockDim.x lives in the implicit
                   // arguments, whose 16-bit fields the kernel would fetch with a vector load and
                   // wait for before anything else)
  // jit_paged_decode_attn_qkv: the step's raw q/k/v rows [B, (H + 2 Hkv) * 128] instead of q, the
  // q and k norm weights, RoPE's inverse frequencies and the norm's eps (null qkv: q as given)
  const uint16_t *qkv;
  const uint16_t *qn_w, *kn_w;
  const float *inv_freq;
  float eps;
};

// xor-16 / xor-32 lane exchanges, one VALU op each (gfx950 permlane swaps): with both
// operands the same value, the two results are the even and the odd row (of each
// row pair, resp. half) -- so any symmetric combination of them is the reduction.
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The K part of kv head kvh in page pg (its V part follows).
__device__ __forceinline__ const uint16_t *head_part(const uint16_t *pool, int pg, int Hkv, int kvh) {
  return pool + ((long long)pg * Hkv + kvh) * 2 * kPageHead;
}

// K fragments of two pages: the A operand of S^T = K . Q^T (lane: slot lr, dims
// 8*lg..8*lg+7 of each 32-dim chunk).
__device__ __forceinline__ void load_k2(Frag8 (&k)[2][4], const uint16_t *pool, int Hkv, int kvh, int pg0, int pg1,
                                        int lr, int lg) {
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const uint16_t *kp = head_part(pool, t ? pg1 : pg0, Hkv, kvh);
#pragma unroll
    for (int cc = 0; cc < 4; cc++) k[t][cc].q = ld_stream16(kp + cc * (kPage * 32) + lr * 32 + 8 * lg);
  }
}

// V fragments of two pages: the A operand of O^T = V^T . P^T (lane: dim 16*cc + lr,
// slots 4*lg..4*lg+3 of each page).
__device__ __forceinline__ void load_v2(uint2 (&v)[2][8], const uint16_t *pool, int Hkv, int kvh, int pg0, int pg1,
                                        int lr, int lg) {
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const uint16_t *vp = head_part(pool, t ? pg1 : pg0, Hkv, kvh) + kPageHead;
#pragma unroll
    for (int cc = 0; cc < 8; cc++) v[t][cc] = ld_stream8(vp + (16 * cc + lr) * kPage + 4 * lg);
  }
}

// keep the bf16 halves of w whose key index (k, k + 1) is below L
__device__ __forceinline__ uint32_t mask_pair(uint32_t w, int k, int L) {
  return (k < L ? (w & 0xffffu) : 0u) | (k + 1 < L ? (w & 0xffff0000u) : 0u);
}

// WS waves share a kv head's chunk of ck keys: wave s streams keys [s * ck / WS, (s + 1) * ck / WS)
// of it, and the workgroup merges the WS (max, sum, o) states in LDS in wave order, so a
// chunk's result depends only on its keys.  More waves with shorter key runs each keep more
// loads in flight than one wave per kv head walking the whole chunk.
constexpr int kStateFloats = 32 + 2;  // o[8][4], max, sum per lane

// Stamps (a build with JIT_ATTN_STAMPS=1 only, bench.py --attn-phases): wave 0 of every workgroup
// records s_memrealtime (100 MHz) at entry (0), once its first step's K has landed (1; that build
// waits for it there), at the end of its key loop (2), after the splits' states have met in LDS (3)
// and at its end (4).
#ifndef JIT_ATTN_STAMPS
#define JIT_ATTN_STAMPS 0
#endif
#if JIT_ATTN_STAMPS
constexpr int kAttnStampSlots = 1 << 14;
__device__ uint64_t g_attn_stamps[kAttnStampSlots][8];
#define ATTN_STAMP(i) ts[i] = __builtin_amdgcn_s_memrealtime()
#else
#define ATTN_STAMP(i) \
  do {                \
  } while (0)
#endif

template <int WS>
__global__ __launch_bounds__(512) void paged_attn_kernel(const AttnArgs a) {
#if JIT_ATTN_STAMPS
  uint64_t ts[5] = {__builtin_amdgcn_s_memrealtime(), 0, 0, 0, 0};
  auto stamp_out = [&]() {
    ts[4] = __builtin_amdgcn_s_memrealtime();
    const int slot = blockIdx.x + gridDim.x * blockIdx.y;
    if (threadIdx.x < 5 && slot < kAttnStampSlots) {
      uint64_t v = ts[0];
      for (int i = 1; i < 5; i++) v = threadIdx.x == i ? ts[i] : v;
      g_attn_stamps[slot][threadIdx.x] = v;
      if (threadIdx.x == 0) g_attn_stamps[slot][7] = 1;
    }
  };
#endif
  static_assert(WS == kAttnSplits, "the chunk rule rounds to whole 32-key steps of each of WS waves");
  extern __shared__ float xstate[];  // [WS - 1][hb][kStateFloats][64]
  const int gc = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = lane_id();
  const int hb = a.hb;
  const int kvl = wave % hb, split = wave / hb;
  const int kvh = blockIdx.y * hb + kvl;
  const bool live = kvh < a.Hkv;  // (dead waves still meet the barrier of the merge)
  const int b = a.chunk_seq[gc];
  const int L = a.lens[b];
  const int c = gc - a.chunk_start[b];
  const int ck = chunk_tokens(L), kRun = ck / WS;
  const int nchunks = (L + ck - 1) / ck;
  const int lr = l & 15, lg = l >> 4;
  const int G = a.G;
  const int wk0 = c * ck + split * kRun;
  const int wk1 = min(c * ck + (split + 1) * kRun, L);
  const int npg = wk1 > wk0 ? (wk1 - wk0 + kPage - 1) / kPage : 0;  // split 0 always holds a key
  const int nst = live ? (npg + 1) >> 1 : 0;                          // 32-key steps
  // the run's page ids, one per lane (at most kRun / 16 <= 64)
  const int my_page = l < npg ? a.page_table[(long long)b * a.max_pages + (wk0 >> 4) + l] : 0;
  const int last = npg - 1;
  // page id i of the chunk (past the last page: the last page again, whose keys are
  // masked, so prefetches need no branch)
  auto page = [&](int i) { return __builtin_amdgcn_readlane(my_page, min(i, last)); };

  Frag8 kf[2][4];
  uint2 vv[2][8];
  // K before V, as in the loop, so a step's K wait leaves its V loads in flight
  auto first_loads = [&]() {
    if (nst > 0) {
      load_k2(kf, a.pool, a.Hkv, kvh, page(0), page(1), lr, lg);
      asm volatile("" ::: "memory");
      load_v2(vv, a.pool, a.Hkv, kvh, page(0), page(1), lr, lg);
    }
  };
  // Q^T fragments (B operand of S^T = K . Q^T): q head lr, dims 8*lg.. of each chunk
  Frag8 qf[4];
#pragma unroll
  for (int cc = 0; cc < 4; cc++) qf[cc].q = make_uint4(0, 0, 0, 0);
  if (a.qkv == nullptr) {
    if (lr < G) {
      const uint16_t *qp = a.q + ((long long)b * a.H + kvh * G + lr) * kD + 8 * lg;
#pragma unroll
      for (int cc = 0; cc < 4; cc++) qf[cc].q = *(const uint4 *)(qp + 32 * cc);
    }
    first_loads();
  } else {
    // The step's own token (position L - 1) from its raw q/k/v row: every workgroup norms and
    // rotates its q heads (qk_head_norm_rope, as jit_qk_norm_rope_append does: the same bits) into
    // LDS, and the workgroup of the sequence's last chunk first writes the token's K and V of its
    // kv heads into the pool.  The barrier's fence orders those stores before this workgroup's
    // reads of the token's page; other workgroups never read it.  A wave whose first step holds
    // that page issues its first loads after the barrier, the others right after requesting the
    // token's values: vector loads complete in order, so values requested behind the first K/V
    // loads would be waited for only once those had landed.
    const int tok = L - 1;
    const bool defer = wk1 == L && tok < wk0 + 32;
    const int nh = a.H + 2 * a.Hkv;
    const uint16_t *row = a.qkv + (long long)b * nh * kD;
    uint16_t *qs = (uint16_t *)(xstate + (WS - 1) * hb * kStateFloats * 64);  // [hb][G][128], past the states
    constexpr int kQHeads = (16 + WS - 1) / WS;  // q heads a wave norms (G <= 16)
    const bool writer = live && c == nchunks - 1 && split < 2;  // the token's K (split 0) or V (split 1)
    uint16_t qx[kQHeads][2], tx[2] = {0, 0}, qw[2] = {0, 0}, kw[2] = {0, 0};
    float fr = 0.0f;
    int pg = 0;
    if (live) {
      fr = a.inv_freq[l];
      qw[0] = a.qn_w[l];
      qw[1] = a.qn_w[l + 64];
#pragma unroll
      for (int i = 0; i < kQHeads; i++) {
        const int hq = split + WS * i;
        if (hq < G) {  // (uniform over the wave)
          const uint16_t *src = row + (kvh * G + hq) * kD;
          qx[i][0] = src[l];
          qx[i][1] = src[l + 64];
        }
      }
      if (writer) {
        pg = a.page_table[(long long)b * a.max_pages + (tok >> 4)];
        const uint16_t *src = row + (a.H + (split ? a.Hkv : 0) + kvh) * kD;
        tx[0] = src[l];
        tx[1] = src[l + 64];
        if (split == 0) {
          kw[0] = a.kn_w[l];
          kw[1] = a.kn_w[l + 64];
        }
      }
    }
    asm volatile("" ::: "memory");  // (the token's loads stay ahead of the first K/V)
    if (!defer) first_loads();
    if (live) {
      const float ang = (float)tok * fr;
      if (writer) {
        const int slot = tok & (kPage - 1);
        uint16_t *hp = (uint16_t *)a.pool + ((long long)pg * a.Hkv + kvh) * 2 * kPageHead;
        if (split == 0) {  // K: normed and rotated, into the chunk-major K part
          uint32_t o1, o2;
          qk_head_norm_rope(bf2f(tx[0]), bf2f(tx[1]), bf2f(kw[0]), bf2f(kw[1]), a.eps, ang, o1, o2);
          hp[k_page_offset(slot, l)] = (uint16_t)o1;
          hp[k_page_offset(slot, l + 64)] = (uint16_t)o2;
        } else {  // V: as it is, into the dim-major V part
          hp[kPageHead + l * kPage + slot] = tx[0];
          hp[kPageHead + (l + 64) * kPage + slot] = tx[1];
        }
      }
#pragma unroll
      for (int i = 0; i < kQHeads; i++) {
        const int hq = split + WS * i;
        if (hq < G) {  // (uniform over the wave)
          uint32_t o1, o2;
          qk_head_norm_rope(bf2f(qx[i][0]), bf2f(qx[i][1]), bf2f(qw[0]), bf2f(qw[1]), a.eps, ang, o1, o2);
          qs[(kvl * G + hq) * kD + l] = (uint16_t)o1;
          qs[(kvl * G + hq) * kD + l + 64] = (uint16_t)o2;
        }
      }
    }
    __syncthreads();
    if (live && lr < G) {
#pragma unroll
      for (int cc = 0; cc < 4; cc++) qf[cc].q = *(const uint4 *)(qs + (kvl * G + lr) * kD + 8 * lg + 32 * cc);
    }
    if (defer) first_loads();
  }
  // Lane (lr, lg) owns q head lr throughout: scores S^T[key 4*lg + i][head lr], the
  // running max / sum of head lr, and O^T[dim 16*cc + 4*lg + i][head lr].
  float m_run = -INFINITY, l_run = 0.0f;
  f32x4 o[8];
#pragma unroll
  for (int cc = 0; cc < 8; cc++) o[cc] = f32x4{0.f, 0.f, 0.f, 0.f};

#if JIT_ATTN_STAMPS
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("" ::: "memory");
  ATTN_STAMP(1);
#endif
  for (int st = 0; st < nst; st++) {
    const int k0 = wk0 + 32 * st;
    f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
      s0 = mfma16x16x32(kf[0][cc], qf[cc], s0);
      s1 = mfma16x16x32(kf[1][cc], qf[cc], s1);
    }
    // K registers are free: the next step's K is in flight during softmax and P.V
    load_k2(kf, a.pool, a.Hkv, kvh, page(2 * st + 2), page(2 * st + 3), lr, lg);
    // keys past the run are masked on its last step only; the scale is applied inside the
    // exponent's fma (the max of the raw scores times the positive scale is the scaled max)
    float p0[4], p1[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      p0[i] = s0[i];
      p1[i] = s1[i];
    }
    if (k0 + 32 > wk1) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int key = k0 + 4 * lg + i;
        p0[i] = key < wk1 ? p0[i] : -INFINITY;
        p1[i] = key + 16 < wk1 ? p1[i] : -INFINITY;
      }
    }
    float tmax = fmaxf(p0[0], p1[0]);
#pragma unroll
    for (int i = 1; i < 4; i++) tmax = fmaxf(tmax, fmaxf(p0[i], p1[i]));
    tmax = max_xor32(max_xor16(tmax)) * a.qk_scale;
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      p0[i] = __builtin_amdgcn_exp2f(fmaf(p0[i], a.qk_scale, -m_new));
      p1[i] = __builtin_amdgcn_exp2f(fmaf(p1[i], a.qk_scale, -m_new));
      psum += p0[i] + p1[i];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // P^T fragments (B operand): head lr, k slots 8*lg + j = key 4*lg + j of the first
    // page (j < 4) and of the second (j >= 4) -- the lane's own probabilities, as bf16
    // high parts (pf) and bf16 residuals (pl): O^T += V^T . pf^T + V^T . pl^T keeps P at
    // 16 significant bits, as the reference's fp32 P.V does (one bf16 P rounds each
    // probability by up to 2^-9 and moves ~40% of the bf16 outputs by an ulp)
    Frag8 pf, pl;
    split_bf16x2(p0[0], p0[1], pf.u[0], pl.u[0]);
    split_bf16x2(p0[2], p0[3], pf.u[1], pl.u[1]);
    split_bf16x2(p1[0], p1[1], pf.u[2], pl.u[2]);
    split_bf16x2(p1[2], p1[3], pf.u[3], pl.u[3]);
    if (lr >= G) {
      pf.q = make_uint4(0, 0, 0, 0);
      pl.q = make_uint4(0, 0, 0, 0);
    }
    // the tail page may hold stale slots past L: their p is 0, make their V 0 too
    if (k0 + 32 > L) {
      const int kb = k0 + 4 * lg;
#pragma unroll
      for (int cc = 0; cc < 8; cc++) {
        vv[0][cc].x = mask_pair(vv[0][cc].x, kb, L);
        vv[0][cc].y = mask_pair(vv[0][cc].y, kb + 2, L);
        vv[1][cc].x = mask_pair(vv[1][cc].x, kb + 16, L);
        vv[1][cc].y = mask_pair(vv[1][cc].y, kb + 18, L);
      }
    }
    // rescale only when some head's running max moved (alpha == 1 is a no-op)
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int cc = 0; cc < 8; cc++)
#pragma unroll
        for (int i = 0; i < 4; i++) o[cc][i] *= alpha;
    }
    Frag8 vf[8];
#pragma unroll
    for (int cc = 0; cc < 8; cc++) {
      vf[cc].u[0] = vv[0][cc].x;
      vf[cc].u[1] = vv[0][cc].y;
      vf[cc].u[2] = vv[1][cc].x;
      vf[cc].u[3] = vv[1][cc].y;
      o[cc] = mfma16x16x32(vf[cc], pf, o[cc]);
    }
#pragma unroll
    for (int cc = 0; cc < 8; cc++) o[cc] = mfma16x16x32(vf[cc], pl, o[cc]);
    load_v2(vv, a.pool, a.Hkv, kvh, page(2 * st + 2), page(2 * st + 3), lr, lg);
    // keep these loads in this step: sunk into the next step they would only be
    // issued once that step's K has arrived
    asm volatile("" ::: "memory");
  }
  ATTN_STAMP(2);
  if (WS > 1) {  // the splits' states meet: split 0 of each kv head adds splits 1.. in order
    if (split > 0) {
      float *st = xstate + (((split - 1) * hb + kvl) * kStateFloats) * 64 + l;
#pragma unroll
      for (int cc = 0; cc < 8; cc++)
#pragma unroll
        for (int i = 0; i < 4; i++) st[(4 * cc + i) * 64] = o[cc][i];
      st[32 * 64] = m_run;
      st[33 * 64] = l_run;
    }
    __syncthreads();
    ATTN_STAMP(3);
    if (split > 0 || !live) return;
#pragma unroll
    for (int sp = 1; sp < WS; sp++) {
      const float *st = xstate + (((sp - 1) * hb + kvl) * kStateFloats) * 64 + l;
      const float m2 = st[32 * 64], l2 = st[33 * 64];
      const float M = fmaxf(m_run, m2);  // split 0 holds a key: M is finite
      const float f0 = exp2f(m_run - M), f1 = exp2f(m2 - M);
#pragma unroll
      for (int cc = 0; cc < 8; cc++)
#pragma unroll
        for (int i = 0; i < 4; i++) o[cc][i] = o[cc][i] * f0 + st[(4 * cc + i) * 64] * f1;
      l_run = l_run * f0 + l2 * f1;
      m_run = M;
    }
  } else if (!live) {
    return;
  }
#if JIT_ATTN_STAMPS
  if (wave == 0) stamp_out();
#endif
  // per-head sum over the four lane groups
  const float l_tot = sum_xor32(sum_xor16(l_run));
  if (lr >= G) return;
  const long long row = (long long)b * a.H + kvh * G + lr;  // this lane's q head
  if (nchunks == 1) {
    const float inv = 1.0f / l_tot;
#pragma unroll
    for (int cc = 0; cc < 8; cc++) {
      uint2 w;
      w.x = pack_bf16x2(o[cc][0] * inv, o[cc][1] * inv);
      w.y = pack_bf16x2(o[cc][2] * inv, o[cc][3] * inv);
      *(uint2 *)(a.out + row * kD + 16 * cc + 4 * lg) = w;
    }
  } else {
    const long long r = (long long)gc * a.H + kvh * G + lr;
#pragma unroll
    for (int cc = 0; cc < 8; cc++)
      *(float4 *)(a.part_o + r * kD + 16 * cc + 4 * lg) = make_float4(o[cc][0], o[cc][1], o[cc][2], o[cc][3]);
    if (lg == 0) {
      a.part_ml[r * 2 + 0] = m_run;
      a.part_ml[r * 2 + 1] = l_tot;
    }
  }
}

// Merge of a sequence's chunk partials: one workgroup of 512 threads per (sequence,
// q head).  The partials were written by workgroups on other XCDs, so every read
// here misses this XCD's L2; the chunks are spread over 16 chunk lanes (thread =
// chunk lane x 32 dim quads) so that many of those reads are in flight at once
// instead of one per chunk in a serial chain.  Lane j merges chunks j, j + 16, ...
// online (running max, one pass over the partials), and the 16 lane states are
// merged in lane order: a fixed order that depends only on the sequence's chunk count.
constexpr int kMergeLanes = 16;

__global__ __launch_bounds__(512) void attn_merge_kernel(const int32_t *__restrict__ chunk_start,
                                                         const float *__restrict__ part_o,
                                                         const float *__restrict__ part_ml, int H,
                                                         uint16_t *__restrict__ out) {
  const int b = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
  // the sequence's chunks from the plan's prefix alone (one load of two adjacent words, where
  // lens[b] and then the prefix were two round trips in a row; the plan is lens' chunk split)
  const long long c0 = chunk_start[b];
  const int n = chunk_start[b + 1] - (int)c0;
  if (n <= 1) return;
  __shared__ float4 s_o[kMergeLanes][32];
  __shared__ float s_m[kMergeLanes], s_l[kMergeLanes];
  const int cl = t >> 5, dq = t & 31;
  float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
  float m_run = -INFINITY, Ls = 0.0f;  // every chunk holds a key: its max is finite
  // four iterations' loads go out together (bs = 1's 128 chunks, 8 a lane: attention 88.6 -> 88.1-88.3
  // us; 2 before).  8 would take the kernel past 64 VGPRs, one wave a SIMD fewer, and cost config 2's
  // 1,024 merge workgroups 0.7 us.  The arithmetic and its order are the same at any unroll.
#pragma unroll 4
  for (int c = cl; c < n; c += kMergeLanes) {
    const long long r = (c0 + c) * H + h;
    const float2 ml = *(const float2 *)(part_ml + r * 2);
    const float4 o = *(const float4 *)(part_o + r * kD + 4 * dq);
    const float mn = fmaxf(m_run, ml.x);
    const float fa = exp2f(m_run - mn), fb = exp2f(ml.x - mn);
    Ls = Ls * fa + ml.y * fb;
    O.x = O.x * fa + o.x * fb;
    O.y = O.y * fa + o.y * fb;
    O.z = O.z * fa + o.z * fb;
    O.w = O.w * fa + o.w * fb;
    m_run = mn;
  }
  s_o[cl][dq] = O;
  if (dq == 0) {
    s_m[cl] = m_run;
    s_l[cl] = Ls;
  }
  __syncthreads();
  if (t >= 32) return;
  float M = s_m[0];
#pragma unroll
  for (int j = 1; j < kMergeLanes; j++) M = fmaxf(M, s_m[j]);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float lsum = 0.0f;
#pragma unroll
  for (int j = 0; j < kMergeLanes; j++) {  // lanes without a chunk hold m = -inf: weight 0
    const float f = exp2f(s_m[j] - M);
    const float4 v = s_o[j][t];
    acc.x += v.x * f;
    acc.y += v.y * f;
    acc.z += v.z * f;
    acc.w += v.w * f;
    lsum += s_l[j] * f;
  }
  const float inv = 1.0f / lsum;
  uint2 w;
  w.x = pack_bf16x2(acc.x * inv, acc.y * inv);
  w.y = pack_bf16x2(acc.z * inv, acc.w * inv);
  *(uint2 *)(out + ((long long)b * H + h) * kD + 4 * t) = w;
}

#ifndef JIT_PF_PSPLIT
#define JIT_PF_PSPLIT 1  // prefill P.V with P as bf16 high part + bf16 residual (two MFMAs)
#endif

// ---------------------------------------------------------------- prefill (causal chunks)
// Causal attention of prefill chunks over the paged pool: query token t of a chunk (at
// position ctx + t of its sequence) attends keys 0 .. ctx + t, whose K/V the chunk's
// append already wrote (mx.fast.scaled_dot_product_attention with mask = "causal" over the
// slot's keys, Q36/model/attention.py:70-74).  A workgroup owns kPfWaves * kPfTiles 16-row
// q tiles of one kv head -- a tile's rows are 16 / G tokens x the G q heads that share the
// kv head -- and streams the keys up to its last token in steps of kPfHalves x 32 keys through
// LDS (one barrier and one softmax update a step), so each
// K/V byte it reads serves all its tokens; per step and tile the arithmetic is the decode
// kernel's (S^T = K . Q^T, online softmax in the exp2 domain, O^T += V^T . P^T), with keys
// past a row's position masked.  A token's result depends only on its q row and its keys:
// the steps and their order are the same wherever the token's tile sits.
constexpr int kPfWaves = 8, kPfTiles = 2;
constexpr int kPfHalves = 4;                                           // 32-key halves of a step
constexpr int kPfStages = 2;                                           // LDS ring depth (steps)
constexpr int kPfChunks = kPfHalves * 4 * kPageHead * 2 / 1024 / kPfWaves;  // 1 KB chunks of a step per wave
// each wave stages the K and V of one page per step (4 parts of 4 KB in 1 KB chunks)
static_assert(kPfChunks == 8 && kPfWaves == 2 * kPfHalves, "one page per wave per step");
static_assert(kPfStages == 2, "the page-id prefetch below runs one step ahead of the staging");

// Key parts.  A token's keys are cut at the fixed positions kPfPartKeys, 2 kPfPartKeys, ...
// (whole 128-key steps), and each part of a row block is a work item of its own, so a chunk
// deep into a long context becomes several items of at most kPfPartSteps steps that the
// dispatcher can place beside the short ones (config 3: the longest item falls from 68 steps to
// 48, against a mean of 46).  A token whose keys all precede kPfPartKeys is finished by its one
// item; the others leave fp32 partials (m, l, o) per part, which prefill_merge_kernel combines in
// part order.  The cuts depend only on key positions, so a token's bits still depend only on its
// q row and its keys.
#ifndef JIT_PF_PART_STEPS
#define JIT_PF_PART_STEPS 48
#endif
constexpr int kPfPartSteps = JIT_PF_PART_STEPS;
constexpr int kPfPartKeys = kPfPartSteps * 32 * kPfHalves;
constexpr int kPfSlot = kD + 4;  // floats of one (token, part, head) partial: o, max, sum, 2 pad (16 B rows)

struct PrefillArgs {
  const uint16_t *q;          // [T, H, 128] bf16 (normed, rotated)
  const uint16_t *pool;
  const int32_t *page_table;  // [S, max_pages]
  const int32_t *blk_chunk;   // [nblk] chunk of each workgroup
  const int32_t *blk_q0;      // [nblk] first token (within the chunk) of each workgroup
  const int32_t *blk_part;    // [nblk] key part of each workgroup
  const int32_t *chunk_seq, *chunk_ctx, *chunk_len, *chunk_row;  // [C]
  uint16_t *out;              // [T, H, 128] bf16
  float *part;                // [T][pmax][H][kPfSlot] fp32: o[128], max, sum (tokens of several parts)
  int max_pages, H, Hkv, G, pmax;
  float qk_scale;             // scale * log2(e)
};

__global__ __launch_bounds__(64 * kPfWaves) void prefill_attn_kernel(const PrefillArgs a) {
  // a ring of kPfStages steps of kPfHalves x 32 keys, each half K0, V0, K1, V1 of its two pages
  // (4 KB each), filled by direct global->LDS loads kPfStages - 1 steps ahead of the step
  // being computed
  __shared__ __attribute__((aligned(16))) uint16_t kvs[kPfStages][kPfHalves * 4 * kPageHead];
  // one dimension, the kv heads of an item adjacent: the hardware dispatches workgroups in index
  // order, so the plan's longest-first order holds across the kv heads (a (item, kv head) grid
  // dispatched every item of kv head 0 before any of kv head 1)
  const int item = blockIdx.x / a.Hkv, kvh = blockIdx.x % a.Hkv;
  const int ch = a.blk_chunk[item], q0 = a.blk_q0[item], part = a.blk_part[item];
  const int seq = a.chunk_seq[ch], ctx = a.chunk_ctx[ch], len = a.chunk_len[ch], row0 = a.chunk_row[ch];
  const int G = a.G, TR = 16 / G, tpw = kPfTiles * TR;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = lane_id();
  const int lr = l & 15, lg = l >> 4;
  const int tlast = min(q0 + kPfWaves * tpw, len) - 1;  // the workgroup's last token
  const int kend = ctx + tlast + 1;                     // its keys: [0, kend)
  const int nst = (kend + 32 * kPfHalves - 1) / (32 * kPfHalves), npages = (kend + 15) >> 4;
  // this item's steps: part `part` of the keys (the plan makes an item only for parts that hold a
  // key of the block's last token)
  const int st0 = part * kPfPartSteps, st1 = min(nst, st0 + kPfPartSteps);
  const int32_t *prow = a.page_table + (long long)seq * a.max_pages;
  // wave w stages on step st page 2 kPfHalves st + w of the workgroup's keys (a page past the keys
  // repeats the last one); lane i reads the page of wave i % kPfWaves, so that the ids stay in a
  // vector register until the step that stages them reads its lane
  auto pages_of_step = [&](int st) {
    return prow[min(2 * kPfHalves * st + (l & (kPfWaves - 1)), npages - 1)];
  };

  // the lane's q row in tile j: token t (clamped into the chunk), head kvh * G + lr % G
  int tok[kPfTiles];
  bool store[kPfTiles];
  Frag8 qf[kPfTiles][4];
  float m_run[kPfTiles], l_run[kPfTiles];
  f32x4 o[kPfTiles][8];
#pragma unroll
  for (int j = 0; j < kPfTiles; j++) {
    const int t = q0 + wave * tpw + j * TR + lr / G;
    store[j] = t < len;
    tok[j] = min(t, len - 1);
    const uint16_t *qp = a.q + ((long long)(row0 + tok[j]) * a.H + kvh * G + lr % G) * kD + 8 * lg;
#pragma unroll
    for (int cc = 0; cc < 4; cc++) qf[j][cc].q = *(const uint4 *)(qp + 32 * cc);
    m_run[j] = -INFINITY;
    l_run[j] = 0.0f;
#pragma unroll
    for (int cc = 0; cc < 8; cc++) o[j][cc] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // the first position among each tile's rows (uniform over the wave)
  int tile_first[kPfTiles];
#pragma unroll
  for (int j = 0; j < kPfTiles; j++) tile_first[j] = ctx + min(q0 + wave * tpw + j * TR, len - 1);
  __syncthreads();

  // staging of step st into stage st % kPfStages: chunk c = kPfChunks * wave + u (1 KB, one
  // load instruction of the wave) of the step's four parts -- K of page 2st, V of page 2st, K of
  // page 2st + 1, V of page 2st + 1 (a page past the keys repeats the last one: its slots are
  // masked, and the steps past the end are loaded and never read, so every wave always has
  // (kPfStages - 1) * kPfChunks loads issued after a step's own)
  // The loads are issued from inline assembly: the compiler then keeps no track of them (its
  // own waits would otherwise include them before every LDS read, as it cannot tell the
  // stages apart), and the explicit waits below order them; its waits for other loads only
  // grow more conservative.
  const uint32_t kvs_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)&kvs[0][0];
#define PF_STAGE(st, pv)                                                                               \
  {                                                                                                    \
  const int pg = __builtin_amdgcn_readlane(pv, wave);                                                  \
  _Pragma("unroll") for (int u = 0; u < kPfChunks; u++) {                                              \
    const int c = kPfChunks * wave + u, part = c >> 2;  /* part: K or V (part & 1) of page pg */       \
    const uint16_t *src = head_part(a.pool, pg, a.Hkv, kvh) + (part & 1) * kPageHead + (c & 3) * 512 + 8 * l; \
    const uint32_t dst = __builtin_amdgcn_readfirstlane(                                               \
        kvs_lds + 2 * (((st) % kPfStages) * kPfHalves * 4 * kPageHead + 512 * c));                     \
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(dst) : "memory", "m0"); \
  }                                                                                                    \
  }
  // the q fragments have landed before the first staged load is issued: the compiler's waits
  // for them would otherwise sit inside the loop, where they would also wait for the staging
#pragma unroll
  for (int j = 0; j < kPfTiles; j++)
#pragma unroll
    for (int cc = 0; cc < 4; cc++)
      asm volatile("" ::"v"(qf[j][cc].u[0]), "v"(qf[j][cc].u[1]), "v"(qf[j][cc].u[2]), "v"(qf[j][cc].u[3]));
  PF_STAGE(st0, pages_of_step(st0));
  // the pages of the next step to stage, read one step ahead so that their latency hides behind a
  // step's arithmetic (the wait for them is the loop's own wait for the staging)
  int pv_next = pages_of_step(st0 + 1);
  // the wait that leaves the loads of the next kPfStages - 2 steps in flight, and no lgkm or
  // export wait (vmcnt is split over bits 3:0 and 15:14)
  constexpr int kPfVm = (kPfStages - 2) * kPfChunks;
  constexpr int kPfWait = (kPfVm & 15) | ((kPfVm >> 4) << 14) | (7 << 4) | (15 << 8);
  for (int st = st0; st < st1; st++) {
    // this wave's loads of step st have landed and its reads of step st - 1 are done; after
    // the barrier so are every wave's, and stage (st - 1) % kPfStages may be refilled
    // (the empty asm statements keep the compiler from moving LDS accesses across the barrier,
    // which is issued bare: a __syncthreads fence would wait for every load in flight)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kPfWait);
    __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    PF_STAGE(st + 1, pv_next);
    pv_next = pages_of_step(st + 2);
    const uint16_t *kvst = kvs[st % kPfStages];
    const int k0 = 32 * kPfHalves * st;
    // the step's slots past the workgroup's keys (its last step only) may hold stale bits, which a
    // p of 0 would not cancel (0 x NaN): their V is zeroed in the stage before any wave reads it
    // (one more barrier, on that step only)
    if (k0 + 32 * kPfHalves > kend) {
      uint16_t *vst = kvs[st % kPfStages];
      for (int e = tid; e < kPfHalves * 2 * kPageHead; e += 64 * kPfWaves) {
        const int slot = e % kPage, dim = (e / kPage) % kD, pgh = e / kPageHead;  // pgh: page 2 h + p of the step
        if (k0 + kPage * pgh + slot >= kend) vst[(2 * pgh + 1) * kPageHead + dim * kPage + slot] = 0;
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    // Key order within each 32-key half h (keys k0 + 32 h ..): the P.V MFMA's k index 8 lg + j
    // (lane group lg) is key 8 lg + j of the half (page lg / 2, slot 8 (lg % 2) + j), so a
    // lane's V operand is 8 consecutive slots of one page -- 16 contiguous bytes of the page's
    // dim-major V part.  Score tile t therefore holds in its row 4 lg + i key 8 lg + 4 t + i:
    // its A operand row r (lane lr = r) reads the K row of key 8 (r / 4) + 4 t + r % 4, and
    // each lane's 8 scores of a half are then exactly its P^T operand (tile 0: j < 4, tile 1:
    // j >= 4).
    // phase 1: scores of every tile and half, one score tile of K fragments at a time
    f32x4 sc[kPfTiles][kPfHalves][2];
#pragma unroll
    for (int h = 0; h < kPfHalves; h++)
#pragma unroll
      for (int t = 0; t < 2; t++) {
        Frag8 kf[4];
        const int kr = 8 * (lr >> 2) + 4 * t + (lr & 3);  // the key of this lane's A row
        const uint16_t *kvsc = kvst + h * 4 * kPageHead;
#pragma unroll
        for (int cc = 0; cc < 4; cc++)
          kf[cc].q = *(const uint4 *)(kvsc + 2 * (kr >> 4) * kPageHead + cc * (kPage * 32) + (kr & 15) * 32 + 8 * lg);
#pragma unroll
        for (int j = 0; j < kPfTiles; j++) {  // (a tile past the step's keys discards its scores)
          sc[j][h][t] = mfma16x16x32(kf[0], qf[j][0], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int cc = 1; cc < 4; cc++) sc[j][h][t] = mfma16x16x32(kf[cc], qf[j][cc], sc[j][h][t]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    // online softmax of every tile over the step's keys: the masked scores' running max first
    // (the o rescale happens before the step's first P.V MFMA).  Keys past a row's position are
    // masked on the steps that reach into the tile's rows (a tile whose rows all precede the
    // step's keys is masked whole: its p are 0 and its state is left as it was); the scale is
    // applied inside the exponent (max of the raw scores times the positive scale is the max of
    // the scaled ones).
    float m_step[kPfTiles], alpha[kPfTiles], psum[kPfTiles];
#pragma unroll
    for (int j = 0; j < kPfTiles; j++) {
      if (k0 + 32 * kPfHalves - 1 > tile_first[j]) {
        const int pos = ctx + tok[j];
#pragma unroll
        for (int h = 0; h < kPfHalves; h++)
#pragma unroll
          for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const int key = k0 + 32 * h + 8 * lg + 4 * t + i;
              sc[j][h][t][i] = key <= pos ? sc[j][h][t][i] : -INFINITY;
            }
      }
      float tmax = sc[j][0][0][0];
#pragma unroll
      for (int h = 0; h < kPfHalves; h++)
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int i = 0; i < 4; i++) tmax = fmaxf(tmax, sc[j][h][t][i]);
      tmax = max_xor32(max_xor16(tmax)) * a.qk_scale;
      // finite for every row with a key in this part (its first key is in the part's first step);
      // a row without one (a token before the part's first key) turns NaN in its own column only
      // and is never stored
      m_step[j] = fmaxf(m_run[j], tmax);
      alpha[j] = __builtin_amdgcn_exp2f(m_run[j] - m_step[j]);
      psum[j] = 0.0f;
      if (__any(alpha[j] != 1.0f)) {
#pragma unroll
        for (int cc = 0; cc < 8; cc++)
#pragma unroll
          for (int i = 0; i < 4; i++) o[j][cc][i] *= alpha[j];
      }
    }
    // O^T += V^T . P^T, software-pipelined over the halves: the probabilities of half h + 1 are
    // computed (vector ALU) while the P.V MFMAs of half h run on the matrix cores.  P^T
    // fragments of a half are bf16 high parts (pw) and, with JIT_PF_PSPLIT, bf16 residuals (pl),
    // in two buffers by the half's parity; the lane's 8 keys of a half are slots 8 (lg % 2) .. + 7
    // of page lg / 2.
    uint32_t pw[2][kPfTiles][4];
#if JIT_PF_PSPLIT
    uint32_t pl[2][kPfTiles][4];
#endif
    auto probs = [&](const int h) {
#pragma unroll
      for (int j = 0; j < kPfTiles; j++) {
        float p[2][4];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            p[t][i] = __builtin_amdgcn_exp2f(fmaf(sc[j][h][t][i], a.qk_scale, -m_step[j]));
            psum[j] += p[t][i];
          }
#if JIT_PF_PSPLIT
        split_bf16x2(p[0][0], p[0][1], pw[h & 1][j][0], pl[h & 1][j][0]);
        split_bf16x2(p[0][2], p[0][3], pw[h & 1][j][1], pl[h & 1][j][1]);
        split_bf16x2(p[1][0], p[1][1], pw[h & 1][j][2], pl[h & 1][j][2]);
        split_bf16x2(p[1][2], p[1][3], pw[h & 1][j][3], pl[h & 1][j][3]);
#else
        pw[h & 1][j][0] = pack_bf16x2_rne(p[0][0], p[0][1]);
        pw[h & 1][j][1] = pack_bf16x2_rne(p[0][2], p[0][3]);
        pw[h & 1][j][2] = pack_bf16x2_rne(p[1][0], p[1][1]);
        pw[h & 1][j][3] = pack_bf16x2_rne(p[1][2], p[1][3]);
#endif
      }
    };
    probs(0);
#pragma unroll
    for (int h = 0; h < kPfHalves; h++) {
      // (one region per half: its P.V MFMAs and the next half's probabilities)
      if (h + 1 < kPfHalves) probs(h + 1);
      const uint16_t *kvsc = kvst + h * 4 * kPageHead;
#pragma unroll
      for (int hv = 0; hv < 2; hv++) {
        Frag8 vf[4];
#pragma unroll
        for (int c4 = 0; c4 < 4; c4++)
          vf[c4].q = *(const uint4 *)(kvsc + (2 * (lg >> 1) + 1) * kPageHead + (16 * (4 * hv + c4) + lr) * kPage +
                                      8 * (lg & 1));
#pragma unroll
        for (int j = 0; j < kPfTiles; j++) {
          Frag8 pf;
#pragma unroll
          for (int i = 0; i < 4; i++) pf.u[i] = pw[h & 1][j][i];
#pragma unroll
          for (int c4 = 0; c4 < 4; c4++) o[j][4 * hv + c4] = mfma16x16x32(vf[c4], pf, o[j][4 * hv + c4]);
#if JIT_PF_PSPLIT
#pragma unroll
          for (int i = 0; i < 4; i++) pf.u[i] = pl[h & 1][j][i];
#pragma unroll
          for (int c4 = 0; c4 < 4; c4++) o[j][4 * hv + c4] = mfma16x16x32(vf[c4], pf, o[j][4 * hv + c4]);
#endif
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < kPfTiles; j++) {
      l_run[j] = l_run[j] * alpha[j] + psum[j];
      m_run[j] = m_step[j];
    }
  }
#undef PF_STAGE
  __builtin_amdgcn_s_waitcnt(0);  // no load may still write the LDS when the workgroup ends
#pragma unroll
  for (int j = 0; j < kPfTiles; j++) {
    const float l_tot = sum_xor32(sum_xor16(l_run[j]));
    if (!store[j]) continue;
    const int parts = (ctx + tok[j]) / kPfPartKeys + 1;  // the token's key parts
    const long long hrow = (long long)(row0 + tok[j]) * a.H + kvh * G + lr % G;
    if (parts == 1) {  // (then part == 0): the token's whole result
      const float inv = 1.0f / l_tot;
      uint16_t *op = a.out + hrow * kD + 4 * lg;
#pragma unroll
      for (int cc = 0; cc < 8; cc++) {
        uint2 w;
        w.x = pack_bf16x2(o[j][cc][0] * inv, o[j][cc][1] * inv);
        w.y = pack_bf16x2(o[j][cc][2] * inv, o[j][cc][3] * inv);
        *(uint2 *)(op + 16 * cc) = w;
      }
    } else if (part < parts) {  // this part's (max, sum, unnormalised o) of the token
      float *ps = a.part + (((long long)(row0 + tok[j]) * a.pmax + part) * a.H + kvh * G + lr % G) * kPfSlot;
#pragma unroll
      for (int cc = 0; cc < 8; cc++)
        *(float4 *)(ps + 16 * cc + 4 * lg) = make_float4(o[j][cc][0], o[j][cc][1], o[j][cc][2], o[j][cc][3]);
      if (lg == 0) *(float2 *)(ps + kD) = make_float2(m_run[j], l_tot);
    }
  }
}

// Merge of a token's key parts (tokens at or past kPfPartKeys): one workgroup of 8 H threads per
// token, thread (h, d) owning 16 dims of head h; the parts are combined online in part order
// (running max in the exp2 domain, as the parts were formed), then normalised and rounded as a
// whole-token result is.  Grid: (the longest chunk, chunks); other tokens exit at once.
__global__ __launch_bounds__(512) void prefill_merge_kernel(const int32_t *__restrict__ chunk_ctx,
                                                            const int32_t *__restrict__ chunk_len,
                                                            const int32_t *__restrict__ chunk_row,
                                                            const float *__restrict__ part, int H, int pmax,
                                                            uint16_t *__restrict__ out) {
  const int c = blockIdx.y, t = blockIdx.x;
  if (t >= chunk_len[c]) return;
  const int parts = (chunk_ctx[c] + t) / kPfPartKeys + 1;
  if (parts < 2) return;
  const long long row = chunk_row[c] + t;
  const int h = threadIdx.x >> 3, d0 = 16 * (threadIdx.x & 7);
  float M = -INFINITY, Ls = 0.0f;
  float O[16];
#pragma unroll
  for (int i = 0; i < 16; i++) O[i] = 0.0f;
  for (int p = 0; p < parts; p++) {
    const float *ps = part + ((row * pmax + p) * H + h) * kPfSlot;
    const float2 ml = *(const float2 *)(ps + kD);
    const float4 *po = (const float4 *)(ps + d0);
    const float mn = fmaxf(M, ml.x);
    const float fa = exp2f(M - mn), fb = exp2f(ml.x - mn);
    Ls = Ls * fa + ml.y * fb;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float4 v = po[q];
      O[4 * q] = O[4 * q] * fa + v.x * fb;
      O[4 * q + 1] = O[4 * q + 1] * fa + v.y * fb;
      O[4 * q + 2] = O[4 * q + 2] * fa + v.z * fb;
      O[4 * q + 3] = O[4 * q + 3] * fa + v.w * fb;
    }
    M = mn;
  }
  const float inv = 1.0f / Ls;
  uint4 w[2];
  uint32_t *wu = (uint32_t *)w;
#pragma unroll
  for (int i = 0; i < 8; i++) wu[i] = pack_bf16x2(O[2 * i] * inv, O[2 * i + 1] * inv);
  uint4 *op = (uint4 *)(out + (row * H + h) * kD + d0);
  op[0] = w[0];
  op[1] = w[1];
}

}  // namespace

extern "C" int jit_prefill_block_tokens(int H, int Hkv) {
  if (H <= 0 || Hkv <= 0 || H % Hkv != 0 || 16 % (H / Hkv) != 0) return -1;
  return kPfWaves * kPfTiles * 16 / (H / Hkv);
}

extern "C" int jit_prefill_part_keys(void) { return kPfPartKeys; }

extern "C" long long jit_prefill_workspace_bytes(int T, int pmax, int H) {
  if (T < 0 || pmax < 1 || H <= 0) return -1;
  return pmax > 1 ? (long long)T * pmax * H * kPfSlot * (long long)sizeof(float) : 0;
}

extern "C" int jit_paged_prefill_attn(const uint16_t *q, const uint16_t *pool, const int32_t *page_table,
                                      int max_pages, const int32_t *chunk_seq, const int32_t *chunk_ctx,
                                      const int32_t *chunk_len, const int32_t *chunk_row, int C,
                                      const int32_t *blk_chunk, const int32_t *blk_q0, const int32_t *blk_part,
                                      int nblk, int pmax, int max_len, int H, int Hkv, float scale,
                                      void *workspace, uint16_t *out, void *stream) {
  if (C < 0 || nblk < 0 || H <= 0 || Hkv <= 0 || max_pages <= 0 || pmax < 1 || max_len < 0)
    return jit::fail(JIT_EINVAL, "paged_prefill_attn: bad dims C=%d nblk=%d H=%d Hkv=%d pmax=%d max_len=%d", C,
                     nblk, H, Hkv, pmax, max_len);
  if (H % Hkv != 0) return jit::fail(JIT_EINVAL, "%d query heads do not share %d KV heads evenly", H, Hkv);
  if (16 % (H / Hkv) != 0)
    return jit::fail(JIT_EUNSUPPORTED, "paged_prefill_attn covers H / Hkv in {1, 2, 4, 8, 16}, got %d", H / Hkv);
  if (pmax > 1 && H > 64)
    return jit::fail(JIT_EUNSUPPORTED, "paged_prefill_attn merges key parts of up to 64 query heads, got %d", H);
  if (C == 0 || nblk == 0) return JIT_OK;
  if (!q || !pool || !page_table || !chunk_seq || !chunk_ctx || !chunk_len || !chunk_row || !blk_chunk ||
      !blk_q0 || !blk_part || !out || (pmax > 1 && !workspace))
    return jit::fail(JIT_EINVAL, "paged_prefill_attn: null pointer");
  const PrefillArgs a{q, pool, page_table, blk_chunk, blk_q0, blk_part, chunk_seq, chunk_ctx, chunk_len, chunk_row,
                      out, (float *)workspace, max_pages, H, Hkv, H / Hkv, pmax, scale * 1.44269504088896341f};
  prefill_attn_kernel<<<dim3(nblk * Hkv), 64 * kPfWaves, 0, (hipStream_t)stream>>>(a);
  int rc = jit::check_launch("jit_paged_prefill_attn");
  if (rc || pmax == 1 || max_len == 0) return rc;
  prefill_merge_kernel<<<dim3(max_len, C), 8 * H, 0, (hipStream_t)stream>>>(chunk_ctx, chunk_len, chunk_row,
                                                                              (const float *)workspace, H, pmax, out);
  return jit::check_launch("jit_paged_prefill_attn");
}



extern "C" int jit_kv_append_paged(const uint16_t *k, const uint16_t *v, int B, int Hkv,
                                   const int32_t *pos, const int32_t *page_table, int max_pages,
                                   uint16_t *pool, void *stream) {
  if (B < 0 || Hkv <= 0 || max_pages <= 0)
    return jit::fail(JIT_EINVAL, "kv_append_paged: bad dims B=%d Hkv=%d max_pages=%d", B, Hkv, max_pages);
  if (B == 0) return JIT_OK;
  if (!k || !v || !pos || !page_table || !pool) return jit::fail(JIT_EINVAL, "kv_append_paged: null pointer");
  kv_append_kernel<<<B, 256, 0, (hipStream_t)stream>>>(k, v, Hkv, pos, page_table, max_pages, pool);
  return jit::check_launch("jit_kv_append_paged");
}

extern "C" int jit_attn_plan(const int32_t *lens_host, int B, int32_t *chunk_start_host,
                             int32_t *chunk_seq_host, int seq_cap) {
  if (B < 0 || (B > 0 && (!lens_host || !chunk_start_host)))
    return jit::fail(JIT_EINVAL, "attn_plan: bad arguments");
  int total = 0;
  for (int b = 0; b < B; b++) {
    const int L = lens_host[b];
    if (L < 1) return jit::fail(JIT_EINVAL, "attn_plan: sequence %d has length %d (must be >= 1)", b, L);
    const int ck = jit_attn_chunk_tokens(L);
    chunk_start_host[b] = total;
    const int n = (L + ck - 1) / ck;
    if (chunk_seq_host) {
      if (total + n > seq_cap) return jit::fail(JIT_EINVAL, "attn_plan: chunk_seq capacity %d too small", seq_cap);
      for (int i = 0; i < n; i++) chunk_seq_host[total + i] = b;
    }
    total += n;
  }
  chunk_start_host[B] = total;
  return total;
}

extern "C" int64_t jit_attn_workspace_bytes(int total_chunks, int H) {
  return (int64_t)total_chunks * H * (kD + 2) * (int64_t)sizeof(float);
}

namespace {

// The two launches of a decode-attention call: the split-K chunks, then the chunk-order merge.
// `workspace` holds the fp32 partials of multi-chunk sequences (every partial the merge reads
// is written by the first launch of the same call, so nothing in it has to start at zero).
// The raw-row inputs of the fused entry (jit_paged_decode_attn_qkv).
struct FusedQkv {
  const uint16_t *qkv, *q_norm_w, *k_norm_w;
  const float *inv_freq;
  float eps;
};

int decode_attn_launch(const uint16_t *q, const uint16_t *pool, const int32_t *page_table, int max_pages,
                       const int32_t *lens, const int32_t *chunk_start, const int32_t *chunk_seq, int B, int H,
                       int Hkv, float scale, int total_chunks, void *workspace, uint16_t *out, hipStream_t st,
                       const char *what, const FusedQkv *fq = nullptr) {
  float *part_o = (float *)workspace;
  float *part_ml = part_o + (long long)total_chunks * H * kD;
  constexpr int WS = kAttnSplits;
  const int hb = Hkv < kAttnHeadsPerBlock ? Hkv : kAttnHeadsPerBlock;  // kv heads per workgroup (WS waves each)
  AttnArgs a{q, pool, page_table, lens, chunk_start, chunk_seq, part_o, part_ml, out,
             max_pages, H, Hkv, H / Hkv, scale * 1.44269504088896341f, hb,
             fq ? fq->qkv : nullptr, fq ? fq->q_norm_w : nullptr, fq ? fq->k_norm_w : nullptr,
             fq ? fq->inv_freq : nullptr, fq ? fq->eps : 0.0f};
  // the splits' states, and with fq the staged q heads of the workgroup's kv heads
  const size_t lds = (size_t)(WS - 1) * hb * kStateFloats * 64 * sizeof(float) +
                     (fq ? (size_t)hb * (H / Hkv) * kD * sizeof(uint16_t) : 0);
  paged_attn_kernel<WS><<<dim3(total_chunks, (Hkv + hb - 1) / hb), 64 * hb * WS, lds, st>>>(a);
  int rc = jit::check_launch(what);
  if (rc) return rc;
  attn_merge_kernel<<<dim3(B, H), 512, 0, st>>>(chunk_start, part_o, part_ml, H, out);
  return jit::check_launch(what);
}

// Scalar contract shared by both decode-attention entry points (host only, before any launch).
int decode_attn_contract(int B, int H, int Hkv, int max_pages, int total_chunks, const char *what) {
  if (B < 0 || H <= 0 || Hkv <= 0 || max_pages <= 0 || total_chunks < 0)
    return jit::fail(JIT_EINVAL, "%s: bad dims B=%d H=%d Hkv=%d", what, B, H, Hkv);
  if (H % Hkv != 0) return jit::fail(JIT_EINVAL, "%d query heads do not share %d KV heads evenly", H, Hkv);
  if (H / Hkv > 16) return jit::fail(JIT_EUNSUPPORTED, "%s covers H / Hkv <= 16, got %d", what, H / Hkv);
  return JIT_OK;
}

// ------------------------------------------------------------ allocation-free variant
// The split-K partials of jit_paged_decode_attn_noalloc live in this file-scope device array
// instead of a caller's workspace: every device the library runs on holds its own copy until
// the process ends.  On the host, `scratch` names a host-side stand-in, not device memory, so
// it is never passed to a kernel, a copy or a fill: host code uses only the per-device address
// hipGetSymbolAddress returns (g_scratch_dev), taken once per device with that device current.
static __device__ __align__(256) unsigned char scratch[JIT_ATTN_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_dev[kMaxDevices];

// The current device's address of `scratch` (looked up on the first call on that device).
int scratch_of_current_device(void **ptr, const char *what) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return jit::fail(JIT_ELAUNCH, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return jit::fail(JIT_EUNSUPPORTED, "%s: device %d is past the %d devices the scratch table covers", what, dev,
                     kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return jit::fail(JIT_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev,
                       hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *ptr = g_scratch_dev[dev];
  return JIT_OK;
}

}  // namespace

extern "C" int jit_paged_decode_attn(const uint16_t *q, const uint16_t *pool,
                                     const int32_t *page_table, int max_pages, const int32_t *lens,
                                     const int32_t *chunk_start, const int32_t *chunk_seq, int B,
                                     int H, int Hkv, float scale, int total_chunks, void *workspace,
                                     uint16_t *out, void *stream) {
  int rc = decode_attn_contract(B, H, Hkv, max_pages, total_chunks, "paged_decode_attn");
  if (rc) return rc;
  if (B == 0 || total_chunks == 0) return JIT_OK;
  if (!q || !pool || !page_table || !lens || !chunk_start || !chunk_seq || !workspace || !out)
    return jit::fail(JIT_EINVAL, "paged_decode_attn: null pointer");
  return decode_attn_launch(q, pool, page_table, max_pages, lens, chunk_start, chunk_seq, B, H, Hkv, scale,
                            total_chunks, workspace, out, (hipStream_t)stream, "jit_paged_decode_attn");
}

extern "C" int jit_paged_decode_attn_qkv(const uint16_t *qkv, const uint16_t *q_norm_w, const uint16_t *k_norm_w,
                                         float eps, const float *inv_freq, uint16_t *pool, const int32_t *page_table,
                                         int max_pages, const int32_t *lens, const int32_t *chunk_start,
                                         const int32_t *chunk_seq, int B, int H, int Hkv, float scale,
                                         int total_chunks, void *workspace, uint16_t *out, void *stream) {
  int rc = decode_attn_contract(B, H, Hkv, max_pages, total_chunks, "paged_decode_attn_qkv");
  if (rc) return rc;
  if (B == 0 || total_chunks == 0) return JIT_OK;
  if (!qkv || !q_norm_w || !k_norm_w || !inv_freq || !pool || !page_table || !lens || !chunk_start || !chunk_seq ||
      !workspace || !out)
    return jit::fail(JIT_EINVAL, "paged_decode_attn_qkv: null pointer");
  const FusedQkv fq{qkv, q_norm_w, k_norm_w, inv_freq, eps};
  return decode_attn_launch(nullptr, pool, page_table, max_pages, lens, chunk_start, chunk_seq, B, H, Hkv, scale,
                            total_chunks, workspace, out, (hipStream_t)stream, "jit_paged_decode_attn_qkv", &fq);
}

extern "C" int jit_paged_decode_attn_noalloc(const uint16_t *q, const uint16_t *pool, const int32_t *page_table,
                                             int max_pages, const int32_t *lens, const int32_t *chunk_start,
                                             const int32_t *chunk_seq, int B, int H, int Hkv, float scale,
                                             int total_chunks, uint16_t *out, void *stream) {
  int rc = decode_attn_contract(B, H, Hkv, max_pages, total_chunks, "paged_decode_attn_noalloc");
  if (rc) return rc;
  const int64_t need = jit_attn_workspace_bytes(total_chunks, H);
  if (need > (int64_t)JIT_ATTN_SCRATCH_BYTES)
    return jit::fail(JIT_EUNSUPPORTED,
                     "paged_decode_attn_noalloc: %d chunks x %d heads need %lld bytes of partials, past the "
                     "%d-byte scratch (use jit_paged_decode_attn with a workspace)",
                     total_chunks, H, (long long)need, (int)JIT_ATTN_SCRATCH_BYTES);
  if (B == 0 || total_chunks == 0) return JIT_OK;
  if (!q || !pool || !page_table || !lens || !chunk_start || !chunk_seq || !out)
    return jit::fail(JIT_EINVAL, "paged_decode_attn_noalloc: null pointer");
  void *ws = nullptr;
  rc = scratch_of_current_device(&ws, "paged_decode_attn_noalloc");
  if (rc) return rc;
  return decode_attn_launch(q, pool, page_table, max_pages, lens, chunk_start, chunk_seq, B, H, Hkv, scale,
                            total_chunks, ws, out, (hipStream_t)stream, "jit_paged_decode_attn_noalloc");
}

#if JIT_ATTN_STAMPS
// The stamps of the last decode-attention launch (bench.py --attn-phases).
extern "C" int jit_attn_stamps_clear(void *stream) {
  void *p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_attn_stamps)) != hipSuccess) return JIT_ELAUNCH;
  return hipMemsetAsync(p, 0, sizeof(g_attn_stamps), (hipStream_t)stream) == hipSuccess ? 0 : JIT_ELAUNCH;
}
extern "C" int jit_attn_stamps_read(uint64_t *host, int slots) {
  if (!host || slots < 0 || slots > kAttnStampSlots) return JIT_EINVAL;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_attn_stamps), (size_t)slots * 8 * sizeof(uint64_t), 0,
                             hipMemcpyDeviceToHost) == hipSuccess ? 0 : JIT_ELAUNCH;
}
#endif
