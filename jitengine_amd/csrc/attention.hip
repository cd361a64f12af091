// Paged KV pool append and split-K paged GQA decode attention for gfx950.
//
// Pool page (one layer): [2][Hkv][16 * 128] bf16 -- K slot-major ([slot][d],
// 4 KiB per kv head), V dim-major ([d][slot], 4 KiB per kv head).
//
// Attention work item: one workgroup per (chunk of one sequence, kv head); its 4
// waves split the chunk's pages and each streams 2 pages (32 keys) per step:
//   S^T[16 keys x 16 q heads] = K_page . Q^T     (4 MFMA 16x16x32 per page; the
//        K page feeds the A operand directly: lane = slot, 16 B of d per MFMA)
//   online softmax in the exp2 domain (fp32 running max / sum per q head)
//   O[16 q heads x 128 d] += P . V               (8 MFMA 16x16x32 per 2 pages; the
//        V page's dim-major rows feed the B operand with 8-byte loads)
// so each K/V byte is read once for all G = H / Hkv query heads of its kv head
// (G <= 16; rows G..15 of the tiles are padding).  The waves merge in LDS; a
// sequence of one chunk writes its output directly, longer ones write fp32
// (max, sum, o[128]) partials that attn_merge_kernel combines in chunk order.
#include "common.hpp"

namespace {

constexpr int kD = JIT_HEAD_DIM;      // 128
constexpr int kPage = JIT_PAGE_TOKENS;  // 16
constexpr int kPageHead = kPage * kD;   // bf16 elements of one (page, part, kv head)

}  // namespace

// Chunk length rule: a pure function of the sequence's own length (so results
// do not depend on the batch), 256 keys up to 16K tokens, 512 beyond.
extern "C" int jit_attn_chunk_tokens(int len) { return len <= 16384 ? 256 : 512; }

__device__ __forceinline__ int chunk_tokens_dev(int len) { return len <= 16384 ? 256 : 512; }

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
    pool[((long long)page * 2 * Hkv + h) * kPageHead + slot * kD + d] = k[src];
    pool[(((long long)page * 2 + 1) * Hkv + h) * kPageHead + d * kPage + slot] = v[src];
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
};

__global__ __launch_bounds__(256) void paged_attn_kernel(const AttnArgs a) {
  __shared__ float sm[4][16], sl[4][16];
  __shared__ float so[4][16][kD];
  const int gc = blockIdx.x, kvh = blockIdx.y;
  const int b = a.chunk_seq[gc];
  const int L = a.lens[b];
  const int CK = chunk_tokens_dev(L);
  const int c = gc - a.chunk_start[b];
  const int nchunks = (L + CK - 1) / CK;
  const int wave = threadIdx.x >> 6, l = lane_id();
  const int lr = l & 15, lg = l >> 4;
  const int G = a.G;
  const int per_wave = CK / 4;
  const int wk0 = c * CK + wave * per_wave;
  const int wk1 = min(wk0 + per_wave, L);
  const int32_t *prow = a.page_table + (long long)b * a.max_pages;
  const long long part_stride = (long long)2 * a.Hkv * kPageHead;  // bf16 per page

  Frag8 qf[4];
  if (lr < G) {
    const uint16_t *qp = a.q + ((long long)b * a.H + kvh * G + lr) * kD + 8 * lg;
#pragma unroll
    for (int cc = 0; cc < 4; cc++) qf[cc].q = *(const uint4 *)(qp + 32 * cc);
  } else {
#pragma unroll
    for (int cc = 0; cc < 4; cc++) qf[cc].q = make_uint4(0, 0, 0, 0);
  }
  float m_run = -INFINITY, l_run = 0.0f;
  f32x4 o[8];
#pragma unroll
  for (int cc = 0; cc < 8; cc++) o[cc] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = wk0; k0 < wk1; k0 += 32) {
    const bool has1 = k0 + 16 < wk1;
    const int pg0 = prow[k0 >> 4];
    const int pg1 = has1 ? prow[(k0 >> 4) + 1] : pg0;
    const uint16_t *kp0 = a.pool + (long long)pg0 * part_stride + (long long)kvh * kPageHead;
    const uint16_t *kp1 = a.pool + (long long)pg1 * part_stride + (long long)kvh * kPageHead;
    const uint16_t *vp0 = kp0 + (long long)a.Hkv * kPageHead;
    const uint16_t *vp1 = kp1 + (long long)a.Hkv * kPageHead;
    Frag8 kf0[4], kf1[4];
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
      kf0[cc].q = *(const uint4 *)(kp0 + lr * kD + 32 * cc + 8 * lg);
      kf1[cc].q = has1 ? *(const uint4 *)(kp1 + lr * kD + 32 * cc + 8 * lg) : make_uint4(0, 0, 0, 0);
    }
    uint2 va[8], vb[8];
#pragma unroll
    for (int cc = 0; cc < 8; cc++) {
      va[cc] = *(const uint2 *)(vp0 + (16 * cc + lr) * kPage + 4 * lg);
      vb[cc] = has1 ? *(const uint2 *)(vp1 + (16 * cc + lr) * kPage + 4 * lg) : make_uint2(0, 0);
    }
    f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
      s0 = mfma16x16x32(kf0[cc], qf[cc], s0);
      s1 = mfma16x16x32(kf1[cc], qf[cc], s1);
    }
    // lane holds S^T[key 4*lg + i][head lr] of both pages
    float p0[4], p1[4], tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int key0 = k0 + 4 * lg + i, key1 = key0 + 16;
      p0[i] = key0 < wk1 ? s0[i] * a.qk_scale : -INFINITY;
      p1[i] = key1 < wk1 ? s1[i] * a.qk_scale : -INFINITY;
      tmax = fmaxf(tmax, fmaxf(p0[i], p1[i]));
    }
    tmax = fmaxf(tmax, shfl_xor_f(tmax, 16));
    tmax = fmaxf(tmax, shfl_xor_f(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      p0[i] = exp2f(p0[i] - m_new);
      p1[i] = exp2f(p1[i] - m_new);
      psum += p0[i] + p1[i];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    Frag8 pf;
    if (lr < G) {
      pf.u[0] = pack_bf16x2(p0[0], p0[1]);
      pf.u[1] = pack_bf16x2(p0[2], p0[3]);
      pf.u[2] = pack_bf16x2(p1[0], p1[1]);
      pf.u[3] = pack_bf16x2(p1[2], p1[3]);
    } else {
      pf.q = make_uint4(0, 0, 0, 0);
    }
    // the tail page may hold stale slots past L: their p is 0, make their V 0 too
    if (k0 + 32 > L) {
#pragma unroll
      for (int cc = 0; cc < 8; cc++) {
        const int kb0 = k0 + 4 * lg, kb1 = kb0 + 16;
        va[cc].x = (kb0 + 0 < L ? (va[cc].x & 0xffffu) : 0u) | (kb0 + 1 < L ? (va[cc].x & 0xffff0000u) : 0u);
        va[cc].y = (kb0 + 2 < L ? (va[cc].y & 0xffffu) : 0u) | (kb0 + 3 < L ? (va[cc].y & 0xffff0000u) : 0u);
        vb[cc].x = (kb1 + 0 < L ? (vb[cc].x & 0xffffu) : 0u) | (kb1 + 1 < L ? (vb[cc].x & 0xffff0000u) : 0u);
        vb[cc].y = (kb1 + 2 < L ? (vb[cc].y & 0xffffu) : 0u) | (kb1 + 3 < L ? (vb[cc].y & 0xffff0000u) : 0u);
      }
    }
    // O rows are q heads 4*lg + i: fetch their rescale factors from the lanes
    // that own those heads in the score layout
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; i++) al[i] = shfl_f(alpha, 4 * lg + i);
#pragma unroll
    for (int cc = 0; cc < 8; cc++) {
      Frag8 vf;
      vf.u[0] = va[cc].x;
      vf.u[1] = va[cc].y;
      vf.u[2] = vb[cc].x;
      vf.u[3] = vb[cc].y;
#pragma unroll
      for (int i = 0; i < 4; i++) o[cc][i] *= al[i];
      o[cc] = mfma16x16x32(pf, vf, o[cc]);
    }
  }
  float l_tot = l_run + shfl_xor_f(l_run, 16);
  l_tot = l_tot + shfl_xor_f(l_tot, 32);
  if (lg == 0) {
    sm[wave][lr] = m_run;
    sl[wave][lr] = l_tot;
  }
#pragma unroll
  for (int cc = 0; cc < 8; cc++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int hh = 4 * lg + i;
      if (hh < G) so[wave][hh][16 * cc + lr] = o[cc][i];
    }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * kD; idx += 256) {
    const int hh = idx / kD, d = idx % kD;
    float M = sm[0][hh];
#pragma unroll
    for (int w = 1; w < 4; w++) M = fmaxf(M, sm[w][hh]);
    float Ls = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float f = exp2f(sm[w][hh] - M);
      Ls += sl[w][hh] * f;
      O += so[w][hh][d] * f;
    }
    const int h = kvh * G + hh;
    if (nchunks == 1) {
      a.out[((long long)b * a.H + h) * kD + d] = (uint16_t)f2bf(O / Ls);
    } else {
      a.part_o[((long long)gc * a.H + h) * kD + d] = O;
      if (d == 0) {
        a.part_ml[((long long)gc * a.H + h) * 2 + 0] = M;
        a.part_ml[((long long)gc * a.H + h) * 2 + 1] = Ls;
      }
    }
  }
}

// Merge of a sequence's chunk partials in chunk order: one workgroup of 128
// threads (one per d) per (sequence, q head).
__global__ __launch_bounds__(128) void attn_merge_kernel(const int32_t *__restrict__ lens,
                                                         const int32_t *__restrict__ chunk_start,
                                                         const float *__restrict__ part_o,
                                                         const float *__restrict__ part_ml, int H,
                                                         uint16_t *__restrict__ out) {
  const int b = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int L = lens[b];
  const int CK = chunk_tokens_dev(L);
  const int n = (L + CK - 1) / CK;
  if (n <= 1) return;
  const long long c0 = chunk_start[b];
  float M = -INFINITY;
  for (int c = 0; c < n; c++) M = fmaxf(M, part_ml[((c0 + c) * H + h) * 2]);
  float Ls = 0.0f, O = 0.0f;
  for (int c = 0; c < n; c++) {
    const long long r = (c0 + c) * H + h;
    const float f = exp2f(part_ml[r * 2] - M);
    Ls += part_ml[r * 2 + 1] * f;
    O += part_o[r * kD + d] * f;
  }
  out[((long long)b * H + h) * kD + d] = (uint16_t)f2bf(O / Ls);
}

}  // namespace

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

extern "C" int jit_paged_decode_attn(const uint16_t *q, const uint16_t *pool,
                                     const int32_t *page_table, int max_pages, const int32_t *lens,
                                     const int32_t *chunk_start, const int32_t *chunk_seq, int B,
                                     int H, int Hkv, float scale, int total_chunks, void *workspace,
                                     uint16_t *out, void *stream) {
  if (B < 0 || H <= 0 || Hkv <= 0 || max_pages <= 0 || total_chunks < 0)
    return jit::fail(JIT_EINVAL, "paged_decode_attn: bad dims B=%d H=%d Hkv=%d", B, H, Hkv);
  if (H % Hkv != 0) return jit::fail(JIT_EINVAL, "%d query heads do not share %d KV heads evenly", H, Hkv);
  if (H / Hkv > 16) return jit::fail(JIT_EUNSUPPORTED, "paged_decode_attn covers H / Hkv <= 16, got %d", H / Hkv);
  if (B == 0 || total_chunks == 0) return JIT_OK;
  if (!q || !pool || !page_table || !lens || !chunk_start || !chunk_seq || !workspace || !out)
    return jit::fail(JIT_EINVAL, "paged_decode_attn: null pointer");
  float *part_o = (float *)workspace;
  float *part_ml = part_o + (long long)total_chunks * H * kD;
  AttnArgs a{q, pool, page_table, lens, chunk_start, chunk_seq, part_o, part_ml, out,
             max_pages, H, Hkv, H / Hkv, scale * 1.44269504088896341f};
  hipStream_t st = (hipStream_t)stream;
  paged_attn_kernel<<<dim3(total_chunks, Hkv), 256, 0, st>>>(a);
  int rc = jit::check_launch("jit_paged_decode_attn");
  if (rc) return rc;
  attn_merge_kernel<<<dim3(B, H), 128, 0, st>>>(lens, chunk_start, part_o, part_ml, H, out);
  return jit::check_launch("jit_paged_decode_attn merge");
}
