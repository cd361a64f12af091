// Router top-k and token-to-expert packing for gfx950.
//
// Compiled with -ffp-contract=off: the softmax must produce the same fp32 bits
// as the CPU restatement, because the expert indices derived from it are
// compared bit for bit.  Every floating-point step below is a single IEEE
// operation (add, multiply, divide, fused multiply-add, round-to-integer) in a
// fixed order.
#pragma clang fp contract(off)

#include "common.hpp"
#include "fmath.hpp"
#include "route.hpp"

namespace {

using fmath::exp_neg;
using route::key_bf16;
using route::order_key;
using route::row_keys;
using route::wave_max_u32;

constexpr int kRowsPerBlock = 4;  // one wave64 per token row
constexpr int kMaxN = 1024;

// One wave per row.  Lane l owns experts l, l+64, ...: it sums their exps in that
// order, the wave adds the 64 partial sums by a butterfly over offsets 32..1
// (every lane ends with the same total), then every gate is e_i * (1 / total)
// rounded to bf16.  The top-k is the rank rule of the reference: the rank of
// gate i counts the gates below it, ties broken by index, and ranks >= N-k fill
// slots rank-(N-k) in ascending (value, index) order.  The wave finds them as k
// rounds of a maximum over (value, index) keys, round t filling slot k-1-t -- the
// same slots the ranks give, with no pairwise comparison.
// One row on one wave: softmax (unless FROM_GATES) and the top-k slots, written to
// inds / scores.  `skey` is the wave's LDS scratch of k entries.
template <int NPL, bool FROM_GATES>
__device__ __forceinline__ void topk_row(const uint16_t *__restrict__ lg, int row, int N, int k, int norm,
                                         uint32_t *__restrict__ inds, uint16_t *__restrict__ scores,
                                         uint16_t *__restrict__ gates_out, uint32_t *skey, int l) {
  uint32_t key[NPL];
  row_keys<NPL, FROM_GATES>(lg, row, N, l, key, gates_out);
  if (k <= 64) {  // (uniform) slot j's key stays in lane j: no LDS round trip per slot
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
    const float tot = scores != nullptr ? route::slots_total(mine, k) : 0.0f;
    if (l < k) {
      inds[(size_t)row * k + l] = mine & 0xffffu;
      if (scores != nullptr) {
        const float sc = bf2f(key_bf16(mine));
        scores[(size_t)row * k + l] = (uint16_t)(norm ? f2bf(sc / tot) : f2bf(sc));
      }
    }
    return;
  }
  // every valid key is > 0 (its value field is >= 0x007f); a taken key becomes 0
  for (int t = 0; t < k; t++) {
    uint32_t m = key[0];
#pragma unroll
    for (int j = 1; j < NPL; j++) m = key[j] > m ? key[j] : m;
    m = wave_max_u32(m);
#pragma unroll
    for (int j = 0; j < NPL; j++) key[j] = key[j] == m ? 0u : key[j];
    if (l == 0) skey[k - 1 - t] = m;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float tot = 0.0f;
  if (scores != nullptr)
    for (int j = 0; j < k; j++) tot = bf2f(f2bf(tot + bf2f(key_bf16(skey[j]))));
  for (int j = l; j < k; j += 64) {
    const uint32_t m = skey[j];
    inds[(size_t)row * k + j] = m & 0xffffu;
    if (scores != nullptr) {
      const float sc = bf2f(key_bf16(m));
      scores[(size_t)row * k + j] = (uint16_t)(norm ? f2bf(sc / tot) : f2bf(sc));
    }
  }
}

template <int NPL, bool FROM_GATES>
__global__ __launch_bounds__(256) void router_topk_kernel(const uint16_t *__restrict__ src, int rows,
                                                          int N, int k, int norm,
                                                          uint32_t *__restrict__ inds,
                                                          uint16_t *__restrict__ scores,
                                                          uint16_t *__restrict__ gates_out) {
  __shared__ uint32_t skey[kRowsPerBlock][kMaxN];
  const int w = threadIdx.x >> 6, l = lane_id();
  const int row = blockIdx.x * kRowsPerBlock + w;
  if (row >= rows) return;  // the whole wave: row is uniform
  topk_row<NPL, FROM_GATES>(src + (size_t)row * N, row, N, k, norm, inds, scores, gates_out, skey[w], l);
}

template <bool FROM_GATES>
int launch_router(const uint16_t *src, int rows, int N, int k, int norm, uint32_t *inds,
                  uint16_t *scores, uint16_t *gates_out, hipStream_t st) {
  const dim3 grid((rows + kRowsPerBlock - 1) / kRowsPerBlock), block(256);
  const int npl = (N + 63) / 64;
  if (npl <= 1)
    router_topk_kernel<1, FROM_GATES><<<grid, block, 0, st>>>(src, rows, N, k, norm, inds, scores, gates_out);
  else if (npl <= 2)
    router_topk_kernel<2, FROM_GATES><<<grid, block, 0, st>>>(src, rows, N, k, norm, inds, scores, gates_out);
  else if (npl <= 4)
    router_topk_kernel<4, FROM_GATES><<<grid, block, 0, st>>>(src, rows, N, k, norm, inds, scores, gates_out);
  else if (npl <= 8)
    router_topk_kernel<8, FROM_GATES><<<grid, block, 0, st>>>(src, rows, N, k, norm, inds, scores, gates_out);
  else
    router_topk_kernel<16, FROM_GATES><<<grid, block, 0, st>>>(src, rows, N, k, norm, inds, scores, gates_out);
  return jit::check_launch(FROM_GATES ? "jit_topk" : "jit_router_topk");
}

// --------------------------------------------------------------- packing
constexpr int kPackThreads = 1024;  // the largest workgroup (and expert count) of the packing

__device__ __forceinline__ int wave_incl_scan(int x, int l) {
  // within each 16-lane row by row shifts 1, 2, 4, 8 (lanes past a row's start add 0), then the
  // rows' totals (integers: any order gives the same sums)
#define JIT_SCAN_STEP(ctrl) x += __builtin_amdgcn_update_dpp(0, x, ctrl, 0xF, 0xF, true)
  JIT_SCAN_STEP(0x111);
  JIT_SCAN_STEP(0x112);
  JIT_SCAN_STEP(0x114);
  JIT_SCAN_STEP(0x118);
#undef JIT_SCAN_STEP
  const int t0 = __builtin_amdgcn_readlane(x, 15), t1 = __builtin_amdgcn_readlane(x, 31);
  const int t2 = __builtin_amdgcn_readlane(x, 47);
  const int row = l >> 4;
  return x + (row >= 1 ? t0 : 0) + (row >= 2 ? t1 : 0) + (row >= 3 ? t2 : 0);
}

// The per-expert tables from each expert's pair count c (thread t: expert t, t < E; threads past
// E pass c = 0): counts, first sorted positions, the ascending list of non-empty experts (their
// segments) and meta = (segments, largest segment, bad pairs, 0).  nxt[t] receives expert t's
// first position.  One workgroup of TH >= E threads.
template <int TH>
__device__ __forceinline__ void pack_tables(int c, int bad, int E, int *nxt, int32_t *__restrict__ expert_cnt,
                                            int32_t *__restrict__ expert_off, int32_t *__restrict__ seg_expert,
                                            int32_t *__restrict__ seg_start, int32_t *__restrict__ seg_cnt,
                                            int32_t *__restrict__ meta) {
  __shared__ int wsum[(TH / 64)], wflag[(TH / 64)], wmax[(TH / 64)];
  const int t = threadIdx.x, w = t >> 6, l = t & 63;
  const int f = c > 0 ? 1 : 0;
  const int cs = wave_incl_scan(c, l);
  const int fs = wave_incl_scan(f, l);
  int mx = c;
  mx = (int)wave_max_u32((uint32_t)mx);  // (counts are >= 0)
  if (l == 63) {
    wsum[w] = cs;
    wflag[w] = fs;
    wmax[w] = mx;
  }
  __syncthreads();
  int cbase = 0, fbase = 0, tot_f = 0, tot_m = 0;
  for (int ww = 0; ww < (TH / 64); ww++) {
    if (ww < w) {
      cbase += wsum[ww];
      fbase += wflag[ww];
    }
    tot_f += wflag[ww];
    tot_m = max(tot_m, wmax[ww]);
  }
  const int off = cbase + cs - c;
  nxt[t] = off;
  if (t < E) {
    expert_cnt[t] = c;
    expert_off[t] = off;
    if (f) {
      const int u = fbase + fs - 1;
      seg_expert[u] = t;
      seg_start[u] = off;
      seg_cnt[u] = c;
    }
  }
  if (t == 0) {
    meta[0] = tot_f;
    meta[1] = tot_m;
    meta[2] = bad;
    meta[3] = 0;
  }
}

// Placement of the pairs base .. base + TH - 1 (flat order) at their sorted positions, given each
// expert's next free position in nxt (advanced past the tile's pairs on return): within a wave,
// lanes holding the same expert id find each other with ballots over the id's bits, so a pair's
// position is its expert's running offset plus the pairs of that expert in earlier waves of the
// tile plus its rank among its own wave's lanes -- a stable counting sort.  A pair with an id
// past E gets inv = -1 and no position.
template <int TH, typename IndFn>
__device__ __forceinline__ void pack_place_tile(IndFn ind, int base, int P, int k, int E, int *nxt,
                                                unsigned short (*wcnt)[TH], int32_t *__restrict__ order,
                                                int32_t *__restrict__ pair_row, int32_t *__restrict__ inv) {
  const int t = threadIdx.x, w = t >> 6, l = t & 63;
  const int nbits = 32 - __clz(E);  // enough bits for ids 0..E (E = "no expert")
  const int p = base + t;
  uint32_t e = p < P ? ind(p) : (uint32_t)E;
  if (e > (uint32_t)E) e = (uint32_t)E;
  unsigned long long m = ~0ull;
  for (int bt = 0; bt < nbits; bt++) {
    const int bit = (e >> bt) & 1u;
    const unsigned long long bal = __ballot(bit);
    m &= bit ? bal : ~bal;
  }
  const int rank = __popcll(m & ((1ull << l) - 1ull));
  const int total = __popcll(m);
  for (int idx = t; idx < (TH / 64) * E; idx += TH) wcnt[idx / E][idx % E] = 0;
  __syncthreads();
  if (e < (uint32_t)E && rank == total - 1) wcnt[w][e] = (unsigned short)total;
  __syncthreads();
  if (e < (uint32_t)E) {
    int pos = nxt[e] + rank;
    for (int ww = 0; ww < w; ww++) pos += wcnt[ww][e];
    order[pos] = p;
    pair_row[pos] = p / k;
    inv[p] = pos;
  } else if (p < P) {
    inv[p] = -1;
  }
  __syncthreads();
  if (t < E) {
    int s = 0;
    for (int ww = 0; ww < (TH / 64); ww++) s += wcnt[ww][t];
    nxt[t] += s;
  }
  __syncthreads();
}

// The packing, run by one workgroup of TH threads (TH >= E): (1) per-expert counts in LDS; (2)
// the tables; (3) the pairs placed in tiles of TH in flat order.  ind(p) is flat pair p's expert id.
template <int TH, typename IndFn>
__device__ __forceinline__ void pack_body(IndFn ind, int P, int k, int E, int32_t *__restrict__ order,
                                          int32_t *__restrict__ pair_row, int32_t *__restrict__ inv,
                                          int32_t *__restrict__ expert_cnt, int32_t *__restrict__ expert_off,
                                          int32_t *__restrict__ seg_expert, int32_t *__restrict__ seg_start,
                                          int32_t *__restrict__ seg_cnt, int32_t *__restrict__ meta) {
  __shared__ int cnt[TH];
  __shared__ int nxt[TH];
  __shared__ unsigned short wcnt[(TH / 64)][TH];
  __shared__ int bad;
  const int t = threadIdx.x;
  cnt[t] = 0;
  if (t == 0) bad = 0;
  __syncthreads();
  for (int p = t; p < P; p += TH) {
    const uint32_t e = ind(p);
    if (e < (uint32_t)E)
      atomicAdd(&cnt[e], 1);
    else
      atomicAdd(&bad, 1);
  }
  __syncthreads();
  pack_tables<TH>(cnt[t], bad, E, nxt, expert_cnt, expert_off, seg_expert, seg_start, seg_cnt, meta);
  for (int base = 0; base < P; base += TH)
    pack_place_tile<TH>(ind, base, P, k, E, nxt, wcnt, order, pair_row, inv);
}

// The packing of a long batch over many workgroups (the one-workgroup kernel walks its tiles one
// after another), in three launches over a workspace of per-tile counts ws[tiles][E + 1] (slot E:
// the tile's bad pairs), tiles of kPackThreads pairs:
//   pack_count_kernel: each tile's expert counts;
//   pack_scan_kernel (one workgroup): each expert's total, the tables, and in ws each tile's
//     pairs of each expert before it (the tile's offset within the expert's segment);
//   pack_place_kernel: each tile placed from its experts' first positions plus those offsets.
// The result is the stable order (expert, flat index) itself, so the same tables as the one
// workgroup's, bit for bit.
__global__ __launch_bounds__(kPackThreads) void pack_count_kernel(const uint32_t *__restrict__ inds, int P, int E,
                                                                  int32_t *__restrict__ ws) {
  __shared__ int cnt[kPackThreads + 1];
  const int t = threadIdx.x, tile = blockIdx.x;
  for (int e = t; e <= E; e += kPackThreads) cnt[e] = 0;
  __syncthreads();
  const int p = tile * kPackThreads + t;
  if (p < P) {
    const uint32_t e = inds[p];
    atomicAdd(&cnt[e < (uint32_t)E ? e : (uint32_t)E], 1);
  }
  __syncthreads();
  for (int e = t; e <= E; e += kPackThreads) ws[(long long)tile * (E + 1) + e] = cnt[e];
}

template <int TH>
__global__ __launch_bounds__(TH) void pack_scan_kernel(int tiles, int E, int32_t *__restrict__ ws,
                                                       int32_t *__restrict__ expert_cnt, int32_t *__restrict__ expert_off,
                                                       int32_t *__restrict__ seg_expert, int32_t *__restrict__ seg_start,
                                                       int32_t *__restrict__ seg_cnt, int32_t *__restrict__ meta) {
  __shared__ int nxt[TH];
  const int t = threadIdx.x;
  int run = 0;
  if (t <= E) {  // experts, and slot E (the bad pairs)
    // the tiles' counts in batches whose loads are all issued before the first store (a store
    // between them would order each load behind the previous one's round trip)
    constexpr int kBatch = 16;
    for (int i0 = 0; i0 < tiles; i0 += kBatch) {
      int v[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; j++) v[j] = i0 + j < tiles ? ws[(long long)(i0 + j) * (E + 1) + t] : 0;
#pragma unroll
      for (int j = 0; j < kBatch; j++)
        if (i0 + j < tiles) {
          ws[(long long)(i0 + j) * (E + 1) + t] = run;
          run += v[j];
        }
    }
  }
  __shared__ int bad;
  if (t == E) bad = run;
  __syncthreads();
  pack_tables<TH>(t < E ? run : 0, bad, E, nxt, expert_cnt, expert_off, seg_expert, seg_start, seg_cnt, meta);
}

__global__ __launch_bounds__(kPackThreads) void pack_place_kernel(const uint32_t *__restrict__ inds, int P, int k,
                                                                  int E, const int32_t *__restrict__ ws,
                                                                  const int32_t *__restrict__ expert_off,
                                                                  int32_t *__restrict__ order,
                                                                  int32_t *__restrict__ pair_row,
                                                                  int32_t *__restrict__ inv) {
  __shared__ int nxt[kPackThreads];
  __shared__ unsigned short wcnt[kPackThreads / 64][kPackThreads];
  const int t = threadIdx.x, tile = blockIdx.x;
  for (int e = t; e < E; e += kPackThreads) nxt[e] = expert_off[e] + ws[(long long)tile * (E + 1) + e];
  __syncthreads();
  pack_place_tile<kPackThreads>([&](int p) { return inds[p]; }, tile * kPackThreads, P, k, E, nxt, wcnt, order,
                                pair_row, inv);
}

template <int TH>
__global__ __launch_bounds__(TH) void moe_pack_kernel(
    const uint32_t *__restrict__ inds, int P, int k, int E, int32_t *__restrict__ order,
    int32_t *__restrict__ pair_row, int32_t *__restrict__ inv, int32_t *__restrict__ expert_cnt,
    int32_t *__restrict__ expert_off, int32_t *__restrict__ seg_expert,
    int32_t *__restrict__ seg_start, int32_t *__restrict__ seg_cnt, int32_t *__restrict__ meta) {
  pack_body<TH>([&](int p) { return inds[p]; }, P, k, E, order, pair_row, inv, expert_cnt, expert_off, seg_expert,
            seg_start, seg_cnt, meta);
}

// Top-k of a few rows and their packing in one launch (a decode step of at most
// kRoutePackRows rows, e.g. one sequence): the same topk_row and pack_body as the two
// kernels above, so the same bits, one launch fewer.  Two waves take the rows in turn;
// the packing reads the indices they wrote after the workgroup barrier.
constexpr int kRoutePackRows = 4;

template <int NPL>
__global__ __launch_bounds__(128) void route_pack_kernel(
    const uint16_t *__restrict__ logits, int rows, int N, int k, int norm, uint32_t *__restrict__ inds,
    uint16_t *__restrict__ scores, int32_t *__restrict__ order, int32_t *__restrict__ pair_row,
    int32_t *__restrict__ inv, int32_t *__restrict__ expert_cnt, int32_t *__restrict__ expert_off,
    int32_t *__restrict__ seg_expert, int32_t *__restrict__ seg_start, int32_t *__restrict__ seg_cnt,
    int32_t *__restrict__ meta) {
  __shared__ uint32_t skey[2][kMaxN];
  const int w = threadIdx.x >> 6, l = lane_id();
  for (int row = w; row < rows; row += 2)
    topk_row<NPL, false>(logits + (size_t)row * N, row, N, k, norm, inds, scores, nullptr, skey[w], l);
  __syncthreads();
  pack_body<128>([&](int p) { return inds[p]; }, rows * k, k, N, order, pair_row, inv, expert_cnt, expert_off,
                 seg_expert, seg_start, seg_cnt, meta);
}

}  // namespace

extern "C" int jit_route_pack(const uint16_t *logits, int rows, int N, int k, int norm, uint32_t *inds,
                              uint16_t *scores, int32_t *order, int32_t *pair_row, int32_t *inv,
                              int32_t *expert_cnt, int32_t *expert_off, int32_t *seg_expert, int32_t *seg_start,
                              int32_t *seg_cnt, int32_t *meta, void *stream) {
  if (rows < 0 || N <= 0 || !(0 < k && k <= N))
    return jit::fail(JIT_EINVAL, "route_pack takes rows >= 0 and 0 < k <= N, got rows=%d N=%d k=%d", rows, N, k);
  if (rows > kRoutePackRows || N % 32 != 0 || N > 128)
    return jit::fail(JIT_EUNSUPPORTED, "route_pack covers rows <= %d and N %% 32 == 0, N <= 128, got rows=%d N=%d",
                     kRoutePackRows, rows, N);
  if (!expert_cnt || !expert_off || !seg_expert || !seg_start || !seg_cnt || !meta)
    return jit::fail(JIT_EINVAL, "route_pack: null pointer");
  if (rows > 0 && (!logits || !inds || !scores || !order || !pair_row || !inv))
    return jit::fail(JIT_EINVAL, "route_pack: null pointer");
  const hipStream_t st = (hipStream_t)stream;
  if (N <= 64)
    route_pack_kernel<1><<<1, 128, 0, st>>>(logits, rows, N, k, norm, inds, scores, order, pair_row, inv, expert_cnt,
                                           expert_off, seg_expert, seg_start, seg_cnt, meta);
  else
    route_pack_kernel<2><<<1, 128, 0, st>>>(logits, rows, N, k, norm, inds, scores, order, pair_row, inv, expert_cnt,
                                           expert_off, seg_expert, seg_start, seg_cnt, meta);
  return jit::check_launch("jit_route_pack");
}

extern "C" int jit_router_topk(const uint16_t *logits, int rows, int N, int k, int norm,
                               uint32_t *inds, uint16_t *scores, uint16_t *gates_out,
                               void *stream) {
  if (rows < 0 || N <= 0 || !(0 < k && k <= N))
    return jit::fail(JIT_EINVAL, "router_topk takes rows >= 0 and 0 < k <= N, got rows=%d N=%d k=%d",
                     rows, N, k);
  if (N % 32 != 0 || N > kMaxN)
    return jit::fail(JIT_EUNSUPPORTED, "router_topk covers N %% 32 == 0 and N <= %d, got N=%d", kMaxN, N);
  if (rows == 0) return JIT_OK;
  if (!logits || !inds || !scores) return jit::fail(JIT_EINVAL, "router_topk: null pointer");
  return launch_router<false>(logits, rows, N, k, norm, inds, scores, gates_out, (hipStream_t)stream);
}

extern "C" int jit_topk(const uint16_t *gates, int rows, int N, int k, uint32_t *inds, void *stream) {
  if (rows < 0 || N <= 0 || !(0 < k && k <= N))
    return jit::fail(JIT_EINVAL, "top-k takes 0 < k <= %d gates, not k = %d", N, k);
  if (N > kMaxN) return jit::fail(JIT_EUNSUPPORTED, "topk covers N <= %d, got N=%d", kMaxN, N);
  if (rows == 0) return JIT_OK;
  if (!gates || !inds) return jit::fail(JIT_EINVAL, "topk: null pointer");
  return launch_router<true>(gates, rows, N, k, 0, inds, nullptr, nullptr, (hipStream_t)stream);
}

extern "C" int jit_moe_pack(const uint32_t *inds, int P, int k, int E, int32_t *order,
                            int32_t *pair_row, int32_t *inv, int32_t *expert_cnt,
                            int32_t *expert_off, int32_t *seg_expert, int32_t *seg_start,
                            int32_t *seg_cnt, int32_t *meta, void *stream) {
  if (P < 0 || k <= 0 || E <= 0 || P % k != 0)
    return jit::fail(JIT_EINVAL, "moe_pack takes P >= 0 pairs in rows of k > 0 and E > 0, got P=%d k=%d E=%d",
                     P, k, E);
  if (E > kPackThreads) return jit::fail(JIT_EUNSUPPORTED, "moe_pack covers E <= %d, got %d", kPackThreads, E);
  if (!expert_cnt || !expert_off || !seg_expert || !seg_start || !seg_cnt || !meta)
    return jit::fail(JIT_EINVAL, "moe_pack: null pointer");
  if (P > 0 && (!inds || !order || !pair_row || !inv)) return jit::fail(JIT_EINVAL, "moe_pack: null pointer");
  // a decode batch's few pairs take the smallest workgroup that owns every expert (fewer waves
  // at each of the placement's barriers), and more than 128 pairs 256 threads (fewer tiles, each
  // behind the same barriers: config 2's 256 pairs over 128 experts 3.90 -> 3.17 us); long batches
  // take 1024 threads a tile
  const hipStream_t st = (hipStream_t)stream;
#define JIT_PACK(TH) moe_pack_kernel<TH><<<1, TH, 0, st>>>(inds, P, k, E, order, pair_row, inv, expert_cnt, \
                                                           expert_off, seg_expert, seg_start, seg_cnt, meta)
  if (P <= 128 && E <= 128)
    JIT_PACK(128);
  else if (P <= 2048 && E <= 256)
    JIT_PACK(256);
  else
    JIT_PACK(1024);
#undef JIT_PACK
  return jit::check_launch("jit_moe_pack");
}

// Long batches take the three-launch packing over a workspace of per-tile counts.
static bool pack_multi(int P, int E) { return P > 2 * kPackThreads && E < kPackThreads; }

extern "C" long long jit_moe_pack_workspace_bytes(int P, int E) {
  if (P <= 0 || E <= 0 || !pack_multi(P, E)) return 0;
  return (long long)((P + kPackThreads - 1) / kPackThreads) * (E + 1) * (long long)sizeof(int32_t);
}

extern "C" int jit_moe_pack_ws(const uint32_t *inds, int P, int k, int E, int32_t *order, int32_t *pair_row,
                               int32_t *inv, int32_t *expert_cnt, int32_t *expert_off, int32_t *seg_expert,
                               int32_t *seg_start, int32_t *seg_cnt, int32_t *meta, void *workspace,
                               long long workspace_bytes, void *stream) {
  const long long need = jit_moe_pack_workspace_bytes(P, E);
  if (need == 0)
    return jit_moe_pack(inds, P, k, E, order, pair_row, inv, expert_cnt, expert_off, seg_expert, seg_start, seg_cnt,
                        meta, stream);
  if (k <= 0 || P % k != 0)
    return jit::fail(JIT_EINVAL, "moe_pack takes P >= 0 pairs in rows of k > 0 and E > 0, got P=%d k=%d E=%d",
                     P, k, E);
  if (!inds || !order || !pair_row || !inv || !expert_cnt || !expert_off || !seg_expert || !seg_start ||
      !seg_cnt || !meta)
    return jit::fail(JIT_EINVAL, "moe_pack: null pointer");
  if (!workspace || workspace_bytes < need)
    return jit::fail(JIT_EINVAL, "moe_pack: workspace of %lld bytes, %lld needed", workspace_bytes, need);
  const hipStream_t st = (hipStream_t)stream;
  const int tiles = (P + kPackThreads - 1) / kPackThreads;
  int32_t *ws = (int32_t *)workspace;
  pack_count_kernel<<<tiles, kPackThreads, 0, st>>>(inds, P, E, ws);
  pack_scan_kernel<kPackThreads><<<1, kPackThreads, 0, st>>>(tiles, E, ws, expert_cnt, expert_off, seg_expert,
                                                             seg_start, seg_cnt, meta);
  pack_place_kernel<<<tiles, kPackThreads, 0, st>>>(inds, P, k, E, ws, expert_off, order, pair_row, inv);
  return jit::check_launch("jit_moe_pack_ws");
}
