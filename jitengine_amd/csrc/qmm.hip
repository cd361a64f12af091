// 4-bit affine (MLX layout, group 64) quantized projections on gfx950 matrix
// cores, for dense projections and for expert segments of packed pairs.
//
// MFMA tile: v_mfma_f32_16x16x32_bf16 computes C[16 tokens x 16 weight rows],
// tokens on the M side (A operand = activations), weight rows on the N side
// (B operand = nibbles).  Each lane owns one weight row (l % 16) and, per quant
// group of 64 k, the two 32-bit words (16 nibbles) its lane group (l / 16) feeds
// into the group's two MFMAs -- every MFMA sees k values of a single group, so
// the group's scale and bias apply to the MFMA result, not to each weight:
//   sum_k x_k (s q_k + b) = s * sum_k x_k (q_k + 128) + (b - 128 s) * sum_k x_k.
// A nibble q becomes the bf16 value 128 + q with one AND-OR (bit pattern 0x43pq),
// and sum_k x_k comes from one more MFMA against an all-ones B operand, so the
// vector work per weight word is 7 integer ops.  Words are used in the packed
// nibble order (nibbles_natural below), whose unpacking yields k in natural order,
// so the activations are fed to the matrix cores as loaded.
//
// Work split: a workgroup owns 16 * NB output rows of one expert (or of the dense
// matrix) and splits K over its waves (KSPLIT = blockDim / 64); each wave owns
// GPW consecutive groups.  A wave issues every weight, scale and bias load of its
// K-slice before any math -- 9 KB in flight per wave for the gate||up shape (a
// 16-row gate block and its up block, 8 groups) -- and keeps the slice in
// registers while it walks the expert's token
// tiles of 16, so an expert's weights leave HBM once however many tokens it has.
// The waves' partial sums meet in LDS and are added in wave order (a fixed
// order: results do not depend on the batch).
#include "qtile.hpp"
#include "route.hpp"
#include "rowops.hpp"

namespace {

struct QmmArgs {
  const uint16_t *x;          // activations, row stride K (bf16)
  const int32_t *row_index;   // x row of each sorted position (gate||up; null: the position itself)
  const int32_t *cnt;         // pairs per expert (null: dense, T tokens)
  const int32_t *off;         // first sorted position per expert
  const uint32_t *w;          // weight stack [E, rows_w, K / 8]
  const uint16_t *s, *b;      // scales, biases [E, rows_w, K / 64]
  uint16_t *out;              // [positions, N] bf16
  int K, N, T;
  long long w_estride, g_estride;  // per expert: 32-bit words and bf16 entries (MLX layout), or
                                   // bytes of tiles (packed layout; g_estride unused)
  int rows_w;                      // weight rows per expert (2N with SWIGLU)
  int E;                           // experts of the stack (the grid may have fewer rows)
  // ROUTED (a one-token step routing itself): the token's router logits [E], top-k and renorm,
  // and the packing tables the launch writes for the later launches (down, combine)
  const uint16_t *logits;
  int k, norm;
  uint32_t *inds;
  uint16_t *scores;
  int32_t *order, *pair_row, *inv, *t_cnt, *t_off, *seg_expert, *seg_start, *seg_cnt, *meta;
  // PRO (a one-row dense projection that builds its own input row; x unused): 1 = bf16(pr_a +
  // pr_resid) then RMSNorm with pr_w (workgroup 0 writes the sum to pr_sum and the normed row to
  // pr_norm); 2 = the MoE combine of the expert outputs pr_a through pr_inv / pr_scores plus
  // pr_resid, then RMSNorm (workgroup 0 writes the combined row to pr_sum)
  const uint16_t *pr_a, *pr_resid, *pr_w, *pr_scores;
  const int32_t *pr_inv;
  int pr_k;
  float pr_eps;
  uint16_t *pr_sum, *pr_norm;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The wave's integer sum (exact, so the pairing does not matter), by VALU lane exchanges: the
// permlane swaps across rows, then DPP row rotations within each 16-lane row.
__device__ __forceinline__ int wave_sum_i(int v) {
  auto r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  v = (int)(r[0] + r[1]);
  r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  v = (int)(r[0] + r[1]);
  v += __builtin_amdgcn_update_dpp(v, v, 0x128, 0xF, 0xF, false);  // row_ror:8
  v += __builtin_amdgcn_update_dpp(v, v, 0x124, 0xF, 0xF, false);  // row_ror:4
  v += __builtin_amdgcn_update_dpp(v, v, 0x122, 0xF, 0xF, false);  // row_ror:2
  v += __builtin_amdgcn_update_dpp(v, v, 0x121, 0xF, 0xF, false);  // row_ror:1
  return v;
}
constexpr uint32_t kXOutOfRange = 0x80000000u;  // a byte offset past the activation buffer's range

using qtile::kNibbleBytes;
using qtile::kScaleBytes;
using qtile::kTileBytes;
using qtile::nibbles_natural;
using qtile::unpack_nibbles;
using qtile::unpack_nibbles2;
#define UNPACK_CONSTANTS(m, c) QTILE_UNPACK_CONSTANTS(m, c)

using qtile::swiglu_bf16;

// The outputs of a workgroup of 4 or more row blocks without SwiGLU (down) leave the LDS reduction
// as 16-byte stores of 8 adjacent outputs per thread: each thread's one item instead of a wave's
// 5-6 rounds of 2-byte stores per lane (config 2: down 23.5 -> 21.2 us, the same bits).  Narrower
// workgroups keep the per-lane stores (the dense projections' 32 items would sit on one wave:
// o_proj 6.8 -> 7.1 us).  JIT_QMM_VEC_EPILOGUE=0 builds the per-lane stores everywhere.
#ifndef JIT_QMM_VEC_EPILOGUE
#define JIT_QMM_VEC_EPILOGUE 1
#endif
constexpr bool kVecEpilogue = JIT_QMM_VEC_EPILOGUE;
constexpr int kVecEpilogueMinNb = 4;

// Phase stamps (a build with JIT_QMM_STAMPS=1 only, bench.py --gemv-phases): wave 0 of every
// workgroup that has work records s_memrealtime (a constant 100 MHz clock shared by the device) at
// kernel entry (0), once its expert's count is known and its first loads go out (1), once every load
// of its first pass has landed (2; that build waits for all of them there instead of group by group),
// when the pass's arithmetic is done (3), after the K-split partial sums have met in LDS (4) and at
// its end (5).
#ifndef JIT_QMM_STAMPS
#define JIT_QMM_STAMPS 0
#endif
#if JIT_QMM_STAMPS
constexpr int kStampSlots = 1 << 16;
__device__ uint64_t g_qmm_stamps[kStampSlots][8];
#define QMM_STAMP(i)                                        \
  do {                                                      \
    if (stamp_pass == 0) ts[i] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define QMM_STAMP(i) \
  do {               \
  } while (0)
#endif

template <int NB, int GPW, bool SWIGLU, bool PACKED, int TT = 1, bool COMPACT = false, bool ROUTED = false,
          int PRO = 0>
__global__ __launch_bounds__(512) void qmm_kernel(const QmmArgs a) {
#if JIT_QMM_STAMPS
  uint64_t ts[6] = {__builtin_amdgcn_s_memrealtime(), 0, 0, 0, 0, 0};
  int stamp_pass = 0;
#endif
  static_assert(!PACKED || GPW % 2 == 0, "packed tiles hold pairs of groups");
  constexpr int NBW = SWIGLU ? 2 * NB : NB;  // weight row blocks (gate and up blocks with SWIGLU)
  extern __shared__ float red[];             // [KSPLIT][TT][NBW][4][64]
  const int ksplit = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = lane_id();
  const int lr = l & 15, lg = l >> 4;
  static_assert(!ROUTED || (COMPACT && TT == 1), "a routed step is one token over the compact grid");
  static_assert(PRO == 0 || (!SWIGLU && TT == 1 && !COMPACT), "a row prologue goes with a one-row dense projection");
  int e = 0, cnt, off;
  if constexpr (ROUTED) {
    // One token routes itself (the router's top-k on every wave: route::topk_slot_key, the
    // router kernels' own arithmetic): grid row y takes the y-th smallest of the token's k expert
    // ids -- the packing's order, one pair each at position y.  Workgroup (0, 0) also writes the
    // packing tables (jit_route_pack's, for one token) that the later launches read.
    const uint32_t slot = route::topk_slot_key<2>(a.logits, a.E, a.k, l);  // lane j < k: slot j
    const int id = (int)(slot & 0xffffu);
    int rank = 0;  // among the k distinct ids
    for (int j = 0; j < a.k; j++) rank += __builtin_amdgcn_readlane(id, j) < id ? 1 : 0;
    const int y = blockIdx.y;
    const unsigned long long at = __ballot(l < a.k && rank == y);
    e = __builtin_amdgcn_readlane(id, __ffsll((long long)at) - 1);
    cnt = 1;
    off = y;
    if (blockIdx.x == 0 && y == 0 && wave == 0) {
      const float tot = route::slots_total(slot, a.k);
      if (l < a.k) {
        const float sc = bf2f(route::key_bf16(slot));
        a.inds[l] = (uint32_t)id;
        a.scores[l] = (uint16_t)(a.norm ? f2bf(sc / tot) : f2bf(sc));
        a.inv[l] = rank;
        a.order[rank] = l;
        a.pair_row[rank] = 0;
        a.seg_expert[rank] = id;
        a.seg_start[rank] = rank;
        a.seg_cnt[rank] = 1;
      }
      for (int x = l; x < a.E; x += 64) {
        int c = 0, below = 0;
        for (int j = 0; j < a.k; j++) {
          const int o = __builtin_amdgcn_readlane(id, j);
          c += o == x ? 1 : 0;
          below += o < x ? 1 : 0;
        }
        a.t_cnt[x] = c;
        a.t_off[x] = below;
      }
      if (l < 4) a.meta[l] = l == 0 ? a.k : (l == 1 ? 1 : 0);  // segments, largest, bad pairs, 0
    }
  } else if (a.cnt && !COMPACT) {
    e = blockIdx.y;
    cnt = a.cnt[e];
    off = a.off[e];
  } else if (a.cnt) {
    // COMPACT (a step of P < E pairs, min(E, P) grid rows): workgroup row y takes the y-th
    // expert that has pairs (experts in id order), so such a step launches no workgroups for
    // idle experts.  Its offset is the pairs of the experts before it (the packing sorts pairs
    // by expert).  (A grid of E rows keeps the direct lookup: every wave of a full grid reading
    // all the counts would crowd the one L2 channel that holds them.)
    // The counts of up to kScanAhead * 64 experts are requested together before the first ballot
    // (one round trip instead of one per 64 experts; a stack of more experts reads the rest as
    // it goes).
    constexpr int kScanAhead = 4;
    const int y = blockIdx.y;
    int seen = 0, before = 0;
    int cpre[kScanAhead];
#pragma unroll
    for (int j = 0; j < kScanAhead; j++) cpre[j] = 64 * j + l < a.E ? a.cnt[64 * j + l] : 0;
    e = -1;
    for (int base = 0; base < a.E; base += 64) {  // uniform loop
      int c = cpre[0];
#pragma unroll
      for (int j = 1; j < kScanAhead; j++)
        if (base == 64 * j) c = cpre[j];
      if (base >= 64 * kScanAhead) c = base + l < a.E ? a.cnt[base + l] : 0;
      const unsigned long long m = __ballot(c > 0);
      const int n = __popcll(m);
      if (y < seen + n) {
        const int rank = __popcll(m & ((1ull << l) - 1ull));
        const int bit = __ffsll((long long)__ballot(c > 0 && rank == y - seen)) - 1;
        e = base + bit;
        cnt = __builtin_amdgcn_readlane(c, bit);
        off = before + wave_sum_i(l < bit ? c : 0);
        break;
      }
      seen += n;
      before += wave_sum_i(c);
    }
    if (e < 0) return;  // fewer experts with pairs than grid rows (uniform over the workgroup)
  } else {
    cnt = a.T;
    off = 0;
  }
  if (cnt <= 0) return;  // uniform over the workgroup
  QMM_STAMP(1);
  const int n0 = blockIdx.x * (16 * NB);
  const int G = a.K >> 6, KW = a.K >> 3;
  const int g0 = wave * GPW;
  // token passes of 16 * TT tokens; with gridDim.z > 1 the passes are dealt to z
  // workgroups of the same rows (a dense decode batch split over more workgroups)
  const int tfirst = 16 * TT * blockIdx.z, tstride = 16 * TT * gridDim.z;
  if (tfirst >= cnt) return;  // uniform over the workgroup

  // The prologue issues every load of the first pass before its first wait: the row indices of
  // the first pass's tokens (before the weights: vector loads complete in order, so an index
  // loaded after the weights would hold the activation loads back until every weight load had
  // landed), the weight slice, then the activations, whose offsets need the indices.  The scale
  // shuffles, which need the scale loads, come after all of them; the scheduling barriers keep
  // the compiler from hoisting an offset or a shuffle (and the wait it implies) above a load.
  // Only the gate||up instances (SWIGLU) gather token rows through a row index (launch_qmm checks
  // it); down and the dense projections read their rows in place, with no load and no wait.
  auto row_of = [&](int tok) {
    const int pos = off + (tok < cnt ? tok : 0);
    if constexpr (ROUTED) return 0;  // (the one token's row)
    else if constexpr (SWIGLU) return a.row_index[pos];
    else return pos;
  };
  // a row as a byte offset into x for the activation loads; a token past the expert's count gets
  // an offset past the buffer's range, whose loads return zeros without reading memory
  auto x_off = [&](int tok, int row) {
    return tok < cnt ? (int)((uint32_t)row * (uint32_t)a.K * 2u) : (int)kXOutOfRange;
  };
  // activations through a buffer resource (2 GiB range: x holds fewer bytes), so that the lanes
  // of padding tokens (a 16-token tile over an expert's ~2 decode tokens) fetch nothing
  const __amdgpu_buffer_rsrc_t xbuf = __builtin_amdgcn_make_buffer_rsrc((void *)a.x, (short)0, 0x7fffffff, 0x00020000);
  int row0[TT];
#pragma unroll
  for (int tt = 0; tt < TT; tt++) row0[tt] = row_of(tfirst + 16 * tt + lr);

  // PRO 1: the input row's operands requested before the weight slice (vector loads complete in
  // order: requested behind it, they would land only once all of it had; router launch 3.67 ->
  // 3.25 us at bs = 1).  PRO 2's combine reads its rows through the slots' positions, after the
  // weights: requesting all of the token's rows ahead instead was slower (6.6 -> 7.9 us).
  const int pro_n = threadIdx.x * 8;
  const bool pro_on = PRO != 0 && threadIdx.x < 256 && pro_n < a.K;
  uint4 pro_wq = make_uint4(0u, 0u, 0u, 0u), pro_av = make_uint4(0u, 0u, 0u, 0u), pro_rv = make_uint4(0u, 0u, 0u, 0u);
  // workgroup 0's copies of the row (the sum, and for PRO 1 the normed row), stored at the kernel's
  // end: a store counts on the same in-order counter as the loads, so one issued before the weights'
  // wait would be waited for there as well
  uint4 pro_sum_q = make_uint4(0u, 0u, 0u, 0u), pro_norm_q = make_uint4(0u, 0u, 0u, 0u);
  if constexpr (PRO == 1) {
    if (pro_on) {
      pro_wq = *(const uint4 *)(a.pr_w + pro_n);
      pro_av = *(const uint4 *)(a.pr_a + pro_n);
      pro_rv = *(const uint4 *)(a.pr_resid + pro_n);
    }
    asm volatile("" ::: "memory");
  }

  // ---- the wave's whole weight slice: GPW groups x NBW row blocks
  uint2 wv[GPW][NBW];
  uint32_t sv[NBW][(GPW + 1) / 2], bv[NBW][(GPW + 1) / 2];  // bf16 pairs (groups 2j, 2j+1)
  uint2 sbl[NBW];  // packed layout: the lane's 8 bytes of its block's scale tile, shuffled later
#pragma unroll
  for (int rb = 0; rb < NBW; rb++) {
    // rows past N (a partial last tile) read row block n0 instead; only stores are guarded
    const int ob = SWIGLU ? (rb % NB) : rb;
    const int rowo = n0 + 16 * ob < a.N ? n0 + 16 * ob : n0;
    const int rowb = (SWIGLU && rb >= NB ? a.N : 0) + rowo;  // first row of the block
    if (PACKED) {
      static_assert(GPW / 2 <= 4, "one scale load covers at most 4 group pairs");
      const int GP = a.K >> 7;
      const uint8_t *blk = (const uint8_t *)a.w + (long long)e * a.w_estride + (long long)(rowb >> 4) * GP * kTileBytes;
      const uint8_t *nb = blk + (g0 >> 1) * kNibbleBytes;
      // lane group lg fetches pair min(lg, GPW/2 - 1) (lanes past the slice re-read its last pair)
      sbl[rb] = ld_stream8(blk + (long long)GP * kNibbleBytes +
                           ((g0 >> 1) + min(lg, GPW / 2 - 1)) * kScaleBytes + 8 * lr);
#pragma unroll
      for (int j = 0; j < GPW / 2; j++) {
        const uint4 q = ld_stream16(nb + j * kNibbleBytes + 16 * l);
        wv[2 * j][rb] = make_uint2(q.x, q.y);
        wv[2 * j + 1][rb] = make_uint2(q.z, q.w);
      }
    } else {
      const long long row = (long long)rowb + lr;
      const uint32_t *wp = a.w + e * a.w_estride + row * KW + 8 * g0 + 2 * lg;
      const uint16_t *sp = a.s + e * a.g_estride + row * G + g0;
      const uint16_t *bp = a.b + e * a.g_estride + row * G + g0;
#pragma unroll
      for (int g = 0; g < GPW; g++) {
        const uint2 wm = ld_stream8(wp + 8 * g);
        wv[g][rb] = make_uint2(nibbles_natural(wm.x), nibbles_natural(wm.y));
      }
#pragma unroll
      for (int j = 0; j < (GPW + 1) / 2; j++) {
        const uint32_t s0 = sp[2 * j], b0 = bp[2 * j];
        const uint32_t s1 = (2 * j + 1 < GPW) ? sp[2 * j + 1] : 0u;
        const uint32_t b1 = (2 * j + 1 < GPW) ? bp[2 * j + 1] : 0u;
        sv[rb][j] = s0 | (s1 << 16);
        bv[rb][j] = b0 | (b1 << 16);
      }
    }
  }
  Frag8 ones;
#pragma unroll
  for (int i = 0; i < 4; i++) ones.u[i] = 0x3F803F80u;
  UNPACK_CONSTANTS(um, uc);

  // TT token tiles of 16 per pass: their activations are loaded together, their
  // partial sums meet in LDS once (one barrier round and one epilogue per pass)
  // (the first pass is peeled off so that its activation loads follow the weight loads
  // directly, with no merge of load paths in front of them)
  // activation fragments (natural k order, as the unpacked weights); lanes past the
  // last token load from outside the buffer's range (no branch around the loads): zeros,
  // which feed only output rows of tokens that are never stored
  // PRO: the row, after the K-split partials' region of the LDS (8 floats of reduction, then K bf16)
  float *pro_red = red + ksplit * TT * NBW * 4 * 64;
  const uint8_t *pro_row = (const uint8_t *)(pro_red + 8);
  auto load_x = [&](const int t0, const int (&rows)[TT], Frag8 (&xa)[TT][GPW][2]) {
    if constexpr (PRO != 0) {  // the one token's lanes read the row from LDS, the padding lanes zeros
#pragma unroll
      for (int g = 0; g < GPW; g++) {
        const uint8_t *xp = pro_row + 2 * (64 * g0 + 16 * lg) + 128 * g;
        xa[0][g][0].q = lr == 0 ? *(const uint4 *)xp : make_uint4(0u, 0u, 0u, 0u);
        xa[0][g][1].q = lr == 0 ? *(const uint4 *)(xp + 16) : make_uint4(0u, 0u, 0u, 0u);
      }
      return;
    }
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
      const uint32_t xo = (uint32_t)x_off(t0 + 16 * tt + lr, rows[tt]) + 2u * (64 * g0 + 16 * lg);  // (out of range stays out)
#pragma unroll
      for (int g = 0; g < GPW; g++) {
        const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(xbuf, xo + 128 * g, 0, 0);
        const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(xbuf, xo + 128 * g + 16, 0, 0);
        xa[tt][g][0].q = make_uint4(v0.x, v0.y, v0.z, v0.w);
        xa[tt][g][1].q = make_uint4(v1.x, v1.y, v1.z, v1.w);
      }
    }
  };
  auto pass = [&](const int t0, const Frag8 (&xa)[TT][GPW][2]) {
    f32x4 acc[TT][NBW];
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
#pragma unroll
      for (int rb = 0; rb < NBW; rb++) acc[tt][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < GPW; g++) {
      f32x4 X[TT];
#pragma unroll
      for (int tt = 0; tt < TT; tt++) {
        X[tt] = mfma16x16x32(xa[tt][g][0], ones, f32x4{0.f, 0.f, 0.f, 0.f});
        X[tt] = mfma16x16x32(xa[tt][g][1], ones, X[tt]);
      }
#pragma unroll
      for (int rb = 0; rb < NBW; rb++) {
        // the packed words are loop-invariant across token tiles; this empty register
        // constraint keeps their unpacking here instead of hoisted (8 VGPRs per word pair)
        uint32_t w0 = wv[g][rb].x, w1 = wv[g][rb].y;
        asm volatile("" : "+v"(w0), "+v"(w1));
        // (the paired 64-bit shifts save 3 instructions a word pair; the other instances keep the
        // 32-bit shifts, which need no adjacent register pair: down would pass 168 VGPRs and lose a
        // wave per SIMD)
        Frag8 B0, B1;
        if constexpr (SWIGLU) {
          unpack_nibbles2(w0, w1, um, uc, B0, B1);
        } else {
          B0 = unpack_nibbles(w0, um, uc);
          B1 = unpack_nibbles(w1, um, uc);
        }
        const float sc = (g & 1) ? bf2f_hi(sv[rb][g >> 1]) : bf2f(sv[rb][g >> 1] & 0xffffu);
        const float bi = (g & 1) ? bf2f_hi(bv[rb][g >> 1]) : bf2f(bv[rb][g >> 1] & 0xffffu);
        const float bq = fmaf(-128.0f, sc, bi);
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
          f32x4 C = mfma16x16x32(xa[tt][g][0], B0, f32x4{0.f, 0.f, 0.f, 0.f});
          C = mfma16x16x32(xa[tt][g][1], B1, C);
#pragma unroll
          for (int i = 0; i < 4; i++) acc[tt][rb][i] = fmaf(bq, X[tt][i], fmaf(sc, C[i], acc[tt][rb][i]));
        }
      }
      // keep each group's nibble unpacking next to its MFMAs (hoisting every group's
      // unpacked fragments ahead would cost 8 registers per (group, block))
      __builtin_amdgcn_sched_barrier(0);
    }
    QMM_STAMP(3);
    // ---- the waves' partial sums meet in LDS; lane l holds C[token 4*lg + i][row lr]
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
#pragma unroll
      for (int rb = 0; rb < NBW; rb++)
#pragma unroll
        for (int i = 0; i < 4; i++) red[(((wave * TT + tt) * NBW + rb) * 4 + i) * 64 + l] = acc[tt][rb][i];
    __syncthreads();
    QMM_STAMP(4);
    if constexpr (!SWIGLU && kVecEpilogue && NB >= kVecEpilogueMinNb) {
      // each thread owns 8 adjacent outputs of one token: (tile, token, row octet) items spread over
      // the threads, the partial sums read as two 16-byte LDS reads per wave slice and added in wave
      // order as below, the outputs stored as one 16-byte store
      const int nthr = ksplit * 64;
      for (int it = threadIdx.x; it < TT * 16 * 2 * NB; it += nthr) {
        const int half = it & 1, tok = (it >> 1) & 15, rest = it >> 5;
        const int ob = rest % NB, tt = rest / NB;
        const int t = t0 + 16 * tt + tok;
        if (n0 + 16 * ob >= a.N || t >= cnt) continue;
        const int lane0 = 16 * (tok >> 2) + 8 * half;
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int ks = 0; ks < ksplit; ks++) {
          const float *pr = red + (((ks * TT + tt) * NBW + ob) * 4 + (tok & 3)) * 64 + lane0;
          const float4 p0 = *(const float4 *)pr, p1 = *(const float4 *)(pr + 4);
          v[0] += p0.x;
          v[1] += p0.y;
          v[2] += p0.z;
          v[3] += p0.w;
          v[4] += p1.x;
          v[5] += p1.y;
          v[6] += p1.z;
          v[7] += p1.w;
        }
        const uint4 w = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                                   pack_bf16x2(v[6], v[7]));
        *(uint4 *)(a.out + (long long)(off + t) * a.N + n0 + 16 * ob + 8 * half) = w;
      }
      __syncthreads();
      return;
    }
    // (tile, output block, token row i) triples are spread over the waves
    for (int idx = wave; idx < TT * 4 * NB; idx += ksplit) {
      const int tt = idx / (4 * NB), ob = (idx >> 2) % NB, i = idx & 3;
      const int t = t0 + 16 * tt + 4 * lg + i;
      if (n0 + 16 * ob >= a.N) continue;
      float v = 0.0f, u = 0.0f;
      for (int ks = 0; ks < ksplit; ks++) {
        v += red[(((ks * TT + tt) * NBW + ob) * 4 + i) * 64 + l];
        if (SWIGLU) u += red[(((ks * TT + tt) * NBW + NB + ob) * 4 + i) * 64 + l];
      }
      if (t < cnt) {
        uint16_t *o = a.out + (long long)(off + t) * a.N + n0 + 16 * ob + lr;
        *o = (uint16_t)(SWIGLU ? swiglu_bf16(v, u) : f2bf(v));
      }
    }
    __syncthreads();
  };
  if constexpr (PRO != 0) {
    // The input row, built as rmsnorm_kernel (PRO 1) or combine_rmsnorm_kernel (PRO 2) builds it
    // (rowops: thread t < 256 owns elements 8t .. 8t + 7), while the weight loads above are in
    // flight; every workgroup builds it (no exchange), workgroup 0 also writes it out.
    const int D = a.K, n = pro_n;
    const bool on = pro_on;
    const uint4 wq = PRO == 1 ? pro_wq : (on ? *(const uint4 *)(a.pr_w + n) : make_uint4(0u, 0u, 0u, 0u));
    float v[8];
    float ss = 0.0f;
    if (on) {
      if constexpr (PRO == 1) {
        const uint4 av = pro_av, rv = pro_rv;
        const uint32_t aw[4] = {av.x, av.y, av.z, av.w}, rw[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          v[i] = bf2f(aw[i >> 1] & 0xffffu);
          v[i + 1] = bf2f_hi(aw[i >> 1]);
          v[i] += bf2f(rw[i >> 1] & 0xffffu);
          v[i + 1] += bf2f_hi(rw[i >> 1]);
          round_bf2(v[i], v[i + 1]);
        }
      } else {
        rowops::combine8(a.pr_a, a.pr_inv, a.pr_scores, a.pr_k, D, a.pr_resid, 0, n, v);
      }
      pro_sum_q = rowops::pack8(v);
#pragma unroll
      for (int i = 0; i < 8; i++) ss = fmaf(v[i], v[i], ss);
    }
    const float tot = rowops::block_sum_256(ss, pro_red);
    const float rs = rsqrtf(tot / (float)D + a.pr_eps);
    if (on) {
      float o[8];
      rowops::norm8(v, rs, wq, o);
      const uint4 q = rowops::pack8(o);
      *(uint4 *)(pro_row + 2 * n) = q;
      pro_norm_q = q;
    }
    __syncthreads();
  }
  {
    Frag8 xa[TT][GPW][2];
    __builtin_amdgcn_sched_barrier(0);
    load_x(tfirst, row0, xa);
    __builtin_amdgcn_sched_barrier(0);
    if (PACKED) {
#pragma unroll
      for (int rb = 0; rb < NBW; rb++)
#pragma unroll
        for (int j = 0; j < GPW / 2; j++) {
          sv[rb][j] = (uint32_t)__shfl((int)sbl[rb].x, 16 * j + lr, 64);
          bv[rb][j] = (uint32_t)__shfl((int)sbl[rb].y, 16 * j + lr, 64);
        }
    }
#if JIT_QMM_STAMPS
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("" ::: "memory");
#endif
    QMM_STAMP(2);
    pass(tfirst, xa);
#if JIT_QMM_STAMPS
    stamp_pass = 1;
#endif
  }
  for (int t0 = tfirst + tstride; t0 < cnt; t0 += tstride) {
    int rows[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) rows[tt] = row_of(t0 + 16 * tt + lr);
    Frag8 xa[TT][GPW][2];
    load_x(t0, rows, xa);
    pass(t0, xa);
  }
  if constexpr (PRO != 0) {
    if (pro_on && blockIdx.x == 0 && blockIdx.z == 0) {
      *(uint4 *)(a.pr_sum + pro_n) = pro_sum_q;
      if constexpr (PRO == 1) *(uint4 *)(a.pr_norm + pro_n) = pro_norm_q;
    }
  }
#if JIT_QMM_STAMPS
  ts[5] = __builtin_amdgcn_s_memrealtime();
  const long long slot = blockIdx.x + (long long)gridDim.x * (blockIdx.y + (long long)gridDim.y * blockIdx.z);
  if (threadIdx.x < 6 && slot < kStampSlots) {
    uint64_t v = ts[0];
#pragma unroll
    for (int i = 1; i < 6; i++) v = threadIdx.x == i ? ts[i] : v;
    g_qmm_stamps[slot][threadIdx.x] = v;
  }
  if (threadIdx.x == 6 && slot < kStampSlots) g_qmm_stamps[slot][6] = 1;  // (a workgroup with work)
#endif
}

template <int NB, int GPW, bool SWIGLU, bool PACKED, int TT = 1, bool COMPACT = false, bool ROUTED = false,
          int PRO = 0>
int launch_qmm(const QmmArgs &a, int E, hipStream_t st, const char *what, int zsplit = 1) {
  constexpr int NBW = SWIGLU ? 2 * NB : NB;
  const int G = a.K / 64;
  const int ksplit = G / GPW;
  if (ksplit * GPW != G || ksplit < 1 || ksplit > 8)
    return jit::fail(JIT_EUNSUPPORTED, "%s: K=%d does not split into %d-group wave slices", what, a.K, GPW);
  if (SWIGLU != (a.row_index != nullptr || ROUTED))
    return jit::fail(JIT_EINVAL, "%s: a row index goes with the gate||up instances only", what);
  const dim3 grid((a.N + 16 * NB - 1) / (16 * NB), E, zsplit), block(64 * ksplit);
  const size_t lds = (size_t)ksplit * TT * NBW * 4 * 64 * sizeof(float) +
                     (PRO ? 8 * sizeof(float) + (size_t)a.K * sizeof(uint16_t) : 0);
  qmm_kernel<NB, GPW, SWIGLU, PACKED, TT, COMPACT, ROUTED, PRO><<<grid, block, lds, st>>>(a);
  return jit::check_launch(what);
}

// Groups per wave for a dense projection: the smallest even slice that splits K over at
// most 8 waves (the packed and direct layouts use the same split, so they agree bit for bit).
int dense_gpw(int K) {
  const int G = K / 64;
  for (int gpw = 2; gpw <= 8; gpw += 2)
    if (G % gpw == 0 && G / gpw <= 8) return gpw;
  return 0;
}

// Dense launch shape: up to two token tiles per pass (one reduction round for a
// 32-row decode batch), and 32 output rows per workgroup for a wide matrix with a
// short K-slice per wave (the activations each workgroup pulls through L2 then
// serve twice the rows).  The shape never changes a result: each output sums the
// same groups in the same order.
#ifndef JIT_DENSE_ZMAX
#define JIT_DENSE_ZMAX 4
#endif
#ifndef JIT_DENSE_WIDE_N
#define JIT_DENSE_WIDE_N 4096
#endif
template <bool PACKED, int GPW>
int launch_dense_gpw(const QmmArgs &a, hipStream_t st, const char *what) {
  // a decode batch's 16-token tiles go to separate workgroups (up to JIT_DENSE_ZMAX), so a
  // matrix of few row blocks still fills the chip and each workgroup pulls one tile's
  // activations; longer batches take two tiles per pass
  // (a prefill-sized batch spreads its 32-token passes over workgroups too: one pass each)
  const int tiles = (a.T + 15) / 16;
  const bool wide = GPW <= 4 && a.N >= JIT_DENSE_WIDE_N;
  if (tiles <= JIT_DENSE_ZMAX)
    return wide ? launch_qmm<2, GPW, false, PACKED, 1>(a, 1, st, what, tiles)
                : launch_qmm<1, GPW, false, PACKED, 1>(a, 1, st, what, tiles);
  const int passes = (tiles + 1) / 2;
  return wide ? launch_qmm<2, GPW, false, PACKED, 2>(a, 1, st, what, passes)
              : launch_qmm<1, GPW, false, PACKED, 2>(a, 1, st, what, passes);
}

template <bool PACKED>
int launch_dense(const QmmArgs &a, hipStream_t st) {
  const char *what = PACKED ? "jit_qmm_packed" : "jit_qmm";
  switch (dense_gpw(a.K)) {
    case 2: return launch_dense_gpw<PACKED, 2>(a, st, what);
    case 4: return launch_dense_gpw<PACKED, 4>(a, st, what);
    case 6: return launch_dense_gpw<PACKED, 6>(a, st, what);
    case 8: return launch_dense_gpw<PACKED, 8>(a, st, what);
    default: return jit::fail(JIT_EUNSUPPORTED, "%s covers K %% 256 == 0 and K <= 4096, got %d", what, a.K);
  }
}

// One-time repack of an MLX-layout stack into the packed layout above: one wave per
// (16-row block, group pair).
__global__ __launch_bounds__(64) void q4_prepack_kernel(const uint32_t *__restrict__ w,
                                                        const uint16_t *__restrict__ s,
                                                        const uint16_t *__restrict__ b, int N, int K,
                                                        uint8_t *__restrict__ out) {
  const long long tile = blockIdx.x;
  const int l = threadIdx.x, lr = l & 15, lg = l >> 4;
  const int GP = K >> 7, NRB = N >> 4, G = K >> 6, KW = K >> 3;
  const int gp = (int)(tile % GP);
  const int rbi = (int)((tile / GP) % NRB);
  const long long e = tile / ((long long)GP * NRB);
  const long long row = e * N + rbi * 16 + lr;
  const uint32_t *wr = w + row * KW + 16 * gp + 2 * lg;
  uint4 q;
  q.x = nibbles_natural(wr[0]);
  q.y = nibbles_natural(wr[1]);
  q.z = nibbles_natural(wr[8]);
  q.w = nibbles_natural(wr[9]);
  uint8_t *blk = out + (tile / GP) * GP * kTileBytes;  // the (expert, row block)'s block
  *(uint4 *)(blk + gp * kNibbleBytes + 16 * l) = q;
  if (lg == 0) {
    const uint16_t *sr = s + row * G + 2 * gp, *br = b + row * G + 2 * gp;
    *(uint2 *)(blk + (long long)GP * kNibbleBytes + gp * kScaleBytes + 8 * lr) =
        make_uint2((uint32_t)sr[0] | ((uint32_t)sr[1] << 16), (uint32_t)br[0] | ((uint32_t)br[1] << 16));
  }
}

}  // namespace

extern "C" int64_t jit_q4_packed_bytes(int E, int N, int K) {
  if (E <= 0 || N <= 0 || K <= 0 || N % 16 != 0 || K % 128 != 0) return -1;
  return (int64_t)E * (N / 16) * (K / 128) * kTileBytes;
}

extern "C" int jit_q4_prepack(const uint32_t *w, const uint16_t *scales, const uint16_t *biases, int E,
                              int N, int K, void *packed, void *stream) {
  if (E <= 0 || N <= 0 || K <= 0) return jit::fail(JIT_EINVAL, "q4_prepack: bad dims E=%d N=%d K=%d", E, N, K);
  if (N % 16 != 0 || K % 128 != 0)
    return jit::fail(JIT_EUNSUPPORTED, "q4_prepack covers N %% 16 == 0 and K %% 128 == 0, got N=%d K=%d", N, K);
  if (!w || !scales || !biases || !packed) return jit::fail(JIT_EINVAL, "q4_prepack: null pointer");
  const long long tiles = (long long)E * (N / 16) * (K / 128);
  if (tiles > 0x7fffffffLL) return jit::fail(JIT_EUNSUPPORTED, "q4_prepack: %lld tiles", tiles);
  q4_prepack_kernel<<<(unsigned)tiles, 64, 0, (hipStream_t)stream>>>(w, scales, biases, N, K, (uint8_t *)packed);
  return jit::check_launch("jit_q4_prepack");
}

// The kernels read activations through a buffer resource of a 2 GiB range (byte offsets in 32
// bits, past-the-end offsets for padding tokens).
static bool x_in_range(long long rows, int K) { return rows * K * 2 + 4096 < 0x7fffffffLL; }

static int qmm_common(const uint16_t *x, int T, int K, int N, uint16_t *y, const char *what) {
  if (T < 0 || K <= 0 || N <= 0) return jit::fail(JIT_EINVAL, "%s: bad dims T=%d K=%d N=%d", what, T, K, N);
  if (K % 256 != 0 || N % 16 != 0 || K > 4096)
    return jit::fail(JIT_EUNSUPPORTED, "%s covers K %% 256 == 0, K <= 4096 and N %% 16 == 0, got K=%d N=%d",
                     what, K, N);
  if (T > 0 && (!x || !y)) return jit::fail(JIT_EINVAL, "%s: null pointer", what);
  if (!x_in_range(T, K)) return jit::fail(JIT_EUNSUPPORTED, "%s: x of %d x %d bf16 exceeds 2 GiB", what, T, K);
  return JIT_OK;
}

extern "C" int jit_qmm(const uint16_t *x, int T, int K, const uint32_t *w, const uint16_t *scales,
                       const uint16_t *biases, int N, uint16_t *y, void *stream) {
  if (int rc = qmm_common(x, T, K, N, y, "qmm")) return rc;
  if (T == 0) return JIT_OK;
  if (!w || !scales || !biases) return jit::fail(JIT_EINVAL, "qmm: null pointer");
  QmmArgs a{x, nullptr, nullptr, nullptr, w, scales, biases, y, K, N, T, 0, 0, N};
  return launch_dense<false>(a, (hipStream_t)stream);
}

extern "C" int jit_qmm_packed(const uint16_t *x, int T, int K, const void *packed, int N, uint16_t *y,
                              void *stream) {
  if (int rc = qmm_common(x, T, K, N, y, "qmm_packed")) return rc;
  if (T == 0) return JIT_OK;
  if (!packed) return jit::fail(JIT_EINVAL, "qmm_packed: null pointer");
  QmmArgs a{x, nullptr, nullptr, nullptr, (const uint32_t *)packed, nullptr, nullptr, y, K, N, T, 0, 0, N};
  return launch_dense<true>(a, (hipStream_t)stream);
}

// One row's dense projection with its input row built in the launch (PRO 1 / 2): the launch shape of
// jit_qmm_packed for one token, so each output sums the same groups in the same order.
template <int PRO, int GPW>
int launch_dense_pro_gpw(const QmmArgs &a, hipStream_t st, const char *what) {
  const bool wide = GPW <= 4 && a.N >= JIT_DENSE_WIDE_N;
  return wide ? launch_qmm<2, GPW, false, true, 1, false, false, PRO>(a, 1, st, what, 1)
              : launch_qmm<1, GPW, false, true, 1, false, false, PRO>(a, 1, st, what, 1);
}

template <int PRO>
int launch_dense_pro(const QmmArgs &a, hipStream_t st, const char *what) {
  if (a.K % 256 != 0 || a.K > 2048 || a.N % 16 != 0)
    return jit::fail(JIT_EUNSUPPORTED, "%s covers D %% 256 == 0, D <= 2048 and N %% 16 == 0, got D=%d N=%d", what,
                     a.K, a.N);
  switch (dense_gpw(a.K)) {
    case 2: return launch_dense_pro_gpw<PRO, 2>(a, st, what);
    case 4: return launch_dense_pro_gpw<PRO, 4>(a, st, what);
    case 6: return launch_dense_pro_gpw<PRO, 6>(a, st, what);
    case 8: return launch_dense_pro_gpw<PRO, 8>(a, st, what);
    default: return jit::fail(JIT_EUNSUPPORTED, "%s: no wave split for D=%d", what, a.K);
  }
}

// rmsnorm of bf16(a + resid) (jit_rmsnorm with a residual, for one row) followed by jit_qmm_packed of the
// normed row, in one launch: h_out = the sum, hn_out = the normed row, y = hn . W^T.
extern "C" int jit_qmm_packed_add_rmsnorm(const uint16_t *a_row, const uint16_t *resid, const uint16_t *w, float eps,
                                          int D, const void *packed, int N, uint16_t *h_out, uint16_t *hn_out,
                                          uint16_t *y, void *stream) {
  if (D <= 0 || N <= 0) return jit::fail(JIT_EINVAL, "qmm_packed_add_rmsnorm: bad dims D=%d N=%d", D, N);
  if (!a_row || !resid || !w || !packed || !h_out || !hn_out || !y)
    return jit::fail(JIT_EINVAL, "qmm_packed_add_rmsnorm: null pointer");
  QmmArgs a{nullptr, nullptr, nullptr, nullptr, (const uint32_t *)packed, nullptr, nullptr, y, D, N, 1, 0, 0, N};
  a.pr_a = a_row;
  a.pr_resid = resid;
  a.pr_w = w;
  a.pr_eps = eps;
  a.pr_sum = h_out;
  a.pr_norm = hn_out;
  return launch_dense_pro<1>(a, (hipStream_t)stream, "jit_qmm_packed_add_rmsnorm");
}

// jit_moe_combine_rmsnorm for one row followed by jit_qmm_packed of the normed row, in one launch:
// y_out = the combined row (the next layer's residual), out = rmsnorm(y_out) . W^T.
extern "C" int jit_qmm_packed_combine_rmsnorm(const uint16_t *r, const int32_t *inv, const uint16_t *scores, int k,
                                              const uint16_t *resid, const uint16_t *w, float eps, int D,
                                              const void *packed, int N, uint16_t *y_out, uint16_t *out,
                                              void *stream) {
  if (D <= 0 || N <= 0 || k <= 0)
    return jit::fail(JIT_EINVAL, "qmm_packed_combine_rmsnorm: bad dims D=%d N=%d k=%d", D, N, k);
  if (!r || !inv || !scores || !w || !packed || !y_out || !out)
    return jit::fail(JIT_EINVAL, "qmm_packed_combine_rmsnorm: null pointer");
  QmmArgs a{nullptr, nullptr, nullptr, nullptr, (const uint32_t *)packed, nullptr, nullptr, out, D, N, 1, 0, 0, N};
  a.pr_a = r;
  a.pr_inv = inv;
  a.pr_scores = scores;
  a.pr_k = k;
  a.pr_resid = resid;
  a.pr_w = w;
  a.pr_eps = eps;
  a.pr_sum = y_out;
  return launch_dense_pro<2>(a, (hipStream_t)stream, "jit_qmm_packed_combine_rmsnorm");
}

// Expert GEMV shapes (groups of 64 per wave; row blocks of 16 per workgroup), chosen by timing
// sweeps on MI355X over the config-2 routing.
#ifndef JIT_GU_GPW
#define JIT_GU_GPW 8
#endif
#ifndef JIT_DN_NB
#define JIT_DN_NB 4
#endif
#ifndef JIT_DN_GPW
#define JIT_DN_GPW 4
#endif
constexpr int kGuGpw = JIT_GU_GPW, kDnNb = JIT_DN_NB, kDnGpw = JIT_DN_GPW;

static int gate_up_check(const uint16_t *x, int K, const int32_t *pair_row, const int32_t *cnt,
                         const int32_t *off, int E, int I, int P, uint16_t *h) {
  if (K <= 0 || I <= 0 || E <= 0 || P < 0)
    return jit::fail(JIT_EINVAL, "moe_gate_up: bad dims K=%d I=%d E=%d P=%d", K, I, E, P);
  if (K % 512 != 0 || K > 4096 || I % 16 != 0)
    return jit::fail(JIT_EUNSUPPORTED, "moe_gate_up covers K %% 512 == 0, K <= 4096 and I %% 16 == 0, got K=%d I=%d",
                     K, I);
  if (P > 0 && (!x || !pair_row || !cnt || !off || !h)) return jit::fail(JIT_EINVAL, "moe_gate_up: null pointer");
  if (!x_in_range(P, K))  // x has at most P rows (every row routes at least one pair)
    return jit::fail(JIT_EUNSUPPORTED, "moe_gate_up: %d pairs of K=%d exceed the 2 GiB activation range", P, K);
  return JIT_OK;
}

extern "C" int jit_moe_gate_up_swiglu(const uint16_t *x, int K, const int32_t *pair_row,
                                      const int32_t *expert_cnt, const int32_t *expert_off, int E,
                                      const uint32_t *w, const uint16_t *scales,
                                      const uint16_t *biases, int I, int P, uint16_t *h,
                                      void *stream) {
  if (int rc = gate_up_check(x, K, pair_row, expert_cnt, expert_off, E, I, P, h)) return rc;
  if (P == 0) return JIT_OK;
  if (!w || !scales || !biases) return jit::fail(JIT_EINVAL, "moe_gate_up: null pointer");
  QmmArgs a{x, pair_row, expert_cnt, expert_off, w, scales, biases, h, K, I, 0,
            (long long)2 * I * (K / 8), (long long)2 * I * (K / 64), 2 * I, E};
  if (P < E) return launch_qmm<1, kGuGpw, true, false, 1, true>(a, P, (hipStream_t)stream, "jit_moe_gate_up_swiglu");
  return launch_qmm<1, kGuGpw, true, false>(a, E, (hipStream_t)stream, "jit_moe_gate_up_swiglu");
}

extern "C" int jit_moe_gate_up_swiglu_packed(const uint16_t *x, int K, const int32_t *pair_row,
                                             const int32_t *expert_cnt, const int32_t *expert_off, int E,
                                             const void *packed, int I, int P, uint16_t *h, void *stream) {
  if (int rc = gate_up_check(x, K, pair_row, expert_cnt, expert_off, E, I, P, h)) return rc;
  if (P == 0) return JIT_OK;
  if (!packed) return jit::fail(JIT_EINVAL, "moe_gate_up_packed: null pointer");
  QmmArgs a{x, pair_row, expert_cnt, expert_off, (const uint32_t *)packed, nullptr, nullptr, h, K, I, 0,
            jit_q4_packed_bytes(1, 2 * I, K), 0, 2 * I, E};
  if (P < E) return launch_qmm<1, kGuGpw, true, true, 1, true>(a, P, (hipStream_t)stream, "jit_moe_gate_up_swiglu_packed");
  return launch_qmm<1, kGuGpw, true, true>(a, E, (hipStream_t)stream, "jit_moe_gate_up_swiglu_packed");
}

// A one-token step routed inside the gate||up launch (jit_route_pack + jit_moe_gate_up_swiglu_packed
// for one token, one launch): every workgroup takes the token's top-k from its router logits, and
// the packing tables are written for the down and combine launches that follow.
extern "C" int jit_moe_gate_up_swiglu_routed_packed(const uint16_t *x, int K, const uint16_t *logits, int E, int k,
                                                    int norm, const void *packed, int I, uint16_t *h, uint32_t *inds,
                                                    uint16_t *scores, int32_t *order, int32_t *pair_row, int32_t *inv,
                                                    int32_t *expert_cnt, int32_t *expert_off, int32_t *seg_expert,
                                                    int32_t *seg_start, int32_t *seg_cnt, int32_t *meta,
                                                    void *stream) {
  if (K <= 0 || I <= 0 || E <= 0 || !(0 < k && k <= E))
    return jit::fail(JIT_EINVAL, "moe_gate_up_routed: bad dims K=%d I=%d E=%d k=%d", K, I, E, k);
  if (K % 512 != 0 || K > 4096 || I % 16 != 0 || E % 32 != 0 || E > 128 || k >= E || k > 64)
    return jit::fail(JIT_EUNSUPPORTED,
                     "moe_gate_up_routed covers K %% 512 == 0, K <= 4096, I %% 16 == 0, E %% 32 == 0, E <= 128 and "
                     "k < E, k <= 64, got K=%d I=%d E=%d k=%d", K, I, E, k);
  if (!x || !logits || !packed || !h || !inds || !scores || !order || !pair_row || !inv || !expert_cnt ||
      !expert_off || !seg_expert || !seg_start || !seg_cnt || !meta)
    return jit::fail(JIT_EINVAL, "moe_gate_up_routed: null pointer");
  QmmArgs a{x, nullptr, nullptr, nullptr, (const uint32_t *)packed, nullptr, nullptr, h, K, I, 0,
            jit_q4_packed_bytes(1, 2 * I, K), 0, 2 * I, E, logits, k, norm ? 1 : 0, inds, scores, order, pair_row,
            inv, expert_cnt, expert_off, seg_expert, seg_start, seg_cnt, meta};
  return launch_qmm<1, kGuGpw, true, true, 1, true, true>(a, k, (hipStream_t)stream,
                                                          "jit_moe_gate_up_swiglu_routed_packed");
}

static int down_check(const uint16_t *h, int I, const int32_t *cnt, const int32_t *off, int E, int D, int P,
                      uint16_t *r) {
  if (I <= 0 || D <= 0 || E <= 0 || P < 0)
    return jit::fail(JIT_EINVAL, "moe_down: bad dims I=%d D=%d E=%d P=%d", I, D, E, P);
  if (I % 256 != 0 || I > 2048 || D % 16 != 0)
    return jit::fail(JIT_EUNSUPPORTED, "moe_down covers I %% 256 == 0, I <= 2048 and D %% 16 == 0, got I=%d D=%d",
                     I, D);
  if (P > 0 && (!h || !cnt || !off || !r)) return jit::fail(JIT_EINVAL, "moe_down: null pointer");
  if (!x_in_range(P, I)) return jit::fail(JIT_EUNSUPPORTED, "moe_down: h of %d x %d bf16 exceeds 2 GiB", P, I);
  return JIT_OK;
}

extern "C" int jit_moe_down(const uint16_t *h, int I, const int32_t *expert_cnt,
                            const int32_t *expert_off, int E, const uint32_t *w,
                            const uint16_t *scales, const uint16_t *biases, int D, int P, uint16_t *r,
                            void *stream) {
  if (int rc = down_check(h, I, expert_cnt, expert_off, E, D, P, r)) return rc;
  if (P == 0) return JIT_OK;
  if (!w || !scales || !biases) return jit::fail(JIT_EINVAL, "moe_down: null pointer");
  QmmArgs a{h, nullptr, expert_cnt, expert_off, w, scales, biases, r, I, D, 0,
            (long long)D * (I / 8), (long long)D * (I / 64), D, E};
  if (P < E) return launch_qmm<kDnNb, kDnGpw, false, false, 1, true>(a, P, (hipStream_t)stream, "jit_moe_down");
  return launch_qmm<kDnNb, kDnGpw, false, false>(a, E, (hipStream_t)stream, "jit_moe_down");
}

extern "C" int jit_moe_down_packed(const uint16_t *h, int I, const int32_t *expert_cnt,
                                   const int32_t *expert_off, int E, const void *packed, int D, int P,
                                   uint16_t *r, void *stream) {
  if (int rc = down_check(h, I, expert_cnt, expert_off, E, D, P, r)) return rc;
  if (P == 0) return JIT_OK;
  if (!packed) return jit::fail(JIT_EINVAL, "moe_down_packed: null pointer");
  QmmArgs a{h, nullptr, expert_cnt, expert_off, (const uint32_t *)packed, nullptr, nullptr, r, I, D, 0,
            jit_q4_packed_bytes(1, D, I), 0, D, E};
  if (P < E) return launch_qmm<kDnNb, kDnGpw, false, true, 1, true>(a, P, (hipStream_t)stream, "jit_moe_down_packed");
  return launch_qmm<kDnNb, kDnGpw, false, true>(a, E, (hipStream_t)stream, "jit_moe_down_packed");
}

#if JIT_QMM_STAMPS
// The stamps of the last launches (bench.py --gemv-phases): clear, then copy out kStampSlots x 8 words.
extern "C" int jit_qmm_stamps_clear(void *stream) {
  void *p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_qmm_stamps)) != hipSuccess) return JIT_ELAUNCH;
  return hipMemsetAsync(p, 0, sizeof(g_qmm_stamps), (hipStream_t)stream) == hipSuccess ? 0 : JIT_ELAUNCH;
}
extern "C" int jit_qmm_stamps_read(uint64_t *host, int slots) {
  if (!host || slots < 0 || slots > kStampSlots) return JIT_EINVAL;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_qmm_stamps), (size_t)slots * 8 * sizeof(uint64_t), 0,
                             hipMemcpyDeviceToHost) == hipSuccess ? 0 : JIT_ELAUNCH;
}
#endif
