// Expert GEMMs over long expert segments (chunked prefill, configs with many rows
// per expert) on gfx950 matrix cores: the sorted-segment gather_qmm of the
// reference's prefill (Q36/kernels/gather_qmm_prefill.py:1-257, MLX's quantized
// block loader + tile MMA), whose arithmetic it keeps: every weight is
// dequantized to bf16, w = bf16(s * q + b), and the MMA accumulates bf16
// products in fp32.  Rows are independent, so a row's result does not depend on
// how many rows its expert has.
//
// Work split: a workgroup of 8 waves (two a SIMD) owns 256 weight rows of one expert
// (down: 16 row blocks; gate||up: 8 gate blocks and the 8 up blocks of the same
// output columns, so SwiGLU is fused) and every token of the expert's segment, in
// chunks of up to 16 * TTS tokens.  Each wave owns 2 row blocks (gate||up: a gate
// block and its up block).  K is walked in steps of one group pair (128 k): the wave
// dequantizes its 2 row blocks' pair into bf16 MFMA B fragments once (one fma and
// half a convert per weight) and uses them against every token tile of the chunk,
// whose activations the workgroup stages in LDS (gathered through pair_row for
// gate||up).  The next step's packed weights and activations are loaded while the
// current step computes.  Two waves a SIMD let one wave's dequantization (vector ALU)
// run while the other's MFMAs keep the matrix core busy.  fp32 accumulators: TTS x 2
// tiles of 16 x 16 per wave.
#include "qtile.hpp"

namespace {

constexpr int kSegWaves = 8;
constexpr int kSegRB = 2;                 // row blocks per wave
constexpr int kSegThreads = 64 * kSegWaves;
constexpr int kSegRows = 16 * kSegRB * kSegWaves;  // weight rows per workgroup
constexpr int kSegTT = 10;                // token tiles per chunk of an expert segment (160 tokens)
// (a dense batch, one matrix with its token chunks spread over workgroups, sizes its chunks to the
// CUs: jit_qmm_seg)
#ifndef JIT_SEG_AHEAD
#define JIT_SEG_AHEAD 1
#endif
constexpr int kSegAhead = JIT_SEG_AHEAD;  // token tiles whose fragment reads run ahead of the MFMAs
#ifndef JIT_SEG_IGLP
#define JIT_SEG_IGLP 0
#endif

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // (HIP's uint4 is a union-based struct)

struct SegArgs {
  const uint16_t *x;          // activations [rows, K] bf16
  const int32_t *row_index;   // x row of each sorted position (null: the position itself)
  const int32_t *cnt, *off;   // pairs per expert, first sorted position per expert (null: a
                              // dense matrix, E = 1, rows 0 .. T - 1)
  const uint8_t *w;           // packed stack [E, rows_w, K]
  uint16_t *out;              // [P, N] bf16 in sorted order
  long long w_estride;        // packed bytes per expert
  int K, N;                   // N: output columns (I for gate||up, D for down)
  int T;                      // rows of a dense matrix (cnt null)
  int nx, groups;             // column blocks per group; groups = experts (or a dense matrix's token chunks)
};

// Workgroup -> (group, column block), XCD-aware.  MI355X deals the workgroups of a launch to its
// 8 XCDs round-robin (workgroup i to XCD i % 8), and each XCD has its own L2.  All column blocks
// of one group (an expert's segment, or one token chunk of a dense matrix) read the same
// activation rows, so they are given consecutive slots of one XCD: group g goes to XCD g % 8,
// and its nx blocks follow each other there, resident together, so the rows leave HBM (or the
// last-level cache) once per group instead of once per column block.  The grid is padded to
// 8 * ceil(groups / 8) groups; the padding's workgroups exit at once.
__device__ __forceinline__ bool seg_block(const SegArgs &a, int &g, int &cb) {
  const int L = blockIdx.x, xcd = L & 7, slot = L >> 3;
  g = xcd + 8 * (slot / a.nx);
  cb = slot % a.nx;
  return g < a.groups;
}

inline dim3 seg_grid(int nx, int groups) { return dim3(nx * 8 * ((groups + 7) / 8)); }

// 8 packed-order nibbles of a word -> 8 bf16 weights bf16(s * q + b) in natural k order.
// The masked words pass through an empty asm so that each byte converts with one
// v_cvt_f32_ubyteN (the compiler would otherwise extract every nibble separately), and the
// weights are rounded in pairs (one v_cvt_pk_bf16_f32 each; s q + b is finite).
__device__ __forceinline__ Frag8 dequant_word(uint32_t w, float s, float b) {
  uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  asm volatile("" : "+v"(lo), "+v"(hi));
  // packed order: nibble positions 0..7 hold q0 q2 q4 q6 q1 q3 q5 q7, so the bytes of
  // lo are (q0, q4, q1, q5) and those of hi (q2, q6, q3, q7)
  const float q0 = (float)(lo & 0xffu), q4 = (float)((lo >> 8) & 0xffu);
  const float q1 = (float)((lo >> 16) & 0xffu), q5 = (float)(lo >> 24);
  const float q2 = (float)(hi & 0xffu), q6 = (float)((hi >> 8) & 0xffu);
  const float q3 = (float)((hi >> 16) & 0xffu), q7 = (float)(hi >> 24);
  Frag8 f;
  f.u[0] = pack_bf16x2_rne(fmaf(s, q0, b), fmaf(s, q1, b));
  f.u[1] = pack_bf16x2_rne(fmaf(s, q2, b), fmaf(s, q3, b));
  f.u[2] = pack_bf16x2_rne(fmaf(s, q4, b), fmaf(s, q5, b));
  f.u[3] = pack_bf16x2_rne(fmaf(s, q6, b), fmaf(s, q7, b));
  return f;
}

// LDS of a workgroup:
//   two activation stages: one K step's activations, 16 TTS token rows of 128 k (256 B, no
//     padding).  Row r's 16 B piece c sits in slot c ^ (r % 16), so the 16 rows one fragment
//     read touches (same piece, rows 16 t .. 16 t + 15) fall in 16 different slots: the reads
//     are free of bank conflicts without the padding the direct global->LDS loads (1 KB = 4
//     whole rows per wave instruction) could not insert;
//   three weight stages: per wave its 2 row blocks' nibble tiles of one K step (2 x 1 KB) and
//     their scale tiles (2 x 128 B, then copies of them: the instruction writes 1 KB);
//   the chunk's activation row indices.
// (per chunk of TTS token tiles: the expert segments take kSegTT, dense batches 5, 8 or 10, jit_qmm_seg)
constexpr int seg_stage_bytes(int tts) { return 16 * tts * 256; }
constexpr int kSegWLoads = kSegRB + 1;  // direct loads of a wave's weights per K step
constexpr int kSegWWave = kSegWLoads * 1024;
constexpr int kSegWStageBytes = kSegWaves * kSegWWave;
constexpr int seg_w_off(int tts) { return 2 * seg_stage_bytes(tts); }
constexpr int seg_row_off(int tts) { return seg_w_off(tts) + 3 * kSegWStageBytes; }
constexpr int seg_lds_bytes(int tts) { return seg_row_off(tts) + 16 * tts * (int)sizeof(int); }
static_assert(seg_lds_bytes(kSegTT) <= 160 * 1024, "gfx950 gives a workgroup at most 160 KB of LDS");

// s_waitcnt vmcnt(N), nothing else.  Direct loads are counted by hand: the compiler does not see
// the ones issued by inline assembly.
template <int N>
__device__ __forceinline__ void seg_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// A workgroup barrier that waits for nothing else: every wave has already waited for its own
// direct loads (__syncthreads()'s fence would also wait for the loads still in flight).
__device__ __forceinline__ void seg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ void seg_load_lds(const void *src, uint32_t dst) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(dst) : "memory", "m0");
}

// DENSE: one dense matrix (E = 1, cnt null), one token chunk per group.
//
// Pipeline over the K steps p (one group pair each).  Per wave and step, TTS / 2 + 3 direct
// loads: TTS / 2 of activations (4 rows of each of half the token tiles: waves 0-3 stage the
// even tiles, 4-7 the odd ones) and 3 of its packed weights.
//   top of step p: wait for step p's activations (requested at the top of step p - 1), one
//     barrier; request step p + 1's activations into the other stage and step p + 2's weights;
//   group 0's token tiles against B fragments dequantized during step p - 1, with the
//     dequantization of this step's group 1 between their MFMAs;
//   wait for step p + 1's weights (the wave's own: no barrier), then group 1's token tiles
//     with the dequantization of step p + 1's group 0 between their MFMAs.
// Each tile's activation fragments are read kSegAhead tiles ahead of its MFMAs.  Weights are
// requested one and a half steps before they are dequantized, activations (mostly L2 hits:
// an expert's column blocks run on one XCD) a step before they are read.
template <bool SWIGLU, bool DENSE = false, int TTS = kSegTT>
__global__ __launch_bounds__(kSegThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void seg_kernel(const SegArgs a) {
  static_assert(TTS % 2 == 0 && TTS >= 2 * kSegRB, "the halves of the waves stage alternate token tiles");
  constexpr int kTokens = 16 * TTS, kStage = seg_stage_bytes(TTS), kXLoads = TTS / 2;
  extern __shared__ __attribute__((aligned(16))) uint8_t seg_lds[];
  int *xrow = (int *)(seg_lds + seg_row_off(TTS));
  int grp, cb;
  if (!seg_block(a, grp, cb)) return;  // grid padding (uniform over the workgroup)
  const int e = DENSE ? 0 : grp;
  const int cnt = DENSE ? a.T : a.cnt[e], off = DENSE ? 0 : a.off[e];
  if (cnt <= 0) return;  // uniform over the workgroup
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = lane_id();
  const int lr = l & 15, lg = l >> 4;
  const int tid = threadIdx.x;
  const int GP = a.K >> 7;  // K steps (group pairs)
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)seg_lds);

  // the wave's 2 row blocks (index of the first row / 16 inside the expert's stack)
  int rbk[kSegRB];
#pragma unroll
  for (int r = 0; r < kSegRB; r++) {
    if (SWIGLU)  // gate block 8 cb + wave, and the up block of the same columns
      rbk[r] = (r ? a.N / 16 : 0) + cb * 8 + wave;
    else
      rbk[r] = cb * 16 + kSegRB * wave + r;
  }
  const uint8_t *wexp = a.w + (long long)e * a.w_estride;
  const long long tile_row = (long long)GP * qtile::kTileBytes;  // bytes of one row block's tiles
  // weight staging: nibble instruction r moves row block r's tile (lane l: its 16 B piece); the
  // scale instruction's lane l moves piece l % 8 of row block (l / 8) % 2's scale tile
  const uint8_t *wnib = wexp + 16 * l;
  const int rb_s = (l >> 3) & 1 ? rbk[1] : rbk[0];
  const uint8_t *wscl = wexp + rb_s * tile_row + (long long)GP * qtile::kNibbleBytes + 16 * (l & 7);
  const uint32_t wlds = lds0 + seg_w_off(TTS) + wave * kSegWWave;  // + stage * kSegWStageBytes
  const uint8_t *wmine = seg_lds + seg_w_off(TTS) + wave * kSegWWave;
  auto load_w = [&](int p) {
    const uint32_t st = wlds + (p % 3) * kSegWStageBytes;
#pragma unroll
    for (int r = 0; r < kSegRB; r++)
      seg_load_lds(wnib + rbk[r] * tile_row + p * qtile::kNibbleBytes, __builtin_amdgcn_readfirstlane(st + r * 1024));
    seg_load_lds(wscl + p * qtile::kScaleBytes, __builtin_amdgcn_readfirstlane(st + kSegRB * 1024));
  };
  // B fragment h of group g, row block r, from the staged step p: bf16(s q + b) of the lane's
  // word h of the group (the nibble tile's 16 B piece holds group 0's two words, then group 1's)
  auto dequant_word_at = [&](int p, int g, int r, int h, Frag8 (&bw)[kSegRB][2]) {
    const uint8_t *st = wmine + (p % 3) * kSegWStageBytes;
    const uint32_t q = *(const uint32_t *)(st + r * 1024 + 16 * l + 8 * g + 4 * h);
    const uint2 sb = *(const uint2 *)(st + kSegRB * 1024 + r * 128 + 8 * lr);
    const float sc = g ? bf2f_hi(sb.x) : bf2f(sb.x & 0xffffu);
    const float bi = g ? bf2f_hi(sb.y) : bf2f(sb.y & 0xffffu);
    bw[r][h] = dequant_word(q, sc, bi);
  };
  auto dequant_rb = [&](int p, int g, int r, Frag8 (&bw)[kSegRB][2]) {
    dequant_word_at(p, g, r, 0, bw);
    dequant_word_at(p, g, r, 1, bw);
  };
  // activation staging: the wave's instruction i moves rows 4 (wave % 4) .. + 3 (1 KB) of token
  // tile j = 2 i + wave / 4; lane l fetches the piece its slot l % 16 holds in row 16 j + srow
  const int srow = 4 * (wave & 3) + (l >> 4), jhalf = wave >> 2;
  const int spiece = (l & 15) ^ srow;
  // fragment reads: lane (lr, lg) reads pieces 8 g + 2 lg and + 1 of row 16 t + lr
  const int frow = lr * 256;

  const int cend = DENSE ? min(cnt, (grp + 1) * kTokens) : cnt;
  for (int c0 = DENSE ? grp * kTokens : 0; c0 < cend; c0 += kTokens) {
    const int nt = min(kTokens, cnt - c0);
    __syncthreads();  // the previous chunk's reads of the stages and of xrow are done
    for (int j = tid; j < kTokens; j += kSegThreads) {
      const int pos = off + c0 + min(j, nt - 1);  // rows past the segment re-read its last row
      xrow[j] = a.row_index ? a.row_index[pos] : pos;
    }
    __syncthreads();
    uint32_t xsrc[kXLoads];  // element offsets of this lane's pieces (x holds < 2^32 elements)
#pragma unroll
    for (int i = 0; i < kXLoads; i++)
      xsrc[i] = (uint32_t)xrow[16 * (2 * i + jhalf) + srow] * (uint32_t)a.K + 8 * spiece;
    auto load_x = [&](int p) {
      const uint32_t st = lds0 + (p & 1) * kStage + 4 * (wave & 3) * 256;
#pragma unroll
      for (int i = 0; i < kXLoads; i++)
        seg_load_lds(a.x + xsrc[i] + 128 * p, __builtin_amdgcn_readfirstlane(st + 16 * (2 * i + jhalf) * 256));
    };

    f32x4 acc[TTS][kSegRB];
#pragma unroll
    for (int t = 0; t < TTS; t++)
#pragma unroll
      for (int r = 0; r < kSegRB; r++) acc[t][r] = f32x4{0.f, 0.f, 0.f, 0.f};
    Frag8 bw0[kSegRB][2], bw1[kSegRB][2];

    // all TTS token tiles of group g of step p against bw, with no branch (tiles past the
    // chunk compute on rows that are never stored: a branch per tile would keep the
    // dequantization from being scheduled between the MFMAs); side(t) is the dequantization of
    // one B fragment (word t % 2 of row block t / 2) interleaved with tile t's MFMAs (t < 8)
    auto tiles = [&](int p, int g, Frag8 (&bw)[kSegRB][2], auto &&side) {
      const uint8_t *xs = seg_lds + (p & 1) * kStage + frow;
      const int pa = 8 * g + 2 * lg;
      const int o0 = 16 * (pa ^ lr), o1 = 16 * ((pa + 1) ^ lr);
      Frag8 xa[kSegAhead + 1][2];
#pragma unroll
      for (int t = 0; t < kSegAhead; t++) {
        xa[t][0].q = *(const uint4 *)(xs + t * 16 * 256 + o0);
        xa[t][1].q = *(const uint4 *)(xs + t * 16 * 256 + o1);
      }
#pragma unroll
      for (int t = 0; t < TTS; t++) {
        if (t + kSegAhead < TTS) {
          Frag8 *n = xa[(t + kSegAhead) % (kSegAhead + 1)];
          n[0].q = *(const uint4 *)(xs + (t + kSegAhead) * 16 * 256 + o0);
          n[1].q = *(const uint4 *)(xs + (t + kSegAhead) * 16 * 256 + o1);
        }
        const Frag8 *c = xa[t % (kSegAhead + 1)];
#pragma unroll
        for (int r = 0; r < kSegRB; r++) {
          acc[t][r] = mfma16x16x32(c[0], bw[r][0], acc[t][r]);
          acc[t][r] = mfma16x16x32(c[1], bw[r][1], acc[t][r]);
        }
        if (t < 2 * kSegRB) side(t);
#if JIT_SEG_IGLP
        // one MFMA, then three VALU instructions of the side dequantization, eight times: the
        // VALU work issues while the matrix core runs instead of between bursts of MFMAs
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < 2 * kSegRB; i++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
#endif
      }
      // (a chunk of fewer tiles than B fragments runs the rest of them after its tiles)
#pragma unroll
      for (int t = TTS; t < 2 * kSegRB; t++) side(t);
    };

    // prologue: step 0's activations and weights, step 1's weights; group 0 of step 0
    load_x(0);
    load_w(0);
    if (GP > 1) load_w(1);
    if (GP > 1)
      seg_wait_vm<kSegWLoads>();
    else
      seg_wait_vm<0>();
    seg_barrier();
#pragma unroll
    for (int r = 0; r < kSegRB; r++) dequant_rb(0, 0, r, bw0);
    for (int p = 0; p < GP; p++) {
      if (p > 0) {
        // step p's activations: the loads issued after them are step p + 1's weights
        if (p + 1 < GP)
          seg_wait_vm<kSegWLoads>();
        else
          seg_wait_vm<0>();
        seg_barrier();
      }
      if (p + 1 < GP) load_x(p + 1);
      if (p + 2 < GP) load_w(p + 2);
      tiles(p, 0, bw0, [&](int t) { dequant_word_at(p, 1, t >> 1, t & 1, bw1); });
      // step p + 1's weights: issued after them, step p + 1's activations (TTS / 2 loads) and
      // step p + 2's weights, as far as those exist
      if (p + 2 < GP)
        seg_wait_vm<kXLoads + kSegWLoads>();
      else if (p + 1 < GP)
        seg_wait_vm<kXLoads>();
      // (after the last step the dequantization below reads a stale stage and is unused)
      tiles(p, 1, bw1, [&](int t) { dequant_word_at(p + 1, 0, t >> 1, t & 1, bw0); });
    }

    // SwiGLU's sigmoid by table (qtile::swiglu_bf16_tab, exhaustively equal to the bf16 steps): every
    // wave is done with the stages, so the table (7.7 KB) takes the start of the LDS, one entry
    // or so a thread instead of ~45 instructions for each of a lane's ~40 outputs
    const uint16_t *sig_tab = (const uint16_t *)seg_lds;
    if constexpr (SWIGLU) {
      __syncthreads();
      for (int i = tid; i < qtile::kSigEntries; i += kSegThreads) ((uint16_t *)seg_lds)[i] = qtile::sigmoid_entry(i);
      __syncthreads();
    }
    // lane l holds C[token 16 t + 4 lg + i][row 16 rbk[r] + lr].  No branch per token: the
    // stores go through a buffer resource (the launch checks that the output spans less than
    // 2 GiB), and a token past the chunk gets an offset past its range, whose store is dropped.
    // (Whole tiles past the chunk are skipped: a branch uniform over the wave.)
    const __amdgpu_buffer_rsrc_t obuf = __builtin_amdgcn_make_buffer_rsrc((void *)a.out, (short)0, 0x7fffffff, 0x00020000);
    const int ntiles = (nt + 15) >> 4;
#pragma unroll
    for (int t = 0; t < TTS; t++) {
      if (t >= ntiles) continue;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int tok = 16 * t + 4 * lg + i;
        const uint32_t ro = tok < nt ? (uint32_t)(off + c0 + tok) * (uint32_t)a.N * 2u : 0x80000000u;
        if (SWIGLU) {
          __builtin_amdgcn_raw_buffer_store_b16((unsigned short)qtile::swiglu_bf16_tab(acc[t][0][i], acc[t][1][i], sig_tab), obuf,
                                                (int)(ro + 2u * (16 * rbk[0] + lr)), 0, 0);
        } else {
#pragma unroll
          for (int r = 0; r < kSegRB; r++)
            __builtin_amdgcn_raw_buffer_store_b16((unsigned short)f2bf(acc[t][r][i]), obuf,
                                                  (int)(ro + 2u * (16 * rbk[r] + lr)), 0, 0);
        }
      }
    }
  }
}

// The kernels take more LDS than the static limit: raise their dynamic limit once.
template <bool SWIGLU, bool DENSE, int TTS>
void seg_prepare() {
  static const bool done = [] {
    (void)hipFuncSetAttribute((const void *)&seg_kernel<SWIGLU, DENSE, TTS>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, seg_lds_bytes(TTS));
    return true;
  }();
  (void)done;
}

}  // namespace

extern "C" int jit_moe_gate_up_swiglu_seg(const uint16_t *x, int K, const int32_t *pair_row,
                                          const int32_t *expert_cnt, const int32_t *expert_off, int E,
                                          const void *packed, int I, int P, uint16_t *h, void *stream) {
  if (K <= 0 || I <= 0 || E <= 0 || P < 0)
    return jit::fail(JIT_EINVAL, "moe_gate_up_seg: bad dims K=%d I=%d E=%d P=%d", K, I, E, P);
  if (K % 128 != 0 || I % 128 != 0)
    return jit::fail(JIT_EUNSUPPORTED, "moe_gate_up_seg covers K %% 128 == 0 and I %% 128 == 0, got K=%d I=%d", K,
                     I);
  if (P == 0) return JIT_OK;
  if (!x || !pair_row || !expert_cnt || !expert_off || !packed || !h)
    return jit::fail(JIT_EINVAL, "moe_gate_up_seg: null pointer");
  if ((long long)P * I * 2 >= (1LL << 31))
    return jit::fail(JIT_EUNSUPPORTED, "moe_gate_up_seg: h of %d x %d bf16 exceeds 2 GiB", P, I);
  SegArgs a{x, pair_row, expert_cnt, expert_off, (const uint8_t *)packed, h, jit_q4_packed_bytes(1, 2 * I, K), K, I, 0,
            I / 128, E};
  seg_prepare<true, false, kSegTT>();
  seg_kernel<true><<<seg_grid(a.nx, E), kSegThreads, seg_lds_bytes(kSegTT), (hipStream_t)stream>>>(a);
  return jit::check_launch("jit_moe_gate_up_swiglu_seg");
}

extern "C" int jit_moe_down_seg(const uint16_t *h, int I, const int32_t *expert_cnt, const int32_t *expert_off,
                                int E, const void *packed, int D, int P, uint16_t *r, void *stream) {
  if (I <= 0 || D <= 0 || E <= 0 || P < 0)
    return jit::fail(JIT_EINVAL, "moe_down_seg: bad dims I=%d D=%d E=%d P=%d", I, D, E, P);
  if (I % 128 != 0 || D % kSegRows != 0)
    return jit::fail(JIT_EUNSUPPORTED, "moe_down_seg covers I %% 128 == 0 and D %% %d == 0, got I=%d D=%d", kSegRows,
                     I, D);
  if (P == 0) return JIT_OK;
  if (!h || !expert_cnt || !expert_off || !packed || !r) return jit::fail(JIT_EINVAL, "moe_down_seg: null pointer");
  if ((long long)P * D * 2 >= (1LL << 31))
    return jit::fail(JIT_EUNSUPPORTED, "moe_down_seg: r of %d x %d bf16 exceeds 2 GiB", P, D);
  SegArgs a{h, nullptr, expert_cnt, expert_off, (const uint8_t *)packed, r, jit_q4_packed_bytes(1, D, I), I, D, 0,
            D / kSegRows, E};
  seg_prepare<false, false, kSegTT>();
  seg_kernel<false><<<seg_grid(a.nx, E), kSegThreads, seg_lds_bytes(kSegTT), (hipStream_t)stream>>>(a);
  return jit::check_launch("jit_moe_down_seg");
}

extern "C" int jit_qmm_seg(const uint16_t *x, int T, int K, const void *packed, int N, uint16_t *y, void *stream) {
  if (T < 0 || K <= 0 || N <= 0) return jit::fail(JIT_EINVAL, "qmm_seg: bad dims T=%d K=%d N=%d", T, K, N);
  if (K % 128 != 0 || N % kSegRows != 0)
    return jit::fail(JIT_EUNSUPPORTED, "qmm_seg covers K %% 128 == 0 and N %% %d == 0, got K=%d N=%d", kSegRows, K,
                     N);
  if (T == 0) return JIT_OK;
  if (!x || !packed || !y) return jit::fail(JIT_EINVAL, "qmm_seg: null pointer");
  if ((long long)T * N * 2 >= (1LL << 31))
    return jit::fail(JIT_EUNSUPPORTED, "qmm_seg: y of %d x %d bf16 exceeds 2 GiB", T, N);
  // The chunk (token tiles per workgroup, even: the two halves of the waves stage alternate
  // tiles) is the smallest of 4, 6, 8, 10 whose workgroups fill the CUs in one round: chunks of
  // 10 can leave most CUs idle (config 3's o_proj, N = 2048 over 2,108 tokens: 112 workgroups),
  // while smaller chunks only add dequantization.  Batches too long for one round take chunks of
  // 10.
  const int nx = N / kSegRows, cus = jit::cu_count();
  auto groups = [&](int tts) { return (T + 16 * tts - 1) / (16 * tts); };
  const hipStream_t st = (hipStream_t)stream;
#define JIT_QMM_SEG(TTS)                                                                                       \
  {                                                                                                            \
    SegArgs a{x, nullptr, nullptr, nullptr, (const uint8_t *)packed, y, 0, K, N, T, nx, groups(TTS)};          \
    seg_prepare<false, true, TTS>();                                                                           \
    seg_kernel<false, true, TTS><<<seg_grid(nx, groups(TTS)), kSegThreads, seg_lds_bytes(TTS), st>>>(a);      \
  }
  if (nx * groups(4) <= cus)
    JIT_QMM_SEG(4)
  else if (nx * groups(6) <= cus)
    JIT_QMM_SEG(6)
  else if (nx * groups(8) <= cus)
    JIT_QMM_SEG(8)
  else
    JIT_QMM_SEG(10)
#undef JIT_QMM_SEG
  return jit::check_launch("jit_qmm_seg");
}
