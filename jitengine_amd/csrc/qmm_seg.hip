// Expert GEMMs over long expert segments (chunked prefill, configs with many rows
// per expert) on gfx950 matrix cores: the sorted-segment gather_qmm of the
// reference's prefill (Q36/kernels/gather_qmm_prefill.py:1-257, MLX's quantized
// block loader + tile MMA), whose arithmetic it keeps: every weight is
// dequantized to bf16, w = bf16(s * q + b), and the MMA accumulates bf16
// products in fp32.  Rows are independent, so a row's result does not depend on
// how many rows its expert has.
//
// Work split: a workgroup of 4 waves owns 256 weight rows of one expert (down:
// 16 row blocks; gate||up: 8 gate blocks and the 8 up blocks of the same output
// columns, so SwiGLU is fused) and every token of the expert's segment, in
// chunks of up to 16 * TTMAX tokens.  Each wave owns 4 row blocks.  K is walked in
// steps of one group pair (128 k): the wave dequantizes its 4 row blocks' pair
// into bf16 MFMA B fragments once (one fma and half a convert per weight) and uses
// them against every token tile of the chunk, whose activations the workgroup
// stages in LDS (gathered through pair_row for gate||up).  The next step's packed
// weights and activations are loaded while the current step computes.  fp32
// accumulators: TTMAX x 4 tiles of 16 x 16 per wave.
#include "qtile.hpp"

namespace {

constexpr int kSegWaves = 4;
constexpr int kSegRB = 4;                 // row blocks per wave
constexpr int kSegRows = 16 * kSegRB * kSegWaves;  // weight rows per workgroup
constexpr int kSegTT = 10;                // token tiles per chunk (160 tokens)
constexpr int kSegTokens = 16 * kSegTT;
#ifndef JIT_SEG_XPAD
#define JIT_SEG_XPAD 8
#endif
constexpr int kXStride = 128 + JIT_SEG_XPAD;  // LDS row stride of the staged activations (bf16)

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
// v_cvt_f32_ubyteN (the compiler would otherwise extract every nibble separately).
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
  f.v[0] = (__bf16)fmaf(s, q0, b);
  f.v[1] = (__bf16)fmaf(s, q1, b);
  f.v[2] = (__bf16)fmaf(s, q2, b);
  f.v[3] = (__bf16)fmaf(s, q3, b);
  f.v[4] = (__bf16)fmaf(s, q4, b);
  f.v[5] = (__bf16)fmaf(s, q5, b);
  f.v[6] = (__bf16)fmaf(s, q6, b);
  f.v[7] = (__bf16)fmaf(s, q7, b);
  return f;
}

// DENSE: one dense matrix (E = 1, cnt null), one token chunk per group
template <bool SWIGLU, bool DENSE = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void seg_kernel(const SegArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kSegTokens * kXStride];
  __shared__ int xrow[kSegTokens];
  int grp, cb;
  if (!seg_block(a, grp, cb)) return;  // grid padding (uniform over the workgroup)
  const int e = DENSE ? 0 : grp;
  const int cnt = DENSE ? a.T : a.cnt[e], off = DENSE ? 0 : a.off[e];
  if (cnt <= 0) return;  // uniform over the workgroup
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = lane_id();
  const int lr = l & 15, lg = l >> 4;
  const int tid = threadIdx.x;
  const int GP = a.K >> 7;  // K steps (group pairs)

  // the wave's 4 row blocks (index of the first row / 16 inside the expert's stack)
  int rbk[kSegRB];
#pragma unroll
  for (int r = 0; r < kSegRB; r++) {
    if (SWIGLU)  // gate blocks 8 cb + 2 wave + r (r < 2), and the up blocks of the same columns
      rbk[r] = (r >= 2 ? a.N / 16 : 0) + cb * 8 + 2 * wave + (r & 1);
    else
      rbk[r] = cb * 16 + 4 * wave + r;
  }
  const uint8_t *wexp = a.w + (long long)e * a.w_estride;

  // token chunks: every chunk of an expert segment in turn; one chunk (the group) of a dense batch
  const int cend = DENSE ? min(cnt, (grp + 1) * kSegTokens) : cnt;
  for (int c0 = DENSE ? grp * kSegTokens : 0; c0 < cend; c0 += kSegTokens) {
    const int nt = min(kSegTokens, cnt - c0);
    const int ntiles = (nt + 15) >> 4;
    __syncthreads();  // the previous chunk's LDS reads are done
    for (int j = tid; j < kSegTokens; j += 256) {
      const int pos = off + c0 + min(j, nt - 1);  // rows past the segment re-read its last row
      xrow[j] = a.row_index ? a.row_index[pos] : pos;
    }
    __syncthreads();

    // staging of one K step's activations: thread t moves 16 B piece (t % 16) of rows
    // t / 16 + 16 i; packed weights of one K step: per row block the pair's nibble tile
    // (16 B per lane) and its scale tile (scale pair, bias pair of row lr)
    u32x4 xv[kSegTT];
    uint4 wq[kSegRB];
    uint2 wsb[kSegRB];
    uint32_t xsrc[kSegTT];  // element offsets of this thread's pieces (x holds < 2^32 elements)
#pragma unroll
    for (int i = 0; i < kSegTT; i++) xsrc[i] = (uint32_t)xrow[(tid >> 4) + 16 * i] * (uint32_t)a.K + 8 * (tid & 15);
#define SEG_LOAD_STEP(p)                                                                                   \
  {                                                                                                        \
    _Pragma("unroll") for (int i = 0; i < kSegTT; i++) if ((tid >> 4) + 16 * i < 16 * ntiles) xv[i] =      \
        *(const u32x4 *)(a.x + xsrc[i] + 128 * (p));                                                       \
    _Pragma("unroll") for (int r = 0; r < kSegRB; r++) {                                                   \
      const uint8_t *blk = wexp + (long long)rbk[r] * GP * qtile::kTileBytes;                              \
      wq[r] = *(const uint4 *)(blk + (p) * qtile::kNibbleBytes + 16 * l);                                  \
      wsb[r] = *(const uint2 *)(blk + (long long)GP * qtile::kNibbleBytes + (p) * qtile::kScaleBytes + 8 * lr); \
    }                                                                                                      \
  }

    f32x4 acc[kSegTT][kSegRB];
#pragma unroll
    for (int t = 0; t < kSegTT; t++)
#pragma unroll
      for (int r = 0; r < kSegRB; r++) acc[t][r] = f32x4{0.f, 0.f, 0.f, 0.f};

    SEG_LOAD_STEP(0);
    for (int p = 0; p < GP; p++) {
      __syncthreads();  // every wave is done reading the previous step's activations
#pragma unroll
      for (int i = 0; i < kSegTT; i++) {
        const int row = (tid >> 4) + 16 * i;
        if (row < 16 * ntiles) *(u32x4 *)(xs + row * kXStride + 8 * (tid & 15)) = xv[i];
      }
      __syncthreads();
      uint4 cq[kSegRB];
      uint2 csb[kSegRB];
#pragma unroll
      for (int r = 0; r < kSegRB; r++) {
        cq[r] = wq[r];
        csb[r] = wsb[r];
      }
      if (p + 1 < GP) SEG_LOAD_STEP(p + 1);  // the next step's loads fly while this one computes
#pragma unroll
      for (int g = 0; g < 2; g++) {
        // B fragments of group g of the pair: row block r, half hf (k 16 lg + 8 hf .. + 8)
        Frag8 bw[kSegRB][2];
#pragma unroll
        for (int r = 0; r < kSegRB; r++) {
          const float sc = g ? bf2f_hi(csb[r].x) : bf2f(csb[r].x & 0xffffu);
          const float bi = g ? bf2f_hi(csb[r].y) : bf2f(csb[r].y & 0xffffu);
          bw[r][0] = dequant_word(g ? cq[r].z : cq[r].x, sc, bi);
          bw[r][1] = dequant_word(g ? cq[r].w : cq[r].y, sc, bi);
        }
#pragma unroll
        for (int t = 0; t < kSegTT; t++) {
          if (t < ntiles) {
            const uint16_t *xr = xs + (16 * t + lr) * kXStride + 64 * g + 16 * lg;
            Frag8 xa[2];
            xa[0].q = *(const uint4 *)xr;
            xa[1].q = *(const uint4 *)(xr + 8);
#pragma unroll
            for (int r = 0; r < kSegRB; r++) {
              acc[t][r] = mfma16x16x32(xa[0], bw[r][0], acc[t][r]);
              acc[t][r] = mfma16x16x32(xa[1], bw[r][1], acc[t][r]);
            }
          }
          // at most the next tile's activation reads ahead of its MFMAs (each tile's
          // fragments are 8 registers)
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
#undef SEG_LOAD_STEP

    // lane l holds C[token 16 t + 4 lg + i][row 16 rbk[r] + lr]
#pragma unroll
    for (int t = 0; t < kSegTT; t++) {
      if (t >= ntiles) continue;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int tok = 16 * t + 4 * lg + i;
        if (tok >= nt) continue;
        uint16_t *o = a.out + (long long)(off + c0 + tok) * a.N;
        if (SWIGLU) {
#pragma unroll
          for (int r = 0; r < 2; r++) o[16 * rbk[r] + lr] = (uint16_t)qtile::swiglu_bf16(acc[t][r][i], acc[t][r + 2][i]);
        } else {
#pragma unroll
          for (int r = 0; r < kSegRB; r++) o[16 * rbk[r] + lr] = (uint16_t)f2bf(acc[t][r][i]);
        }
      }
    }
  }
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
  SegArgs a{x, pair_row, expert_cnt, expert_off, (const uint8_t *)packed, h, jit_q4_packed_bytes(1, 2 * I, K), K, I, 0,
            I / 128, E};
  seg_kernel<true><<<seg_grid(a.nx, E), 256, 0, (hipStream_t)stream>>>(a);
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
  SegArgs a{h, nullptr, expert_cnt, expert_off, (const uint8_t *)packed, r, jit_q4_packed_bytes(1, D, I), I, D, 0,
            D / kSegRows, E};
  seg_kernel<false><<<seg_grid(a.nx, E), 256, 0, (hipStream_t)stream>>>(a);
  return jit::check_launch("jit_moe_down_seg");
}

extern "C" int jit_qmm_seg(const uint16_t *x, int T, int K, const void *packed, int N, uint16_t *y, void *stream) {
  if (T < 0 || K <= 0 || N <= 0) return jit::fail(JIT_EINVAL, "qmm_seg: bad dims T=%d K=%d N=%d", T, K, N);
  if (K % 128 != 0 || N % kSegRows != 0)
    return jit::fail(JIT_EUNSUPPORTED, "qmm_seg covers K %% 128 == 0 and N %% %d == 0, got K=%d N=%d", kSegRows, K,
                     N);
  if (T == 0) return JIT_OK;
  if (!x || !packed || !y) return jit::fail(JIT_EINVAL, "qmm_seg: null pointer");
  const int chunks = (T + kSegTokens - 1) / kSegTokens;
  SegArgs a{x, nullptr, nullptr, nullptr, (const uint8_t *)packed, y, 0, K, N, T, N / kSegRows, chunks};
  seg_kernel<false, true><<<seg_grid(a.nx, chunks), 256, 0, (hipStream_t)stream>>>(a);
  return jit::check_launch("jit_qmm_seg");
}
