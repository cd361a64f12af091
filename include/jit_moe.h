/*
 * jit_moe.h -- C-ABI of the MI355X (gfx950) ragged-batch MoE decode step.
 *
 * One shared library (jitengine_amd/_lib/libjit_moe.so) exports these entry
 * points.  They replace the Metal kernels of JITEngine's hot path; each
 * declaration names the reference interface it stands in for (paths relative to
 * the reference repository; Q36 = engines/qwen3.6-35b-a3b-m4pro/src/
 * jitengine_qwen3_6_35b_a3b_m4pro, FN = engines/qwen3.8-flash-next-m4pro/src/
 * jitengine_qwen3_8_flash_next_m4pro, FL = engines/flint-m4pro/src/
 * jitengine_flint_m4pro).
 *
 * Conventions
 *  - Every pointer argument is a device pointer unless its name ends in _host.
 *  - bf16 tensors are uint16_t bit patterns; all tensors are dense row-major.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *  - Entry points check their scalar contract on the host before any launch and
 *    return JIT_EINVAL (contract break, the reference's ValueError) or
 *    JIT_EUNSUPPORTED (a shape outside the kernel's coverage, where the
 *    reference would take its stock MLX fallback); JIT_ELAUNCH reports a HIP
 *    launch failure.  jit_last_error() describes the last failure on the
 *    calling thread.
 *  - No entry point allocates device memory: workspaces are arguments (or, for
 *    jit_paged_decode_attn_noalloc, a fixed array inside the library).
 *  - Calls are asynchronous on `stream`; device-side contents (expert ids,
 *    page ids) are trusted, as the reference's kernels trust theirs
 *    ("entry points validate nothing; callers gate them", FN/kernels/README.md:4).
 *
 * MLX 4-bit affine layout (Q36/linear.py:101-128): a quantized matrix [N, K] is
 * w uint32 [N, K/8] (element j = nibble j%8 of word j/8, low nibble first),
 * scales and biases bf16 [N, K/64]; value = scale * q + bias.  An expert stack
 * prepends an expert axis [E, N, ...].
 */
#ifndef JIT_MOE_H
#define JIT_MOE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JIT_OK 0
#define JIT_EINVAL (-1)
#define JIT_EUNSUPPORTED (-2)
#define JIT_ELAUNCH (-3)

/* Paged KV pool geometry fixed by the kernels. */
#define JIT_PAGE_TOKENS 16
#define JIT_HEAD_DIM 128

/* Human-readable description of the last error returned on this thread. */
const char *jit_last_error(void);

/* Library version (monotonic integer). */
int jit_version(void);

/* ---------------------------------------------------------------- router --
 * router_topk(logits[..., N] bf16, k, norm) -> (inds uint32[..., k],
 * scores bf16[..., k]): softmax (fp32, stored bf16), exact top-k by rank in
 * ascending (value, index) order, gathered gates, optional renormalisation by
 * their sequential bf16 sum.
 * Replaces Q36/kernels/router_topk.py:177-192 (router_topk) and the stock chain
 * of Q36/model/moe.py:304-315.  Contract: rows >= 0, 0 < k <= N (else
 * JIT_EINVAL, Q36/kernels/router_topk.py:41-42); N % 32 == 0 and N <= 1024
 * (else JIT_EUNSUPPORTED, router_supported :171-174).
 * gates_out (optional, may be NULL): the bf16 gates [rows, N]. */
int jit_router_topk(const uint16_t *logits, int rows, int N, int k, int norm, uint32_t *inds,
                    uint16_t *scores, uint16_t *gates_out, void *stream);

/* topk(gates, k): the rank top-k alone on given bf16 gates [rows, N].
 * Replaces Q36/kernels/router_topk.py:36-66 (topk / topk_stable).
 * Contract: 0 < k <= N (JIT_EINVAL); N <= 1024 (JIT_EUNSUPPORTED). */
int jit_topk(const uint16_t *gates, int rows, int N, int k, uint32_t *inds, void *stream);

/* --------------------------------------------------------------- packing --
 * Token-to-expert packing of the P = rows*k flat (row, slot) pairs of inds:
 * a stable sort by expert id.  Replaces Q36/model/moe.py:151-159 (_sort_pairs:
 * argsort, inverse argsort, order // k) and FN/model/moe/expert_mlp.py:39-49,
 * 147-163 (stable argsort + np.unique -> seg_slot, seg_start, seg_cnt,
 * pair_row).  Outputs (int32):
 *   order[P]      flat pair index at sorted position p
 *   pair_row[P]   order[p] / k (the activation row of sorted position p)
 *   inv[P]        sorted position of flat pair f
 *   expert_cnt[E], expert_off[E]    pairs per expert and first sorted position
 *   seg_expert[E], seg_start[E], seg_cnt[E]   the first meta[0] entries list
 *                 the non-empty experts in ascending order (the entries past
 *                 them are not written)
 *   meta[4]       {n_seg, max_cnt, bad_ids, 0}; bad_ids counts ids >= E (such
 *                 pairs are dropped: they appear in no segment)
 * Contract: P >= 0, k > 0, 0 < E <= 1024. */
int jit_moe_pack(const uint32_t *inds, int P, int k, int E, int32_t *order, int32_t *pair_row,
                 int32_t *inv, int32_t *expert_cnt, int32_t *expert_off, int32_t *seg_expert,
                 int32_t *seg_start, int32_t *seg_cnt, int32_t *meta, void *stream);

/* Bytes of device workspace jit_moe_pack_ws takes for P pairs over E experts: 4 (E + 1) per tile of
 * 1024 pairs when P > 2048 and E < 1024, else 0 (no workspace needed). */
long long jit_moe_pack_workspace_bytes(int P, int E);

/* jit_moe_pack with a device workspace of jit_moe_pack_workspace_bytes(P, E) bytes (contents on
 * entry do not matter): a long batch (a chunked-prefill step's B * k pairs,
 * Q36/model/moe.py:151-159 over the prefill rows) is packed by many workgroups in three launches
 * -- per-tile expert counts, one scan, per-tile placement -- instead of one workgroup walking every
 * tile.  The same tables, bit for bit (the stable order is unique).  With a workspace of 0 bytes
 * needed it is jit_moe_pack; a smaller workspace than needed returns JIT_EINVAL. */
int jit_moe_pack_ws(const uint32_t *inds, int P, int k, int E, int32_t *order, int32_t *pair_row, int32_t *inv,
                    int32_t *expert_cnt, int32_t *expert_off, int32_t *seg_expert, int32_t *seg_start,
                    int32_t *seg_cnt, int32_t *meta, void *workspace, long long workspace_bytes, void *stream);

/* The router top-k of at most 4 rows followed by their packing, in one launch: the same
 * outputs, bit for bit, as jit_router_topk (inds [rows, k], scores) then jit_moe_pack over
 * P = rows * k pairs of E = N experts (their two contracts, plus rows <= 4 and N <= 128:
 * JIT_EUNSUPPORTED otherwise).  For the decode step of one sequence (the reference's solo path,
 * Q36/model/moe.py:304-315 then :151-159), where the second launch costs as much as the work. */
int jit_route_pack(const uint16_t *logits, int rows, int N, int k, int norm, uint32_t *inds, uint16_t *scores,
                   int32_t *order, int32_t *pair_row, int32_t *inv, int32_t *expert_cnt, int32_t *expert_off,
                   int32_t *seg_expert, int32_t *seg_start, int32_t *seg_cnt, int32_t *meta, void *stream);

/* ------------------------------------------------ quantized projections --
 * Dense 4-bit projection y[T, N] = x[T, K] . dequant(W[N, K])^T, fp32
 * accumulation, bf16 out: QLinear.__call__ / .rows (Q36/linear.py:219-313,
 * the qmv arithmetic of Q36/kernels/qmv_mrow.py), used for the router logits
 * (Q36/model/moe.py:296-302) and the attention projections.
 * Contract: T >= 0, N % 16 == 0, K % 256 == 0, K <= 4096 (JIT_EUNSUPPORTED
 * otherwise). */
int jit_qmm(const uint16_t *x, int T, int K, const uint32_t *w, const uint16_t *scales,
            const uint16_t *biases, int N, uint16_t *y, void *stream);

/* Packed tile layout of a quantized stack (the build's MI355X layout; no
 * counterpart in the reference, whose loader keeps the MLX layout,
 * Q36/linear.py:101-128).  The same bytes as the MLX layout, reordered once at
 * load time: per (expert, block of 16 rows) GP = K / 128 nibble tiles of 1 KB,
 * one per pair of groups -- 64 lanes x 16 B of nibble words in the order the
 * MFMA B operand consumes them (lane 16*j + r: words 2j, 2j+1 of the pair's
 * first group and 2j, 2j+1 of its second group, row r; each word's nibbles
 * reordered to q0 q2 q4 q6 q1 q3 q5 q7) -- followed by GP scale tiles of 128 B,
 * 16 rows x (scale pair, bias pair) bf16.  A wave reads a nibble tile with one
 * fully coalesced 1 KB load and the scales of 4 consecutive pairs with one 512 B
 * load (the MLX layout in MFMA fragment order is read in 32-byte pieces per row,
 * which caps HBM reads well below the streaming rate).
 * jit_q4_packed_bytes: bytes of the packed stack [E, N, K] (-1 if N % 16 or
 * K % 128 != 0).  jit_q4_prepack: w, scales, biases (MLX layout) -> packed. */
int64_t jit_q4_packed_bytes(int E, int N, int K);
int jit_q4_prepack(const uint32_t *w, const uint16_t *scales, const uint16_t *biases, int E, int N,
                   int K, void *packed, void *stream);

/* jit_qmm on a packed matrix (bitwise jit_qmm's result on the same weights). */
int jit_qmm_packed(const uint16_t *x, int T, int K, const void *packed, int N, uint16_t *y,
                   void *stream);

/* Grouped gate||up projection with fused SwiGLU over packed pairs:
 * for every sorted pair p of expert e, g, u = x[pair_row[p]] . dequant(Wgu_e)^T
 * (gate rows [0, I), up rows [I, 2I) of the fused [E, 2I, K] stack),
 * h[p] = bf16(bf16(g * sigmoid(g)) * u) with g, u and sigmoid(g) rounded to bf16.
 * Replaces expert_gate_up_exact(_rows) (Q36/kernels/expert_solo.py:67-116,
 * 213-232,359-401), the stock gate_up.gather + swiglu (Q36/model/moe.py:
 * 191-193, Q36/kernels/elementwise.py:14-15) and FN's grouped_swiglu
 * (FN/kernels/grouped_expert_qmv.py:345-371).  x [B, K] bf16; h [P, I] bf16 in
 * sorted pair order.  Contract: I % 16 == 0, K % 512 == 0, K <= 4096, 0 < E.
 * Expert segments come from jit_moe_pack (expert_cnt, expert_off, pair_row). */
int jit_moe_gate_up_swiglu(const uint16_t *x, int K, const int32_t *pair_row,
                           const int32_t *expert_cnt, const int32_t *expert_off, int E,
                           const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
                           int I, int P, uint16_t *h, void *stream);

/* The same on a packed [E, 2I, K] stack (bitwise the unpacked call's result). */
int jit_moe_gate_up_swiglu_packed(const uint16_t *x, int K, const int32_t *pair_row,
                                  const int32_t *expert_cnt, const int32_t *expert_off, int E,
                                  const void *packed, int I, int P, uint16_t *h, void *stream);

/* One token's routing and its gate||up in one launch: jit_route_pack for one row (the top-k of
 * logits [E] with renormalisation when norm != 0, Q36/kernels/router_topk.py:72-192, and the
 * packing of its k pairs, Q36/model/moe.py:129-159) followed by jit_moe_gate_up_swiglu_packed of
 * x [1, K] -- the same bits, one launch fewer.  Every workgroup takes the top-k itself (no
 * exchange); the launch also writes jit_route_pack's outputs (inds [k], scores [k] and the packing
 * tables, as for one row) for the down and combine launches that read them.  h [k, I] in sorted
 * pair order.  Contract: K % 512 == 0, K <= 4096, I % 16 == 0, E % 32 == 0, E <= 128, 0 < k < E,
 * k <= 64 (JIT_EINVAL / JIT_EUNSUPPORTED). */
int jit_moe_gate_up_swiglu_routed_packed(const uint16_t *x, int K, const uint16_t *logits, int E, int k,
                                         int norm, const void *packed, int I, uint16_t *h, uint32_t *inds,
                                         uint16_t *scores, int32_t *order, int32_t *pair_row, int32_t *inv,
                                         int32_t *expert_cnt, int32_t *expert_off, int32_t *seg_expert,
                                         int32_t *seg_start, int32_t *seg_cnt, int32_t *meta, void *stream);

/* Elementwise SwiGLU of bf16 gate and up values: h[i] = bf16(bf16(g[i] * SigmoidX(g[i])) * u[i]),
 * SigmoidX's steps each rounded to bf16 (e = bf16(exp|g|), d = bf16(1 + e), y = bf16(1 / d),
 * g < 0 ? y : bf16(1 - y)) -- exactly the epilogue of jit_moe_gate_up_swiglu* on given operands.
 * Replaces the stock swiglu (Q36/kernels/elementwise.py:14-15, nn.silu(gate) * x in bf16, used by
 * Q36/model/moe.py:189-197).  g, u, h: n bf16 values, 16-byte aligned.  NaN inputs give NaN
 * outputs (payload bits unspecified). */
int jit_swiglu(const uint16_t *g, const uint16_t *u, int64_t n, uint16_t *h, void *stream);

/* Grouped down projection over packed pairs: r[p] = bf16(h[p] . dequant(Wd_e)^T)
 * for every sorted pair p of expert e (the down gather of Q36/model/moe.py:193;
 * the per-expert GEMV inside expert_down_exact(_par),
 * Q36/kernels/expert_solo.py:118-164,262-356).  h [P, I], r [P, D] bf16.
 * Contract: D % 16 == 0, I % 256 == 0, I <= 2048. */
int jit_moe_down(const uint16_t *h, int I, const int32_t *expert_cnt, const int32_t *expert_off,
                 int E, const uint32_t *w, const uint16_t *scales, const uint16_t *biases, int D,
                 int P, uint16_t *r, void *stream);

/* The same on a packed [E, D, I] stack (bitwise the unpacked call's result). */
int jit_moe_down_packed(const uint16_t *h, int I, const int32_t *expert_cnt,
                        const int32_t *expert_off, int E, const void *packed, int D, int P,
                        uint16_t *r, void *stream);

/* Expert GEMMs for long expert segments (chunked prefill: at least 4 pairs per
 * expert on average, the reference's switch in Q36/model/moe.py:161-175): the
 * sorted-segment gather_qmm of Q36/kernels/gather_qmm_prefill.py:1-257
 * (seg_gather_qmm), on matrix-core tiles.  Its arithmetic is that of the
 * reference's tile GEMM (MLX's quantized block loader): every weight is
 * dequantized to bf16, w = bf16(fma(s, q, b)), and bf16 products accumulate in
 * fp32; rows are independent.  Packed stacks only (jit_q4_prepack).
 * Segments, pair_row and the sorted output order are those of
 * jit_moe_gate_up_swiglu / jit_moe_down.
 * gate||up + SwiGLU: x [B, K] -> h [P, I]; contract K % 128 == 0, I % 128 == 0.
 * down: h [P, I] -> r [P, D]; contract I % 128 == 0, D % 256 == 0. */
int jit_moe_gate_up_swiglu_seg(const uint16_t *x, int K, const int32_t *pair_row,
                               const int32_t *expert_cnt, const int32_t *expert_off, int E,
                               const void *packed, int I, int P, uint16_t *h, void *stream);
int jit_moe_down_seg(const uint16_t *h, int I, const int32_t *expert_cnt, const int32_t *expert_off,
                     int E, const void *packed, int D, int P, uint16_t *r, void *stream);

/* A prefill-sized dense projection y[T, N] = x[T, K] . W[N, K]^T on the segment GEMM's
 * tiles, with its arithmetic: bf16-dequantized weights, fp32 accumulate -- that of
 * MLX's affine_qmm_t for long inputs, which the reference's dense prefill kernel keeps
 * (Q36/kernels/qmm_prefill.py:1-6,86-90; called from QLinear.__call__,
 * Q36/linear.py:219-231).  W packed (jit_q4_prepack); the token chunks are spread over
 * workgroups.  Contract: K % 128 == 0, N % 256 == 0. */
int jit_qmm_seg(const uint16_t *x, int T, int K, const void *packed, int N, uint16_t *y, void *stream);

/* Weighted combine in slot order: y[b] = sum_j bf16(r[inv[b*k+j]] * score[b, j])
 * with each product rounded to bf16 and a sequential bf16 sum over j = 0..k-1
 * (Q36/kernels/expert_solo.py:1-6,155-163,307-315; stock
 * (e * scores[..., None]).sum(-2), Q36/model/moe.py:286).  With resid != NULL,
 * y[b] = bf16(resid[b] + that sum) (with_residual, Q36/model/moe.py:119-123). */
int jit_moe_combine(const uint16_t *r, const int32_t *inv, const uint16_t *scores, int B, int k,
                    int D, const uint16_t *resid, uint16_t *y, void *stream);

/* jit_moe_combine followed by jit_rmsnorm of its output y with weight w (the
 * next decoder layer's input norm, Q36/model/model.py:65-80) in one launch: y as
 * jit_moe_combine writes it and xn = rmsnorm(y) * w, bit for bit the two calls.
 * Contract: that of both calls (D % 8 == 0, D <= 2048). */
int jit_moe_combine_rmsnorm(const uint16_t *r, const int32_t *inv, const uint16_t *scores, int B, int k,
                            int D, const uint16_t *resid, uint16_t *y, const uint16_t *w, float eps,
                            uint16_t *xn, void *stream);

/* ----------------------------------------------------- decoder block glue --
 * RMSNorm of rows x [rows, D] (mx.fast.rms_norm as the decoder layer applies it,
 * Q36/model/model.py:65-80; Q36/model/attention.py:59-60): sum(x^2) in fp32,
 * y = bf16(w * bf16(x * rsqrt(mean + eps))).  With resid != NULL the normed row
 * is h = bf16(x + resid) (the residual add in front of the post-attention
 * norm), written to h_out when that is not NULL.  Contract: D % 8 == 0,
 * D <= 2048. */
int jit_rmsnorm(const uint16_t *x, const uint16_t *resid, int rows, int D, const uint16_t *w,
                float eps, uint16_t *h_out, uint16_t *y, void *stream);

/* One row's residual add and RMSNorm in front of a packed projection, in one launch
 * (jit_rmsnorm with resid followed by jit_qmm_packed of its output, for a one-token step; the
 * post-attention norm and the router projection, Q36/model/model.py:65-80 and
 * Q36/model/moe.py:161-165): h_out = bf16(a_row + resid), hn_out = rmsnorm(h_out) * w and
 * y = hn_out . W^T, each bit for bit what the two calls write.  a_row, resid, w, h_out,
 * hn_out: D bf16; W packed [N, D] (jit_q4_prepack); y: N bf16.
 * Contract: D % 256 == 0, D <= 2048, N % 16 == 0 (JIT_EUNSUPPORTED). */
int jit_qmm_packed_add_rmsnorm(const uint16_t *a_row, const uint16_t *resid, const uint16_t *w, float eps, int D,
                               const void *packed, int N, uint16_t *h_out, uint16_t *hn_out, uint16_t *y,
                               void *stream);

/* One row's MoE combine and the next layer's input RMSNorm in front of that layer's packed qkv
 * projection, in one launch (jit_moe_combine_rmsnorm for B = 1 followed by jit_qmm_packed of its
 * normed row; Q36/model/moe.py:119-123,286, Q36/model/model.py:65-80, Q36/model/attention.py:99):
 * y_out = the combined row as jit_moe_combine writes it (resid may be NULL) and
 * out = rmsnorm(y_out) * w . W^T, each bit for bit what the two calls write.  r, inv, scores, k:
 * as jit_moe_combine with B = 1; W packed [N, D].
 * Contract: D % 256 == 0, D <= 2048, N % 16 == 0, k > 0 (JIT_EUNSUPPORTED / JIT_EINVAL). */
int jit_qmm_packed_combine_rmsnorm(const uint16_t *r, const int32_t *inv, const uint16_t *scores, int k,
                                   const uint16_t *resid, const uint16_t *w, float eps, int D, const void *packed,
                                   int N, uint16_t *y_out, uint16_t *out, void *stream);

/* The attention block between the qkv projection and attention
 * (Qwen3_5MoeAttention.step, Q36/model/attention.py:99-119, without the output
 * gate, which the BASELINE geometry does not have): qkv [B, (H + 2 Hkv) * 128]
 * (q heads, then k heads, then v heads); per head RMSNorm with q_norm_w /
 * k_norm_w [128]; RoPE with traditional = False on q and k (pairs (i, i + 64),
 * angle fp32(pos[b]) * inv_freq[i], inv_freq [64] fp32 = base^(-2i/128));
 * q -> q_out [B, H, 128]; k, v -> the paged pool at position pos[b] (the KV
 * append of KVSlot.append, Q36/kvcache/kv_cache.py:76-85). */
int jit_qk_norm_rope_append(const uint16_t *qkv, int B, int H, int Hkv, const uint16_t *q_norm_w,
                            const uint16_t *k_norm_w, float eps, const float *inv_freq,
                            const int32_t *pos, const int32_t *page_table, int max_pages,
                            uint16_t *pool, uint16_t *q_out, void *stream);

/* --------------------------------------------------------- paged KV pool --
 * Pool layout (the build's design; the reference keeps one contiguous
 * [1, Hkv, cap, Dh] buffer per request, Q36/kvcache/kv_cache.py:27-85):
 * pool [num_pages, Hkv, 2, 16 * 128] bf16 per layer; for each kv head, part 0
 * of a page holds K chunk-major ([d / 32][slot][d % 32]: an MFMA fragment's 16
 * slots x 32 dims are 1 KB contiguous) and part 1 holds V dim-major
 * ([d][slot]), so one kv head's K and V are one contiguous 8 KiB block.  Token
 * t of sequence b is at page page_table[b * max_pages + t / 16], slot t % 16.
 *
 * KV append: write k, v [B, Hkv, 128] of row b at position pos[b]
 * (KVSlot.append, Q36/kvcache/kv_cache.py:76-85).  Contract: Dh == 128. */
int jit_kv_append_paged(const uint16_t *k, const uint16_t *v, int B, int Hkv, const int32_t *pos,
                        const int32_t *page_table, int max_pages, uint16_t *pool, void *stream);

/* Host-only split plan for paged decode attention: sequence b is cut into
 * ceil(lens_host[b] / chunk) chunks of jit_attn_chunk_tokens(lens_host[b])
 * keys, a pure function of the sequence's own length, so a row's result never
 * depends on the rest of the batch (the property of FL/kernels/plan.py:50-57
 * and Q36T/metal/engine/test_engine_consistency.py:43).  Fills
 * chunk_start_host[B + 1] (exclusive prefix) and, when chunk_seq_host is not
 * NULL, chunk_seq_host[c] = the sequence of chunk c (at most seq_cap entries);
 * returns the total chunk count, negative on a contract break (lens < 1, or
 * seq_cap too small). */
int jit_attn_chunk_tokens(int len);
int jit_attn_plan(const int32_t *lens_host, int B, int32_t *chunk_start_host,
                  int32_t *chunk_seq_host, int seq_cap);

/* Workspace bytes jit_paged_decode_attn needs for `total_chunks` chunks. */
int64_t jit_attn_workspace_bytes(int total_chunks, int H);

/* Paged GQA decode attention, one query per row: out[b, h] =
 * softmax(scale * q[b, h] . K_b^T) . V_b over the first lens[b] tokens of
 * sequence b, q head h reading kv head h / (H / Hkv).  Split-K over the key
 * length with fp32 (max, sum, o) partials merged in chunk order.
 * Replaces sdpa_decode / sdpa_decode_rows (Q36/kernels/sdpa_decode.py:448-476,
 * the one- and two-pass kernels :16-74,217-315) and the split-K attention phase
 * of Flint (FL/kernels/plan.py:42-59).  q, out [B, H, 128] bf16; chunk_start
 * [B + 1] and chunk_seq [total_chunks] int32 (device copies of jit_attn_plan's
 * output for these lens); workspace of jit_attn_workspace_bytes(total_chunks, H)
 * bytes.  The pool must hold finite values in every slot of the pages read
 * (the build's pool is zero-initialised).
 * Contract: H % Hkv == 0, H / Hkv <= 16, Dh == 128, B >= 0 (JIT_EINVAL /
 * JIT_EUNSUPPORTED, the checks of Q36/kernels/sdpa_decode.py:77-116). */
int jit_paged_decode_attn(const uint16_t *q, const uint16_t *pool, const int32_t *page_table,
                          int max_pages, const int32_t *lens, const int32_t *chunk_start,
                          const int32_t *chunk_seq, int B, int H, int Hkv, float scale,
                          int total_chunks, void *workspace, uint16_t *out, void *stream);

/* jit_paged_decode_attn fused with the step's own token's jit_qk_norm_rope_append: qkv holds
 * the step's raw rows [B, (H + 2 Hkv) * 128] (the qkv projection's output) instead of q.  Row b's
 * token sits at position lens[b] - 1: its q heads are normed and rotated inside the attention
 * kernel, and its K (normed, rotated) and V are written into the pool at that position through
 * page_table row b before any read of that slot -- the bits of jit_qk_norm_rope_append followed
 * by jit_paged_decode_attn, one launch fewer.  Replaces the same reference calls as the two
 * (Q36/model/attention.py:99-119, Q36/kvcache/kv_cache.py:27-85, Q36/kernels/sdpa_decode.py:448-476).
 * inv_freq [64] fp32; q_norm_w, k_norm_w [128] bf16.  Contract as jit_paged_decode_attn. */
int jit_paged_decode_attn_qkv(const uint16_t *qkv, const uint16_t *q_norm_w, const uint16_t *k_norm_w,
                              float eps, const float *inv_freq, uint16_t *pool, const int32_t *page_table,
                              int max_pages, const int32_t *lens, const int32_t *chunk_start,
                              const int32_t *chunk_seq, int B, int H, int Hkv, float scale,
                              int total_chunks, void *workspace, uint16_t *out, void *stream);

/* jit_paged_decode_attn without a workspace argument: the same kernels and the same bits,
 * with the fp32 split-K partials in a file-scope device array of JIT_ATTN_SCRATCH_BYTES
 * (16 MiB) that each GPU holds from the library's first call on it until the process ends.
 * No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 * calls no allocating routine.  Limit: jit_attn_workspace_bytes(total_chunks, H) <=
 * JIT_ATTN_SCRATCH_BYTES (about 1,000 chunks at H = 32), else JIT_EUNSUPPORTED before any
 * launch.  The scratch address is taken for the device current at the call (the stream must
 * belong to it).  All calls on one GPU share its array: calls that overlap in time on one GPU
 * (other streams, other threads) race on it; calls in one stream are ordered and safe.
 * Nothing in the array needs clearing: each call writes every partial it reads. */
#define JIT_ATTN_SCRATCH_BYTES (16 << 20)
int jit_paged_decode_attn_noalloc(const uint16_t *q, const uint16_t *pool, const int32_t *page_table,
                                  int max_pages, const int32_t *lens, const int32_t *chunk_start,
                                  const int32_t *chunk_seq, int B, int H, int Hkv, float scale,
                                  int total_chunks, uint16_t *out, void *stream);

/* Causal attention of prefill chunks over the paged pool: the other half of a
 * chunked-prefill step (mx.fast.scaled_dot_product_attention with mask = "causal"
 * over the slot's keys, Q36/model/attention.py:70-74, after the chunk's KV append).
 * Chunk c owns q rows chunk_row[c] .. + chunk_len[c] - 1 of q [T, H, 128] (normed,
 * rotated); its token t sits at position chunk_ctx[c] + t of sequence chunk_seq[c]
 * and attends keys 0 .. chunk_ctx[c] + t (the pool must hold them: the chunk's own
 * keys appended).  A token's keys are cut into parts at multiples of
 * jit_prefill_part_keys() (6,144): a token at position pos has pos / 6144 + 1 parts.
 * Work items: nblk (chunk, first token, part) triples blk_chunk, blk_q0, blk_part --
 * row blocks of jit_prefill_block_tokens(H, Hkv) tokens, each with one item per part
 * that holds a key of its last token -- covering every chunk (any order; longest
 * first balances best).  pmax = the most parts of any token; max_len = the longest
 * chunk.  Tokens of one part are written by their item; the others leave fp32
 * partials in workspace (jit_prefill_workspace_bytes(T, pmax, H) bytes, T = the q
 * rows; unused and may be null when pmax == 1), which a second launch merges in part
 * order.  out [T, H, 128] bf16; fp32 online softmax.
 * Contract: H % Hkv == 0, pmax >= 1 (JIT_EINVAL), H / Hkv divides 16, H <= 64 when
 * pmax > 1 (JIT_EUNSUPPORTED).  Any context length. */
int jit_prefill_block_tokens(int H, int Hkv);
int jit_prefill_part_keys(void);
/* Bytes of the partials' workspace: T * pmax * H * 132 * 4 when pmax > 1, 0 when pmax == 1,
 * -1 for T < 0, pmax < 1 or H <= 0. */
long long jit_prefill_workspace_bytes(int T, int pmax, int H);
int jit_paged_prefill_attn(const uint16_t *q, const uint16_t *pool, const int32_t *page_table,
                           int max_pages, const int32_t *chunk_seq, const int32_t *chunk_ctx,
                           const int32_t *chunk_len, const int32_t *chunk_row, int C,
                           const int32_t *blk_chunk, const int32_t *blk_q0, const int32_t *blk_part,
                           int nblk, int pmax, int max_len, int H, int Hkv, float scale,
                           void *workspace, uint16_t *out, void *stream);

/* ------------------------------------------------------------------ step ends and KV pages */

/* Embedding lookup of MLX 4-bit affine rows: out[b] = dequantize(weight[ids[b]]) [B, D] bf16,
 * weight [V, D/8] u32 (nibble i of word j = column 8j + i), scales/biases [V, D/64] bf16, each
 * value bf16(bf16(scale * q) + bias) -- mx.dequantize in bf16 arithmetic
 * (QEmbedding.lookup, Q36/linear.py:680-690).  An id outside [0, V) gives a zero row (callers
 * validate token ids on the host).  Contract: D % 64 == 0 (JIT_EUNSUPPORTED). */
int jit_embed_q4(const int32_t *ids, int B, const uint32_t *weight, const uint16_t *scales,
                 const uint16_t *biases, int V, int D, uint16_t *out, void *stream);

/* Token sampling over rows of bf16 logits [B, V] (Q36/sampler.py).  Up to 64 rows are split
 * over slices of each row, one workgroup a slice, with partials and the draws' histograms in a
 * workspace: the caller's (the _ws entry points, jit_sampler_workspace_bytes() bytes, 16-byte
 * aligned, contents on entry do not matter) or, for the entry points without one, a static device
 * buffer of the same size (8.1 MiB, held on each device the library runs on until the process
 * ends).  Calls that share a workspace -- or the static buffer -- and overlap in time race: give
 * concurrent streams workspaces of their own.  More than 64 rows take one workgroup a row and
 * use no workspace.
 * Shared definitions:
 *   lse  = bf16(m0 + ln(S 2^-42)), m0 the row's largest logit and S = sum floor(e^(x - m0) 2^42);
 *   lp   = bf16(x - lse) (logprobs_from_logits, Q36/sampler.py:295-297).
 * The sums are exact integers, so results do not depend on the order of the additions; the
 * reference's fp32 reductions (MLX's logsumexp, cumsum and sum orders) are not restated.
 * Contract: 1 <= V <= 2^19 (JIT_EUNSUPPORTED beyond); finite or -inf logits with at least one
 * finite value per row (other rows give unspecified tokens, never a fault). */

/* lp [B, V] bf16 = the rows' log-probabilities as defined above. */
int jit_logprobs_rows(const uint16_t *logits, int B, int V, uint16_t *lp, void *stream);

/* Bytes of the workspace the _ws sampling entry points take (the split launches' partials). */
long long jit_sampler_workspace_bytes(void);

/* jit_logprobs_rows, jit_argmax_rows and jit_sample_rows with a caller's workspace of at least
 * jit_sampler_workspace_bytes() bytes (JIT_EINVAL if smaller or not 16-byte aligned; NULL takes the
 * static buffer): the same kernels and the same results, for callers that run samplers on several
 * streams at once.  No counterpart in the reference, whose MLX ops allocate per call. */
int jit_logprobs_rows_ws(const uint16_t *logits, int B, int V, uint16_t *lp, void *workspace,
                         long long workspace_bytes, void *stream);
int jit_argmax_rows_ws(const uint16_t *logits, int B, int V, int32_t *out, void *workspace,
                       long long workspace_bytes, void *stream);
int jit_sample_rows_ws(const uint16_t *logits, int B, int V, double temperature, double top_p, int top_k,
                       const float *u, int32_t *tokens, void *workspace, long long workspace_bytes,
                       void *stream);

/* Greedy choice: out[b] = the first index of the largest lp of row b (Sampler.__call__ with
 * temperature 0: mx.argmax of the log-probabilities, Q36/sampler.py:371-374).  The bf16
 * rounding of x - lse can tie logits that differ, so this is not always the argmax of the
 * logits themselves. */
int jit_argmax_rows(const uint16_t *logits, int B, int V, int32_t *out, void *stream);

/* One draw per row under shared settings (the rows of a Sampler.rows_key group,
 * Q36/sampler.py:479-483): temperature <= 0 is the greedy choice above; otherwise, with
 * inv_t = bf16(fp32(1 / temperature)) and thr = bf16(fp32(1 - top_p)):
 *   order   ascending (lp, index), -0 tying +0 (the stable argsort, :458-459);
 *   top_p   in (0, 1): position r survives iff bf16(sum_{r' <= r} floor(bf16(e^lp) 2^42) 2^-42)
 *           > thr (apply_top_p, :300-312; _sample_exact_full, :460-462); outside (0, 1) all survive;
 *   top_k   in [1, V): of the survivors, the k largest by (value desc, index asc) (apply_top_k,
 *           :315-318; _sample_exact_full's cut, :463-469); 0 or >= V: all survivors;
 *   weights x = bf16(lp inv_t) of the kept, m = max x, W = floor(e^(x - m) 2^42), 0 elsewhere;
 *   draw    C_i = sum_{j < i} W_j, U = floor(u' 2^32 sum(W) 2^-32) with u' = u[b] clamped to
 *           [0, 1 - 2^-24]; tokens[b] = the last i with C_i <= U (the categorical draw as
 *           searchsorted(cdf, u * sum(w), "right") - 1, :470-476).
 * Where no position survives top_p (bf16 mass below 1 - top_p: top_p under about 0.03) the
 * greedy token is drawn; the reference's chains disagree among themselves there.
 * u: [B] fp32 uniforms on the device (jit_threefry_uniform); unused when greedy.
 * Contract breaks (JIT_EINVAL): NaN settings, top_k < 0, null uniforms when sampling;
 * 1 / temperature that rounds to 0 or infinity in bf16 is JIT_EUNSUPPORTED. */
int jit_sample_rows(const uint16_t *logits, int B, int V, double temperature, double top_p, int top_k,
                    const float *u, int32_t *tokens, void *stream);

/* u[b] = min(fp32(y0) / 2^32, 1 - 2^-24), (y0, y1) = Threefry-2x32-20(keys[b] = (k0, k1),
 * counter (0, 0)) (Salmon et al., SC'11): the uniform mx.random.uniform(shape=(1,), key) draws
 * for a step key (Sampler.uniform, Q36/sampler.py:367-369; the fused tail's replay,
 * :160-177).  keys: [B, 2] uint32 on the device. */
int jit_threefry_uniform(const uint32_t *keys, int B, float *u, void *stream);

/* Copy page src[i] to page dst[i] (i < n; device arrays) inside one layer's pool
 * [num_pages, Hkv, 2, 16 * 128] bf16: the copy-on-write of a shared page before a sequence
 * writes into it.  It replaces the reference's snapshot copies of a stored prefix
 * (RequestState.snapshot / restore, Q36/kvcache/state.py:58-149; KVSlot.load,
 * Q36/kvcache/kv_cache.py:38-58): full pages of a prefix are shared, only its partial last
 * page is copied.  A page id outside [0, num_pages) copies nothing. */
int jit_kv_copy_pages(uint16_t *pool, int num_pages, int Hkv, const int32_t *src, const int32_t *dst, int n,
                      void *stream);

#ifdef __cplusplus
}
#endif

#endif /* JIT_MOE_H */
