// The ends of the decode step and the KV pages' copy-on-write:
//   * embedding lookup of MLX 4-bit affine rows (QEmbedding.lookup = mx.dequantize of the
//     gathered rows, Q36/linear.py:680-690),
//   * whole-page copies inside a layer's KV pool (the copy a sequence makes of a shared page
//     before writing into it).
#include "common.hpp"

namespace {

// One workgroup per row; thread t dequantizes packed words t, t + 256, ... (8 values each).
// MLX computes the affine dequantization in bf16 arithmetic: scale * q rounded to bf16, then
// + bias rounded to bf16.  An id outside [0, V) gives a zero row.
__global__ __launch_bounds__(256) void embed_q4_kernel(const int32_t *__restrict__ ids, const uint32_t *__restrict__ w,
                                                       const uint16_t *__restrict__ scales,
                                                       const uint16_t *__restrict__ biases, int V, int D,
                                                       uint16_t *__restrict__ out) {
  const int b = blockIdx.x;
  const int id = ids[b];
  const bool ok = id >= 0 && id < V;
  const int words = D / 8, groups = D / 64;
  for (int j = threadIdx.x; j < words; j += blockDim.x) {
    uint4 o = make_uint4(0u, 0u, 0u, 0u);
    if (ok) {
      const uint32_t q = w[(long long)id * words + j];
      const float s = bf2f(scales[(long long)id * groups + j / 8]);
      const float bb = bf2f(biases[(long long)id * groups + j / 8]);
      uint32_t h[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float sq = bf2f(f2bf(s * (float)((q >> (4 * i)) & 15u)));
        h[i] = f2bf(sq + bb);
      }
      o = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
    }
    *(uint4 *)(out + (long long)b * D + 8 * j) = o;
  }
}

// Workgroup i copies page src[i] to page dst[i] of one layer's pool; page_words = 16-byte words
// of a page (all kv heads' K and V).  A page id outside [0, num_pages) copies nothing.
__global__ __launch_bounds__(256) void kv_copy_pages_kernel(uint4 *__restrict__ pool, const int32_t *__restrict__ src,
                                                            const int32_t *__restrict__ dst, int page_words,
                                                            int num_pages) {
  const int ps = src[blockIdx.x], pd = dst[blockIdx.x];
  if (ps < 0 || ps >= num_pages || pd < 0 || pd >= num_pages) return;
  const long long s = (long long)ps * page_words, d = (long long)pd * page_words;
  for (int j = threadIdx.x; j < page_words; j += blockDim.x) pool[d + j] = pool[s + j];
}

}  // namespace

extern "C" int jit_embed_q4(const int32_t *ids, int B, const uint32_t *weight, const uint16_t *scales,
                            const uint16_t *biases, int V, int D, uint16_t *out, void *stream) {
  if (B < 0 || V <= 0 || D <= 0) return jit::fail(JIT_EINVAL, "embed_q4: bad dims B=%d V=%d D=%d", B, V, D);
  if (D % 64 != 0) return jit::fail(JIT_EUNSUPPORTED, "embed_q4 covers D %% 64 == 0 (group 64), got %d", D);
  if (B == 0) return JIT_OK;
  if (!ids || !weight || !scales || !biases || !out) return jit::fail(JIT_EINVAL, "embed_q4: null pointer");
  embed_q4_kernel<<<B, 256, 0, (hipStream_t)stream>>>(ids, weight, scales, biases, V, D, out);
  return jit::check_launch("jit_embed_q4");
}

extern "C" int jit_kv_copy_pages(uint16_t *pool, int num_pages, int Hkv, const int32_t *src, const int32_t *dst,
                                 int n, void *stream) {
  if (n < 0 || Hkv <= 0 || num_pages <= 0)
    return jit::fail(JIT_EINVAL, "kv_copy_pages: bad dims n=%d Hkv=%d num_pages=%d", n, Hkv, num_pages);
  if (n == 0) return JIT_OK;
  if (!pool || !src || !dst) return jit::fail(JIT_EINVAL, "kv_copy_pages: null pointer");
  const int page_words = Hkv * 2 * JIT_PAGE_TOKENS * JIT_HEAD_DIM * 2 / 16;
  kv_copy_pages_kernel<<<n, 256, 0, (hipStream_t)stream>>>((uint4 *)pool, src, dst, page_words, num_pages);
  return jit::check_launch("jit_kv_copy_pages");
}
