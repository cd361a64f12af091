// The decoder block's small fused kernels for gfx950: RMSNorm (with the residual
// add fused in front), the MoE combine (optionally followed by the next layer's
// input RMSNorm), and the per-head q/k RMSNorm + RoPE + paged KV append that sits
// between the qkv projection and decode attention.
//
// Arithmetic follows the reference's MLX ops (Q36/model/attention.py:42-68,
// 99-119; Q36/model/model.py:65-80): RMSNorm accumulates sum(x^2) in fp32 and
// returns bf16(w * bf16(x * rsqrt(mean + eps))); RoPE (traditional = False)
// rotates the pairs (x[i], x[i + D/2]) by pos * inv_freq[i] in fp32.
#include "common.hpp"
#include "qtile.hpp"
#include "rowops.hpp"

namespace {

using rowops::block_sum_256;
using rowops::combine8;
using rowops::norm8;
using rowops::pack8;

constexpr int kD = JIT_HEAD_DIM;
constexpr int kPage = JIT_PAGE_TOKENS;

// One workgroup (256 threads) per row; each thread owns 8 consecutive elements.
// With `resid`, the row is h = bf16(x + resid) (written to h_out) and h is normed.
// Rows a kernel writes besides its last output are stored at its end: a vector store counts on the
// same in-order counter as the loads, so a store issued before a later load wait (the norm weights'
// after the barrier) would be waited for there as well.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t *__restrict__ x,
                                                      const uint16_t *__restrict__ resid, int D,
                                                      const uint16_t *__restrict__ w, float eps,
                                                      uint16_t *__restrict__ h_out,
                                                      uint16_t *__restrict__ y) {
  __shared__ float red[8];
  const long long row = blockIdx.x;
  float v[8];
  float ss = 0.0f;
  const int n = threadIdx.x * 8;
  const bool on = n < D;
  // the norm weights are requested with the row (a load after the barrier would add a
  // memory round trip to the kernel's critical path)
  const uint4 wq = on ? *(const uint4 *)(w + n) : make_uint4(0u, 0u, 0u, 0u);
  if (on) {
    const uint4 a = *(const uint4 *)(x + row * D + n);
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (i & 1) ? bf2f_hi(aw[i >> 1]) : bf2f(aw[i >> 1] & 0xffffu);
    if (resid) {
      const uint4 r = *(const uint4 *)(resid + row * D + n);
      const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        v[i] += bf2f(rw[i >> 1] & 0xffffu);
        v[i + 1] += bf2f_hi(rw[i >> 1]);
        round_bf2(v[i], v[i + 1]);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) ss = fmaf(v[i], v[i], ss);
  }
  const float tot = block_sum_256(ss, red);
  const float r = rsqrtf(tot / (float)D + eps);
  if (on) {
    float o[8];
    norm8(v, r, wq, o);
    *(uint4 *)(y + row * D + n) = pack8(o);
    if (resid && h_out) *(uint4 *)(h_out + row * D + n) = pack8(v);
  }
}

// Weighted combine: one workgroup per token row, 8 outputs per thread.
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t *__restrict__ r,
                                                      const int32_t *__restrict__ inv,
                                                      const uint16_t *__restrict__ scores, int k, int D,
                                                      const uint16_t *__restrict__ resid,
                                                      uint16_t *__restrict__ y) {
  const long long bt = blockIdx.x;
  for (int n = threadIdx.x * 8; n < D; n += blockDim.x * 8) {
    float acc[8];
    combine8(r, inv, scores, k, D, resid, bt, n, acc);
    *(uint4 *)(y + bt * D + n) = pack8(acc);
  }
}

// The combine of a layer's last step followed by the next layer's input RMSNorm,
// in the thread layout and summation order of rmsnorm_kernel (so xn is bit for bit
// rmsnorm(y)): y = combine (+ resid) is written, and xn = rmsnorm(y) * w.
__global__ __launch_bounds__(256) void combine_rmsnorm_kernel(
    const uint16_t *__restrict__ r, const int32_t *__restrict__ inv, const uint16_t *__restrict__ scores, int k,
    int D, const uint16_t *__restrict__ resid, uint16_t *__restrict__ y, const uint16_t *__restrict__ w, float eps,
    uint16_t *__restrict__ xn) {
  __shared__ float red[8];
  const long long bt = blockIdx.x;
  const int n = threadIdx.x * 8;
  const bool on = n < D;
  const uint4 wq = on ? *(const uint4 *)(w + n) : make_uint4(0u, 0u, 0u, 0u);  // requested up front
  float v[8];
  float ss = 0.0f;
  if (on) {
    combine8(r, inv, scores, k, D, resid, bt, n, v);
#pragma unroll
    for (int i = 0; i < 8; i++) ss = fmaf(v[i], v[i], ss);
  }
  const float tot = block_sum_256(ss, red);
  const float rs = rsqrtf(tot / (float)D + eps);
  if (on) {
    float o[8];
    norm8(v, rs, wq, o);
    *(uint4 *)(xn + bt * D + n) = pack8(o);
    *(uint4 *)(y + bt * D + n) = pack8(v);  // (stored last: see rmsnorm_kernel)
  }
}

// One wave per (token, head) of the fused qkv row [q: H*128 | k: Hkv*128 | v: Hkv*128].
// Lane l owns dims l and l + 64 -- exactly one RoPE pair -- so the per-head
// RMSNorm is a wave butterfly and the rotation needs no exchange.  q heads go to
// q_out; k heads are normed, rotated and written to the pool page slot of pos[b];
// v heads are written to the pool's dim-major V part.
__global__ __launch_bounds__(256) void qk_norm_rope_append_kernel(
    const uint16_t *__restrict__ qkv, int H, int Hkv, const uint16_t *__restrict__ qn_w,
    const uint16_t *__restrict__ kn_w, float eps, const float *__restrict__ inv_freq,
    const int32_t *__restrict__ pos, const int32_t *__restrict__ page_table, int max_pages,
    uint16_t *__restrict__ pool, uint16_t *__restrict__ q_out) {
  const int b = blockIdx.y;
  const int head = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int l = lane_id();
  const int nh = H + 2 * Hkv;
  if (head >= nh) return;
  const uint16_t *src = qkv + ((long long)b * nh + head) * kD;
  const int p = pos[b];
  const int page = page_table[(long long)b * max_pages + p / kPage];
  const int slot = p % kPage;
  // this row's page for kv head h: K part, then V part (kPage * kD bf16 each)
  auto head_part = [&](int h) { return pool + ((long long)page * Hkv + h) * 2 * (kPage * kD); };
  float x1 = bf2f(src[l]), x2 = bf2f(src[l + 64]);
  if (head >= H + Hkv) {  // v: copy into the dim-major V part
    const int h = head - H - Hkv;
    uint16_t *vp = head_part(h) + kPage * kD;
    vp[l * kPage + slot] = src[l];
    vp[(l + 64) * kPage + slot] = src[l + 64];
    return;
  }
  const uint16_t *nw = head < H ? qn_w : kn_w;
  uint32_t o1, o2;
  qk_head_norm_rope(x1, x2, bf2f(nw[l]), bf2f(nw[l + 64]), eps, (float)p * inv_freq[l], o1, o2);
  if (head < H) {
    uint16_t *qo = q_out + ((long long)b * H + head) * kD;
    qo[l] = (uint16_t)o1;
    qo[l + 64] = (uint16_t)o2;
  } else {
    const int h = head - H;
    uint16_t *kp = head_part(h);
    kp[k_page_offset(slot, l)] = (uint16_t)o1;
    kp[k_page_offset(slot, l + 64)] = (uint16_t)o2;
  }
}

// Elementwise SwiGLU on bf16 g, u: the expert GEMM epilogue's chain (qtile::swiglu_bf16) on given
// operands, 8 values per thread.
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t *__restrict__ g, const uint16_t *__restrict__ u,
                                                     long long n, uint16_t *__restrict__ h) {
  const long long i0 = ((long long)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i0 >= n) return;
  if (i0 + 8 <= n) {
    const uint4 gv = *(const uint4 *)(g + i0), uv = *(const uint4 *)(u + i0);
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
    uint32_t hw[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
      hw[j] = qtile::swiglu_bf16(bf2f(gw[j] & 0xffffu), bf2f(uw[j] & 0xffffu)) |
              (qtile::swiglu_bf16(bf2f_hi(gw[j]), bf2f_hi(uw[j])) << 16);
    *(uint4 *)(h + i0) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  } else {
    for (long long i = i0; i < n; i++) h[i] = (uint16_t)qtile::swiglu_bf16(bf2f(g[i]), bf2f(u[i]));
  }
}

}  // namespace

extern "C" int jit_swiglu(const uint16_t *g, const uint16_t *u, int64_t n, uint16_t *h, void *stream) {
  if (n < 0) return jit::fail(JIT_EINVAL, "swiglu: bad length %lld", (long long)n);
  if (n == 0) return JIT_OK;
  if (!g || !u || !h) return jit::fail(JIT_EINVAL, "swiglu: null pointer");
  if (((uintptr_t)g | (uintptr_t)u | (uintptr_t)h) & 15)
    return jit::fail(JIT_EINVAL, "swiglu: g, u and h must be 16-byte aligned");
  const long long blocks = (n + 256 * 8 - 1) / (256 * 8);
  swiglu_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(g, u, (long long)n, h);
  return jit::check_launch("jit_swiglu");
}

extern "C" int jit_rmsnorm(const uint16_t *x, const uint16_t *resid, int rows, int D, const uint16_t *w,
                           float eps, uint16_t *h_out, uint16_t *y, void *stream) {
  if (rows < 0 || D <= 0) return jit::fail(JIT_EINVAL, "rmsnorm: bad dims rows=%d D=%d", rows, D);
  if (D % 8 != 0 || D > 2048) return jit::fail(JIT_EUNSUPPORTED, "rmsnorm covers D %% 8 == 0 and D <= 2048, got %d", D);
  if (rows == 0) return JIT_OK;
  if (!x || !w || !y) return jit::fail(JIT_EINVAL, "rmsnorm: null pointer");
  rmsnorm_kernel<<<rows, 256, 0, (hipStream_t)stream>>>(x, resid, D, w, eps, h_out, y);
  return jit::check_launch("jit_rmsnorm");
}

extern "C" int jit_qk_norm_rope_append(const uint16_t *qkv, int B, int H, int Hkv, const uint16_t *q_norm_w,
                                       const uint16_t *k_norm_w, float eps, const float *inv_freq,
                                       const int32_t *pos, const int32_t *page_table, int max_pages,
                                       uint16_t *pool, uint16_t *q_out, void *stream) {
  if (B < 0 || H <= 0 || Hkv <= 0 || max_pages <= 0)
    return jit::fail(JIT_EINVAL, "qk_norm_rope_append: bad dims B=%d H=%d Hkv=%d", B, H, Hkv);
  if (H % Hkv != 0) return jit::fail(JIT_EINVAL, "%d query heads do not share %d KV heads evenly", H, Hkv);
  if (B == 0) return JIT_OK;
  if (!qkv || !q_norm_w || !k_norm_w || !inv_freq || !pos || !page_table || !pool || !q_out)
    return jit::fail(JIT_EINVAL, "qk_norm_rope_append: null pointer");
  const dim3 grid((H + 2 * Hkv + 3) / 4, B);
  qk_norm_rope_append_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(qkv, H, Hkv, q_norm_w, k_norm_w, eps, inv_freq,
                                                                    pos, page_table, max_pages, pool, q_out);
  return jit::check_launch("jit_qk_norm_rope_append");
}

extern "C" int jit_moe_combine(const uint16_t *r, const int32_t *inv, const uint16_t *scores, int B, int k, int D,
                               const uint16_t *resid, uint16_t *y, void *stream) {
  if (B < 0 || k <= 0 || D <= 0) return jit::fail(JIT_EINVAL, "moe_combine: bad dims B=%d k=%d D=%d", B, k, D);
  if (D % 8 != 0) return jit::fail(JIT_EUNSUPPORTED, "moe_combine covers D %% 8 == 0, got %d", D);
  if (B == 0) return JIT_OK;
  if (!r || !inv || !scores || !y) return jit::fail(JIT_EINVAL, "moe_combine: null pointer");
  combine_kernel<<<B, 256, 0, (hipStream_t)stream>>>(r, inv, scores, k, D, resid, y);
  return jit::check_launch("jit_moe_combine");
}

extern "C" int jit_moe_combine_rmsnorm(const uint16_t *r, const int32_t *inv, const uint16_t *scores, int B, int k,
                                       int D, const uint16_t *resid, uint16_t *y, const uint16_t *w, float eps,
                                       uint16_t *xn, void *stream) {
  if (B < 0 || k <= 0 || D <= 0)
    return jit::fail(JIT_EINVAL, "moe_combine_rmsnorm: bad dims B=%d k=%d D=%d", B, k, D);
  if (D % 8 != 0 || D > 2048)
    return jit::fail(JIT_EUNSUPPORTED, "moe_combine_rmsnorm covers D %% 8 == 0 and D <= 2048, got %d", D);
  if (B == 0) return JIT_OK;
  if (!r || !inv || !scores || !y || !w || !xn) return jit::fail(JIT_EINVAL, "moe_combine_rmsnorm: null pointer");
  combine_rmsnorm_kernel<<<B, 256, 0, (hipStream_t)stream>>>(r, inv, scores, k, D, resid, y, w, eps, xn);
  return jit::check_launch("jit_moe_combine_rmsnorm");
}

