// The non-GEMV single-token ops: RMSNorm, RoPE + KV append (+ QK-norm), SwiGLU.
// reference: crates/whetstone-kernels/cuda/decode.cu.
//
// Precision contract (decode.cu:15-21): reductions and activations in f32,
// narrowing to f16 only where a vector is handed to the next GEMV or to the
// KV cache; the residual stream stays f32.
#include "common.hpp"

// ------------------------------------------------------------------ RMSNorm

// One 512-thread block per row. The scale comes from rms_scale512, the same
// reduction the GEMV's fused RMSNorm prologue uses, so the two produce
// identical f16 vectors.
__global__ __launch_bounds__(512) void rmsnorm_kernel(const float *__restrict__ x,
                                                      const uint16_t *__restrict__ w,
                                                      uint16_t *__restrict__ out, int n,
                                                      float eps) {
  __shared__ float red[16];
  const float *xr = x + (size_t)blockIdx.x * n;
  uint16_t *orow = out + (size_t)blockIdx.x * n;
  const float s = rms_scale512(xr, n, eps, red);
  for (int i = threadIdx.x; i < n; i += 512) orow[i] = f2h(xr[i] * s * h2f(w[i]));
}

extern "C" wst_status_t wst_rmsnorm(const void *x, const void *w, void *out, int32_t n,
                                    float eps) {
  WST_REQUIRE(x && w && out, "wst_rmsnorm: null pointer");
  WST_REQUIRE(n > 0, "wst_rmsnorm: n must be positive");
  rmsnorm_kernel<<<1, 512, 0, WST_STREAM>>>((const float *)x, (const uint16_t *)w,
                                            (uint16_t *)out, n, eps);
  WST_TRY_KERNEL("wst_rmsnorm");
  return WST_OK;
}

// Token-major [n][dim] form (chunk_ops.cu:42-97): one block per token, the same
// kernel, so chunk and single-token outputs agree bit for bit.
extern "C" wst_status_t wst_rmsnorm_chunk(const void *x, const void *w, void *out, int32_t dim,
                                          int32_t n, float eps) {
  WST_REQUIRE(x && w && out, "wst_rmsnorm_chunk: null pointer");
  WST_REQUIRE(dim > 0 && n > 0, "wst_rmsnorm_chunk: bad shape");
  rmsnorm_kernel<<<n, 512, 0, WST_STREAM>>>((const float *)x, (const uint16_t *)w,
                                            (uint16_t *)out, dim, eps);
  WST_TRY_KERNEL("wst_rmsnorm_chunk");
  return WST_OK;
}

// -------------------------------------------------- RoPE + KV cache append

// One block per head (n_q query heads, then n_kv key heads that also copy v).
// `pos_dev` (device, clamped) or, when null, `pos0 + blockIdx.y` for the
// token-major chunk form, where qkv rows are [n][(n_q+2n_kv)*hd].
__global__ __launch_bounds__(1024) void rope_cache_kernel(
    float *__restrict__ qkv, uint16_t *__restrict__ k_cache, uint16_t *__restrict__ v_cache,
    const float *__restrict__ cos_tab, const float *__restrict__ sin_tab, int n_q, int n_kv,
    int hd, const int32_t *__restrict__ pos_dev, int pos0, int max_seq,
    const uint16_t *__restrict__ q_norm_w, const uint16_t *__restrict__ k_norm_w, float eps) {
  __shared__ float red[16];
  const int head = blockIdx.x;
  const int half = hd >> 1;
  const int j = threadIdx.x;
  const bool active = j < half;
  const int raw = pos_dev ? *pos_dev : pos0 + (int)blockIdx.y;
  const int pos = min(max(raw, 0), max_seq - 1);
  float *row = qkv + (size_t)blockIdx.y * (size_t)(n_q + 2 * n_kv) * hd;

  const float c = active ? cos_tab[(size_t)pos * half + j] : 0.0f;
  const float s = active ? sin_tab[(size_t)pos * half + j] : 0.0f;

  if (head < n_q) {
    float *qh = row + (size_t)head * hd;
    float x1 = active ? qh[j] : 0.0f;
    float x2 = active ? qh[j + half] : 0.0f;
    if (q_norm_w) qk_norm(x1, x2, q_norm_w, j, half, hd, eps, active, red);
    if (!active) return;
    qh[j] = rope_lo(x1, x2, c, s);
    qh[j + half] = rope_hi(x1, x2, c, s);
    return;
  }
  const int kvh = head - n_q;
  const float *kh = row + (size_t)(n_q + kvh) * hd;
  const float *vh = row + (size_t)(n_q + n_kv + kvh) * hd;
  float k1 = active ? kh[j] : 0.0f;
  float k2 = active ? kh[j + half] : 0.0f;
  if (k_norm_w) qk_norm(k1, k2, k_norm_w, j, half, hd, eps, active, red);
  if (!active) return;
  const size_t slot = ((size_t)kvh * max_seq + pos) * hd;
  k_cache[slot + j] = f2h(rope_lo(k1, k2, c, s));
  k_cache[slot + j + half] = f2h(rope_hi(k1, k2, c, s));
  v_cache[slot + j] = f2h(vh[j]);
  v_cache[slot + j + half] = f2h(vh[j + half]);
}

static int rope_threads(int head_dim) {
  const int half = head_dim / 2;
  return ((half + 63) / 64) * 64;
}

extern "C" wst_status_t wst_rope_cache(void *qkv, void *k_cache, void *v_cache,
                                       const void *cos_tab, const void *sin_tab, int32_t n_q,
                                       int32_t n_kv, int32_t head_dim, const void *pos,
                                       int32_t max_seq, const void *q_norm_w,
                                       const void *k_norm_w, float eps) {
  WST_REQUIRE(qkv && k_cache && v_cache && cos_tab && sin_tab && pos,
              "wst_rope_cache: null pointer");
  WST_REQUIRE(n_q > 0 && n_kv > 0 && head_dim > 0, "wst_rope_cache: non-positive shape");
  WST_REQUIRE(head_dim % 2 == 0, "wst_rope_cache: head_dim must be even");
  WST_REQUIRE(head_dim <= 2048, "wst_rope_cache: head_dim/2 exceeds a block");
  WST_REQUIRE(max_seq > 0, "wst_rope_cache: empty cache");
  rope_cache_kernel<<<dim3(n_q + n_kv, 1), rope_threads(head_dim), 0, WST_STREAM>>>(
      (float *)qkv, (uint16_t *)k_cache, (uint16_t *)v_cache, (const float *)cos_tab,
      (const float *)sin_tab, n_q, n_kv, head_dim, (const int32_t *)pos, 0, max_seq,
      (const uint16_t *)q_norm_w, (const uint16_t *)k_norm_w, eps);
  WST_TRY_KERNEL("wst_rope_cache");
  return WST_OK;
}

extern "C" wst_status_t wst_rope_cache_chunk(void *qkv, void *k_cache, void *v_cache,
                                             const void *cos_tab, const void *sin_tab,
                                             int32_t n_q, int32_t n_kv, int32_t head_dim,
                                             int32_t pos0, int32_t n, int32_t max_seq,
                                             const void *q_norm_w, const void *k_norm_w,
                                             float eps) {
  WST_REQUIRE(qkv && k_cache && v_cache && cos_tab && sin_tab,
              "wst_rope_cache_chunk: null pointer");
  WST_REQUIRE(n_q > 0 && n_kv > 0 && head_dim > 0 && n > 0 && n <= 65535,
              "wst_rope_cache_chunk: bad shape");
  WST_REQUIRE(head_dim % 2 == 0 && head_dim <= 2048, "wst_rope_cache_chunk: bad head_dim");
  WST_REQUIRE(max_seq > 0 && pos0 >= 0 && pos0 + n <= max_seq,
              "wst_rope_cache_chunk: chunk does not fit the cache");
  rope_cache_kernel<<<dim3(n_q + n_kv, n), rope_threads(head_dim), 0, WST_STREAM>>>(
      (float *)qkv, (uint16_t *)k_cache, (uint16_t *)v_cache, (const float *)cos_tab,
      (const float *)sin_tab, n_q, n_kv, head_dim, nullptr, pos0, max_seq,
      (const uint16_t *)q_norm_w, (const uint16_t *)k_norm_w, eps);
  WST_TRY_KERNEL("wst_rope_cache_chunk");
  return WST_OK;
}

// ------------------------------------------------------------------ SwiGLU

// out = f16(g / (1 + e^-g) * u) for the two halves of each gate|up row
// (decode.cu:235-242); `inter` wide, `n` rows.
__global__ __launch_bounds__(256) void swiglu_kernel(const float *__restrict__ gate_up,
                                                     uint16_t *__restrict__ out, int inter,
                                                     int n) {
  const size_t total = (size_t)inter * n;
  for (size_t k = blockIdx.x * (size_t)256 + threadIdx.x; k < total;
       k += (size_t)gridDim.x * 256) {
    const size_t tok = k / inter, i = k % inter;
    const float *row = gate_up + tok * 2 * inter;
    const float g = row[i];
    out[k] = f2h(g / (1.0f + __expf(-g)) * row[i + inter]);
  }
}

extern "C" wst_status_t wst_swiglu(const void *gate_up, void *out, int32_t n) {
  WST_REQUIRE(gate_up && out, "wst_swiglu: null pointer");
  WST_REQUIRE(n > 0, "wst_swiglu: n must be positive");
  int blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  swiglu_kernel<<<blocks, 256, 0, WST_STREAM>>>((const float *)gate_up, (uint16_t *)out, n, 1);
  WST_TRY_KERNEL("wst_swiglu");
  return WST_OK;
}

extern "C" wst_status_t wst_swiglu_chunk(const void *gate_up, void *out, int32_t inter,
                                         int32_t n) {
  WST_REQUIRE(gate_up && out, "wst_swiglu_chunk: null pointer");
  WST_REQUIRE(inter > 0 && n > 0, "wst_swiglu_chunk: bad shape");
  const size_t total = (size_t)inter * n;
  size_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  swiglu_kernel<<<(int)blocks, 256, 0, WST_STREAM>>>((const float *)gate_up, (uint16_t *)out,
                                                     inter, n);
  WST_TRY_KERNEL("wst_swiglu_chunk");
  return WST_OK;
}
