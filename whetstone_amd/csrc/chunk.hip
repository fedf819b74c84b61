// Multi-token ("chunk") forms of the decode step, for prefill.
// reference: crates/whetstone-kernels/cuda/chunk_gemm.cu, chunk_ops.cu.
//
// Activations are token-major [n][dim]; pos0 is passed by value (a chunk pass
// is not graph-captured, chunk.rs:1-12). Causality is the loop bound: token j
// attends to cache positions [0, pos0 + j].
#include "common.hpp"

#define CHUNK_MAX_TOKENS 256

extern "C" int32_t wst_chunk_max_tokens(void) { return CHUNK_MAX_TOKENS; }

// Implemented in gemm.hip (MFMA).
wst_status_t wst_gemm_mfma(bool hier, const void *w, const void *si, const void *sb,
                           const void *x, const void *bias, void *y, int32_t in_f, int32_t out_f,
                           int32_t n, int32_t accum);

extern "C" wst_status_t wst_gemm_int4_hier(const void *qw, const void *si, const void *sb,
                                           const void *x, const void *bias, void *y,
                                           int32_t in_f, int32_t out_f, int32_t n,
                                           int32_t accum) {
  WST_REQUIRE(qw && si && sb && x && y, "wst_gemm_int4_hier: null pointer");
  WST_REQUIRE(in_f > 0 && out_f > 0 && n > 0, "wst_gemm_int4_hier: non-positive dimension");
  WST_REQUIRE(in_f % 32 == 0, "wst_gemm_int4_hier: in_features must be a multiple of 32");
  WST_REQUIRE(!(((uintptr_t)qw | (uintptr_t)x) & 15u),
              "wst_gemm_int4_hier: qw and x must be 16-byte aligned");
  wst_gemm_mfma(true, qw, si, sb, x, bias, y, in_f, out_f, n, accum);
  WST_TRY_KERNEL("wst_gemm_int4_hier");
  return WST_OK;
}

extern "C" wst_status_t wst_gemm_fp16(const void *w, const void *x, const void *bias, void *y,
                                      int32_t in_f, int32_t out_f, int32_t n, int32_t accum) {
  WST_REQUIRE(w && x && y, "wst_gemm_fp16: null pointer");
  WST_REQUIRE(in_f > 0 && out_f > 0 && n > 0, "wst_gemm_fp16: non-positive dimension");
  WST_REQUIRE(in_f % 8 == 0, "wst_gemm_fp16: in_features must be a multiple of 8");
  if (in_f % 32 == 0 && !(((uintptr_t)w | (uintptr_t)x) & 15u)) {
    wst_gemm_mfma(false, w, nullptr, nullptr, x, bias, y, in_f, out_f, n, accum);
    WST_TRY_KERNEL("wst_gemm_fp16");
    return WST_OK;
  }
  for (int j = 0; j < n; ++j) {  // widths that are not whole 32-column steps
    const wst_status_t st = wst_gemv_fp16_ex(w, (const uint16_t *)x + (size_t)j * in_f, bias,
                                             (float *)y + (size_t)j * out_f, in_f, out_f, accum);
    if (st != WST_OK) return st;
  }
  return WST_OK;
}

// Causal chunk attention (chunk_ops.cu:187-265): one block per (query head,
// token). q is the rotated q of the token's qkv row; the cache already holds
// the chunk's own k/v (wst_rope_cache_chunk ran first). Each of the 4 waves
// sweeps every 4th position with head_dim/64 elements per lane and its own
// online softmax; the waves merge through LDS.
template <int HD>
__global__ __launch_bounds__(256) void attn_chunk_kernel(
    const float *__restrict__ qkv, const uint16_t *__restrict__ k_cache,
    const uint16_t *__restrict__ v_cache, uint16_t *__restrict__ out, int n_q, int n_kv,
    int pos0, int max_seq, float scale) {
  constexpr int EPL = HD / 64;  // elements per lane
  const int head = blockIdx.x, tok = blockIdx.y;
  const int gqa = n_q / n_kv, kvh = head / gqa;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int stride_row = (n_q + 2 * n_kv) * HD;
  const float *q = qkv + (size_t)tok * stride_row + (size_t)head * HD;
  const int seq = min(pos0 + tok + 1, max_seq);

  float qr[EPL], acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    qr[e] = q[lane + 64 * e] * scale;
    acc[e] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  const uint16_t *kb = k_cache + (size_t)kvh * max_seq * HD;
  const uint16_t *vb = v_cache + (size_t)kvh * max_seq * HD;
  for (int t = wave; t < seq; t += 4) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) s = fmaf(qr[e], h2f(kb[(size_t)t * HD + lane + 64 * e]), s);
    s = wave_sum(s);
    const float mn = fmaxf(m, s);
    const float corr = __expf(m - mn);
    const float p = __expf(s - mn);
    l = fmaf(l, corr, p);
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      acc[e] = fmaf(p, h2f(vb[(size_t)t * HD + lane + 64 * e]), acc[e] * corr);
    m = mn;
  }
  __shared__ float sm[4][HD + 2];
#pragma unroll
  for (int e = 0; e < EPL; ++e) sm[wave][2 + lane + 64 * e] = acc[e];
  if (lane == 0) {
    sm[wave][0] = m;
    sm[wave][1] = l;
  }
  __syncthreads();
  for (int d = tid; d < HD; d += 256) {
    float M = -INFINITY;
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm[w][0]);
    float num = 0.0f, den = 0.0f;
    for (int w = 0; w < 4; ++w) {
      const float f = (sm[w][0] == -INFINITY) ? 0.0f : __expf(sm[w][0] - M);
      num = fmaf(sm[w][2 + d], f, num);
      den = fmaf(sm[w][1], f, den);
    }
    out[(size_t)tok * n_q * HD + (size_t)head * HD + d] = f2h(num / den);
  }
}

extern "C" wst_status_t wst_attn_chunk(const void *qkv, const void *k_cache, const void *v_cache,
                                       void *out, int32_t n_q, int32_t n_kv, int32_t head_dim,
                                       int32_t pos0, int32_t n, int32_t max_seq, float scale) {
  WST_REQUIRE(qkv && k_cache && v_cache && out, "wst_attn_chunk: null pointer");
  WST_REQUIRE(n_q > 0 && n_kv > 0 && n_q % n_kv == 0 && n > 0 && n <= 65535,
              "wst_attn_chunk: bad shape");
  WST_REQUIRE(max_seq > 0 && pos0 >= 0 && pos0 + n <= max_seq,
              "wst_attn_chunk: chunk does not fit the cache");
  const dim3 grid(n_q, n);
  switch (head_dim) {
    case 64:
      attn_chunk_kernel<64><<<grid, 256, 0, WST_STREAM>>>(
          (const float *)qkv, (const uint16_t *)k_cache, (const uint16_t *)v_cache,
          (uint16_t *)out, n_q, n_kv, pos0, max_seq, scale);
      break;
    case 128:
      attn_chunk_kernel<128><<<grid, 256, 0, WST_STREAM>>>(
          (const float *)qkv, (const uint16_t *)k_cache, (const uint16_t *)v_cache,
          (uint16_t *)out, n_q, n_kv, pos0, max_seq, scale);
      break;
    case 256:
      attn_chunk_kernel<256><<<grid, 256, 0, WST_STREAM>>>(
          (const float *)qkv, (const uint16_t *)k_cache, (const uint16_t *)v_cache,
          (uint16_t *)out, n_q, n_kv, pos0, max_seq, scale);
      break;
    default:
      WST_REQUIRE(false, "wst_attn_chunk: head_dim must be 64, 128 or 256");
  }
  WST_TRY_KERNEL("wst_attn_chunk");
  return WST_OK;
}
