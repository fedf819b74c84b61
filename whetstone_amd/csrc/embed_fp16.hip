// Row gathers (embedding lookups) and the fp16 GEMV.
// reference: gemv_hier.cu:165-189, 293-307; decode.cu:255-268; gemv_int4.cu:194-305;
// chunk_ops.cu:319-370.
#include "common.hpp"

#define HGROUP 32


// Bit-exact with the quantiser's dequantisation (hier.rs:398-421): s = d*ls,
// m = -dmin*lm, w = q*s + m with each product and the sum rounded separately.
__global__ __launch_bounds__(256) void embed_hier_kernel(const uint32_t *__restrict__ qw,
                                                         const uint8_t *__restrict__ si,
                                                         const uint32_t *__restrict__ sb,
                                                         const int32_t *__restrict__ row_ptr,
                                                         float *__restrict__ out, int in_f,
                                                         int vocab, int n) {
#pragma clang fp contract(off)
  const int tok = blockIdx.y;
  const int row = min(max(row_ptr[tok], 0), vocab - 1);
  const uint32_t p = sb[row];
  const float d = h2f((uint16_t)(p & 0xFFFFu));
  const float dm = h2f((uint16_t)(p >> 16));
  const size_t words = (size_t)in_f / 8, groups = (size_t)in_f / HGROUP;
  for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < in_f; c += gridDim.x * blockDim.x) {
    const uint32_t word = qw[(size_t)row * words + c / 8];
    const float q = (float)((word >> (4 * (c % 8))) & 0xFu);
    const uint8_t idx = si[(size_t)row * groups + c / HGROUP];
    const float s = __fmul_rn(d, (float)(idx & 0xF));
    const float m = __fmul_rn(-dm, (float)(idx >> 4));
    out[(size_t)tok * in_f + c] = __fadd_rn(__fmul_rn(q, s), m);
  }
}

extern "C" wst_status_t wst_embed_int4_hier(const void *qw, const void *si, const void *sb,
                                            const void *row, void *out, int32_t in_f,
                                            int32_t vocab) {
  WST_REQUIRE(qw && si && sb && row && out, "wst_embed_int4_hier: null pointer");
  WST_REQUIRE(in_f > 0 && vocab > 0, "wst_embed_int4_hier: non-positive dimension");
  WST_REQUIRE(in_f % HGROUP == 0, "wst_embed_int4_hier: in_features must be a multiple of 32");
  const int blocks = (in_f + 255) / 256;
  embed_hier_kernel<<<dim3(blocks, 1), 256, 0, WST_STREAM>>>(
      (const uint32_t *)qw, (const uint8_t *)si, (const uint32_t *)sb, (const int32_t *)row,
      (float *)out, in_f, vocab, 1);
  WST_TRY_KERNEL("wst_embed_int4_hier");
  return WST_OK;
}

extern "C" wst_status_t wst_embed_int4_hier_chunk(const void *qw, const void *si,
                                                  const void *sb, const void *tokens, void *out,
                                                  int32_t hidden, int32_t rows, int32_t n) {
  WST_REQUIRE(qw && si && sb && tokens && out, "wst_embed_int4_hier_chunk: null pointer");
  WST_REQUIRE(hidden > 0 && rows > 0 && n > 0, "wst_embed_int4_hier_chunk: bad shape");
  WST_REQUIRE(hidden % HGROUP == 0, "wst_embed_int4_hier_chunk: hidden must be a multiple of 32");
  WST_REQUIRE(n <= 65535, "wst_embed_int4_hier_chunk: too many tokens");
  const int blocks = (hidden + 255) / 256;
  embed_hier_kernel<<<dim3(blocks, n), 256, 0, WST_STREAM>>>(
      (const uint32_t *)qw, (const uint8_t *)si, (const uint32_t *)sb, (const int32_t *)tokens,
      (float *)out, hidden, rows, n);
  WST_TRY_KERNEL("wst_embed_int4_hier_chunk");
  return WST_OK;
}

// ------------------------------------------------------------- fp16 GEMV
//
// Lossless reference path (gemv_int4.cu:194-305): y (+)= W x + b with f16 W.
// A wave owns TILE rows; lanes stride the row 8 halves (16 B) at a time and
// multiply with v_dot2c_f32_f16 into f32.
template <int TILE>
__global__ __launch_bounds__(256) void gemv_fp16_kernel(const uint4 *__restrict__ w,
                                                        const uint4 *__restrict__ x,
                                                        const uint16_t *__restrict__ bias,
                                                        float *__restrict__ y, int in_f,
                                                        int out_f, int accum) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nw = gridDim.x * 4;
  const int V = in_f / 8;
  for (int r0 = wave * TILE; r0 < out_f; r0 += nw * TILE) {
    float acc[TILE];
#pragma unroll
    for (int t = 0; t < TILE; ++t) acc[t] = 0.0f;
    for (int v = lane; v < V; v += 64) {
      const uint4 xv = x[v];
#pragma unroll
      for (int t = 0; t < TILE; ++t) {
        if (r0 + t >= out_f) break;
        const uint4 wv = ld_stream16(w + (size_t)(r0 + t) * V + v);
        acc[t] = __builtin_amdgcn_fdot2(as_h2(wv.x), as_h2(xv.x), acc[t], false);
        acc[t] = __builtin_amdgcn_fdot2(as_h2(wv.y), as_h2(xv.y), acc[t], false);
        acc[t] = __builtin_amdgcn_fdot2(as_h2(wv.z), as_h2(xv.z), acc[t], false);
        acc[t] = __builtin_amdgcn_fdot2(as_h2(wv.w), as_h2(xv.w), acc[t], false);
      }
    }
#pragma unroll
    for (int t = 0; t < TILE; ++t) acc[t] = wave_sum(acc[t]);
    if (lane == 0) {
#pragma unroll
      for (int t = 0; t < TILE; ++t) {
        const int r = r0 + t;
        if (r >= out_f) break;
        float v = acc[t];
        if (bias) v += h2f(bias[r]);
        y[r] = accum ? y[r] + v : v;
      }
    }
  }
}

extern "C" wst_status_t wst_gemv_fp16_ex(const void *w, const void *x, const void *bias, void *y,
                                         int32_t in_f, int32_t out_f, int32_t accum) {
  WST_REQUIRE(w && x && y, "wst_gemv_fp16: null pointer");
  WST_REQUIRE(in_f > 0 && out_f > 0, "wst_gemv_fp16: non-positive dimension");
  WST_REQUIRE(in_f % 8 == 0, "wst_gemv_fp16: in_features must be a multiple of 8");
  const int waves = (out_f + 3) / 4;
  int grid = (waves + 3) / 4;
  const int cap = wst_cu_count() * 16;
  if (grid > cap) grid = cap;
  gemv_fp16_kernel<4><<<grid, 256, 0, WST_STREAM>>>((const uint4 *)w, (const uint4 *)x,
                                                     (const uint16_t *)bias, (float *)y, in_f,
                                                     out_f, accum);
  WST_TRY_KERNEL("wst_gemv_fp16");
  return WST_OK;
}

extern "C" wst_status_t wst_gemv_fp16(const void *w, const void *x, void *y, int32_t in_f,
                                      int32_t out_f) {
  return wst_gemv_fp16_ex(w, x, nullptr, y, in_f, out_f, 0);
}

// Table-row gather of an f16 table (decode.cu:255-268, chunk_ops.cu:319-330).
__global__ void embed_fp16_kernel(const uint16_t *__restrict__ table,
                                  const int32_t *__restrict__ tokens, float *__restrict__ out,
                                  int hidden, int rows) {
  const int tok = blockIdx.y;
  const int row = min(max(tokens[tok], 0), rows - 1);
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
    out[(size_t)tok * hidden + i] = h2f(table[(size_t)row * hidden + i]);
}

extern "C" wst_status_t wst_embed_fp16(const void *table, const void *token, void *out,
                                       int32_t hidden, int32_t rows) {
  WST_REQUIRE(table && out && token, "wst_embed_fp16: null pointer");
  WST_REQUIRE(hidden > 0 && rows > 0, "wst_embed_fp16: bad argument");
  embed_fp16_kernel<<<dim3((hidden + 255) / 256, 1), 256, 0, WST_STREAM>>>(
      (const uint16_t *)table, (const int32_t *)token, (float *)out, hidden, rows);
  WST_TRY_KERNEL("wst_embed_fp16");
  return WST_OK;
}

extern "C" wst_status_t wst_embed_fp16_chunk(const void *table, const void *tokens, void *out,
                                             int32_t hidden, int32_t rows, int32_t n) {
  WST_REQUIRE(table && out && tokens, "wst_embed_fp16_chunk: null pointer");
  WST_REQUIRE(hidden > 0 && rows > 0 && n > 0 && n <= 65535, "wst_embed_fp16_chunk: bad shape");
  embed_fp16_kernel<<<dim3((hidden + 255) / 256, n), 256, 0, WST_STREAM>>>(
      (const uint16_t *)table, (const int32_t *)tokens, (float *)out, hidden, rows);
  WST_TRY_KERNEL("wst_embed_fp16_chunk");
  return WST_OK;
}
