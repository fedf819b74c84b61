// Multi-token GEMMs for the chunked prefill: y[j] (+)= W x[j] + b for j < n,
// x f16 [n][in_f] token-major, y f32 [n][out_f].
// reference: chunk_gemm.cu:65-176 (int4-hier), 183-258 (fp16), 285-332.
//
// MI355X design
// -------------
// * A block computes a 64-row x 128-token tile of y on MFMA
//   (v_mfma_f32_16x16x32_f16: rows x tokens, f32 accumulate). Four waves each
//   own 32 tokens x 64 rows (4 x 2 accumulator tiles).
// * K advances one int4-hier group (32 columns) per step. The step's weights
//   are dequantised into an f16 LDS tile exactly as the quantiser's
//   dequantisation computes them (hier.rs:398-421: s = d*ls, m = -dmin*lm,
//   q*s + m, each operation rounded in f32) and then rounded to f16; x is
//   already f16. The tiles are double-buffered: the next step's packed bytes
//   and activations are loaded into registers while this step's MFMAs run,
//   and one barrier per step separates the buffers.
// * Each weight is dequantised once per 128 tokens; per step a block does
//   2048 dequantisations against 262144 multiply-adds, so the MFMA pipe, not
//   VALU, sets the pace.
// * f16 rather than bf16 tiles: the same MFMA rate, three more mantissa bits
//   (the dequantised weight rounds once, to 11 bits; products and sums are
//   f32).
// * The fp16 form (wst_gemm_fp16, the lossless reference path) runs the same
//   kernel with the W tile copied instead of dequantised.
#include "common.hpp"

#define HGROUP 32
#define GM_BM 64
#define GM_BN 128
#define GM_THREADS 256
#define GM_KS 40  // LDS row stride (halves) of a 32-wide K step: 80 B, conflict-free reads

typedef _Float16 gm_h8 __attribute__((ext_vector_type(8)));
typedef float gm_f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ gm_h8 gm_lds8(const uint16_t *p) {
  return __builtin_bit_cast(gm_h8, *(const uint4 *)p);
}

// HIER: w = (qw, si, sb) int4-hier-g32; else w is f16 [out_f][in_f].
template <bool HIER>
__global__ __launch_bounds__(GM_THREADS) void gemm_mfma_kernel(
    const void *__restrict__ w, const uint8_t *__restrict__ si, const uint32_t *__restrict__ sb,
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ bias, float *__restrict__ y,
    int in_f, int out_f, int n, int accum) {
#pragma clang fp contract(off)
  __shared__ __align__(16) uint16_t wt[2][GM_BM * GM_KS];
  __shared__ __align__(16) uint16_t xt[2][GM_BN * GM_KS];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r0 = blockIdx.x * GM_BM, t0 = blockIdx.y * GM_BN;
  const int G = in_f / HGROUP;

  // Load assignment: W row wr = tid/4 (clamped), 8 columns wc = 8*(tid%4) of
  // the step; x tokens xtok + 64i, the same 8 columns.
  const int wr = tid >> 2, wc = (tid & 3) * 8;
  const int wrow = min(r0 + wr, out_f - 1);
  float d = 0.0f, dm = 0.0f;
  if constexpr (HIER) {
    const uint32_t p = sb[wrow];
    d = h2f((uint16_t)(p & 0xFFFFu));
    dm = h2f((uint16_t)(p >> 16));
  }
  uint32_t wword = 0;
  uint32_t widx = 0;
  uint4 wvec = make_uint4(0, 0, 0, 0);
  uint4 xv[2];
  auto load = [&](int g) {
    if constexpr (HIER) {
      wword = ((const uint32_t *)w)[(size_t)wrow * (in_f / 8) + g * 4 + (tid & 3)];
      widx = si[(size_t)wrow * G + g];
    } else {
      wvec = *(const uint4 *)((const uint16_t *)w + (size_t)wrow * in_f + g * HGROUP + wc);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int tok = min(t0 + wr + 64 * i, n - 1);
      xv[i] = *(const uint4 *)(x + (size_t)tok * in_f + g * HGROUP + wc);
    }
  };
  auto store = [&](int buf) {
    uint4 o;
    if constexpr (HIER) {
      const float s = __fmul_rn(d, (float)(widx & 0xFu));
      const float m = __fmul_rn(-dm, (float)(widx >> 4));
      uint32_t hv[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float lo = __fadd_rn(__fmul_rn((float)((wword >> (8 * k)) & 0xFu), s), m);
        const float hi = __fadd_rn(__fmul_rn((float)((wword >> (8 * k + 4)) & 0xFu), s), m);
        hv[k] = (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
      }
      o = make_uint4(hv[0], hv[1], hv[2], hv[3]);
    } else {
      o = wvec;
    }
    *(uint4 *)&wt[buf][wr * GM_KS + wc] = o;
#pragma unroll
    for (int i = 0; i < 2; ++i) *(uint4 *)&xt[buf][(wr + 64 * i) * GM_KS + wc] = xv[i];
  };

  gm_f4 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = (gm_f4){0.0f, 0.0f, 0.0f, 0.0f};

  load(0);
  store(0);
  __syncthreads();
  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  for (int g = 0; g < G; ++g) {
    const int buf = g & 1;
    if (g + 1 < G) load(g + 1);
    gm_h8 bf[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) bf[b] = gm_lds8(&xt[buf][(wave * 32 + b * 16 + r16) * GM_KS + kq]);
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const gm_h8 af = gm_lds8(&wt[buf][(a * 16 + r16) * GM_KS + kq]);
#pragma unroll
      for (int b = 0; b < 2; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[b], acc[a][b], 0, 0, 0);
    }
    if (g + 1 < G) store(buf ^ 1);
    __syncthreads();
  }

  // C[row][token]: lane holds rows 4*(lane/16)+i of each 16-row tile, token lane%16.
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int tok = t0 + wave * 32 + b * 16 + r16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = r0 + a * 16 + (lane >> 4) * 4 + i;
        if (row < out_f && tok < n) {
          float v = acc[a][b][i];
          if (bias) v += h2f(bias[row]);
          float *dst = y + (size_t)tok * out_f + row;
          *dst = accum ? *dst + v : v;
        }
      }
    }
}

wst_status_t wst_gemm_mfma(bool hier, const void *w, const void *si, const void *sb,
                           const void *x, const void *bias, void *y, int32_t in_f, int32_t out_f,
                           int32_t n, int32_t accum) {
  const dim3 grid((out_f + GM_BM - 1) / GM_BM, (n + GM_BN - 1) / GM_BN);
  if (hier)
    gemm_mfma_kernel<true><<<grid, GM_THREADS, 0, WST_STREAM>>>(
        w, (const uint8_t *)si, (const uint32_t *)sb, (const uint16_t *)x,
        (const uint16_t *)bias, (float *)y, in_f, out_f, n, accum);
  else
    gemm_mfma_kernel<false><<<grid, GM_THREADS, 0, WST_STREAM>>>(
        w, nullptr, nullptr, (const uint16_t *)x, (const uint16_t *)bias, (float *)y, in_f,
        out_f, n, accum);
  return WST_OK;
}
