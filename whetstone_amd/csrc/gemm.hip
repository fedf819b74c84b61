// Multi-token GEMMs for the chunked prefill: y[j] (+)= W x[j] + b for j < n,
// x f16 [n][in_f] token-major, y f32 [n][out_f].
// reference: chunk_gemm.cu:65-176 (int4-hier), 183-258 (fp16), 285-332.
//
// MI355X design
// -------------
// * A block computes a 64-row x 128-token tile of y on MFMA
//   (v_mfma_f32_16x16x32_f16: rows x tokens, f32 accumulate). Four waves each
//   own 32 tokens x 64 rows (4 x 2 accumulator tiles).
// * K advances four int4-hier groups (128 columns) per step. The step's weights
//   are dequantised into an f16 LDS tile exactly as the quantiser's
//   dequantisation computes them (hier.rs:398-421: s = d*ls, m = -dmin*lm,
//   q*s + m, each operation rounded in f32) and then rounded to f16; x is
//   already f16. The tiles are double-buffered in LDS: the next step's packed
//   bytes and activations are in flight while this step's 32 MFMAs per wave
//   run, and one barrier per step separates the buffers. (With one group per
//   step the loop was latency-bound: every step waited a full memory round
//   trip for one group's data.)
// * Split-K: when the output has too few tiles to fill the chip (the o and
//   down projections of small models, any shape at few tokens), the group
//   range is split over blocks. Each split writes its f32 partial tile to a
//   library scratch slot, and a second kernel adds the splits in split order
//   plus the bias and the accumulate, so the result is deterministic for a
//   given shape. Chunk GEMMs are never graph-captured (chunk.rs:1-12), so the
//   slot may grow on first use.
// * Each weight is dequantised once per 128 tokens; per step a block does
//   8192 dequantisations against 1 M multiply-adds, so the MFMA pipe, not
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
#define GM_KG 4                                   // groups per step
#define GM_KC (GM_KG * HGROUP)                    // columns per step
#define GM_KS (GM_KC + 8)                         // LDS row stride (halves): conflict-free reads
#define GM_XP (GM_BN * GM_KC / 8 / GM_THREADS)    // 16-byte x pieces per thread per step
#define GM_WT (GM_BM * GM_KS)                     // halves of one W buffer
#define GM_XT (GM_BN * GM_KS)                     // halves of one x buffer
#define GM_LDS ((2 * GM_WT + 2 * GM_XT) * 2)      // bytes

typedef _Float16 gm_h8 __attribute__((ext_vector_type(8)));
typedef float gm_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t gm_u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ gm_h8 gm_lds8(const uint16_t *p) {
  return __builtin_bit_cast(gm_h8, *(const gm_u4 *)p);
}

// HIER: w = (qw, si, sb) int4-hier-g32; else w is f16 [out_f][in_f].
// Split z = blockIdx.z covers groups [z*gps, min(G, (z+1)*gps)); with one
// split the epilogue writes y, otherwise the f32 tile goes to ws[z].
template <bool HIER>
__global__ __launch_bounds__(GM_THREADS) void gemm_mfma_kernel(
    const void *__restrict__ w, const uint8_t *__restrict__ si, const uint32_t *__restrict__ sb,
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ bias, float *__restrict__ y,
    float *__restrict__ ws, int in_f, int out_f, int n, int accum, int gps) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint16_t gm_lds[];
  uint16_t *wt = gm_lds;            // [2][GM_BM][GM_KS]
  uint16_t *xt = gm_lds + 2 * GM_WT;  // [2][GM_BN][GM_KS]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r0 = blockIdx.x * GM_BM, t0 = blockIdx.y * GM_BN;
  const int G = in_f / HGROUP;
  const int g_begin = blockIdx.z * gps, g_end = min(G, g_begin + gps);
  const int steps = (g_end - g_begin + GM_KG - 1) / GM_KG;

  // W assignment: row wr = tid / 4, group wg = tid % 4 of the step.
  const int wr = tid >> 2, wg = tid & 3;
  const int wrow = min(r0 + wr, out_f - 1);
  float d = 0.0f, dm = 0.0f;
  if constexpr (HIER) {
    const uint32_t p = sb[wrow];
    d = h2f((uint16_t)(p & 0xFFFFu));
    dm = h2f((uint16_t)(p >> 16));
  }
  gm_u4 wv[HIER ? 1 : 4];
  uint32_t widx = 0;
  gm_u4 xv[GM_XP];
  auto load = [&](int step) {  // indices clamped: unconditional loads stay batched
    const int g = g_begin + step * GM_KG;
    const int gw = min(g + wg, G - 1);
    if constexpr (HIER) {
      wv[0] = *(const gm_u4 *)((const uint32_t *)w + (size_t)wrow * (in_f / 8) + gw * 4);
      widx = si[(size_t)wrow * G + gw];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        wv[i] = *(const gm_u4 *)((const uint16_t *)w + (size_t)wrow * in_f + gw * HGROUP + 8 * i);
    }
#pragma unroll
    for (int i = 0; i < GM_XP; ++i) {
      const int piece = tid + GM_THREADS * i;
      const int tok = min(t0 + piece / (GM_KC / 8), n - 1);
      const int col = min(g * HGROUP + 8 * (piece % (GM_KC / 8)), in_f - 8);
      xv[i] = *(const gm_u4 *)(x + (size_t)tok * in_f + col);
    }
  };
  auto store = [&](int step, int buf) {
    // Groups past the split's range hold zero weights (their x is finite).
    const bool live = g_begin + step * GM_KG + wg < g_end;
    uint16_t *dst = wt + buf * GM_WT + wr * GM_KS + wg * HGROUP;
    if constexpr (HIER) {
      const float s = __fmul_rn(d, (float)(widx & 0xFu));
      const float m = __fmul_rn(-dm, (float)(widx >> 4));
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const uint32_t word = wv[0][q4];
        uint32_t hv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float lo = __fadd_rn(__fmul_rn((float)((word >> (8 * k)) & 0xFu), s), m);
          const float hi = __fadd_rn(__fmul_rn((float)((word >> (8 * k + 4)) & 0xFu), s), m);
          hv[k] = live ? ((uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16)) : 0u;
        }
        *(gm_u4 *)(dst + 8 * q4) = (gm_u4){hv[0], hv[1], hv[2], hv[3]};
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) *(gm_u4 *)(dst + 8 * i) = live ? wv[i] : (gm_u4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < GM_XP; ++i) {
      const int piece = tid + GM_THREADS * i;
      *(gm_u4 *)(xt + buf * GM_XT + (piece / (GM_KC / 8)) * GM_KS + 8 * (piece % (GM_KC / 8))) =
          xv[i];
    }
  };

  gm_f4 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = (gm_f4){0.0f, 0.0f, 0.0f, 0.0f};

  load(0);
  store(0, 0);
  __syncthreads();
  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  for (int st = 0; st < steps; ++st) {
    const int buf = st & 1;
    if (st + 1 < steps) load(st + 1);
    const uint16_t *wb = wt + buf * GM_WT, *xb = xt + buf * GM_XT;
#pragma unroll
    for (int kk = 0; kk < GM_KC; kk += 32) {
      gm_h8 bf[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) bf[b] = gm_lds8(xb + (wave * 32 + b * 16 + r16) * GM_KS + kk + kq);
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const gm_h8 af = gm_lds8(wb + (a * 16 + r16) * GM_KS + kk + kq);
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[b], acc[a][b], 0, 0, 0);
      }
    }
    if (st + 1 < steps) store(st + 1, buf ^ 1);
    __syncthreads();
  }

  // C[row][token]: lane holds rows 4*(lane/16)+i of each 16-row tile, token lane%16.
  const bool split = gridDim.z > 1;
  float *part = split ? ws + (size_t)blockIdx.z * n * out_f : nullptr;
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
          if (split) {
            part[(size_t)tok * out_f + row] = v;
          } else {
            if (bias) v += h2f(bias[row]);
            float *dst = y + (size_t)tok * out_f + row;
            *dst = accum ? *dst + v : v;
          }
        }
      }
    }
}

// y = (accum ? y : 0) + (sum of the splits in split order) + bias.
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(const float *__restrict__ ws,
                                                                const uint16_t *__restrict__ bias,
                                                                float *__restrict__ y, int out_f,
                                                                int n, int splits, int accum) {
  const size_t total = (size_t)n * out_f;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    float v = ws[i];
    for (int z = 1; z < splits; ++z) v += ws[(size_t)z * total + i];
    if (bias) v += h2f(bias[i % out_f]);
    y[i] = accum ? y[i] + v : v;
  }
}

wst_status_t wst_gemm_mfma(bool hier, const void *w, const void *si, const void *sb,
                           const void *x, const void *bias, void *y, int32_t in_f, int32_t out_f,
                           int32_t n, int32_t accum) {
  static bool attr[2] = {false, false};
  if (!attr[hier]) {
    const void *k = hier ? (const void *)gemm_mfma_kernel<true> : (const void *)gemm_mfma_kernel<false>;
    (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, GM_LDS);
    attr[hier] = true;
  }
  const int G = in_f / HGROUP;
  const int tiles = ((out_f + GM_BM - 1) / GM_BM) * ((n + GM_BN - 1) / GM_BN);
  // Splits so that the grid covers the chip, each at least one step long.
  int splits = 1, gps = G;
  const int target = wst_cu_count();
  if (tiles < target / 2) {
    const int want = (target + tiles - 1) / tiles;
    gps = (G + want - 1) / want;
    gps = (gps + GM_KG - 1) / GM_KG * GM_KG;
    splits = (G + gps - 1) / gps;
  }
  float *ws = nullptr;
  if (splits > 1) {
    ws = (float *)wst_static_scratch(WST_SCRATCH_GEMM, (size_t)splits * n * out_f * 4);
    if (!ws) return WST_ERR_OOM;
  }
  const dim3 grid((out_f + GM_BM - 1) / GM_BM, (n + GM_BN - 1) / GM_BN, splits);
  if (hier)
    gemm_mfma_kernel<true><<<grid, GM_THREADS, GM_LDS, WST_STREAM>>>(
        w, (const uint8_t *)si, (const uint32_t *)sb, (const uint16_t *)x,
        (const uint16_t *)bias, (float *)y, ws, in_f, out_f, n, accum, gps);
  else
    gemm_mfma_kernel<false><<<grid, GM_THREADS, GM_LDS, WST_STREAM>>>(
        w, nullptr, nullptr, (const uint16_t *)x, (const uint16_t *)bias, (float *)y, ws, in_f,
        out_f, n, accum, gps);
  if (splits > 1) {
    const size_t total = (size_t)n * out_f;
    const int blocks = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
    gemm_split_reduce_kernel<<<blocks, 256, 0, WST_STREAM>>>(ws, (const uint16_t *)bias,
                                                              (float *)y, out_f, n, splits, accum);
  }
  return WST_OK;
}
