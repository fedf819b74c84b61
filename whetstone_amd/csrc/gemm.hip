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
#define GM_WT (GM_BM * GM_KS)                     // halves of one W buffer
#define GM_LDS (2 * GM_WT * 2)                    // bytes: the W double buffer only
#define GM_NKK (GM_KC / 32)                       // MFMA k-steps per step
#define GM_CS (GM_BM + 4)                         // epilogue tile row stride (floats)
static_assert(GM_BN * GM_CS * 4 <= GM_LDS, "the epilogue tile reuses the W buffers");

typedef _Float16 gm_h8 __attribute__((ext_vector_type(8)));
typedef float gm_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t gm_u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ gm_h8 gm_lds8(const uint16_t *p) {
  return __builtin_bit_cast(gm_h8, *(const gm_u4 *)p);
}

// One step's operands in registers: this thread's W piece (packed, or four
// f16 pieces) and this wave's x B-operand fragments, loaded straight from
// memory in the MFMA layout (lane l: token l%16, columns 8*(l/16)..+7).
template <bool HIER>
struct GmStage {
  gm_u4 wv[HIER ? 1 : 4];
  uint32_t widx;
  gm_u4 xb[GM_NKK][2];
};

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
  uint16_t *wt = gm_lds;  // [2][GM_BM][GM_KS]
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
  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  const uint16_t *xrow[2];
#pragma unroll
  for (int b = 0; b < 2; ++b)
    xrow[b] = x + (size_t)min(t0 + wave * 32 + b * 16 + r16, n - 1) * in_f + kq;

  // Loads are unconditional (the step clamped to the last one): a load under
  // a branch would be followed by a wait for every load in flight.
  auto load = [&](GmStage<HIER> &S, int step) {
    step = min(step, steps - 1);
    const int g = g_begin + step * GM_KG;
    const int gw = min(g + wg, G - 1);
    if constexpr (HIER) {
      S.wv[0] = *(const gm_u4 *)((const uint32_t *)w + (size_t)wrow * (in_f / 8) + gw * 4);
      S.widx = si[(size_t)wrow * G + gw];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        S.wv[i] = *(const gm_u4 *)((const uint16_t *)w + (size_t)wrow * in_f + gw * HGROUP + 8 * i);
    }
#pragma unroll
    for (int k = 0; k < GM_NKK; ++k) {
      const int col = min(g * HGROUP + 32 * k, in_f - 32);  // past G: any finite columns
#pragma unroll
      for (int b = 0; b < 2; ++b) S.xb[k][b] = *(const gm_u4 *)(xrow[b] + col);
    }
  };
  auto store = [&](const GmStage<HIER> &S, int step, int buf) {
    // Groups past the split's range hold zero weights (their x is finite).
    const bool live = g_begin + step * GM_KG + wg < g_end;
    uint16_t *dst = wt + buf * GM_WT + wr * GM_KS + wg * HGROUP;
    if constexpr (HIER) {
      // A dead group gets s = m = 0 (every weight +0) by select, not by a
      // branch: a branch here makes the compiler wait for every load in flight.
      const float s = live ? __fmul_rn(d, (float)(S.widx & 0xFu)) : 0.0f;
      const float m = live ? __fmul_rn(-dm, (float)(S.widx >> 4)) : 0.0f;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const uint32_t word = S.wv[0][q4];
        uint32_t hv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float lo = __fadd_rn(__fmul_rn((float)((word >> (8 * k)) & 0xFu), s), m);
          const float hi = __fadd_rn(__fmul_rn((float)((word >> (8 * k + 4)) & 0xFu), s), m);
          hv[k] = (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
        }
        *(gm_u4 *)(dst + 8 * q4) = (gm_u4){hv[0], hv[1], hv[2], hv[3]};
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) *(gm_u4 *)(dst + 8 * i) = S.wv[i] & (gm_u4)(live ? ~0u : 0u);
    }
  };

  gm_f4 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = (gm_f4){0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](const GmStage<HIER> &S, int buf) {
    const uint16_t *wb = wt + buf * GM_WT;
#pragma unroll
    for (int k = 0; k < GM_NKK; ++k) {
      const gm_h8 bf0 = __builtin_bit_cast(gm_h8, S.xb[k][0]);
      const gm_h8 bf1 = __builtin_bit_cast(gm_h8, S.xb[k][1]);
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const gm_h8 af = gm_lds8(wb + (a * 16 + r16) * GM_KS + 32 * k + kq);
        acc[a][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf0, acc[a][0], 0, 0, 0);
        acc[a][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf1, acc[a][1], 0, 0, 0);
      }
    }
  };

  // Three register stages rotate, so two steps' loads are always in flight
  // behind the one being multiplied; the W tile of step st sits in LDS
  // buffer st & 1, written from its registers one step ahead. The order of
  // the products (k ascending) is that of a plain K loop. (Measured against
  // running whole rounds of three steps, which keeps every wait partial but
  // multiplies up to two steps of zero weights: slower, 76k against 93k tok/s
  // of config-4 prefill.)
  GmStage<HIER> S0, S1, S2;
  load(S0, 0);
  load(S1, 1);
  store(S0, 0, 0);
  __syncthreads();
  for (int st = 0; st < steps; st += 3) {
    load(S2, st + 2);
    compute(S0, st & 1);
    store(S1, st + 1, (st + 1) & 1);
    __syncthreads();
    if (st + 1 >= steps) break;
    load(S0, st + 3);
    compute(S1, (st + 1) & 1);
    store(S2, st + 2, st & 1);
    __syncthreads();
    if (st + 2 >= steps) break;
    load(S1, st + 4);
    compute(S2, st & 1);
    store(S0, st + 3, (st + 1) & 1);
    __syncthreads();
  }

  // Epilogue through LDS: C[row][token] (lane: rows 4*(lane/16)+i of each
  // 16-row tile, token lane%16) is stored token-major into the W buffers
  // (free after the loop's last barrier), then each token's 64 rows go out as
  // contiguous 16-byte pieces. Written straight from the accumulators, the
  // f32 outputs were 4-byte stores scattered over 16 rows per instruction, and
  // they cost more than the whole K loop (the gate|up tile: 16 of 28 us).
  float *ct = (float *)gm_lds;  // [GM_BN][GM_CS]
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ct[(wave * 32 + b * 16 + r16) * GM_CS + a * 16 + (lane >> 4) * 4 + i] = acc[a][b][i];
  __syncthreads();
  const bool split = gridDim.z > 1;
  float *dst0 = split ? ws + (size_t)blockIdx.z * n * out_f : y;
  const bool vec = (out_f & 3) == 0;
#pragma unroll
  for (int j = 0; j < GM_BM * GM_BN / 4 / GM_THREADS; ++j) {
    const int idx = tid + GM_THREADS * j;
    const int tl = idx / (GM_BM / 4), rl = (idx % (GM_BM / 4)) * 4;
    const int tok = t0 + tl, row = r0 + rl;
    if (tok >= n || row >= out_f) continue;
    float v[4];
    const float4 cv = *(const float4 *)(ct + tl * GM_CS + rl);
    v[0] = cv.x; v[1] = cv.y; v[2] = cv.z; v[3] = cv.w;
    float *dst = dst0 + (size_t)tok * out_f + row;
    if (!split) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (bias && row + e < out_f) v[e] += h2f(bias[row + e]);
    }
    if (vec) {  // out_f % 4 == 0: the four rows exist and the piece is aligned
      if (!split && accum) {
        const float4 o = *(const float4 *)dst;
        v[0] = o.x + v[0]; v[1] = o.y + v[1]; v[2] = o.z + v[2]; v[3] = o.w + v[3];
      }
      *(float4 *)dst = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (row + e < out_f) dst[e] = (!split && accum) ? dst[e] + v[e] : v[e];
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
