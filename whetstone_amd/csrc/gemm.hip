// Multi-token GEMMs for the chunked prefill: y[j] (+)= W x[j] + b for j < n,
// x f16 [n][in_f] token-major, y f32 [n][out_f].
// reference: chunk_gemm.cu:65-176 (int4-hier), 183-258 (fp16), 285-332.
//
// MI355X design
// -------------
// * A block computes a 64-row x 64-token tile of y on MFMA
//   (v_mfma_f32_16x16x32_f16: rows x tokens, f32 accumulate). Four waves each
//   own 16 tokens x 64 rows (4 accumulator tiles). Measured against 128-token
//   tiles (32 tokens per wave): fewer registers per lane and twice the blocks
//   took the 0.5B gate|up tile from 21.3 to 18.7 us, the dequantisation being
//   done once per 64 tokens instead of 128.
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

#include <mutex>

#define HGROUP 32
#define GM_BM 64
#ifndef GM_BN
#define GM_BN 64  // tokens per block (a multiple of 64)
#endif
#define GM_NB (GM_BN / 64)  // 16-token MFMA B fragments per wave (a wave owns GM_BN / 4 tokens)
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
  gm_u4 xb[GM_NKK][GM_NB];
};

// HIER: w = (qw, si, sb) int4-hier-g32; else w is f16 [out_f][in_f].
// Split z = blockIdx.z covers groups [z*gps, min(G, (z+1)*gps)); with one
// split the epilogue writes y, otherwise the f32 tile goes to ws[z].
// SWI: the gate|up form. Tile row k < 32 is gate row a0 + k and row 32 + k is
// up row inter + a0 + k (a0 = 32 * blockIdx.x, out_f = inter), and the
// epilogue writes act[tok][a0 + k] = f16(silu(gate) * up) (never split).
template <bool HIER, bool SWI>
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
  const int wrow = SWI ? (wr < 32 ? min(r0 / 2 + wr, out_f - 1) : out_f + min(r0 / 2 + wr - 32, out_f - 1))
                      : min(r0 + wr, out_f - 1);
  float d = 0.0f, dm = 0.0f;
  if constexpr (HIER) {
    const uint32_t p = sb[wrow];
    d = h2f((uint16_t)(p & 0xFFFFu));
    dm = h2f((uint16_t)(p >> 16));
  }
  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  const uint16_t *xrow[GM_NB];
#pragma unroll
  for (int b = 0; b < GM_NB; ++b)
    xrow[b] = x + (size_t)min(t0 + wave * 16 * GM_NB + b * 16 + r16, n - 1) * in_f + kq;

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
      for (int b = 0; b < GM_NB; ++b) S.xb[k][b] = *(const gm_u4 *)(xrow[b] + col);
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

  gm_f4 acc[4][GM_NB];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < GM_NB; ++b) acc[a][b] = (gm_f4){0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](const GmStage<HIER> &S, int buf) {
    const uint16_t *wb = wt + buf * GM_WT;
#pragma unroll
    for (int k = 0; k < GM_NKK; ++k) {
      gm_h8 bf[GM_NB];
#pragma unroll
      for (int b = 0; b < GM_NB; ++b) bf[b] = __builtin_bit_cast(gm_h8, S.xb[k][b]);
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const gm_h8 af = gm_lds8(wb + (a * 16 + r16) * GM_KS + 32 * k + kq);
#pragma unroll
        for (int b = 0; b < GM_NB; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[b], acc[a][b], 0, 0, 0);
      }
    }
  };

  // Three register stages rotate, so two steps' loads are always in flight
  // behind the one being multiplied; the W tile of step st sits in LDS
  // buffer st & 1, written from its registers one step ahead. The order of
  // the products (k ascending) is that of a plain K loop. (Measured against
  // running whole rounds of three steps, which keeps every wait partial but
  // multiplies up to two steps of zero weights: slower, 76k against 93k tok/s
  // of config-4 prefill.) Whole rounds run in a loop with no exit inside it,
  // the one or two remaining steps after it: with an exit after each step,
  // the compiler moved the 16 accumulators between AGPRs every step (48
  // v_accvgpr_mov a round).
  GmStage<HIER> S0, S1, S2;
  load(S0, 0);
  load(S1, 1);
  store(S0, 0, 0);
  __syncthreads();
#define GM_STEP_A                      \
  load(S2, st + 2);                    \
  compute(S0, st & 1);                 \
  store(S1, st + 1, (st + 1) & 1);     \
  __syncthreads();
#define GM_STEP_B                      \
  load(S0, st + 3);                    \
  compute(S1, (st + 1) & 1);           \
  store(S2, st + 2, st & 1);           \
  __syncthreads();
#define GM_STEP_C                      \
  load(S1, st + 4);                    \
  compute(S2, st & 1);                 \
  store(S0, st + 3, (st + 1) & 1);     \
  __syncthreads();
  int st = 0;
  for (; st + 3 <= steps; st += 3) {
    GM_STEP_A
    GM_STEP_B
    GM_STEP_C
  }
  if (st < steps) {
    GM_STEP_A
  }
  if (st + 1 < steps) {
    GM_STEP_B
  }
#undef GM_STEP_A
#undef GM_STEP_B
#undef GM_STEP_C

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
    for (int b = 0; b < GM_NB; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ct[(wave * 16 * GM_NB + b * 16 + r16) * GM_CS + a * 16 + (lane >> 4) * 4 + i] =
            acc[a][b][i];
  __syncthreads();
  if constexpr (SWI) {
    // act[tok][a0 + k] for k < 32: the same expression as swiglu_kernel.
    uint16_t *act = (uint16_t *)y;
    const int a0 = r0 / 2;
#pragma unroll
    for (int j = 0; j < GM_BN * 32 / 4 / GM_THREADS; ++j) {
      const int idx = tid + GM_THREADS * j;
      const int tl = idx / 8, kl = (idx % 8) * 4;
      const int tok = t0 + tl;
      if (tok >= n) continue;
      uint16_t hv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float g = ct[tl * GM_CS + kl + e], u = ct[tl * GM_CS + 32 + kl + e];
        hv[e] = f2h(g / (1.0f + __expf(-g)) * u);
      }
      uint16_t *dst = act + (size_t)tok * out_f + a0 + kl;
      if ((out_f & 3) == 0 && a0 + kl + 3 < out_f) {
        *(uint2 *)dst = make_uint2(hv[0] | ((uint32_t)hv[1] << 16), hv[2] | ((uint32_t)hv[3] << 16));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (a0 + kl + e < out_f) dst[e] = hv[e];
      }
    }
    return;
  }
  const bool split = gridDim.z > 1 || ws;
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

// ------------------------------------------------------------ wide tiles
//
// gemm_wide_kernel: the same product on 64-row x 256-token tiles -- a whole
// chunk's tokens -- with the 32x32x16 MFMA (v_mfma_f32_32x32x16_f16). Eight
// waves each own 32 tokens x 64 rows (two 32 x 32 accumulator tiles).
//
// * The weights are dequantised once per 256 tokens. (The 64 x 64 tiles
//   dequantise each weight four times per chunk; on the 7B shapes that VALU
//   work alone was about 40% of their time.) A thread dequantises one packed
//   word (8 weights) per step into the LDS W tile, as w = q * s + m in one f32
//   fma -- q * s is exact in f32 (a 4-bit integer times an f16 times a 4-bit
//   integer), so the single rounding equals the quantiser's two -- rounded to
//   f16. On the 256-token tiles each W tile is dequantised two steps before
//   its use into one of four LDS buffers, with a barrier after every other
//   step (config-4 prefill 450-456k -> 461-465k tok/s; bit-identical); the
//   128-token tiles keep two buffers and a barrier per step.
// * x goes memory -> LDS by DMA (global_load_lds_dwordx4: 16 bytes per lane
//   land at M0 + 16 * lane), three steps in flight in an LDS ring, with no
//   registers held for it. Each wave loads only its own 32 tokens (a
//   coalesced 128-byte row per 8 lanes), so the ring needs no barrier. In LDS
//   a token's 16-byte chunk c sits at slot c ^ (token % 8), and each DMA
//   block of 8 tokens is followed by 64 bytes of padding, so the MFMA operand
//   reads (32 tokens, one chunk) spread over the banks. (Measured against
//   four waves of 64 tokens, which halve the W reads from LDS but leave one
//   wave per SIMD: 7B gate|up 148 against 134 us.)
// * The packed weights (a dword and an index byte per thread per step) are
//   loaded four steps ahead into a register ring.
// * Every load of the loop is issued by inline asm with the wait counted by
//   hand: left to itself the compiler sank each step's loads down to their
//   first use, one step later, leaving one step in flight. Per step a thread
//   issues 4 DMA ops and then 2 weight loads (x(q) just before the weights
//   of step q + 2). When step st is computed, the wait lets through only the
//   ops issued after the later of x(st) and the weights it dequantises next
//   (GwShape::VMCNT: 12 on the 256-token tiles, whose next weights are
//   step st + 2's, issued after x(st); 20 on the 128-token tiles, whose next
//   weights are step st + 1's, issued before x(st)).
// * Hazard of that scheme: the compiler takes an asm load's output register
//   as written when the load issues, so it may copy or rename a ring
//   register while its load is still landing. Each ring slot must keep its
//   physical registers from the prologue through every loop round and the
//   tail, as the shipped variants do (read off their ISA: the same eight or
//   sixteen destination registers in every round). A 128-row variant (four
//   accumulator tiles a wave, 168 VGPRs) broke this: one ring register was
//   renamed across the loop's back edge and rows 96..127 of some tiles came
//   out wrong (tests/test_gpu_kernels.py's 896 -> 33000 case caught it). It
//   is not built.
// * K advances two groups (64 columns) per step; split-K and the epilogue
//   (through LDS, token-major) are those of gemm_mfma_kernel. SWI: rows
//   0..31 of a tile are gate rows a0..a0+31 and rows 32..63 the up rows
//   inter+a0.., and the epilogue writes act = f16(silu(gate) * up).
#define GW_BM 64
#define GW_ROPE_HD 64                   // head_dim of the RoPE epilogue: one tile's rows
#define GW_KG 2
#define GW_KC (GW_KG * HGROUP)          // 64 columns per step
#define GW_KS (GW_KC + 8)               // W tile row stride in halves
#define GW_WT (GW_BM * GW_KS)           // halves of one W buffer
#define GW_NKK (GW_KC / 16)             // MFMA k-steps per step
#define GW_CS (GW_BM + 4)               // epilogue tile row stride (floats)
#define GW_DX 3                         // x steps in flight (LDS ring)
#define GW_DW 4                         // packed-weight steps in flight (registers)
#define GW_XPAD 64                      // bytes between DMA blocks: t and t+8 on other banks
#define GW_XWAVE (4 * (1024 + GW_XPAD)) // bytes of a wave's 32 tokens in one stage
static_assert(GW_DW == GW_DX + 1, "the wait count assumes the weights lead x by one step");

// NWV waves of 32 tokens: 256-token tiles (8 waves, one packed word per
// thread per step) or 128-token tiles (4 waves, two words per thread) for
// shapes whose 256-token tiles leave CUs idle.
template <int NWV>
struct GwShape {
  static constexpr int THREADS = 64 * NWV;
  static constexpr int BN = 32 * NWV;
  static constexpr int RPT = 512 / THREADS;           // W words per thread per step
  static constexpr int XSTAGE = NWV * GW_XWAVE;       // bytes of one x ring stage
  static constexpr int LDS_X = GW_DX * XSTAGE;
  // Steps ahead that W is dequantised into LDS: 2 for the 256-token tiles
  // (four W buffers, a barrier every two steps), 1 for the 128-token ones
  // (two buffers, a barrier every step: with the weights two steps ahead the
  // compiler renamed a register of their load ring across the loop's back
  // edge).
  static constexpr int WA = NWV == 8 ? 2 : 1;
  static constexpr int WB = 2 * WA;                   // W tile buffers
  static constexpr int LDS_W = WB * GW_WT * 2;
  static constexpr int LDS_C = BN * GW_CS * 4;
  static constexpr int LDS = LDS_X + LDS_W > LDS_C ? LDS_X + LDS_W : LDS_C;
  // Ops issued after the later of x(st) and W(st + WA) when step st is
  // multiplied (4 DMA ops and 2 RPT weight loads per step, x(q) issued just
  // before W(q + 2)): WA = 1, after x(st): W(st + 2) and the two steps
  // since; WA = 2, after W(st + 2): the two steps since.
  static constexpr int VMCNT = 4 * (GW_DX - 1) + 2 * RPT * (GW_DX + 1 - WA);
  static_assert(RPT * THREADS == 512, "64 rows x 2 groups x 4 words per step");
  static_assert(LDS <= 160 * 1024, "one CU's LDS");
};

typedef float gm_f16v __attribute__((ext_vector_type(16)));

// The qkv GEMM's RoPE epilogue (ROPE tiles, head_dim 64 = one tile's rows):
// what gemm_reduce_rope_kernel does after an unsplit GEMM, per token.
struct GwRope {
  uint16_t *k_cache, *v_cache;
  const float *cos_tab, *sin_tab;
  const uint16_t *q_norm_w, *k_norm_w;
  int n_q, n_kv, pos0, max_seq;
  float eps;
};

// RT tokens of one head of 64, stage by stage so that the tokens' dependent
// chains (cross-lane swap, norm reduction, square root) overlap: lane j holds
// column j of each (the value after the GEMM and bias); q is QK-normed,
// rotated and stored to its row, k stored to its row as computed and rotated
// into the cache, v stored to its row and the cache. The arithmetic is
// gemm_reduce_rope_kernel's NARROW form (column j in lane j, the rotation
// partner over a 32-lane swap, the norm's pair sums over the wave), so the
// two give the same bits. ok[u]: token u exists (uniform in the wave).
template <int RT>
__device__ __forceinline__ void gw_rope_tokens(const float (&mine)[RT], const bool (&ok)[RT],
                                               const int (&tok)[RT], int h, float *__restrict__ y,
                                               int row_stride, const GwRope &re,
                                               const float (&c)[RT], const float (&s)[RT],
                                               float gq1, float gq2, int lane) {
  const int hd = GW_ROPE_HD;
  const bool hi = lane >= 32;
  int pos[RT];
#pragma unroll
  for (int u = 0; u < RT; ++u) pos[u] = min(max(re.pos0 + tok[u], 0), re.max_seq - 1);
  if (h >= re.n_q + re.n_kv) {  // v
    const int kvh = h - re.n_q - re.n_kv;
#pragma unroll
    for (int u = 0; u < RT; ++u)
      if (ok[u]) {
        y[(size_t)tok[u] * row_stride + h * hd + lane] = mine[u];
        re.v_cache[((size_t)kvh * re.max_seq + pos[u]) * hd + lane] = f2h(mine[u]);
      }
    return;
  }
  const bool is_q = h < re.n_q;
  float x1[RT], x2[RT];
#pragma unroll
  for (int u = 0; u < RT; ++u) {
    const float other = __shfl_xor(mine[u], 32);
    x1[u] = hi ? other : mine[u];
    x2[u] = hi ? mine[u] : other;
  }
  if (is_q ? re.q_norm_w : re.k_norm_w) {
    float ss[RT];
#pragma unroll
    for (int u = 0; u < RT; ++u) ss[u] = wave_sum(!hi ? fmaf(x1[u], x1[u], x2[u] * x2[u]) : 0.0f);
#pragma unroll
    for (int u = 0; u < RT; ++u) {
      const float sc = 1.0f / sqrtf(ss[u] / (float)hd + re.eps);
      x1[u] = x1[u] * sc * gq1;
      x2[u] = x2[u] * sc * gq2;
    }
  }
#pragma unroll
  for (int u = 0; u < RT; ++u) {
    if (!ok[u]) continue;
    const float lo = rope_lo(x1[u], x2[u], c[u], s[u]), hv = rope_hi(x1[u], x2[u], c[u], s[u]);
    float *row = y + (size_t)tok[u] * row_stride;
    if (is_q) {
      row[h * hd + lane] = hi ? hv : lo;
    } else {
      row[h * hd + lane] = mine[u];  // k as computed
      re.k_cache[((size_t)(h - re.n_q) * re.max_seq + pos[u]) * hd + lane] = f2h(hi ? hv : lo);
    }
  }
}

template <bool HIER, bool SWI, int NWV, bool ROPE = false>
__global__ __launch_bounds__(64 * NWV, 1) void gemm_wide_kernel(
    const void *__restrict__ w, const uint8_t *__restrict__ si, const uint32_t *__restrict__ sb,
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ bias, float *__restrict__ y,
    float *__restrict__ ws, int in_f, int out_f, int n, int accum, int gps, GwRope re) {
#pragma clang fp contract(off)
  static_assert(HIER, "the wide tiles take int4-hier weights");
  using S = GwShape<NWV>;
  constexpr int RPT = S::RPT, THREADS = S::THREADS, BN = S::BN;
  extern __shared__ __align__(16) unsigned char gw_lds[];
  const uint32_t lds0 = (uint32_t)(uintptr_t)gw_lds;  // byte address of the ring
  uint16_t *wt = (uint16_t *)(gw_lds + S::LDS_X);      // [2][GW_BM][GW_KS]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: M0 takes it
  const int r0 = blockIdx.x * GW_BM, t0 = blockIdx.y * BN;
  const int G = in_f / HGROUP;
  const int g_begin = blockIdx.z * gps, g_end = min(G, g_begin + gps);
  const int steps = (g_end - g_begin + GW_KG - 1) / GW_KG;

  // W assignment: word u = tid + THREADS j (j < RPT) is tile row wr = u / 8,
  // group wg = (u / 4) % 2 of the step, packed word ww = u % 4 of the group
  // (columns 8 ww .. 8 ww + 7).
  const int wg = (tid >> 2) & 1, ww = tid & 3;
  int wr[RPT];
  uint32_t sbv[RPT];
  const uint32_t *wq_base[RPT];
  const uint8_t *wi_base[RPT];
  float d[RPT], dm[RPT];  // set once the prologue's loads land
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    wr[j] = (tid + THREADS * j) >> 3;
    const int wrow = SWI ? (wr[j] < 32 ? min(r0 / 2 + wr[j], out_f - 1)
                                       : out_f + min(r0 / 2 + wr[j] - 32, out_f - 1))
                         : min(r0 + wr[j], out_f - 1);
    // The row's (d, dmin), loaded with the prologue's loads (by asm, so that
    // the compiler's own wait for it does not wait for those too).
    asm volatile("global_load_dword %0, %1, off" : "=v"(sbv[j]) : "v"(sb + wrow) : "memory");
    // This word's and index's addresses at step 0; a step adds 32 bytes (qw)
    // and 2 (si). The group index is clamped per step.
    wq_base[j] = (const uint32_t *)w + (size_t)wrow * (in_f / 8) + ww;
    wi_base[j] = si + (size_t)wrow * G;
    d[j] = dm[j] = 0.0f;
  }

  // x DMA: instruction i of wave `wave` covers tokens 8i .. 8i+7 of the wave's
  // 32; lane l loads token 8i + l/8, chunk (l % 8) ^ (token % 8).
  uint32_t xoff[4];  // byte offset of the lane's chunk at column 0
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tl = 8 * i + (lane >> 3);
    const int tok = min(t0 + wave * 32 + tl, n - 1);
    const int c = (lane & 7) ^ (tl & 7);
    xoff[i] = (uint32_t)tok * (uint32_t)in_f * 2u + (uint32_t)c * 16u;
  }
  const uint32_t wave_x = lds0 + (uint32_t)wave * GW_XWAVE;

  auto issue_x = [&](int step) {  // 4 DMA ops
    // The stage was last read by this wave's own step - GW_DX: its LDS reads
    // must be complete before the DMA can land (with a barrier after every
    // step, its fence waited for them).
    if constexpr (S::WA == 2) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    step = min(step, steps - 1);
    const int col = min((g_begin + step * GW_KG) * HGROUP, in_f - GW_KC);
    const uint32_t stage = wave_x + (uint32_t)(step % GW_DX) * S::XSTAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t m0 = stage + (uint32_t)i * (1024u + GW_XPAD);
      const uint32_t off = xoff[i] + (uint32_t)col * 2u;
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                   :: "s"(m0), "v"(off), "s"(x) : "memory");
    }
  };
  uint32_t wq[GW_DW][RPT], wi[GW_DW][RPT];
  auto issue_w = [&](int step, uint32_t (&q)[RPT], uint32_t (&ix)[RPT]) {  // 2 RPT ops
    step = min(step, steps - 1);
    const int g = min(g_begin + step * GW_KG + wg, G - 1);
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const uint32_t *qa = wq_base[j] + (size_t)g * 4;
      const uint8_t *ia = wi_base[j] + g;
      asm volatile("global_load_dword %0, %1, off" : "=v"(q[j]) : "v"(qa) : "memory");
      asm volatile("global_load_ubyte %0, %1, off" : "=v"(ix[j]) : "v"(ia) : "memory");
    }
  };
  auto store_w = [&](const uint32_t (&q)[RPT], const uint32_t (&ix)[RPT], int step, int buf) {
    const bool live = g_begin + step * GW_KG + wg < g_end;
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const float s = live ? __fmul_rn(d[j], (float)(ix[j] & 0xFu)) : 0.0f;
      const float m = live ? __fmul_rn(-dm[j], (float)((ix[j] >> 4) & 0xFu)) : 0.0f;
      uint32_t hv[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float lo = __builtin_fmaf((float)((q[j] >> (8 * k)) & 0xFu), s, m);
        const float hi = __builtin_fmaf((float)((q[j] >> (8 * k + 4)) & 0xFu), s, m);
        hv[k] = (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
      }
      *(gm_u4 *)(wt + buf * GW_WT + wr[j] * GW_KS + wg * HGROUP + 8 * ww) =
          (gm_u4){hv[0], hv[1], hv[2], hv[3]};
    }
  };
  // Wait until at most `n` ops are outstanding; the registers of W ring slot
  // `u` are operands, so that no use of them is scheduled above the wait.
#define GW_WAIT(u, n_)                                                               \
  if constexpr (RPT == 1)                                                            \
    asm volatile("s_waitcnt vmcnt(%2)" : "+v"(wq[u][0]), "+v"(wi[u][0])              \
                 : "n"(n_) : "memory");                                              \
  else                                                                               \
    asm volatile("s_waitcnt vmcnt(%4)"                                               \
                 : "+v"(wq[u][0]), "+v"(wi[u][0]), "+v"(wq[u][RPT - 1]), "+v"(wi[u][RPT - 1]) \
                 : "n"(n_) : "memory");

  gm_f16v acc[2];  // [row tile]
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[a][r] = 0.0f;

  const int l32 = lane & 31, kh = lane >> 5;
  // token l32 sits in DMA block l32 / 8, row l32 % 8
  const uint32_t xrow0 = (uint32_t)(l32 >> 3) * (1024u + GW_XPAD) + (uint32_t)(l32 & 7) * 128u;
  auto compute = [&](int step) {
    const uint16_t *wb = wt + (step % S::WB) * GW_WT + l32 * GW_KS + 8 * kh;
    const unsigned char *xs = gw_lds + (wave_x - lds0) + (uint32_t)(step % GW_DX) * S::XSTAGE + xrow0;
#pragma unroll
    for (int k = 0; k < GW_NKK; ++k) {
      const int c = 2 * k + kh;
      const gm_h8 b = *(const gm_h8 *)(xs + (uint32_t)((c ^ (l32 & 7)) * 16));
      const gm_h8 a0 = gm_lds8(wb + 16 * k);
      const gm_h8 a1 = gm_lds8(wb + 32 * GW_KS + 16 * k);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b, acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b, acc[1], 0, 0, 0);
    }
  };

  // Prologue in the loop's issue pattern: W(0), W(1), then x(q) followed by
  // W(q + 2) for q < GW_DX - 1.
  issue_w(0, wq[0], wi[0]);
  issue_w(1, wq[1], wi[1]);
#pragma unroll
  for (int q = 0; q < GW_DX - 1; ++q) {
    issue_x(q);
    issue_w(q + 2, wq[q + 2], wi[q + 2]);
  }
  // WA = 1: sb and W(0) are followed by S::VMCNT ops (W(1), x(0), W(2),
  // x(1), W(3)); WA = 2: sb, W(0) and W(1) by x(0), W(2), x(1), W(3).
  if constexpr (S::WA == 2) {
    static_assert(RPT == 1, "two steps ahead: the 256-token tiles only");
    asm volatile("s_waitcnt vmcnt(%5)"
                 : "+v"(wq[0][0]), "+v"(wi[0][0]), "+v"(wq[1][0]), "+v"(wi[1][0]), "+v"(sbv[0])
                 : "n"(S::VMCNT) : "memory");
  } else if constexpr (RPT == 1) {
    asm volatile("s_waitcnt vmcnt(%3)" : "+v"(wq[0][0]), "+v"(wi[0][0]), "+v"(sbv[0])
                 : "n"(S::VMCNT) : "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(%6)"
                 : "+v"(wq[0][0]), "+v"(wi[0][0]), "+v"(wq[0][RPT - 1]), "+v"(wi[0][RPT - 1]),
                   "+v"(sbv[0]), "+v"(sbv[RPT - 1])
                 : "n"(S::VMCNT) : "memory");
  }
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    d[j] = h2f((uint16_t)(sbv[j] & 0xFFFFu));
    dm[j] = h2f((uint16_t)(sbv[j] >> 16));
  }
  store_w(wq[0], wi[0], 0, 0);
  if constexpr (S::WA == 2) store_w(wq[1], wi[1], 1, 1);
  __syncthreads();

  // One step: issue x(st + GW_DX - 1) and W(st + GW_DW) (into W(st)'s slot,
  // stored WA steps ago), wait for x(st) and W(st + WA), multiply, dequantise
  // W(st + WA) into W buffer (st + WA) % WB. With WA = 1 a barrier after
  // every step. With WA = 2 a barrier after every odd step: W(st + 2) is
  // stored at step st and read at step st + 2, with a barrier after st or
  // st + 1 between; its buffer held W(st - 2), read at step st - 2, with a
  // barrier after st - 2 or st - 1 between. (One barrier a step with two
  // buffers: batched 0.5B gate|up 141 us; none at all, results wrong, 112
  // us.)
#define GW_STEP(U)                                                              \
  {                                                                             \
    const int st = st0 + (U);                                                   \
    issue_x(st + GW_DX - 1);                                                    \
    issue_w(st + GW_DW, wq[(U) % GW_DW], wi[(U) % GW_DW]);                      \
    GW_WAIT(((U) + S::WA) % GW_DW, S::VMCNT)                                    \
    compute(st);                                                                \
    store_w(wq[((U) + S::WA) % GW_DW], wi[((U) + S::WA) % GW_DW], st + S::WA,   \
            (st + S::WA) % S::WB);                                              \
    if (S::WA == 1 || ((U) & 1)) __syncthreads();                               \
  }
  // Whole rounds of GW_DW steps in a loop with no exit inside it, then the
  // remaining steps. (With a `break` after each step inside one loop, the
  // compiler rotated the accumulators through other registers every step:
  // 16 v_mov_b64 behind an MFMA drain.)
  int st0 = 0;
  for (; st0 + GW_DW <= steps; st0 += GW_DW) {
    GW_STEP(0)
    GW_STEP(1)
    GW_STEP(2)
    GW_STEP(3)
  }
  if (st0 < steps) GW_STEP(0)
  if (st0 + 1 < steps) GW_STEP(1)
  if (st0 + 2 < steps) GW_STEP(2)
#undef GW_STEP
#undef GW_WAIT
  // Clamped look-ahead DMAs may still be landing in the ring, which the
  // epilogue tile overlaps; and the look-ahead weight loads of the last
  // steps may still be landing in their ring registers. Those registers are
  // operands of this wait, so the compiler keeps them reserved until it (a
  // dead load destination it took back earlier would be overwritten when the
  // load lands).
  if constexpr (RPT == 1)
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(wq[0][0]), "+v"(wi[0][0]), "+v"(wq[1][0]), "+v"(wi[1][0]),
                   "+v"(wq[2][0]), "+v"(wi[2][0]), "+v"(wq[3][0]), "+v"(wi[3][0])
                 :: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(wq[0][0]), "+v"(wi[0][0]), "+v"(wq[1][0]), "+v"(wi[1][0]),
                   "+v"(wq[2][0]), "+v"(wi[2][0]), "+v"(wq[3][0]), "+v"(wi[3][0]),
                   "+v"(wq[0][1]), "+v"(wi[0][1]), "+v"(wq[1][1]), "+v"(wi[1][1]),
                   "+v"(wq[2][1]), "+v"(wi[2][1]), "+v"(wq[3][1]), "+v"(wi[3][1])
                 :: "memory");
  __syncthreads();

  // RoPE epilogue: the rotation angles of the wave's tokens (every NWV-th of
  // the tile's), loaded while the accumulators go through LDS.
  constexpr int RTOK = ROPE ? BN / NWV : 1;
  float rc[RTOK], rsn[RTOK];
  if constexpr (ROPE) {
    const int half = GW_ROPE_HD / 2, jj = lane & 31;
#pragma unroll
    for (int i = 0; i < RTOK; ++i) {
      const int pos = min(max(re.pos0 + t0 + wave + i * NWV, 0), re.max_seq - 1);
      rc[i] = re.cos_tab[(size_t)pos * half + jj];
      rsn[i] = re.sin_tab[(size_t)pos * half + jj];
    }
  }

  // Epilogue through LDS, token-major: accumulator r of row tile a holds row
  // 32 a + 8 (r / 4) + 4 (lane / 32) + r % 4, token lane % 32 of the wave.
  float *ct = (float *)gw_lds;  // [BN][GW_CS]
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = a * 32 + 8 * (r >> 2) + 4 * kh + (r & 3);
      ct[(wave * 32 + l32) * GW_CS + row] = acc[a][r];
    }
  __syncthreads();
  if constexpr (ROPE) {
    // the tile's 64 rows are head h; each wave takes every NWV-th token
    static_assert(!SWI && GW_BM == GW_ROPE_HD, "the RoPE tiles are one head of the plain GEMM");
    const int h = r0 / GW_BM, half = GW_ROPE_HD / 2, jj = lane & 31;
    const float bj = bias ? h2f(bias[r0 + lane]) : 0.0f;
    const uint16_t *g = h < re.n_q ? re.q_norm_w : re.k_norm_w;
    const float gq1 = g ? h2f(g[jj]) : 0.0f, gq2 = g ? h2f(g[jj + half]) : 0.0f;
    constexpr int RT = 4;
    static_assert(RTOK % RT == 0, "tokens in groups of four");
#pragma unroll
    for (int i0 = 0; i0 < RTOK; i0 += RT) {
      float mine[RT], c[RT], sn[RT];
      bool ok[RT];
      int tok[RT];
#pragma unroll
      for (int u = 0; u < RT; ++u) {
        const int tl = wave + (i0 + u) * NWV;
        tok[u] = t0 + tl;
        ok[u] = tok[u] < n;
        mine[u] = ct[tl * GW_CS + lane];
        if (bias) mine[u] += bj;
        c[u] = rc[i0 + u];
        sn[u] = rsn[i0 + u];
      }
      gw_rope_tokens<RT>(mine, ok, tok, h, y, out_f, re, c, sn, gq1, gq2, lane);
    }
    return;
  }
  if constexpr (SWI) {
    uint16_t *act = (uint16_t *)y;
    const int a0 = r0 / 2;
#pragma unroll
    for (int j = 0; j < BN * 32 / 4 / THREADS; ++j) {
      const int idx = tid + THREADS * j;
      const int tl = idx / 8, kl = (idx % 8) * 4;
      const int tok = t0 + tl;
      if (tok >= n) continue;
      uint16_t hv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float g = ct[tl * GW_CS + kl + e], u = ct[tl * GW_CS + 32 + kl + e];
        hv[e] = f2h(g / (1.0f + __expf(-g)) * u);
      }
      uint16_t *dst = act + (size_t)tok * out_f + a0 + kl;
      if ((out_f & 3) == 0 && a0 + kl + 3 < out_f) {
        *(uint2 *)dst = make_uint2(hv[0] | ((uint32_t)hv[1] << 16), hv[2] | ((uint32_t)hv[3] << 16));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (a0 + kl + e < out_f) dst[e] = hv[e];
      }
    }
    return;
  }
  const bool split = gridDim.z > 1 || ws;
  float *dst0 = split ? ws + (size_t)blockIdx.z * n * out_f : y;
  const bool vec = (out_f & 3) == 0;
#pragma unroll 4
  for (int j = 0; j < GW_BM * BN / 4 / THREADS; ++j) {
    const int idx = tid + THREADS * j;
    const int tl = idx / (GW_BM / 4), rl = (idx % (GW_BM / 4)) * 4;
    const int tok = t0 + tl, row = r0 + rl;
    if (tok >= n || row >= out_f) continue;
    float v[4];
    const float4 cv = *(const float4 *)(ct + tl * GW_CS + rl);
    v[0] = cv.x; v[1] = cv.y; v[2] = cv.z; v[3] = cv.w;
    float *dst = dst0 + (size_t)tok * out_f + row;
    if (!split) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (bias && row + e < out_f) v[e] += h2f(bias[row + e]);
    }
    if (vec) {
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

// sum over the splits of element i (stride `total`), in split order: the
// loads are issued four at a time (a batch past the last split re-reads it),
// the adds stay in order. A 4-way split costs 4 loads, not GM_MAXSPLIT.
#define GM_MAXSPLIT 16
__device__ __forceinline__ float split_sum(const float *__restrict__ ws, size_t i, size_t total,
                                           int splits) {
  if (splits == 1) return ws[i];  // (the batch of four below would load it four times)
  float t = 0.0f;
  for (int z0 = 0; z0 < splits; z0 += 4) {
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = ws[(size_t)min(z0 + e, splits - 1) * total + i];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (z0 + e < splits) t = (z0 + e == 0) ? v[e] : t + v[e];
  }
  return t;
}

// y = (accum ? y : 0) + (sum of the splits in split order) + bias.
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(const float *__restrict__ ws,
                                                                const uint16_t *__restrict__ bias,
                                                                float *__restrict__ y, int out_f,
                                                                int n, int splits, int accum) {
  const size_t total = (size_t)n * out_f;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    float v = split_sum(ws, i, total, splits);
    if (bias) v += h2f(bias[i % out_f]);
    y[i] = accum ? y[i] + v : v;
  }
}

// Fused reduce + RMSNorm (a token per 512-thread block): x = (accum ? x : 0) +
// (sum of the splits in split order) + bias, staged in LDS, then
// h = f16(x * rms * w) with rms_scale512's order, so both outputs equal
// gemm_split_reduce_kernel followed by rmsnorm_kernel bit for bit.
template <int CPT>
__global__ __launch_bounds__(512) void gemm_reduce_norm_kernel(
    const float *__restrict__ ws, const uint16_t *__restrict__ bias, float *__restrict__ y,
    int out_f, int n, int splits, int accum, const uint16_t *__restrict__ nw, float eps,
    uint16_t *__restrict__ h) {
  __shared__ float red[16];
  extern __shared__ float xrow[];  // [out_f]: the reduced row
  const int tok = blockIdx.x;
  const size_t total = (size_t)n * out_f, base = (size_t)tok * out_f;
  if constexpr (CPT > 0) {
    // CPT columns per thread (out_f <= 512 * CPT): every global load (the
    // splits, the bias, the residual, the norm weight) issued before the
    // first wait, the columns past out_f clamped to the last one and not
    // stored.
    float t[CPT], w[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = min((int)threadIdx.x + 512 * k, out_f - 1);
      w[k] = h2f(nw[c]);
      float v = split_sum(ws, base + c, total, splits);
      if (bias) v += h2f(bias[c]);
      t[k] = accum ? y[base + c] + v : v;
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = threadIdx.x + 512 * k;
      if (c < out_f) {
        y[base + c] = t[k];
        xrow[c] = t[k];
      }
    }
    __syncthreads();
    const float sc = rms_scale512(xrow, out_f, eps, red);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = threadIdx.x + 512 * k;
      if (c < out_f) h[base + c] = f2h(t[k] * sc * w[k]);
    }
    return;
  }
  // 1. the reduce, coalesced (thread t: elements t, t+512, ...)
  for (int c = threadIdx.x; c < out_f; c += 512) {
    float t = split_sum(ws, base + c, total, splits);
    if (bias) t += h2f(bias[c]);
    t = accum ? y[base + c] + t : t;
    y[base + c] = t;
    xrow[c] = t;
  }
  __syncthreads();
  // 2. the RMS in rms_scale512's order, from LDS
  const float sc = rms_scale512(xrow, out_f, eps, red);
  // 3. h, coalesced
  for (int c = threadIdx.x; c < out_f; c += 512)
    h[base + c] = f2h(xrow[c] * sc * h2f(nw[c]));
}

// gemm_reduce_norm_kernel for rows of out_f <= 4096 columns, out_f % 8 == 0:
// a token per block of 64 * ceil(out_f / 512) threads, thread t holding the
// eight columns 8t..8t+7 (two 16-byte loads per operand). rms_scale512 gives
// thread t of its 512 exactly these eight columns, in this order, for rows of
// at most 4096 columns, and its threads past the row add zeros, as the missing
// waves here do: both outputs are bit-identical to the 512-thread form. (The
// 512-thread form with two columns a thread ran 16 us over 4096 tokens of 896
// columns: 4096 barrier-bound blocks.)
__global__ __launch_bounds__(512) void gemm_reduce_norm8_kernel(
    const float *__restrict__ ws, const uint16_t *__restrict__ bias, float *__restrict__ y,
    int out_f, int n, int splits, int accum, const uint16_t *__restrict__ nw, float eps,
    uint16_t *__restrict__ h) {
  __shared__ float red[16];
  const int tok = blockIdx.x;
  const size_t total = (size_t)n * out_f, base = (size_t)tok * out_f;
  const int c0 = 8 * (int)threadIdx.x;
  const bool on = c0 < out_f;
  float t[8];
  float acc = 0.0f;
  if (on) {
    float v[8];
    const float4 *w0 = (const float4 *)(ws + base + c0);
    float4 a = w0[0], b = w0[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    for (int z = 1; z < splits; ++z) {  // split order, as split_sum
      const float4 *wz = (const float4 *)(ws + (size_t)z * total + base + c0);
      a = wz[0];
      b = wz[1];
      v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w;
      v[4] += b.x; v[5] += b.y; v[6] += b.z; v[7] += b.w;
    }
    if (bias) {
      const uint4 bb = *(const uint4 *)(bias + c0);
      const uint32_t bw[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] += h2f((uint16_t)(bw[e] & 0xFFFFu));
        v[2 * e + 1] += h2f((uint16_t)(bw[e] >> 16));
      }
    }
    if (accum) {
      const float4 *yr = (const float4 *)(y + base + c0);
      a = yr[0];
      b = yr[1];
      const float yv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = yv[e] + v[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = v[e];
    }
    float4 *yo = (float4 *)(y + base + c0);
    yo[0] = make_float4(t[0], t[1], t[2], t[3]);
    yo[1] = make_float4(t[4], t[5], t[6], t[7]);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf(t[e], t[e], acc);
  }
  acc = block_sum(acc, red);
  const float sc = 1.0f / sqrtf(acc / (float)out_f + eps);
  if (!on) return;
  const uint4 gw = *(const uint4 *)(nw + c0);
  const uint32_t g[4] = {gw.x, gw.y, gw.z, gw.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint16_t lo = f2h(t[2 * e] * sc * h2f((uint16_t)(g[e] & 0xFFFFu)));
    const uint16_t hi = f2h(t[2 * e + 1] * sc * h2f((uint16_t)(g[e] >> 16)));
    o[e] = (uint32_t)lo | ((uint32_t)hi << 16);
  }
  *(uint4 *)(h + base + c0) = make_uint4(o[0], o[1], o[2], o[3]);
}

// Fused reduce + QK-norm + RoPE + KV append (head_dim <= 128, so a head's
// halves are one wave): the head's qkv values are summed from the splits
// (+ bias) exactly as gemm_split_reduce_kernel does and stored to qkv, then
// rotated exactly as rope_cache_kernel does (q back into qkv, k and v to the
// cache). The QK-norm sum is the wave's sum, which is what a one-wave block's
// block_sum returns (its second stage adds the one wave total to 0).
//
// A wave (a block) per token and group of RR_GROUP heads: it issues the
// group's loads and the token's rotation factors before it rotates the first
// head. With a wave per (token, head) item the kernel was bound by waves in
// flight: 73,728 short waves, each a memory round trip (25.7 us over 4096
// tokens x 18 heads with QK-norm, 38 MB; now 21.4 us, 14.1 without QK-norm).
// Over one 256-token chunk (the qkv sum split over K there) groups of eight
// leave too few waves: 9.8 us against 4.3 for a wave per head, so below 1024
// tokens a group is one head. NARROW: head_dim <= 64.
#define RR_WAVES 1
template <bool NARROW, int RR_GROUP>
__global__ __launch_bounds__(64 * RR_WAVES) void gemm_reduce_rope_kernel(
    const float *__restrict__ ws, const uint16_t *__restrict__ bias, float *__restrict__ qkv,
    int splits, int n, uint16_t *__restrict__ k_cache, uint16_t *__restrict__ v_cache,
    const float *__restrict__ cos_tab, const float *__restrict__ sin_tab, int n_q, int n_kv,
    int hd, int pos0, int max_seq, const uint16_t *__restrict__ q_norm_w,
    const uint16_t *__restrict__ k_norm_w, float eps) {
  const int nh = n_q + n_kv, ngrp = (nh + RR_GROUP - 1) / RR_GROUP;
  const int item = blockIdx.x * RR_WAVES + (int)(threadIdx.x >> 6);
  if (item >= n * ngrp) return;  // a whole wave: no barriers below
  const int tok = item / ngrp, grp = item % ngrp;
  const int half = hd >> 1, j = threadIdx.x & 63;
  const int nqkv = (n_q + 2 * n_kv) * hd;
  const size_t total = (size_t)n * nqkv;
  // Lane roles. NARROW (half <= 32): one column per lane (lanes 0..31 the
  // first half, 32..63 the second), the rotation partner over a cross-lane
  // swap; else lane j < half holds columns j and j + half. The norm's sum
  // and every product are the same in both forms.
  const bool hi = NARROW && j >= 32;
  const int jj = NARROW ? (j & 31) : j;
  const bool act = jj < half;
  const int off = jj + (hi ? half : 0);
  constexpr int NV = NARROW ? 2 : 4;  // a kv head's columns per lane (k, then v)
  // column e of head h relative to the row: q heads use e = 0 (and 1 in the
  // wide form), kv heads k then v
  auto col = [&](int h, int e) {
    if (h < n_q) return h * hd + (NARROW ? off : jj + e * half);
    const int kvh = h - n_q;
    const int k0 = (n_q + kvh) * hd, v0 = (n_q + n_kv + kvh) * hd;
    if (NARROW) return (e == 0 ? k0 : v0) + off;
    return (e < 2 ? k0 : v0) + jj + (e & 1) * half;
  };
  auto ncols = [&](int h) { return (h < n_q ? 1 : 2) * (NARROW ? 1 : 2); };
  const float *wrow = ws + (size_t)tok * nqkv;
  float *row = qkv + (size_t)tok * nqkv;
  const int pos = min(max(pos0 + tok, 0), max_seq - 1);
  const float c = act ? cos_tab[(size_t)pos * half + jj] : 0.0f;
  const float s = act ? sin_tab[(size_t)pos * half + jj] : 0.0f;
  {
    const int h0 = grp * RR_GROUP;
    float v[RR_GROUP][NV];
#pragma unroll
    for (int u = 0; u < RR_GROUP; ++u) {
      const int h = h0 + u;
#pragma unroll
      for (int e = 0; e < NV; ++e) {
        float t = 0.0f;
        if (h < nh && act && e < ncols(h)) {
          const int cc = col(h, e);
          t = split_sum(wrow, cc, total, splits);
          if (bias) t += h2f(bias[cc]);
        }
        v[u][e] = t;
      }
    }
#pragma unroll
    for (int u = 0; u < RR_GROUP; ++u) {
      const int h = h0 + u;
      if (h >= nh) break;  // uniform
      const int nc = ncols(h);
      if (act && h >= n_q) {  // k and v: the reduced values, as gemm_split_reduce_kernel
                              // stores them (q's are overwritten below by their rotation)
#pragma unroll
        for (int e = 0; e < NV; ++e)
          if (e < nc) row[col(h, e)] = v[u][e];
      }
      const bool is_q = h < n_q;
      const uint16_t *__restrict__ g = is_q ? q_norm_w : k_norm_w;
      if constexpr (NARROW) {
        const float mine = v[u][0];
        const float other = __shfl_xor(mine, 32);
        float x1 = hi ? other : mine, x2 = hi ? mine : other;
        if (g) {
          const float ss = wave_sum(act && !hi ? fmaf(x1, x1, x2 * x2) : 0.0f);
          const float sc = 1.0f / sqrtf(ss / (float)hd + eps);
          if (act) {
            x1 = x1 * sc * h2f(g[jj]);
            x2 = x2 * sc * h2f(g[jj + half]);
          }
        }
        const float lo = rope_lo(x1, x2, c, s), hv = rope_hi(x1, x2, c, s);
        if (act) {
          if (is_q) {
            row[col(h, 0)] = hi ? hv : lo;
          } else {
            const size_t slot = ((size_t)(h - n_q) * max_seq + pos) * hd;
            k_cache[slot + off] = f2h(hi ? hv : lo);
            v_cache[slot + off] = f2h(v[u][1]);
          }
        }
      } else {
        float x1 = v[u][0], x2 = v[u][1];
        if (g) qk_norm_wave(x1, x2, g, jj, half, hd, eps, act);
        if (act) {
          if (is_q) {
            row[h * hd + jj] = rope_lo(x1, x2, c, s);
            row[h * hd + jj + half] = rope_hi(x1, x2, c, s);
          } else {
            const size_t slot = ((size_t)(h - n_q) * max_seq + pos) * hd;
            k_cache[slot + jj] = f2h(rope_lo(x1, x2, c, s));
            k_cache[slot + jj + half] = f2h(rope_hi(x1, x2, c, s));
            v_cache[slot + jj] = f2h(v[u][2]);
            v_cache[slot + jj + half] = f2h(v[u][3]);
          }
        }
      }
    }
  }
}

namespace {
// The tile family: the 128 x 128 wide tiles (32x32x16 MFMA) unless
// WST_GEMM_TILES=narrow selects the 64 x 64 tiles (16x16x32 MFMA) and
// WST_GEMM_TILES=wide the wide tiles wherever they apply (for measurement);
// unset, the shape picks. One choice for every chunk GEMM form, so fused and
// unfused forms sum alike.
int gemm_tiles_mode() {  // 0 narrow, 1 by shape, 2 wide
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("WST_GEMM_TILES");
    v = (e && e[0] == 'n') ? 0 : (e && e[0] == 'w') ? 2 : 1;
  }
  return v;
}

template <bool HIER, bool SWI>
void set_lds_attr() {
  static bool done = false;
  if (!done) {
    (void)hipFuncSetAttribute((const void *)gemm_mfma_kernel<HIER, SWI>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, GM_LDS);
    if constexpr (HIER) {
      (void)hipFuncSetAttribute((const void *)gemm_wide_kernel<HIER, SWI, 8>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, GwShape<8>::LDS);
      (void)hipFuncSetAttribute((const void *)gemm_wide_kernel<HIER, SWI, 4>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, GwShape<4>::LDS);
    }
    done = true;
  }
}

struct GemmPlan {
  bool wide;
  int nwv;  // wide tiles: waves of 32 tokens (8: 256-token tiles, 4: 128)
  int bm, bn, kg;
  int splits, gps;
  dim3 grid;
};

// WST_GEMM_SPLITS=k caps the split-K count at k (1: no split); a measurement
// knob.
static int gemm_split_cap() {
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("WST_GEMM_SPLITS");
    v = e ? atoi(e) : 0;
  }
  return v;
}

static int gemm_bn_override() {
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("WST_GEMM_BN");
    v = e ? atoi(e) : 0;
  }
  return v;
}

// Splits so that the grid covers the chip, each at least one step long.
// rows: the weight matrix's row count (2 * inter for the SwiGLU form), which
// with in_f and the plan's token count picks the tiles: the wide tiles for
// long rows or many of them, where their deeper pipeline pays, and for any
// shape whose 256-token tiles fill half the CUs without a split (the 0.5B
// qkv and o projections over a 4096-token batched prefill: 30.3 -> 28.6 and
// 25.0 -> 17.0 us, config 4 464-466k -> 475-480k tok/s); otherwise (the
// same projections on one 256-token chunk: wide 9.0 + 3.9 us against narrow
// 7.4 + 3.9 us for qkv) the narrow tiles, since short K split into pieces is
// too short for the wide tiles' pipeline.
// plan_n: the token count whose tiling and split-K plan the launch uses; n
// may exceed it (several chunks in one launch): the grid then repeats the
// plan's token tiles over n, and every token gets the bits a launch of
// plan_n tokens gives it (the tiles are 64, 128 or 256 tokens, which divide
// a chunk). 0: n itself.
GemmPlan plan_gemm(int in_f, int out_f, int n, bool hier = true, int rows = 0, bool swi = false,
                   int plan_n = 0) {
  GemmPlan p;
  if (rows <= 0) rows = out_f;
  const int pn = plan_n > 0 && plan_n < n ? plan_n : n;
  // (The wide tiles address x with 32-bit byte offsets.)
  const int tm = gemm_tiles_mode();
  const int rows_t256 = ((rows + GW_BM - 1) / GW_BM) * ((pn + 255) / 256);
  p.wide = hier && tm > 0 && in_f >= GW_KC &&
           (tm == 2 || in_f >= 2048 || rows >= 4096 || rows_t256 >= wst_cu_count() / 2) &&
           (size_t)n * in_f * 2 < ((size_t)1 << 31);
  // Wide tiles of 128 tokens for the split-K shapes (256-token tiles fewer
  // than half the CUs), where 256-token tiles would leave CUs without a
  // tile: 7B qkv 43.0 -> 36.2 us, 7B down 100.3 -> 95.6 us (0.5B down
  // unchanged). Not where the 256-token tiles already fill about one round
  // of the CUs without splitting (the 0.5B down over a 4096-token batched
  // prefill, 224 tiles: 76.2 -> 65.2 us), nor for the SwiGLU form, which
  // never splits: its 128-token tiles run one wave per SIMD (0.5B gate|up
  // 14.0 -> 16.7 us). WST_GEMM_BN=128|256 forces one.
  p.nwv = 8;
  if (p.wide) {
    const int forced = gemm_bn_override();
    const int t256 = ((out_f + GW_BM - 1) / GW_BM) * ((pn + 255) / 256);
    if (forced == 128 || (forced != 256 && !swi && pn > 128 && t256 < wst_cu_count() / 2))
      p.nwv = 4;
  }
  p.bm = p.wide ? GW_BM : GM_BM;
  p.bn = p.wide ? 32 * p.nwv : GM_BN;
  p.kg = p.wide ? GW_KG : GM_KG;
  const int G = in_f / HGROUP;
  const int tiles = ((out_f + p.bm - 1) / p.bm) * ((pn + p.bn - 1) / p.bn);
  p.splits = 1;
  p.gps = G;
  const int target = wst_cu_count();
  if (tiles < target / 2) {
    int want = (target + tiles - 1) / tiles;
    if (gemm_split_cap() > 0) want = min(want, gemm_split_cap());
    int g = (G + want - 1) / want;
    g = (g + p.kg - 1) / p.kg * p.kg;
    if ((G + g - 1) / g > GM_MAXSPLIT) g = (G + GM_MAXSPLIT - 1) / GM_MAXSPLIT;
    g = (g + p.kg - 1) / p.kg * p.kg;
    p.gps = g;
    p.splits = (G + g - 1) / g;
  }
  p.grid = dim3((out_f + p.bm - 1) / p.bm, (n + p.bn - 1) / p.bn, p.splits);
  return p;
}

template <bool HIER, bool SWI>
void launch_gemm(const GemmPlan &p, const void *w, const void *si, const void *sb, const void *x,
                 const void *bias, void *y, float *ws, int in_f, int out_f, int n, int accum) {
  set_lds_attr<HIER, SWI>();
  if constexpr (HIER) {
    if (p.wide) {
      if (p.nwv == 4)
        gemm_wide_kernel<HIER, SWI, 4><<<p.grid, GwShape<4>::THREADS, GwShape<4>::LDS, WST_STREAM>>>(
            w, (const uint8_t *)si, (const uint32_t *)sb, (const uint16_t *)x,
            (const uint16_t *)bias, (float *)y, ws, in_f, out_f, n, accum, p.gps, GwRope{});
      else
        gemm_wide_kernel<HIER, SWI, 8><<<p.grid, GwShape<8>::THREADS, GwShape<8>::LDS, WST_STREAM>>>(
            w, (const uint8_t *)si, (const uint32_t *)sb, (const uint16_t *)x,
            (const uint16_t *)bias, (float *)y, ws, in_f, out_f, n, accum, p.gps, GwRope{});
      return;
    }
  }
  gemm_mfma_kernel<HIER, SWI><<<p.grid, GM_THREADS, GM_LDS, WST_STREAM>>>(
        w, (const uint8_t *)si, (const uint32_t *)sb, (const uint16_t *)x,
        (const uint16_t *)bias, (float *)y, ws, in_f, out_f, n, accum, p.gps);
}

// The GEMM into the split scratch (always, even with one split): the fused
// reduce kernels read it.
wst_status_t gemm_to_scratch(const void *w, const void *si, const void *sb, const void *x,
                             int in_f, int out_f, int n, float **ws_out, int *splits_out,
                             int plan_n = 0) {
  const GemmPlan p = plan_gemm(in_f, out_f, n, true, 0, false, plan_n);
  float *ws = (float *)wst_static_scratch(WST_SCRATCH_GEMM, (size_t)p.splits * n * out_f * 4);
  if (!ws) return WST_ERR_OOM;
  launch_gemm<true, false>(p, w, si, sb, x, nullptr, nullptr, ws, in_f, out_f, n, 0);
  *ws_out = ws;
  *splits_out = p.splits;
  return WST_OK;
}
}  // namespace

// ws_ext: when non-null, the split partials go there (ws_cap bytes) instead
// of the library's lazily grown scratch slot, and nothing is allocated.
wst_status_t wst_gemm_mfma(bool hier, const void *w, const void *si, const void *sb,
                           const void *x, const void *bias, void *y, int32_t in_f, int32_t out_f,
                           int32_t n, int32_t accum, float *ws_ext, size_t ws_cap,
                           int32_t plan_n) {
  const GemmPlan p = plan_gemm(in_f, out_f, n, hier, 0, false, plan_n);
  const int splits = p.splits;
  float *ws = nullptr;
  if (splits > 1) {
    const size_t need = (size_t)splits * n * out_f * 4;
    if (ws_ext) {
      if (need > ws_cap) {
        snprintf(wst_err_buf, sizeof(wst_err_buf),
                 "split-K partials need %zu bytes, above the %zu-byte static scratch", need, ws_cap);
        return WST_ERR_SHAPE;
      }
      ws = ws_ext;
    } else {
      ws = (float *)wst_static_scratch(WST_SCRATCH_GEMM, need);
      if (!ws) return WST_ERR_OOM;
    }
  }
  if (hier)
    launch_gemm<true, false>(p, w, si, sb, x, bias, y, ws, in_f, out_f, n, accum);
  else
    launch_gemm<false, false>(p, w, nullptr, nullptr, x, bias, y, ws, in_f, out_f, n, accum);
  if (splits > 1) {
    const size_t total = (size_t)n * out_f;
    const int blocks = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
    gemm_split_reduce_kernel<<<blocks, 256, 0, WST_STREAM>>>(ws, (const uint16_t *)bias,
                                                              (float *)y, out_f, n, splits, accum);
  }
  return WST_OK;
}

static wst_status_t chunk_gemm_args(const void *qw, const void *si, const void *sb, const void *x,
                                    int32_t in_f, int32_t out_f, int32_t n, const char *who) {
  if (!(qw && si && sb && x)) {
    snprintf(wst_err_buf, sizeof(wst_err_buf), "%s: null pointer", who);
    return WST_ERR_INVALID_ARG;
  }
  if (in_f <= 0 || out_f <= 0 || n <= 0 || in_f % HGROUP != 0) {
    snprintf(wst_err_buf, sizeof(wst_err_buf), "%s: bad shape", who);
    return WST_ERR_INVALID_ARG;
  }
  if (((uintptr_t)qw | (uintptr_t)x) & 15u) {
    snprintf(wst_err_buf, sizeof(wst_err_buf), "%s: qw and x must be 16-byte aligned", who);
    return WST_ERR_INVALID_ARG;
  }
  return WST_OK;
}

extern "C" wst_status_t wst_gemm_hier_swiglu_chunks(const void *qw, const void *si,
                                                    const void *sb, const void *x, void *act,
                                                    int32_t in_f, int32_t inter, int32_t n,
                                                    int32_t plan_n) {
  wst_status_t st = chunk_gemm_args(qw, si, sb, x, in_f, inter, n, "wst_gemm_hier_swiglu_chunk");
  if (st != WST_OK) return st;
  WST_REQUIRE(act, "wst_gemm_hier_swiglu_chunk: null pointer");
  // Never split: a tile pairs BM/2 gate rows with the matching up rows.
  GemmPlan p = plan_gemm(in_f, inter, n, true, 2 * inter, true, plan_n);
  p.splits = 1;
  p.gps = in_f / HGROUP;
  p.grid = dim3((inter + p.bm / 2 - 1) / (p.bm / 2), (n + p.bn - 1) / p.bn, 1);
  launch_gemm<true, true>(p, qw, si, sb, x, nullptr, act, nullptr, in_f, inter, n, 0);
  WST_TRY_KERNEL("wst_gemm_hier_swiglu_chunk");
  return WST_OK;
}

extern "C" wst_status_t wst_gemm_hier_swiglu_chunk(const void *qw, const void *si,
                                                   const void *sb, const void *x, void *act,
                                                   int32_t in_f, int32_t inter, int32_t n) {
  return wst_gemm_hier_swiglu_chunks(qw, si, sb, x, act, in_f, inter, n, n);
}

extern "C" wst_status_t wst_gemm_hier_norm_chunks(const void *qw, const void *si, const void *sb,
                                                 const void *x, const void *bias, void *y,
                                                 int32_t in_f, int32_t out_f, int32_t n,
                                                 int32_t accum, const void *norm_w, float eps,
                                                 void *h_out, int32_t plan_n) {
  wst_status_t st = chunk_gemm_args(qw, si, sb, x, in_f, out_f, n, "wst_gemm_hier_norm_chunk");
  if (st != WST_OK) return st;
  WST_REQUIRE(y && norm_w && h_out, "wst_gemm_hier_norm_chunk: null pointer");
  WST_REQUIRE(out_f <= 16384, "wst_gemm_hier_norm_chunk: out_features above 16384");
  float *ws;
  int splits;
  st = gemm_to_scratch(qw, si, sb, x, in_f, out_f, n, &ws, &splits, plan_n);
  if (st != WST_OK) return st;
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void *)gemm_reduce_norm_kernel<0>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 16384 * 4);
    attr = true;
  }
  if (out_f % 8 == 0 && out_f <= 4096 && !(((uintptr_t)y | (uintptr_t)h_out | (uintptr_t)norm_w |
                                              (uintptr_t)bias) & 15u)) {
    const int threads = 64 * ((out_f / 8 + 63) / 64);
    gemm_reduce_norm8_kernel<<<n, threads, 0, WST_STREAM>>>(
        ws, (const uint16_t *)bias, (float *)y, out_f, n, splits, accum, (const uint16_t *)norm_w,
        eps, (uint16_t *)h_out);
    WST_TRY_KERNEL("wst_gemm_hier_norm_chunk");
    return WST_OK;
  }
  auto kern = out_f <= 1024   ? gemm_reduce_norm_kernel<2>
              : out_f <= 2048 ? gemm_reduce_norm_kernel<4>
              : out_f <= 4096 ? gemm_reduce_norm_kernel<8>
                              : gemm_reduce_norm_kernel<0>;
  kern<<<n, 512, (size_t)out_f * 4, WST_STREAM>>>(ws, (const uint16_t *)bias, (float *)y, out_f, n,
                                                  splits, accum, (const uint16_t *)norm_w, eps,
                                                  (uint16_t *)h_out);
  WST_TRY_KERNEL("wst_gemm_hier_norm_chunk");
  return WST_OK;
}

extern "C" wst_status_t wst_gemm_hier_norm_chunk(const void *qw, const void *si, const void *sb,
                                                const void *x, const void *bias, void *y,
                                                int32_t in_f, int32_t out_f, int32_t n,
                                                int32_t accum, const void *norm_w, float eps,
                                                void *h_out) {
  return wst_gemm_hier_norm_chunks(qw, si, sb, x, bias, y, in_f, out_f, n, accum, norm_w, eps,
                                   h_out, n);
}

// WST_GEMM_ROPE_EPI=0 keeps the separate reduce + RoPE kernel on the shapes
// the GEMM's own RoPE epilogue covers (for measurement and the parity test).
static bool rope_epilogue_on() {
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("WST_GEMM_ROPE_EPI");
    v = (e && e[0] == '0') ? 0 : 1;
  }
  return v == 1;
}

extern "C" wst_status_t wst_gemm_hier_rope_chunks(const void *qw, const void *si, const void *sb,
                                                 const void *x, const void *bias, void *qkv,
                                                 int32_t in_f, void *k_cache, void *v_cache,
                                                 const void *cos_tab, const void *sin_tab,
                                                 int32_t n_q, int32_t n_kv, int32_t head_dim,
                                                 int32_t pos0, int32_t n, int32_t max_seq,
                                                 const void *q_norm_w, const void *k_norm_w,
                                                 float eps, int32_t plan_n) {
  WST_REQUIRE(n_q > 0 && n_kv > 0 && head_dim > 0 && n > 0 && n <= 65535,
              "wst_gemm_hier_rope_chunk: bad shape");
  WST_REQUIRE(head_dim % 2 == 0 && head_dim <= 128, "wst_gemm_hier_rope_chunk: head_dim above 128");
  const int out_f = (n_q + 2 * n_kv) * head_dim;
  wst_status_t st = chunk_gemm_args(qw, si, sb, x, in_f, out_f, n, "wst_gemm_hier_rope_chunk");
  if (st != WST_OK) return st;
  WST_REQUIRE(qkv && k_cache && v_cache && cos_tab && sin_tab,
              "wst_gemm_hier_rope_chunk: null pointer");
  WST_REQUIRE(max_seq > 0 && pos0 >= 0 && pos0 + n <= max_seq,
              "wst_gemm_hier_rope_chunk: chunk does not fit the cache");
  // head_dim 64 on unsplit 256-token wide tiles (a batched prefill of the
  // 0.5B shape): each tile is one head, and its epilogue applies the norm,
  // the rotation and the cache append itself, in the reduce kernel's
  // arithmetic; no partials, no second launch.
  {
    const GemmPlan p = plan_gemm(in_f, out_f, n, true, 0, false, plan_n);
    if (p.wide && p.nwv == 8 && p.splits == 1 && head_dim == GW_ROPE_HD && rope_epilogue_on()) {
      static bool attr = false;
      if (!attr) {
        (void)hipFuncSetAttribute((const void *)gemm_wide_kernel<true, false, 8, true>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, GwShape<8>::LDS);
        attr = true;
      }
      const GwRope re{(uint16_t *)k_cache, (uint16_t *)v_cache, (const float *)cos_tab,
                      (const float *)sin_tab, (const uint16_t *)q_norm_w,
                      (const uint16_t *)k_norm_w, n_q, n_kv, pos0, max_seq, eps};
      gemm_wide_kernel<true, false, 8, true><<<p.grid, GwShape<8>::THREADS, GwShape<8>::LDS,
                                               WST_STREAM>>>(
          qw, (const uint8_t *)si, (const uint32_t *)sb, (const uint16_t *)x,
          (const uint16_t *)bias, (float *)qkv, nullptr, in_f, out_f, n, 0, p.gps, re);
      WST_TRY_KERNEL("wst_gemm_hier_rope_chunk");
      return WST_OK;
    }
  }
  float *ws;
  int splits;
  st = gemm_to_scratch(qw, si, sb, x, in_f, out_f, n, &ws, &splits, plan_n);
  if (st != WST_OK) return st;
#define RR_LAUNCH(NARROW_, G_)                                                                 \
  do {                                                                                       \
    const int items_ = n * ((n_q + n_kv + (G_) - 1) / (G_));                                 \
    gemm_reduce_rope_kernel<NARROW_, G_><<<(items_ + RR_WAVES - 1) / RR_WAVES, 64 * RR_WAVES, 0, \
                                           WST_STREAM>>>(                                    \
        ws, (const uint16_t *)bias, (float *)qkv, splits, n, (uint16_t *)k_cache,            \
        (uint16_t *)v_cache, (const float *)cos_tab, (const float *)sin_tab, n_q, n_kv,       \
        head_dim, pos0, max_seq, (const uint16_t *)q_norm_w, (const uint16_t *)k_norm_w, eps); \
  } while (0)
  const bool big = n >= 1024;
  if (head_dim <= 64) {
    if (big) RR_LAUNCH(true, 8);
    else RR_LAUNCH(true, 1);
  } else {
    if (big) RR_LAUNCH(false, 8);
    else RR_LAUNCH(false, 1);
  }
#undef RR_LAUNCH
  WST_TRY_KERNEL("wst_gemm_hier_rope_chunk");
  return WST_OK;
}

extern "C" wst_status_t wst_gemm_hier_rope_chunk(const void *qw, const void *si, const void *sb,
                                                const void *x, const void *bias, void *qkv,
                                                int32_t in_f, void *k_cache, void *v_cache,
                                                const void *cos_tab, const void *sin_tab,
                                                int32_t n_q, int32_t n_kv, int32_t head_dim,
                                                int32_t pos0, int32_t n, int32_t max_seq,
                                                const void *q_norm_w, const void *k_norm_w,
                                                float eps) {
  return wst_gemm_hier_rope_chunks(qw, si, sb, x, bias, qkv, in_f, k_cache, v_cache, cos_tab,
                                   sin_tab, n_q, n_kv, head_dim, pos0, n, max_seq, q_norm_w,
                                   k_norm_w, eps, n);
}

// ------------------------------------------- the no-allocation GEMM entry
//
// wst_gemm_int4_hier_noalloc: wst_gemm_int4_hier for callers that cannot
// allocate (graph capture, serving loops). Its split-K partials live in this
// file-scope device array instead of the lazily allocated scratch slot. The
// split plan splits only grids of fewer tiles than half the CUs, at most
// ceil(CUs / tiles) ways, so the partials stay below (CUs + tiles) x (one
// tile, at most 64 x 256 f32 = 64 KiB): under 24 MiB on 256 CUs, which this
// array holds; a larger need is refused.
#define GM_NOALLOC_BYTES (24u << 20)
static __device__ __align__(256) unsigned char scratch[GM_NOALLOC_BYTES];

// The array's device address, looked up once per device with that device
// current (each GPU holds its own copy). In host code `scratch` itself is only
// a stand-in for the symbol and must never be passed to a kernel.
static void *g_noalloc_scratch[64];
static std::mutex g_noalloc_mu;

static float *noalloc_scratch() {
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) {
    snprintf(wst_err_buf, sizeof(wst_err_buf), "wst_gemm_int4_hier_noalloc: no current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc_scratch[d]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      wst_set_error("wst_gemm_int4_hier_noalloc: hipGetSymbolAddress", e);
      return nullptr;
    }
    g_noalloc_scratch[d] = p;
  }
  return (float *)g_noalloc_scratch[d];
}

extern "C" wst_status_t wst_gemm_int4_hier_noalloc(const void *qw, const void *si, const void *sb,
                                                   const void *x, const void *bias, void *y,
                                                   int32_t in_f, int32_t out_f, int32_t n,
                                                   int32_t accum) {
  WST_REQUIRE(qw && si && sb && x && y, "wst_gemm_int4_hier_noalloc: null pointer");
  WST_REQUIRE(in_f > 0 && out_f > 0 && n > 0, "wst_gemm_int4_hier_noalloc: non-positive dimension");
  WST_REQUIRE(in_f % 32 == 0, "wst_gemm_int4_hier_noalloc: in_features must be a multiple of 32");
  WST_REQUIRE(!(((uintptr_t)qw | (uintptr_t)x) & 15u),
              "wst_gemm_int4_hier_noalloc: qw and x must be 16-byte aligned");
  float *ws = noalloc_scratch();
  if (!ws) return WST_ERR_CUDA;
  const wst_status_t st =
      wst_gemm_mfma(true, qw, si, sb, x, bias, y, in_f, out_f, n, accum, ws, GM_NOALLOC_BYTES, 0);
  if (st != WST_OK) return st;
  WST_TRY_KERNEL("wst_gemm_int4_hier_noalloc");
  return WST_OK;
}
