// int4-hier-g32 decode GEMV for gfx950, plus its fused forms (RMSNorm
// prologue, SwiGLU epilogue) used by the engine's step.
//
// Format (docs/FORMAT.md:128-166, hier.rs:62-99): per row an f16 pair (d, dmin),
// per group of 32 weights one byte (ls | lm<<4), per weight a nibble q, and
//     w = q * (d*ls) - dmin*lm.
// The GEMV computes y[r] = (accum ? y[r] : 0) + (sum_c w[r][c] x[c] + bias[r])
// (reference kernel: gemv_hier.cu:70-163).
//
// How it maps onto CDNA4
// ----------------------
// * One lane owns whole groups: a group is 16 bytes of nibbles, exactly one
//   dwordx4 load, and a row-slot of LPR consecutive lanes reads a contiguous
//   run of the row. A wave therefore issues 1 KB-wide coalesced loads, and
//   each lane keeps TILE*NG of them in flight before it does any arithmetic.
// * x is staged once per block in LDS (normalised there when the RMSNorm is
//   fused), then each lane's slice (64 B per group) moves into registers for
//   the rest of the kernel: no LDS traffic in the inner loop. The grid is
//   persistent (a few blocks per CU) so the staging is paid a few times per CU,
//   not once per row. x is permuted so that the nibble pairs produced by one
//   bit-field insert line up with the x pairs they multiply.
// * Unpack without conversions: inserting a nibble into the mantissa of f16
//   1024.0 gives 1024+q exactly; nibbles in bits 4..7 give 1024+16q. One
//   v_bfi_b32 per pair of weights, one shift per word, and v_dot2c_f32_f16
//   multiplies two of them by two activations with an f32 accumulator. The
//   1024 offsets are removed once per group with per-group sums of x computed
//   at start-up:
//       sum_i q_i x_i = DA + DB/16 - (1024*sum_even x + 64*sum_odd x)
//   where DA (DB) accumulates the even (odd) columns. About 1.1 VALU
//   instructions per weight, and every product is accumulated in f32 -- more
//   precise than the reference's f16 half2 accumulation inside a group.
// * Per row: y = d * sum_g ls_g*Q_g - dmin * sum_g lm_g*S_g, reduced across the
//   row-slot with DPP row operations and, for rows split over several waves,
//   through LDS in a fixed order. Results are deterministic and do not depend
//   on TILE, the grid, or which fused form ran: a row's value is a function of
//   (in_f, the row's bytes, x) only. That is what lets the fused kernels be
//   checked bit for bit against the unfused ABI sequence.
#include "common.hpp"

#include <stdlib.h>

#define HGROUP 32
#define HIER_MAGIC 0x64006400u  // f16 1024.0 in both halves

// Bit-field insert (a & m) | (b & ~m) as one v_bfi_b32: the mask lives in a
// VGPR and the magic constant in an SGPR kernel argument. (Left to itself the
// compiler emits v_and + v_or with a literal, one more VALU op per pair.)
__device__ __forceinline__ uint32_t bfi(uint32_t a, uint32_t m, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(a), "s"(b));
  return r;
}

// A lane's resident slice of x for one group: the permuted activation pairs
// and the two correction terms.
struct XGroup {
  uint32_t ea[4], ob[4], ea2[4], ob2[4];  // (x0,x4) (x1,x5) (x2,x6) (x3,x7) per word
  float corr;                             // 1024*sum_even + 64*sum_odd
  float sum;                              // sum of the 32 activations
};

// r[k] holds f16 activations (2k, 2k+1) of the group.
__device__ __forceinline__ void build_xgroup(const uint32_t r[16], XGroup &xg) {
  const wst_h2 one = {(_Float16)1.0f, (_Float16)1.0f};
  float se = 0.0f, so = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t a = r[4 * k], b = r[4 * k + 1], c = r[4 * k + 2], d = r[4 * k + 3];
    xg.ea[k] = (a & 0xFFFFu) | (c << 16);
    xg.ob[k] = (a >> 16) | (c & 0xFFFF0000u);
    xg.ea2[k] = (b & 0xFFFFu) | (d << 16);
    xg.ob2[k] = (b >> 16) | (d & 0xFFFF0000u);
    se = __builtin_amdgcn_fdot2(as_h2(xg.ea[k]), one, se, false);
    se = __builtin_amdgcn_fdot2(as_h2(xg.ea2[k]), one, se, false);
    so = __builtin_amdgcn_fdot2(as_h2(xg.ob[k]), one, so, false);
    so = __builtin_amdgcn_fdot2(as_h2(xg.ob2[k]), one, so, false);
  }
  xg.corr = 1024.0f * se + 64.0f * so;
  xg.sum = se + so;
}

__device__ __forceinline__ void load_xgroup(const uint16_t *__restrict__ x, int g, XGroup &xg) {
  const uint4 *xv = (const uint4 *)(x + (size_t)g * HGROUP);
  uint32_t r[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 v = xv[i];
    r[4 * i + 0] = v.x;
    r[4 * i + 1] = v.y;
    r[4 * i + 2] = v.z;
    r[4 * i + 3] = v.w;
  }
  build_xgroup(r, xg);
}

// sum_i q_i x_i for one packed group (32 nibbles in `p`) against `xg`.
__device__ __forceinline__ float group_dot(const uint4 p, const XGroup &xg, uint32_t magic) {
  const uint32_t w[4] = {p.x, p.y, p.z, p.w};
  float da = 0.0f, db = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t u = w[k], t = w[k] >> 8;
    da = __builtin_amdgcn_fdot2(as_h2(bfi(u, 0x000F000Fu, magic)), as_h2(xg.ea[k]), da, false);
    db = __builtin_amdgcn_fdot2(as_h2(bfi(u, 0x00F000F0u, magic)), as_h2(xg.ob[k]), db, false);
    da = __builtin_amdgcn_fdot2(as_h2(bfi(t, 0x000F000Fu, magic)), as_h2(xg.ea2[k]), da, false);
    db = __builtin_amdgcn_fdot2(as_h2(bfi(t, 0x00F000F0u, magic)), as_h2(xg.ob2[k]), db, false);
  }
  return fmaf(db, 0.0625f, da) - xg.corr;
}

template <int LPR>
__device__ __forceinline__ float slot_sum(float v) {
  if constexpr (LPR == 32) return half_wave_sum(v);
  else return wave_sum(v);
}

// ---------------------------------------------------------------- the kernel
//
// LPR lanes cooperate on a row (32, 64, 128 or 256); each owns NG groups of
// the row (group g = lane_in_row + j*LPR). A unit of work is TILE rows per
// row-slot. Blocks are 256 threads. For LPR <= 64 waves are independent; for
// LPR > 64 the W = LPR/64 waves of a row combine through LDS.
//
// NORM:   x is the f32 residual stream; every block computes its RMS scale and
//         normalises with norm_w on the fly (wst_rmsnorm + GEMV). Block 0
//         also stores h when h_out is non-null.
// SWIGLU: out_f is the intermediate width; unit row r computes gate row r and
//         up row r + out_f of the fused matrix and writes f16(silu(g) * u)
//         (GEMV + wst_swiglu).
template <int LPR, int NG, int TILE, bool NORM, bool SWIGLU>
__global__ __launch_bounds__(256) void gemv_hier_kernel(
    const uint4 *__restrict__ qw, const uint8_t *__restrict__ si,
    const uint32_t *__restrict__ sb, const void *__restrict__ xin,
    const uint16_t *__restrict__ norm_w, float eps, uint16_t *__restrict__ h_out,
    const uint16_t *__restrict__ bias, void *__restrict__ yout, int in_f, int out_f, int accum,
    uint32_t magic) {
  constexpr int SLOTS = 256 / LPR;  // row-slots per block
  constexpr int W = LPR > 64 ? LPR / 64 : 1;
  constexpr int NR = SWIGLU ? 2 : 1;  // matrix rows per unit row
  const int tid = threadIdx.x;
  const int slot = tid / LPR, lr = tid % LPR;
  const int G = in_f / HGROUP;

  __shared__ float red[16];
  __shared__ float wred[4][TILE * NR];
  // The activation vector, staged once per block (f16, in_f entries): every
  // row-slot builds its register slices from here instead of each re-reading
  // x from L2.
  extern __shared__ uint4 xs_raw[];
  uint16_t *xs = (uint16_t *)xs_raw;

  if constexpr (NORM) {
    const float *x = (const float *)xin;
    const float s = rms_scale256(x, in_f, eps, red);
    for (int i = tid; i < in_f; i += 256) xs[i] = f2h(x[i] * s * h2f(norm_w[i]));
  } else {
    const uint4 *x = (const uint4 *)xin;
    for (int i = tid; i < in_f / 8; i += 256) xs_raw[i] = x[i];
  }
  __syncthreads();
  if (NORM && h_out && blockIdx.x == 0)
    for (int i = tid; i < in_f / 8; i += 256) ((uint4 *)h_out)[i] = xs_raw[i];

  XGroup xg[NG];
  bool gv[NG];
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    const int g = lr + j * LPR;
    gv[j] = g < G;
    if (gv[j]) load_xgroup(xs, g, xg[j]);
  }

  const int rows_per_block = SLOTS * TILE;
  const int nunits = (out_f + rows_per_block - 1) / rows_per_block;
  for (int unit = blockIdx.x; unit < nunits; unit += gridDim.x) {
    const int row0 = unit * rows_per_block + slot * TILE;

    uint4 wq[TILE][NR][NG];
    uint32_t idx[TILE][NR][NG];
    uint32_t sbv[TILE][NR];
#pragma unroll
    for (int t = 0; t < TILE; ++t) {
      const bool rv = row0 + t < out_f;
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        const int r = row0 + t + k * out_f;
        sbv[t][k] = rv ? sb[r] : 0u;
#pragma unroll
        for (int j = 0; j < NG; ++j) {
          const size_t at = (size_t)r * G + lr + j * LPR;
          if (rv && gv[j]) {
            wq[t][k][j] = ld_stream16(qw + at);
            idx[t][k][j] = si[at];
          } else {
            wq[t][k][j] = make_uint4(0, 0, 0, 0);
            idx[t][k][j] = 0;
          }
        }
      }
    }

    float part[TILE][NR];
#pragma unroll
    for (int t = 0; t < TILE; ++t) {
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        float as = 0.0f, am = 0.0f;
#pragma unroll
        for (int j = 0; j < NG; ++j) {
          if (!gv[j]) continue;
          const float q = group_dot(wq[t][k][j], xg[j], magic);
          as = fmaf((float)(idx[t][k][j] & 0xFu), q, as);
          am = fmaf((float)(idx[t][k][j] >> 4), xg[j].sum, am);
        }
        const float d = h2f((uint16_t)(sbv[t][k] & 0xFFFFu));
        const float dm = h2f((uint16_t)(sbv[t][k] >> 16));
        part[t][k] = slot_sum<LPR>(d * as - dm * am);
      }
    }

    if constexpr (W > 1) {
      const int wave = tid >> 6;
      if ((tid & 63) == 0) {
#pragma unroll
        for (int t = 0; t < TILE; ++t)
#pragma unroll
          for (int k = 0; k < NR; ++k) wred[wave][t * NR + k] = part[t][k];
      }
      __syncthreads();
      if ((tid & 63) == 0 && (wave % W) == 0) {
#pragma unroll
        for (int t = 0; t < TILE; ++t)
#pragma unroll
          for (int k = 0; k < NR; ++k) {
            float v = 0.0f;
            for (int q = 0; q < W; ++q) v += wred[wave + q][t * NR + k];  // fixed order
            part[t][k] = v;
          }
      }
      __syncthreads();  // `wred` is reused by the next unit
    }

    if (lr == 0) {
#pragma unroll
      for (int t = 0; t < TILE; ++t) {
        const int r = row0 + t;
        if (r >= out_f) continue;
        if constexpr (SWIGLU) {
          const float g = part[t][0], u = part[t][1];
          ((uint16_t *)yout)[r] = f2h(g / (1.0f + __expf(-g)) * u);
        } else {
          float v = part[t][0];
          if (bias) v += h2f(bias[r]);
          float *y = (float *)yout;
          y[r] = accum ? y[r] + v : v;
        }
      }
    }
  }
}

// Fallback for rows wider than 28672 columns: x is re-read from L2 per group
// rather than held in registers. Same arithmetic per group; plain GEMV only.
template <int TILE>
__global__ __launch_bounds__(256) void gemv_hier_wide_kernel(
    const uint4 *__restrict__ qw, const uint8_t *__restrict__ si,
    const uint32_t *__restrict__ sb, const uint16_t *__restrict__ x,
    const uint16_t *__restrict__ bias, float *__restrict__ y, int in_f, int out_f, int accum,
    uint32_t magic) {
  const int tid = threadIdx.x, G = in_f / HGROUP;
  __shared__ float red[4][TILE];
  const int nunits = (out_f + TILE - 1) / TILE;
  for (int unit = blockIdx.x; unit < nunits; unit += gridDim.x) {
    const int row0 = unit * TILE;
    float as[TILE], am[TILE];
#pragma unroll
    for (int t = 0; t < TILE; ++t) as[t] = am[t] = 0.0f;
    for (int g = tid; g < G; g += 256) {
      XGroup xg;
      load_xgroup(x, g, xg);
#pragma unroll
      for (int t = 0; t < TILE; ++t) {
        const int r = row0 + t;
        if (r >= out_f) continue;
        const size_t at = (size_t)r * G + g;
        const uint32_t id = si[at];
        const float q = group_dot(ld_stream16(qw + at), xg, magic);
        as[t] = fmaf((float)(id & 0xFu), q, as[t]);
        am[t] = fmaf((float)(id >> 4), xg.sum, am[t]);
      }
    }
    float part[TILE];
#pragma unroll
    for (int t = 0; t < TILE; ++t) {
      const int r = row0 + t < out_f ? row0 + t : out_f - 1;
      const uint32_t sv = sb[r];
      part[t] = wave_sum(h2f((uint16_t)(sv & 0xFFFFu)) * as[t] - h2f((uint16_t)(sv >> 16)) * am[t]);
    }
    if ((tid & 63) == 0)
#pragma unroll
      for (int t = 0; t < TILE; ++t) red[tid >> 6][t] = part[t];
    __syncthreads();
    if (tid == 0) {
#pragma unroll
      for (int t = 0; t < TILE; ++t) {
        const int r = row0 + t;
        if (r >= out_f) continue;
        float v = red[0][t] + red[1][t] + red[2][t] + red[3][t];
        if (bias) v += h2f(bias[r]);
        y[r] = accum ? y[r] + v : v;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- dispatch

// Tile rule (wide reduction, huge output, everything else), entries 0..3 ->
// TILE 1, 2, 4, 8 rows per row-slot. Same knob and classes as the reference
// (gemv_hier.cu:253-272); the defaults are this kernel's own.
static int g_hier_rule[3] = {1, 2, 2};

extern "C" void wst_gemv_hier_set_rule(int32_t wide, int32_t huge, int32_t other) {
  if (wide >= 0 && wide < 4) g_hier_rule[0] = wide;
  if (huge >= 0 && huge < 4) g_hier_rule[1] = huge;
  if (other >= 0 && other < 4) g_hier_rule[2] = other;
}

extern "C" void wst_gemv_hier_get_rule(int32_t *out) {
  if (!out) return;
  out[0] = g_hier_rule[0];
  out[1] = g_hier_rule[1];
  out[2] = g_hier_rule[2];
}

static int hier_tile_index(int in_f, int rows) {
  if (in_f >= 2048) return g_hier_rule[0];
  if (rows >= 65536) return g_hier_rule[1];
  return g_hier_rule[2];
}

struct HierArgs {
  const void *qw, *si, *sb, *x;
  const void *norm_w;
  float eps;
  void *h_out;
  const void *bias;
  void *y;
  int in_f, out_f, accum;
};

// Persistent grid: a few blocks per CU stream every row; each block stages x
// once. WST_GEMV_BLOCKS_PER_CU overrides the default (for sweeps).
static int blocks_per_cu() {
  static int v = 0;
  if (v == 0) {
    const char *e = getenv("WST_GEMV_BLOCKS_PER_CU");
    v = e ? atoi(e) : 0;
    if (v <= 0 || v > 64) v = 4;
  }
  return v;
}

template <int LPR, int NG, int TILE, bool NORM, bool SWIGLU>
static void launch_t(const HierArgs &a) {
  const int rows_per_block = (256 / LPR) * TILE;
  const int units = (a.out_f + rows_per_block - 1) / rows_per_block;
  const int cap = wst_cu_count() * blocks_per_cu();
  const int grid = units < cap ? units : cap;
  const size_t lds = (size_t)a.in_f * 2;
  gemv_hier_kernel<LPR, NG, TILE, NORM, SWIGLU><<<grid, 256, lds, WST_STREAM>>>(
      (const uint4 *)a.qw, (const uint8_t *)a.si, (const uint32_t *)a.sb, a.x,
      (const uint16_t *)a.norm_w, a.eps, (uint16_t *)a.h_out, (const uint16_t *)a.bias, a.y,
      a.in_f, a.out_f, a.accum, HIER_MAGIC);
}

template <int LPR, int NG, bool NORM, bool SWIGLU>
static void launch_tile(int tile_idx, const HierArgs &a) {
  switch (tile_idx) {
    case 0: launch_t<LPR, NG, 1, NORM, SWIGLU>(a); break;
    case 1: launch_t<LPR, NG, 2, NORM, SWIGLU>(a); break;
    case 3: launch_t<LPR, NG, 8, NORM, SWIGLU>(a); break;
    default: launch_t<LPR, NG, 4, NORM, SWIGLU>(a); break;
  }
}

// Shape -> (lanes per row, groups per lane): at most 3 groups (48 VGPRs of x)
// per lane up to in_f = 24576, 4 up to 28672 (the staged x is in_f*2 bytes of
// LDS; past that the wide kernel reads x from L2).
template <bool NORM, bool SWIGLU>
static bool hier_dispatch(int tile_idx, const HierArgs &a) {
  const int G = a.in_f / HGROUP;
  if (G <= 32) launch_tile<32, 1, NORM, SWIGLU>(tile_idx, a);
  else if (G <= 64) launch_tile<64, 1, NORM, SWIGLU>(tile_idx, a);
  else if (G <= 128) launch_tile<64, 2, NORM, SWIGLU>(tile_idx, a);
  else if (G <= 192) launch_tile<64, 3, NORM, SWIGLU>(tile_idx, a);
  else if (G <= 384) launch_tile<128, 3, NORM, SWIGLU>(tile_idx, a);
  else if (G <= 768) launch_tile<256, 3, NORM, SWIGLU>(tile_idx, a);
  else if (G <= 896) launch_tile<256, 4, NORM, SWIGLU>(tile_idx, a);
  else return false;
  return true;
}

static wst_status_t check_common(const void *qw, const void *si, const void *sb, const void *x,
                                 const void *y, int32_t in_f, int32_t out_f, const char *who) {
  if (!(qw && si && sb && x && y)) {
    snprintf(wst_err_buf, sizeof(wst_err_buf), "%s: null pointer", who);
    return WST_ERR_INVALID_ARG;
  }
  if (in_f <= 0 || out_f <= 0) {
    snprintf(wst_err_buf, sizeof(wst_err_buf), "%s: non-positive dimension", who);
    return WST_ERR_INVALID_ARG;
  }
  if (in_f % HGROUP != 0) {
    snprintf(wst_err_buf, sizeof(wst_err_buf), "%s: in_features must be a multiple of 32", who);
    return WST_ERR_INVALID_ARG;
  }
  // Groups and activations are read 16 bytes at a time.
  if (((uintptr_t)qw | (uintptr_t)x) & 15u) {
    snprintf(wst_err_buf, sizeof(wst_err_buf), "%s: qw and x must be 16-byte aligned", who);
    return WST_ERR_INVALID_ARG;
  }
  return WST_OK;
}

extern "C" wst_status_t wst_gemv_int4_hier_ex(const void *qw, const void *si, const void *sb,
                                              const void *x, const void *bias, void *y,
                                              int32_t in_f, int32_t out_f, int32_t accum) {
  const wst_status_t st = check_common(qw, si, sb, x, y, in_f, out_f, "wst_gemv_int4_hier");
  if (st != WST_OK) return st;
  const HierArgs a{qw, si, sb, x, nullptr, 0.0f, nullptr, bias, y, in_f, out_f, accum};
  if (!hier_dispatch<false, false>(hier_tile_index(in_f, out_f), a)) {
    const int units = (out_f + 3) / 4;
    const int cap = wst_cu_count() * 16;
    gemv_hier_wide_kernel<4><<<units < cap ? units : cap, 256, 0, WST_STREAM>>>(
        (const uint4 *)qw, (const uint8_t *)si, (const uint32_t *)sb, (const uint16_t *)x,
        (const uint16_t *)bias, (float *)y, in_f, out_f, accum, HIER_MAGIC);
  }
  WST_TRY_KERNEL("wst_gemv_int4_hier");
  return WST_OK;
}

extern "C" wst_status_t wst_gemv_hier_rmsnorm(const void *qw, const void *si, const void *sb,
                                              const void *x, const void *norm_w, float eps,
                                              void *h_out, const void *bias, void *y,
                                              int32_t in_f, int32_t out_f, int32_t accum) {
  const wst_status_t st = check_common(qw, si, sb, x, y, in_f, out_f, "wst_gemv_hier_rmsnorm");
  if (st != WST_OK) return st;
  WST_REQUIRE(norm_w, "wst_gemv_hier_rmsnorm: null norm weight");
  WST_REQUIRE(in_f <= 28672, "wst_gemv_hier_rmsnorm: in_features above 28672");
  WST_REQUIRE(!(((uintptr_t)norm_w | (uintptr_t)h_out) & 15u),
              "wst_gemv_hier_rmsnorm: norm weight and h must be 16-byte aligned");
  const HierArgs a{qw, si, sb, x, norm_w, eps, h_out, bias, y, in_f, out_f, accum};
  hier_dispatch<true, false>(hier_tile_index(in_f, out_f), a);
  WST_TRY_KERNEL("wst_gemv_hier_rmsnorm");
  return WST_OK;
}

extern "C" wst_status_t wst_gemv_hier_swiglu(const void *qw, const void *si, const void *sb,
                                             const void *x, const void *norm_w, float eps,
                                             void *out, int32_t in_f, int32_t inter) {
  const wst_status_t st = check_common(qw, si, sb, x, out, in_f, inter, "wst_gemv_hier_swiglu");
  if (st != WST_OK) return st;
  WST_REQUIRE(in_f <= 28672, "wst_gemv_hier_swiglu: in_features above 28672");
  WST_REQUIRE(!((uintptr_t)norm_w & 15u), "wst_gemv_hier_swiglu: norm weight must be 16-byte aligned");
  const HierArgs a{qw, si, sb, x, norm_w, eps, nullptr, nullptr, out, in_f, inter, 0};
  const int ti = hier_tile_index(in_f, 2 * inter);
  if (norm_w) hier_dispatch<true, true>(ti, a);
  else hier_dispatch<false, true>(ti, a);
  WST_TRY_KERNEL("wst_gemv_hier_swiglu");
  return WST_OK;
}
