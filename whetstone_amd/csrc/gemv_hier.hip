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
//   dwordx4 load, and a row-slot of 64 consecutive lanes (32 when a row has at
//   most 32 groups) reads a contiguous run of the row. A wave therefore issues
//   1 KB-wide coalesced loads. Waves are independent (no barriers after the
//   prologue) and the kernel is kept near 64 VGPRs so 8 waves share a SIMD:
//   at this size occupancy, not per-wave prefetch depth, is what keeps enough
//   bytes in flight to stream HBM3E (measured: 5.9 TB/s of 8 on the 7B
//   gate|up shape with this arithmetic, vs 4 TB/s at 100+ VGPRs).
// * x lives in LDS as a per-group table prepared once per block: the 32
//   activations of a group, permuted so that the nibble pairs produced by one
//   bit-field insert line up with the activation pairs they multiply, plus the
//   group's two correction sums. Entries are 80 bytes apart, which keeps a
//   wave's ds_read_b128 free of bank conflicts.
// * Unpack without conversions: inserting a nibble into the mantissa of f16
//   1024.0 gives 1024+q exactly; nibbles in bits 4..7 give 1024+16q. One
//   v_bfi_b32 per pair of weights, one shift per word, and v_dot2c_f32_f16
//   multiplies two of them by two activations with an f32 accumulator:
//       sum_i q_i x_i = DA + DB/16 - (1024*sum_even x + 64*sum_odd x)
//   where DA (DB) accumulates the even (odd) columns. About 1.1 VALU
//   instructions per weight, every product accumulated in f32 -- more precise
//   than the reference's f16 half2 accumulation inside a group.
// * Per row: y = d * sum_g ls_g*Q_g - dmin * sum_g lm_g*S_g, reduced across the
//   row-slot with DPP. A row's value depends only on (in_f, the row's bytes,
//   x): not on TILE, the grid, or which fused form ran, so the fused kernels
//   can be checked bit for bit against the unfused ABI sequence.
#include "common.hpp"

#include <stdlib.h>

#define HGROUP 32
#define HIER_MAGIC 0x64006400u  // f16 1024.0 in both halves
#define GEMV_THREADS 512
#define XG_WORDS 20      // LDS words per group entry (18 used)
#define GEMV_MAX_G 768   // groups per row handled by the LDS-table kernel

// Bit-field insert (a & m) | (b & ~m) as one v_bfi_b32: the mask lives in a
// VGPR and the magic constant in an SGPR kernel argument. (Left to itself the
// compiler emits v_and + v_or with a literal, one more VALU op per pair.)
__device__ __forceinline__ uint32_t bfi(uint32_t a, uint32_t m, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(a), "s"(b));
  return r;
}

// A group's activations as the unpack consumes them.
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

__device__ __forceinline__ void store_xgroup(uint32_t *e, const XGroup &xg) {
  uint4 *v = (uint4 *)e;
  v[0] = make_uint4(xg.ea[0], xg.ea[1], xg.ea[2], xg.ea[3]);
  v[1] = make_uint4(xg.ob[0], xg.ob[1], xg.ob[2], xg.ob[3]);
  v[2] = make_uint4(xg.ea2[0], xg.ea2[1], xg.ea2[2], xg.ea2[3]);
  v[3] = make_uint4(xg.ob2[0], xg.ob2[1], xg.ob2[2], xg.ob2[3]);
  e[16] = __float_as_uint(xg.corr);
  e[17] = __float_as_uint(xg.sum);
}

__device__ __forceinline__ void load_xgroup_lds(const uint32_t *e, XGroup &xg) {
  const uint4 *v = (const uint4 *)e;
  const uint4 a = v[0], b = v[1], c = v[2], d = v[3];
  xg.ea[0] = a.x; xg.ea[1] = a.y; xg.ea[2] = a.z; xg.ea[3] = a.w;
  xg.ob[0] = b.x; xg.ob[1] = b.y; xg.ob[2] = b.z; xg.ob[3] = b.w;
  xg.ea2[0] = c.x; xg.ea2[1] = c.y; xg.ea2[2] = c.z; xg.ea2[3] = c.w;
  xg.ob2[0] = d.x; xg.ob2[1] = d.y; xg.ob2[2] = d.z; xg.ob2[3] = d.w;
  xg.corr = __uint_as_float(e[16]);
  xg.sum = __uint_as_float(e[17]);
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
// LPR (32 or 64) lanes own a row; lane lr holds groups lr, lr+LPR, ... (NG of
// them). A unit is TILE rows per row-slot; units are handed to waves
// round-robin over the whole grid, so after the prologue every wave runs on
// its own.
//
// NORM:   x is the f32 residual stream; the prologue computes the RMS scale
//         (the same reduction as the RMSNorm kernel) and normalises with
//         norm_w while building the table (wst_rmsnorm + GEMV). Block 0 also
//         stores h when h_out is non-null.
// SWIGLU: out_f is the intermediate width; unit row r computes gate row r and
//         up row r + out_f of the fused matrix and writes f16(silu(g) * u)
//         (GEMV + wst_swiglu).
template <int LPR, int NG, int TILE, bool NORM, bool SWIGLU>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_hier_kernel(
    const uint4 *__restrict__ qw, const uint8_t *__restrict__ si,
    const uint32_t *__restrict__ sb, const void *__restrict__ xin,
    const uint16_t *__restrict__ norm_w, float eps, uint16_t *__restrict__ h_out,
    const uint16_t *__restrict__ bias, void *__restrict__ yout, int in_f, int out_f, int accum,
    uint32_t magic) {
  constexpr int SLOTS = 64 / LPR;    // row-slots per wave
  constexpr int NR = SWIGLU ? 2 : 1;  // matrix rows per unit row
  const int tid = threadIdx.x, lane = tid & 63;
  const int slot = lane / LPR, lr = lane % LPR;
  const int G = in_f / HGROUP;

  __shared__ float red[16];
  extern __shared__ uint32_t xgt[];  // [G][XG_WORDS]

  // ---- prologue: the x table
  float s = 0.0f;
  if constexpr (NORM) {
    // rms_scale256's reduction, spread over 512 threads with the upper 256
    // contributing exact zeros: same bits as the RMSNorm kernel.
    // The first 16 strided values are loaded together (one round trip), then
    // accumulated in index order.
    const float *x = (const float *)xin;
    float acc = 0.0f;
    if (tid < 256) {
      float v[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int i = tid + 256 * k;
        v[k] = i < in_f ? x[i] : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (tid + 256 * k < in_f) acc = fmaf(v[k], v[k], acc);
      for (int i = tid + 256 * 16; i < in_f; i += 256) acc = fmaf(x[i], x[i], acc);
    }
    s = 1.0f / sqrtf(block_sum(acc, red) / (float)in_f + eps);
  }
  for (int g = tid; g < G; g += GEMV_THREADS) {
    uint32_t r[16];
    if constexpr (NORM) {
      const float4 *xv = (const float4 *)((const float *)xin + (size_t)g * HGROUP);
      const uint4 *wv = (const uint4 *)(norm_w + (size_t)g * HGROUP);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 a = xv[2 * i], b = xv[2 * i + 1];
        const uint4 ww = wv[i];
        const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        const uint32_t wp[4] = {ww.x, ww.y, ww.z, ww.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint16_t lo = f2h(xs[2 * k] * s * h2f((uint16_t)(wp[k] & 0xFFFFu)));
          const uint16_t hi = f2h(xs[2 * k + 1] * s * h2f((uint16_t)(wp[k] >> 16)));
          r[4 * i + k] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
      }
      if (h_out && blockIdx.x == 0) {
        uint4 *hv = (uint4 *)(h_out + (size_t)g * HGROUP);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          hv[i] = make_uint4(r[4 * i], r[4 * i + 1], r[4 * i + 2], r[4 * i + 3]);
      }
    } else {
      const uint4 *xv = (const uint4 *)((const uint16_t *)xin + (size_t)g * HGROUP);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 v = xv[i];
        r[4 * i] = v.x;
        r[4 * i + 1] = v.y;
        r[4 * i + 2] = v.z;
        r[4 * i + 3] = v.w;
      }
    }
    XGroup xg;
    build_xgroup(r, xg);
    store_xgroup(xgt + (size_t)g * XG_WORDS, xg);
  }
  __syncthreads();

  // ---- rows
  const int nunits = (out_f + SLOTS * TILE - 1) / (SLOTS * TILE);
  const int tw = gridDim.x * (GEMV_THREADS / 64);
  for (int unit = blockIdx.x * (GEMV_THREADS / 64) + (tid >> 6); unit < nunits; unit += tw) {
    const int row0 = (unit * SLOTS + slot) * TILE;
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
          const int g = lr + j * LPR;
          const size_t at = (size_t)r * G + g;
          if (rv && g < G) {
            wq[t][k][j] = ld_stream16(qw + at);
            idx[t][k][j] = si[at];
          } else {
            wq[t][k][j] = make_uint4(0, 0, 0, 0);
            idx[t][k][j] = 0;
          }
        }
      }
    }
    float as[TILE][NR], am[TILE][NR];
#pragma unroll
    for (int t = 0; t < TILE; ++t)
#pragma unroll
      for (int k = 0; k < NR; ++k) as[t][k] = am[t][k] = 0.0f;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int g = lr + j * LPR;
      if (g >= G) continue;
      XGroup xg;
      load_xgroup_lds(xgt + (size_t)g * XG_WORDS, xg);
#pragma unroll
      for (int t = 0; t < TILE; ++t)
#pragma unroll
        for (int k = 0; k < NR; ++k) {
          const float q = group_dot(wq[t][k][j], xg, magic);
          as[t][k] = fmaf((float)(idx[t][k][j] & 0xFu), q, as[t][k]);
          am[t][k] = fmaf((float)(idx[t][k][j] >> 4), xg.sum, am[t][k]);
        }
    }
#pragma unroll
    for (int t = 0; t < TILE; ++t) {
      float part[NR];
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        const float d = h2f((uint16_t)(sbv[t][k] & 0xFFFFu));
        const float dm = h2f((uint16_t)(sbv[t][k] >> 16));
        part[k] = slot_sum<LPR>(d * as[t][k] - dm * am[t][k]);
      }
      const int r = row0 + t;
      if (lr == 0 && r < out_f) {
        if constexpr (SWIGLU) {
          const float g = part[0], up = part[NR - 1];
          ((uint16_t *)yout)[r] = f2h(g / (1.0f + __expf(-g)) * up);
        } else {
          float v = part[0];
          if (bias) v += h2f(bias[r]);
          float *y = (float *)yout;
          y[r] = accum ? y[r] + v : v;
        }
      }
    }
  }
}

// Fallback for rows wider than GEMV_MAX_G groups: x is re-read from L2 per
// group. Same arithmetic per group; plain GEMV only.
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
      uint32_t r[16];
      const uint4 *xv = (const uint4 *)(x + (size_t)g * HGROUP);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 v = xv[i];
        r[4 * i] = v.x;
        r[4 * i + 1] = v.y;
        r[4 * i + 2] = v.z;
        r[4 * i + 3] = v.w;
      }
      XGroup xg;
      build_xgroup(r, xg);
#pragma unroll
      for (int t = 0; t < TILE; ++t) {
        const int rr = row0 + t;
        if (rr >= out_f) continue;
        const size_t at = (size_t)rr * G + g;
        const uint32_t id = si[at];
        const float q = group_dot(ld_stream16(qw + at), xg, magic);
        as[t] = fmaf((float)(id & 0xFu), q, as[t]);
        am[t] = fmaf((float)(id >> 4), xg.sum, am[t]);
      }
    }
    float part[TILE];
#pragma unroll
    for (int t = 0; t < TILE; ++t) {
      const int rr = row0 + t < out_f ? row0 + t : out_f - 1;
      const uint32_t sv = sb[rr];
      part[t] = wave_sum(h2f((uint16_t)(sv & 0xFFFFu)) * as[t] - h2f((uint16_t)(sv >> 16)) * am[t]);
    }
    if ((tid & 63) == 0)
#pragma unroll
      for (int t = 0; t < TILE; ++t) red[tid >> 6][t] = part[t];
    __syncthreads();
    if (tid == 0) {
#pragma unroll
      for (int t = 0; t < TILE; ++t) {
        const int rr = row0 + t;
        if (rr >= out_f) continue;
        float v = red[0][t] + red[1][t] + red[2][t] + red[3][t];
        if (bias) v += h2f(bias[rr]);
        y[rr] = accum ? y[rr] + v : v;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- dispatch

// Tile rule (wide reduction, huge output, everything else), entries 0..3 ->
// TILE 1, 2, 4, 8 rows per row-slot, clamped so a lane holds at most 16
// groups per unit. Same knob and classes as the reference
// (gemv_hier.cu:253-272); the defaults are this kernel's own.
static int g_hier_rule[3] = {0, 0, 1};

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

// Blocks per CU of the persistent grid. WST_GEMV_BLOCKS_PER_CU overrides the
// default (for sweeps).
static int blocks_per_cu() {
  static int v = 0;
  if (v == 0) {
    const char *e = getenv("WST_GEMV_BLOCKS_PER_CU");
    v = e ? atoi(e) : 0;
    if (v <= 0 || v > 64) v = 4;
  }
  return v;
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

template <int LPR, int NG, int TILE, bool NORM, bool SWIGLU>
static void launch_t(const HierArgs &a) {
  const int rows_per_wave = (64 / LPR) * TILE;
  const int units = (a.out_f + rows_per_wave - 1) / rows_per_wave;
  const int blocks = (units + GEMV_THREADS / 64 - 1) / (GEMV_THREADS / 64);
  const int cap = wst_cu_count() * blocks_per_cu();
  const int grid = blocks < cap ? blocks : cap;
  const size_t lds = (size_t)(a.in_f / HGROUP) * XG_WORDS * 4;
  gemv_hier_kernel<LPR, NG, TILE, NORM, SWIGLU><<<grid, GEMV_THREADS, lds, WST_STREAM>>>(
      (const uint4 *)a.qw, (const uint8_t *)a.si, (const uint32_t *)a.sb, a.x,
      (const uint16_t *)a.norm_w, a.eps, (uint16_t *)a.h_out, (const uint16_t *)a.bias, a.y,
      a.in_f, a.out_f, a.accum, HIER_MAGIC);
}

template <int LPR, int NG, bool NORM, bool SWIGLU>
static void launch_tile(int tile_idx, const HierArgs &a) {
  constexpr int NR = SWIGLU ? 2 : 1;
  int t = tile_idx;
  while (t > 0 && (1 << t) * NG * NR > 16) --t;  // register budget
  switch (t) {
    case 0: launch_t<LPR, NG, 1, NORM, SWIGLU>(a); break;
    case 1: if constexpr (2 * NG * NR <= 16) launch_t<LPR, NG, 2, NORM, SWIGLU>(a); break;
    case 2: if constexpr (4 * NG * NR <= 16) launch_t<LPR, NG, 4, NORM, SWIGLU>(a); break;
    default: if constexpr (8 * NG * NR <= 16) launch_t<LPR, NG, 8, NORM, SWIGLU>(a); break;
  }
}

// Shape -> (lanes per row, groups per lane).
template <bool NORM, bool SWIGLU>
static bool hier_dispatch(int tile_idx, const HierArgs &a) {
  const int G = a.in_f / HGROUP;
  const int ng = (G + 63) / 64;
  if (G <= 32) launch_tile<32, 1, NORM, SWIGLU>(tile_idx, a);
  else if (ng == 1) launch_tile<64, 1, NORM, SWIGLU>(tile_idx, a);
  else if (ng == 2) launch_tile<64, 2, NORM, SWIGLU>(tile_idx, a);
  else if (ng == 3) launch_tile<64, 3, NORM, SWIGLU>(tile_idx, a);
  else if (ng == 4) launch_tile<64, 4, NORM, SWIGLU>(tile_idx, a);
  else if (ng <= 6) launch_tile<64, 6, NORM, SWIGLU>(tile_idx, a);
  else if (ng <= 8) launch_tile<64, 8, NORM, SWIGLU>(tile_idx, a);
  else if (ng <= 10) launch_tile<64, 10, NORM, SWIGLU>(tile_idx, a);
  else if (ng <= 12) launch_tile<64, 12, NORM, SWIGLU>(tile_idx, a);
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
  if (in_f / HGROUP > GEMV_MAX_G || !hier_dispatch<false, false>(hier_tile_index(in_f, out_f), a)) {
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
  WST_REQUIRE(in_f / HGROUP <= GEMV_MAX_G, "wst_gemv_hier_rmsnorm: in_features above 24576");
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
  WST_REQUIRE(in_f / HGROUP <= GEMV_MAX_G, "wst_gemv_hier_swiglu: in_features above 24576");
  WST_REQUIRE(!((uintptr_t)norm_w & 15u), "wst_gemv_hier_swiglu: norm weight must be 16-byte aligned");
  const HierArgs a{qw, si, sb, x, norm_w, eps, nullptr, nullptr, out, in_f, inter, 0};
  const int ti = hier_tile_index(in_f, 2 * inter);
  if (norm_w) hier_dispatch<true, true>(ti, a);
  else hier_dispatch<false, true>(ti, a);
  WST_TRY_KERNEL("wst_gemv_hier_swiglu");
  return WST_OK;
}
