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
//   dwordx4 load, and a row's 64 (or 64*WPR) lanes read a contiguous run of it,
//   so a wave issues 1 KB-wide coalesced loads.
// * The arithmetic is integer. Counted with rocprofv3 (SQ_INSTS_VALU) the
//   earlier f16 formulation (nibble inserted into the mantissa of 1024.0, then
//   v_dot2c_f32_f16) cost ~277 VALU instructions per row pair per lane-group on
//   the 7B gate|up shape, about 9.5 us of SIMD time per 17 us launch: VALU was
//   a co-bottleneck with HBM. Here each group of activations is held as a
//   14-bit fixed-point integer split into four signed base-16 digits, and the
//   packed nibbles feed v_dot8_i32_i4 directly: one xor and four dot8 per 8
//   weights, no unpacking (see the activation table below).
// * x lives in LDS as that per-group table, built once per block from the
//   thread's own 8-column blocks while the block's first weight loads are in
//   flight (activation loads are issued first; a wave's loads return in
//   order). Entries are 80 bytes apart.
// * The grid is persistent: as many blocks as the CUs hold resident (two per
//   CU by default), units dealt round-robin so slot counts differ by at most
//   one. (WST_GEMV_GRID=balanced instead sizes the grid so every slot gets the
//   same count.)
// * Per row: y = d * sum_g ls_g*Q_g - dmin * sum_g lm_g*S_g, reduced across the
//   row's lanes with DPP (and LDS when a row spans waves). A row's value
//   depends only on (in_f, the row's bytes, x): not on the grid or on which
//   fused form ran, so the fused kernels are checked bit for bit against the
//   unfused ABI sequence.
// * The table can come from the producer of x instead (XT: wst_gemv_hier_xq
//   copies it memory -> LDS by DMA; TW: the SwiGLU form writes the table of
//   its own output, taking its rows 32 at a time so a block holds every
//   output of an entry). Both give the bits of the form that builds it.
// * Rows wider than GEMV_MAX_G groups fall back to a simple kernel with the f16
//   formulation (x read from L2).
#include "common.hpp"
#include "hier_xq.hpp"

#include <stdlib.h>

#define HGROUP 32
#define HIER_MAGIC 0x64006400u  // f16 1024.0 in both halves
#define GEMV_THREADS 512
#define XG_WORDS 20      // LDS words per group entry (18 used)
#define SUBS_OF(rpb) ((rpb) < 32 ? 32 / (rpb) : 1)
#define XT_CHUNKS(xb) ((5 * (xb) + 3) / 4)  // table chunks per thread for XB blocks of 8

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

// The attention slices as a GEMV input (AM forms): x[h*hd + d] is the merge
// of head h's per-slice partials (attention.hip's layout: numerators
// [n_q][nsplit][hd], then (max, sum) pairs [n_q][nsplit][2]) for the
// ceil(seq/P) slices holding cached positions, computed exactly as
// attn_merge_kernel computes it and rounded to f16.
#define AM_MAX_SLICES 8
struct AttnIn {
  const int32_t *pos;
  int nsplit, hd, n_q, max_seq, P;
};

// Eight merged attention outputs (columns 8b .. 8b+7, one head) as f16, the
// arithmetic of attn_merge_kernel for at most AM_MAX_SLICES slices (one
// batch: every live slice in slice order, after the batch's maximum). Every
// load is issued unconditionally (slice indices clamped), then dead slices
// are replaced by select.
// MS: the slices read (4 or AM_MAX_SLICES); slices past nsplit are clamped
// and replaced, so a cache of at most 4 slices gives the same bits either way.
template <int MS>
__device__ __forceinline__ uint4 merge8(const AttnIn &am, const float *partials, int b) {
  const int c0 = 8 * b, h = c0 / am.hd, d0 = c0 % am.hd;
  const float *pacc = partials;
  const float *pml = partials + (size_t)am.n_q * am.nsplit * am.hd;
  const size_t row0 = (size_t)h * am.nsplit;
  const int pos = *am.pos;
  float ms[MS], ls[MS], vs[MS][8];
#pragma unroll
  for (int sl = 0; sl < MS; ++sl) {
    const size_t r = row0 + min(sl, am.nsplit - 1);
    const float2 mlv = *(const float2 *)(pml + r * 2);
    ms[sl] = mlv.x;
    ls[sl] = mlv.y;
    const float4 v0 = *(const float4 *)(pacc + r * am.hd + d0);
    const float4 v1 = *(const float4 *)(pacc + r * am.hd + d0 + 4);
    vs[sl][0] = v0.x; vs[sl][1] = v0.y; vs[sl][2] = v0.z; vs[sl][3] = v0.w;
    vs[sl][4] = v1.x; vs[sl][5] = v1.y; vs[sl][6] = v1.z; vs[sl][7] = v1.w;
  }
  const int seq = min(max(pos, 0) + 1, am.max_seq);
  const int nactive = (seq + am.P - 1) / am.P;
  float M = -INFINITY;
#pragma unroll
  for (int sl = 0; sl < MS; ++sl) {
    const bool live = sl < nactive;
    ms[sl] = live ? ms[sl] : -INFINITY;
    ls[sl] = live ? ls[sl] : 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) vs[sl][e] = live ? vs[sl][e] : 0.0f;
    M = fmaxf(M, ms[sl]);
  }
  float f[MS];  // one exp per slice, shared by the eight columns
  float den = 0.0f;         // the merge kernel's a *= 0, den *= 0 from -inf
#pragma unroll
  for (int sl = 0; sl < MS; ++sl) {
    f[sl] = (ms[sl] == -INFINITY) ? 0.0f : __expf(ms[sl] - M);
    den = fmaf(ls[sl], f[sl], den);
  }
  uint16_t o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float a = 0.0f;
#pragma unroll
    for (int sl = 0; sl < MS; ++sl) a = fmaf(vs[sl][e], f[sl], a);
    o[e] = f2h(a / den);
  }
  return make_uint4(o[0] | ((uint32_t)o[1] << 16), o[2] | ((uint32_t)o[3] << 16),
                    o[4] | ((uint32_t)o[5] << 16), o[6] | ((uint32_t)o[7] << 16));
}

// The argmax epilogue (AX forms). Every block stores the largest argmax key
// of the rows it wrote (the order-preserving key of sample.cu:28-37) to its
// own slot of `keys`, a plain store; a one-block kernel launched after the
// GEMV takes the maximum of the slots, writes the token and advances the
// position. (An earlier form folded the keys with chains of agent-scope
// atomics into group maxima, the last block finishing: about 6 us on the 0.5B
// head, against about 2 us for the second launch.)
#define AX_MAX_BLOCKS 8192
struct ArgmaxOut {
  int32_t *out, *pos;
  int max_seq;
  unsigned long long *keys;  // [gridDim.x]
};

// Sum over a row's lanes when a row spans LPR <= 64 lanes of one wave (every
// lane of the row gets the sum).
template <int LPR>
__device__ __forceinline__ float slot_sum(float v) {
  if constexpr (LPR == 8) return dpp_sum8(v);
  else if constexpr (LPR == 16) return dpp_sum16(v);
  else if constexpr (LPR == 32) return half_wave_sum(v);
  else return wave_sum(v);
}

// ---------------------------------------------------------------- the kernel
//
// y for one or two rows (SWIGLU: gate row r and up row r + nunits).
//
// NG groups per lane, WPR waves per row (a row's lanes are lr = 0..64*WPR-1,
// lane lr holding groups lr, lr + 64*WPR, ...), XB activation blocks of 8 per
// thread (in_f <= XB * 8 * NT), NT threads per block. A block works on
// NT/64/WPR rows at a time; units (rows, or row pairs) are dealt to the block's
// row slots round-robin over the grid.
//
// Each thread first issues the loads of its activation blocks, then the loads
// of its first unit's packed bytes; the table is built while those are in
// flight (a wave's loads return in order, so the table waits only for x).
//
// NORM:   x is the f32 residual stream; h = f16(x * rms * w) is formed in
//         registers (the RMS with the same reduction as wst_rmsnorm), block 0
//         also stores h when h_out is non-null. Requires NT == NORM_THREADS.
// SWIGLU: nunits is the intermediate width; the unit writes f16(silu(g) * u).
//
// qw, si, xin and norm_w are deliberately not __restrict__: loads through
// restrict-const pointers count as invariant, and the compiler then issues
// the weight loads ahead of the activation loads.
//
// PD: units in flight per row slot (1: the next unit's loads are issued after
// the current unit's compute; PD > 1: PD - 1 more units are always in flight).
// RPW: rows per wave for short rows (WPR == 1): a row is 64 / RPW lanes of a
// wave, so a wave streams RPW rows at once.
// AX: the argmax epilogue above (plain rows only).
template <int NG, int WPR, int XB, int NT, bool NORM, bool SWIGLU, int PD, int RPW = 1,
          int AM = 0, bool AX = false, bool XT = false, bool TW = false>
__global__ __launch_bounds__(NT) void gemv_hier_kernel(
    const uint4 *qw, const uint8_t *si,
    const uint32_t *__restrict__ sb, const void *xin,
    const uint16_t *norm_w, float eps, uint16_t *__restrict__ h_out,
    const uint16_t *__restrict__ bias, void *__restrict__ yout, int in_f, int nunits,
    int accum, AttnIn am, ArgmaxOut ax, uint32_t *__restrict__ tw) {
  static_assert(!NORM || NT == NORM_THREADS, "the RMS reduction order assumes 512 threads");
  static_assert(!AX || !SWIGLU, "the argmax epilogue takes plain rows");
  static_assert(!XT || (!NORM && !AM), "a prebuilt table replaces the activation loads");
  static_assert(!TW || (SWIGLU && PD == 1), "the table of the output: SwiGLU rows, one unit in flight");
  constexpr int NR = SWIGLU ? 2 : 1;
  static_assert(RPW == 1 || WPR == 1, "rows share a wave only when a row is one wave or less");
  constexpr int NW = NT / 64;
  constexpr int RPB = NW / WPR * RPW;
  constexpr int LPR = WPR > 1 ? 64 * WPR : 64 / RPW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rs = (wave / WPR) * RPW + (RPW > 1 ? lane / LPR : 0);
  const int lr = WPR > 1 ? (wave % WPR) * 64 + lane : lane % LPR;
  const int G = in_f / HGROUP, NB8 = in_f / 8;
  __shared__ float red[2][NW][NR];
  __shared__ float bred[16];
  __shared__ uint16_t tws[TW ? 2 * RPB * SUBS_OF(RPB) : 1];  // TW: outputs of two group units
  extern __shared__ uint32_t xgt[];  // [G][XQ_WORDS]

  // 1. this thread's activation blocks b = tid + NT*i (and norm gains)
  float xf[NORM ? XB : 1][8];
  uint4 xh[NORM ? 1 : XB];
  uint4 nwv[NORM ? XB : 1];
  // XT: the table itself, G entries of XQ_WORDS words (5 16-byte chunks),
  // copied memory -> LDS by DMA (global_load_lds_dwordx4: lane l's 16 bytes
  // land at M0 + 16 l), no registers held; in_f <= 8 * XB * NT bounds it by
  // XTL * NT chunks (the launch sizes the LDS for that many: clamped lanes
  // write copies of the last chunk past the table).
  // Every load below is unconditional (indices clamped, values masked): the
  // code stays straight-line, so the compiler counts the loads in flight and
  // waits for exactly the ones it needs (a load under a branch is followed by
  // a wait for everything outstanding).
  if constexpr (XT) {
    const uint32_t l0 = (uint32_t)(uintptr_t)xgt;
#pragma unroll
    for (int i = 0; i < XT_CHUNKS(XB); ++i) {
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(l0 + 16u * (uint32_t)(wave * 64 + NT * i));
      const uint32_t off = 16u * (uint32_t)min(tid + NT * i, G * (XQ_WORDS / 4) - 1);
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                   :: "s"(m0), "v"(off), "s"(xin) : "memory");
    }
  }
#pragma unroll
  for (int i = 0; i < (XT ? 0 : XB); ++i) {
    const int b = tid + NT * i;
    if constexpr (NORM) {
      const int bc = min(b, NB8 - 1);
      const float4 *xv = (const float4 *)((const float *)xin + (size_t)bc * 8);
      const float4 a = xv[0], c = xv[1];
      xf[i][0] = a.x; xf[i][1] = a.y; xf[i][2] = a.z; xf[i][3] = a.w;
      xf[i][4] = c.x; xf[i][5] = c.y; xf[i][6] = c.z; xf[i][7] = c.w;
      nwv[i] = *(const uint4 *)(norm_w + (size_t)bc * 8);
    } else if constexpr (AM) {
      xh[i] = merge8<AM>(am, (const float *)xin, min(b, NB8 - 1));
    } else {
      xh[i] = *(const uint4 *)((const uint16_t *)xin + (size_t)min(b, NB8 - 1) * 8);
    }
  }

  // The activation loads are issued before the weight loads (a wave's loads
  // return in order, so the table waits only for them); the non-restrict
  // pointers keep the compiler from hoisting the weights above them.

  // 2. the first PD units' packed bytes
  const int stride = gridDim.x * RPB;
  // First row of the block's t-th unit slot set. TW: a block takes whole
  // groups of 32 consecutive rows (one group unit per 32 / RPB iterations,
  // or RPB / 32 group units per iteration), so that it holds every output
  // of a table entry; otherwise units are dealt round-robin.
  constexpr int SUBS = RPB < 32 ? 32 / RPB : 1;
  static_assert(!TW || 32 % RPB == 0 || RPB % 32 == 0, "whole groups per block");
  auto row0 = [&](int t) -> int {
    if constexpr (TW && RPB < 32)
      return 32 * (blockIdx.x + (t / SUBS) * gridDim.x) + RPB * (t % SUBS);
    else
      return blockIdx.x * RPB + t * stride;
  };
  struct Buf {
    uint4 wq[NR][NG];
    uint32_t idx[NR][NG];
    uint32_t sbv[NR];
  };
  Buf bufs[PD];
  auto load_unit = [&](Buf &B, int row) {  // row clamped: past the end loads are unused
    const int rc = min(row, nunits - 1);
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const int r = rc + k * nunits;
      B.sbv[k] = sb[r];
      const uint4 *qr = qw + (size_t)r * G;
      const uint8_t *sr = si + (size_t)r * G;
#pragma unroll
      for (int j = 0; j < NG; ++j) {
        const int g = min(lr + j * LPR, G - 1);  // lanes past G compute nothing
        B.wq[k][j] = ld_stream16(qr + g);
        B.idx[k][j] = sr[g];
      }
    }
  };
  // (units 1..PD-1 go out after the table: issued here they would queue the
  // activation fetch behind them; 0.5B head 5.06 -> 5.21 TB/s over six A/B
  // pairs)
  load_unit(bufs[0], row0(0) + rs);

  // 3. the RMS scale (rms_scale512's order: thread t, blocks t, t+512, ...)
  float s = 1.0f;
  if constexpr (NORM) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < XB; ++i) {
      if (tid + NT * i >= NB8)  // clamped duplicates contribute nothing
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[i][e] = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf(xf[i][e], xf[i][e], acc);
    }
    s = 1.0f / sqrtf(block_sum(acc, bred) / (float)in_f + eps);
  }

  // 4. the table
  if constexpr (XT) {
    // The DMA went out before the first unit's loads (2 per group and row:
    // packed bytes and scale index; later units go out after the table);
    // waiting for all but those many leaves the weights in flight. (Where the
    // compiler loads the row scales with vector loads too, the wait also
    // covers the first of the weights.)
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * NR * NG) : "memory");
  }
#pragma unroll
  for (int i = 0; i < (XT ? 0 : XB); ++i) {
    const int b = tid + NT * i;
    uint16_t h[8];
    if constexpr (NORM) {
      const uint32_t nw[4] = {nwv[i].x, nwv[i].y, nwv[i].z, nwv[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        h[2 * k] = f2h(xf[i][2 * k] * s * h2f((uint16_t)(nw[k] & 0xFFFFu)));
        h[2 * k + 1] = f2h(xf[i][2 * k + 1] * s * h2f((uint16_t)(nw[k] >> 16)));
      }
      if (h_out && blockIdx.x == 0 && b < NB8)
        *(uint4 *)(h_out + (size_t)b * 8) =
            make_uint4(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16),
                       h[4] | ((uint32_t)h[5] << 16), h[6] | ((uint32_t)h[7] << 16));
    } else {
      const uint32_t w[4] = {xh[i].x, xh[i].y, xh[i].z, xh[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        h[2 * k] = (uint16_t)(w[k] & 0xFFFFu);
        h[2 * k + 1] = (uint16_t)(w[k] >> 16);
      }
    }
    build_xq(h, b, b < NB8, xgt);
  }
  __syncthreads();
#pragma unroll
  for (int i = 1; i < PD; ++i) load_unit(bufs[i], row0(i) + rs);

  // A lane's groups are the same for every unit, so with at most two groups
  // per lane their table entries move to registers once, here, instead of
  // being read from LDS for every unit (76 bytes per group and unit).
  constexpr bool HOIST = NG <= 2;
  uint4 hl[HOIST ? NG : 1][4];
  int hc8[HOIST ? NG : 1];
  float hS[HOIST ? NG : 1], hsc[HOIST ? NG : 1];
  if constexpr (HOIST) {
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const uint32_t *e = xgt + (size_t)min(lr + j * LPR, G - 1) * XQ_WORDS;
#pragma unroll
      for (int q = 0; q < 4; ++q) hl[j][q] = *(const uint4 *)(e + 4 * q);
      hc8[j] = (int)e[16];
      hS[j] = __uint_as_float(e[17]);
      hsc[j] = __uint_as_float(e[18]);
    }
  }

  // 5. rows. The trip count is the same for every wave of the block (the
  // WPR > 1 reduction synchronises the block).
  // Every block has at least one unit (the launch sizes the grid so), and a
  // do-while keeps the first unit's loads where they are issued: under a
  // `base < nunits` guard the compiler would move them past the barrier.
  int it = 0;
  unsigned long long best = 0ull;  // AX: largest key of the rows this thread wrote
  // One unit from B; B is then refilled with the unit PD strides ahead, issued
  // after the compute and before the reductions and stores.
  auto process = [&](Buf &B) {
    const int row = row0(it) + rs;
    // The epilogue's operands are fetched now, ahead of the next unit's weight
    // loads, so that waiting for them later does not wait for those too.
    float yv = 0.0f, bv = 0.0f;
    if constexpr (!SWIGLU) {
      const int rowc = min(row, nunits - 1);
      yv = ((const float *)yout)[rowc];
      bv = h2f((bias ? bias : (const uint16_t *)sb)[rowc]);  // sb: any readable row
    }
    float as[NR], am[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) as[k] = am[k] = 0.0f;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int g = lr + j * LPR;
      if (g >= G) continue;
      uint4 l0, l1, l2, l3;
      int c8;
      float S, sc;
      if constexpr (HOIST) {
        l0 = hl[j][0]; l1 = hl[j][1]; l2 = hl[j][2]; l3 = hl[j][3];
        c8 = hc8[j];
        S = hS[j];
        sc = hsc[j];
      } else {
        const uint32_t *e = xgt + (size_t)g * XQ_WORDS;
        l0 = *(const uint4 *)(e); l1 = *(const uint4 *)(e + 4);
        l2 = *(const uint4 *)(e + 8); l3 = *(const uint4 *)(e + 12);
        c8 = (int)e[16];
        S = __uint_as_float(e[17]);
        sc = __uint_as_float(e[18]);
      }
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        const uint4 p = B.wq[k][j];
        const uint32_t w0 = p.x ^ 0x88888888u, w1 = p.y ^ 0x88888888u;
        const uint32_t w2 = p.z ^ 0x88888888u, w3 = p.w ^ 0x88888888u;
        int a0 = sdot8(w0, l0.x, c8), a1 = sdot8z(w0, l0.y);
        int a2 = sdot8z(w0, l0.z), a3 = sdot8z(w0, l0.w);
        a0 = sdot8(w1, l1.x, a0); a1 = sdot8(w1, l1.y, a1);
        a2 = sdot8(w1, l1.z, a2); a3 = sdot8(w1, l1.w, a3);
        a0 = sdot8(w2, l2.x, a0); a1 = sdot8(w2, l2.y, a1);
        a2 = sdot8(w2, l2.z, a2); a3 = sdot8(w2, l2.w, a3);
        a0 = sdot8(w3, l3.x, a0); a1 = sdot8(w3, l3.y, a1);
        a2 = sdot8(w3, l3.z, a2); a3 = sdot8(w3, l3.w, a3);
        const int t = a0 + (a1 << 4) + (a2 << 8) + (a3 << 12);  // sum_i q_i X_i
        const uint32_t id = B.idx[k][j];
        as[k] = fmaf((float)(id & 0xFu) * sc, (float)t, as[k]);
        am[k] = fmaf((float)(id >> 4), S, am[k]);
      }
    }
    float lv[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const float d = h2f((uint16_t)(B.sbv[k] & 0xFFFFu));
      const float dm = h2f((uint16_t)(B.sbv[k] >> 16));
      lv[k] = d * as[k] - dm * am[k];
    }
    // The next unit's loads. With one unit in flight they are skipped when
    // that unit lies past the last row (a wave-uniform branch): issued
    // anyway, clamped to the last row, every wave of the grid ended on a
    // request to the same few cache lines (7B step 788 -> 797-804 tok/s,
    // 0.5B 1,806 -> 1,878-1,901). The next compute waits for this unit's
    // loads in any case. With two or more in flight the branch made the
    // compiler wait for every outstanding load (7B head 48.3 -> 54.1 us), so
    // those keep the clamped loads.
    if (PD > 1 || row0(it + PD) + rs < nunits) load_unit(B, row0(it + PD) + rs);
    float part[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) part[k] = WPR > 1 ? wave_sum(lv[k]) : slot_sum<LPR>(lv[k]);
    if constexpr (WPR > 1) {
      if (lane == 0)
#pragma unroll
        for (int k = 0; k < NR; ++k) red[it & 1][wave][k] = part[k];
      __syncthreads();
      if (lane == 0 && (wave % WPR) == 0) {
#pragma unroll
        for (int k = 0; k < NR; ++k) {
          float v = red[it & 1][wave][k];
#pragma unroll
          for (int w = 1; w < WPR; ++w) v += red[it & 1][wave + w][k];
          part[k] = v;
        }
      }
    }
    if (lr == 0 && row < nunits) {
      if constexpr (SWIGLU) {
        const float g = part[0], up = part[NR - 1];
        const uint16_t a = f2h(g / (1.0f + __expf(-g)) * up);
        ((uint16_t *)yout)[row] = a;
        if constexpr (TW) tws[((it / SUBS) & 1) * RPB * SUBS + RPB * (it % SUBS) + rs] = a;
      } else {
        float v = part[0];
        if (bias) v += bv;
        const float yr = accum ? yv + v : v;
        ((float *)yout)[row] = yr;
        if constexpr (AX) {
          const unsigned long long key = argmax_key(yr, row);
          best = key > best ? key : best;
        }
      }
    }
    if constexpr (TW) {
      // The last iteration of a group unit: its table entries (one quad of
      // lanes per 32 outputs, as the GEMV prologue builds them).
      if (it % SUBS == SUBS - 1) {
        __syncthreads();
        const uint16_t *src = tws + ((it / SUBS) & 1) * RPB * SUBS;
        const int nq = RPB * SUBS / 8;  // threads of 8 outputs: 4 per group
        const int r8 = row0(it - SUBS + 1) + 8 * tid;
        if (tid < nq && r8 < nunits) {  // whole groups: nunits is a multiple of 32
          uint16_t h[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) h[e] = src[8 * tid + e];
          build_xq(h, r8 / 8, true, tw);
        }
      }
    }
    ++it;
  };
  do {
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      process(bufs[i]);
      if (PD > 1 && row0(it) >= nunits) break;
    }
  } while (row0(it) < nunits);
  if constexpr (AX) {
    __shared__ unsigned long long wbest[NW];
    best = wave_max_u64(best);
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (tid == 0) {
      unsigned long long b = wbest[0];
#pragma unroll
      for (int w = 1; w < NW; ++w) b = wbest[w] > b ? wbest[w] : b;
      ax.keys[blockIdx.x] = b;
    }
  }
}

// The argmax over the head blocks' keys (one block of 1024 threads), then
// the token and the position advance.
__global__ __launch_bounds__(1024) void argmax_keys_kernel(
    const unsigned long long *__restrict__ keys, int n, int32_t *__restrict__ out,
    int32_t *__restrict__ pos, int max_seq) {
  __shared__ unsigned long long wbest[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  unsigned long long b = 0ull;
  for (int i = tid; i < n; i += 1024) b = keys[i] > b ? keys[i] : b;
  b = wave_max_u64(b);
  if (lane == 0) wbest[wave] = b;
  __syncthreads();
  if (tid == 0) {
    unsigned long long m = wbest[0];
#pragma unroll
    for (int w = 1; w < 16; ++w) m = wbest[w] > m ? wbest[w] : m;
    *out = (int32_t)(~(uint32_t)(m & 0xFFFFFFFFull));
    if (pos) {
      const int p = *pos + 1;
      *pos = p < max_seq ? p : max_seq;
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

// Measurement form (WST_GEMV_EXACT=1, plain GEMV only): the same row formula
// with the activations as f16 values, not the 14-bit table: per group
// Q = sum q_i x_i and S = sum x_i in f32 (each product exact), one wave per
// row, lanes over groups l, l + 64, ..., then the wave sum. It exists to
// measure what the table's rounding costs end to end; it is not fast.
__global__ __launch_bounds__(256) void gemv_hier_exact_kernel(
    const uint4 *__restrict__ qw, const uint8_t *__restrict__ si,
    const uint32_t *__restrict__ sb, const uint16_t *__restrict__ x,
    const uint16_t *__restrict__ bias, float *__restrict__ y, int in_f, int out_f, int accum) {
  const int lane = threadIdx.x & 63, G = in_f / HGROUP;
  for (int row = blockIdx.x * 4 + (threadIdx.x >> 6); row < out_f; row += gridDim.x * 4) {
    float as = 0.0f, am = 0.0f;
    for (int g = lane; g < G; g += 64) {
      const size_t at = (size_t)row * G + g;
      const uint4 p = qw[at];
      const uint32_t w[4] = {p.x, p.y, p.z, p.w};
      float q = 0.0f, sx = 0.0f;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const float xv = h2f(x[(size_t)g * HGROUP + i]);
        q = fmaf((float)((w[i / 8] >> (4 * (i % 8))) & 0xFu), xv, q);
        sx += xv;
      }
      const uint32_t id = si[at];
      as = fmaf((float)(id & 0xFu), q, as);
      am = fmaf((float)(id >> 4), sx, am);
    }
    const uint32_t sv = sb[row];
    float v = wave_sum(h2f((uint16_t)(sv & 0xFFFFu)) * as - h2f((uint16_t)(sv >> 16)) * am);
    if (lane == 0) {
      if (bias) v += h2f(bias[row]);
      y[row] = accum ? y[row] + v : v;
    }
  }
}

static bool gemv_exact() {
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("WST_GEMV_EXACT");
    v = e && e[0] == '1';
  }
  return v == 1;
}

// ---------------------------------------------------------------- dispatch

// The (wide, huge, other) rule of the reference (gemv_hier.cu:253-272) picks
// rows per thread tile there. This kernel's mapping depends only on in_f, so
// the rule is kept (and reported) for API compatibility but selects nothing:
// every rule gives the same bits, as the reference requires of its rules.
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

// Upper bound on resident blocks per CU used to size the persistent grid.
// WST_GEMV_BLOCKS_PER_CU overrides it (for sweeps).
static int blocks_per_cu() {
  static int v = 0;
  if (v == 0) {
    const char *e = getenv("WST_GEMV_BLOCKS_PER_CU");
    v = e ? atoi(e) : 0;
    if (v <= 0 || v > 64) v = 2;
  }
  return v;
}

// The grid: every resident block, units dealt round-robin (slot counts
// differ by at most one). WST_GEMV_GRID=balanced gives instead just enough
// blocks that every slot gets the same count, which leaves CUs with one block
// where others have two (7B: qkv 288 blocks, gate|up 474 on 256 CUs).
// Measured on the 7B step: qkv 6.0 -> 5.1 us, gate|up 15.5 -> 15.3 us,
// 778 -> 793 tok/s; the 0.5B step is unchanged. A row's bits do not depend
// on the grid.
static bool gemv_full_grid() {
  const char *e = getenv("WST_GEMV_GRID");
  return !(e && e[0] == 'b');
}

struct HierArgs {
  const void *qw, *si, *sb, *x;  // x: the partials for the AM form
  const void *norm_w;
  float eps;
  void *h_out;
  const void *bias;
  void *y;
  int in_f, nunits, accum;
  AttnIn am;
  ArgmaxOut ax;
  uint32_t *tw;  // TW: the output's table
};

// Units in flight per row slot. Measured on the 7B shapes: a second buffer
// helps only when a slot streams many units (the head, ~37 per slot); for the
// block GEMVs (1 to 5 units per slot) the extra up-front loads cost more than
// they hide (7B step 790 -> 738 tok/s with two everywhere). A row's bits do
// not depend on this. WST_GEMV_PD=1..4 forces one choice.
static int gemv_pd_override() {
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("WST_GEMV_PD");
    v = e ? atoi(e) : 0;
  }
  return v;
}

template <int NG, int WPR, int XB, int NT, bool NORM, bool SWIGLU, int PD, int RPW, int AM,
          bool AX, bool XT, bool TW>
static int launch_pd(const HierArgs &a) {
  auto kern = gemv_hier_kernel<NG, WPR, XB, NT, NORM, SWIGLU, PD, RPW, AM, AX, XT, TW>;
  size_t lds = (size_t)(a.in_f / HGROUP) * XQ_WORDS * 4;
  if (XT && lds < (size_t)XT_CHUNKS(XB) * NT * 16) lds = (size_t)XT_CHUNKS(XB) * NT * 16;
  // Resident blocks per CU for this instance and LDS size, queried once.
  static thread_local size_t q_lds = (size_t)-1;
  static thread_local int q_res = 1;
  if (lds != q_lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, NT, lds) != hipSuccess || n <= 0)
      n = 1;
    q_res = n < blocks_per_cu() ? n : blocks_per_cu();
    q_lds = lds;
  }
  // Persistent grid: at most k units per row slot.
  // Rows a block takes at a time (TW: whole groups of 32).
  constexpr int RPB = NT / 64 / WPR * RPW;
  constexpr int PER = TW && RPB < 32 ? 32 : RPB;
  const int cap = wst_cu_count() * q_res * PER;
  const int k = (a.nunits + cap - 1) / cap;
  int grid = (a.nunits + k * PER - 1) / (k * PER);
  if (gemv_full_grid()) {  // every resident slot, counts differing by at most one
    const int full = wst_cu_count() * q_res, need = (a.nunits + PER - 1) / PER;
    grid = full < need ? full : need;
  }
  // AX: one key slot per block (the grid is persistent: fewer blocks cover
  // every unit)
  if (AX && grid > AX_MAX_BLOCKS) grid = AX_MAX_BLOCKS;
  kern<<<grid, NT, lds, WST_STREAM>>>(
      (const uint4 *)a.qw, (const uint8_t *)a.si, (const uint32_t *)a.sb, a.x,
      (const uint16_t *)a.norm_w, a.eps, (uint16_t *)a.h_out, (const uint16_t *)a.bias, a.y,
      a.in_f, a.nunits, a.accum, a.am, a.ax, a.tw);
  return grid;
}

template <int NG, int WPR, int XB, int NT, bool NORM, bool SWIGLU, int RPW = 1, int AM = 0,
          bool AX = false, bool XT = false, bool TW = false>
static int launch_q(const HierArgs &a) {
  if constexpr (TW) {  // the table epilogue runs with one unit in flight
    return launch_pd<NG, WPR, XB, NT, NORM, SWIGLU, 1, RPW, AM, AX, XT, TW>(a);
  } else {
    int pd = gemv_pd_override();
    if (pd < 1 || pd > 4) {
      const int slots = wst_cu_count() * blocks_per_cu() * (NT / 64 / WPR * RPW);
      pd = a.nunits >= 8 * slots ? 2 : 1;
    }
    if (pd == 1) return launch_pd<NG, WPR, XB, NT, NORM, SWIGLU, 1, RPW, AM, AX, XT, TW>(a);
    if (pd == 3) return launch_pd<NG, WPR, XB, NT, NORM, SWIGLU, 3, RPW, AM, AX, XT, TW>(a);
    if (pd == 4) return launch_pd<NG, WPR, XB, NT, NORM, SWIGLU, 4, RPW, AM, AX, XT, TW>(a);
    return launch_pd<NG, WPR, XB, NT, NORM, SWIGLU, 2, RPW, AM, AX, XT, TW>(a);
  }
}

static int gemv_rpw_override() {
  const char *e = getenv("WST_GEMV_RPW");
  return e ? atoi(e) : 0;
}

// in_f -> (groups per lane, waves per row, activation blocks per thread,
// threads). NORM forms use 512 threads (their RMS order); plain forms with
// long rows use 1024 so a CU builds its table once.
#define GEMV_MAX_G 1280  // groups per row handled by the table kernel

template <bool NORM, bool SWIGLU, int AM = 0, bool AX = false, bool XT = false,
          bool TW = false>
// Returns the grid launched, 0 when in_f is outside the table kernel.
static int hier_dispatch(const HierArgs &a) {
  const int G = a.in_f / HGROUP;
  // Rows of at most 32 groups (in_f <= 1024, e.g. the 0.5B hidden 896) share a
  // wave: with one row per wave, 28 groups left 36 of 64 lanes idle and a
  // wave streamed 448 bytes per unit. Measured on the 0.5B lm_head (151936 x
  // 896, weights cold): 28.0 us one row per wave, 18.0 two, 15.4-16.0 four,
  // 15.1-15.4 eight (four groups per lane); but eight per wave slows the
  // latency-bound block GEMVs of that model (config-2 decode 1559 -> 1435
  // tok/s), so four is the default for every shape (a row's bits must not
  // depend on the output count). WST_GEMV_RPW=1|2|8 selects the others.
  const int rpw = gemv_rpw_override();
  if (G <= 16 && rpw != 1) return launch_q<1, 1, 1, 512, NORM, SWIGLU, 4, AM, AX, XT, TW>(a);
  else if (G <= 32 && rpw == 2) return launch_q<1, 1, 1, 512, NORM, SWIGLU, 2, AM, AX, XT, TW>(a);
  else if (G <= 32 && rpw == 8) return launch_q<4, 1, 1, 512, NORM, SWIGLU, 8, AM, AX, XT, TW>(a);
  else if (G <= 32 && rpw != 1) return launch_q<2, 1, 1, 512, NORM, SWIGLU, 4, AM, AX, XT, TW>(a);
  else if (G <= 64) return launch_q<1, 1, 1, 512, NORM, SWIGLU, 1, AM, AX, XT, TW>(a);
  else if (G <= 128) return launch_q<2, 1, 1, 512, NORM, SWIGLU, 1, AM, AX, XT, TW>(a);
  else if (G <= 192) return launch_q<3, 1, 2, 512, NORM, SWIGLU, 1, AM, AX, XT, TW>(a);
  else if (G <= 256) return launch_q<4, 1, 2, 512, NORM, SWIGLU, 1, AM, AX, XT, TW>(a);
  else if constexpr (NORM) {
    if (G <= 512) return launch_q<4, 2, 4, 512, NORM, SWIGLU, 1, AM, AX, XT, TW>(a);
    else return 0;
  } else {
    if (G <= 640) return launch_q<5, 2, 3, 1024, NORM, SWIGLU, 1, AM, AX, XT, TW>(a);
    else if (G <= GEMV_MAX_G) return launch_q<5, 4, 5, 1024, NORM, SWIGLU, 1, AM, AX, XT, TW>(a);
    else return 0;
  }
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
  const HierArgs a{qw, si, sb, x, nullptr, 0.0f, nullptr, bias, y, in_f, out_f, accum, {}, {}};
  if (gemv_exact()) {
    const int blocks = (out_f + 3) / 4, cap = wst_cu_count() * 8;
    gemv_hier_exact_kernel<<<blocks < cap ? blocks : cap, 256, 0, WST_STREAM>>>(
        (const uint4 *)qw, (const uint8_t *)si, (const uint32_t *)sb, (const uint16_t *)x,
        (const uint16_t *)bias, (float *)y, in_f, out_f, accum);
  } else if (!hier_dispatch<false, false>(a)) {
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
  WST_REQUIRE(in_f / HGROUP <= 512, "wst_gemv_hier_rmsnorm: in_features above 16384");
  WST_REQUIRE(!(((uintptr_t)norm_w | (uintptr_t)h_out) & 15u),
              "wst_gemv_hier_rmsnorm: norm weight and h must be 16-byte aligned");
  const HierArgs a{qw, si, sb, x, norm_w, eps, h_out, bias, y, in_f, out_f, accum, {}, {}};
  hier_dispatch<true, false>(a);
  WST_TRY_KERNEL("wst_gemv_hier_rmsnorm");
  return WST_OK;
}

extern "C" wst_status_t wst_gemv_hier_swiglu(const void *qw, const void *si, const void *sb,
                                             const void *x, const void *norm_w, float eps,
                                             void *out, int32_t in_f, int32_t inter) {
  const wst_status_t st = check_common(qw, si, sb, x, out, in_f, inter, "wst_gemv_hier_swiglu");
  if (st != WST_OK) return st;
  WST_REQUIRE(in_f / HGROUP <= (norm_w ? 512 : GEMV_MAX_G),
              "wst_gemv_hier_swiglu: in_features above 16384 (40960 without the norm)");
  WST_REQUIRE(!((uintptr_t)norm_w & 15u), "wst_gemv_hier_swiglu: norm weight must be 16-byte aligned");
  const HierArgs a{qw, si, sb, x, norm_w, eps, nullptr, nullptr, out, in_f, inter, 0, {}, {}};
  if (norm_w) hier_dispatch<true, true>(a);
  else hier_dispatch<false, true>(a);
  WST_TRY_KERNEL("wst_gemv_hier_swiglu");
  return WST_OK;
}

// The activation table of an f16 vector as the GEMV prologue builds it
// (hier_xq.hpp): G = in_f / 32 entries of XQ_WORDS words. One thread per 8
// columns; the four of a group are a quad.
__global__ __launch_bounds__(256) void xq_table_kernel(const uint16_t *__restrict__ x,
                                                       uint32_t *__restrict__ table, int nb8) {
  const int b = blockIdx.x * 256 + threadIdx.x;
  const bool valid = b < nb8;
  const uint4 v = *(const uint4 *)(x + (size_t)min(b, nb8 - 1) * 8);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint16_t h[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    h[2 * k] = (uint16_t)(w[k] & 0xFFFFu);
    h[2 * k + 1] = (uint16_t)(w[k] >> 16);
  }
  build_xq(h, b, valid, table);
}

extern "C" wst_status_t wst_hier_xq_table(const void *x, void *table, int32_t in_f) {
  WST_REQUIRE(x && table, "wst_hier_xq_table: null pointer");
  WST_REQUIRE(in_f > 0 && in_f % HGROUP == 0, "wst_hier_xq_table: in_features must be a positive multiple of 32");
  WST_REQUIRE(!(((uintptr_t)x | (uintptr_t)table) & 15u), "wst_hier_xq_table: x and table must be 16-byte aligned");
  const int nb8 = in_f / 8;
  xq_table_kernel<<<(nb8 + 255) / 256, 256, 0, WST_STREAM>>>((const uint16_t *)x, (uint32_t *)table, nb8);
  WST_TRY_KERNEL("wst_hier_xq_table");
  return WST_OK;
}

// wst_gemv_int4_hier_ex with the activation table already built (by
// wst_hier_xq_table or a producer's epilogue) in place of x: the same bits.
extern "C" wst_status_t wst_gemv_hier_xq(const void *qw, const void *si, const void *sb,
                                         const void *table, const void *bias, void *y,
                                         int32_t in_f, int32_t out_f, int32_t accum) {
  const wst_status_t st = check_common(qw, si, sb, table, y, in_f, out_f, "wst_gemv_hier_xq");
  if (st != WST_OK) return st;
  const HierArgs a{qw, si, sb, table, nullptr, 0.0f, nullptr, bias, y, in_f, out_f, accum, {}, {}};
  if (!hier_dispatch<false, false, 0, false, true>(a)) {
    snprintf(wst_err_buf, sizeof(wst_err_buf), "wst_gemv_hier_xq: in_features above 40960");
    return WST_ERR_SHAPE;
  }
  WST_TRY_KERNEL("wst_gemv_hier_xq");
  return WST_OK;
}

// wst_gemv_hier_swiglu that also writes the activation table of its output
// (inter / 32 entries of XQ_WORDS words, as wst_hier_xq_table(out) writes
// them), so that the GEMV consuming it need not build the table. inter must
// be a multiple of 32.
extern "C" wst_status_t wst_gemv_hier_swiglu_xq(const void *qw, const void *si, const void *sb,
                                                const void *x, const void *norm_w, float eps,
                                                void *out, void *table, int32_t in_f,
                                                int32_t inter) {
  const wst_status_t st = check_common(qw, si, sb, x, out, in_f, inter, "wst_gemv_hier_swiglu_xq");
  if (st != WST_OK) return st;
  WST_REQUIRE(table, "wst_gemv_hier_swiglu_xq: null table");
  WST_REQUIRE(inter % HGROUP == 0, "wst_gemv_hier_swiglu_xq: intermediate size must be a multiple of 32");
  WST_REQUIRE(!((uintptr_t)table & 15u), "wst_gemv_hier_swiglu_xq: table must be 16-byte aligned");
  WST_REQUIRE(in_f / HGROUP <= (norm_w ? 512 : GEMV_MAX_G),
              "wst_gemv_hier_swiglu_xq: in_features above 16384 (40960 without the norm)");
  WST_REQUIRE(!((uintptr_t)norm_w & 15u), "wst_gemv_hier_swiglu_xq: norm weight must be 16-byte aligned");
  HierArgs a{qw, si, sb, x, norm_w, eps, nullptr, nullptr, out, in_f, inter, 0, {}, {}};
  a.tw = (uint32_t *)table;
  if (norm_w) hier_dispatch<true, true, 0, false, false, true>(a);
  else hier_dispatch<false, true, 0, false, false, true>(a);
  WST_TRY_KERNEL("wst_gemv_hier_swiglu_xq");
  return WST_OK;
}

// The attention slice merge fused into the GEMV that consumes it (the o
// projection): y (+)= W merge(partials), bit-identical to attn_merge_kernel
// followed by wst_gemv_int4_hier_ex. For caches of at most AM_MAX_SLICES
// slices (max_seq <= 8 * 16384 / head_dim, where the slices are 16384 /
// head_dim positions long).
extern "C" wst_status_t wst_gemv_hier_attn(const void *qw, const void *si, const void *sb,
                                           const void *partials, void *y, int32_t n_q,
                                           int32_t head_dim, const void *pos, int32_t max_seq,
                                           int32_t out_f, int32_t accum) {
  const int32_t in_f = n_q * head_dim;
  const wst_status_t st = check_common(qw, si, sb, partials, y, in_f, out_f, "wst_gemv_hier_attn");
  if (st != WST_OK) return st;
  WST_REQUIRE(pos, "wst_gemv_hier_attn: null position");
  WST_REQUIRE(head_dim == 64 || head_dim == 128, "wst_gemv_hier_attn: head_dim must be 64 or 128");
  WST_REQUIRE(max_seq > 0, "wst_gemv_hier_attn: empty cache");
  const int P = wst_attn_slice_len(head_dim, max_seq);
  const int nsplit = (max_seq + P - 1) / P;
  WST_REQUIRE(nsplit <= AM_MAX_SLICES, "wst_gemv_hier_attn: more than 8 attention slices");
  HierArgs a{qw, si, sb, partials, nullptr, 0.0f, nullptr, nullptr, y, in_f, out_f, accum,
             {(const int32_t *)pos, nsplit, head_dim, n_q, max_seq, P}, {}};
  const bool ok = nsplit <= 4 ? hier_dispatch<false, false, 4>(a)
                              : hier_dispatch<false, false, AM_MAX_SLICES>(a);
  if (!ok) {
    snprintf(wst_err_buf, sizeof(wst_err_buf), "wst_gemv_hier_attn: in_features above 40960");
    return WST_ERR_SHAPE;
  }
  WST_TRY_KERNEL("wst_gemv_hier_attn");
  return WST_OK;
}

// The head of the decode step with its argmax: wst_gemv_hier_rmsnorm (accum
// 0, no bias) followed by wst_argmax_advance(y, out_idx, out_f, pos,
// max_seq) in one launch (pos may be null: no advance).
extern "C" wst_status_t wst_gemv_hier_rmsnorm_argmax(const void *qw, const void *si,
                                                     const void *sb, const void *x,
                                                     const void *norm_w, float eps, void *h_out,
                                                     void *y, int32_t in_f, int32_t out_f,
                                                     void *out_idx, void *pos, int32_t max_seq) {
  const wst_status_t st =
      check_common(qw, si, sb, x, y, in_f, out_f, "wst_gemv_hier_rmsnorm_argmax");
  if (st != WST_OK) return st;
  WST_REQUIRE(norm_w && out_idx, "wst_gemv_hier_rmsnorm_argmax: null pointer");
  WST_REQUIRE(!pos || max_seq > 0, "wst_gemv_hier_rmsnorm_argmax: bad max_seq");
  WST_REQUIRE(in_f / HGROUP <= 512, "wst_gemv_hier_rmsnorm_argmax: in_features above 16384");
  WST_REQUIRE(!(((uintptr_t)norm_w | (uintptr_t)h_out) & 15u),
              "wst_gemv_hier_rmsnorm_argmax: norm weight and h must be 16-byte aligned");
  unsigned long long *keys = (unsigned long long *)wst_static_scratch(
      WST_SCRATCH_HEADMAX, AX_MAX_BLOCKS * sizeof(unsigned long long));
  if (!keys) return WST_ERR_OOM;
  const HierArgs a{qw, si, sb, x, norm_w, eps, h_out, nullptr, y, in_f, out_f, 0, {},
                   {(int32_t *)out_idx, (int32_t *)pos, max_seq, keys}};
  const int nblocks = hier_dispatch<true, false, 0, true>(a);
  WST_REQUIRE(nblocks > 0 && nblocks <= AX_MAX_BLOCKS,
              "wst_gemv_hier_rmsnorm_argmax: grid outside the key slots");
  argmax_keys_kernel<<<1, 1024, 0, WST_STREAM>>>(keys, nblocks, (int32_t *)out_idx,
                                                 (int32_t *)pos, max_seq);
  WST_TRY_KERNEL("wst_gemv_hier_rmsnorm_argmax");
  return WST_OK;
}
