// Batch=1 GQA decode attention over the f16 KV cache.
// reference: crates/whetstone-kernels/cuda/attention.cu (split over the
// sequence, softmax per slice, associative merge of the slices).
//
// MI355X design
// -------------
// * One block per (kv head, slice of P cached positions), P*hd/32 threads, so
//   each thread stages four positions of one 16-byte chunk; P = 16384 / hd
//   (wst_attn_slice_len). Every K/V row is read from memory once and used for
//   all n_q/n_kv query heads of the group.
// * The block stages its slice in LDS with one batch of 16-byte loads (K as
//   rows of positions, V transposed: rows of dims) and computes both products
//   on MFMA (v_mfma_f32_16x16x32_f16, f32 accumulate):
//     scores  S[h][p] = q_h . k_p : rows the block's heads (padded to 16),
//             16 positions per tile;
//     softmax a wave per head: one max, one exp per (head, position), one sum;
//     P.V     O[h][d] = sum_p P[h][p] V[p][d] : 16 dims per tile.
//   q and P enter the MFMA as their f16 hi part plus the f16 rounding of the
//   rest, so the products keep ~22 bits; K and V are f16 already. The f32
//   FMA formulation of the same block spent ~4 us of a 7.8 us single-slice
//   launch on VALU; on MFMA the compute is a few hundred cycles.
// * Each slice writes its unnormalised numerators and (max, sum) to the
//   partials; a second kernel (one 256-thread block per head and 32 dims)
//   merges them: eight lanes per dim each merge every eighth slice, all loads
//   issued with the position load, then a fixed tree over the eight. Measured
//   against merging in the last block of each kv head to finish: that costs a
//   device-scope hand-off plus one CU pulling all of a kv head's partials,
//   about 4.7 us; the separate merge about 3.
// * The grid covers max_seq; only the ceil(seq/P) slices holding cached
//   positions do work, so a captured graph serves every position.
// * A slice is one tile of P positions by default. WST_ATTN_TILES makes it
//   several, looped with an online softmax (measured: with at most 8 slices
//   the o GEMV can merge them and the merge launch goes, but on the 7B cache
//   the tile loop and the larger merge in o cost more than the launch saves).
// * ROPE form (wst_attn_decode_fused): each block applies QK-norm and RoPE to
//   the q heads it needs exactly as wst_rope_cache does (same per-head
//   reduction, same fma shapes) while its K/V loads are in flight; the block
//   whose slice holds the current position appends that position's k and v to
//   the cache and puts them into its LDS tile. No other block reads that
//   position, so no cross-block wait is needed, and the result is
//   bit-identical to wst_rope_cache followed by wst_attn_decode.
// * Deterministic: every sum runs in a fixed order.
#include "common.hpp"
#include "hier_xq.hpp"

#include <stdlib.h>

#define ATTN_MAX_GQA 8
#define ATTN_MERGE_LANES 8   // lanes per dim in the merge (slices dealt round-robin)
#define ATTN_MERGE_BATCH 16  // slices each lane fetches per round trip

template <int HD, int P_>
struct AttnShape {
  static constexpr int P = P_;              // positions per block
  static constexpr int CH = HD / 8;         // 16-byte chunks per row
  static constexpr int T = P * HD / 32;     // threads: four positions of one chunk each
  static constexpr int NW = T / 64;         // waves
  // Row strides in halves, padded by 16 bytes so that the 16 rows an MFMA
  // operand read touches fall in different LDS banks.
  static constexpr int KS = HD + 8;  // K tile  [P][KS]      (rows: positions)
  static constexpr int VS = P + 8;   // V^T tile [HD][VS]    (rows: dims)
  static constexpr int QS = HD + 8;  // q hi/lo  [16][QS]    (rows: heads)
  static constexpr int PS = P + 8;   // p hi/lo  [16][PS]    (rows: heads)
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = K_OFF + P * KS * 2;
  static constexpr int QH_OFF = V_OFF + HD * VS * 2;
  static constexpr int QL_OFF = QH_OFF + 16 * QS * 2;
  static constexpr int S_OFF = QL_OFF + 16 * QS * 2;   // scores [16][P] f32
  static constexpr int PH_OFF = S_OFF + 16 * P * 4;
  static constexpr int PL_OFF = PH_OFF + 16 * PS * 2;
  static constexpr int ML_OFF = PL_OFF + 16 * PS * 2;  // per head (m, l, rescale)
  static constexpr int LDS = ML_OFF + 16 * 3 * 4;
  static_assert(P % 32 == 0 && HD % 32 == 0, "MFMA tiles");
};

// Query-head groups per kv head (grid z): the heads of a kv head are split over
// this many blocks per slice, each staging the same K/V tile, so that a slice's
// score and P.V work is spread over more CUs. Every head's arithmetic is the
// same in any group. Default: one group, or one block per head when the grid
// would have fewer than 64 blocks (0.5B: 2 kv heads x 4 slices, attention 4.85
// -> 4.2 us; x 17 slices at a 4.3k cache, decode 1,440 -> 1,482 tok/s; on the
// 7B grid of 76 blocks two or more groups measured equal or slower).
// WST_ATTN_HEAD_GROUPS overrides.
static int attn_head_groups(int gqa, int blocks) {
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("WST_ATTN_HEAD_GROUPS");
    v = e ? atoi(e) : 0;
  }
  int z = v > 0 ? v : (blocks < 64 ? gqa : 1);
  z = z < gqa ? z : gqa;
  const int hpz = (gqa + z - 1) / z;  // heads per group; every group gets >= 1
  return (gqa + hpz - 1) / hpz;
}

// Tiles are 16384 / hd positions (128 at hd 128): measured on the 7B shape
// at 2k context (4 kv heads), 32- and 64-position tiles launch 4-2x the
// blocks but run slower (slice kernel 6.8 us at 32 against 5.6 us at 128;
// step 754 / 779 / 774 tok/s at 32 / 64 / 128), since every block pays the
// same chain of dependent phases. WST_ATTN_SLICE=<positions> (32, 64, 128 or
// 256, within 16384 / hd and at least 64 threads) overrides, for measurement.
static int attn_tile_len(int hd) {
  static int forced = -1;
  if (forced < 0) {
    const char *e = getenv("WST_ATTN_SLICE");
    forced = e ? atoi(e) : 0;
  }
  const int pmax = 16384 / hd;
  if (forced == 32 || forced == 64 || forced == 128 || forced == 256)
    if (forced <= pmax && forced * hd >= 2048) return forced;
  return pmax;
}

// Tiles per slice (1 to 4, the default tile length only). WST_ATTN_TILES=n
// forces n; WST_ATTN_TILES=auto takes the fewest that leave at most 8 slices
// (AM_MAX_SLICES: the o GEMV can then merge them itself).
static int attn_tiles(int hd, int max_seq) {
  static int forced = -1;
  if (forced < 0) {
    const char *e = getenv("WST_ATTN_TILES");
    forced = !e ? 1 : (e[0] == 'a' ? 0 : atoi(e));
    if (forced < 0 || forced > 4) forced = 1;
  }
  const int P = attn_tile_len(hd);
  if (P != 16384 / hd || hd > 128) return 1;
  if (forced > 0) return forced;
  const int ntiles = (max_seq + P - 1) / P;
  const int t = (ntiles + 7) / 8;
  return t < 1 ? 1 : (t > 4 ? 4 : t);
}

// Positions per slice: the tile length times the tiles per slice.
int wst_attn_slice_len(int hd, int max_seq) {
  return attn_tile_len(hd) * attn_tiles(hd, max_seq);
}

static inline int attn_slices(int head_dim, int max_seq) {
  const int p = wst_attn_slice_len(head_dim, max_seq);
  return (max_seq + p - 1) / p;
}

struct RopeArgs {
  const float *cos_tab, *sin_tab;
  const uint16_t *q_norm_w, *k_norm_w;
  float eps;
};

__device__ __forceinline__ void unpack8(const uint4 v, float *f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = h2f((uint16_t)(w[i] & 0xFFFFu));
    f[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
  }
}

typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Eight halves (16 bytes) from LDS as an MFMA operand.
__device__ __forceinline__ h16x8 lds_h8(const uint16_t *p) {
  return __builtin_bit_cast(h16x8, *(const uint4 *)p);
}

// Column of position p in row d of the V^T tile: 8-position blocks are
// permuted by xor with d / 8, so that the 8-byte stores of a wave (16 or more
// chunks of 8 dims at once) spread over all LDS banks, while every aligned run
// of 8 positions an MFMA operand reads stays contiguous.
template <int P>
__device__ __forceinline__ int vt_col(int d, int p) {
  return (((p >> 3) ^ ((d >> 3) & (P / 8 - 1))) << 3) | (p & 7);
}

// q (already scaled) as its f16 hi part and the f16 rounding of the rest.
__device__ __forceinline__ void store_q(uint16_t *qh, uint16_t *ql, int at, float v) {
  const uint16_t h = f2h(v);
  qh[at] = h;
  ql[at] = f2h(v - h2f(h));
}

// NTL: tiles of P positions per slice. A slice of NTL * P positions is
// processed tile by tile with an online softmax: per head the running (m, l)
// live in LDS, the P.V accumulators in the MFMA result registers, each rescaled
// by exp(m_old - m_new) before the next tile's products are added; the next
// tile's K/V loads are issued as soon as the current one is in LDS. With
// NTL = 1 the arithmetic is that of a single tile (the rescale of a zero
// accumulator by zero adds nothing).
template <int HD, int P_, bool ROPE, int NTL>
__global__ __launch_bounds__(P_ * HD / 32) void attn_decode_kernel(
    const float *__restrict__ qkv, uint16_t *__restrict__ k_cache,
    uint16_t *__restrict__ v_cache, float *__restrict__ partials, int n_q, int n_kv,
    const int32_t *__restrict__ pos_dev, int max_seq, float scale, RopeArgs ra) {
  using S = AttnShape<HD, P_>;
  constexpr int P = S::P, CH = S::CH, T = S::T, NW = S::NW;
  constexpr int SP = P * NTL;  // positions per slice
  constexpr int ND = (HD / 16 + NW - 1) / NW;  // 16-dim output tiles per wave
  (void)CH;
  extern __shared__ __align__(16) unsigned char lds[];
  uint16_t *ktile = (uint16_t *)(lds + S::K_OFF);
  uint16_t *vtile = (uint16_t *)(lds + S::V_OFF);
  uint16_t *qh = (uint16_t *)(lds + S::QH_OFF);
  uint16_t *ql = (uint16_t *)(lds + S::QL_OFF);
  float *sc = (float *)(lds + S::S_OFF);
  uint16_t *ph = (uint16_t *)(lds + S::PH_OFF);
  uint16_t *pl = (uint16_t *)(lds + S::PL_OFF);
  float *ml = (float *)(lds + S::ML_OFF);  // per head: m, l, and the tile's rescale

  const int gqa = n_q / n_kv;
  const int kvh = blockIdx.x, split = blockIdx.y, nsplit = gridDim.y;
  // This block's query heads: group blockIdx.z of the kv head's gqa heads.
  const int hpz = (gqa + gridDim.z - 1) / gridDim.z;
  const int h0 = blockIdx.z * hpz;
  const int hb = min(hpz, gqa - h0);  // >= 1: the launch keeps gridDim.z <= gqa
  const int qh0 = kvh * gqa + h0;     // first global query head
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  const int pos = min(max(*pos_dev, 0), max_seq - 1);
  const int seq = min(max(*pos_dev, 0) + 1, max_seq);
  const int nactive = (seq + SP - 1) / SP;
  if (split >= nactive) return;  // no cached positions here (uniform per block)
  const int t0 = split * SP, tend = min(t0 + SP, seq);

  const uint16_t *kb = k_cache + (size_t)kvh * max_seq * HD;
  const uint16_t *vb = v_cache + (size_t)kvh * max_seq * HD;

  // ---- phase A: the first tile's K and V requests go out first, all at once.
  // Thread t holds 16-byte chunk ch = t % CH (dims 8ch..8ch+7) of the four
  // consecutive positions 4 (t / CH) + i of a tile.
  constexpr int LD = P * CH / T;
  static_assert(LD == 4, "four positions per thread");
  const int lch = tid % CH, lrow = 4 * (tid / CH);
  uint4 kr[LD], vr[LD];
  auto load_tile = [&](int tt0) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int t = min(tt0 + lrow + i, seq - 1);  // clamped: unconditional loads stay batched
      kr[i] = *(const uint4 *)(kb + (size_t)t * HD + lch * 8);
      vr[i] = *(const uint4 *)(vb + (size_t)t * HD + lch * 8);
    }
  };
  load_tile(t0);

  // q for the group's heads, pre-scaled (attention.cu:98-101), into LDS.
  const bool owner = ROPE && pos >= t0 && pos < tend;  // the slice holds `pos`
  uint16_t knew = 0, vnew = 0, knew2 = 0, vnew2 = 0;  // owner: this position's k, v
  if constexpr (ROPE) {
    // One wave per head, as wst_rope_cache runs one 64-thread block per head
    // (hd <= 128): lane j owns elements j and j + hd/2.
    constexpr int HALF = HD / 2;
    const int j = lane;
    const bool active = j < HALF;
    const float c = active ? ra.cos_tab[(size_t)pos * HALF + j] : 0.0f;
    const float s = active ? ra.sin_tab[(size_t)pos * HALF + j] : 0.0f;
    for (int h = wave; h < hb + 1; h += NW) {
      const bool is_k = h == hb;
      if (is_k && !owner) continue;
      const float *src = is_k ? qkv + (size_t)(n_q + kvh) * HD : qkv + (size_t)(qh0 + h) * HD;
      float x1 = active ? src[j] : 0.0f;
      float x2 = active ? src[j + HALF] : 0.0f;
      const uint16_t *g = is_k ? ra.k_norm_w : ra.q_norm_w;
      if (g) {
        // Single-wave form of qk_norm: for one wave block_sum == 0 + wave_sum.
        const float a = active ? fmaf(x1, x1, x2 * x2) : 0.0f;
        const float ss = 0.0f + wave_sum(a);
        const float sc_ = 1.0f / sqrtf(ss / (float)HD + ra.eps);
        if (active) {
          x1 = x1 * sc_ * h2f(g[j]);
          x2 = x2 * sc_ * h2f(g[j + HALF]);
        }
      }
      if (!active) continue;
      const float lo = rope_lo(x1, x2, c, s), hi = rope_hi(x1, x2, c, s);
      if (!is_k) {
        store_q(qh, ql, h * S::QS + j, lo * scale);
        store_q(qh, ql, h * S::QS + j + HALF, hi * scale);
      } else {
        const float *vh = qkv + (size_t)(n_q + n_kv + kvh) * HD;
        knew = f2h(lo);
        knew2 = f2h(hi);
        vnew = f2h(vh[j]);
        vnew2 = f2h(vh[j + HALF]);
        if (blockIdx.z == 0) {  // every head group forms the row; one appends it
          const size_t slot = ((size_t)kvh * max_seq + pos) * HD;
          k_cache[slot + j] = knew;
          k_cache[slot + j + HALF] = knew2;
          v_cache[slot + j] = vnew;
          v_cache[slot + j + HALF] = vnew2;
        }
      }
    }
  } else {
    // At most 8 * HD values: unconditional (clamped) loads, so they share one
    // round trip.
    constexpr int QL = (ATTN_MAX_GQA * HD + T - 1) / T;
    const int nqv = hb * HD;
    float qv[QL];
#pragma unroll
    for (int i = 0; i < QL; ++i) qv[i] = qkv[(size_t)qh0 * HD + min(tid + i * T, nqv - 1)];
#pragma unroll
    for (int i = 0; i < QL; ++i) {
      const int e = tid + i * T;
      if (e < nqv) store_q(qh, ql, (e / HD) * S::QS + e % HD, qv[i] * scale);
    }
  }
  if (tid < hb) {
    ml[tid * 3] = -INFINITY;
    ml[tid * 3 + 1] = 0.0f;
  }

  f32x4 oc[ND];
#pragma unroll
  for (int n = 0; n < ND; ++n) oc[n] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  for (int jt = 0; jt < NTL; ++jt) {
    const int tt0 = t0 + jt * P;
    if (tt0 >= tend) break;  // uniform
    const int tt1 = min(tt0 + P, tend);
    if (jt > 0) __syncthreads();  // every wave is done with the previous tile's LDS

    // Tiles into LDS; rows past the cached positions are zero (their scores
    // are masked, and a zero V row keeps 0 * v finite).
    uint32_t vw[LD][4];
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const uint32_t mk = tt0 + lrow + i < tt1 ? 0xFFFFFFFFu : 0u;  // a mask, not a select of
      const uint4 a = kr[i], b = vr[i];                               // addresses (which spills)
      *(uint4 *)(ktile + (lrow + i) * S::KS + lch * 8) =
          make_uint4(a.x & mk, a.y & mk, a.z & mk, a.w & mk);
      vw[i][0] = b.x & mk;
      vw[i][1] = b.y & mk;
      vw[i][2] = b.z & mk;
      vw[i][3] = b.w & mk;
    }
    // V^T: dim d's four positions as one 8-byte store (halves picked by byte
    // permutes), at the swizzled column of vt_col.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int odd = 0; odd < 2; ++odd) {
        const uint32_t sel = odd ? 0x07060302u : 0x05040100u;
        const uint32_t lo = __builtin_amdgcn_perm(vw[1][e], vw[0][e], sel);
        const uint32_t hi = __builtin_amdgcn_perm(vw[3][e], vw[2][e], sel);
        const int d = lch * 8 + 2 * e + odd;
        *(uint2 *)(vtile + d * S::VS + vt_col<P>(d, lrow)) = make_uint2(lo, hi);
      }
    }
    // the next tile's loads go out now (the registers are consumed)
    if (NTL > 1 && jt + 1 < NTL && tt0 + P < tend) load_tile(tt0 + P);
    if constexpr (ROPE) {
      const bool here = owner && pos >= tt0 && pos < tt1;  // uniform
      if (here) {
        __syncthreads();  // the tile row of `pos` holds the cache's old contents
        if (wave == hb % NW && lane < HD / 2) {
          const int row = pos - tt0;
          ktile[row * S::KS + lane] = knew;
          ktile[row * S::KS + lane + HD / 2] = knew2;
          vtile[lane * S::VS + vt_col<P>(lane, row)] = vnew;
          vtile[(lane + HD / 2) * S::VS + vt_col<P>(lane + HD / 2, row)] = vnew2;
        }
      }
    }
    __syncthreads();

    // ---- phase B: scores S[h][p] = q_h . k_p on MFMA (16x16x32 f16, f32
    // accumulate): rows are the block's heads (up to 16; rows past hb carry
    // whatever the LDS held and are never read back), columns 16 positions per
    // tile, q as its f16 hi and lo parts so the products keep ~22 bits of q.
    {
      const int r16 = lane & 15, kq = (lane >> 4) * 8;
      for (int nt = wave; nt < P / 16; nt += NW) {
        f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < HD; kk += 32) {
          const h16x8 b = lds_h8(ktile + (nt * 16 + r16) * S::KS + kk + kq);
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(lds_h8(qh + r16 * S::QS + kk + kq), b, c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(lds_h8(ql + r16 * S::QS + kk + kq), b, c, 0, 0, 0);
        }
        const int p = nt * 16 + r16;
        const bool valid = tt0 + p < tt1;
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[((lane >> 4) * 4 + i) * P + p] = valid ? c[i] : -INFINITY;
      }
    }
    __syncthreads();

    // ---- phase C: softmax over the tile, a wave per head, against the
    // running maximum; the weights go to LDS as f16 hi and lo parts for the
    // P.V MFMAs, and the running (m, l) and the accumulators' rescale to ml.
    for (int hh = wave; hh < hb; hh += NW) {
      constexpr int R = (P + 63) / 64;
      float v[R];
      float m = -INFINITY;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int p = lane + 64 * r;
        v[r] = p < P ? sc[hh * P + p] : -INFINITY;
        m = fmaxf(m, v[r]);
      }
      m = wave_max(m);  // finite: every tile processed holds a cached position
      const float m_old = ml[hh * 3];
      const float mn = fmaxf(m_old, m);
      const float corr = (m_old == -INFINITY) ? 0.0f : __expf(m_old - mn);
      float l = 0.0f;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int p = lane + 64 * r;
        const float e = (v[r] == -INFINITY) ? 0.0f : __expf(v[r] - mn);
        const uint16_t eh = f2h(e);
        if (p < P) {
          ph[hh * S::PS + p] = eh;
          pl[hh * S::PS + p] = f2h(e - h2f(eh));
        }
        l += e;
      }
      l = wave_sum(l);
      if (lane == 0) {
        ml[hh * 3] = mn;
        ml[hh * 3 + 1] = ml[hh * 3 + 1] * corr + l;
        ml[hh * 3 + 2] = corr;
      }
    }
    __syncthreads();

    // ---- phase D: O[h][d] = corr_h O[h][d] + sum_p P[h][p] V[p][d] on MFMA
    // (V^T rows are dims).
    {
      const int r16 = lane & 15, kq = (lane >> 4) * 8;
#pragma unroll
      for (int n = 0; n < ND; ++n) {
        const int nd = wave + n * NW;
        if (nd >= HD / 16) break;
        const int d = nd * 16 + r16;
        f32x4 c = oc[n];
        if (NTL > 1) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int h = (lane >> 4) * 4 + i;
            c[i] *= h < hb ? ml[h * 3 + 2] : 0.0f;
          }
        }
#pragma unroll 4
        for (int kk = 0; kk < P; kk += 32) {
          const h16x8 b = lds_h8(vtile + d * S::VS + vt_col<P>(d, kk + kq));
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(lds_h8(ph + r16 * S::PS + kk + kq), b, c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(lds_h8(pl + r16 * S::PS + kk + kq), b, c, 0, 0, 0);
        }
        oc[n] = c;
      }
    }
  }

  // This slice's result straight from the accumulators.
  float *pacc = partials;
  float *pml = partials + (size_t)n_q * nsplit * HD;
  {
    const int r16 = lane & 15;
#pragma unroll
    for (int n = 0; n < ND; ++n) {
      const int nd = wave + n * NW;
      if (nd >= HD / 16) break;
      const int d = nd * 16 + r16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = (lane >> 4) * 4 + i;
        if (h >= hb) continue;
        const size_t row = (size_t)(qh0 + h) * nsplit + split;
        pacc[row * HD + d] = oc[n][i];
        if (d == 0) {
          pml[row * 2] = ml[h * 3];
          pml[row * 2 + 1] = ml[h * 3 + 1];
        }
      }
    }
  }
}

// ---------------------------------------------------------------- slice merge
//
// out[h][d] = sum_s e^(m_s - M) acc_s[d] / sum_s e^(m_s - M) l_s with M the
// largest slice maximum (attention.cu:170-193). One block of 32*NL threads per
// (head, 32 dims); lane group j = tid / 32 (of NL: 2 up to 32 slices, 8
// beyond) merges slices j, j + NL, j + 2 NL, ... of dim d = tid % 32 in
// ascending order, then the groups are combined by a fixed tree (j with
// j + NL/2, then + NL/4, ...).
// When the cache has at most 8 slices (SPREAD false), group 0 takes them all,
// in slice order: the arithmetic of the merge inside the o GEMV (merge8 in
// gemv_hier.hip), so both forms give the same bits.
// A group's first B slices are loaded together with the position (slice
// indices clamped to the partials' extent), and slices past the cached ones
// are replaced afterwards: up to 128 slices cost one memory round trip per
// B NL slices. With NL = 2, B is the smallest of 4, 8, 12, 16 that holds a
// group's slices in one batch: fewer clamped loads, and the same bits as any
// larger single batch (a dead slice adds exactly nothing).
struct MergeState {
  float M, den, a;
};

__device__ __forceinline__ void merge_combine(MergeState &x, const MergeState &y) {
  if (y.M == -INFINITY) return;  // an empty partner adds nothing
  const float Mn = fmaxf(x.M, y.M);
  const float fo = (x.M == -INFINITY) ? 0.0f : __expf(x.M - Mn);
  const float ft = __expf(y.M - Mn);
  x.den = x.den * fo + y.den * ft;
  x.a = x.a * fo + y.a * ft;
  x.M = Mn;
}

template <int NL, bool SPREAD, int B = ATTN_MERGE_BATCH>
__global__ __launch_bounds__(32 * NL) void attn_merge_kernel(const float *__restrict__ partials,
                                                         uint16_t *__restrict__ out, int n_q,
                                                         int hd, int nsplit,
                                                         const int32_t *__restrict__ pos_dev,
                                                         int max_seq, int P,
                                                         uint32_t *__restrict__ tw) {
  __shared__ float hx[NL][32][3];
  __shared__ uint16_t mo[32];
  const int h = blockIdx.x, d0 = blockIdx.y * 32, tid = threadIdx.x;
  const int j = tid >> 5, d = d0 + (tid & 31);
  const float *pacc = partials;
  const float *pml = partials + (size_t)n_q * nsplit * hd;
  const size_t row0 = (size_t)h * nsplit;
  const int pos = *pos_dev;
  // SPREAD: group j owns slices j + NL*i; else group 0 owns slices i.
  const int first = SPREAD ? j : (j == 0 ? 0 : nsplit);
  const int stride = SPREAD ? NL : 1;
  MergeState st{-INFINITY, 0.0f, 0.0f};
  int nactive = 1;
  for (int c = first; c < nsplit; c += B * stride) {
    if (c != first && c >= nactive) break;  // nactive is known after the first batch
    float ms[B], ls[B], vs[B];
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const size_t r = row0 + min(c + i * stride, nsplit - 1);
      const float2 mlv = *(const float2 *)(pml + r * 2);
      ms[i] = mlv.x;
      ls[i] = mlv.y;
      vs[i] = pacc[r * hd + d];
    }
    const int seq = min(max(pos, 0) + 1, max_seq);
    nactive = (seq + P - 1) / P;
    // Slices past the cached positions hold stale partials: replaced, not
    // multiplied by zero, so nothing non-finite can enter.
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const bool live = c + i * stride < nactive;
      ms[i] = live ? ms[i] : -INFINITY;
      ls[i] = live ? ls[i] : 0.0f;
      vs[i] = live ? vs[i] : 0.0f;
    }
    float Mn = st.M;
#pragma unroll
    for (int i = 0; i < B; ++i) Mn = fmaxf(Mn, ms[i]);
    if (Mn != -INFINITY) {  // else nothing live in this batch for this group
      const float fo = (st.M == -INFINITY) ? 0.0f : __expf(st.M - Mn);
      st.a *= fo;
      st.den *= fo;
#pragma unroll
      for (int i = 0; i < B; ++i) {
        const float f = (ms[i] == -INFINITY) ? 0.0f : __expf(ms[i] - Mn);
        st.a = fmaf(vs[i], f, st.a);
        st.den = fmaf(ls[i], f, st.den);
      }
      st.M = Mn;
    }
  }
  hx[j][tid & 31][0] = st.M;
  hx[j][tid & 31][1] = st.den;
  hx[j][tid & 31][2] = st.a;
  __syncthreads();
#pragma unroll
  for (int w = NL / 2; w >= 1; w >>= 1) {
    if (j < w) {
      const MergeState o{hx[j + w][tid & 31][0], hx[j + w][tid & 31][1], hx[j + w][tid & 31][2]};
      merge_combine(st, o);
      hx[j][tid & 31][0] = st.M;
      hx[j][tid & 31][1] = st.den;
      hx[j][tid & 31][2] = st.a;
    }
    __syncthreads();
  }
  if (j == 0) {
    const uint16_t v = f2h(st.a / st.den);
    out[(size_t)h * hd + d] = v;
    mo[tid] = v;
  }
  if (tw) {  // the block's 32 outputs are one group of the consumer's table
    __syncthreads();
    if (tid < 4) {
      uint16_t hv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) hv[e] = mo[8 * tid + e];
      build_xq(hv, (h * hd + d0) / 8 + tid, true, tw);
    }
  }
}

template <int HD, int P, bool ROPE, int NTL = 1>
static void attn_go(const dim3 grid, const void *qkv, void *k_cache, void *v_cache,
                    void *partials, int n_q, int n_kv, const void *pos, int max_seq, float scale,
                    const RopeArgs &ra) {
  using S = AttnShape<HD, P>;
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void *)attn_decode_kernel<HD, P, ROPE, NTL>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, S::LDS);
    attr_set = true;
  }
  attn_decode_kernel<HD, P, ROPE, NTL><<<grid, S::T, S::LDS, WST_STREAM>>>(
      (const float *)qkv, (uint16_t *)k_cache, (uint16_t *)v_cache, (float *)partials, n_q,
      n_kv, (const int32_t *)pos, max_seq, scale, ra);
}

// The slice kernel, then the merge.
template <bool ROPE>
static void attn_launch(int head_dim, const void *qkv, void *k_cache, void *v_cache,
                        void *partials, void *out, int n_q, int n_kv, const void *pos,
                        int max_seq, float scale, const RopeArgs &ra, bool merge = true,
                        uint32_t *tw = nullptr) {
  const int PT = attn_tile_len(head_dim), NTL = attn_tiles(head_dim, max_seq);
  const int P = PT * NTL;  // positions per slice
  const int nsplit = (max_seq + P - 1) / P;
  const dim3 grid(n_kv, nsplit, attn_head_groups(n_q / n_kv, n_kv * nsplit));
#define ATTN_GO(hd_, p_) attn_go<hd_, p_, ROPE>(grid, qkv, k_cache, v_cache, partials, n_q, \
                                                n_kv, pos, max_seq, scale, ra)
#define ATTN_GO_T(hd_, p_, t_) attn_go<hd_, p_, ROPE, t_>(grid, qkv, k_cache, v_cache, partials, \
                                                          n_q, n_kv, pos, max_seq, scale, ra)
  switch (NTL > 1 ? -(head_dim * 10 + NTL) : head_dim * 1000 + PT) {
    case -(64 * 10 + 2): ATTN_GO_T(64, 256, 2); break;
    case -(64 * 10 + 3): ATTN_GO_T(64, 256, 3); break;
    case -(64 * 10 + 4): ATTN_GO_T(64, 256, 4); break;
    case -(128 * 10 + 2): ATTN_GO_T(128, 128, 2); break;
    case -(128 * 10 + 3): ATTN_GO_T(128, 128, 3); break;
    case -(128 * 10 + 4): ATTN_GO_T(128, 128, 4); break;
    case 64 * 1000 + 32: ATTN_GO(64, 32); break;
    case 64 * 1000 + 64: ATTN_GO(64, 64); break;
    case 64 * 1000 + 128: ATTN_GO(64, 128); break;
    case 64 * 1000 + 256: ATTN_GO(64, 256); break;
    case 128 * 1000 + 32: ATTN_GO(128, 32); break;
    case 128 * 1000 + 64: ATTN_GO(128, 64); break;
    case 128 * 1000 + 128: ATTN_GO(128, 128); break;
    default:
      if constexpr (!ROPE) {
        if (PT == 32) attn_go<256, 32, false>(grid, qkv, k_cache, v_cache, partials, n_q, n_kv,
                                             pos, max_seq, scale, ra);
        else attn_go<256, 64, false>(grid, qkv, k_cache, v_cache, partials, n_q, n_kv, pos,
                                     max_seq, scale, ra);
      }
      break;
  }
#undef ATTN_GO
#undef ATTN_GO_T
  if (merge) {
    const dim3 mg(n_q, head_dim / 32);
    const float *pa = (const float *)partials;
    const int32_t *pp = (const int32_t *)pos;
    uint16_t *o = (uint16_t *)out;
#define ATTN_MERGE(sp_, b_)                                                              \
  attn_merge_kernel<2, sp_, b_><<<mg, 64, 0, WST_STREAM>>>(pa, o, n_q, head_dim, nsplit, pp, \
                                                          max_seq, P, tw)
    if (nsplit <= 4) ATTN_MERGE(false, 4);
    else if (nsplit <= 8) ATTN_MERGE(false, 8);
    else if (nsplit <= 16) ATTN_MERGE(true, 8);
    else if (nsplit <= 24) ATTN_MERGE(true, 12);
    else if (nsplit <= 2 * ATTN_MERGE_BATCH) ATTN_MERGE(true, 16);
#undef ATTN_MERGE
    else
      attn_merge_kernel<ATTN_MERGE_LANES, true><<<mg, 32 * ATTN_MERGE_LANES, 0, WST_STREAM>>>(
          pa, o, n_q, head_dim, nsplit, pp, max_seq, P, tw);
  }
}

extern "C" int32_t wst_attn_slice_positions(int32_t head_dim, int32_t max_seq) {
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return 0;
  if (max_seq <= 0) return 0;
  return wst_attn_slice_len(head_dim, max_seq);
}

extern "C" int32_t wst_attn_partial_floats(int32_t n_q, int32_t head_dim, int32_t max_seq) {
  if (n_q <= 0 || head_dim <= 0 || max_seq <= 0) return 0;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return 0;
  return n_q * attn_slices(head_dim, max_seq) * (head_dim + 2);
}

static wst_status_t attn_check(const void *q, const void *k_cache, const void *v_cache,
                               const void *partials, const void *out, int32_t n_q, int32_t n_kv,
                               int32_t head_dim, const void *pos, int32_t max_seq) {
  WST_REQUIRE(q && k_cache && v_cache && out && pos && partials,
              "wst_attn_decode: null pointer");
  WST_REQUIRE(n_q > 0 && n_kv > 0 && head_dim > 0, "wst_attn_decode: non-positive shape");
  WST_REQUIRE(n_q % n_kv == 0,
              "wst_attn_decode: query heads must be a multiple of key/value heads");
  WST_REQUIRE(n_q / n_kv <= ATTN_MAX_GQA,
              "wst_attn_decode: more than 8 query heads per kv head");
  WST_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
              "wst_attn_decode: head_dim must be 64, 128 or 256");
  WST_REQUIRE(max_seq > 0, "wst_attn_decode: empty cache");
  WST_REQUIRE(n_kv <= 4096, "wst_attn_decode: too many kv heads");
  WST_REQUIRE(attn_slices(head_dim, max_seq) <= 65535, "wst_attn_decode: max_seq too large");
  WST_REQUIRE(!(((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)partials) & 15u),
              "wst_attn_decode: caches and partials must be 16-byte aligned");
  return WST_OK;
}


extern "C" wst_status_t wst_attn_decode(const void *q, const void *k_cache, const void *v_cache,
                                        void *partials, void *out, int32_t n_q, int32_t n_kv,
                                        int32_t head_dim, const void *pos, int32_t max_seq,
                                        float scale) {
  const wst_status_t st =
      attn_check(q, k_cache, v_cache, partials, out, n_q, n_kv, head_dim, pos, max_seq);
  if (st != WST_OK) return st;
  const RopeArgs ra{nullptr, nullptr, nullptr, nullptr, 0.0f};
  attn_launch<false>(head_dim, q, (void *)k_cache, (void *)v_cache, partials, out, n_q, n_kv,
                     pos, max_seq, scale, ra);
  WST_TRY_KERNEL("wst_attn_decode");
  return WST_OK;
}

extern "C" wst_status_t wst_attn_decode_fused(void *qkv, void *k_cache, void *v_cache,
                                              const void *cos_tab, const void *sin_tab,
                                              void *partials, void *out, int32_t n_q,
                                              int32_t n_kv, int32_t head_dim, const void *pos,
                                              int32_t max_seq, float scale,
                                              const void *q_norm_w, const void *k_norm_w,
                                              float eps) {
  const wst_status_t st =
      attn_check(qkv, k_cache, v_cache, partials, out, n_q, n_kv, head_dim, pos, max_seq);
  if (st != WST_OK) return st;
  WST_REQUIRE(cos_tab && sin_tab, "wst_attn_decode_fused: null rope table");
  WST_REQUIRE(head_dim <= 128, "wst_attn_decode_fused: head_dim must be 64 or 128");
  const RopeArgs ra{(const float *)cos_tab, (const float *)sin_tab, (const uint16_t *)q_norm_w,
                    (const uint16_t *)k_norm_w, eps};
  attn_launch<true>(head_dim, qkv, k_cache, v_cache, partials, out, n_q, n_kv, pos, max_seq,
                    scale, ra);
  WST_TRY_KERNEL("wst_attn_decode_fused");
  return WST_OK;
}

// wst_attn_decode_fused whose merge also writes the activation table of
// its output (n_q * head_dim / 32 entries, as wst_hier_xq_table(out) writes
// them) for the GEMV that consumes it (wst_gemv_hier_xq).
extern "C" wst_status_t wst_attn_decode_fused_xq(void *qkv, void *k_cache, void *v_cache,
                                                 const void *cos_tab, const void *sin_tab,
                                                 void *partials, void *out, void *table,
                                                 int32_t n_q, int32_t n_kv, int32_t head_dim,
                                                 const void *pos, int32_t max_seq, float scale,
                                                 const void *q_norm_w, const void *k_norm_w,
                                                 float eps) {
  const wst_status_t st =
      attn_check(qkv, k_cache, v_cache, partials, out, n_q, n_kv, head_dim, pos, max_seq);
  if (st != WST_OK) return st;
  WST_REQUIRE(cos_tab && sin_tab, "wst_attn_decode_fused_xq: null rope table");
  WST_REQUIRE(table && !((uintptr_t)table & 15u), "wst_attn_decode_fused_xq: table must be non-null and 16-byte aligned");
  WST_REQUIRE(head_dim <= 128, "wst_attn_decode_fused_xq: head_dim must be 64 or 128");
  const RopeArgs ra{(const float *)cos_tab, (const float *)sin_tab, (const uint16_t *)q_norm_w,
                    (const uint16_t *)k_norm_w, eps};
  attn_launch<true>(head_dim, qkv, k_cache, v_cache, partials, out, n_q, n_kv, pos, max_seq,
                    scale, ra, true, (uint32_t *)table);
  WST_TRY_KERNEL("wst_attn_decode_fused_xq");
  return WST_OK;
}

// wst_attn_decode_fused without the merge: the slices' partials are left for
// a consumer that merges them itself (wst_gemv_hier_attn).
extern "C" wst_status_t wst_attn_decode_slices(void *qkv, void *k_cache, void *v_cache,
                                               const void *cos_tab, const void *sin_tab,
                                               void *partials, int32_t n_q, int32_t n_kv,
                                               int32_t head_dim, const void *pos,
                                               int32_t max_seq, float scale,
                                               const void *q_norm_w, const void *k_norm_w,
                                               float eps) {
  const wst_status_t st =
      attn_check(qkv, k_cache, v_cache, partials, partials, n_q, n_kv, head_dim, pos, max_seq);
  if (st != WST_OK) return st;
  WST_REQUIRE(cos_tab && sin_tab, "wst_attn_decode_slices: null rope table");
  WST_REQUIRE(head_dim <= 128, "wst_attn_decode_slices: head_dim must be 64 or 128");
  const RopeArgs ra{(const float *)cos_tab, (const float *)sin_tab, (const uint16_t *)q_norm_w,
                    (const uint16_t *)k_norm_w, eps};
  attn_launch<true>(head_dim, qkv, k_cache, v_cache, partials, nullptr, n_q, n_kv, pos, max_seq,
                    scale, ra, false);
  WST_TRY_KERNEL("wst_attn_decode_slices");
  return WST_OK;
}
