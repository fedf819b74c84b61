// Batch=1 GQA decode attention over the f16 KV cache.
// reference: crates/whetstone-kernels/cuda/attention.cu (split over the
// sequence, softmax per slice, associative merge of the slices).
//
// MI355X design
// -------------
// * One 512-thread block per (kv head, slice of P cached positions), P*hd =
//   16384 (P = 256 / 128 / 64 at hd 64 / 128 / 256). Every K/V row is read
//   from memory once and used for all n_q/n_kv query heads of the group.
// * The block stages its slice of K and V in LDS (32 KB each) with one batch of
//   16-byte loads -- one memory round trip -- and then works from LDS:
//     scores   a lane per position, the wave's 64 positions against one query
//              head at a time (q broadcast from LDS): hd FMAs per score, no
//              cross-lane reduction;
//     softmax  a wave per query head over the slice: one max, one exp per
//              (head, position), one sum;
//     P.V      a lane per (head, 8 output dims, 32 positions), reduced over the
//              position groups through LDS.
//   So each exp is computed once (the previous lane-per-dimension layout
//   recomputed the online-softmax exps on every lane of a position and was
//   compute bound).
// * Slices merge in the last block of each kv head to finish (a device-scope
//   counter that the merging block resets: the whole attention is one launch
//   and needs no memset inside a graph), fetching the partials in batches of
//   16 slices per round trip and combining them in slice order. A context
//   that fits one slice skips the partials entirely.
// * The grid covers max_seq; only the ceil(seq/P) slices holding cached
//   positions do work, so a captured graph serves every position.
// * ROPE form (wst_attn_decode_fused): each block applies QK-norm and RoPE to
//   the q heads it needs exactly as wst_rope_cache does (same per-head
//   reduction, same fma shapes) while its K/V loads are in flight; the block
//   whose slice holds the current position appends that position's k and v to
//   the cache and puts them into its LDS tile. No other block reads that
//   position, so no cross-block wait is needed, and the result is
//   bit-identical to wst_rope_cache followed by wst_attn_decode.
// * Deterministic: every sum runs in a fixed order.
#include "common.hpp"

#define ATTN_THREADS 512
#define ATTN_WAVES 8
#define ATTN_MAX_GQA 8
#define ATTN_TILE 16384      // P * hd: halves of K (and of V) a block stages
#define ATTN_MERGE_BATCH 16  // slices fetched per round trip in the merge

template <int HD>
struct AttnShape {
  static constexpr int P = ATTN_TILE / HD;                  // positions per block
  static constexpr int KS = HD + 8;                         // K row stride (halves): +16 B
  static constexpr int G = ATTN_THREADS / P;                // head groups, score phase
  static constexpr int WPG = P / 64;                        // waves per head group
  static constexpr int HPT = (ATTN_MAX_GQA + G - 1) / G;    // heads per lane, score phase
  static constexpr int PG = ATTN_THREADS / HD;              // position groups, P.V phase
  static constexpr int PPG = P / PG;                        // positions per group (32)
  static constexpr int CH = HD / 8;                         // 16-byte chunks per row
  // LDS (bytes): K tile | V tile | q (scaled) | scores | per-head (m, l)
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = K_OFF + P * KS * 2;
  static constexpr int Q_OFF = V_OFF + P * HD * 2;
  static constexpr int S_OFF = Q_OFF + ATTN_MAX_GQA * HD * 4;
  static constexpr int ML_OFF = S_OFF + ATTN_MAX_GQA * P * 4;
  static constexpr int LDS = ML_OFF + ATTN_MAX_GQA * 2 * 4;
  // The P.V reduction buffer [PG][8][HD] f32 reuses the K tile.
  static_assert(PG * ATTN_MAX_GQA * HD * 4 <= P * KS * 2, "reduction buffer fits the K tile");
  static_assert(PPG == 32, "32 positions per P.V group");
};

static inline int attn_slices(int head_dim, int max_seq) {
  const int p = ATTN_TILE / head_dim;
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

template <int HD, bool ROPE>
__global__ __launch_bounds__(ATTN_THREADS, 1) void attn_decode_kernel(
    const float *__restrict__ qkv, uint16_t *__restrict__ k_cache,
    uint16_t *__restrict__ v_cache, float *__restrict__ partials, uint16_t *__restrict__ out,
    unsigned int *__restrict__ counters, int n_q, int n_kv,
    const int32_t *__restrict__ pos_dev, int max_seq, float scale, RopeArgs ra) {
  using S = AttnShape<HD>;
  constexpr int P = S::P, CH = S::CH;
  extern __shared__ __align__(16) unsigned char lds[];
  uint16_t *ktile = (uint16_t *)(lds + S::K_OFF);
  uint16_t *vtile = (uint16_t *)(lds + S::V_OFF);
  float *qs = (float *)(lds + S::Q_OFF);
  float *sc = (float *)(lds + S::S_OFF);
  float *ml = (float *)(lds + S::ML_OFF);
  float *red = (float *)(lds + S::K_OFF);

  const int gqa = n_q / n_kv;
  const int kvh = blockIdx.x, split = blockIdx.y, nsplit = gridDim.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  const int pos = min(max(*pos_dev, 0), max_seq - 1);
  const int seq = min(max(*pos_dev, 0) + 1, max_seq);
  const int nactive = (seq + P - 1) / P;
  if (split >= nactive) return;  // no cached positions here (uniform per block)
  const int t0 = split * P, t1 = min(t0 + P, seq);

  const uint16_t *kb = k_cache + (size_t)kvh * max_seq * HD;
  const uint16_t *vb = v_cache + (size_t)kvh * max_seq * HD;

  // ---- phase A: the slice's K and V requests go out first, all at once.
  constexpr int LD = P * CH / ATTN_THREADS;  // 16-byte chunks per thread per tile (4)
  uint4 kr[LD], vr[LD];
#pragma unroll
  for (int i = 0; i < LD; ++i) {
    const int c = tid + i * ATTN_THREADS, row = c / CH, ch = c % CH;
    const int t = min(t0 + row, seq - 1);  // clamped: unconditional loads stay batched
    kr[i] = *(const uint4 *)(kb + (size_t)t * HD + ch * 8);
    vr[i] = *(const uint4 *)(vb + (size_t)t * HD + ch * 8);
  }

  // q for the group's heads, pre-scaled (attention.cu:98-101), into LDS.
  const bool owner = ROPE && pos >= t0 && pos < t1;
  uint16_t knew = 0, vnew = 0, knew2 = 0, vnew2 = 0;  // owner: this position's k, v
  if constexpr (ROPE) {
    // One wave per head, as wst_rope_cache runs one 64-thread block per head
    // (hd <= 128): lane j owns elements j and j + hd/2.
    constexpr int HALF = HD / 2;
    const int j = lane;
    const bool active = j < HALF;
    const float c = active ? ra.cos_tab[(size_t)pos * HALF + j] : 0.0f;
    const float s = active ? ra.sin_tab[(size_t)pos * HALF + j] : 0.0f;
    for (int h = wave; h < gqa + 1; h += ATTN_WAVES) {
      const bool is_k = h == gqa;
      if (is_k && !owner) continue;
      const float *src = is_k ? qkv + (size_t)(n_q + kvh) * HD : qkv + (size_t)(kvh * gqa + h) * HD;
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
        qs[h * HD + j] = lo * scale;
        qs[h * HD + j + HALF] = hi * scale;
      } else {
        const float *vh = qkv + (size_t)(n_q + n_kv + kvh) * HD;
        knew = f2h(lo);
        knew2 = f2h(hi);
        vnew = f2h(vh[j]);
        vnew2 = f2h(vh[j + HALF]);
        const size_t slot = ((size_t)kvh * max_seq + pos) * HD;
        k_cache[slot + j] = knew;
        k_cache[slot + j + HALF] = knew2;
        v_cache[slot + j] = vnew;
        v_cache[slot + j + HALF] = vnew2;
      }
    }
  } else {
    // At most 8 * 256 values: four unconditional (clamped) loads per thread,
    // so they share one round trip.
    constexpr int QL = ATTN_MAX_GQA * HD / ATTN_THREADS;
    const int nqv = gqa * HD;
    float qv[QL];
#pragma unroll
    for (int i = 0; i < QL; ++i) qv[i] = qkv[(size_t)kvh * nqv + min(tid + i * ATTN_THREADS, nqv - 1)];
#pragma unroll
    for (int i = 0; i < QL; ++i)
      if (tid + i * ATTN_THREADS < nqv) qs[tid + i * ATTN_THREADS] = qv[i] * scale;
  }

  // Tiles into LDS; rows past the cached positions are zero (their scores are
  // masked, and a zero V row keeps 0 * v finite).
#pragma unroll
  for (int i = 0; i < LD; ++i) {
    const int c = tid + i * ATTN_THREADS, row = c / CH, ch = c % CH;
    const uint32_t mk = t0 + row < t1 ? 0xFFFFFFFFu : 0u;  // a mask, not a select of
    const uint4 a = kr[i], b = vr[i];                      // addresses (which spills)
    *(uint4 *)(ktile + row * S::KS + ch * 8) = make_uint4(a.x & mk, a.y & mk, a.z & mk, a.w & mk);
    *(uint4 *)(vtile + row * HD + ch * 8) = make_uint4(b.x & mk, b.y & mk, b.z & mk, b.w & mk);
  }
  if constexpr (ROPE) {
    __syncthreads();  // the tile row of `pos` holds the cache's old contents
    if (owner && wave == gqa % ATTN_WAVES && lane < HD / 2) {
      const int row = pos - t0;
      ktile[row * S::KS + lane] = knew;
      ktile[row * S::KS + lane + HD / 2] = knew2;
      vtile[row * HD + lane] = vnew;
      vtile[row * HD + lane + HD / 2] = vnew2;
    }
  }
  __syncthreads();

  // ---- phase B: scores. Wave w: head group g, positions pb..pb+63 (one per lane).
  {
    const int g = wave / S::WPG;
    const int p = (wave % S::WPG) * 64 + lane;
    float s[S::HPT];
#pragma unroll
    for (int i = 0; i < S::HPT; ++i) s[i] = 0.0f;
    const uint16_t *krow = ktile + p * S::KS;
#pragma unroll 4
    for (int c = 0; c < CH; ++c) {
      float kf[8];
      unpack8(*(const uint4 *)(krow + c * 8), kf);
#pragma unroll
      for (int i = 0; i < S::HPT; ++i) {
        const int h = g + i * S::G;
        if (h < gqa) {  // uniform across the wave
          const float4 qa = *(const float4 *)(qs + h * HD + c * 8);
          const float4 qb = *(const float4 *)(qs + h * HD + c * 8 + 4);
          float a = s[i];
          a = fmaf(qa.x, kf[0], a);
          a = fmaf(qa.y, kf[1], a);
          a = fmaf(qa.z, kf[2], a);
          a = fmaf(qa.w, kf[3], a);
          a = fmaf(qb.x, kf[4], a);
          a = fmaf(qb.y, kf[5], a);
          a = fmaf(qb.z, kf[6], a);
          a = fmaf(qb.w, kf[7], a);
          s[i] = a;
        }
      }
    }
    const bool valid = t0 + p < t1;
#pragma unroll
    for (int i = 0; i < S::HPT; ++i) {
      const int h = g + i * S::G;
      if (h < gqa) sc[h * P + p] = valid ? s[i] : -INFINITY;
    }
  }
  __syncthreads();

  // ---- phase C: softmax over the slice, a wave per head.
  if (wave < gqa) {
    constexpr int R = P / 64;
    float v[R];
    float m = -INFINITY;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      v[r] = sc[wave * P + lane + 64 * r];
      m = fmaxf(m, v[r]);
    }
    m = wave_max(m);  // finite: every active slice holds a cached position
    float l = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float e = (v[r] == -INFINITY) ? 0.0f : __expf(v[r] - m);
      sc[wave * P + lane + 64 * r] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      ml[wave * 2] = m;
      ml[wave * 2 + 1] = l;
    }
  }
  __syncthreads();

  // ---- phase D: P.V. Lane (position group pg, head h, 8 dims dc).
  {
    const int pg = tid / HD, rem = tid % HD, h = rem / CH, dc = rem % CH;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    if (h < gqa) {
      const float *w = sc + h * P + pg * S::PPG;
      const uint16_t *vcol = vtile + (pg * S::PPG) * HD + dc * 8;
#pragma unroll 8
      for (int j = 0; j < S::PPG; ++j) {
        const float pj = w[j];
        float vf[8];
        unpack8(*(const uint4 *)(vcol + j * HD), vf);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(pj, vf[i], acc[i]);
      }
    }
    // K tile is dead since phase B: reuse it for the group reduction.
    float4 *dst = (float4 *)(red + ((pg * ATTN_MAX_GQA + h) * HD + dc * 8));
    dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  __syncthreads();

  // ---- phase E: this slice's result.
  float *pacc = partials;
  float *pml = partials + (size_t)n_q * nsplit * HD;
  for (int k = tid; k < gqa * HD; k += ATTN_THREADS) {
    const int h = k / HD, d = k % HD;
    float a = 0.0f;
#pragma unroll
    for (int pg = 0; pg < S::PG; ++pg) a += red[(pg * ATTN_MAX_GQA + h) * HD + d];
    if (nactive == 1) {
      out[(size_t)(kvh * gqa + h) * HD + d] = f2h(a / ml[h * 2 + 1]);
    } else {
      const size_t row = (size_t)(kvh * gqa + h) * nsplit + split;
      pacc[row * HD + d] = a;
      if (d == 0) {
        pml[row * 2] = ml[h * 2];
        pml[row * 2 + 1] = ml[h * 2 + 1];
      }
    }
  }
  if (nactive == 1) return;
  if (!last_block_done(counters + kvh, (unsigned int)nactive)) return;

  // ---- slice merge for the gqa heads of this kv head (attention.cu:170-193):
  // one thread per (head, 4 dims) fetches the slices' (m, l) and numerators in
  // batches of ATTN_MERGE_BATCH (one round trip each) and combines them in
  // slice order, rescaling the running sum when a batch raises the maximum.
  for (int k = tid; k < gqa * (HD / 4); k += ATTN_THREADS) {
    const int h = k / (HD / 4), d4 = k % (HD / 4);
    const size_t row0 = (size_t)(kvh * gqa + h) * nsplit;
    float M = -INFINITY, den = 0.0f;
    float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int c0 = 0; c0 < nactive; c0 += ATTN_MERGE_BATCH) {
      float ms[ATTN_MERGE_BATCH], ls[ATTN_MERGE_BATCH];
      float4 vs[ATTN_MERGE_BATCH];
      // Unconditional loads (a clamped slice index) so that all of them are
      // in flight together; guarded loads compile to one round trip each.
#pragma unroll
      for (int i = 0; i < ATTN_MERGE_BATCH; ++i) {
        const int s = c0 + i;
        const size_t r = row0 + (s < nactive ? s : nactive - 1);
        const float2 mlv = *(const float2 *)(pml + r * 2);
        ms[i] = s < nactive ? mlv.x : -INFINITY;
        ls[i] = mlv.y;
        vs[i] = ((const float4 *)(pacc + r * HD))[d4];
      }
      float Mn = M;
#pragma unroll
      for (int i = 0; i < ATTN_MERGE_BATCH; ++i) Mn = fmaxf(Mn, ms[i]);
      const float fo = (M == -INFINITY) ? 0.0f : __expf(M - Mn);
      a.x *= fo;
      a.y *= fo;
      a.z *= fo;
      a.w *= fo;
      den *= fo;
#pragma unroll
      for (int i = 0; i < ATTN_MERGE_BATCH; ++i) {
        // slices past nactive carry m = -inf: f = 0 adds exact zeros
        const float f = (ms[i] == -INFINITY) ? 0.0f : __expf(ms[i] - Mn);
        a.x = fmaf(vs[i].x, f, a.x);
        a.y = fmaf(vs[i].y, f, a.y);
        a.z = fmaf(vs[i].z, f, a.z);
        a.w = fmaf(vs[i].w, f, a.w);
        den = fmaf(ls[i], f, den);
      }
      M = Mn;
    }
    uint16_t *o = out + (size_t)(kvh * gqa + h) * HD + d4 * 4;
    o[0] = f2h(a.x / den);
    o[1] = f2h(a.y / den);
    o[2] = f2h(a.z / den);
    o[3] = f2h(a.w / den);
  }
}

template <int HD, bool ROPE>
static void attn_go(const dim3 grid, const void *qkv, void *k_cache, void *v_cache,
                    void *partials, void *out, unsigned int *counters, int n_q, int n_kv,
                    const void *pos, int max_seq, float scale, const RopeArgs &ra) {
  static bool attr_set = false;
  if (!attr_set) {
    hipFuncSetAttribute((const void *)attn_decode_kernel<HD, ROPE>,
                        hipFuncAttributeMaxDynamicSharedMemorySize, AttnShape<HD>::LDS);
    attr_set = true;
  }
  attn_decode_kernel<HD, ROPE><<<grid, ATTN_THREADS, AttnShape<HD>::LDS, WST_STREAM>>>(
      (const float *)qkv, (uint16_t *)k_cache, (uint16_t *)v_cache, (float *)partials,
      (uint16_t *)out, counters, n_q, n_kv, (const int32_t *)pos, max_seq, scale, ra);
}

template <bool ROPE>
static void attn_launch(int head_dim, const void *qkv, void *k_cache, void *v_cache,
                        void *partials, void *out, unsigned int *counters, int n_q, int n_kv,
                        const void *pos, int max_seq, float scale, const RopeArgs &ra) {
  const dim3 grid(n_kv, attn_slices(head_dim, max_seq));
  switch (head_dim) {
    case 64:
      attn_go<64, ROPE>(grid, qkv, k_cache, v_cache, partials, out, counters, n_q, n_kv, pos,
                        max_seq, scale, ra);
      break;
    case 128:
      attn_go<128, ROPE>(grid, qkv, k_cache, v_cache, partials, out, counters, n_q, n_kv, pos,
                         max_seq, scale, ra);
      break;
    default:
      if constexpr (!ROPE)
        attn_go<256, false>(grid, qkv, k_cache, v_cache, partials, out, counters, n_q, n_kv,
                            pos, max_seq, scale, ra);
      break;
  }
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

static unsigned int *attn_counters() {
  return (unsigned int *)wst_static_scratch(WST_SCRATCH_ATTN, 4096 * sizeof(unsigned int));
}

extern "C" wst_status_t wst_attn_decode(const void *q, const void *k_cache, const void *v_cache,
                                        void *partials, void *out, int32_t n_q, int32_t n_kv,
                                        int32_t head_dim, const void *pos, int32_t max_seq,
                                        float scale) {
  const wst_status_t st =
      attn_check(q, k_cache, v_cache, partials, out, n_q, n_kv, head_dim, pos, max_seq);
  if (st != WST_OK) return st;
  unsigned int *counters = attn_counters();
  if (!counters) return WST_ERR_OOM;
  const RopeArgs ra{nullptr, nullptr, nullptr, nullptr, 0.0f};
  attn_launch<false>(head_dim, q, (void *)k_cache, (void *)v_cache, partials, out, counters, n_q,
                     n_kv, pos, max_seq, scale, ra);
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
  unsigned int *counters = attn_counters();
  if (!counters) return WST_ERR_OOM;
  const RopeArgs ra{(const float *)cos_tab, (const float *)sin_tab, (const uint16_t *)q_norm_w,
                    (const uint16_t *)k_norm_w, eps};
  attn_launch<true>(head_dim, qkv, k_cache, v_cache, partials, out, counters, n_q, n_kv, pos,
                    max_seq, scale, ra);
  WST_TRY_KERNEL("wst_attn_decode_fused");
  return WST_OK;
}
