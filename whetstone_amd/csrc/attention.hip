// Batch=1 GQA decode attention over the f16 KV cache.
// reference: crates/whetstone-kernels/cuda/attention.cu (split over the
// sequence, online softmax per slice, associative merge).
//
// MI355X design
// -------------
// * One 512-thread block per (kv head, sequence slice) rather than per
//   (query head, slice): every K/V element is read from memory once and used
//   for all n_q/n_kv query heads of the group, instead of relying on L2 hits
//   that a per-XCD L2 does not guarantee across blocks.
// * A position's head vector is split over hd/8 lanes, 16 B (8 halves) per
//   lane per load. Each wave sweeps ATTN_UNROLL steps of 64/(hd/8) positions
//   per iteration and issues all of an iteration's K/V loads before it uses
//   any; at the configurations' contexts a slice is one iteration, so the
//   whole slice is requested in one round trip.
// * Scores reduce across the hd/8 lanes of a position; each position-group of
//   lanes keeps its own online-softmax state per query head, merged across
//   groups by lane shuffles and across the 8 waves through LDS.
// * The slice merge is done by the last block of each kv head to finish (a
//   device-scope counter that the merging block resets), so the whole
//   attention is one launch and the counter needs no memset inside a graph.
//   The merging threads fetch every slice's partial in one batch of loads.
//   Slices and waves merge in a fixed order: results are deterministic.
// * ROPE form (wst_attn_decode_fused): each block applies QK-norm and RoPE to
//   the q heads it needs exactly as wst_rope_cache does (same per-head
//   reduction, same fma shapes) while its first K/V loads are in flight; the
//   block whose slice holds the current position appends that position's k
//   and v to the cache and uses them from LDS. No other block reads that
//   position, so no cross-block wait is needed, and the result is bit-identical
//   to wst_rope_cache followed by wst_attn_decode.
#include "common.hpp"

#include <stdlib.h>

#define ATTN_MAX_GQA 8
#define ATTN_MAX_SPLITS 16
#define ATTN_MERGE_BATCH 16  // slices fetched per round trip in the merge
#define ATTN_UNROLL 4
#define ATTN_WAVES 8
#define ATTN_THREADS (64 * ATTN_WAVES)

static inline int attn_splits(int n_kv, int max_seq) {
  // Slices of at least 128 cached positions, at most 16 of them (the merge
  // then fetches every slice in one batch), and no more than about one block
  // per CU. (Measured on the 7B shape at ctx 2048: 32 slices of 64 positions
  // are slower -- the merge and the last-block hand-off grow with the slice
  // count faster than the per-slice sweep shrinks.)
  // WST_ATTN_SPLITS caps the slice count (for sweeps).
  static int cap_env = -1;
  if (cap_env < 0) {
    const char *e = getenv("WST_ATTN_SPLITS");
    cap_env = e ? atoi(e) : 0;
  }
  int s = (wst_cu_count() + n_kv - 1) / n_kv;
  if (cap_env > 0 && s > cap_env) s = cap_env;
  const int by_len = (max_seq + 127) / 128;
  if (s > by_len) s = by_len;
  if (s > ATTN_MAX_SPLITS) s = ATTN_MAX_SPLITS;
  if (s < 1) s = 1;
  return s;
}

// Merges online-softmax state (mo, lo, acco) into (m, l, acc).
__device__ __forceinline__ void softmax_merge(float &m, float &l, float *acc, float mo,
                                              float lo, const float *acco) {
  const float mn = fmaxf(m, mo);
  const float a = (m == -INFINITY) ? 0.0f : __expf(m - mn);
  const float b = (mo == -INFINITY) ? 0.0f : __expf(mo - mn);
  l = l * a + lo * b;
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = acc[i] * a + acco[i] * b;
  m = mn;
}

struct RopeArgs {
  const float *cos_tab, *sin_tab;
  const uint16_t *q_norm_w, *k_norm_w;
  float eps;
};

// Sum over the LP lanes of a position (aligned groups of 8, 16 or 32 lanes),
// returned in all of them. DPP row operations (quad swaps, half-row and row
// mirrors, then the gfx950 row swap): a few VALU cycles per step, where lane
// shuffles through LDS cost a round trip each and made the score reduction the
// kernel's bottleneck.
template <int LP>
__device__ __forceinline__ float pos_group_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror: lane i + lane 7-i of each 8
  if constexpr (LP >= 16) v += dpp_f<0x140>(v);  // row_mirror
  if constexpr (LP >= 32) v = xrow16_sum(v);
  return v;
}

__device__ __forceinline__ void unpack8(const uint4 v, float *f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = h2f((uint16_t)(w[i] & 0xFFFFu));
    f[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
  }
}

template <int LP, bool ROPE>  // LP = lanes per position = hd / 8
__global__ __launch_bounds__(ATTN_THREADS) void attn_decode_kernel(
    const float *__restrict__ qkv, uint16_t *__restrict__ k_cache,
    uint16_t *__restrict__ v_cache, float *__restrict__ partials, uint16_t *__restrict__ out,
    unsigned int *__restrict__ counters, int n_q, int n_kv,
    const int32_t *__restrict__ pos_dev, int max_seq, float scale, int splits, RopeArgs ra) {
  constexpr int HD = LP * 8;
  constexpr int PPW = 64 / LP;  // positions per wave step
  constexpr int STEP = ATTN_WAVES * PPW * ATTN_UNROLL;  // positions per block iteration
  constexpr int MAXG = HD > 128 ? 4 : ATTN_MAX_GQA;  // LDS: at most 4 heads at hd 256
  const int gqa = n_q / n_kv;
  const int kvh = blockIdx.x, split = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int sub = lane % LP, pg = lane / LP;

  const int pos = min(max(*pos_dev, 0), max_seq - 1);
  const int seq = min(max(*pos_dev, 0) + 1, max_seq);
  const int per = (seq + splits - 1) / splits;
  const int t0 = split * per;
  const int t1 = min(t0 + per, seq);

  const uint16_t *kb = k_cache + (size_t)kvh * max_seq * HD;
  const uint16_t *vb = v_cache + (size_t)kvh * max_seq * HD;

  // First iteration's K/V requests go out before anything else.
  uint4 kq[ATTN_UNROLL], vq[ATTN_UNROLL];
  int base = t0 + wave * PPW * ATTN_UNROLL;
#pragma unroll
  for (int u = 0; u < ATTN_UNROLL; ++u) {
    const int t = base + u * PPW + pg;
    if (t < t1) {
      kq[u] = *(const uint4 *)(kb + (size_t)t * HD + sub * 8);
      vq[u] = *(const uint4 *)(vb + (size_t)t * HD + sub * 8);
    }
  }

  __shared__ float qs[MAXG * HD];
  __shared__ uint16_t kv_now[2 * HD];  // ROPE: this position's k and v (f16)
  const bool owner = ROPE && pos >= t0 && pos < t1;
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
      const float *src = is_k ? qkv + (size_t)(n_q + kvh) * HD : qkv + (size_t)(kvh * gqa + h) * HD;
      float x1 = active ? src[j] : 0.0f;
      float x2 = active ? src[j + HALF] : 0.0f;
      const uint16_t *g = is_k ? ra.k_norm_w : ra.q_norm_w;
      if (g) {
        // Single-wave form of qk_norm: for one wave block_sum == 0 + wave_sum.
        const float a = active ? fmaf(x1, x1, x2 * x2) : 0.0f;
        const float ss = 0.0f + wave_sum(a);
        const float sc = 1.0f / sqrtf(ss / (float)HD + ra.eps);
        if (active) {
          x1 = x1 * sc * h2f(g[j]);
          x2 = x2 * sc * h2f(g[j + HALF]);
        }
      }
      if (!active) continue;
      const float lo = rope_lo(x1, x2, c, s), hi = rope_hi(x1, x2, c, s);
      if (!is_k) {
        qs[h * HD + j] = lo;
        qs[h * HD + j + HALF] = hi;
      } else if (owner) {
        const float *vh = qkv + (size_t)(n_q + n_kv + kvh) * HD;
        const uint16_t k1 = f2h(lo), k2 = f2h(hi), v1 = f2h(vh[j]), v2 = f2h(vh[j + HALF]);
        kv_now[j] = k1;
        kv_now[j + HALF] = k2;
        kv_now[HD + j] = v1;
        kv_now[HD + j + HALF] = v2;
        const size_t slot = ((size_t)kvh * max_seq + pos) * HD;
        k_cache[slot + j] = k1;
        k_cache[slot + j + HALF] = k2;
        v_cache[slot + j] = v1;
        v_cache[slot + j + HALF] = v2;
      }
    }
  } else {
    for (int k = tid; k < gqa * HD; k += ATTN_THREADS)
      qs[k] = qkv[(size_t)kvh * gqa * HD + k];
  }
  __syncthreads();

  // q slices for every head of the group, pre-scaled (attention.cu:98-101).
  float qr[MAXG][8];
#pragma unroll
  for (int h = 0; h < MAXG; ++h) {
#pragma unroll
    for (int i = 0; i < 8; ++i) qr[h][i] = h < gqa ? qs[h * HD + sub * 8 + i] * scale : 0.0f;
  }

  float m[MAXG], l[MAXG], acc[MAXG][8];
#pragma unroll
  for (int h = 0; h < MAXG; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.0f;
  }

  while (base < t1) {
    const int next = base + STEP;
#pragma unroll
    for (int u = 0; u < ATTN_UNROLL; ++u) {
      const int t = base + u * PPW + pg;
      if (t >= t1) continue;  // uniform across the position's lanes
      float kf[8], vf[8];
      if (owner && t == pos) {
        unpack8(*(const uint4 *)(kv_now + sub * 8), kf);
        unpack8(*(const uint4 *)(kv_now + HD + sub * 8), vf);
      } else {
        unpack8(kq[u], kf);
        unpack8(vq[u], vf);
      }
#pragma unroll
      for (int h = 0; h < MAXG; ++h) {
        if (h >= gqa) break;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = fmaf(qr[h][i], kf[i], s);
        s = pos_group_sum<LP>(s);
        const float mn = fmaxf(m[h], s);
        const float corr = __expf(m[h] - mn);
        const float p = __expf(s - mn);
        l[h] = fmaf(l[h], corr, p);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(p, vf[i], acc[h][i] * corr);
        m[h] = mn;
      }
    }
    base = next;
    if (base < t1) {
#pragma unroll
      for (int u = 0; u < ATTN_UNROLL; ++u) {
        const int t = base + u * PPW + pg;
        if (t < t1) {
          kq[u] = *(const uint4 *)(kb + (size_t)t * HD + sub * 8);
          vq[u] = *(const uint4 *)(vb + (size_t)t * HD + sub * 8);
        }
      }
    }
  }

  // Merge the position groups of this wave (lanes with equal `sub`): groups
  // 8 lanes apart by a DPP row rotation, 16 and 32 apart by the row swaps.
  // softmax_merge is exactly commutative, so both partners end with the same
  // bits.
  if constexpr (LP == 8) {
#pragma unroll
    for (int h = 0; h < MAXG; ++h) {
      if (h >= gqa) break;
      float ao[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) ao[i] = dpp_f<0x128>(acc[h][i]);  // row_ror:8
      softmax_merge(m[h], l[h], acc[h], dpp_f<0x128>(m[h]), dpp_f<0x128>(l[h]), ao);
    }
  }
#pragma unroll
  for (int o = (LP > 16 ? LP : 16); o < 64; o <<= 1) {
#pragma unroll
    for (int h = 0; h < MAXG; ++h) {
      if (h >= gqa) break;
      const RowPair pm = o == 16 ? xrow16(m[h]) : xrow32(m[h]);
      const RowPair pl = o == 16 ? xrow16(l[h]) : xrow32(l[h]);
      float aa[8], ab[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const RowPair pa = o == 16 ? xrow16(acc[h][i]) : xrow32(acc[h][i]);
        aa[i] = pa.a;
        ab[i] = pa.b;
      }
      m[h] = pm.a;
      l[h] = pl.a;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] = aa[i];
      softmax_merge(m[h], l[h], acc[h], pm.b, pl.b, ab);
    }
  }

  // Merge the waves through LDS: [wave][head][HD + 2].
  __shared__ float sm[ATTN_WAVES * MAXG * (HD + 2)];
  if (pg == 0) {
#pragma unroll
    for (int h = 0; h < MAXG; ++h) {
      if (h >= gqa) break;
      float *e = sm + (wave * MAXG + h) * (HD + 2);
      if (sub == 0) {
        e[0] = m[h];
        e[1] = l[h];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) e[2 + sub * 8 + i] = acc[h][i];
    }
  }
  __syncthreads();

  // This slice's partial: acc [n_q][splits][HD], then (m, l) [n_q][splits][2].
  float *pacc = partials;
  float *pml = partials + (size_t)n_q * splits * HD;
  for (int k = tid; k < gqa * HD; k += ATTN_THREADS) {
    const int h = k / HD, d = k % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < ATTN_WAVES; ++w) M = fmaxf(M, sm[(w * MAXG + h) * (HD + 2)]);
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int w = 0; w < ATTN_WAVES; ++w) {
      const float *e = sm + (w * MAXG + h) * (HD + 2);
      const float f = (e[0] == -INFINITY) ? 0.0f : __expf(e[0] - M);
      num = fmaf(e[2 + d], f, num);
      den = fmaf(e[1], f, den);
    }
    const size_t row = (size_t)(kvh * gqa + h) * splits + split;
    pacc[row * HD + d] = num;
    if (d == 0) {
      pml[row * 2] = M;
      pml[row * 2 + 1] = den;
    }
  }

  if (!last_block_done(counters + kvh, (unsigned int)splits)) return;

  // Slice merge for the gqa heads of this kv head (attention.cu:170-193): one
  // thread per (head, 4 dims) fetches the slices' (m, l) and numerators in
  // batches of ATTN_MERGE_BATCH (one round trip each) and combines them in
  // slice order, rescaling the running sum when a batch raises the maximum.
  for (int k = tid; k < gqa * (HD / 4); k += ATTN_THREADS) {
    const int h = k / (HD / 4), d4 = k % (HD / 4);
    const size_t row0 = (size_t)(kvh * gqa + h) * splits;
    float M = -INFINITY, den = 0.0f;
    float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int c0 = 0; c0 < splits; c0 += ATTN_MERGE_BATCH) {
      float ms[ATTN_MERGE_BATCH], ls[ATTN_MERGE_BATCH];
      float4 vs[ATTN_MERGE_BATCH];
      // Unconditional loads (a clamped slice index) so that all of them are
      // in flight together; guarded loads compile to one round trip each.
#pragma unroll
      for (int i = 0; i < ATTN_MERGE_BATCH; ++i) {
        const int s = c0 + i;
        const size_t r = row0 + (s < splits ? s : splits - 1);
        const float2 ml = *(const float2 *)(pml + r * 2);
        ms[i] = s < splits ? ml.x : -INFINITY;
        ls[i] = ml.y;
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
        if (c0 + i >= splits) break;  // uniform; loads are already done
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

template <bool ROPE>
static void attn_launch(int head_dim, const void *qkv, void *k_cache, void *v_cache,
                        void *partials, void *out, unsigned int *counters, int n_q, int n_kv,
                        const void *pos, int max_seq, float scale, int splits,
                        const RopeArgs &ra) {
  const dim3 grid(n_kv, splits);
#define WST_ATTN_GO(LP)                                                                     \
  attn_decode_kernel<LP, ROPE><<<grid, ATTN_THREADS, 0, WST_STREAM>>>(                      \
      (const float *)qkv, (uint16_t *)k_cache, (uint16_t *)v_cache, (float *)partials,      \
      (uint16_t *)out, counters, n_q, n_kv, (const int32_t *)pos, max_seq, scale, splits, ra)
  switch (head_dim) {
    case 64: WST_ATTN_GO(8); break;
    case 128: WST_ATTN_GO(16); break;
    default:
      if constexpr (!ROPE) WST_ATTN_GO(32);
      break;
  }
#undef WST_ATTN_GO
}

extern "C" int32_t wst_attn_partial_floats(int32_t n_q, int32_t head_dim, int32_t max_seq) {
  if (n_q <= 0 || head_dim <= 0 || max_seq <= 0) return 0;
  // Sized for the smallest n_kv (1), which has the most splits.
  return n_q * attn_splits(1, max_seq) * (head_dim + 2);
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
  WST_REQUIRE(head_dim != 256 || n_q / n_kv <= 4,
              "wst_attn_decode: head_dim 256 supports at most 4 query heads per kv head");
  WST_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
              "wst_attn_decode: head_dim must be 64, 128 or 256");
  WST_REQUIRE(max_seq > 0, "wst_attn_decode: empty cache");
  WST_REQUIRE(n_kv <= 4096, "wst_attn_decode: too many kv heads");
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
                     n_kv, pos, max_seq, scale, attn_splits(n_kv, max_seq), ra);
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
                    max_seq, scale, attn_splits(n_kv, max_seq), ra);
  WST_TRY_KERNEL("wst_attn_decode_fused");
  return WST_OK;
}
