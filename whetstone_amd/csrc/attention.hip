// Batch=1 GQA decode attention over the f16 KV cache.
// reference: crates/whetstone-kernels/cuda/attention.cu (split over the
// sequence, online softmax per slice, associative merge).
//
// MI355X design
// -------------
// * One block per (kv head, sequence slice) rather than per (query head,
//   slice): every K/V element is read from memory once and used for all
//   n_q/n_kv query heads of the group, instead of relying on L2 hits that a
//   per-XCD L2 does not guarantee across blocks.
// * A position's head vector is split over hd/8 lanes, 16 B (8 halves) per
//   lane per load, so one wave reads 64/(hd/8) positions of K and V per step
//   with dwordx4 loads.
// * Scores reduce across the hd/8 lanes of a position; each position-group of
//   lanes keeps its own online-softmax state per query head, merged across
//   groups by lane shuffles and across the 4 waves through LDS.
// * The slice merge is done by the last block of each kv head to finish (a
//   device-scope counter that the merging block resets), so the whole
//   attention is one launch and the counter needs no memset inside a graph.
//   Slices and waves are merged in a fixed order: results are deterministic.
// * ROPE form (wst_attn_decode_fused): each block first applies QK-norm and
//   RoPE to the q heads it needs, exactly as wst_rope_cache does (same
//   per-head reduction, same fma shapes), keeps them in LDS, and the block
//   whose slice holds the current position appends that position's k and v to
//   the cache before reading it. No other block reads that position, so no
//   cross-block wait is needed, and the result is bit-identical to
//   wst_rope_cache followed by wst_attn_decode.
#include "common.hpp"

#define ATTN_MAX_GQA 8
#define ATTN_MAX_SPLITS 64
#define ATTN_UNROLL 4

static inline int attn_splits(int n_kv, int max_seq) {
  // ~2 blocks per CU, but never slices thinner than 128 cached positions: a
  // slice is one or two unrolled sweeps of a block, and the merge reads every
  // slice's partial.
  int s = (2 * wst_cu_count() + n_kv - 1) / n_kv;
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

template <int LP, bool ROPE>  // LP = lanes per position = hd / 8
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const float *__restrict__ qkv, uint16_t *__restrict__ k_cache,
    uint16_t *__restrict__ v_cache, float *__restrict__ partials, uint16_t *__restrict__ out,
    unsigned int *__restrict__ counters, int n_q, int n_kv,
    const int32_t *__restrict__ pos_dev, int max_seq, float scale, int splits, RopeArgs ra) {
  constexpr int HD = LP * 8;
  constexpr int PPW = 64 / LP;  // positions per wave step
  const int gqa = n_q / n_kv;
  const int kvh = blockIdx.x, split = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int sub = lane % LP, pg = lane / LP;

  const int pos = min(max(*pos_dev, 0), max_seq - 1);
  const int seq = min(max(*pos_dev, 0) + 1, max_seq);
  const int per = (seq + splits - 1) / splits;
  const int t0 = split * per;
  const int t1 = min(t0 + per, seq);

  __shared__ float qs[ROPE ? ATTN_MAX_GQA * HD : 1];
  if constexpr (ROPE) {
    // One wave per head, as wst_rope_cache runs one 64-thread block per head
    // (hd <= 128): lane j owns elements j and j + hd/2.
    __shared__ float red[4][16];
    constexpr int HALF = HD / 2;
    const int j = lane;
    const bool active = j < HALF;
    const float c = active ? ra.cos_tab[(size_t)pos * HALF + j] : 0.0f;
    const float s = active ? ra.sin_tab[(size_t)pos * HALF + j] : 0.0f;
    const bool owner = pos >= t0 && pos < t1;  // this block appends k/v
    for (int h = wave; h < gqa + 1; h += 4) {
      const bool is_k = h == gqa;
      const float *src = is_k ? qkv + (size_t)(n_q + kvh) * HD : qkv + (size_t)(kvh * gqa + h) * HD;
      float x1 = active ? src[j] : 0.0f;
      float x2 = active ? src[j + HALF] : 0.0f;
      const uint16_t *g = is_k ? ra.k_norm_w : ra.q_norm_w;
      if (g) {
        // Single-wave form of qk_norm: for one wave block_sum == wave_sum.
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
        const size_t slot = ((size_t)kvh * max_seq + pos) * HD;
        const float *vh = qkv + (size_t)(n_q + n_kv + kvh) * HD;
        k_cache[slot + j] = f2h(lo);
        k_cache[slot + j + HALF] = f2h(hi);
        v_cache[slot + j] = f2h(vh[j]);
        v_cache[slot + j + HALF] = f2h(vh[j + HALF]);
      }
    }
    (void)red;
    __syncthreads();
  }

  // q slices for every head of the group, pre-scaled (attention.cu:98-101).
  float qr[ATTN_MAX_GQA][8];
#pragma unroll
  for (int h = 0; h < ATTN_MAX_GQA; ++h) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = 0.0f;
      if (h < gqa) v = ROPE ? qs[h * HD + sub * 8 + i] : qkv[(size_t)(kvh * gqa + h) * HD + sub * 8 + i];
      qr[h][i] = v * scale;
    }
  }

  float m[ATTN_MAX_GQA], l[ATTN_MAX_GQA], acc[ATTN_MAX_GQA][8];
#pragma unroll
  for (int h = 0; h < ATTN_MAX_GQA; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.0f;
  }

  // Each wave sweeps ATTN_UNROLL steps of PPW positions per iteration; all the
  // K/V loads of an iteration are issued before any is consumed.
  const uint16_t *kb = k_cache + (size_t)kvh * max_seq * HD;
  const uint16_t *vb = v_cache + (size_t)kvh * max_seq * HD;
  for (int base = t0 + wave * PPW * ATTN_UNROLL; base < t1; base += 4 * PPW * ATTN_UNROLL) {
    uint4 kq[ATTN_UNROLL], vq[ATTN_UNROLL];
#pragma unroll
    for (int u = 0; u < ATTN_UNROLL; ++u) {
      const int t = base + u * PPW + pg;
      if (t < t1) {
        kq[u] = *(const uint4 *)(kb + (size_t)t * HD + sub * 8);
        vq[u] = *(const uint4 *)(vb + (size_t)t * HD + sub * 8);
      }
    }
#pragma unroll
    for (int u = 0; u < ATTN_UNROLL; ++u) {
      if (base + u * PPW + pg >= t1) continue;  // uniform across the position's lanes
      float kf[8], vf[8];
      const uint32_t kw[4] = {kq[u].x, kq[u].y, kq[u].z, kq[u].w};
      const uint32_t vw[4] = {vq[u].x, vq[u].y, vq[u].z, vq[u].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kf[2 * i] = h2f((uint16_t)(kw[i] & 0xFFFFu));
        kf[2 * i + 1] = h2f((uint16_t)(kw[i] >> 16));
        vf[2 * i] = h2f((uint16_t)(vw[i] & 0xFFFFu));
        vf[2 * i + 1] = h2f((uint16_t)(vw[i] >> 16));
      }
#pragma unroll
      for (int h = 0; h < ATTN_MAX_GQA; ++h) {
        if (h >= gqa) break;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = fmaf(qr[h][i], kf[i], s);
#pragma unroll
        for (int o = 1; o < LP; o <<= 1) s += __shfl_xor(s, o, 64);
        const float mn = fmaxf(m[h], s);
        const float corr = __expf(m[h] - mn);
        const float p = __expf(s - mn);
        l[h] = fmaf(l[h], corr, p);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(p, vf[i], acc[h][i] * corr);
        m[h] = mn;
      }
    }
  }

  // Merge the position groups of this wave (lanes with equal `sub`).
#pragma unroll
  for (int o = LP; o < 64; o <<= 1) {
#pragma unroll
    for (int h = 0; h < ATTN_MAX_GQA; ++h) {
      if (h >= gqa) break;
      const float mo = __shfl_xor(m[h], o, 64);
      const float lo = __shfl_xor(l[h], o, 64);
      float ao[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) ao[i] = __shfl_xor(acc[h][i], o, 64);
      softmax_merge(m[h], l[h], acc[h], mo, lo, ao);
    }
  }

  // Merge the 4 waves through LDS: [wave][head][HD + 2].
  __shared__ float sm[4 * ATTN_MAX_GQA * (HD + 2)];
  if (pg == 0) {
#pragma unroll
    for (int h = 0; h < ATTN_MAX_GQA; ++h) {
      if (h >= gqa) break;
      float *e = sm + (wave * ATTN_MAX_GQA + h) * (HD + 2);
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
  for (int k = tid; k < gqa * HD; k += 256) {
    const int h = k / HD, d = k % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm[(w * ATTN_MAX_GQA + h) * (HD + 2)]);
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float *e = sm + (w * ATTN_MAX_GQA + h) * (HD + 2);
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

  // Slice merge for the gqa heads of this kv head (attention.cu:170-193), in
  // three parallel phases so no thread walks the slices with dependent loads:
  // (1) every (head, slice) max/denominator into LDS, (2) per head the global
  // max, the slice weights and the denominator, (3) per (head, 4 dims) the
  // weighted sum of the slice numerators, float4 loads unrolled.
  __shared__ float fsh[ATTN_MAX_GQA * ATTN_MAX_SPLITS], lsh[ATTN_MAX_GQA * ATTN_MAX_SPLITS];
  __shared__ float densh[ATTN_MAX_GQA];
  for (int k = tid; k < gqa * splits; k += 256) {
    const size_t row = (size_t)kvh * gqa * splits + k;  // == (kvh*gqa + h)*splits + s
    fsh[k] = pml[row * 2];
    lsh[k] = pml[row * 2 + 1];
  }
  __syncthreads();
  if (tid < gqa) {
    const float *mh = fsh + tid * splits;
    float M = -INFINITY;
    for (int s = 0; s < splits; ++s) M = fmaxf(M, mh[s]);
    float den = 0.0f;
    for (int s = 0; s < splits; ++s) {
      const float f = (mh[s] == -INFINITY) ? 0.0f : __expf(mh[s] - M);
      den = fmaf(lsh[tid * splits + s], f, den);
      fsh[tid * splits + s] = f;
    }
    densh[tid] = den;
  }
  __syncthreads();
  for (int k = tid; k < gqa * (HD / 4); k += 256) {
    const int h = k / (HD / 4), d4 = k % (HD / 4);
    const float4 *src = (const float4 *)(pacc + (size_t)(kvh * gqa + h) * splits * HD) + d4;
    const float *f = fsh + h * splits;
    float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 8
    for (int s = 0; s < splits; ++s) {
      const float4 v = src[(size_t)s * (HD / 4)];
      a.x = fmaf(v.x, f[s], a.x);
      a.y = fmaf(v.y, f[s], a.y);
      a.z = fmaf(v.z, f[s], a.z);
      a.w = fmaf(v.w, f[s], a.w);
    }
    const float den = densh[h];
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
  attn_decode_kernel<LP, ROPE><<<grid, 256, 0, WST_STREAM>>>(                               \
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
  WST_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
              "wst_attn_decode: head_dim must be 64, 128 or 256");
  WST_REQUIRE(max_seq > 0, "wst_attn_decode: empty cache");
  WST_REQUIRE(n_kv <= 4096, "wst_attn_decode: too many kv heads");
  WST_REQUIRE(!(((uintptr_t)k_cache | (uintptr_t)v_cache) & 15u),
              "wst_attn_decode: caches must be 16-byte aligned");
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
