// Multi-token ("chunk") forms of the decode step, for prefill.
// reference: crates/whetstone-kernels/cuda/chunk_gemm.cu, chunk_ops.cu.
//
// Activations are token-major [n][dim]; pos0 is passed by value (a chunk pass
// is not graph-captured, chunk.rs:1-12). Causality is the loop bound: token j
// attends to cache positions [0, pos0 + j].
#include "common.hpp"

#define CHUNK_MAX_TOKENS 256

extern "C" int32_t wst_chunk_max_tokens(void) { return CHUNK_MAX_TOKENS; }

// Implemented in gemm.hip (MFMA).
wst_status_t wst_gemm_mfma(bool hier, const void *w, const void *si, const void *sb,
                           const void *x, const void *bias, void *y, int32_t in_f, int32_t out_f,
                           int32_t n, int32_t accum, float *ws_ext = nullptr, size_t ws_cap = 0,
                           int32_t plan_n = 0);

extern "C" wst_status_t wst_gemm_int4_hier_chunks(const void *qw, const void *si, const void *sb,
                                                  const void *x, const void *bias, void *y,
                                                  int32_t in_f, int32_t out_f, int32_t n,
                                                  int32_t accum, int32_t plan_n) {
  WST_REQUIRE(qw && si && sb && x && y, "wst_gemm_int4_hier: null pointer");
  WST_REQUIRE(in_f > 0 && out_f > 0 && n > 0, "wst_gemm_int4_hier: non-positive dimension");
  WST_REQUIRE(in_f % 32 == 0, "wst_gemm_int4_hier: in_features must be a multiple of 32");
  WST_REQUIRE(!(((uintptr_t)qw | (uintptr_t)x) & 15u),
              "wst_gemm_int4_hier: qw and x must be 16-byte aligned");
  const wst_status_t st =
      wst_gemm_mfma(true, qw, si, sb, x, bias, y, in_f, out_f, n, accum, nullptr, 0, plan_n);
  if (st != WST_OK) return st;
  WST_TRY_KERNEL("wst_gemm_int4_hier");
  return WST_OK;
}

extern "C" wst_status_t wst_gemm_int4_hier(const void *qw, const void *si, const void *sb,
                                           const void *x, const void *bias, void *y,
                                           int32_t in_f, int32_t out_f, int32_t n,
                                           int32_t accum) {
  return wst_gemm_int4_hier_chunks(qw, si, sb, x, bias, y, in_f, out_f, n, accum, n);
}

extern "C" wst_status_t wst_gemm_fp16(const void *w, const void *x, const void *bias, void *y,
                                      int32_t in_f, int32_t out_f, int32_t n, int32_t accum) {
  WST_REQUIRE(w && x && y, "wst_gemm_fp16: null pointer");
  WST_REQUIRE(in_f > 0 && out_f > 0 && n > 0, "wst_gemm_fp16: non-positive dimension");
  WST_REQUIRE(in_f % 8 == 0, "wst_gemm_fp16: in_features must be a multiple of 8");
  if (in_f % 32 == 0 && !(((uintptr_t)w | (uintptr_t)x) & 15u)) {
    const wst_status_t st = wst_gemm_mfma(false, w, nullptr, nullptr, x, bias, y, in_f, out_f, n,
                                          accum);
    if (st != WST_OK) return st;
    WST_TRY_KERNEL("wst_gemm_fp16");
    return WST_OK;
  }
  for (int j = 0; j < n; ++j) {  // widths that are not whole 32-column steps
    const wst_status_t st = wst_gemv_fp16_ex(w, (const uint16_t *)x + (size_t)j * in_f, bias,
                                             (float *)y + (size_t)j * out_f, in_f, out_f, accum);
    if (st != WST_OK) return st;
  }
  return WST_OK;
}

// Causal chunk attention (chunk_ops.cu:187-265) for head_dim 256: one block
// per (query head, token). q is the rotated q of the token's qkv row; the cache already holds
// the chunk's own k/v (wst_rope_cache_chunk ran first). Each of the 4 waves
// sweeps every 4th position with head_dim/64 elements per lane and its own
// online softmax; the waves merge through LDS.
template <int HD>
__global__ __launch_bounds__(256) void attn_chunk_kernel(
    const float *__restrict__ qkv, const uint16_t *__restrict__ k_cache,
    const uint16_t *__restrict__ v_cache, uint16_t *__restrict__ out, int n_q, int n_kv,
    int pos0, int max_seq, float scale) {
  constexpr int EPL = HD / 64;  // elements per lane
  const int head = blockIdx.x, tok = blockIdx.y;
  const int gqa = n_q / n_kv, kvh = head / gqa;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int stride_row = (n_q + 2 * n_kv) * HD;
  const float *q = qkv + (size_t)tok * stride_row + (size_t)head * HD;
  const int seq = min(pos0 + tok + 1, max_seq);

  float qr[EPL], acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    qr[e] = q[lane + 64 * e] * scale;
    acc[e] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  const uint16_t *kb = k_cache + (size_t)kvh * max_seq * HD;
  const uint16_t *vb = v_cache + (size_t)kvh * max_seq * HD;
  for (int t = wave; t < seq; t += 4) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) s = fmaf(qr[e], h2f(kb[(size_t)t * HD + lane + 64 * e]), s);
    s = wave_sum(s);
    const float mn = fmaxf(m, s);
    const float corr = __expf(m - mn);
    const float p = __expf(s - mn);
    l = fmaf(l, corr, p);
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      acc[e] = fmaf(p, h2f(vb[(size_t)t * HD + lane + 64 * e]), acc[e] * corr);
    m = mn;
  }
  __shared__ float sm[4][HD + 2];
#pragma unroll
  for (int e = 0; e < EPL; ++e) sm[wave][2 + lane + 64 * e] = acc[e];
  if (lane == 0) {
    sm[wave][0] = m;
    sm[wave][1] = l;
  }
  __syncthreads();
  for (int d = tid; d < HD; d += 256) {
    float M = -INFINITY;
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm[w][0]);
    float num = 0.0f, den = 0.0f;
    for (int w = 0; w < 4; ++w) {
      const float f = (sm[w][0] == -INFINITY) ? 0.0f : __expf(sm[w][0] - M);
      num = fmaf(sm[w][2 + d], f, num);
      den = fmaf(sm[w][1], f, den);
    }
    out[(size_t)tok * n_q * HD + (size_t)head * HD + d] = f2h(num / den);
  }
}

// ------------------------------------------------------ MFMA chunk attention
//
// The same causal attention (chunk_ops.cu:187-265) as flash attention on
// v_mfma_f32_16x16x32_f16, for head_dim 64 and 128:
// * one 512-thread block per (query head, 16 query tokens); its eight waves
//   take key tiles of 32 positions round-robin, each with its own online
//   softmax, and merge once at the end through LDS;
// * scores S = q . k^T: q (already rotated, times log2(e)/sqrt(hd), so the
//   softmax is in base 2) enters as its f16 hi part plus the f16 rounding of
//   the rest, so the products keep ~22 bits; K rows load coalesced (a
//   128-byte row per eight lanes) into LDS, and the B operand (16 bytes of one
//   position per lane) is read from there (loaded straight into that layout,
//   each load touched sixteen part rows: hd 128 was 13% slower);
// * P . V: P (hi + lo, as q) and V are turned into MFMA operands with the
//   gfx950 transposing LDS read (ds_read_b64_tr_b16): within 16 lanes, lane L's
//   element i comes from lane 4i + L/4's element L%4, so V stays row-major in
//   LDS as loaded and P is stored [position][token] straight from the score
//   accumulators -- no transposing stores;
// * the next key tile's loads are issued before the current tile's compute.
// Causality is a mask: token j keeps positions <= pos0 + j.
typedef _Float16 ac_h8 __attribute__((ext_vector_type(8)));
typedef short ac_s4 __attribute__((ext_vector_type(4)));
typedef short ac_s8 __attribute__((ext_vector_type(8)));
typedef float ac_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t ac_u4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) ac_s4 ac_lds_s4;

#define AC_WAVES 8
#define AC_TT 16  // query tokens per block
#define AC_KT 32  // key positions per wave iteration

template <int HD>
struct AcShape {
  static constexpr int KS = HD / 32;              // k-steps of the scores
  static constexpr int NT = HD / 16;              // 16-dim output tiles
  static constexpr int VR = HD + 16;              // V row stride (halves)
  static constexpr int KR = HD + 8;               // K row stride (halves)
  static constexpr int PR = AC_TT;                // P row stride (halves): [pos][tok]
  static constexpr int VU = AC_KT * HD / 8 / 64;  // 16-byte V pieces per lane per tile
  static constexpr int WAVE_HALVES = AC_KT * VR + AC_KT * KR + 2 * AC_KT * PR;
  static constexpr int LDS = AC_WAVES * WAVE_HALVES * 2;
  static_assert(16 * (HD + 2) * 4 <= WAVE_HALVES * 2, "the merge rows fit a wave's region");
};

// Eight halves as an MFMA operand from two transposing reads (rows r and r + 4
// of the 16-lane pattern each lane's address selects).
__device__ __forceinline__ ac_h8 tr_pair(const uint16_t *a0, const uint16_t *a1) {
  const ac_s4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((ac_lds_s4 *)a0);
  const ac_s4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((ac_lds_s4 *)a1);
  return __builtin_bit_cast(ac_h8, __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <int HD>
__global__ __launch_bounds__(AC_WAVES * 64) void attn_chunk_mfma_kernel(
    const float *__restrict__ qkv, const uint16_t *__restrict__ k_cache,
    const uint16_t *__restrict__ v_cache, uint16_t *__restrict__ out, int n_q, int n_kv,
    int pos0, int n, int max_seq, float scale) {
  using S = AcShape<HD>;
  extern __shared__ __align__(16) uint16_t ac_lds[];
  // Token groups in reverse order: blocks are dispatched in index order, and
  // the last tokens attend to the most positions, so the longest blocks start
  // first and the short ones fill in behind them (a batched prefill's causal
  // work spans 16x between its first and last chunk).
  const int head = blockIdx.x, t0 = (gridDim.y - 1 - blockIdx.y) * AC_TT;
  const int kvh = head / (n_q / n_kv);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the tile loop is scalar
  const int r16 = lane & 15, kg = lane >> 4;
  uint16_t *vs = ac_lds + wave * S::WAVE_HALVES;  // V tile [AC_KT][VR], row-major
  uint16_t *ph = vs + AC_KT * S::VR;              // P hi [AC_KT][PR] ([pos][tok])
  uint16_t *pl = ph + AC_KT * S::PR;              // P lo
  uint16_t *ks = pl + AC_KT * S::PR;              // K tile [AC_KT][KR], row-major
  const int stride_row = (n_q + 2 * n_kv) * HD;
  const uint16_t *kb = k_cache + (size_t)kvh * max_seq * HD;
  const uint16_t *vb = v_cache + (size_t)kvh * max_seq * HD;

  // q of token t0 + r16 as the A operand: dims 32s + 8kg + i, hi and lo parts,
  // scaled by log2(e) as well, so that the scores are in base 2 and the
  // softmax exponentials are bare exp2.
  const float qscale = scale * 1.44269504088896340736f;
  ac_h8 qh[S::KS], ql[S::KS];
  {
    const float *q = qkv + (size_t)min(t0 + r16, n - 1) * stride_row + (size_t)head * HD;
#pragma unroll
    for (int s = 0; s < S::KS; ++s) {
      const float4 a = *(const float4 *)(q + 32 * s + 8 * kg);
      const float4 b = *(const float4 *)(q + 32 * s + 8 * kg + 4);
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = v[i] * qscale;
        const _Float16 h = (_Float16)x;
        qh[s][i] = h;
        ql[s][i] = (_Float16)(x - (float)h);
      }
    }
  }
  const int tlast = min(t0 + AC_TT, n) - 1;
  const int kend = min(pos0 + tlast + 1, max_seq);  // positions [0, kend) are attended
  const int ntiles = (kend + AC_KT - 1) / AC_KT;

  // Loads of key tile kt as buffer loads over [0, kend) of the head's cache
  // rows. The whole byte offset (the lane's within the tile plus the tile's)
  // goes in the vector offset, which is the offset the buffer range check
  // compares with num_records, so positions at or past kend read zeros
  // whatever the cache holds there (their scores are masked, their P is zero),
  // and no load reaches past the allocation. K and V rows both load as
  // 16-byte pieces, eight lanes to a 128-byte row, and go through LDS.
  const uint32_t kv_bytes = (uint32_t)kend * HD * 2u;
  // 0x00020000: word 3 of a raw gfx9 buffer resource (32-bit data format,
  // no swizzle); a load past kv_bytes returns zeros.
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void *)kb, 0, (int)kv_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void *)vb, 0, (int)kv_bytes, 0x00020000);
  const uint32_t voff = (uint32_t)((lane / (HD / 8)) * HD + 8 * (lane % (HD / 8))) * 2u;
#define AC_LOAD_TILE(KR_, VR_, KT)                                                          \
  do {                                                                                      \
    const uint32_t so_ = (uint32_t)(KT) * (AC_KT * HD * 2);                                \
    _Pragma("unroll") for (int j = 0; j < S::VU; ++j) KR_[j] =                              \
        __builtin_amdgcn_raw_buffer_load_b128(krs, so_ + voff + j * (64 / (HD / 8)) * HD * 2, \
                                              0, 0);                                        \
    _Pragma("unroll") for (int j = 0; j < S::VU; ++j) VR_[j] =                              \
        __builtin_amdgcn_raw_buffer_load_b128(vrs, so_ + voff + j * (64 / (HD / 8)) * HD * 2, \
                                              0, 0);                                        \
  } while (0)
  ac_u4 kr[S::VU], vr[S::VU];

  float m[4], l[4];
  ac_f4 o[S::NT];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.0f;
  }
#pragma unroll
  for (int t = 0; t < S::NT; ++t) o[t] = (ac_f4){0.0f, 0.0f, 0.0f, 0.0f};

  int kt = wave;
  AC_LOAD_TILE(kr, vr, min(kt, max(ntiles - 1, 0)));
  while (kt < ntiles) {
    const int p0 = kt * AC_KT;
    // K and V tiles into LDS (rows past kend hold zeros; their P is zero)
#pragma unroll
    for (int j = 0; j < S::VU; ++j) {
      const int u = lane + 64 * j, pr = u / (HD / 8), ch = u % (HD / 8);
      *(ac_u4 *)(ks + pr * S::KR + 8 * ch) = kr[j];
      *(ac_u4 *)(vs + pr * S::VR + 8 * ch) = vr[j];
    }
    // scores for positions p0 + 16 t2 + r16, tokens 4kg + i
    ac_f4 sc[2];
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      ac_f4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < S::KS; ++s) {
        const ac_h8 b = *(const ac_h8 *)(ks + (16 * t2 + r16) * S::KR + 32 * s + 8 * kg);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[s], b, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[s], b, c, 0, 0, 0);
      }
      sc[t2] = c;
    }
    // the next tile's loads go out now (the registers above are consumed)
    const int next = kt + AC_WAVES;
    AC_LOAD_TILE(kr, vr, min(next, ntiles - 1));
    // online softmax per token row (register i), the row spread over 16 lanes.
    // A tile wholly below the block's first token's limit and the cache end
    // (most of them) needs no mask: the same values without the selects.
    float corr[4];
    const bool full = p0 + AC_KT - 1 <= pos0 + t0 && p0 + AC_KT <= kend;  // uniform
    if (full) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float mx = dpp_max16(__builtin_elementwise_maximum(sc[0][i], sc[1][i]));
        const float mn = __builtin_elementwise_maximum(m[i], mx);
        corr[i] = (m[i] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m[i] - mn);
        const float pv0 = __builtin_amdgcn_exp2f(sc[0][i] - mn);
        const float pv1 = __builtin_amdgcn_exp2f(sc[1][i] - mn);
        l[i] = l[i] * corr[i] + pv0 + pv1;  // this lane's columns; rows reduce at the end
        m[i] = mn;
        sc[0][i] = pv0;
        sc[1][i] = pv1;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int lim = pos0 + t0 + 4 * kg + i;  // last position this token attends
        float sv[2];
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          const int p = p0 + 16 * t2 + r16;
          sv[t2] = (p <= lim && p < kend) ? sc[t2][i] : -INFINITY;
        }
        const float mx = dpp_max16(__builtin_elementwise_maximum(sv[0], sv[1]));
        const float mn = __builtin_elementwise_maximum(m[i], mx);
        corr[i] = (m[i] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m[i] - mn);
        float pv[2];
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
          pv[t2] = (sv[t2] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sv[t2] - mn);
        l[i] = l[i] * corr[i] + pv[0] + pv[1];
        m[i] = mn;
        sc[0][i] = pv[0];
        sc[1][i] = pv[1];
      }
    }
    // P (hi, lo) to LDS as [pos][tok]: one 8-byte store per tile and part
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      uint16_t hv[4], lv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const _Float16 h = (_Float16)sc[t2][i];
        hv[i] = __builtin_bit_cast(uint16_t, h);
        lv[i] = __builtin_bit_cast(uint16_t, (_Float16)(sc[t2][i] - (float)h));
      }
      const int row = 16 * t2 + r16;
      *(uint2 *)(ph + row * S::PR + 4 * kg) =
          make_uint2(hv[0] | ((uint32_t)hv[1] << 16), hv[2] | ((uint32_t)hv[3] << 16));
      *(uint2 *)(pl + row * S::PR + 4 * kg) =
          make_uint2(lv[0] | ((uint32_t)lv[1] << 16), lv[2] | ((uint32_t)lv[3] << 16));
    }
    // O's rescale, skipped when no row's maximum moved in the whole wave
    // (every factor 1: the products would be exact copies).
    const bool same = corr[0] == 1.0f && corr[1] == 1.0f && corr[2] == 1.0f && corr[3] == 1.0f;
    if (!__all(same)) {  // some lane of the wave has a factor != 1
#pragma clang loop unroll(full)
      for (int t = 0; t < S::NT; ++t)
#pragma clang loop unroll(full)
        for (int i = 0; i < 4; ++i) o[t][i] *= corr[i];
    }
    // A operand: P[tok = r16][pos = 8kg + i]; source lane s reads row 8kg + s/4 (+4), cols 4(s%4)
    const int sr = 8 * kg + (r16 >> 2), sc4 = 4 * (r16 & 3);
    const ac_h8 pah = tr_pair(ph + sr * S::PR + sc4, ph + (sr + 4) * S::PR + sc4);
    const ac_h8 pal = tr_pair(pl + sr * S::PR + sc4, pl + (sr + 4) * S::PR + sc4);
#pragma clang loop unroll(full)
    for (int t = 0; t < S::NT; ++t) {
      // B operand: V[pos = 8kg + i][dim = 16t + r16]
      const ac_h8 bv = tr_pair(vs + sr * S::VR + 16 * t + sc4, vs + (sr + 4) * S::VR + 16 * t + sc4);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pah, bv, o[t], 0, 0, 0);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pal, bv, o[t], 0, 0, 0);
    }
    kt = next;
  }
#undef AC_LOAD_TILE

  // merge the waves: rows 4kg + i, per wave (m, l, O[row][HD])
  float *mb = (float *)vs;  // this wave's region, [16][HD + 2]
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lr = dpp_sum16(l[i]);
    const int row = 4 * kg + i;
    if (r16 == 0) {
      mb[row * (HD + 2)] = m[i];
      mb[row * (HD + 2) + 1] = lr;
    }
#pragma unroll
    for (int t = 0; t < S::NT; ++t) mb[row * (HD + 2) + 2 + 16 * t + r16] = o[t][i];
  }
  __syncthreads();
  const int rows = min(AC_TT, n - t0);
  for (int idx = tid; idx < rows * HD; idx += AC_WAVES * 64) {
    const int row = idx / HD, d = idx % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < AC_WAVES; ++w)
      M = fmaxf(M, ((const float *)(ac_lds + w * S::WAVE_HALVES))[row * (HD + 2)]);
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int w = 0; w < AC_WAVES; ++w) {
      const float *wb = (const float *)(ac_lds + w * S::WAVE_HALVES) + row * (HD + 2);
      const float f = (wb[0] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(wb[0] - M);  // base 2
      num = fmaf(wb[2 + d], f, num);
      den = fmaf(wb[1], f, den);
    }
    out[(size_t)(t0 + row) * n_q * HD + (size_t)head * HD + d] = f2h(num / den);
  }
}

template <int HD>
static void attn_chunk_mfma(const void *qkv, const void *k_cache, const void *v_cache, void *out,
                            int n_q, int n_kv, int pos0, int n, int max_seq, float scale) {
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void *)attn_chunk_mfma_kernel<HD>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, AcShape<HD>::LDS);
    attr = true;
  }
  const dim3 grid(n_q, (n + AC_TT - 1) / AC_TT);
  attn_chunk_mfma_kernel<HD><<<grid, AC_WAVES * 64, AcShape<HD>::LDS, WST_STREAM>>>(
      (const float *)qkv, (const uint16_t *)k_cache, (const uint16_t *)v_cache, (uint16_t *)out,
      n_q, n_kv, pos0, n, max_seq, scale);
}

extern "C" wst_status_t wst_attn_chunk(const void *qkv, const void *k_cache, const void *v_cache,
                                       void *out, int32_t n_q, int32_t n_kv, int32_t head_dim,
                                       int32_t pos0, int32_t n, int32_t max_seq, float scale) {
  WST_REQUIRE(qkv && k_cache && v_cache && out, "wst_attn_chunk: null pointer");
  WST_REQUIRE(n_q > 0 && n_kv > 0 && n_q % n_kv == 0 && n > 0 && n <= 65535,
              "wst_attn_chunk: bad shape");
  WST_REQUIRE(max_seq > 0 && pos0 >= 0 && pos0 + n <= max_seq,
              "wst_attn_chunk: chunk does not fit the cache");
  WST_REQUIRE(!(((uintptr_t)qkv | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15u),
              "wst_attn_chunk: qkv and the caches must be 16-byte aligned");
  // The MFMA kernel addresses a head's cache rows with 32-bit buffer offsets.
  WST_REQUIRE((int64_t)max_seq * head_dim * 2 < ((int64_t)1 << 31),
              "wst_attn_chunk: a head's cache rows exceed 2 GiB");
  const dim3 grid(n_q, n);
  switch (head_dim) {
    case 64:
      attn_chunk_mfma<64>(qkv, k_cache, v_cache, out, n_q, n_kv, pos0, n, max_seq, scale);
      break;
    case 128:
      attn_chunk_mfma<128>(qkv, k_cache, v_cache, out, n_q, n_kv, pos0, n, max_seq, scale);
      break;
    case 256:
      attn_chunk_kernel<256><<<grid, 256, 0, WST_STREAM>>>(
          (const float *)qkv, (const uint16_t *)k_cache, (const uint16_t *)v_cache,
          (uint16_t *)out, n_q, n_kv, pos0, max_seq, scale);
      break;
    default:
      WST_REQUIRE(false, "wst_attn_chunk: head_dim must be 64, 128 or 256");
  }
  WST_TRY_KERNEL("wst_attn_chunk");
  return WST_OK;
}
