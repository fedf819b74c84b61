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
// v_mfma_f32_16x16x32_f16, for head_dim 64 and 128, in transposed form:
// S^T = K . q^T and O^T = V^T . P^T, keys on the MFMA's M side and tokens on
// its N side.
// * One block per (query head, 16 TG query tokens), AC_WAVES waves; a wave
//   takes key tiles of 32 positions round-robin with its own online softmax
//   for all the block's tokens (TG groups of 16: one K fragment and one V^T
//   fragment feed TG MFMAs), and the waves merge once at the end through LDS.
// * A lane holds one token per group (r16) and eight of the tile's keys
//   (16 t2 + 4 kg + i): a token's softmax state (m, l) is one scalar per lane;
//   its tile maximum is a local maximum of eight and two cross-row swaps; one
//   rescale factor covers the lane's O^T column.
// * Scores: q (already rotated, times log2(e)/sqrt(hd), so the softmax is in
//   base 2) enters as its f16 hi part plus the f16 rounding of the rest, so
//   the products keep ~22 bits. K and V rows load coalesced (16-byte pieces,
//   a 128-byte row per eight lanes) into row-major LDS tiles; the next tile's
//   loads are issued before the current tile's softmax.
// * P^T never goes through LDS: the score accumulators, exponentiated and
//   rounded to f16, are the B operand of O^T = V^T . P^T as they stand, the
//   MFMA's K index k = 8 kg + j standing for key 4 kg + j
//   (j < 4) and 16 + 4 kg + j - 4 (j >= 4); the V^T operand is gathered in
//   that key order by the gfx950 transposing LDS read (ds_read_b64_tr_b16:
//   within 16 lanes, lane L's element i comes from lane 4i + L/4's element
//   L%4), rows 4 kg + s/4 and 16 + 4 kg + s/4 of the row-major V tile.
// * The reference maximum m moves only when a tile's maximum passes it by more
//   than 8 (base 2): the exponentials stay at most 2^8, far inside f16 and
//   f32, and O's rescale is rare instead of taken on almost every tile by
//   some token of the wave's. Softmax is exact for any reference point; only
//   roundings move.
// * P in one f16 (round to nearest, relative error <= 2^-11 per weight,
//   averaging over the keys) where q keeps its hi + lo parts: a score error
//   is an exponent error, a P error only a weight error, and the output is
//   rounded to f16 (2^-11) anyway. With P as f16 hi + lo too
//   (WST_ATTN_CHUNK_PLO=1, twice the P.V MFMAs and ~40 more VALU a tile)
//   0.5B 4096 tokens took 88.5 against 75.1 us, 7B 367 against 317 us, and
//   the chunked prefill's logits moved by nothing measurable (0.0068 and
//   0.0065 from the sequential prefill's, rescore off).
// Causality is a mask: token j keeps positions <= pos0 + j.
//
// A token's result does not depend on TG: its valid keys fall in the same
// tiles, taken by the same wave in the same order (a block's extra tiles are
// wholly masked for it: no term and no rescale), so TG is picked by the token
// count alone (WST_ATTN_CHUNK_TG=1|2 forces one).
//
// Measured (0.5B shape, 14/2 heads of 64, 4096 tokens from position 0): 75 us
// (400 TFLOP/s causal) with TG 2 (with P as hi + lo: 87 us; TG 1 106 us).
// The untransposed form (scores S = q . K^T, P through LDS, a row spread
// over 16 lanes, O's accumulators in AGPRs) took 142-187 us; K operands
// loaded straight from the cache instead of through LDS, 113-160 us.
typedef _Float16 ac_h8 __attribute__((ext_vector_type(8)));
typedef short ac_s4 __attribute__((ext_vector_type(4)));
typedef float ac_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t ac_u4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) ac_s4 ac_lds_s4;

#define AC_WAVES 4
#define AC_KT 32  // key positions per wave iteration

template <int HD, int TG>
struct AcShape {
  static constexpr int KS = HD / 32;              // k-steps of the scores
  static constexpr int NT = HD / 16;              // 16-dim output tiles
  static constexpr int VR = HD + 16;              // V row stride (halves)
  static constexpr int KR = HD + 8;               // K row stride (halves)
  static constexpr int VU = AC_KT * HD / 8 / 64;  // 16-byte K and V pieces per lane per tile
  static constexpr int TILES = AC_KT * VR + AC_KT * KR;
  static constexpr int MERGE = 16 * TG * (HD + 2) * 2;  // the merge rows (floats), in halves
  static constexpr int WAVE_HALVES = TILES > MERGE ? TILES : MERGE;
  static constexpr int LDS = AC_WAVES * WAVE_HALVES * 2;
};

// Eight halves as an MFMA operand from two transposing reads (rows r and r' of
// the 16-lane pattern each lane's address selects).
__device__ __forceinline__ ac_h8 tr_pair(const uint16_t *a0, const uint16_t *a1) {
  const ac_s4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((ac_lds_s4 *)a0);
  const ac_s4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((ac_lds_s4 *)a1);
  return __builtin_bit_cast(ac_h8, __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7));
}

__device__ __forceinline__ float row4_max(float v) {  // over the lanes r16 + 16 kg
  RowPair p = xrow16(v);
  v = __builtin_elementwise_maximum(p.a, p.b);
  p = xrow32(v);
  return __builtin_elementwise_maximum(p.a, p.b);
}

template <int HD, int TG, bool PLO = true>
__global__ __launch_bounds__(AC_WAVES * 64) void attn_chunk_mfma_kernel(
    const float *__restrict__ qkv, const uint16_t *__restrict__ k_cache,
    const uint16_t *__restrict__ v_cache, uint16_t *__restrict__ out, int n_q, int n_kv,
    int pos0, int n, int max_seq, float scale) {
  using S = AcShape<HD, TG>;
  constexpr int TT = 16 * TG;  // the block's tokens
  extern __shared__ __align__(16) uint16_t ac_lds[];
  // Token groups in reverse order: blocks are dispatched in index order, and
  // the last tokens attend to the most positions, so the longest blocks start
  // first and the short ones fill in behind them (a batched prefill's causal
  // work spans 16x between its first and last chunk).
  const int head = blockIdx.x, t0 = (gridDim.y - 1 - blockIdx.y) * TT;
  const int kvh = head / (n_q / n_kv);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the tile loop is scalar
  const int r16 = lane & 15, kg = lane >> 4;
  uint16_t *vs = ac_lds + wave * S::WAVE_HALVES;  // V tile [AC_KT][VR], row-major
  uint16_t *ks = vs + AC_KT * S::VR;              // K tile [AC_KT][KR], row-major
  const int stride_row = (n_q + 2 * n_kv) * HD;
  const uint16_t *kb = k_cache + (size_t)kvh * max_seq * HD;
  const uint16_t *vb = v_cache + (size_t)kvh * max_seq * HD;

  // q^T of token t0 + 16g + r16 as the B operand: dims 32s + 8kg + i, hi and
  // lo parts
  const float qscale = scale * 1.44269504088896340736f;
  ac_h8 qh[TG][S::KS], ql[TG][S::KS];
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    const float *q = qkv + (size_t)min(t0 + 16 * g + r16, n - 1) * stride_row + (size_t)head * HD;
#pragma unroll
    for (int s = 0; s < S::KS; ++s) {
      const float4 a = *(const float4 *)(q + 32 * s + 8 * kg);
      const float4 b = *(const float4 *)(q + 32 * s + 8 * kg + 4);
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = v[i] * qscale;
        const _Float16 h = (_Float16)x;
        qh[g][s][i] = h;
        ql[g][s][i] = (_Float16)(x - (float)h);
      }
    }
  }
  const int tlast = min(t0 + TT, n) - 1;
  const int kend = min(pos0 + tlast + 1, max_seq);  // positions [0, kend) are attended
  const int ntiles = (kend + AC_KT - 1) / AC_KT;

  // Loads of key tile kt as buffer loads over [0, kend) of the head's cache
  // rows. The whole byte offset (the lane's within the tile plus the tile's)
  // goes in the vector offset, which is the offset the buffer range check
  // compares with num_records, so positions at or past kend read zeros
  // whatever the cache holds there (their scores are masked, their P is zero),
  // and no load reaches past the allocation.
  const uint32_t kv_bytes = (uint32_t)kend * HD * 2u;
  // 0x00020000: word 3 of a raw gfx9 buffer resource (32-bit data format,
  // no swizzle); a load past kv_bytes returns zeros.
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void *)kb, 0, (int)kv_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void *)vb, 0, (int)kv_bytes, 0x00020000);
  const uint32_t voff = (uint32_t)((lane / (HD / 8)) * HD + 8 * (lane % (HD / 8))) * 2u;
  ac_u4 kr[S::VU], vr[S::VU];
  auto load_tile = [&](int kt) {
    const uint32_t so = (uint32_t)kt * (AC_KT * HD * 2);
#pragma unroll
    for (int j = 0; j < S::VU; ++j)
      kr[j] = __builtin_amdgcn_raw_buffer_load_b128(krs, so + voff + j * (64 / (HD / 8)) * HD * 2,
                                                    0, 0);
#pragma unroll
    for (int j = 0; j < S::VU; ++j)
      vr[j] = __builtin_amdgcn_raw_buffer_load_b128(vrs, so + voff + j * (64 / (HD / 8)) * HD * 2,
                                                    0, 0);
  };

  float m[TG], l[TG];  // per group: this lane's token; l over this lane's keys
  ac_f4 o[TG][S::NT];  // O^T: dims 16t + 4kg + i of token 16g + r16
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int t = 0; t < S::NT; ++t) o[g][t] = (ac_f4){0.0f, 0.0f, 0.0f, 0.0f};
  }

  int kt = wave;
  load_tile(min(kt, max(ntiles - 1, 0)));
  while (kt < ntiles) {
    const int p0 = kt * AC_KT;
    // K and V tiles into LDS (rows past kend hold zeros; their P is zero)
#pragma unroll
    for (int j = 0; j < S::VU; ++j) {
      const int u = lane + 64 * j, pr = u / (HD / 8), ch = u % (HD / 8);
      *(ac_u4 *)(ks + pr * S::KR + 8 * ch) = kr[j];
      *(ac_u4 *)(vs + pr * S::VR + 8 * ch) = vr[j];
    }
    // S^T for keys p0 + 16 t2 + 4kg + i, tokens 16g + r16; the A operand
    // (key 16 t2 + r16, dims 32s + 8kg + i) read once for every group
    ac_f4 sc[TG][2];
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
#pragma unroll
      for (int g = 0; g < TG; ++g) sc[g][t2] = (ac_f4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < S::KS; ++s) {
        const ac_h8 a = *(const ac_h8 *)(ks + (16 * t2 + r16) * S::KR + 32 * s + 8 * kg);
#pragma unroll
        for (int g = 0; g < TG; ++g) {
          sc[g][t2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[g][s], sc[g][t2], 0, 0, 0);
          sc[g][t2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[g][s], sc[g][t2], 0, 0, 0);
        }
      }
    }
    // the next tile's loads go out now (the registers above are consumed)
    load_tile(min(kt + AC_WAVES, ntiles - 1));
    // A tile wholly below the block's first token's limit and the cache end
    // (most of them) needs no mask.
    const bool full = p0 + AC_KT - 1 <= pos0 + t0 && p0 + AC_KT <= kend;  // uniform
    float corr[TG];
    ac_h8 pbh[TG], pbl[TG];
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      if (!full) {
        const int lim = pos0 + t0 + 16 * g + r16;  // the last position this token attends
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int p = p0 + 16 * t2 + 4 * kg + i;
            if (!(p <= lim && p < kend)) sc[g][t2][i] = -INFINITY;
          }
      }
#define AC_MAX(a, b) __builtin_elementwise_maximum(a, b)
      float mx = AC_MAX(AC_MAX(AC_MAX(sc[g][0][0], sc[g][0][1]), AC_MAX(sc[g][0][2], sc[g][0][3])),
                        AC_MAX(AC_MAX(sc[g][1][0], sc[g][1][1]), AC_MAX(sc[g][1][2], sc[g][1][3])));
#undef AC_MAX
      mx = row4_max(mx);
      // m moves only past m + 8; mx = -inf (no key of this token in the
      // tile) leaves it
      const bool bump = mx > m[g] + 8.0f;
      const float mn = bump ? mx : m[g];
      corr[g] = !bump ? 1.0f : (m[g] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m[g] - mn);
      // exp2(-inf - mref) = 0 for a masked score; mref is finite so that a
      // token with no key yet (mn = -inf) gets 0, not NaN
      const float mref = (mn == -INFINITY) ? 0.0f : mn;
      float pv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pv[j] = __builtin_amdgcn_exp2f(sc[g][j >> 2][j & 3] - mref);
      // P^T as the B operand (k = 8kg + j <-> key, above): one f16 each, or
      // (PLO) hi parts converted in pairs and lo parts
      float psum = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        psum += pv[j];
        psum += pv[j + 1];
        if constexpr (PLO) {
          const auto h2 = __builtin_amdgcn_cvt_pkrtz(pv[j], pv[j + 1]);
          pbh[g][j] = h2[0];
          pbh[g][j + 1] = h2[1];
          pbl[g][j] = (_Float16)(pv[j] - (float)h2[0]);
          pbl[g][j + 1] = (_Float16)(pv[j + 1] - (float)h2[1]);
        } else {
          pbh[g][j] = (_Float16)pv[j];
          pbh[g][j + 1] = (_Float16)pv[j + 1];
        }
      }
      l[g] = l[g] * corr[g] + psum;
      m[g] = mn;
    }
    // O's rescale, skipped when no token's factor in the wave moved (every
    // factor 1: the products would be exact copies)
    bool same = true;
#pragma unroll
    for (int g = 0; g < TG; ++g) same = same && corr[g] == 1.0f;
    if (!__all(same)) {
#pragma unroll
      for (int g = 0; g < TG; ++g)
#pragma clang loop unroll(full)
        for (int t = 0; t < S::NT; ++t)
#pragma clang loop unroll(full)
          for (int i = 0; i < 4; ++i) o[g][t][i] *= corr[g];
    }
    // V^T operand: lane s of a 16-lane group reads key rows 4kg + s/4 and
    // 16 + 4kg + s/4, dims 16t + 4(s%4); one read serves every group
    const int sr = 4 * kg + (r16 >> 2), sc4 = 4 * (r16 & 3);
#pragma clang loop unroll(full)
    for (int t = 0; t < S::NT; ++t) {
      const ac_h8 va =
          tr_pair(vs + sr * S::VR + 16 * t + sc4, vs + (sr + 16) * S::VR + 16 * t + sc4);
#pragma unroll
      for (int g = 0; g < TG; ++g) {
        o[g][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pbh[g], o[g][t], 0, 0, 0);
        if constexpr (PLO)
          o[g][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pbl[g], o[g][t], 0, 0, 0);
      }
    }
    kt += AC_WAVES;
  }

  // merge the waves: per wave (m, l, O[tok][HD]), rows 16g + r16
  float *mb = (float *)vs;  // this wave's region, [TT][HD + 2]
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    const int row = 16 * g + r16;
    const float lr = row4_sum(l[g]);
    if (kg == 0) {
      mb[row * (HD + 2)] = m[g];
      mb[row * (HD + 2) + 1] = lr;
    }
#pragma unroll
    for (int t = 0; t < S::NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) mb[row * (HD + 2) + 2 + 16 * t + 4 * kg + i] = o[g][t][i];
  }
  __syncthreads();
  const int rows = min(TT, n - t0);
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

template <int HD, int TG, bool PLO>
static void attn_chunk_mfma_tgp(const void *qkv, const void *k_cache, const void *v_cache,
                                void *out, int n_q, int n_kv, int pos0, int n, int max_seq,
                                float scale) {
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void *)attn_chunk_mfma_kernel<HD, TG, PLO>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, AcShape<HD, TG>::LDS);
    attr = true;
  }
  const dim3 grid(n_q, (n + 16 * TG - 1) / (16 * TG));
  attn_chunk_mfma_kernel<HD, TG, PLO><<<grid, AC_WAVES * 64, AcShape<HD, TG>::LDS, WST_STREAM>>>(
      (const float *)qkv, (const uint16_t *)k_cache, (const uint16_t *)v_cache, (uint16_t *)out,
      n_q, n_kv, pos0, n, max_seq, scale);
}
template <int HD, int TG>
static void attn_chunk_mfma_tg(const void *qkv, const void *k_cache, const void *v_cache,
                               void *out, int n_q, int n_kv, int pos0, int n, int max_seq,
                               float scale) {
  const char *v = getenv("WST_ATTN_CHUNK_PLO");  // 1: P as f16 hi + lo
  if (v && v[0] == '1')
    attn_chunk_mfma_tgp<HD, TG, true>(qkv, k_cache, v_cache, out, n_q, n_kv, pos0, n, max_seq,
                                      scale);
  else
    attn_chunk_mfma_tgp<HD, TG, false>(qkv, k_cache, v_cache, out, n_q, n_kv, pos0, n, max_seq,
                                       scale);
}

// Two groups of 16 tokens per wave from 512 tokens up (0.5B shape, 4096
// tokens: 87 against 106 us); one below (7B shape, 256 tokens: 10.0 against
// 11.7 us, the blocks twice as many).
template <int HD>
static void attn_chunk_mfma(const void *qkv, const void *k_cache, const void *v_cache, void *out,
                            int n_q, int n_kv, int pos0, int n, int max_seq, float scale) {
  const char *v = getenv("WST_ATTN_CHUNK_TG");
  const int tg = (v && (v[0] == '1' || v[0] == '2')) ? v[0] - '0' : (n >= 512 ? 2 : 1);
  if (tg == 2)
    attn_chunk_mfma_tg<HD, 2>(qkv, k_cache, v_cache, out, n_q, n_kv, pos0, n, max_seq, scale);
  else
    attn_chunk_mfma_tg<HD, 1>(qkv, k_cache, v_cache, out, n_q, n_kv, pos0, n, max_seq, scale);
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
