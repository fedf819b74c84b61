/* CPU oracle for the batch=1 int4-hier-g32 decode path. TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
 * this file, and only as the checker (or the timed CPU baseline). The product
 * library never links it.
 *
 * Compiled with -ffp-contract=off: every f32 expression below rounds after each
 * operation, exactly as Rust (which never contracts) does in the reference
 * quantiser. Citations are to the Whetstone source tree.
 *
 * Pinning (what checks each function; "parity unpinned" where nothing does):
 *   f16 conversion      exhaustive round trip + numpy float16 on random f32
 *   fixture normal      integer-exact definition, moments, GPU bit-exact
 *   fit_group           brute-force weighted least squares on tiny groups;
 *                       reference invariants (hier.rs:438-557)
 *   quantize/dequant    reference invariant tests restated; closed forms
 *   gemv                numpy float64 matmul of the dequantized matrix
 *   rmsnorm/swiglu/rope closed forms and numpy (decode_kernels.rs:31-126)
 *   attention           one position = v; two positions = explicit softmax
 *   argmax              planted index, low-index ties, negative ordering
 *   head ladder         reference rescore tests restated (rescore_kernels.rs)
 *   forward (textbook)  HF transformers Qwen2 in float64 on the same weights
 *   forward (mirrored)  textbook forward within fp16 tolerance
 *   dense f16 tables    (mirrored step) tables set to the f16 rounding of the
 *                       dequantised int4 ones give the int4 logits within f16
 *                       noise; the f16 GEMV by numpy float64 matmul
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------ f16 <-> f32 */

/* IEEE binary16 from f32, round to nearest even, with subnormals, overflow to
 * infinity and NaN kept quiet. This is the rounding `half` 2.7.1
 * (`f16::from_f32`, used throughout hier.rs) implements. */
uint16_t orc_f32_to_f16(float v) {
  uint32_t x;
  memcpy(&x, &v, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFFu) {
    if (man) return (uint16_t)(sign | 0x7E00u | (man >> 13)); /* NaN stays NaN */
    return (uint16_t)(sign | 0x7C00u);
  }
  const int e = (int)exp - 127 + 15;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u); /* overflow */
  if (e <= 0) {
    /* subnormal (or zero) in f16 */
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const int shift = 14 - e; /* 14..24 */
    uint32_t h = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* may carry into exp: correct */
  return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t x;
  if (exp == 0) {
    if (man == 0) {
      x = sign;
    } else {
      int e = -1;
      do {
        e++;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
    }
  } else if (exp == 0x1Fu) {
    x = sign | 0x7F800000u | (man << 13);
  } else {
    x = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

void orc_f32_to_f16_n(const float *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}
void orc_f16_to_f32_n(const uint16_t *src, float *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(src[i]);
}

/* f16 -> f32 through a 64K-entry table of orc_f16_to_f32's own results. */
static float g_h2f[65536];
static int g_h2f_ready = 0;
static void h2f_init(void) {
  for (uint32_t i = 0; i < 65536; ++i) g_h2f[i] = orc_f16_to_f32((uint16_t)i);
  __atomic_store_n(&g_h2f_ready, 1, __ATOMIC_RELEASE);
}
static inline float h2f(uint16_t h) {
  if (__builtin_expect(!__atomic_load_n(&g_h2f_ready, __ATOMIC_ACQUIRE), 0)) {
#pragma omp critical(orc_h2f_init)
    if (!g_h2f_ready) h2f_init();
  }
  return g_h2f[h];
}
static inline uint16_t f2h(float f) { return orc_f32_to_f16(f); }

/* ------------------------------------------------ arithmetic variants
 *
 * The default oracle evaluates every sum in f64 and rounds once at the
 * reference's narrowing points. The variants below exist to measure how much
 * the decode logits depend on choices the reference leaves to the kernel:
 *
 *   acc = ORC_ACC_F32_SEQ   every reduction (GEMV dot, RMSNorm and QK-norm
 *                           sums of squares, attention scores, softmax
 *                           denominator and P.V numerators) is an f32 sum in
 *                           ascending index order, as a scalar loop computes it
 *   acc = ORC_ACC_F32_LANE  the same f32 terms summed as 64 lane-strided
 *                           partials (term i to lane i % 64, ascending within a
 *                           lane) reduced by a halving tree, as a wave does
 *
 * The two f32 variants differ only in summation order; every term and every
 * other rounding is the same expression in both. xq = 1 rounds each group of
 * 32 int4-GEMV activations to the 14-bit fixed point of the GPU kernel's
 * activation table, X = rint(h * 2^(28-e)) * 2^(e-28) with e the f16 exponent
 * field of the group's largest |h| (clamped to 1..30). */
static int g_acc = ORC_ACC_F64;
static int g_xq = 0;

void orc_set_variant(int acc, int xq) {
  g_acc = acc;
  g_xq = xq;
}

static float sum_f32(const float *t, int64_t n) {
  if (g_acc == ORC_ACC_F32_SEQ) {
    float a = 0.0f;
    for (int64_t i = 0; i < n; ++i) a += t[i];
    return a;
  }
  float p[64];
  for (int i = 0; i < 64; ++i) p[i] = 0.0f;
  for (int64_t i = 0; i < n; ++i) p[i & 63] += t[i];
  for (int w = 32; w >= 1; w >>= 1)
    for (int i = 0; i < w; ++i) p[i] += p[i + w];
  return p[0];
}

/* The GPU activation table's value of each f16 activation (xq = 1). */
void orc_xq14(const uint16_t *x, int64_t n, double *out) {
  for (int64_t g = 0; g < n; g += 32) {
    const int64_t e_ = g + 32 < n ? g + 32 : n;
    uint16_t mx = 0;
    for (int64_t c = g; c < e_; ++c) {
      const uint16_t a = x[c] & 0x7FFFu;
      if (a > mx) mx = a;
    }
    int ef = mx >> 10;
    ef = ef < 1 ? 1 : (ef > 30 ? 30 : ef);
    const double sc = ldexp(1.0, ef - 28);
    for (int64_t c = g; c < e_; ++c) out[c] = (double)rintf(h2f(x[c]) * (float)ldexp(1.0, 28 - ef)) * sc;
  }
}

/* ------------------------------------------- ORC_ACC_REF: the reference's own
 * arithmetic on its CUDA build (acc = ORC_ACC_REF)
 *
 * Every reduction in the order and precision the reference's kernels compute
 * it, on a device with `g_ref_sms` multiprocessors (the attention split count
 * depends on it, attention.cu:201-218; default 30, the fallback the reference
 * itself uses and the RTX 2060 its README quotes):
 *
 *   int4 GEMV   gemv_hier.cu:91-163, hier.cuh:24-60: lane l of a 32-lane warp
 *               takes groups l, l+32, ...; per group an f16 x-sum (`__hadd2`:
 *               even and odd columns in two f16 lanes, 16 steps each, one RNE
 *               rounding per step), an f16 dot (`__hfma2` of (q-8) and x, 16
 *               steps per half, ONE rounding per step), both halves widened and
 *               added in f32, then fmaf(s, dot, acc), fmaf(fmaf(8,s,m), sx, acc);
 *               the lanes' partials summed by the xor butterfly (a halving tree)
 *   fp16 GEMV   gemv_int4.cu:194-229: lane l takes half2 pairs l, l+32, ...,
 *               two fmaf per pair, butterfly
 *   RMSNorm     decode.cu:46-100: n <= 1024: one element per thread of
 *               ceil(n/32)*32, x*x; else 256 threads, fmaf over i = t, t+256..;
 *               block_reduce_sum (common.cuh:149-161: butterfly per warp, warp
 *               sums through warp 0's butterfly); f16(x*inv*w)
 *   QK-norm     common.cuh:185-202: fmaf(x1,x1,x2*x2) per lane, block sum
 *   RoPE        decode.cu:150-174: x1*c - x2*s and x2*c + x1*s as nvcc
 *               contracts them (LLVM fuses the left product of an fsub/fadd:
 *               fmaf(x1,c,-(x2*s)), fmaf(x2,c,x1*s)) -- an assumption, nvcc's
 *               default -fmad=true leaves the form to the compiler
 *   attention   attention.cu:57-193: splits per pick_splits, 8 warps per split
 *               block, warp w takes positions t0+w, t0+w+8, ..., score by a
 *               per-lane fmaf chain over d = lane+32i and the butterfly, online
 *               softmax per warp, the block's warps merged in order, then the
 *               splits merged in order
 *   SwiGLU      decode.cu:240-242: f16((g * (1/(1+exp(-g)))) * u)
 *   rescore     head_rescore.cu:272-281: 256 threads, fmaf, block sum
 *   embedding   gemv_hier.cu:186: q*(d*ls) - dm*lm, contracted to
 *               fmaf(q, d*ls, -(dm*lm))
 *
 * Not restated: the reference's `__expf` and `rsqrtf` are hardware
 * approximations (a few ulp); ref_exp (f64 exp rounded to f32) and 1/sqrtf
 * stand in for them. Their
 * difference is a relative 1e-7-scale perturbation of single values, far below
 * the f16 roundings above. */
#define HGROUP 32
static int g_ref_sms = 30;

void orc_set_ref_sms(int sms) { g_ref_sms = sms > 0 ? sms : 30; }

/* exp for the REF mode: the f64 exponential rounded to f32 (correctly rounded
 * but for ties closer than 2^-29 relative), standing in for __expf. */
static inline float ref_exp(float x) { return (float)exp((double)x); }

/* IEEE binary16 round-to-nearest-even of a double (exact for the values the
 * f16 arithmetic below produces: multiples of 2^-24 far inside double's range). */
uint16_t orc_d2h(double v) {
  uint64_t b;
  memcpy(&b, &v, 8);
  const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
  const int ex = (int)((b >> 52) & 0x7FF);
  const uint64_t man = b & ((1ull << 52) - 1);
  if (ex == 0x7FF) return man ? (uint16_t)(sign | 0x7E00u) : (uint16_t)(sign | 0x7C00u);
  if (ex == 0) return sign; /* double subnormals are far below f16's half-ulp */
  const int e = ex - 1023;
  if (e > 15) return (uint16_t)(sign | 0x7C00u);
  const uint64_t m = man | (1ull << 52); /* value = m * 2^(e-52) */
  /* f16 quantum: 2^(e-10) for normals, 2^-24 below 2^-14 */
  const int qexp = (e >= -14 ? e : -14) - 10;
  const int shift = qexp - (e - 52); /* bits of m below the quantum */
  if (shift > 60) return sign;
  const uint64_t q = m >> shift, rem = m & ((1ull << shift) - 1), half = 1ull << (shift - 1);
  uint64_t r = q + ((rem > half || (rem == half && (q & 1))) ? 1 : 0);
  /* r is the magnitude in units of 2^qexp; f16 bits = biased exponent field
   * of the quantum's binade plus r, carry into the exponent included */
  uint32_t bits;
  if (qexp == -24) {
    bits = (uint32_t)r; /* subnormal (r == 1024 is the smallest normal) */
  } else {
    /* r in [1024, 2048]: (biased exponent e + 15) << 10 | (r - 1024) */
    bits = ((uint32_t)(e + 14) << 10) + (uint32_t)r;
  }
  if (bits >= 0x7C00u) return (uint16_t)(sign | 0x7C00u);
  return (uint16_t)(sign | bits);
}

/* __hadd / __hfma on one f16 lane: the exact result (every product and sum of
 * these f16 values is exact in double) rounded once. */
uint16_t orc_ref_hadd(uint16_t a, uint16_t b) {
  return orc_d2h((double)h2f(a) + (double)h2f(b));
}
uint16_t orc_ref_hfma(uint16_t a, uint16_t b, uint16_t c) {
  return orc_d2h((double)h2f(a) * (double)h2f(b) + (double)h2f(c));
}

/* The xor butterfly of warp_reduce_sum (common.cuh:127-132) as lane 0 sees it:
 * p[i] += p[i + off] for off = 16, 8, 4, 2, 1. */
static float ref_warp_sum(float *p) {
  for (int off = 16; off >= 1; off >>= 1)
    for (int i = 0; i < off; ++i) p[i] += p[i + off];
  return p[0];
}

/* block_reduce_sum (common.cuh:149-161) over `nthreads` per-thread values. */
static float ref_block_sum(const float *v, int nthreads) {
  const int nwarps = (nthreads + 31) / 32;
  float ws[32];
  for (int w = 0; w < nwarps; ++w) {
    float p[32];
    for (int l = 0; l < 32; ++l) p[l] = (w * 32 + l < nthreads) ? v[w * 32 + l] : 0.0f;
    ws[w] = ref_warp_sum(p);
  }
  float p[32];
  for (int l = 0; l < 32; ++l) p[l] = l < nwarps ? ws[l] : 0.0f;
  return ref_warp_sum(p);
}

/* f16 RNE of n * 2^-24 for an integer n (every f16 value, and every exact
 * sum or (q-8)*x product of them, is such a multiple); the result again in
 * units of 2^-24. *ovf is set when the f16 result would be infinite. */
static inline int64_t rnd16_units(int64_t n, int *ovf) {
  const uint64_t a = (uint64_t)(n < 0 ? -n : n);
  if (a < 2048u) return n; /* subnormals and the lowest binade: exact */
  const int sh = 53 - __builtin_clzll(a); /* bit length - 11 */
  const uint64_t q = a >> sh, rem = a & ((1ull << sh) - 1), half = 1ull << (sh - 1);
  const uint64_t r = (q + ((rem > half || (rem == half && (q & 1))) ? 1 : 0)) << sh;
  if (r >= (65520ull << 24)) *ovf = 1;
  return n < 0 ? -(int64_t)r : (int64_t)r;
}

/* The same row arithmetic as ref_gemv_row below on integer f16 images
 * (X[c] = x[c] * 2^24). A group's f16 x-sum and f16 dot do not depend on the
 * lane that computes them, so the x-sums (sx[g], shared by every row) and the
 * row's dots are formed first, four groups at a time for instruction-level
 * parallelism, then each lane folds its groups in the kernel's order. Returns 0
 * if an f16 partial overflowed. */
static void ref_xsums_units(const int64_t *X, int64_t groups, float *sx, int *ovf) {
  const float u = 0x1p-24f;
  for (int64_t v = 0; v < groups; ++v) {
    const int64_t *xg = X + v * HGROUP;
    int64_t xs0 = 0, xs1 = 0;
    for (int i = 0; i < 16; ++i) {
      xs0 = rnd16_units(xs0 + xg[2 * i], ovf);
      xs1 = rnd16_units(xs1 + xg[2 * i + 1], ovf);
    }
    sx[v] = (float)xs0 * u + (float)xs1 * u;
  }
}

static int ref_gemv_row_units(const uint32_t *qr, const uint8_t *sr, uint32_t sbw,
                              const int64_t *X, const float *sx, int64_t groups,
                              float *dot, float *out) {
  const float d = h2f((uint16_t)(sbw & 0xFFFFu));
  const float dm = h2f((uint16_t)(sbw >> 16));
  const float u = 0x1p-24f;
  int ovf = 0;
  for (int64_t v0 = 0; v0 < groups; v0 += 4) {
    const int nv = groups - v0 < 4 ? (int)(groups - v0) : 4;
    int64_t acc[4][2] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};
    for (int w = 0; w < 4; ++w)
      for (int i = 0; i < 4; ++i)
        for (int k = 0; k < nv; ++k) {
          const int64_t v = v0 + k;
          const uint32_t word = qr[v * 4 + w];
          const int64_t *xg = X + v * HGROUP;
          const int64_t q0 = (int64_t)((word >> (8 * i)) & 0xFu) - 8;
          const int64_t q1 = (int64_t)((word >> (8 * i + 4)) & 0xFu) - 8;
          acc[k][0] = rnd16_units(q0 * xg[8 * w + 2 * i] + acc[k][0], &ovf);
          acc[k][1] = rnd16_units(q1 * xg[8 * w + 2 * i + 1] + acc[k][1], &ovf);
        }
    for (int k = 0; k < nv; ++k) dot[v0 + k] = (float)acc[k][0] * u + (float)acc[k][1] * u;
  }
  if (ovf) return 0;
  float lanes[32];
  for (int lane = 0; lane < 32; ++lane) {
    float a = 0.0f;
    for (int64_t v = lane; v < groups; v += 32) {
      const uint8_t idx = sr[v];
      const float s = d * (float)(idx & 0xF);
      const float m = -dm * (float)(idx >> 4);
      a = fmaf(s, dot[v], a);
      a = fmaf(fmaf(8.0f, s, m), sx[v], a);
    }
    lanes[lane] = a;
  }
  *out = ref_warp_sum(lanes);
  return 1;
}

/* One row of gemv_int4_hier_kernel (gemv_hier.cu:118-163), lane partials
 * folded by the butterfly; x given as f16 bits. */
static float ref_gemv_row(const uint32_t *qr, const uint8_t *sr, uint32_t sbw,
                          const uint16_t *x, int64_t groups) {
  const float d = h2f((uint16_t)(sbw & 0xFFFFu));
  const float dm = h2f((uint16_t)(sbw >> 16));
  float acc[32];
  for (int lane = 0; lane < 32; ++lane) {
    float a = 0.0f;
    for (int64_t v = lane; v < groups; v += 32) {
      const uint16_t *xg = x + v * HGROUP;
      uint16_t xs0 = 0, xs1 = 0;
      for (int i = 0; i < 16; ++i) {
        xs0 = orc_ref_hadd(xs0, xg[2 * i]);
        xs1 = orc_ref_hadd(xs1, xg[2 * i + 1]);
      }
      const float sx = h2f(xs0) + h2f(xs1);
      const uint8_t idx = sr[v];
      const float s = d * (float)(idx & 0xF);
      const float m = -dm * (float)(idx >> 4);
      uint16_t d0 = 0, d1 = 0;
      for (int w = 0; w < 4; ++w) {
        const uint32_t word = qr[v * 4 + w];
        for (int i = 0; i < 4; ++i) {
          const double q0 = (double)((word >> (8 * i)) & 0xFu) - 8.0;
          const double q1 = (double)((word >> (8 * i + 4)) & 0xFu) - 8.0;
          d0 = orc_d2h(q0 * (double)h2f(xg[8 * w + 2 * i]) + (double)h2f(d0));
          d1 = orc_d2h(q1 * (double)h2f(xg[8 * w + 2 * i + 1]) + (double)h2f(d1));
        }
      }
      const float dotf = h2f(d0) + h2f(d1);
      a = fmaf(s, dotf, a);
      a = fmaf(fmaf(8.0f, s, m), sx, a);
    }
    acc[lane] = a;
  }
  return ref_warp_sum(acc);
}

/* attention.cu:201-218: slices per head such that 2 blocks per SM are busy,
 * at most 16, none thinner than the 8 warps of a split block. */
int orc_ref_attn_splits(int n_q, int max_seq) {
  int splits = (2 * g_ref_sms + n_q - 1) / n_q;
  if (splits < 1) splits = 1;
  if (splits > 16) splits = 16;
  while (splits > 1 && max_seq / splits < 8) splits--;
  return splits;
}

/* attention.cu:57-193 as the reference computes it (see the ORC_ACC_REF note). */
static void ref_attn_decode(const float *q, const uint16_t *k_cache, const uint16_t *v_cache,
                            uint16_t *out, int n_q, int gqa, int hd, int seq, int max_seq,
                            float scale) {
  const int splits = orc_ref_attn_splits(n_q, max_seq);
  const int epl = hd / 32, per = (seq + splits - 1) / splits;
  float *part = (float *)malloc((size_t)splits * (hd + 2) * sizeof(float));
  for (int h = 0; h < n_q; ++h) {
    const int kvh = h / gqa;
    const uint16_t *kb = k_cache + (size_t)kvh * max_seq * hd;
    const uint16_t *vb = v_cache + (size_t)kvh * max_seq * hd;
    float qs[1024];
    for (int i = 0; i < hd; ++i) qs[i] = q[(size_t)h * hd + i] * scale;
    for (int sp = 0; sp < splits; ++sp) {
      float *o = part + (size_t)sp * (hd + 2);
      const int t0 = sp * per, t1 = t0 + per < seq ? t0 + per : seq;
      if (t0 >= t1) {
        o[0] = -INFINITY;
        o[1] = 0.0f;
        for (int i = 0; i < hd; ++i) o[2 + i] = 0.0f;
        continue;
      }
      float m_s[8], l_s[8], acc_s[8][1024];
      for (int w = 0; w < 8; ++w) {
        float m = -INFINITY, l = 0.0f;
        for (int i = 0; i < hd; ++i) acc_s[w][i] = 0.0f;
        for (int t = t0 + w; t < t1; t += 8) {
          const uint16_t *kt = kb + (size_t)t * hd, *vt = vb + (size_t)t * hd;
          float p[32];
          for (int lane = 0; lane < 32; ++lane) {
            float a = 0.0f;
            for (int i = 0; i < epl; ++i) a = fmaf(qs[lane + 32 * i], h2f(kt[lane + 32 * i]), a);
            p[lane] = a;
          }
          const float sc = ref_warp_sum(p);
          const float m_new = fmaxf(m, sc);
          const float corr = ref_exp(m - m_new);
          const float pr = ref_exp(sc - m_new);
          for (int d = 0; d < hd; ++d) acc_s[w][d] = fmaf(pr, h2f(vt[d]), acc_s[w][d] * corr);
          l = fmaf(l, corr, pr);
          m = m_new;
        }
        m_s[w] = m;
        l_s[w] = l;
      }
      float M = -INFINITY;
      for (int w = 0; w < 8; ++w) M = fmaxf(M, m_s[w]);
      for (int d = 0; d < hd; ++d) {
        float num = 0.0f;
        for (int w = 0; w < 8; ++w) num = fmaf(acc_s[w][d], ref_exp(m_s[w] - M), num);
        o[2 + d] = num;
      }
      float den = 0.0f;
      for (int w = 0; w < 8; ++w) den = fmaf(l_s[w], ref_exp(m_s[w] - M), den);
      o[0] = M;
      o[1] = den;
    }
    /* attn_merge_kernel, attention.cu:172-193 */
    float M = -INFINITY;
    for (int sp = 0; sp < splits; ++sp) M = fmaxf(M, part[(size_t)sp * (hd + 2)]);
    for (int d = 0; d < hd; ++d) {
      float num = 0.0f, den = 0.0f;
      for (int sp = 0; sp < splits; ++sp) {
        const float *pp = part + (size_t)sp * (hd + 2);
        const float f = ref_exp(pp[0] - M);
        num = fmaf(pp[2 + d], f, num);
        den = fmaf(pp[1], f, den);
      }
      out[(size_t)h * hd + d] = f2h(num / den);
    }
  }
  free(part);
}

/* ---------------------------------------------------- fixture generator */

/* splitmix64 (Steele, Lea, Flood 2014): the published finaliser. */
uint64_t orc_splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

/* Sum of twelve 16-bit uniforms, re-centred: an integer N in [-393210, 393210]
 * with mean 0 and variance 65536^2 (Irwin-Hall(12) has variance 1). The value
 * is f32(N) * 2^-16 * std, one rounding, so any IEEE machine reproduces it. */
float orc_fixture_normal(uint64_t seed, uint64_t stream, uint64_t index, float std_) {
  /* Element j = 3*index + k of the splitmix64 sequence keyed by (seed, stream). */
  const uint64_t key = orc_splitmix64(seed ^ orc_splitmix64(stream + 0x632BE59BD9B4E019ull));
  int64_t s = 0;
  for (uint64_t k = 0; k < 3; ++k) {
    const uint64_t h = orc_splitmix64(key + (index * 3u + k) * 0x9E3779B97F4A7C15ull);
    s += (int64_t)(h & 0xFFFFu) + (int64_t)((h >> 16) & 0xFFFFu) +
         (int64_t)((h >> 32) & 0xFFFFu) + (int64_t)(h >> 48);
  }
  const int32_t n = (int32_t)(s * 2 + 12 - 12 * 65536); /* 2*(S + 6 - 6*65536) */
  /* n/2 is the centred sum in units of 2^-16; n * 2^-17 is exact in f32. */
  return ((float)n * 7.62939453125e-06f) * std_;
}

void orc_fixture_normal_n(uint64_t seed, uint64_t stream, uint64_t index0, float std_,
                          float *out, size_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
  for (size_t i = 0; i < n; ++i) out[i] = orc_fixture_normal(seed, stream, index0 + i, std_);
}

/* ------------------------------------------------------ int4-hier-g32 */

#define QMAX 15.0f
#define SMAX 15.0f

/* Rust's saturating float->int cast: NaN -> 0, clamps to the target range. */
static inline uint32_t rust_as_u(float v, float hi) {
  if (isnan(v)) return 0;
  if (v <= 0.0f) return 0;
  if (v >= hi) return (uint32_t)hi;
  return (uint32_t)v;
}

/* Rust f32::clamp(lo, hi): NaN stays NaN. */
static inline float rclamp(float v, float lo, float hi) {
  if (v < lo) v = lo;
  if (v > hi) v = hi;
  return v;
}

/* make_qkx2_quants fit of one group: crates/whetstone-quant/src/hier.rs:113-195.
 * Sequential f32 sums in index order, f32::round = roundf (half away from 0). */
void orc_fit_group(const float *x, int n_, float *out_scale, float *out_min) {
  const int NSTEP = 20;
  const float RMIN = -1.0f, RDELTA = 0.1f;
  const float n = (float)n_;

  float ss = 0.0f;
  for (int i = 0; i < n_; ++i) ss = ss + x[i] * x[i];
  const float av = sqrtf(ss / n);

  float lo = INFINITY, hi = -INFINITY;
  for (int i = 0; i < n_; ++i) lo = fminf(lo, x[i]);
  lo = fminf(lo, 0.0f);
  for (int i = 0; i < n_; ++i) hi = fmaxf(hi, x[i]);
  const float rng = hi - lo;
  if (!isfinite(rng) || rng <= 0.0f) {
    *out_scale = 0.0f;
    *out_min = fminf(lo, 0.0f);
    return;
  }

  float w[64];
  for (int i = 0; i < n_; ++i) w[i] = av + fabsf(x[i]);
  float sum_w = 0.0f, sum_x = 0.0f;
  for (int i = 0; i < n_; ++i) sum_w = sum_w + w[i];
  for (int i = 0; i < n_; ++i) sum_x = sum_x + w[i] * x[i];

  float best_scale = rng / QMAX;
  float best_min = lo;
  float best_err = 0.0f;
  {
    const float s = best_scale;
    for (int i = 0; i < n_; ++i) {
      const float q = rclamp(roundf((x[i] - lo) / s), 0.0f, QMAX);
      const float d = q * s + lo - x[i];
      best_err = best_err + w[i] * d * d;
    }
  }

  for (int step = 0; step <= NSTEP; ++step) {
    const float iscale = (QMAX + RMIN + RDELTA * (float)step) / rng;
    float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
    float lvl[64];
    for (int i = 0; i < n_; ++i) {
      const float l = rclamp(roundf(iscale * (x[i] - lo)), 0.0f, QMAX);
      lvl[i] = l;
      sum_l = sum_l + w[i] * l;
      sum_l2 = sum_l2 + w[i] * l * l;
      sum_xl = sum_xl + w[i] * l * x[i];
    }
    const float det = sum_w * sum_l2 - sum_l * sum_l;
    if (det <= 0.0f) continue;
    float scale = (sum_w * sum_xl - sum_x * sum_l) / det;
    float mn = (sum_l2 * sum_x - sum_l * sum_xl) / det;
    if (mn > 0.0f) {
      mn = 0.0f;
      scale = (sum_l2 > 0.0f) ? sum_xl / sum_l2 : scale;
    }
    float err = 0.0f;
    for (int i = 0; i < n_; ++i) {
      const float d = scale * lvl[i] + mn - x[i];
      err = err + w[i] * d * d;
    }
    if (err < best_err) {
      best_err = err;
      best_scale = scale;
      best_min = mn;
    }
  }
  *out_scale = best_scale;
  *out_min = best_min;
}

/* hier.rs:219-233 */
uint16_t orc_shared_scale(float v) {
  if (isnan(v) || v <= 0.0f) return f2h(1.0f);
  const uint16_t h = f2h(v);
  if (h2f(h) > 0.0f) {
    if ((h & 0x7C00u) != 0x7C00u) return h;
    return 0x7BFFu; /* f16::MAX */
  }
  return 1u; /* smallest positive subnormal */
}

/* hier.rs:250-303 */
static void pack_row(const float *row, int64_t groups, float *ss, float *sm, uint32_t *qw_row,
                     uint8_t *si_row, uint32_t *sb_row, double *num, double *den) {
  float max_scale = 0.0f, max_min = 0.0f;
  for (int64_t g = 0; g < groups; ++g) {
    float s, m;
    orc_fit_group(row + g * HGROUP, HGROUP, &s, &m);
    ss[g] = s;
    sm[g] = m;
    max_scale = fmaxf(max_scale, s);
    max_min = fmaxf(max_min, -m);
  }
  const uint16_t d = orc_shared_scale(max_scale > 0.0f ? max_scale / SMAX : 1.0f);
  const int dm_pos = max_min > 0.0f;
  const uint16_t dm = orc_shared_scale(dm_pos ? max_min / SMAX : 1.0f);
  *sb_row = (uint32_t)d | ((uint32_t)dm << 16);
  const float df = h2f(d), dmf = h2f(dm);

  for (int64_t g = 0; g < groups; ++g) {
    const uint32_t ls = rust_as_u(rclamp(roundf(ss[g] / df), 1.0f, SMAX), 255.0f);
    uint32_t lm = 0;
    if (dm_pos) lm = rust_as_u(rclamp(roundf(fmaxf(-sm[g], 0.0f) / dmf), 0.0f, SMAX), 255.0f);
    si_row[g] = (uint8_t)(ls | (lm << 4));
    const float s = df * (float)(uint8_t)ls;
    const float m = -dmf * (float)(uint8_t)lm;
    for (int i = 0; i < HGROUP; ++i) {
      const int64_t col = g * HGROUP + i;
      const float v = row[col];
      const float qf = rclamp(roundf((v - m) / s), 0.0f, QMAX);
      const uint32_t q = rust_as_u(qf, 4294967295.0f);
      qw_row[col / 8] |= q << (4 * (col % 8));
      const double e = (double)(v - (qf * s + m));
      *num += e * e;
      *den += (double)v * (double)v;
    }
  }
}

/* hier.rs:351-391 */
int orc_quantize_int4_hier(const float *w, int64_t in_f, int64_t out_f, uint32_t *qw,
                           uint8_t *si, uint32_t *sb, double *err2_out, double *ref2_out) {
  if (in_f <= 0 || out_f <= 0 || in_f % HGROUP != 0) return 5;
  const int64_t groups = in_f / HGROUP, words = in_f / 8;
  memset(qw, 0, (size_t)(out_f * words) * 4);
  double num = 0.0, den = 0.0;
#pragma omp parallel reduction(+ : num, den)
  {
    float *ss = (float *)malloc((size_t)groups * sizeof(float));
    float *sm = (float *)malloc((size_t)groups * sizeof(float));
#pragma omp for schedule(dynamic, 16)
    for (int64_t r = 0; r < out_f; ++r)
      pack_row(w + r * in_f, groups, ss, sm, qw + r * words, si + r * groups, sb + r, &num,
               &den);
    free(ss);
    free(sm);
  }
  if (err2_out) *err2_out = num;
  if (ref2_out) *ref2_out = den;
  return 0;
}

/* hier.rs:398-421: s = d*ls, m = -dm*lm, w = q*s + m, two f32 roundings. */
void orc_dequantize_row(const uint32_t *qw, const uint8_t *si, const uint32_t *sb,
                        int64_t in_f, int64_t row, float *dst) {
  const int64_t groups = in_f / HGROUP, words = in_f / 8;
  const uint32_t sbw = sb[row];
  const float d = h2f((uint16_t)(sbw & 0xFFFFu));
  const float dm = h2f((uint16_t)(sbw >> 16));
  const uint32_t *qr = qw + row * words;
  const uint8_t *sr = si + row * groups;
  for (int64_t g = 0; g < groups; ++g) {
    const uint8_t idx = sr[g];
    const float s = d * (float)(idx & 0xF);
    const float m = -dm * (float)(idx >> 4);
    for (int i = 0; i < HGROUP; ++i) {
      const int64_t col = g * HGROUP + i;
      const float q = (float)((qr[col / 8] >> (4 * (col % 8))) & 0xFu);
      dst[col] = q * s + m;
    }
  }
}

void orc_dequantize_int4_hier(const uint32_t *qw, const uint8_t *si, const uint32_t *sb,
                              int64_t in_f, int64_t out_f, float *out) {
#pragma omp parallel for schedule(static) if (out_f * in_f > 65536)
  for (int64_t r = 0; r < out_f; ++r) orc_dequantize_row(qw, si, sb, in_f, r, out + r * in_f);
}

/* ------------------------------------------------------------ decode ops */

/* The GEMV's contract: gemv_hier.cu:70-163 computes, per row,
 *   y = (accum ? y : 0) + (dot + bias)
 * where dot = sum_c dequant(w)[c] * x[c]. The oracle evaluates dot in f64 from
 * the exact f32 dequantized weights (hier.rs:398-421) and f16 x. */
void orc_gemv_int4_hier(const uint32_t *qw, const uint8_t *si, const uint32_t *sb,
                        const uint16_t *x, const uint16_t *bias, float *y, int64_t in_f,
                        int64_t out_f, int accum) {
  if (g_acc == ORC_ACC_REF) {
    const int64_t groups = in_f / HGROUP;
    int64_t *X = (int64_t *)malloc((size_t)in_f * sizeof(int64_t));
    float *sx = (float *)malloc((size_t)groups * sizeof(float));
    int finite = 1, ovf = 0;
    for (int64_t c = 0; c < in_f; ++c) {
      finite &= (x[c] & 0x7C00u) != 0x7C00u;
      X[c] = finite ? (int64_t)ldexp((double)h2f(x[c]), 24) : 0;
    }
    if (finite) ref_xsums_units(X, groups, sx, &ovf);
    const int fast = finite && !ovf;
#pragma omp parallel
    {
      float *dot = (float *)malloc((size_t)groups * sizeof(float));
#pragma omp for schedule(static)
      for (int64_t r = 0; r < out_f; ++r) {
        float rr;
        if (!fast ||
            !ref_gemv_row_units(qw + r * (in_f / 8), si + r * groups, sb[r], X, sx, groups, dot, &rr))
          rr = ref_gemv_row(qw + r * (in_f / 8), si + r * groups, sb[r], x, groups);
        if (bias) rr += h2f(bias[r]);
        y[r] = accum ? y[r] + rr : rr;
      }
      free(dot);
    }
    free(X);
    free(sx);
    return;
  }
  double *xd = (double *)malloc((size_t)in_f * sizeof(double));
  if (g_xq)
    orc_xq14(x, in_f, xd);
  else
    for (int64_t c = 0; c < in_f; ++c) xd[c] = (double)h2f(x[c]);
#pragma omp parallel
  {
    float *row = (float *)malloc((size_t)in_f * sizeof(float));
    float *t = (float *)malloc((size_t)in_f * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < out_f; ++r) {
      orc_dequantize_row(qw, si, sb, in_f, r, row);
      float rr;
      if (g_acc != ORC_ACC_F64) {
        for (int64_t c = 0; c < in_f; ++c) t[c] = row[c] * (float)xd[c];
        rr = sum_f32(t, in_f);
        if (bias) rr += h2f(bias[r]);
      } else {
        double acc = 0.0;
        for (int64_t c = 0; c < in_f; ++c) acc += (double)row[c] * xd[c];
        if (bias) acc += (double)h2f(bias[r]);
        rr = (float)acc;
      }
      y[r] = accum ? y[r] + rr : rr;
    }
    free(row);
    free(t);
  }
  free(xd);
}

/* gemv_int4.cu:194-229 (fp16 weights), same epilogue. */
void orc_gemv_fp16(const uint16_t *w, const uint16_t *x, const uint16_t *bias, float *y,
                   int64_t in_f, int64_t out_f, int accum) {
  if (g_acc == ORC_ACC_REF) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < out_f; ++r) {
      const uint16_t *wr = w + r * in_f;
      float p[32];
      for (int lane = 0; lane < 32; ++lane) {
        float a = 0.0f;
        for (int64_t c = lane; c < in_f / 2; c += 32) {
          a = fmaf(h2f(wr[2 * c]), h2f(x[2 * c]), a);
          a = fmaf(h2f(wr[2 * c + 1]), h2f(x[2 * c + 1]), a);
        }
        p[lane] = a;
      }
      float rr = ref_warp_sum(p);
      if (bias) rr += h2f(bias[r]);
      y[r] = accum ? y[r] + rr : rr;
    }
    return;
  }
#pragma omp parallel
  {
    float *t = (float *)malloc((size_t)in_f * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < out_f; ++r) {
      float rr;
      if (g_acc != ORC_ACC_F64) {
        for (int64_t c = 0; c < in_f; ++c) t[c] = h2f(w[r * in_f + c]) * h2f(x[c]);
        rr = sum_f32(t, in_f);
        if (bias) rr += h2f(bias[r]);
      } else {
        double acc = 0.0;
        for (int64_t c = 0; c < in_f; ++c) acc += (double)h2f(w[r * in_f + c]) * (double)h2f(x[c]);
        if (bias) acc += (double)h2f(bias[r]);
        rr = (float)acc;
      }
      y[r] = accum ? y[r] + rr : rr;
    }
    free(t);
  }
}

/* decode.cu:46-82: out = f16(x * rsqrt(mean(x^2) + eps) * w). */
void orc_rmsnorm(const float *x, const uint16_t *w, uint16_t *out, int n, float eps) {
  if (g_acc == ORC_ACC_REF) {
    const int T = n <= 1024 ? (n + 31) / 32 * 32 : 256;
    float *t = (float *)calloc((size_t)T, sizeof(float));
    if (n <= 1024) {
      for (int i = 0; i < n; ++i) t[i] = x[i] * x[i];
    } else {
      for (int th = 0; th < T; ++th)
        for (int i = th; i < n; i += T) t[th] = fmaf(x[i], x[i], t[th]);
    }
    const float inv = 1.0f / sqrtf(ref_block_sum(t, T) / (float)n + eps);
    for (int i = 0; i < n; ++i) out[i] = f2h(x[i] * inv * h2f(w[i]));
    free(t);
    return;
  }
  if (g_acc != ORC_ACC_F64) {
    float *t = (float *)malloc((size_t)n * sizeof(float));
    for (int i = 0; i < n; ++i) t[i] = x[i] * x[i];
    const float inv = 1.0f / sqrtf(sum_f32(t, n) / (float)n + eps);
    for (int i = 0; i < n; ++i) out[i] = f2h(x[i] * inv * h2f(w[i]));
    free(t);
    return;
  }
  double ss = 0.0;
  for (int i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
  const double inv = 1.0 / sqrt(ss / (double)n + (double)eps);
  for (int i = 0; i < n; ++i) out[i] = f2h((float)((double)x[i] * inv * (double)h2f(w[i])));
}

/* decode.rs:95-147 (no scaling): invf = theta^(-j/half) in f64, angle p*invf in
 * f64, cos/sin narrowed to f32. Layout [max_seq][half]. */
void orc_rope_table(int max_seq, int head_dim, double theta, float *cos_tab, float *sin_tab) {
  const int half = head_dim / 2;
  for (int j = 0; j < half; ++j) {
    const double invf = pow(theta, -(double)j / (double)half);
    for (int p = 0; p < max_seq; ++p) {
      const double a = (double)p * invf;
      cos_tab[(size_t)p * half + j] = (float)cos(a);
      sin_tab[(size_t)p * half + j] = (float)sin(a);
    }
  }
}

/* common.cuh:185-202: per-head RMS over hd entries, shared gain [hd]. */
static void qk_norm_head(double *v, int hd, const uint16_t *g, float eps) {
  if (g_acc != ORC_ACC_F64) {
    float t[1024];
    for (int i = 0; i < hd; ++i) t[i] = (float)v[i] * (float)v[i];
    const float inv = 1.0f / sqrtf(sum_f32(t, hd) / (float)hd + eps);
    for (int i = 0; i < hd; ++i) v[i] = (double)((float)v[i] * inv * h2f(g[i]));
    return;
  }
  double ss = 0.0;
  for (int i = 0; i < hd; ++i) ss += v[i] * v[i];
  const double inv = 1.0 / sqrt(ss / (double)hd + (double)eps);
  for (int i = 0; i < hd; ++i) v[i] = v[i] * inv * (double)h2f(g[i]);
}

/* decode.cu:112-178: optional QK-norm, then half rotation of q (in place) and
 * k (into the f16 cache at [kvh][pos][hd]); v copied to the f16 cache. */
void orc_rope_cache(float *qkv, uint16_t *k_cache, uint16_t *v_cache, const float *cos_tab,
                    const float *sin_tab, int n_q, int n_kv, int hd, int pos, int max_seq,
                    const uint16_t *q_norm_w, const uint16_t *k_norm_w, float eps) {
  const int half = hd / 2;
  if (pos < 0) pos = 0;
  if (pos > max_seq - 1) pos = max_seq - 1;
  const float *c = cos_tab + (size_t)pos * half;
  const float *s = sin_tab + (size_t)pos * half;
  if (g_acc == ORC_ACC_REF) {
    const int T = (half + 31) / 32 * 32;
    for (int h = 0; h < n_q + n_kv; ++h) {
      float *src = qkv + (size_t)h * hd;
      float x1[512], x2[512], t[544];
      for (int j = 0; j < half; ++j) {
        x1[j] = src[j];
        x2[j] = src[j + half];
      }
      const uint16_t *g = h < n_q ? q_norm_w : k_norm_w;
      if (g) {
        for (int j = 0; j < T; ++j) t[j] = j < half ? fmaf(x1[j], x1[j], x2[j] * x2[j]) : 0.0f;
        const float inv = 1.0f / sqrtf(ref_block_sum(t, T) / (float)hd + eps);
        for (int j = 0; j < half; ++j) {
          x1[j] = x1[j] * inv * h2f(g[j]);
          x2[j] = x2[j] * inv * h2f(g[j + half]);
        }
      }
      float r[1024];
      for (int j = 0; j < half; ++j) {
        r[j] = fmaf(x1[j], c[j], -(x2[j] * s[j]));
        r[j + half] = fmaf(x2[j], c[j], x1[j] * s[j]);
      }
      if (h < n_q) {
        for (int i = 0; i < hd; ++i) src[i] = r[i];
      } else {
        const int kvh = h - n_q;
        const size_t slot = ((size_t)kvh * max_seq + pos) * hd;
        const float *vv = qkv + (size_t)(n_q + n_kv + kvh) * hd;
        for (int i = 0; i < hd; ++i) {
          k_cache[slot + i] = f2h(r[i]);
          v_cache[slot + i] = f2h(vv[i]);
        }
      }
    }
    return;
  }
  double v[1024];
  for (int h = 0; h < n_q + n_kv; ++h) {
    float *src = qkv + (size_t)h * hd;
    for (int i = 0; i < hd; ++i) v[i] = (double)src[i];
    const uint16_t *g = h < n_q ? q_norm_w : k_norm_w;
    if (g) qk_norm_head(v, hd, g, eps);
    float r[1024];
    for (int j = 0; j < half; ++j) {
      r[j] = (float)(v[j] * (double)c[j] - v[j + half] * (double)s[j]);
      r[j + half] = (float)(v[j + half] * (double)c[j] + v[j] * (double)s[j]);
    }
    if (h < n_q) {
      for (int i = 0; i < hd; ++i) src[i] = r[i];
    } else {
      const int kvh = h - n_q;
      const size_t slot = ((size_t)kvh * max_seq + pos) * hd;
      const float *vv = qkv + (size_t)(n_q + n_kv + kvh) * hd;
      for (int i = 0; i < hd; ++i) {
        k_cache[slot + i] = f2h(r[i]);
        v_cache[slot + i] = f2h(vv[i]);
      }
    }
  }
}

/* attention.cu:57-193: q scaled by `scale` (in f32, once), softmax over the
 * seq = min(pos+1, max_seq) cached positions of kv head h/(n_q/n_kv), f16 out. */
void orc_attn_decode(const float *q, const uint16_t *k_cache, const uint16_t *v_cache,
                     uint16_t *out, int n_q, int n_kv, int hd, int pos, int max_seq,
                     float scale) {
  int seq = (pos < 0 ? 0 : pos) + 1;
  if (seq > max_seq) seq = max_seq;
  const int gqa = n_q / n_kv;
  if (g_acc == ORC_ACC_REF) {
    ref_attn_decode(q, k_cache, v_cache, out, n_q, gqa, hd, seq, max_seq, scale);
    return;
  }
  if (g_acc != ORC_ACC_F64) {
    float *e = (float *)malloc((size_t)seq * sizeof(float));
    float *t = (float *)malloc((size_t)(seq > hd ? seq : hd) * sizeof(float));
    for (int h = 0; h < n_q; ++h) {
      const int kvh = h / gqa;
      float qs[1024];
      for (int i = 0; i < hd; ++i) qs[i] = q[(size_t)h * hd + i] * scale;
      float m = -INFINITY;
      for (int p = 0; p < seq; ++p) {
        const uint16_t *kt = k_cache + ((size_t)kvh * max_seq + p) * hd;
        for (int i = 0; i < hd; ++i) t[i] = qs[i] * h2f(kt[i]);
        e[p] = sum_f32(t, hd);
        if (e[p] > m) m = e[p];
      }
      for (int p = 0; p < seq; ++p) e[p] = expf(e[p] - m);
      const float den = sum_f32(e, seq);
      for (int i = 0; i < hd; ++i) {
        for (int p = 0; p < seq; ++p)
          t[p] = e[p] * h2f(v_cache[((size_t)kvh * max_seq + p) * hd + i]);
        out[(size_t)h * hd + i] = f2h(sum_f32(t, seq) / den);
      }
    }
    free(e);
    free(t);
    return;
  }
  /* Heads are independent: one per thread, each summing in the same order. */
#pragma omp parallel if (seq * hd > 65536)
  {
    double *sc = (double *)malloc((size_t)seq * sizeof(double));
#pragma omp for schedule(static)
    for (int h = 0; h < n_q; ++h) {
      const int kvh = h / gqa;
      double qs[1024], num[1024];
      for (int i = 0; i < hd; ++i) qs[i] = (double)(q[(size_t)h * hd + i] * scale);
      double m = -INFINITY;
      for (int t = 0; t < seq; ++t) {
        const uint16_t *kt = k_cache + ((size_t)kvh * max_seq + t) * hd;
        double a = 0.0;
        for (int i = 0; i < hd; ++i) a += qs[i] * (double)h2f(kt[i]);
        sc[t] = a;
        if (a > m) m = a;
      }
      double den = 0.0;
      for (int t = 0; t < seq; ++t) {
        sc[t] = exp(sc[t] - m);
        den += sc[t];
      }
      /* num[i] = sum_t sc[t] * v[t][i], t ascending for every i */
      for (int i = 0; i < hd; ++i) num[i] = 0.0;
      for (int t = 0; t < seq; ++t) {
        const uint16_t *vt = v_cache + ((size_t)kvh * max_seq + t) * hd;
        for (int i = 0; i < hd; ++i) num[i] += sc[t] * (double)h2f(vt[i]);
      }
      for (int i = 0; i < hd; ++i) out[(size_t)h * hd + i] = f2h((float)(num[i] / den));
    }
    free(sc);
  }
}

/* decode.cu:235-242: out = f16(g * sigmoid(g) * u), g = first half. */
void orc_swiglu(const float *gate_up, uint16_t *out, int n) {
  if (g_acc == ORC_ACC_REF) {
    for (int i = 0; i < n; ++i) {
      const float g = gate_up[i];
      out[i] = f2h(g * (1.0f / (1.0f + ref_exp(-g))) * gate_up[i + n]);
    }
    return;
  }
  for (int i = 0; i < n; ++i) {
    const double g = gate_up[i], u = gate_up[i + n];
    out[i] = f2h((float)(g / (1.0 + exp(-g)) * u));
  }
}

/* sample.cu:28-37: order-preserving key, value high, complemented index low. */
uint64_t orc_argmax_key(float v, int32_t idx) {
  uint32_t b;
  memcpy(&b, &v, 4);
  const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)k << 32) | (uint64_t)(~(uint32_t)idx);
}

/* sample.cu:39-88: max key over all entries; index = ~low32. */
int32_t orc_argmax(const float *logits, int n) {
  uint64_t best = 0;
  for (int i = 0; i < n; ++i) {
    const uint64_t k = orc_argmax_key(logits[i], i);
    if (k > best) best = k;
  }
  return (int32_t)(~(uint32_t)(best & 0xFFFFFFFFu));
}

/* head_rescore.cu:62-180: max, counts for 12 rungs 2^c/64, pick the smallest
 * rung with count >= k, step down while count > cap, thresh = max - margin. */
float orc_head_threshold(const float *logits, int n, int k, int cap, int32_t *count,
                         int32_t *rung) {
  float mx = -INFINITY;
  for (int i = 0; i < n; ++i) mx = fmaxf(mx, logits[i]);
  int32_t counts[12] = {0};
  for (int i = 0; i < n; ++i) {
    const float d = mx - logits[i];
    for (int c = 0; c < 12; ++c)
      if (d <= 0.015625f * (float)(1 << c)) counts[c]++;
  }
  int pick = 11;
  for (int c = 0; c < 12; ++c)
    if (counts[c] >= k) {
      pick = c;
      break;
    }
  while (pick > 0 && counts[pick] > cap) --pick;
  const float thresh = mx - 0.015625f * (float)(1 << pick);
  int32_t cnt = 0;
  for (int i = 0; i < n; ++i)
    if (!(logits[i] < thresh)) cnt++;
  if (count) *count = cnt;
  if (rung) *rung = pick;
  return thresh;
}

/* head_rescore.cu:215-284: every logit >= thresh recomputed as the f32 result of
 * the fp16 head row dotted with the fp16 x (f64 inside here). */
void orc_head_rescore(const uint16_t *head, const uint16_t *x, float *logits, int n,
                      int hidden, float thresh) {
  for (int r = 0; r < n; ++r) {
    if (logits[r] < thresh) continue;
    if (g_acc == ORC_ACC_REF) {
      float t[256];
      for (int th = 0; th < 256; ++th) {
        t[th] = 0.0f;
        for (int i = th; i < hidden; i += 256)
          t[th] = fmaf(h2f(head[(size_t)r * hidden + i]), h2f(x[i]), t[th]);
      }
      logits[r] = ref_block_sum(t, 256);
      continue;
    }
    double acc = 0.0;
    for (int i = 0; i < hidden; ++i)
      acc += (double)h2f(head[(size_t)r * hidden + i]) * (double)h2f(x[i]);
    logits[r] = (float)acc;
  }
}

/* ----------------------------------------------------------- the model */

typedef struct {
  uint32_t *qw;
  uint8_t *si;
  uint32_t *sb;
  int64_t in_f, out_f;
} hmat_t;

typedef struct {
  hmat_t qkv, o, gate_up, down;
  uint16_t *qkv_bias; /* [(nq+2nkv)hd] or NULL */
  uint16_t *in_norm, *post_norm; /* [H] */
  uint16_t *q_norm, *k_norm;     /* [hd] or NULL */
} layer_t;

struct orc_model {
  orc_config_t c;
  hmat_t embed, lm_head; /* lm_head.qw == NULL when tied */
  uint16_t *final_norm;
  uint16_t *rescore; /* [V][H] fp16 copy of the head, or NULL */
  /* Dense f16 [V][H] embedding / output projection (a converted model's fp16
   * tables, model.rs Embedding::Fp16 and DeviceLinear::Fp16), or NULL. Used by
   * the mirrored step only. */
  uint16_t *embed16, *head16;
  layer_t *layers;
};

/* embed_int4_hier_kernel (gemv_hier.cu:168-189): q*(d*ls) - dm*lm, as nvcc
 * contracts it (ORC_ACC_REF only; the default keeps hier.rs's two roundings). */
static void ref_embed_row(const hmat_t *e, int64_t row, float *dst) {
  const int64_t in_f = e->in_f, groups = in_f / HGROUP, words = in_f / 8;
  const uint32_t sbw = e->sb[row];
  const float d = h2f((uint16_t)(sbw & 0xFFFFu));
  const float dm = h2f((uint16_t)(sbw >> 16));
  for (int64_t c = 0; c < in_f; ++c) {
    const float q = (float)((e->qw[row * words + c / 8] >> (4 * (c % 8))) & 0xFu);
    const uint8_t idx = e->si[row * groups + c / HGROUP];
    dst[c] = fmaf(q, d * (float)(idx & 0xF), -(dm * (float)(idx >> 4)));
  }
}

/* Fixture streams: one per (layer, tensor); the GPU generator uses the same. */
enum { ST_Q = 0, ST_K = 1, ST_V = 2, ST_O = 3, ST_GATE = 4, ST_UP = 5, ST_DOWN = 6,
       ST_QN = 7, ST_KN = 8 };
#define STREAM(l, t) ((uint64_t)(l) * 16u + (uint64_t)(t) + 16u)
#define ST_EMBED 1u
#define ST_HEAD 2u

static void hmat_alloc(hmat_t *m, int64_t in_f, int64_t out_f) {
  m->in_f = in_f;
  m->out_f = out_f;
  m->qw = (uint32_t *)calloc((size_t)(out_f * in_f / 8), 4);
  m->si = (uint8_t *)calloc((size_t)(out_f * in_f / 32), 1);
  m->sb = (uint32_t *)calloc((size_t)out_f, 4);
}
static void hmat_free(hmat_t *m) {
  free(m->qw);
  free(m->si);
  free(m->sb);
}

/* Packs rows [row0, row0+rows) of `m` from stream `st` (rows of that tensor
 * start at 0), chunked so host memory stays bounded. */
static void pack_part(hmat_t *m, int64_t row0, int64_t rows, uint64_t seed, uint64_t st,
                      float *fp16_copy_dst_unused) {
  (void)fp16_copy_dst_unused;
  const int64_t in_f = m->in_f, chunk = 4096;
  float *buf = (float *)malloc((size_t)(chunk * in_f) * sizeof(float));
  for (int64_t r = 0; r < rows; r += chunk) {
    const int64_t nr = rows - r < chunk ? rows - r : chunk;
    orc_fixture_normal_n(seed, st, (uint64_t)(r * in_f), 0.02f, buf, (size_t)(nr * in_f));
    const int64_t R = row0 + r;
    orc_quantize_int4_hier(buf, in_f, nr, m->qw + R * (in_f / 8), m->si + R * (in_f / 32),
                           m->sb + R, NULL, NULL);
  }
  free(buf);
}

static uint16_t *f16_fill(size_t n, float v) {
  uint16_t *p = (uint16_t *)malloc(n * 2);
  const uint16_t h = f2h(v);
  for (size_t i = 0; i < n; ++i) p[i] = h;
  return p;
}

static orc_model_t *model_build(const orc_config_t *cfg, uint64_t seed, int pack);

orc_model_t *orc_model_synthetic(const orc_config_t *cfg, uint64_t seed) {
  return model_build(cfg, seed, 1);
}

orc_model_t *orc_model_alloc(const orc_config_t *cfg, uint64_t seed) {
  return model_build(cfg, seed, 0);
}

static orc_model_t *model_build(const orc_config_t *cfg, uint64_t seed, int pack) {
  orc_model_t *m = (orc_model_t *)calloc(1, sizeof(orc_model_t));
  m->c = *cfg;
  const orc_config_t *c = cfg;
  const int64_t H = c->hidden, hd = c->head_dim, I = c->inter, V = c->vocab;
  const int64_t nq = (int64_t)c->n_q * hd, nk = (int64_t)c->n_kv * hd;

  hmat_alloc(&m->embed, H, V);
  if (pack) pack_part(&m->embed, 0, V, seed, ST_EMBED, NULL);
  if (!c->tied) {
    hmat_alloc(&m->lm_head, H, V);
    if (pack) pack_part(&m->lm_head, 0, V, seed, ST_HEAD, NULL);
  }
  m->final_norm = f16_fill((size_t)H, 1.0f);
  if (c->rescore_k > 0) {
    m->rescore = (uint16_t *)malloc((size_t)(V * H) * 2);
    const uint64_t st = c->tied ? ST_EMBED : ST_HEAD;
    float *buf = (float *)malloc((size_t)H * sizeof(float));
    for (int64_t r = 0; r < V; ++r) {
      orc_fixture_normal_n(seed, st, (uint64_t)(r * H), 0.02f, buf, (size_t)H);
      orc_f32_to_f16_n(buf, m->rescore + r * H, (size_t)H);
    }
    free(buf);
  }
  m->layers = (layer_t *)calloc((size_t)c->n_layers, sizeof(layer_t));
  for (int l = 0; l < c->n_layers; ++l) {
    layer_t *L = &m->layers[l];
    hmat_alloc(&L->qkv, H, nq + 2 * nk);
    if (pack) pack_part(&L->qkv, 0, nq, seed, STREAM(l, ST_Q), NULL);
    if (pack) pack_part(&L->qkv, nq, nk, seed, STREAM(l, ST_K), NULL);
    if (pack) pack_part(&L->qkv, nq + nk, nk, seed, STREAM(l, ST_V), NULL);
    hmat_alloc(&L->o, nq, H);
    if (pack) pack_part(&L->o, 0, H, seed, STREAM(l, ST_O), NULL);
    hmat_alloc(&L->gate_up, H, 2 * I);
    if (pack) pack_part(&L->gate_up, 0, I, seed, STREAM(l, ST_GATE), NULL);
    if (pack) pack_part(&L->gate_up, I, I, seed, STREAM(l, ST_UP), NULL);
    hmat_alloc(&L->down, I, H);
    if (pack) pack_part(&L->down, 0, H, seed, STREAM(l, ST_DOWN), NULL);
    L->qkv_bias = c->qkv_bias ? f16_fill((size_t)(nq + 2 * nk), 0.0f) : NULL;
    L->in_norm = f16_fill((size_t)H, 1.0f);
    L->post_norm = f16_fill((size_t)H, 1.0f);
    if (c->qk_norm) {
      float g[1024];
      L->q_norm = (uint16_t *)malloc((size_t)hd * 2);
      L->k_norm = (uint16_t *)malloc((size_t)hd * 2);
      orc_fixture_normal_n(seed, STREAM(l, ST_QN), 0, 0.02f, g, (size_t)hd);
      for (int64_t i = 0; i < hd; ++i) L->q_norm[i] = f2h(1.0f + g[i]);
      orc_fixture_normal_n(seed, STREAM(l, ST_KN), 0, 0.02f, g, (size_t)hd);
      for (int64_t i = 0; i < hd; ++i) L->k_norm[i] = f2h(1.0f + g[i]);
    }
  }
  return m;
}

void orc_model_free(orc_model_t *m) {
  if (!m) return;
  hmat_free(&m->embed);
  hmat_free(&m->lm_head);
  free(m->final_norm);
  free(m->rescore);
  free(m->embed16);
  free(m->head16);
  for (int l = 0; l < m->c.n_layers; ++l) {
    layer_t *L = &m->layers[l];
    hmat_free(&L->qkv);
    hmat_free(&L->o);
    hmat_free(&L->gate_up);
    hmat_free(&L->down);
    free(L->qkv_bias);
    free(L->in_norm);
    free(L->post_norm);
    free(L->q_norm);
    free(L->k_norm);
  }
  free(m->layers);
  free(m);
}

static hmat_t *find_mat(orc_model_t *m, const char *name) {
  if (strcmp(name, "embed") == 0) return &m->embed;
  if (strcmp(name, "lm_head") == 0) return m->c.tied ? &m->embed : &m->lm_head;
  int l = 0;
  char what[32];
  if (sscanf(name, "L%d.%31s", &l, what) == 2 && l >= 0 && l < m->c.n_layers) {
    layer_t *L = &m->layers[l];
    if (strcmp(what, "qkv") == 0) return &L->qkv;
    if (strcmp(what, "o") == 0) return &L->o;
    if (strcmp(what, "gate_up") == 0) return &L->gate_up;
    if (strcmp(what, "down") == 0) return &L->down;
  }
  return NULL;
}

int orc_model_tensor(orc_model_t *m, const char *name, const uint32_t **qw,
                     const uint8_t **si, const uint32_t **sb, int64_t *in_f, int64_t *out_f) {
  hmat_t *h = find_mat(m, name);
  if (!h) return 2;
  *qw = h->qw;
  *si = h->si;
  *sb = h->sb;
  *in_f = h->in_f;
  *out_f = h->out_f;
  return 0;
}

/* Replaces the embedding ("embed") or the output projection ("head") by a dense
 * f16 [vocab][hidden] table (copied). With a tied model the embedding table
 * also serves as the head. Returns 0, or -1 for an unknown name. */
int orc_model_set_dense(orc_model_t *m, const char *which, const uint16_t *table) {
  const size_t n = (size_t)m->c.vocab * (size_t)m->c.hidden;
  uint16_t **dst = strcmp(which, "embed") == 0 ? &m->embed16
                   : strcmp(which, "head") == 0 ? &m->head16
                                                : NULL;
  if (!dst) return -1;
  free(*dst);
  *dst = (uint16_t *)malloc(n * 2);
  memcpy(*dst, table, n * 2);
  return 0;
}

const uint16_t *orc_model_fp16(orc_model_t *m, const char *name, int64_t *n) {
  const int64_t H = m->c.hidden, hd = m->c.head_dim;
  if (strcmp(name, "final_norm") == 0) {
    *n = H;
    return m->final_norm;
  }
  if (strcmp(name, "rescore") == 0) {
    *n = m->rescore ? (int64_t)m->c.vocab * H : 0;
    return m->rescore;
  }
  int l = 0;
  char what[32];
  if (sscanf(name, "L%d.%31s", &l, what) == 2 && l >= 0 && l < m->c.n_layers) {
    layer_t *L = &m->layers[l];
    if (strcmp(what, "in_norm") == 0) { *n = H; return L->in_norm; }
    if (strcmp(what, "post_norm") == 0) { *n = H; return L->post_norm; }
    if (strcmp(what, "q_norm") == 0) { *n = L->q_norm ? hd : 0; return L->q_norm; }
    if (strcmp(what, "k_norm") == 0) { *n = L->k_norm ? hd : 0; return L->k_norm; }
    if (strcmp(what, "qkv_bias") == 0) {
      *n = L->qkv_bias ? (int64_t)(m->c.n_q + 2 * m->c.n_kv) * hd : 0;
      return L->qkv_bias;
    }
  }
  *n = 0;
  return NULL;
}

/* ------------------------------------------------------- decode state */

struct orc_state {
  const orc_model_t *m;
  int max_seq, mode, pos;
  int n_layers; /* kept so the state can be freed after its model */
  uint16_t **kc, **vc;  /* mode 0: f16 caches per layer */
  double **kd, **vd;    /* mode 1: f64 caches per layer */
  float *cos_tab, *sin_tab;
};

orc_state_t *orc_state_new(const orc_model_t *m, int max_seq, int mode) {
  orc_state_t *s = (orc_state_t *)calloc(1, sizeof(orc_state_t));
  s->m = m;
  s->max_seq = max_seq;
  s->mode = mode;
  s->n_layers = m->c.n_layers;
  const orc_config_t *c = &m->c;
  const size_t n = (size_t)c->n_kv * max_seq * c->head_dim;
  if (mode == 0) {
    s->kc = (uint16_t **)calloc((size_t)c->n_layers, sizeof(void *));
    s->vc = (uint16_t **)calloc((size_t)c->n_layers, sizeof(void *));
    for (int l = 0; l < c->n_layers; ++l) {
      s->kc[l] = (uint16_t *)calloc(n, 2);
      s->vc[l] = (uint16_t *)calloc(n, 2);
    }
  } else {
    s->kd = (double **)calloc((size_t)c->n_layers, sizeof(void *));
    s->vd = (double **)calloc((size_t)c->n_layers, sizeof(void *));
    for (int l = 0; l < c->n_layers; ++l) {
      s->kd[l] = (double *)calloc(n, 8);
      s->vd[l] = (double *)calloc(n, 8);
    }
  }
  const size_t t = (size_t)max_seq * (c->head_dim / 2);
  s->cos_tab = (float *)malloc(t * 4);
  s->sin_tab = (float *)malloc(t * 4);
  orc_rope_table(max_seq, c->head_dim, c->rope_theta, s->cos_tab, s->sin_tab);
  return s;
}

void orc_state_free(orc_state_t *s) {
  if (!s) return;
  for (int l = 0; l < s->n_layers; ++l) {
    if (s->kc) { free(s->kc[l]); free(s->vc[l]); }
    if (s->kd) { free(s->kd[l]); free(s->vd[l]); }
  }
  free(s->kc); free(s->vc); free(s->kd); free(s->vd);
  free(s->cos_tab); free(s->sin_tab);
  free(s);
}

int orc_state_pos(const orc_state_t *s) { return s->pos; }
void orc_state_set_pos(orc_state_t *s, int pos) { s->pos = pos; }

/* Synthetic context: cache entry (layer l, kv head h, position t, dim i) is
 * f16(N(0,1)) from stream 1000+l, index ((h*2 + {0:k,1:v}) * max_pos + t) * hd + i
 * with max_pos = 1<<20, so the values do not depend on the cache capacity. */
void orc_state_fill_kv(orc_state_t *s, uint64_t seed, int n) {
  const orc_config_t *c = &s->m->c;
  const int hd = c->head_dim;
  for (int l = 0; l < c->n_layers; ++l)
    for (int h = 0; h < c->n_kv; ++h)
      for (int kv = 0; kv < 2; ++kv)
        for (int t = 0; t < n && t < s->max_seq; ++t) {
          const uint64_t base = (((uint64_t)(h * 2 + kv) << 20) + (uint64_t)t) * (uint64_t)hd;
          for (int i = 0; i < hd; ++i) {
            const uint16_t v = f2h(orc_fixture_normal(seed, 1000u + (uint64_t)l, base + i, 1.0f));
            const size_t at = ((size_t)h * s->max_seq + t) * hd + i;
            if (s->mode == 0) {
              (kv ? s->vc[l] : s->kc[l])[at] = v;
            } else {
              (kv ? s->vd[l] : s->kd[l])[at] = (double)h2f(v);
            }
          }
        }
}

/* f64 GEMV on the dequantized matrix with an f64 input (textbook mode). */
static void gemv_f64(const hmat_t *w, const double *x, double *y) {
  const int64_t in_f = w->in_f;
#pragma omp parallel
  {
    float *row = (float *)malloc((size_t)in_f * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < w->out_f; ++r) {
      orc_dequantize_row(w->qw, w->si, w->sb, in_f, r, row);
      double acc = 0.0;
      for (int64_t c = 0; c < in_f; ++c) acc += (double)row[c] * x[c];
      y[r] = acc;
    }
    free(row);
  }
}

static void rms_f64(const double *x, const uint16_t *w, double *out, int n, float eps) {
  double ss = 0.0;
  for (int i = 0; i < n; ++i) ss += x[i] * x[i];
  const double inv = 1.0 / sqrt(ss / (double)n + (double)eps);
  for (int i = 0; i < n; ++i) out[i] = x[i] * inv * (double)h2f(w[i]);
}

/* One decode step.
 * Mode 0 restates Engine::step_eager (crates/whetstone-core/src/engine.rs:512-572)
 * with the kernels' storage types: x f32, h f16, qkv f32, KV f16, attn f16,
 * gate_up f32, act f16, logits f32.
 * Mode 1 is the same order in f64 with no narrowing (the textbook forward of
 * bench/reference_numpy.py:148-194, made incremental with an f64 KV cache). */
int32_t orc_step(orc_state_t *s, int32_t token, float *logits_out) {
  const orc_model_t *m = s->m;
  const orc_config_t *c = &m->c;
  const int H = c->hidden, hd = c->head_dim, nq = c->n_q, nkv = c->n_kv, I = c->inter,
            V = c->vocab;
  const int nqkv = (nq + 2 * nkv) * hd;
  const hmat_t *head = c->tied ? &m->embed : &m->lm_head;
  int pos = s->pos;
  if (pos > s->max_seq - 1) pos = s->max_seq - 1;
  if (token < 0) token = 0;
  if (token > V - 1) token = V - 1;
  const float scale = (float)(1.0 / sqrt((double)hd));
  float *logits = logits_out;

  if (s->mode == 0) {
    float *x = (float *)malloc((size_t)H * 4);
    uint16_t *h = (uint16_t *)malloc((size_t)H * 2);
    float *qkv = (float *)malloc((size_t)nqkv * 4);
    uint16_t *attn = (uint16_t *)malloc((size_t)nq * hd * 2);
    float *gu = (float *)malloc((size_t)2 * I * 4);
    uint16_t *act = (uint16_t *)malloc((size_t)I * 2);
    if (m->embed16) {  /* decode.cu:259-268: the f16 row widened to f32 */
      for (int i = 0; i < H; ++i) x[i] = h2f(m->embed16[(size_t)token * H + i]);
    } else if (g_acc == ORC_ACC_REF) {
      ref_embed_row(&m->embed, token, x);
    } else {
      orc_dequantize_row(m->embed.qw, m->embed.si, m->embed.sb, H, token, x);
    }
    for (int l = 0; l < c->n_layers; ++l) {
      const layer_t *L = &m->layers[l];
      orc_rmsnorm(x, L->in_norm, h, H, c->eps);
      orc_gemv_int4_hier(L->qkv.qw, L->qkv.si, L->qkv.sb, h, L->qkv_bias, qkv, H, nqkv, 0);
      orc_rope_cache(qkv, s->kc[l], s->vc[l], s->cos_tab, s->sin_tab, nq, nkv, hd, pos,
                     s->max_seq, L->q_norm, L->k_norm, c->eps);
      orc_attn_decode(qkv, s->kc[l], s->vc[l], attn, nq, nkv, hd, pos, s->max_seq, scale);
      orc_gemv_int4_hier(L->o.qw, L->o.si, L->o.sb, attn, NULL, x, nq * hd, H, 1);
      orc_rmsnorm(x, L->post_norm, h, H, c->eps);
      orc_gemv_int4_hier(L->gate_up.qw, L->gate_up.si, L->gate_up.sb, h, NULL, gu, H, 2 * I, 0);
      orc_swiglu(gu, act, I);
      orc_gemv_int4_hier(L->down.qw, L->down.si, L->down.sb, act, NULL, x, I, H, 1);
    }
    orc_rmsnorm(x, m->final_norm, h, H, c->eps);
    const uint16_t *head16 = c->tied ? m->embed16 : m->head16;
    if (head16)
      orc_gemv_fp16(head16, h, NULL, logits, H, V, 0);
    else
      orc_gemv_int4_hier(head->qw, head->si, head->sb, h, NULL, logits, H, V, 0);
    if (m->rescore && c->rescore_k > 0) {
      const int k = c->rescore_k;
      int cap = 16 * k;
      if (cap > V) cap = V;
      if (cap < k) cap = k;
      int32_t cnt = 0;
      const float th = orc_head_threshold(logits, V, k, cap, &cnt, NULL);
      if (cnt <= cap) orc_head_rescore(m->rescore, h, logits, V, H, th);
    }
    free(x); free(h); free(qkv); free(attn); free(gu); free(act);
  } else {
    double *x = (double *)malloc((size_t)H * 8);
    double *h = (double *)malloc((size_t)H * 8);
    double *qkv = (double *)malloc((size_t)nqkv * 8);
    double *attn = (double *)malloc((size_t)nq * hd * 8);
    double *gu = (double *)malloc((size_t)2 * I * 8);
    double *act = (double *)malloc((size_t)I * 8);
    double *tmp = (double *)malloc((size_t)(H > V ? H : V) * 8);
    double *sc = (double *)malloc((size_t)s->max_seq * 8);
    {
      float *row = (float *)malloc((size_t)H * 4);
      orc_dequantize_row(m->embed.qw, m->embed.si, m->embed.sb, H, token, row);
      for (int i = 0; i < H; ++i) x[i] = row[i];
      free(row);
    }
    const int half = hd / 2;
    for (int l = 0; l < c->n_layers; ++l) {
      const layer_t *L = &m->layers[l];
      rms_f64(x, L->in_norm, h, H, c->eps);
      gemv_f64(&L->qkv, h, qkv);
      if (L->qkv_bias)
        for (int i = 0; i < nqkv; ++i) qkv[i] += (double)h2f(L->qkv_bias[i]);
      for (int hh = 0; hh < nq + nkv; ++hh) {
        double *v = qkv + (size_t)hh * hd;
        const uint16_t *g = hh < nq ? L->q_norm : L->k_norm;
        if (g) qk_norm_head(v, hd, g, c->eps);
        double r[1024];
        for (int j = 0; j < half; ++j) {
          const double invf = pow(c->rope_theta, -(double)j / (double)half);
          const double a = (double)pos * invf, cs = cos(a), sn = sin(a);
          r[j] = v[j] * cs - v[j + half] * sn;
          r[j + half] = v[j + half] * cs + v[j] * sn;
        }
        if (hh < nq) {
          memcpy(v, r, (size_t)hd * 8);
        } else {
          const int kvh = hh - nq;
          const size_t slot = ((size_t)kvh * s->max_seq + pos) * hd;
          memcpy(s->kd[l] + slot, r, (size_t)hd * 8);
          memcpy(s->vd[l] + slot, qkv + (size_t)(nq + nkv + kvh) * hd, (size_t)hd * 8);
        }
      }
      const int seq = pos + 1, gqa = nq / nkv;
      const double dscale = 1.0 / sqrt((double)hd);
      for (int hh = 0; hh < nq; ++hh) {
        const int kvh = hh / gqa;
        double mx = -INFINITY;
        for (int t = 0; t < seq; ++t) {
          const double *kt = s->kd[l] + ((size_t)kvh * s->max_seq + t) * hd;
          double a = 0.0;
          for (int i = 0; i < hd; ++i) a += qkv[(size_t)hh * hd + i] * kt[i];
          sc[t] = a * dscale;
          if (sc[t] > mx) mx = sc[t];
        }
        double den = 0.0;
        for (int t = 0; t < seq; ++t) { sc[t] = exp(sc[t] - mx); den += sc[t]; }
        for (int i = 0; i < hd; ++i) {
          double num = 0.0;
          for (int t = 0; t < seq; ++t)
            num += sc[t] * s->vd[l][((size_t)kvh * s->max_seq + t) * hd + i];
          attn[(size_t)hh * hd + i] = num / den;
        }
      }
      gemv_f64(&L->o, attn, tmp);
      for (int i = 0; i < H; ++i) x[i] += tmp[i];
      rms_f64(x, L->post_norm, h, H, c->eps);
      gemv_f64(&L->gate_up, h, gu);
      for (int i = 0; i < I; ++i) act[i] = gu[i] / (1.0 + exp(-gu[i])) * gu[i + I];
      gemv_f64(&L->down, act, tmp);
      for (int i = 0; i < H; ++i) x[i] += tmp[i];
    }
    rms_f64(x, m->final_norm, h, H, c->eps);
    gemv_f64(head, h, tmp);
    for (int i = 0; i < V; ++i) logits[i] = (float)tmp[i];
    free(x); free(h); free(qkv); free(attn); free(gu); free(act); free(tmp); free(sc);
  }
  s->pos = s->pos + 1 < s->max_seq ? s->pos + 1 : s->max_seq;
  return orc_argmax(logits, V);
}

/* bench/reference_numpy.py:148-194, restated: the whole sequence recomputed,
 * f64 everywhere, cos/sin from f64 angles, causal softmax, last-position logits.
 * Weights are the dequantized int4-hier matrices (hier.rs:398-421). */
void orc_forward_full(const orc_model_t *m, const int32_t *ids, int n, double *logits_out) {
  const orc_config_t *c = &m->c;
  const int H = c->hidden, hd = c->head_dim, nq = c->n_q, nkv = c->n_kv, I = c->inter,
            V = c->vocab, half = hd / 2;
  const int nqkv = (nq + 2 * nkv) * hd;
  double *x = (double *)calloc((size_t)n * H, 8);
  double *h = (double *)calloc((size_t)n * H, 8);
  double *qkv = (double *)calloc((size_t)n * nqkv, 8);
  double *ctx = (double *)calloc((size_t)n * nq * hd, 8);
  double *gu = (double *)calloc((size_t)n * 2 * I, 8);
  double *act = (double *)calloc((size_t)n * I, 8);
  double *tmp = (double *)calloc((size_t)(H > V ? H : V), 8);
  double *sc = (double *)calloc((size_t)n, 8);
  float *row = (float *)malloc((size_t)H * 4);
  for (int t = 0; t < n; ++t) {
    int id = ids[t] < 0 ? 0 : (ids[t] >= V ? V - 1 : ids[t]);
    orc_dequantize_row(m->embed.qw, m->embed.si, m->embed.sb, H, id, row);
    for (int i = 0; i < H; ++i) x[(size_t)t * H + i] = row[i];
  }
  free(row);
  for (int l = 0; l < c->n_layers; ++l) {
    const layer_t *L = &m->layers[l];
    for (int t = 0; t < n; ++t) {
      rms_f64(x + (size_t)t * H, L->in_norm, h + (size_t)t * H, H, c->eps);
      gemv_f64(&L->qkv, h + (size_t)t * H, qkv + (size_t)t * nqkv);
      if (L->qkv_bias)
        for (int i = 0; i < nqkv; ++i) qkv[(size_t)t * nqkv + i] += (double)h2f(L->qkv_bias[i]);
      for (int hh = 0; hh < nq + nkv; ++hh) {
        double *v = qkv + (size_t)t * nqkv + (size_t)hh * hd;
        const uint16_t *g = hh < nq ? L->q_norm : L->k_norm;
        if (g) qk_norm_head(v, hd, g, c->eps);
        double r[1024];
        for (int j = 0; j < half; ++j) {
          const double inv = 1.0 / pow(c->rope_theta, (double)j / (double)half);
          const double a = (double)t * inv;
          r[j] = v[j] * cos(a) - v[j + half] * sin(a);
          r[j + half] = v[j + half] * cos(a) + v[j] * sin(a);
        }
        memcpy(v, r, (size_t)hd * 8);
      }
    }
    const int gqa = nq / nkv;
    for (int t = 0; t < n; ++t)
      for (int hh = 0; hh < nq; ++hh) {
        const int kvh = hh / gqa;
        const double *q = qkv + (size_t)t * nqkv + (size_t)hh * hd;
        double mx = -INFINITY;
        for (int u = 0; u <= t; ++u) {
          const double *k = qkv + (size_t)u * nqkv + (size_t)(nq + kvh) * hd;
          double a = 0.0;
          for (int i = 0; i < hd; ++i) a += q[i] * k[i];
          sc[u] = a / sqrt((double)hd);
          if (sc[u] > mx) mx = sc[u];
        }
        double den = 0.0;
        for (int u = 0; u <= t; ++u) { sc[u] = exp(sc[u] - mx); den += sc[u]; }
        for (int i = 0; i < hd; ++i) {
          double num = 0.0;
          for (int u = 0; u <= t; ++u)
            num += sc[u] / den * qkv[(size_t)u * nqkv + (size_t)(nq + nkv + kvh) * hd + i];
          ctx[((size_t)t * nq + hh) * hd + i] = num;
        }
      }
    for (int t = 0; t < n; ++t) {
      gemv_f64(&L->o, ctx + (size_t)t * nq * hd, tmp);
      for (int i = 0; i < H; ++i) x[(size_t)t * H + i] += tmp[i];
      rms_f64(x + (size_t)t * H, L->post_norm, h + (size_t)t * H, H, c->eps);
      gemv_f64(&L->gate_up, h + (size_t)t * H, gu + (size_t)t * 2 * I);
      for (int i = 0; i < I; ++i) {
        const double g = gu[(size_t)t * 2 * I + i], u = gu[(size_t)t * 2 * I + I + i];
        act[(size_t)t * I + i] = g / (1.0 + exp(-g)) * u;
      }
      gemv_f64(&L->down, act + (size_t)t * I, tmp);
      for (int i = 0; i < H; ++i) x[(size_t)t * H + i] += tmp[i];
    }
  }
  rms_f64(x + (size_t)(n - 1) * H, m->final_norm, h, H, c->eps);
  gemv_f64(c->tied ? &m->embed : &m->lm_head, h, logits_out);
  free(x); free(h); free(qkv); free(ctx); free(gu); free(act); free(tmp); free(sc);
}
