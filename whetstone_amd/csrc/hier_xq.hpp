// The int4-hier GEMV's activation table (shared by the GEMV prologue and by
// the kernels that produce a GEMV input, such as the attention merge).
#pragma once
#include "common.hpp"

// The activation table. For each group of 32 columns the block holds, in LDS:
//   L[k][j]  k = 0..3 (8 columns each), j = 0..3: digit j of X_c for the 8
//            columns c = 8k..8k+7, nibble i <-> column 8k+i (the packed
//            weights' own nibble order), as signed 4-bit values in [-8, 7]
//   C8       8 * sum_c X_c
//   S        sc * sum_c X_c (the sum of the quantised values, exact in f32)
//   sc       2^(e-28), e = f16 exponent field of max_c |h_c| (at least 1)
// where X_c = rint(h_c / sc) is h in units of sc: |X_c| < 2^14, so X is h to
// 14 bits of the group's largest value (f16 itself carries 11), exactly for
// every h_c within 4 binades of that maximum. X_c = sum_j 16^j D_j with
// balanced digits D_j in [-8, 7]; D_j is hex digit j of X_c + 0x8888, minus 8.
//
// One packed word w (8 nibbles q) against digit word j gives, in one
// v_dot8_i32_i4 on (w xor 0x88888888) = (q - 8 per nibble),
//     sum_i (q_i - 8) D_j,i
// and sum_i q_i X_i = sum_j 16^j (that) + 8 sum_i X_i, all exact in int32.
// A group then contributes  ls * sc * (sum q X)  to the row's d-term and
// lm * S to its dmin-term:  y = d * sum_g ls_g Q_g - dmin * sum_g lm_g S_g.
// Per 8 weights: one xor and four dot8 (the f16 route needs nine VALU ops).
//
// The table is built from the f16 vector the GEMV multiplies: h itself for the
// plain form, f16(x * rms * w) for the NORM form (the same bits wst_rmsnorm
// writes), so every form of a row computes the same value.
#define XQ_WORDS 20  // 16 digit words + C8, S, sc, pad
#define NORM_THREADS 512

__device__ __forceinline__ int sdot8(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot8((int)a, (int)b, c, false);
}
// First link of a dot chain: the three-operand form with an inline zero, so no
// accumulator is cleared by a separate move.
__device__ __forceinline__ int sdot8z(uint32_t a, uint32_t b) {
  int r;
  asm("v_dot8_i32_i4 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// Table entry for one quarter (8 columns, words k = b & 3) of group b >> 2.
// The four quarters of a group are four adjacent lanes: quad DPP ops combine
// them, so all lanes of a quad must call this together (valid or not).
__device__ __forceinline__ void build_xq(const uint16_t h[8], int b, bool valid,
                                         uint32_t *__restrict__ xgt) {
  // Group max |h| as f16 bits (monotone in magnitude): pairs of halves at once.
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) w[k] = ((uint32_t)h[2 * k] | ((uint32_t)h[2 * k + 1] << 16)) & 0x7FFF7FFFu;
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  u16x2 m2 = __builtin_elementwise_max(__builtin_bit_cast(u16x2, w[0]), __builtin_bit_cast(u16x2, w[1]));
  m2 = __builtin_elementwise_max(m2, __builtin_elementwise_max(__builtin_bit_cast(u16x2, w[2]),
                                                               __builtin_bit_cast(u16x2, w[3])));
  uint32_t mx = max((uint32_t)m2.x, (uint32_t)m2.y);
  mx = max(mx, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, 0xB1, 0xF, 0xF, false));
  mx = max(mx, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, 0x4E, 0xF, 0xF, false));
  int ef = (int)(mx >> 10);
  ef = ef < 1 ? 1 : (ef > 30 ? 30 : ef);
  const float inv = __builtin_bit_cast(float, (uint32_t)(127 + 28 - ef) << 23);
  const float sc = __builtin_bit_cast(float, (uint32_t)(127 - 28 + ef) << 23);
  // X_e and U_e = X_e + 0x8888 (16 bits: |X_e| < 2^14), packed in pairs.
  uint32_t P[4];
  int sx = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int X0 = (int)__builtin_rintf(h2f(h[2 * k]) * inv);
    const int X1 = (int)__builtin_rintf(h2f(h[2 * k + 1]) * inv);
    sx += X0 + X1;
    P[k] = (uint32_t)(X0 + 0x8888) | ((uint32_t)(X1 + 0x8888) << 16);
  }
  // Nibble transpose: digit word j holds hex digit j of U_0..U_7 (nibble e for
  // element e). E_k bytes 0/1 are bytes k of digit words 0/2, O_k of 1/3.
  uint32_t E[4], O[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    E[k] = (P[k] & 0x0F0Fu) | ((P[k] >> 12) & 0xF0F0u);
    O[k] = ((P[k] >> 4) & 0x0F0Fu) | ((P[k] >> 16) & 0xF0F0u);
  }
  const uint32_t e01 = __builtin_amdgcn_perm(E[1], E[0], 0x05010400u);
  const uint32_t e23 = __builtin_amdgcn_perm(E[3], E[2], 0x05010400u);
  const uint32_t o01 = __builtin_amdgcn_perm(O[1], O[0], 0x05010400u);
  const uint32_t o23 = __builtin_amdgcn_perm(O[3], O[2], 0x05010400u);
  // Hex digit u of U is the balanced digit plus 8; as a signed nibble the
  // digit is u xor 8.
  const uint32_t L0 = __builtin_amdgcn_perm(e23, e01, 0x05040100u) ^ 0x88888888u;
  const uint32_t L2 = __builtin_amdgcn_perm(e23, e01, 0x07060302u) ^ 0x88888888u;
  const uint32_t L1 = __builtin_amdgcn_perm(o23, o01, 0x05040100u) ^ 0x88888888u;
  const uint32_t L3 = __builtin_amdgcn_perm(o23, o01, 0x07060302u) ^ 0x88888888u;
  sx += __builtin_amdgcn_update_dpp(0, sx, 0xB1, 0xF, 0xF, false);
  sx += __builtin_amdgcn_update_dpp(0, sx, 0x4E, 0xF, 0xF, false);
  if (valid) {
    uint32_t *e = xgt + (size_t)(b >> 2) * XQ_WORDS;
    const int k = b & 3;
    *(uint4 *)(e + 4 * k) = make_uint4(L0, L1, L2, L3);
    if (k == 0) {
      e[16] = (uint32_t)(8 * sx);
      e[17] = __float_as_uint((float)sx * sc);  // S = sum of the quantised h
      e[18] = __float_as_uint(sc);
    }
  }
}

