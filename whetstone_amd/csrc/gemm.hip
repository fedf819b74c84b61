// Multi-token int4-hier-g32 GEMM: y[j] (+)= W x[j] + b for j < n.
// reference: chunk_gemm.cu:65-176, 285-332.
#include "common.hpp"

wst_status_t wst_gemm_int4_hier_impl(const void *qw, const void *si, const void *sb,
                                     const void *x, const void *bias, void *y, int32_t in_f,
                                     int32_t out_f, int32_t n, int32_t accum) {
  for (int j = 0; j < n; ++j) {
    const wst_status_t st = wst_gemv_int4_hier_ex(qw, si, sb, (const uint16_t *)x + (size_t)j * in_f,
                                                  bias, (float *)y + (size_t)j * out_f, in_f,
                                                  out_f, accum);
    if (st != WST_OK) return st;
  }
  return WST_OK;
}
