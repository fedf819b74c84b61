// Reference ABI symbols outside the batch=1 int4-hier-g32 decode path: the
// int4-g128 format and its variant sweep (gemv_int4.cu, gemv_variants.cu),
// the NVIDIA tensor-core probe (probe.cu) and MoE (moe.cu). They are exported
// so a caller built against the reference still links, and refuse with
// WST_ERR_UNSUPPORTED_ARCH and a message (status code of whetstone.h:25).
#include "common.hpp"

static wst_status_t unsupported(const char *what) {
  snprintf(wst_err_buf, sizeof(wst_err_buf),
           "%s: not part of the MI355X decode backend (int4-hier-g32 only)", what);
  return WST_ERR_UNSUPPORTED_ARCH;
}

extern "C" {
wst_status_t wst_gemv_int4_g128(const void *, const void *, const void *, void *, int32_t,
                                int32_t) {
  return unsupported("wst_gemv_int4_g128");
}
wst_status_t wst_bench_gemv(int32_t, int32_t, int32_t, int32_t, double *, double *) {
  return unsupported("wst_bench_gemv");
}
wst_status_t wst_gemv_int4_g128_ex(const void *, const void *, const void *, const void *, void *,
                                   int32_t, int32_t, int32_t) {
  return unsupported("wst_gemv_int4_g128_ex");
}
int32_t wst_gemv_variant_count(void) { return 0; }
int32_t wst_gemv_default_variant(void) { return -1; }
int32_t wst_gemv_variant_for_shape(int32_t, int32_t) { return -1; }
void wst_gemv_set_shape_rule(int32_t, int32_t, int32_t) {}
void wst_gemv_get_shape_rule(int32_t *out) {
  if (out) out[0] = out[1] = out[2] = -1;
}
const char *wst_gemv_variant_name(int32_t) { return "unsupported"; }
wst_status_t wst_gemv_int4_variant(int32_t, const void *, const void *, const void *,
                                   const void *, void *, int32_t, int32_t, int32_t) {
  return unsupported("wst_gemv_int4_variant");
}
wst_status_t wst_bench_gemv_variant(int32_t, int32_t, int32_t, int32_t, double *, double *) {
  return unsupported("wst_bench_gemv_variant");
}
wst_status_t wst_embed_int4_g128(const void *, const void *, const void *, void *, int32_t,
                                 int32_t) {
  return unsupported("wst_embed_int4_g128");
}
wst_status_t wst_embed_int4_g128_chunk(const void *, const void *, const void *, void *, int32_t,
                                       int32_t, int32_t) {
  return unsupported("wst_embed_int4_g128_chunk");
}
wst_status_t wst_probe(wst_probe_t *out, int32_t) {
  if (out) memset(out, 0, sizeof(*out));
  return unsupported("wst_probe");
}
wst_status_t wst_moe_router(const void *, int32_t, int32_t, int32_t, void *, void *) {
  return unsupported("wst_moe_router");
}
wst_status_t wst_moe_accumulate(void *, const void *, const void *, int32_t, int32_t) {
  return unsupported("wst_moe_accumulate");
}
}
