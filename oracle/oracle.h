/* CPU oracle for the batch=1 int4-hier-g32 decode path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or
 * calls this code. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker or the timed CPU baseline.
 *
 * Every function restates the reference's algorithm and cites the file:line it
 * follows (paths relative to the Whetstone source tree). How each function is
 * pinned is recorded in tests/test_oracle_*.py; see the per-function notes.
 *
 * Build: `make -C oracle` -> oracle/liboracle.so (gcc, -ffp-contract=off, so
 * every f32 expression rounds exactly where the Rust reference rounds).
 */
#ifndef WHETSTONE_ORACLE_H
#define WHETSTONE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ f16 <-> f32 */
uint16_t orc_f32_to_f16(float v);            /* IEEE binary16, round to nearest even */
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_n(const float *src, uint16_t *dst, size_t n);
void orc_f16_to_f32_n(const uint16_t *src, float *dst, size_t n);

/* ---------------------------------------------------- fixture generator */
uint64_t orc_splitmix64(uint64_t x);
/* Irwin-Hall(12) approximation of N(0, std^2), integer-exact, so a HIP kernel
 * with the same definition reproduces it bit for bit. */
float orc_fixture_normal(uint64_t seed, uint64_t stream, uint64_t index, float std_);
void orc_fixture_normal_n(uint64_t seed, uint64_t stream, uint64_t index0, float std_,
                          float *out, size_t n);

/* ------------------------------------------------------ int4-hier-g32 */
/* Returns 0 on success, 5 (shape) on a bad shape. Packs row-major
 * [out][in] f32 into qw [out][in/8] u32, si [out][in/32] u8, sb [out] u32.
 * err2_out/ref2_out (nullable) receive sum (w - w_hat)^2 and sum w^2. */
int orc_quantize_int4_hier(const float *w, int64_t in_f, int64_t out_f, uint32_t *qw,
                           uint8_t *si, uint32_t *sb, double *err2_out, double *ref2_out);
void orc_fit_group(const float *x, int n, float *scale, float *mn);
uint16_t orc_shared_scale(float v);
void orc_dequantize_int4_hier(const uint32_t *qw, const uint8_t *si, const uint32_t *sb,
                              int64_t in_f, int64_t out_f, float *out);
void orc_dequantize_row(const uint32_t *qw, const uint8_t *si, const uint32_t *sb,
                        int64_t in_f, int64_t row, float *out);

/* ------------------------------------------------ arithmetic variants */
/* Process-wide switches for the drift study (not thread-safe; default 0, 0):
 * acc ORC_ACC_F64 (f64 sums, rounded once), ORC_ACC_F32_SEQ (f32 sums in
 * ascending order), ORC_ACC_F32_LANE (f32 sums as 64 lane-strided partials
 * and a halving tree); xq = 1 rounds int4-GEMV activations to the GPU
 * activation table's 14-bit per-group fixed point. */
#define ORC_ACC_F64 0
#define ORC_ACC_F32_SEQ 1
#define ORC_ACC_F32_LANE 2
/* ORC_ACC_REF: every reduction in the order and precision of the reference's
 * CUDA kernels (f16 __hfma2/__hadd2 group sums in the int4 GEMV, 32-lane
 * butterflies, block reductions, per-warp online softmax and the split merge),
 * on a device of orc_set_ref_sms() multiprocessors (default 30). */
#define ORC_ACC_REF 3
void orc_set_ref_sms(int sms);
/* Splits per head of the reference's attention at that SM count. */
int orc_ref_attn_splits(int n_q, int max_seq);
/* IEEE binary16 RNE of a double; one f16 lane of __hadd2 / __hfma2. */
uint16_t orc_d2h(double v);
uint16_t orc_ref_hadd(uint16_t a, uint16_t b);
uint16_t orc_ref_hfma(uint16_t a, uint16_t b, uint16_t c);
void orc_set_variant(int acc, int xq);
/* The activation table's value of each f16 activation (groups of 32). */
void orc_xq14(const uint16_t *x, int64_t n, double *out);

/* ------------------------------------------------------------ decode ops */
/* y[r] = (accum ? y[r] : 0) + bias[r] + sum_c dequant[r][c] * f16(x)[c], f64 inside. */
void orc_gemv_int4_hier(const uint32_t *qw, const uint8_t *si, const uint32_t *sb,
                        const uint16_t *x, const uint16_t *bias, float *y, int64_t in_f,
                        int64_t out_f, int accum);
void orc_gemv_fp16(const uint16_t *w, const uint16_t *x, const uint16_t *bias, float *y,
                   int64_t in_f, int64_t out_f, int accum);
void orc_rmsnorm(const float *x, const uint16_t *w, uint16_t *out, int n, float eps);
void orc_rope_table(int max_seq, int head_dim, double theta, float *cos_tab, float *sin_tab);
void orc_rope_cache(float *qkv, uint16_t *k_cache, uint16_t *v_cache, const float *cos_tab,
                    const float *sin_tab, int n_q, int n_kv, int hd, int pos, int max_seq,
                    const uint16_t *q_norm_w, const uint16_t *k_norm_w, float eps);
void orc_attn_decode(const float *q, const uint16_t *k_cache, const uint16_t *v_cache,
                     uint16_t *out, int n_q, int n_kv, int hd, int pos, int max_seq,
                     float scale);
void orc_swiglu(const float *gate_up, uint16_t *out, int n);
int32_t orc_argmax(const float *logits, int n);
uint64_t orc_argmax_key(float v, int32_t idx);
/* Head rescore ladder: returns the threshold; *count receives how many logits
 * clear it (uncapped), exactly as head_max/counts/pick compute it. */
float orc_head_threshold(const float *logits, int n, int k, int cap, int32_t *count,
                         int32_t *rung);
/* Overwrites every logit >= thresh (when count <= cap) with the fp16 dot. */
void orc_head_rescore(const uint16_t *head, const uint16_t *x, float *logits, int n,
                      int hidden, float thresh);

/* ----------------------------------------------------------- the model */
typedef struct {
  int32_t n_layers, hidden, n_q, n_kv, head_dim, inter, vocab;
  int32_t tied;          /* lm_head = embed */
  int32_t qkv_bias;      /* 1: q/k/v biases present (Qwen2), zero-valued in fixtures */
  int32_t qk_norm;       /* 1: per-head q/k RMSNorm gains */
  int32_t rescore_k;     /* 0: no fp16 head copy */
  float eps;
  double rope_theta;
} orc_config_t;

typedef struct orc_model orc_model_t;
typedef struct orc_state orc_state_t;

/* Seeded synthetic model: every Linear and the Embedding ~N(0,0.02) f32, packed
 * to hier-g32; q/k/v biases 0; norm gains 1; QK-norm gains 1+N(0,0.02). */
orc_model_t *orc_model_synthetic(const orc_config_t *cfg, uint64_t seed);
/* The same model with its packed matrices allocated but left zero, for a
 * caller that copies packed bytes in through orc_model_tensor's pointers (the
 * bench's CPU leg copies the device model's bytes). */
orc_model_t *orc_model_alloc(const orc_config_t *cfg, uint64_t seed);
void orc_model_free(orc_model_t *m);
/* Raw views of the packed tensors, for tests that compare bytes.
 * name: "embed", "lm_head", "L<l>.qkv", "L<l>.o", "L<l>.gate_up", "L<l>.down". */
int orc_model_tensor(orc_model_t *m, const char *name, const uint32_t **qw,
                     const uint8_t **si, const uint32_t **sb, int64_t *in_f, int64_t *out_f);
const uint16_t *orc_model_fp16(orc_model_t *m, const char *name, int64_t *n);
int orc_model_set_dense(orc_model_t *m, const char *which, const uint16_t *table);

/* mode 0: precision-mirrored (f16 at the kernels' narrowing points),
 * mode 1: textbook f64 (no narrowing, f64 KV cache). */
orc_state_t *orc_state_new(const orc_model_t *m, int max_seq, int mode);
void orc_state_free(orc_state_t *s);
int orc_state_pos(const orc_state_t *s);
void orc_state_set_pos(orc_state_t *s, int pos);
/* One decode step for `token` at the current position; logits f32 [vocab] out.
 * Runs the head rescore when the model has one. Returns the device-style
 * argmax (ties to the lowest index). */
int32_t orc_step(orc_state_t *s, int32_t token, float *logits_out);
/* Fill the KV caches of every layer for positions [0, n) with ~N(0,1) f16 from
 * (seed, stream 1000+layer), the way the GPU engine's synthetic context does. */
void orc_state_fill_kv(orc_state_t *s, uint64_t seed, int n);
/* The reference's own CPU forward: full recompute of all ids, f64, returns the
 * last position's logits (bench/reference_numpy.py:148-194). */
void orc_forward_full(const orc_model_t *m, const int32_t *ids, int n, double *logits_out);
int orc_threads(void);

#ifdef __cplusplus
}
#endif
#endif
