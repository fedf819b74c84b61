/* whetstone.h -- the C ABI of the MI355X (gfx950) decode backend.
 *
 * This is the drop-in boundary. A caller built against the reference's kernel
 * library (crates/whetstone-kernels/cuda/whetstone.h plus the extern block in
 * crates/whetstone-kernels/src/ffi.rs:134-473) links against
 * libwhetstone_hip.so instead and needs no source change: every symbol below
 * keeps the reference's name, argument order, argument meaning, status codes
 * and ownership rules. Each declaration cites the reference line it replaces.
 *
 * Rules (same as the reference, whetstone.h:1-9):
 *   - plain C types only; void* is a device pointer unless named *_host;
 *   - every entry point returns wst_status_t, results go through out-params;
 *   - nothing throws, aborts or longjmps across this boundary;
 *   - all work is queued on the calling thread's per-thread default stream
 *     (hipStreamPerThread), asynchronously; wst_memcpy_* block.
 *
 * Symbols of the reference that are outside the decode path (the int4-g128
 * format, its variant sweep, the tensor-core probe, MoE) are exported as stubs
 * that return WST_ERR_UNSUPPORTED_ARCH with a message, so a caller still links.
 */
#ifndef WHETSTONE_H
#define WHETSTONE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference: whetstone.h:21-28 */
typedef enum {
  WST_OK = 0,
  WST_ERR_CUDA = 1, /* the underlying HIP call failed; see wst_last_error */
  WST_ERR_INVALID_ARG = 2,
  WST_ERR_UNSUPPORTED_ARCH = 3,
  WST_ERR_OOM = 4,
  WST_ERR_SHAPE = 5,
} wst_status_t;

/* ------------------------------------------------------------------ device */

/* reference: whetstone.h:32-57. Same layout. On gfx950 `major.minor` is the
 * gfx IP version (9.5), `sm_count` the compute-unit count, `warp_size` 64. The
 * capability flags report the CDNA4 equivalents (MFMA for tensor cores, fp8
 * MFMA for has_fp8); the NVIDIA-only bmma/cp.async flags are 0. */
typedef struct {
  char name[256];
  int32_t major;
  int32_t minor;
  int32_t sm_count;
  int32_t clock_khz;
  int32_t mem_clock_khz;
  int32_t mem_bus_width;
  int32_t max_threads_per_block;
  int32_t max_smem_per_block;
  int32_t warp_size;
  int32_t l2_bytes;
  uint64_t mem_total;
  uint64_t mem_free;
  double bandwidth_gbs;
  int32_t has_tensor_cores;
  int32_t has_imma;
  int32_t has_bmma_xor;
  int32_t has_bmma_and;
  int32_t has_cp_async;
  int32_t has_sparse_tc;
  int32_t has_fp8;
} wst_device_info_t;

/* reference: whetstone.h:62-67 */
typedef struct {
  uint32_t device_info_size;
  uint32_t device_info_align;
  uint32_t probe_size;
  uint32_t probe_align;
} wst_abi_layout_t;

void wst_abi_layout(wst_abi_layout_t *out);                       /* whetstone.h:69 */
wst_status_t wst_device_count(int32_t *out_count);                 /* whetstone.h:71 */
wst_status_t wst_device_set(int32_t ordinal);                      /* whetstone.h:72 */
wst_status_t wst_device_info(int32_t ordinal, wst_device_info_t *out_info); /* :73 */
wst_status_t wst_device_synchronize(void);                         /* whetstone.h:74 */
const char *wst_last_error(void);                                  /* whetstone.h:77 */

/* ------------------------------------------------------------------ memory */

wst_status_t wst_malloc(void **out_ptr, size_t bytes);             /* whetstone.h:81 */
wst_status_t wst_free(void *ptr);                                  /* whetstone.h:82 */
/* whetstone.h:88-89. Host-resident weights (PCIe offload) are outside the
 * single-GPU resident decode path: returns WST_ERR_UNSUPPORTED_ARCH, and
 * wst_host_alloc_supported() returns 0. */
wst_status_t wst_malloc_host(void **out_ptr, size_t bytes);
int32_t wst_host_alloc_supported(void);
wst_status_t wst_memset(void *dst, int32_t value, size_t bytes);   /* whetstone.h:90 */
wst_status_t wst_memcpy_h2d(void *dst, const void *src_host, size_t bytes); /* :91 */
wst_status_t wst_memcpy_d2h(void *dst_host, const void *src, size_t bytes); /* :92 */
wst_status_t wst_memcpy_d2d(void *dst, const void *src, size_t bytes);      /* :93 */

/* ------------------------------------------------------- capability probe */

/* reference: whetstone.h:103-113. NVIDIA tensor-core probe: stub. */
typedef struct {
  double fp16_wmma_tflops;
  double int8_wmma_tops;
  double int4_wmma_tops;
  double bin_bmma_tops;
  double dp4a_tops;
  double popc_tops;
  int32_t xnor_identity_ok;
} wst_probe_t;
wst_status_t wst_probe(wst_probe_t *out, int32_t iters);

/* --------------------------------------------------------------- bandwidth */

/* reference: whetstone.h:122 (runtime.cu:210-260). 128-bit streaming read over
 * a buffer of `bytes`, timed with events; returns GB/s. */
wst_status_t wst_bench_bandwidth(size_t bytes, int32_t reps, double *out_gbs);

/* ------------------------------------------------- int4-g128 (stubs) */
/* reference: whetstone.h:135-183. The g128 format is in no configuration of
 * this build; these return WST_ERR_UNSUPPORTED_ARCH. */
wst_status_t wst_gemv_int4_g128(const void *qw, const void *sz, const void *x, void *y,
                                int32_t in_f, int32_t out_f);
wst_status_t wst_bench_gemv(int32_t in_f, int32_t out_f, int32_t reps, int32_t use_int4,
                            double *out_gbs, double *out_ms);
wst_status_t wst_gemv_int4_g128_ex(const void *qw, const void *sz, const void *x,
                                   const void *bias, void *y, int32_t in_f, int32_t out_f,
                                   int32_t accum);
int32_t wst_gemv_variant_count(void);
int32_t wst_gemv_default_variant(void);
int32_t wst_gemv_variant_for_shape(int32_t in_f, int32_t out_f);
void wst_gemv_set_shape_rule(int32_t wide, int32_t huge, int32_t other);
void wst_gemv_get_shape_rule(int32_t *out);
const char *wst_gemv_variant_name(int32_t variant);
wst_status_t wst_gemv_int4_variant(int32_t variant, const void *qw, const void *sz,
                                   const void *x, const void *bias, void *y, int32_t in_f,
                                   int32_t out_f, int32_t accum);
wst_status_t wst_bench_gemv_variant(int32_t variant, int32_t in_f, int32_t out_f,
                                    int32_t reps, double *out_gbs, double *out_ms);
wst_status_t wst_embed_int4_g128(const void *qw, const void *sz, const void *token,
                                 void *out, int32_t hidden, int32_t rows);
wst_status_t wst_embed_int4_g128_chunk(const void *qw, const void *sz, const void *tokens,
                                       void *out, int32_t hidden, int32_t rows, int32_t n);

/* ------------------------------------------------------------ fp16 GEMV */

/* reference: whetstone.h:140-141, 176-177 (gemv_int4.cu:194-305).
 * y[out_f] (+)= W[out_f][in_f] . x[in_f] + bias; W, x, bias f16, y f32. */
wst_status_t wst_gemv_fp16(const void *w, const void *x, void *y, int32_t in_f,
                           int32_t out_f);
wst_status_t wst_gemv_fp16_ex(const void *w, const void *x, const void *bias, void *y,
                              int32_t in_f, int32_t out_f, int32_t accum);

/* ------------------------------------------------------ int4-hier-g32 GEMV */

/* reference: ffi.rs:276-286, gemv_hier.cu:274-291.
 *   qw   [out_f][in_f/8]  u32, nibble i of word k = column 8k+i
 *   si   [out_f][in_f/32] u8,  ls | lm<<4
 *   sb   [out_f]          u32, f16 d (low) | f16 dmin (high)
 *   x    [in_f]  f16; bias [out_f] f16 or NULL; y [out_f] f32
 *   y[r] = (accum ? y[r] : 0) + bias[r] + sum_g [ d*ls_g * sum_i q_i x_i - dmin*lm_g * sum_i x_i ]
 * in_f must be a positive multiple of 32. */
wst_status_t wst_gemv_int4_hier_ex(const void *qw, const void *si, const void *sb,
                                   const void *x, const void *bias, void *y, int32_t in_f,
                                   int32_t out_f, int32_t accum);
/* reference: ffi.rs:288-289, gemv_hier.cu:255-267. The (wide, huge, other) tile
 * rule: each entry 0..3 selects rows-per-lane-slot 1, 2, 4 or 8 for shapes with
 * in_f >= 2048, out_f >= 65536, and everything else. Out-of-range entries are
 * ignored. Every rule computes the same result. */
void wst_gemv_hier_set_rule(int32_t wide, int32_t huge, int32_t other);
void wst_gemv_hier_get_rule(int32_t *out);
/* reference: ffi.rs:291-298, gemv_hier.cu:293-307. out[c] = dequant(row)[c] in
 * f32 for row = clamp(*row, 0, vocab-1), bit-exact with the quantiser's
 * dequantisation (s = d*ls, m = -dmin*lm, w = q*s + m, no fused multiply-add). */
wst_status_t wst_embed_int4_hier(const void *qw, const void *si, const void *sb,
                                 const void *row, void *out, int32_t in_f, int32_t vocab);

/* ------------------------------------------------------------ decode layers */

/* reference: whetstone.h:209 (decode.cu:84-100). out = f16(x*rsqrt(mean x^2+eps)*w) */
wst_status_t wst_rmsnorm(const void *x, const void *w, void *out, int32_t n, float eps);

/* reference: whetstone.h:233-236 (decode.cu:180-208). Optional per-head QK
 * RMSNorm, then the half-rotation RoPE of q in place and k into the f16 cache
 * [n_kv][max_seq][head_dim] at clamp(*pos, 0, max_seq-1); v copied to the cache. */
wst_status_t wst_rope_cache(void *qkv, void *k_cache, void *v_cache, const void *cos_tab,
                            const void *sin_tab, int32_t n_q, int32_t n_kv,
                            int32_t head_dim, const void *pos, int32_t max_seq,
                            const void *q_norm_w, const void *k_norm_w, float eps);

/* reference: whetstone.h:251-254 (attention.cu:219-245). GQA attention of q
 * [n_q][head_dim] f32 over the first min(*pos+1, max_seq) cache entries, f16 out. */
wst_status_t wst_attn_decode(const void *q, const void *k_cache, const void *v_cache,
                             void *partials, void *out, int32_t n_q, int32_t n_kv,
                             int32_t head_dim, const void *pos, int32_t max_seq,
                             float scale);
/* reference: whetstone.h:257 (attention.cu:249-253). Floats of `partials`
 * scratch wst_attn_decode needs for these dimensions. */
int32_t wst_attn_partial_floats(int32_t n_q, int32_t head_dim, int32_t max_seq);

/* reference: whetstone.h:261. out[i] = f16(silu(gu[i]) * gu[i+n]) */
wst_status_t wst_swiglu(const void *gate_up, void *out, int32_t n);

/* reference: whetstone.h:264-265. Row clamp(*token) of an f16 table, as f32. */
wst_status_t wst_embed_fp16(const void *table, const void *token, void *out,
                            int32_t hidden, int32_t rows);

/* ------------------------------------------------------------ graphs */

/* reference: whetstone.h:280-284, graph.cu:47-107. Capture of the calling
 * thread's per-thread stream (thread-local mode), instantiate, launch. */
wst_status_t wst_graph_capture_begin(void);
wst_status_t wst_graph_capture_end(void **out_exec);
wst_status_t wst_graph_launch(void *exec);
wst_status_t wst_graph_destroy(void *exec);
wst_status_t wst_stream_sync(void);

/* reference: whetstone.h:289-292, graph.cu:121-145 */
wst_status_t wst_event_create(void **out);
wst_status_t wst_event_record(void *ev);
wst_status_t wst_event_elapsed_ms(void *a, void *b, float *out);
wst_status_t wst_event_destroy(void *ev);

/* reference: whetstone.h:295 (decode.cu:210-226). pos = min(pos+1, max_seq). */
wst_status_t wst_advance_pos(void *pos, int32_t max_seq);

/* ---------------------------------------------------------------- sampling */

/* reference: whetstone.h:300 (sample.cu:182-200). Index of the largest logit
 * into a device i32; ties go to the lowest index; +NaN above +inf; +0 above -0. */
wst_status_t wst_argmax(const void *logits, void *out_idx, int32_t n);

/* reference: whetstone.h:308 (sample.cu:163-180). acc[0] += -log softmax(logits)[target],
 * acc[1] += 1, on the device. */
wst_status_t wst_nll(const void *logits, int32_t target, void *acc, int32_t n);

/* ------------------------------------------------------ top-k head rescore */

/* reference: whetstone.h:343-351 (head_rescore.cu:182-297).
 * scratch: at least nblocks + 1 + 12 floats (layout [nblocks] f32 partial
 * maxima | 1 f32 max | 12 i32 rung counts). The threshold is max - 2^c/64 for
 * the smallest rung c admitting >= k logits, stepped down while it admits > cap;
 * out_count is reset to 0 for wst_head_compact. */
wst_status_t wst_head_threshold(const void *logits, int32_t n, int32_t k, int32_t cap,
                                void *scratch, int32_t nblocks, void *out_thresh,
                                void *out_count);
wst_status_t wst_head_compact(const void *logits, int32_t n, const void *thresh,
                              void *count, void *out_idx, int32_t cap);
wst_status_t wst_head_rescore(const void *head, const void *x, const void *idx,
                              const void *count, void *logits, int32_t hidden,
                              int32_t cap, int32_t grid);

/* ------------------------------------------------------- mixture of experts */
/* reference: whetstone.h:362-369. No MoE model executes: stubs. */
wst_status_t wst_moe_router(const void *logits, int32_t n_experts, int32_t k,
                            int32_t norm_topk, void *out_idx, void *out_w);
wst_status_t wst_moe_accumulate(void *dst, const void *src, const void *weights,
                                int32_t slot, int32_t n);

/* ------------------------------------------------------- multi-token chunk */

/* reference: whetstone.h:311-378 (chunk_gemm.cu, chunk_ops.cu). Token-major
 * [n][dim] activations; pos0 by value. */
int32_t wst_chunk_max_tokens(void);
wst_status_t wst_gemm_int4_hier(const void *qw, const void *si, const void *sb,
                                const void *x, const void *bias, void *y, int32_t in_f,
                                int32_t out_f, int32_t n, int32_t accum);
wst_status_t wst_gemm_fp16(const void *w, const void *x, const void *bias, void *y,
                           int32_t in_f, int32_t out_f, int32_t n, int32_t accum);
wst_status_t wst_rmsnorm_chunk(const void *x, const void *w, void *out, int32_t dim,
                               int32_t n, float eps);
wst_status_t wst_rope_cache_chunk(void *qkv, void *k_cache, void *v_cache,
                                  const void *cos_tab, const void *sin_tab, int32_t n_q,
                                  int32_t n_kv, int32_t head_dim, int32_t pos0, int32_t n,
                                  int32_t max_seq, const void *q_norm_w,
                                  const void *k_norm_w, float eps);
wst_status_t wst_attn_chunk(const void *qkv, const void *k_cache, const void *v_cache,
                            void *out, int32_t n_q, int32_t n_kv, int32_t head_dim,
                            int32_t pos0, int32_t n, int32_t max_seq, float scale);
wst_status_t wst_swiglu_chunk(const void *gate_up, void *out, int32_t inter, int32_t n);
wst_status_t wst_embed_fp16_chunk(const void *table, const void *tokens, void *out,
                                  int32_t hidden, int32_t rows, int32_t n);
wst_status_t wst_embed_int4_hier_chunk(const void *qw, const void *si, const void *sb,
                                       const void *tokens, void *out, int32_t hidden,
                                       int32_t rows, int32_t n);
wst_status_t wst_argmax_chunk(const void *logits, void *out, int32_t vocab, int32_t n);

#ifdef __cplusplus
}
#endif

#endif /* WHETSTONE_H */
