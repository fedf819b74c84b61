/* whetstone_ext.h -- entry points of libwhetstone_hip.so that have NO
 * counterpart in the reference's C ABI.
 *
 * Same conventions as whetstone.h (status codes, per-thread stream, device
 * pointers). Two groups:
 *
 *  1. Fixture generation on the device. The reference quantises on the host in
 *     Rust (crates/whetstone-quant/src/hier.rs); a 7B-shaped model is 7 G
 *     weights, minutes of host time, so the synthetic configurations are
 *     generated and packed on the GPU instead. The device packer follows
 *     hier.rs:113-391 operation for operation and is checked bit-exact
 *     against the host restatement.
 *
 *  2. Fused decode-step kernels used by the engine's fast path. Each computes
 *     exactly what a sequence of reference ABI calls computes (named in its
 *     comment), in fewer launches.
 */
#ifndef WHETSTONE_EXT_H
#define WHETSTONE_EXT_H

#include <stddef.h>
#include <stdint.h>

#include "whetstone.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------ fixture generation */

/* out[i] = fixture normal (seed, stream, index0 + i) * std as f32: the sum of
 * twelve 16-bit uniforms drawn from splitmix64, re-centred, times 2^-16*std. */
wst_status_t wst_fixture_normal_f32(void *out, size_t n, uint64_t seed, uint64_t stream,
                                    uint64_t index0, float std_);
/* Same values narrowed to f16, plus an f32 offset added before narrowing
 * (norm gains are 1 + N(0, 0.02)). */
wst_status_t wst_fixture_normal_f16(void *out, size_t n, uint64_t seed, uint64_t stream,
                                    uint64_t index0, float std_, float offset);
/* Generates rows [0, rows) of a tensor from (seed, stream) -- element (r, c) is
 * fixture normal index r*in_f + c, times std -- and packs them to hier-g32 into
 * rows [row0, row0+rows) of (qw, si, sb). Bit-exact with the host quantiser. */
wst_status_t wst_fixture_pack_hier(void *qw, void *si, void *sb, int64_t in_f,
                                   int64_t row0, int64_t rows, uint64_t seed,
                                   uint64_t stream, float std_);
/* Packs a caller-provided f32 matrix [rows][in_f] (device) into hier-g32. */
wst_status_t wst_quantize_int4_hier(const void *w, void *qw, void *si, void *sb,
                                    int64_t in_f, int64_t rows);
/* Fills a KV cache [n_kv][max_seq][hd] f16 for positions [0, n): element
 * (h, t, i) of k (kv=0) or v (kv=1) is f16(fixture normal (seed, stream,
 * ((h*2+kv)<<20 + t)*hd + i)). */
wst_status_t wst_fixture_fill_kv(void *k_cache, void *v_cache, int32_t n_kv,
                                 int32_t max_seq, int32_t head_dim, int32_t n,
                                 uint64_t seed, uint64_t stream);

/* ------------------------------------------------ fused decode-step kernels */

/* wst_rmsnorm(x, w, h) followed by wst_gemv_int4_hier_ex(W, h, bias, y, accum):
 * every block recomputes the RMS of x (f32 [in_f]) and narrows x*inv*w to f16
 * in registers, so the normalised vector never round-trips through memory.
 * Also writes h (f16 [in_f]) from block 0 when h_out is non-NULL (the head
 * rescore reads it). */
wst_status_t wst_gemv_hier_rmsnorm(const void *qw, const void *si, const void *sb,
                                   const void *x, const void *norm_w, float eps,
                                   void *h_out, const void *bias, void *y, int32_t in_f,
                                   int32_t out_f, int32_t accum);

/* wst_gemv_int4_hier_ex over a fused gate|up matrix followed by wst_swiglu:
 * row r of the gate half and row r of the up half are computed by the same
 * lanes, and out[r] = f16(silu(g) * u) is written directly. Optional RMSNorm
 * prologue when norm_w is non-NULL (as wst_gemv_hier_rmsnorm). */
wst_status_t wst_gemv_hier_swiglu(const void *qw, const void *si, const void *sb,
                                  const void *x, const void *norm_w, float eps,
                                  void *out, int32_t in_f, int32_t inter);

/* wst_rope_cache + wst_attn_decode: the slice kernel (RoPE, KV append,
 * per-slice softmax on MFMA) then the slice merge. */
wst_status_t wst_attn_decode_fused(void *qkv, void *k_cache, void *v_cache,
                                   const void *cos_tab, const void *sin_tab, void *partials,
                                   void *out, int32_t n_q, int32_t n_kv, int32_t head_dim,
                                   const void *pos, int32_t max_seq, float scale,
                                   const void *q_norm_w, const void *k_norm_w, float eps);

/* wst_gemv_hier_rmsnorm(W, x, norm_w, eps, h_out, bias NULL, y, accum 0)
 * followed by wst_argmax_advance(y, out_idx, out_f, pos, max_seq), in one
 * call: the GEMV's blocks store the argmax key of the rows they write, and a
 * one-block kernel after it takes their maximum, writes out_idx and advances
 * pos (pos NULL: no advance). The step's head when nothing (rescore) runs
 * between the logits and the argmax. The per-block keys live in one library
 * scratch slot per device, shared by every stream: calls on one GPU must not
 * overlap (issue them on one stream, or order them), or one call can read
 * another's keys. */
wst_status_t wst_gemv_hier_rmsnorm_argmax(const void *qw, const void *si, const void *sb,
                                          const void *x, const void *norm_w, float eps,
                                          void *h_out, void *y, int32_t in_f, int32_t out_f,
                                          void *out_idx, void *pos, int32_t max_seq);

/* wst_argmax(logits, out_idx) followed by wst_advance_pos(pos, max_seq). */
wst_status_t wst_argmax_advance(const void *logits, void *out_idx, int32_t n, void *pos,
                                int32_t max_seq);

/* wst_head_threshold + wst_head_compact + wst_head_rescore in two launches:
 * the threshold ladder, then every logit >= threshold recomputed from the f16
 * head by the block that found it. Rescores all selected rows whenever their
 * count is <= cap (the reference's deterministic regime); above cap, none. */
wst_status_t wst_head_rescore_fused(const void *head, const void *x, void *logits,
                                    int32_t n, int32_t hidden, int32_t k, int32_t cap,
                                    void *scratch, int32_t nblocks);

/* Cached positions per attention slice that wst_attn_decode and its fused
 * forms use for a cache of max_seq positions: 16384 / head_dim (0 for an
 * unsupported head_dim or an empty cache). */
int32_t wst_attn_slice_positions(int32_t head_dim, int32_t max_seq);

/* wst_attn_decode_fused without its merge kernel: the slices' partials are
 * left for wst_gemv_hier_attn. */
wst_status_t wst_attn_decode_slices(void *qkv, void *k_cache, void *v_cache,
                                    const void *cos_tab, const void *sin_tab, void *partials,
                                    int32_t n_q, int32_t n_kv, int32_t head_dim, const void *pos,
                                    int32_t max_seq, float scale, const void *q_norm_w,
                                    const void *k_norm_w, float eps);
/* The slice merge (attn_merge_kernel) fused into the o GEMV:
 * y (+)= W merge(partials), with in_f = n_q * head_dim; bit-identical to
 * wst_attn_decode's merge followed by wst_gemv_int4_hier_ex. head_dim 64 or
 * 128 and at most 8 slices (max_seq <= 8 * 16384 / head_dim). */
wst_status_t wst_gemv_hier_attn(const void *qw, const void *si, const void *sb,
                                const void *partials, void *y, int32_t n_q, int32_t head_dim,
                                const void *pos, int32_t max_seq, int32_t out_f, int32_t accum);

/* The int4-hier GEMV's activation table, built once by the producer of the
 * GEMV's input instead of by every block of the GEMV. For an f16 vector of
 * in_f values (in_f a multiple of 32) the table is in_f / 32 entries of 80
 * bytes (20 u32: per group of 32 values its 14-bit fixed-point digits for
 * v_dot8, 8*sum, the sum as f32 and the group scale; word 19 unused). The
 * forms below write or read it; each gives the same bits as the form
 * without it. */
wst_status_t wst_hier_xq_table(const void *x, void *table, int32_t in_f);

/* wst_gemv_int4_hier_ex with the input's table (from wst_hier_xq_table or a
 * producer below) in place of x. */
wst_status_t wst_gemv_hier_xq(const void *qw, const void *si, const void *sb,
                              const void *table, const void *bias, void *y, int32_t in_f,
                              int32_t out_f, int32_t accum);

/* wst_gemv_hier_swiglu that also writes the table of out (inter / 32 entries;
 * inter a multiple of 32): the down projection's input. */
wst_status_t wst_gemv_hier_swiglu_xq(const void *qw, const void *si, const void *sb,
                                     const void *x, const void *norm_w, float eps, void *out,
                                     void *table, int32_t in_f, int32_t inter);

/* wst_attn_decode_fused whose merge also writes the table of out
 * (n_q * head_dim / 32 entries): the o projection's input. */
wst_status_t wst_attn_decode_fused_xq(void *qkv, void *k_cache, void *v_cache,
                                      const void *cos_tab, const void *sin_tab, void *partials,
                                      void *out, void *table, int32_t n_q, int32_t n_kv,
                                      int32_t head_dim, const void *pos, int32_t max_seq,
                                      float scale, const void *q_norm_w, const void *k_norm_w,
                                      float eps);

/* Chunk (prefill) fused forms, each bit-identical to the unfused ABI sequence
 * it replaces (tested so):
 *
 * wst_gemm_int4_hier(gate|up, x -> gu [n][2*inter]) + wst_swiglu_chunk(gu ->
 * act): act f16 [n][inter]; qw/si/sb are the fused gate|up matrix
 * [2*inter][in_f] (gate rows first). It never splits K, so where the unfused
 * GEMM would (outputs too few to fill the chip) the f32 sums are added in
 * another order and act may differ in the last place. */
wst_status_t wst_gemm_hier_swiglu_chunk(const void *qw, const void *si, const void *sb,
                                        const void *x, void *act, int32_t in_f, int32_t inter,
                                        int32_t n);
/* wst_gemm_int4_hier(..., y, accum) + wst_rmsnorm_chunk(y, norm_w, h_out):
 * y f32 [n][out_f] (the residual stream), h_out f16 [n][out_f];
 * out_f <= 16384. */
wst_status_t wst_gemm_hier_norm_chunk(const void *qw, const void *si, const void *sb,
                                      const void *x, const void *bias, void *y, int32_t in_f,
                                      int32_t out_f, int32_t n, int32_t accum,
                                      const void *norm_w, float eps, void *h_out);
/* wst_gemm_int4_hier(qkv weights, x -> qkv, bias) + wst_rope_cache_chunk:
 * qkv f32 [n][(n_q+2*n_kv)*head_dim] ends as the unfused pair leaves it
 * (q rotated, k and v as computed), k/v rows appended to the caches at
 * pos0 .. pos0+n-1; head_dim <= 128. */
wst_status_t wst_gemm_hier_rope_chunk(const void *qw, const void *si, const void *sb,
                                      const void *x, const void *bias, void *qkv, int32_t in_f,
                                      void *k_cache, void *v_cache, const void *cos_tab,
                                      const void *sin_tab, int32_t n_q, int32_t n_kv,
                                      int32_t head_dim, int32_t pos0, int32_t n,
                                      int32_t max_seq, const void *q_norm_w,
                                      const void *k_norm_w, float eps);

/* The same four chunk GEMM forms (and the plain one) over n tokens that hold
 * several chunks, with the tiling and split-K plan of a plan_n-token chunk
 * repeated over the n tokens: each token gets the bits a call of plan_n
 * tokens gives it (n = plan_n is the call above); plan_n = 0 plans for the
 * n tokens themselves. The batched prefill uses them to run a layer's op for
 * every full chunk in one launch. */
wst_status_t wst_gemm_int4_hier_chunks(const void *qw, const void *si, const void *sb,
                                       const void *x, const void *bias, void *y, int32_t in_f,
                                       int32_t out_f, int32_t n, int32_t accum, int32_t plan_n);
wst_status_t wst_gemm_hier_swiglu_chunks(const void *qw, const void *si, const void *sb,
                                         const void *x, void *act, int32_t in_f, int32_t inter,
                                         int32_t n, int32_t plan_n);
wst_status_t wst_gemm_hier_norm_chunks(const void *qw, const void *si, const void *sb,
                                       const void *x, const void *bias, void *y, int32_t in_f,
                                       int32_t out_f, int32_t n, int32_t accum,
                                       const void *norm_w, float eps, void *h_out,
                                       int32_t plan_n);
wst_status_t wst_gemm_hier_rope_chunks(const void *qw, const void *si, const void *sb,
                                       const void *x, const void *bias, void *qkv, int32_t in_f,
                                       void *k_cache, void *v_cache, const void *cos_tab,
                                       const void *sin_tab, int32_t n_q, int32_t n_kv,
                                       int32_t head_dim, int32_t pos0, int32_t n,
                                       int32_t max_seq, const void *q_norm_w,
                                       const void *k_norm_w, float eps, int32_t plan_n);

/* ------------------------------------------------------------ measurement */

/* One launch of the library's streaming-read kernel (16-byte nontemporal
 * loads, four in flight per lane, 8 blocks of 256 per CU) over bytes of buf
 * (16-byte aligned); sink is 16 writable bytes. The floor a GEMV of the same
 * bytes is compared with (bench.py --config 1). */
wst_status_t wst_stream_read(const void *buf, size_t bytes, void *sink);

/* ------------------------------------------------- no-allocation entry */

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): wst_gemm_int4_hier with the same arguments and the same
 * kernels, but its split-K partial sums go to a static 24 MiB device array
 * (one per GPU, held until the process ends) instead of the library's lazily
 * allocated scratch. Nothing is allocated or freed. A shape whose partials
 * need more than 24 MiB is refused with WST_ERR_SHAPE (the split plan keeps
 * them below (CUs + output tiles) x 64 KiB, under 24 MiB on 256 CUs). Every call on
 * one GPU shares that array: calls that overlap on one GPU (other threads'
 * streams) race. The partials are fully written before they are read, so no
 * state carries over between calls. */
wst_status_t wst_gemm_int4_hier_noalloc(const void *qw, const void *si, const void *sb,
                                        const void *x, const void *bias, void *y,
                                        int32_t in_f, int32_t out_f, int32_t n, int32_t accum);

#ifdef __cplusplus
}
#endif

#endif /* WHETSTONE_EXT_H */
