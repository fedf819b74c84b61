/* whetstone_engine.h -- the batch=1 decode engine above the C ABI.
 *
 * A C++ restatement of the reference's caller side (crates/whetstone-core:
 * Engine in engine.rs, ModelWeights in model.rs, the safe bindings of
 * whetstone-kernels/src), which cannot be built here (no Rust toolchain). It
 * drives libwhetstone_hip.so only through include/whetstone.h and
 * include/whetstone_ext.h, and exposes a C API so Python (tests, bench.py) and
 * any FFI can run the token loop.
 *
 * Two step implementations compute the same bits:
 *   WSE_STEP_REFERENCE  the reference's launch sequence (engine.rs:512-572):
 *                       rmsnorm, GEMV, rope_cache, attn (split+merge), GEMV,
 *                       rmsnorm, GEMV, swiglu, GEMV per layer; ~11 launches/layer
 *   WSE_STEP_FUSED      the MI355X sequence: RMSNorm folded into the GEMV
 *                       prologue, RoPE/KV-append folded into attention, SwiGLU
 *                       into the gate|up epilogue; 5 launches per layer.
 */
#ifndef WHETSTONE_ENGINE_H
#define WHETSTONE_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#include "whetstone.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Model dimensions (crates/whetstone-core/src/config.rs:26-87, the subset the
 * decode path reads). */
typedef struct {
  int32_t n_layers, hidden, n_q, n_kv, head_dim, inter, vocab;
  int32_t tied;      /* lm_head is the embedding matrix */
  int32_t qkv_bias;  /* q/k/v carry biases (Qwen2) */
  int32_t qk_norm;   /* per-head q/k RMSNorm gains (Qwen3-style) */
  int32_t rescore_k; /* > 0: keep an f16 head copy and rescore the top k */
  float eps;
  double rope_theta;
  /* RoPE frequency schedule (decode.rs RopeScaling): 0 none, 1 Llama-3
   * piecewise (factor, low/high frequency factors, original context). */
  int32_t rope_llama3;
  int32_t rope_orig_max;
  double rope_factor, rope_low_freq, rope_high_freq;
} wse_config_t;

typedef struct wse_model wse_model_t;
/* Message of the last engine-level refusal on this thread (kernel-level
 * failures report through wst_last_error). Never NULL. */
const char *wse_last_error(void);
typedef struct wse_engine wse_engine_t;

enum { WSE_STEP_REFERENCE = 0, WSE_STEP_FUSED = 1 };

/* Stage buckets of wse_engine_profile (engine/profile.rs:172-307). */
enum {
  WSE_STAGE_EMBED = 0,
  WSE_STAGE_QKV = 1,     /* (rmsnorm +) qkv GEMV */
  WSE_STAGE_ATTN = 2,    /* (rope +) attention */
  WSE_STAGE_O = 3,
  WSE_STAGE_GATE_UP = 4, /* (rmsnorm +) gate|up GEMV (+ swiglu) */
  WSE_STAGE_DOWN = 5,
  WSE_STAGE_HEAD = 6,    /* final norm + head GEMV */
  WSE_STAGE_RESCORE = 7,
  WSE_STAGE_SAMPLE = 8,  /* argmax + position advance */
  WSE_STAGES = 9
};

/* Seeded synthetic weights generated and packed on the device: every Linear
 * and the Embedding ~N(0,0.02) -> int4-hier-g32, q/k/v biases 0, norm gains 1,
 * QK-norm gains 1+N(0,0.02), f16 head copy when rescore_k > 0. Same streams as
 * the CPU oracle (oracle/oracle.c), so both hold identical bytes. */
wst_status_t wse_model_synthetic(const wse_config_t *cfg, uint64_t seed, wse_model_t **out);
void wse_model_free(wse_model_t *m);
/* Device pointers of a packed matrix: "embed", "lm_head", "L<l>.qkv",
 * "L<l>.o", "L<l>.gate_up", "L<l>.down". */
wst_status_t wse_model_tensor(wse_model_t *m, const char *name, void **qw, void **si, void **sb,
                              int64_t *in_f, int64_t *out_f);
/* Device pointer and length of an f16 tensor of the model: "final_norm",
 * "rescore" (the head's f16 copy), "embed16" / "lm_head16" (dense tables),
 * "L<l>.in_norm", "L<l>.post_norm", "L<l>.qkv_bias", "L<l>.q_norm",
 * "L<l>.k_norm". WST_ERR_SHAPE when the model has no such tensor. */
wst_status_t wse_model_vector(wse_model_t *m, const char *name, void **ptr, int64_t *n);
/* Weight bytes a decode step streams (packed matrices + norms + biases). */
uint64_t wse_model_weight_bytes(const wse_model_t *m);
/* The model's dimensions and flags as built or loaded. */
wst_status_t wse_model_config(const wse_model_t *m, wse_config_t *out);

/* ----------------------------------------------------------- .wstone files
 * The converted-model container (crates/whetstone-quant/src/format.rs,
 * docs/FORMAT.md). Refusals return WST_ERR_INVALID_ARG (format, config) or
 * WST_ERR_SHAPE with the reason in wse_last_error(). */

/* The container's 64-bit hash (format.rs:225-232): FNV-1a's offset basis and
 * xor-then-multiply, with the multiplier 0x1000000001B3 the reference uses. */
uint64_t wse_fnv1a(const void *bytes, size_t n);
/* Parses and validates a file's header as format.rs:427-516 does: magic,
 * version, header hash, the JSON, every blob range inside the file and
 * 256-byte aligned, and the blobs each kind requires. verify != 0 also checks
 * every payload hash (format.rs:518-547). Host only; needs no GPU. */
wst_status_t wse_wstone_check(const char *path, int32_t verify, int32_t *n_tensors);
/* The embedded config.json parsed and validated (config.rs:26-262: defaults,
 * architecture whitelist, MoE and unsupported RoPE scaling refused). Host only. */
wst_status_t wse_wstone_config(const char *path, wse_config_t *out);
/* The same parse and validation of a config.json text. Host only. */
wst_status_t wse_config_from_json(const char *json, wse_config_t *out);
/* Loads a file into a device model (model.rs:454-638): q|k|v and gate|up
 * fused by row append, q/k/v biases fused with zero fill, QK-norm gains when
 * present (both or neither), embedding and head as int4_hier_g32 or f16.
 * rescore_k: < 0 uses 64 when the file carries the head's ".rescore" f16 copy
 * (model.rs:814), 0 disables the rescore, > 0 sets k. */
wst_status_t wse_model_load_wstone(const char *path, int32_t rescore_k, wse_model_t **out);

wst_status_t wse_engine_create(wse_model_t *m, int32_t max_seq, int32_t step_mode,
                               wse_engine_t **out);
void wse_engine_free(wse_engine_t *e);
wst_status_t wse_engine_reset(wse_engine_t *e);
int32_t wse_engine_pos(const wse_engine_t *e);
wst_status_t wse_engine_set_pos(wse_engine_t *e, int32_t pos);
/* Synthetic context: KV caches of every layer filled for positions [0, n) with
 * f16 N(0,1) from (seed, stream 1000+layer); position set to n. */
wst_status_t wse_engine_fill_kv(wse_engine_t *e, uint64_t seed, int32_t n);
/* Engine::forward (engine.rs:418-430): token -> device cursor, one step. */
wst_status_t wse_engine_forward(wse_engine_t *e, int32_t token);
/* Engine::step (engine.rs:480-499): one step on the token already in the
 * device cursor (graph launch when captured). */
wst_status_t wse_engine_step(wse_engine_t *e);
/* Engine::capture_graph (engine.rs:357-393): warm-up step, rewind, capture. */
wst_status_t wse_engine_capture_graph(wse_engine_t *e);
/* Engine::chunk_width (engine.rs:682-698): tokens per chunk pass, the
 * kernels' wst_chunk_max_tokens() or WHETSTONE_CHUNK_WIDTH=k (k >= 1) clamped
 * to it. */
wst_status_t wse_engine_chunk_width(wse_engine_t *e, int32_t *out);
wst_status_t wse_engine_max_seq(const wse_engine_t *e, int32_t *out);
/* Engine::forward_chunk_ex (engine.rs:731-844): 1 <= n <= chunk width tokens
 * appended at the current position in one pass over the weights. With
 * want_logits the final norm, the head (a chunk GEMM over all n rows, no
 * rescore) and the per-row argmax run; the last row's logits and pick go to
 * the single-token buffers, so step() and token() continue from there. */
wst_status_t wse_engine_forward_chunk(wse_engine_t *e, const int32_t *ids_host, int32_t n,
                                      int32_t want_logits);
/* Engine::chunk_picks (engine.rs:850-865): the greedy pick of each of the
 * first n rows of the last chunk pass that computed logits. */
wst_status_t wse_engine_chunk_picks(wse_engine_t *e, int32_t n, int32_t *out_host);
/* Engine::rewind (engine.rs:870-881): moves the cache cursor back to pos
 * (<= the current position); later entries are overwritten, not cleared. */
wst_status_t wse_engine_rewind(wse_engine_t *e, int32_t pos);
/* Engine::prefill (engine.rs:890-905): chunks of the chunk width; only the
 * last chunk computes logits (every row's, as forward_chunk), leaving the
 * last row's greedy pick in the token cursor. */
wst_status_t wse_engine_prefill(wse_engine_t *e, const int32_t *ids_host, int32_t n,
                                 int32_t chunked);
/* Greedy generation (engine.rs:909-956): prefill, then up to n_new tokens,
 * each read back (4 bytes) from the device cursor. Generation stops early when
 * the context is full; *n_out receives how many tokens were written. */
wst_status_t wse_engine_generate(wse_engine_t *e, const int32_t *prompt_host, int32_t n_prompt,
                                 int32_t n_new, int32_t chunked, int32_t *out_tokens_host,
                                 int32_t *n_out);
wst_status_t wse_engine_token(wse_engine_t *e, int32_t *out);
/* SpecConfig / SpecStats (speculate.rs:58-115). */
typedef struct {
  int32_t draft;     /* tokens per verification pass, the confirmed one included */
  int32_t ngram_max; /* longest n-gram matched against the history */
  int32_t ngram_min; /* shortest n-gram accepted as a match */
} wse_spec_config_t;
typedef struct {
  int64_t rounds, empty_rounds, proposed, accepted;
} wse_spec_stats_t;
/* speculate::propose (speculate.rs:122-150): up to `want` tokens that followed
 * the most recent earlier occurrence of the history's last n tokens, trying n
 * from min(ngram_max, n_history - 1) down to ngram_min. Returns the count
 * written to out (0: no match). Host-only. */
int32_t wse_spec_propose(const int32_t *history, int32_t n_history, int32_t ngram_max,
                         int32_t ngram_min, int32_t want, int32_t *out);
/* speculate::generate (speculate.rs:152-260): greedy generation with the
 * n-gram draft verified by chunk passes of min(chunk width, draft) tokens.
 * Writes up to max_new tokens to out_tokens_host and their count to n_out. */
wst_status_t wse_speculate_generate(wse_engine_t *e, const int32_t *prompt_host, int32_t n_prompt,
                                    int32_t max_new, const wse_spec_config_t *cfg,
                                    int32_t *out_tokens_host, int32_t *n_out,
                                    wse_spec_stats_t *stats);
/* SamplingConfig (engine.rs:104-124). temperature <= 0 means greedy; top_p >= 1,
 * top_k = 0, min_p = 0 and repeat_penalty = 1 each disable their filter. */
typedef struct {
  float temperature;
  float top_p;
  int32_t top_k;
  float min_p;
  float repeat_penalty;
  int32_t repeat_last_n;
  uint64_t seed;
} wse_sampling_config_t;
/* sample_with (engine.rs:987-1096), host only: repetition penalty over the last
 * repeat_last_n of recent[0..n_recent) (oldest first; applied in place to
 * logits, once per occurrence), then argmax (ties to the last maximum) when
 * temperature <= 0, else a pool of the top min(top_k or 512, 512) logits
 * (equal logits ordered by index, where the reference leaves it unspecified),
 * temperature, min-p, top-p and one draw with
 * u = splitmix64(seed ^ step * 0x9E3779B97F4A7C15) / 2^64 * mass. */
int32_t wse_sample_with(float *logits, int32_t n, const wse_sampling_config_t *cfg,
                        uint64_t step, const int32_t *recent, int32_t n_recent);
uint64_t wse_splitmix64(uint64_t z);
/* Engine::sample (engine.rs:648-673): cfg NULL is Sampler::Greedy (the device
 * cursor's token, a 4-byte read); otherwise the logits come to the host, are
 * sampled with the engine's recent-token window (the last 2048 tokens fed or
 * chosen since the last reset), and the choice is written to the device
 * cursor. The chosen token joins the window. */
wst_status_t wse_engine_sample(wse_engine_t *e, const wse_sampling_config_t *cfg, uint64_t step,
                               int32_t *out);
/* Engine::generate with a sampler (engine.rs:909-956): prefill, then
 * next = sample(0); for each step: emit next, stop at the cache end, step,
 * next = sample(step + 1). Writes up to n_new tokens and their count. */
wst_status_t wse_engine_generate_sampled(wse_engine_t *e, const int32_t *prompt_host,
                                         int32_t n_prompt, int32_t n_new, int32_t chunked,
                                         const wse_sampling_config_t *cfg,
                                         int32_t *out_tokens_host, int32_t *n_out);
/* The recent-token window (oldest first): writes up to cap tokens, returns
 * the window's length. Engine::unnote (engine.rs:462-467) drops the last k. */
int32_t wse_engine_recent(const wse_engine_t *e, int32_t *out, int32_t cap);
void wse_engine_unnote(wse_engine_t *e, int32_t k);
/* Writes `token` into the device token cursor (the next step's input). */
wst_status_t wse_engine_set_token(wse_engine_t *e, int32_t token);
wst_status_t wse_engine_logits(wse_engine_t *e, float *out_host);
/* One eager step with an event at every stage boundary; adds the elapsed ms
 * per stage into stage_ms[WSE_STAGES] and launch counts into counts. */
wst_status_t wse_engine_profile_step(wse_engine_t *e, double *stage_ms, int32_t *counts);
/* Average duration of one launch of a stage's kernel in the fused step, timed
 * with events on the calling thread's stream over `reps` sweeps that launch
 * every layer's instance back to back (HEAD: the one head GEMV per sweep), and
 * the algorithmic bytes one launch moves (packed weights, norm gains, biases,
 * activations read and written; ATTN: the K/V rows of every cached position).
 * Stages QKV, ATTN, O, GATE_UP, DOWN, HEAD; WSE_STEP_FUSED engines only.
 * Activations are overwritten and the current position's K/V rewritten with
 * the same values; the position and token cursor are unchanged. */
wst_status_t wse_engine_time_stage(wse_engine_t *e, int32_t stage, int32_t reps,
                                   double *us_per_launch, uint64_t *bytes_per_launch);
/* Engine::cross_entropy (engine.rs:585-618): for each of the first
 * min(n_tokens / window, max_windows) windows, reset the cache and feed
 * tokens 0..window-2 of the window, adding -log softmax(logits)[next token]
 * on the device (wst_nll). Returns the summed NLL (nats) and the number of
 * predicted positions; perplexity = exp(nll_sum / positions). The window must
 * hold at least 2 tokens and fit the cache (WST_ERR_SHAPE otherwise). */
wst_status_t wse_engine_cross_entropy(wse_engine_t *e, const int32_t *tokens_host,
                                      int64_t n_tokens, int32_t window, int32_t max_windows,
                                      double *nll_sum, int64_t *positions);
/* Algorithmic bytes of one decode step at the current position. */
uint64_t wse_engine_step_bytes(const wse_engine_t *e);

#ifdef __cplusplus
}
#endif

#endif /* WHETSTONE_ENGINE_H */
