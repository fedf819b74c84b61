// The batch=1 decode engine: a C++ restatement of the reference's caller side
// (crates/whetstone-core/src/engine.rs Engine, model.rs ModelWeights, and the
// shape checks of crates/whetstone-kernels/src/*.rs). It talks to the GPU only
// through the C ABI of libwhetstone_hip.so (include/whetstone.h,
// include/whetstone_ext.h) -- the same boundary the reference's Rust engine
// crosses -- and is compiled as plain host C++.
#include "whetstone_engine.h"

#include <errno.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <deque>
#include <string>
#include <vector>

#include "engine_internal.hpp"
#include "whetstone.h"
#include "whetstone_ext.h"

namespace wse {

thread_local char g_msg[512];

wst_status_t shape_error(const char *fmt, const char *what) {
  snprintf(g_msg, sizeof(g_msg), fmt, what);
  return WST_ERR_SHAPE;
}

}  // namespace wse

using namespace wse;

namespace {

// Fixture streams, shared with the CPU oracle (oracle/oracle.c).
enum { ST_Q = 0, ST_K = 1, ST_V = 2, ST_O = 3, ST_GATE = 4, ST_UP = 5, ST_DOWN = 6, ST_QN = 7, ST_KN = 8 };
inline uint64_t stream_of(int l, int t) { return (uint64_t)l * 16u + (uint64_t)t + 16u; }
constexpr uint64_t ST_EMBED = 1, ST_HEAD = 2;

}  // namespace

struct wse_engine {
  wse_model *m = nullptr;
  int max_seq = 0, mode = WSE_STEP_FUSED, pos = 0;
  void *x = nullptr, *h = nullptr, *qkv = nullptr, *attn = nullptr, *gu = nullptr,
       *act = nullptr, *logits = nullptr, *token = nullptr, *pos_dev = nullptr;
  // The int4-hier GEMV activation table of the o and down inputs, written by
  // their producers (the attention merge, the gate|up SwiGLU) in the fused step.
  void *xq = nullptr;
  std::vector<void *> kc, vc;
  void *partials = nullptr, *cos_tab = nullptr, *sin_tab = nullptr;
  // head rescore (rescore.rs:75-118)
  int rs_k = 0, rs_cap = 0, rs_grid = 0, rs_nblocks = 0;
  void *rs_thresh = nullptr, *rs_scratch = nullptr, *rs_count = nullptr, *rs_idx = nullptr;
  void *graph = nullptr;
  // chunk scratch, allocated on first use
  int chunk_width = 0;
  void *c_tokens = nullptr, *c_x = nullptr, *c_h = nullptr, *c_qkv = nullptr, *c_attn = nullptr,
       *c_act = nullptr;
  void *c_logits = nullptr, *c_picks = nullptr;  // the chunk head's, on first use
  // Buffers of a prefill whose full chunks share their launches (b_cap tokens).
  int b_cap = 0;
  void *b_tokens = nullptr, *b_x = nullptr, *b_h = nullptr, *b_qkv = nullptr,
       *b_attn = nullptr, *b_act = nullptr;
  void *nll_acc = nullptr;                       // cross_entropy's (sum, count), on first use
  std::deque<int32_t> recent;                    // repetition-penalty window (RECENT_CAP)
  bool c_ran = false;                            // a chunk pass has left picks
  std::vector<void *> events;
  Arena arena;
};

wst_status_t wse::alloc_mat(Arena &a, Mat &m, int64_t in_f, int64_t out_f) {
  m.in_f = in_f;
  m.out_f = out_f;
  TRY(a.alloc(&m.qw, (size_t)(out_f * in_f / 2), false));
  TRY(a.alloc(&m.si, (size_t)(out_f * in_f / 32), false));
  TRY(a.alloc(&m.sb, (size_t)(out_f * 4), false));
  return WST_OK;
}

wst_status_t wse::check_config(const wse_config_t *c) {
  if (!c || c->n_layers <= 0 || c->hidden <= 0 || c->n_q <= 0 || c->n_kv <= 0 ||
      c->head_dim <= 0 || c->inter <= 0 || c->vocab <= 0) {
    snprintf(g_msg, sizeof(g_msg), "config: non-positive dimension");
    return WST_ERR_SHAPE;
  }
  if (c->hidden % 32 || c->inter % 32 || (c->n_q * c->head_dim) % 32 || c->n_q % c->n_kv ||
      c->head_dim % 2) {
    snprintf(g_msg, sizeof(g_msg),
             "config: hidden, intermediate and n_q*head_dim must be multiples of 32, n_q a "
             "multiple of n_kv, head_dim even (config.rs:206-247)");
    return WST_ERR_SHAPE;
  }
  return WST_OK;
}

extern "C" {

const char *wse_last_error(void) { return g_msg; }

// ------------------------------------------------------------------- model


static wst_status_t pack_part(Mat &m, int64_t row0, int64_t rows, uint64_t seed, uint64_t stream) {
  return wst_fixture_pack_hier(m.qw, m.si, m.sb, m.in_f, row0, rows, seed, stream, 0.02f);
}

static wst_status_t f16_fill(Arena &a, void **out, size_t n, uint64_t seed, uint64_t stream,
                             float std_, float offset) {
  TRY(a.alloc(out, n * 2, false));
  return wst_fixture_normal_f16(*out, n, seed, stream, 0, std_, offset);
}


static wst_status_t model_build(wse_model *m, uint64_t seed) {
  const wse_config_t &c = m->c;
  const int64_t H = c.hidden, hd = c.head_dim, I = c.inter, V = c.vocab;
  const int64_t nq = (int64_t)c.n_q * hd, nk = (int64_t)c.n_kv * hd;
  Arena &a = m->arena;
  TRY(alloc_mat(a, m->embed, H, V));
  TRY(pack_part(m->embed, 0, V, seed, ST_EMBED));
  if (!c.tied) {
    TRY(alloc_mat(a, m->lm_head, H, V));
    TRY(pack_part(m->lm_head, 0, V, seed, ST_HEAD));
  }
  TRY(f16_fill(a, &m->final_norm, (size_t)H, seed, 0, 0.0f, 1.0f));
  if (c.rescore_k > 0)
    TRY(f16_fill(a, &m->rescore, (size_t)(V * H), seed, c.tied ? ST_EMBED : ST_HEAD, 0.02f, 0.0f));
  m->layers.resize((size_t)c.n_layers);
  for (int l = 0; l < c.n_layers; ++l) {
    Layer &L = m->layers[(size_t)l];
    TRY(alloc_mat(a, L.qkv, H, nq + 2 * nk));
    TRY(pack_part(L.qkv, 0, nq, seed, stream_of(l, ST_Q)));
    TRY(pack_part(L.qkv, nq, nk, seed, stream_of(l, ST_K)));
    TRY(pack_part(L.qkv, nq + nk, nk, seed, stream_of(l, ST_V)));
    TRY(alloc_mat(a, L.o, nq, H));
    TRY(pack_part(L.o, 0, H, seed, stream_of(l, ST_O)));
    TRY(alloc_mat(a, L.gate_up, H, 2 * I));
    TRY(pack_part(L.gate_up, 0, I, seed, stream_of(l, ST_GATE)));
    TRY(pack_part(L.gate_up, I, I, seed, stream_of(l, ST_UP)));
    TRY(alloc_mat(a, L.down, I, H));
    TRY(pack_part(L.down, 0, H, seed, stream_of(l, ST_DOWN)));
    if (c.qkv_bias) TRY(a.alloc(&L.qkv_bias, (size_t)(nq + 2 * nk) * 2, true));
    TRY(f16_fill(a, &L.in_norm, (size_t)H, seed, 0, 0.0f, 1.0f));
    TRY(f16_fill(a, &L.post_norm, (size_t)H, seed, 0, 0.0f, 1.0f));
    if (c.qk_norm) {
      TRY(f16_fill(a, &L.q_norm, (size_t)hd, seed, stream_of(l, ST_QN), 0.02f, 1.0f));
      TRY(f16_fill(a, &L.k_norm, (size_t)hd, seed, stream_of(l, ST_KN), 0.02f, 1.0f));
    }
  }
  return wst_device_synchronize();
}

wst_status_t wse_model_synthetic(const wse_config_t *cfg, uint64_t seed, wse_model_t **out) {
  if (!out) return WST_ERR_INVALID_ARG;
  *out = nullptr;
  TRY(check_config(cfg));
  wse_model *m = new wse_model();
  m->c = *cfg;
  const wst_status_t st = model_build(m, seed);
  if (st != WST_OK) {
    wse_model_free(m);
    return st;
  }
  *out = m;
  return WST_OK;
}

void wse_model_free(wse_model_t *m) {
  if (!m) return;
  m->arena.free_all();
  delete m;
}

wst_status_t wse_model_tensor(wse_model_t *m, const char *name, void **qw, void **si, void **sb,
                              int64_t *in_f, int64_t *out_f) {
  if (!m || !name || !qw || !si || !sb || !in_f || !out_f) return WST_ERR_INVALID_ARG;
  const Mat *p = nullptr;
  if (!strcmp(name, "embed")) p = &m->embed;
  else if (!strcmp(name, "lm_head")) p = &m->head();
  else {
    int l = -1;
    char what[32] = {0};
    if (sscanf(name, "L%d.%31s", &l, what) == 2 && l >= 0 && l < m->c.n_layers) {
      const Layer &L = m->layers[(size_t)l];
      if (!strcmp(what, "qkv")) p = &L.qkv;
      else if (!strcmp(what, "o")) p = &L.o;
      else if (!strcmp(what, "gate_up")) p = &L.gate_up;
      else if (!strcmp(what, "down")) p = &L.down;
    }
  }
  if (!p) return shape_error("unknown tensor %s", name);
  *qw = p->qw;
  *si = p->si;
  *sb = p->sb;
  *in_f = p->in_f;
  *out_f = p->out_f;
  return WST_OK;
}

wst_status_t wse_model_vector(wse_model_t *m, const char *name, void **ptr, int64_t *n) {
  if (!m || !name || !ptr || !n) return WST_ERR_INVALID_ARG;
  const wse_config_t &c = m->c;
  void *p = nullptr;
  int64_t len = 0;
  if (!strcmp(name, "final_norm")) {
    p = m->final_norm;
    len = c.hidden;
  } else if (!strcmp(name, "rescore")) {
    p = m->rescore;
    len = (int64_t)c.vocab * c.hidden;
  } else if (!strcmp(name, "embed16")) {
    p = m->embed.w16;
    len = (int64_t)c.vocab * c.hidden;
  } else if (!strcmp(name, "lm_head16")) {
    p = m->head().w16;
    len = (int64_t)c.vocab * c.hidden;
  } else {
    int l = -1;
    char what[32] = {0};
    if (sscanf(name, "L%d.%31s", &l, what) == 2 && l >= 0 && l < c.n_layers) {
      const Layer &L = m->layers[(size_t)l];
      if (!strcmp(what, "in_norm")) {
        p = L.in_norm;
        len = c.hidden;
      } else if (!strcmp(what, "post_norm")) {
        p = L.post_norm;
        len = c.hidden;
      } else if (!strcmp(what, "qkv_bias")) {
        p = L.qkv_bias;
        len = (int64_t)(c.n_q + 2 * c.n_kv) * c.head_dim;
      } else if (!strcmp(what, "q_norm")) {
        p = L.q_norm;
        len = c.head_dim;
      } else if (!strcmp(what, "k_norm")) {
        p = L.k_norm;
        len = c.head_dim;
      }
    }
  }
  if (!p) return shape_error("no f16 vector %s in this model", name);
  *ptr = p;
  *n = len;
  return WST_OK;
}

// config.rs:347-362 (decode_resident) restated for this layout: every packed
// matrix the step streams, plus norm gains and biases. The embedding-row gather
// and the rescore copy are excluded, as the reference excludes them.
uint64_t wse_model_weight_bytes(const wse_model_t *m) {
  if (!m) return 0;
  const wse_config_t &c = m->c;
  uint64_t b = m->head().bytes();
  for (const Layer &L : m->layers) b += L.qkv.bytes() + L.o.bytes() + L.gate_up.bytes() + L.down.bytes();
  b += (uint64_t)(2 * c.n_layers + 1) * (uint64_t)c.hidden * 2;
  if (c.qkv_bias) b += (uint64_t)c.n_layers * (uint64_t)(c.n_q + 2 * c.n_kv) * c.head_dim * 2;
  if (c.qk_norm) b += (uint64_t)c.n_layers * 2 * (uint64_t)c.head_dim * 2;
  return b;
}

// ------------------------------------------------------------------ engine

static wst_status_t rope_table(wse_engine *e) {
  // decode.rs:95-147: invf = theta^(-j/half) in f64 (Llama-3 schedule: divided
  // by factor past the low-frequency wavelength, blended across the band
  // between), angle p*invf in f64, narrowed to f32.
  const wse_config_t &c = e->m->c;
  const int hd = c.head_dim, half = hd / 2;
  std::vector<float> cs((size_t)e->max_seq * half), sn((size_t)e->max_seq * half);
  for (int j = 0; j < half; ++j) {
    double invf = pow(c.rope_theta, -(double)j / (double)half);
    if (c.rope_llama3) {
      const double orig = (double)c.rope_orig_max;
      const double low_wl = orig / c.rope_low_freq, high_wl = orig / c.rope_high_freq;
      const double wavelen = 2.0 * M_PI / invf;
      if (wavelen > low_wl) {
        invf /= c.rope_factor;
      } else if (wavelen > high_wl) {
        const double smooth =
            (orig / wavelen - c.rope_low_freq) / (c.rope_high_freq - c.rope_low_freq);
        invf = (1.0 - smooth) * (invf / c.rope_factor) + smooth * invf;
      }
    }
    for (int p = 0; p < e->max_seq; ++p) {
      const double a = (double)p * invf;
      cs[(size_t)p * half + j] = (float)cos(a);
      sn[(size_t)p * half + j] = (float)sin(a);
    }
  }
  TRY(e->arena.alloc(&e->cos_tab, cs.size() * 4, false));
  TRY(e->arena.alloc(&e->sin_tab, sn.size() * 4, false));
  TRY(wst_memcpy_h2d(e->cos_tab, cs.data(), cs.size() * 4));
  TRY(wst_memcpy_h2d(e->sin_tab, sn.data(), sn.size() * 4));
  return WST_OK;
}

static wst_status_t engine_build(wse_engine *e) {
  const wse_config_t &c = e->m->c;
  const size_t H = (size_t)c.hidden, hd = (size_t)c.head_dim, I = (size_t)c.inter,
               V = (size_t)c.vocab;
  const size_t nqkv = (size_t)(c.n_q + 2 * c.n_kv) * hd;
  Arena &a = e->arena;
  TRY(a.alloc(&e->x, H * 4, true));
  TRY(a.alloc(&e->h, H * 2, true));
  TRY(a.alloc(&e->qkv, nqkv * 4, true));
  TRY(a.alloc(&e->attn, (size_t)c.n_q * hd * 2, true));
  TRY(a.alloc(&e->gu, 2 * I * 4, true));
  TRY(a.alloc(&e->act, I * 2, true));
  TRY(a.alloc(&e->xq, (I > (size_t)c.n_q * hd ? I : (size_t)c.n_q * hd) / 32 * 80, true));
  TRY(a.alloc(&e->logits, V * 4, true));
  TRY(a.alloc(&e->token, 4, true));
  TRY(a.alloc(&e->pos_dev, 4, true));
  const size_t kv = (size_t)c.n_kv * (size_t)e->max_seq * hd * 2;
  e->kc.resize((size_t)c.n_layers);
  e->vc.resize((size_t)c.n_layers);
  for (int l = 0; l < c.n_layers; ++l) {
    TRY(a.alloc(&e->kc[(size_t)l], kv, true));
    TRY(a.alloc(&e->vc[(size_t)l], kv, true));
  }
  const int pf = wst_attn_partial_floats(c.n_q, c.head_dim, e->max_seq);
  TRY(a.alloc(&e->partials, (size_t)(pf > 0 ? pf : 1) * 4, true));
  TRY(rope_table(e));
  if (c.rescore_k > 0 && e->m->rescore) {
    // rescore.rs:90-118
    e->rs_k = c.rescore_k;
    e->rs_cap = c.rescore_k * 16 < c.vocab ? c.rescore_k * 16 : c.vocab;
    if (e->rs_cap < e->rs_k) e->rs_cap = e->rs_k;
    e->rs_grid = e->rs_cap < 256 ? e->rs_cap : 256;
    int nb = (c.vocab + 255) / 256;
    e->rs_nblocks = nb < 1 ? 1 : (nb > 512 ? 512 : nb);
    TRY(a.alloc(&e->rs_thresh, 4, true));
    TRY(a.alloc(&e->rs_scratch, (size_t)(e->rs_nblocks + 1 + 12) * 4, true));
    TRY(a.alloc(&e->rs_count, 4, true));
    TRY(a.alloc(&e->rs_idx, (size_t)e->rs_cap * 4, true));
  }
  return WST_OK;
}

wst_status_t wse_engine_create(wse_model_t *m, int32_t max_seq, int32_t step_mode,
                               wse_engine_t **out) {
  if (!m || !out || max_seq <= 0) return WST_ERR_INVALID_ARG;
  *out = nullptr;
  wse_engine *e = new wse_engine();
  e->m = m;
  e->max_seq = max_seq;
  e->mode = step_mode == WSE_STEP_REFERENCE ? WSE_STEP_REFERENCE : WSE_STEP_FUSED;
  if (e->mode == WSE_STEP_FUSED && m->c.head_dim > 128) e->mode = WSE_STEP_REFERENCE;
  const wst_status_t st = engine_build(e);
  if (st != WST_OK) {
    wse_engine_free(e);
    return st;
  }
  *out = e;
  return WST_OK;
}

void wse_engine_free(wse_engine_t *e) {
  if (!e) return;
  if (e->graph) wst_graph_destroy(e->graph);
  for (void *ev : e->events) wst_event_destroy(ev);
  e->arena.free_all();
  delete e;
}

int32_t wse_engine_pos(const wse_engine_t *e) { return e ? e->pos : -1; }

wst_status_t wse_engine_set_pos(wse_engine_t *e, int32_t pos) {
  if (!e || pos < 0 || pos > e->max_seq) return WST_ERR_INVALID_ARG;
  e->pos = pos;
  return wst_memcpy_h2d(e->pos_dev, &pos, 4);
}

// Engine::reset (engine.rs:434-439): position zero and an empty window.
wst_status_t wse_engine_reset(wse_engine_t *e) {
  if (!e) return WST_ERR_INVALID_ARG;
  e->recent.clear();
  return wse_engine_set_pos(e, 0);
}

// Engine::note (engine.rs:469-474): the last RECENT_CAP = 2048 tokens.
static void note(wse_engine *e, int32_t t) {
  if (e->recent.size() == 2048) e->recent.pop_front();
  e->recent.push_back(t);
}

void wse_engine_unnote(wse_engine_t *e, int32_t k) {
  if (!e) return;
  for (int32_t i = 0; i < k && !e->recent.empty(); ++i) e->recent.pop_back();
}

int32_t wse_engine_recent(const wse_engine_t *e, int32_t *out, int32_t cap) {
  if (!e) return 0;
  int32_t i = 0;
  for (int32_t t : e->recent) {
    if (out && i < cap) out[i] = t;
    ++i;
  }
  return i;
}

wst_status_t wse_engine_fill_kv(wse_engine_t *e, uint64_t seed, int32_t n) {
  if (!e || n < 0 || n > e->max_seq) return WST_ERR_INVALID_ARG;
  const wse_config_t &c = e->m->c;
  for (int l = 0; l < c.n_layers; ++l)
    TRY(wst_fixture_fill_kv(e->kc[(size_t)l], e->vc[(size_t)l], c.n_kv, e->max_seq, c.head_dim, n,
                            seed, 1000u + (uint64_t)l));
  TRY(wst_device_synchronize());
  return wse_engine_set_pos(e, n);
}

// ----------------------------------------------------------- the decode step

struct Marks {
  wse_engine *e;
  bool on;
  int next = 0;
  std::vector<int> stage;  // stage of the interval ending at each mark
  wst_status_t mark(int st) {
    if (!on) return WST_OK;
    if ((size_t)next >= e->events.size()) {
      void *ev = nullptr;
      TRY(wst_event_create(&ev));
      e->events.push_back(ev);
    }
    stage.push_back(st);
    return wst_event_record(e->events[(size_t)next++]);
  }
};

// Engine::step_eager (engine.rs:512-572) in either launch sequence.
// The embedding gather and the output projection: int4-hier or, for models
// converted with an f16 head (the reference converter's default), dense f16.
static wst_status_t embed_token(wse_engine *e) {
  const wse_model &m = *e->m;
  if (m.embed.dense())
    return wst_embed_fp16(m.embed.w16, e->token, e->x, m.c.hidden, m.c.vocab);
  return wst_embed_int4_hier(m.embed.qw, m.embed.si, m.embed.sb, e->token, e->x, m.c.hidden,
                             m.c.vocab);
}

// Final RMSNorm of x_last (f32 [H]) into e->h, then logits = head . h.
static wst_status_t head_logits(wse_engine *e, const void *x_last, bool fused) {
  const wse_model &m = *e->m;
  const Mat &head = m.head();
  const int H = m.c.hidden, V = m.c.vocab;
  if (head.dense()) {
    TRY(wst_rmsnorm(x_last, m.final_norm, e->h, H, m.c.eps));
    return wst_gemv_fp16(head.w16, e->h, e->logits, H, V);
  }
  if (fused)
    return wst_gemv_hier_rmsnorm(head.qw, head.si, head.sb, x_last, m.final_norm, m.c.eps, e->h,
                                 nullptr, e->logits, H, V, 0);
  TRY(wst_rmsnorm(x_last, m.final_norm, e->h, H, m.c.eps));
  return wst_gemv_int4_hier_ex(head.qw, head.si, head.sb, e->h, nullptr, e->logits, H, V, 0);
}

// The fused step merges the attention slices inside the o GEMV (one launch
// fewer per layer) when the cache has at most 8 slices of 16384 / head_dim
// positions; WSE_MERGE_IN_O=0 keeps the separate merge kernel.
static bool merge_in_o(const wse_engine *e) {
  const int hd = e->m->c.head_dim;
  if (e->mode != WSE_STEP_FUSED || (hd != 64 && hd != 128)) return false;
  const char *v = getenv("WSE_MERGE_IN_O");
  if (v && v[0] == '0') return false;
  const int P = wst_attn_slice_positions(hd, e->max_seq);
  return P > 0 && (e->max_seq + P - 1) / P <= 8;
}

// WSE_HEAD_ARGMAX=0 keeps the separate argmax launch after the head GEMV.
// The gate|up SwiGLU GEMV builds the down GEMV's activation table, so that
// the down GEMV's blocks do not each build it (both forms give the same
// bits). Used where the gate|up GEMV already takes rows 32 at a time (rows of
// at most 32 groups, four per wave: the 0.5B shape); on wider rows the
// grouping into 32-row units unbalances its grid (7B: 592 units on 512
// blocks) by more than the down GEMV saves. WSE_XQ=0 switches it off, 1
// forces it on every shape, 2 adds the attention merge building the o GEMV's
// table (measured slower on the 7B shape: the build lengthens the merge).
static int xq_mode() {
  const char *v = getenv("WSE_XQ");
  return v ? atoi(v) : -1;
}
static bool xq_on(const wse_engine *e) {
  const wse_config_t &c = e->m->c;
  if (e->mode != WSE_STEP_FUSED || c.inter % 32 != 0) return false;
  const int m = xq_mode();
  return m < 0 ? c.hidden <= 1024 : m >= 1;
}
static bool xq_o_on(const wse_engine *e) { return xq_on(e) && xq_mode() >= 2; }

static bool head_argmax_on() {
  const char *v = getenv("WSE_HEAD_ARGMAX");
  return !(v && v[0] == '0');
}

static wst_status_t step_eager(wse_engine *e, Marks &mk) {
  const wse_model &m = *e->m;
  const wse_config_t &c = m.c;
  const int H = c.hidden, hd = c.head_dim, nq = c.n_q, nkv = c.n_kv, I = c.inter, V = c.vocab;
  const int nqkv = (nq + 2 * nkv) * hd;
  const float eps = c.eps;
  const float scale = (float)(1.0 / sqrt((double)hd));
  const bool fused = e->mode == WSE_STEP_FUSED;
  const bool mio = merge_in_o(e);
  const bool xq = xq_on(e);

  TRY(mk.mark(-1));
  TRY(embed_token(e));
  TRY(mk.mark(WSE_STAGE_EMBED));
  for (int l = 0; l < c.n_layers; ++l) {
    const Layer &L = m.layers[(size_t)l];
    void *kc = e->kc[(size_t)l], *vc = e->vc[(size_t)l];
    if (fused) {
      TRY(wst_gemv_hier_rmsnorm(L.qkv.qw, L.qkv.si, L.qkv.sb, e->x, L.in_norm, eps, nullptr,
                                L.qkv_bias, e->qkv, H, nqkv, 0));
      TRY(mk.mark(WSE_STAGE_QKV));
      if (mio) {
        TRY(wst_attn_decode_slices(e->qkv, kc, vc, e->cos_tab, e->sin_tab, e->partials, nq, nkv,
                                   hd, e->pos_dev, e->max_seq, scale, L.q_norm, L.k_norm, eps));
        TRY(mk.mark(WSE_STAGE_ATTN));
        TRY(wst_gemv_hier_attn(L.o.qw, L.o.si, L.o.sb, e->partials, e->x, nq, hd, e->pos_dev,
                               e->max_seq, H, 1));
      } else if (xq_o_on(e)) {
        TRY(wst_attn_decode_fused_xq(e->qkv, kc, vc, e->cos_tab, e->sin_tab, e->partials,
                                     e->attn, e->xq, nq, nkv, hd, e->pos_dev, e->max_seq, scale,
                                     L.q_norm, L.k_norm, eps));
        TRY(mk.mark(WSE_STAGE_ATTN));
        TRY(wst_gemv_hier_xq(L.o.qw, L.o.si, L.o.sb, e->xq, nullptr, e->x, nq * hd, H, 1));
      } else {
        TRY(wst_attn_decode_fused(e->qkv, kc, vc, e->cos_tab, e->sin_tab, e->partials, e->attn,
                                  nq, nkv, hd, e->pos_dev, e->max_seq, scale, L.q_norm, L.k_norm,
                                  eps));
        TRY(mk.mark(WSE_STAGE_ATTN));
        TRY(wst_gemv_int4_hier_ex(L.o.qw, L.o.si, L.o.sb, e->attn, nullptr, e->x, nq * hd, H, 1));
      }
      TRY(mk.mark(WSE_STAGE_O));
      if (xq)
        TRY(wst_gemv_hier_swiglu_xq(L.gate_up.qw, L.gate_up.si, L.gate_up.sb, e->x, L.post_norm,
                                    eps, e->act, e->xq, H, I));
      else
        TRY(wst_gemv_hier_swiglu(L.gate_up.qw, L.gate_up.si, L.gate_up.sb, e->x, L.post_norm,
                                 eps, e->act, H, I));
      TRY(mk.mark(WSE_STAGE_GATE_UP));
    } else {
      TRY(wst_rmsnorm(e->x, L.in_norm, e->h, H, eps));
      TRY(wst_gemv_int4_hier_ex(L.qkv.qw, L.qkv.si, L.qkv.sb, e->h, L.qkv_bias, e->qkv, H, nqkv, 0));
      TRY(mk.mark(WSE_STAGE_QKV));
      TRY(wst_rope_cache(e->qkv, kc, vc, e->cos_tab, e->sin_tab, nq, nkv, hd, e->pos_dev,
                         e->max_seq, L.q_norm, L.k_norm, eps));
      TRY(wst_attn_decode(e->qkv, kc, vc, e->partials, e->attn, nq, nkv, hd, e->pos_dev,
                          e->max_seq, scale));
      TRY(mk.mark(WSE_STAGE_ATTN));
      TRY(wst_gemv_int4_hier_ex(L.o.qw, L.o.si, L.o.sb, e->attn, nullptr, e->x, nq * hd, H, 1));
      TRY(mk.mark(WSE_STAGE_O));
      TRY(wst_rmsnorm(e->x, L.post_norm, e->h, H, eps));
      TRY(wst_gemv_int4_hier_ex(L.gate_up.qw, L.gate_up.si, L.gate_up.sb, e->h, nullptr, e->gu, H,
                                2 * I, 0));
      TRY(wst_swiglu(e->gu, e->act, I));
      TRY(mk.mark(WSE_STAGE_GATE_UP));
    }
    if (fused && xq)
      TRY(wst_gemv_hier_xq(L.down.qw, L.down.si, L.down.sb, e->xq, nullptr, e->x, I, H, 1));
    else
      TRY(wst_gemv_int4_hier_ex(L.down.qw, L.down.si, L.down.sb, e->act, nullptr, e->x, I, H, 1));
    TRY(mk.mark(WSE_STAGE_DOWN));
  }
  // The argmax rides on the head GEMV when nothing runs between the logits and
  // the pick (no rescore) and the head is int4.
  const bool head_ax = fused && e->rs_k == 0 && !m.head().dense() && head_argmax_on();
  if (head_ax) {
    const Mat &hm = m.head();
    TRY(wst_gemv_hier_rmsnorm_argmax(hm.qw, hm.si, hm.sb, e->x, m.final_norm, eps, e->h,
                                     e->logits, H, V, e->token, e->pos_dev, e->max_seq));
  } else {
    TRY(head_logits(e, e->x, fused));
  }
  TRY(mk.mark(WSE_STAGE_HEAD));
  if (e->rs_k > 0) {
    if (fused) {
      TRY(wst_head_rescore_fused(m.rescore, e->h, e->logits, V, H, e->rs_k, e->rs_cap,
                                 e->rs_scratch, e->rs_nblocks));
    } else {
      TRY(wst_head_threshold(e->logits, V, e->rs_k, e->rs_cap, e->rs_scratch, e->rs_nblocks,
                             e->rs_thresh, e->rs_count));
      TRY(wst_head_compact(e->logits, V, e->rs_thresh, e->rs_count, e->rs_idx, e->rs_cap));
      TRY(wst_head_rescore(m.rescore, e->h, e->rs_idx, e->rs_count, e->logits, H, e->rs_cap,
                           e->rs_grid));
    }
    TRY(mk.mark(WSE_STAGE_RESCORE));
  }
  if (head_ax) {
    // done by the head's last block
  } else if (fused) {
    TRY(wst_argmax_advance(e->logits, e->token, V, e->pos_dev, e->max_seq));
  } else {
    TRY(wst_argmax(e->logits, e->token, V));
    TRY(wst_advance_pos(e->pos_dev, e->max_seq));
  }
  TRY(mk.mark(WSE_STAGE_SAMPLE));
  return WST_OK;
}

static wst_status_t check_room(wse_engine *e) {
  if (e->pos >= e->max_seq) {
    snprintf(g_msg, sizeof(g_msg), "context is full at %d tokens", e->max_seq);
    return WST_ERR_SHAPE;
  }
  return WST_OK;
}

wst_status_t wse_engine_step(wse_engine_t *e) {
  if (!e) return WST_ERR_INVALID_ARG;
  TRY(check_room(e));
  if (e->graph) {
    TRY(wst_graph_launch(e->graph));
  } else {
    Marks mk{e, false};
    TRY(step_eager(e, mk));
  }
  e->pos += 1;
  return WST_OK;
}

wst_status_t wse_engine_forward(wse_engine_t *e, int32_t token) {
  if (!e) return WST_ERR_INVALID_ARG;
  TRY(check_room(e));
  TRY(wst_memcpy_h2d(e->token, &token, 4));
  note(e, token);
  return wse_engine_step(e);
}

wst_status_t wse_engine_capture_graph(wse_engine_t *e) {
  if (!e) return WST_ERR_INVALID_ARG;
  if (e->graph) return WST_OK;
  // The warm-up step writes the KV slot at the current position: with a full
  // context that slot holds a cached token and must not be overwritten.
  TRY(check_room(e));
  // Warm every lazily initialised path (static scratch, cached device facts)
  // outside the capture, then rewind (engine.rs:357-393).
  const int saved = e->pos;
  int32_t tok = 0;
  TRY(wst_memcpy_d2h(&tok, e->token, 4));
  {
    Marks mk{e, false};
    TRY(step_eager(e, mk));
  }
  TRY(wst_device_synchronize());
  TRY(wse_engine_set_pos(e, saved));
  TRY(wst_memcpy_h2d(e->token, &tok, 4));
  TRY(wst_graph_capture_begin());
  Marks mk{e, false};
  const wst_status_t st = step_eager(e, mk);
  void *exec = nullptr;
  const wst_status_t st2 = wst_graph_capture_end(&exec);  // always end the capture
  TRY(st);
  TRY(st2);
  e->graph = exec;
  return WST_OK;
}

wst_status_t wse_engine_profile_step(wse_engine_t *e, double *stage_ms, int32_t *counts) {
  if (!e || !stage_ms) return WST_ERR_INVALID_ARG;
  TRY(check_room(e));
  Marks mk{e, true};
  TRY(step_eager(e, mk));
  e->pos += 1;
  for (int i = 1; i < mk.next; ++i) {
    float ms = 0.0f;
    TRY(wst_event_elapsed_ms(e->events[(size_t)i - 1], e->events[(size_t)i], &ms));
    const int st = mk.stage[(size_t)i];
    if (st >= 0 && st < WSE_STAGES) {
      stage_ms[st] += ms;
      if (counts) counts[st] += 1;
    }
  }
  return WST_OK;
}

// One launch of `stage`'s fused kernel for layer l (the same call step_eager
// makes), and its algorithmic bytes.
static wst_status_t stage_launch(wse_engine *e, int stage, int l, uint64_t *bytes) {
  const wse_model &m = *e->m;
  const wse_config_t &c = m.c;
  const int H = c.hidden, hd = c.head_dim, nq = c.n_q, nkv = c.n_kv, I = c.inter, V = c.vocab;
  const int nqkv = (nq + 2 * nkv) * hd;
  const float eps = c.eps;
  const Layer &L = m.layers[(size_t)l];
  const uint64_t seq = (uint64_t)(e->pos + 1 < e->max_seq ? e->pos + 1 : e->max_seq);
  switch (stage) {
    case WSE_STAGE_QKV:
      *bytes = L.qkv.bytes() + (uint64_t)H * 6 + (L.qkv_bias ? (uint64_t)nqkv * 2 : 0) +
               (uint64_t)nqkv * 4;
      return wst_gemv_hier_rmsnorm(L.qkv.qw, L.qkv.si, L.qkv.sb, e->x, L.in_norm, eps, nullptr,
                                   L.qkv_bias, e->qkv, H, nqkv, 0);
    case WSE_STAGE_ATTN:
      if (merge_in_o(e)) {  // the slices only; the partials go to the o GEMV
        *bytes = 2 * (uint64_t)nkv * seq * (uint64_t)hd * 2 + (uint64_t)nqkv * 4;
        return wst_attn_decode_slices(e->qkv, e->kc[(size_t)l], e->vc[(size_t)l], e->cos_tab,
                                      e->sin_tab, e->partials, nq, nkv, hd, e->pos_dev,
                                      e->max_seq, (float)(1.0 / sqrt((double)hd)), L.q_norm,
                                      L.k_norm, eps);
      }
      *bytes = 2 * (uint64_t)nkv * seq * (uint64_t)hd * 2 + (uint64_t)nqkv * 4 + (uint64_t)nq * hd * 2;
      if (xq_o_on(e))
        return wst_attn_decode_fused_xq(e->qkv, e->kc[(size_t)l], e->vc[(size_t)l], e->cos_tab,
                                        e->sin_tab, e->partials, e->attn, e->xq, nq, nkv, hd,
                                        e->pos_dev, e->max_seq, (float)(1.0 / sqrt((double)hd)),
                                        L.q_norm, L.k_norm, eps);
      return wst_attn_decode_fused(e->qkv, e->kc[(size_t)l], e->vc[(size_t)l], e->cos_tab,
                                   e->sin_tab, e->partials, e->attn, nq, nkv, hd, e->pos_dev,
                                   e->max_seq, (float)(1.0 / sqrt((double)hd)), L.q_norm,
                                   L.k_norm, eps);
    case WSE_STAGE_O:
      if (merge_in_o(e)) {  // reads the live slices' partials instead of the f16 vector
        const uint64_t P = (uint64_t)wst_attn_slice_positions(hd, e->max_seq);
        const uint64_t live = (seq + P - 1) / P;
        *bytes = L.o.bytes() + (uint64_t)nq * live * (uint64_t)(hd + 2) * 4 + (uint64_t)H * 8;
        return wst_gemv_hier_attn(L.o.qw, L.o.si, L.o.sb, e->partials, e->x, nq, hd, e->pos_dev,
                                  e->max_seq, H, 1);
      }
      *bytes = L.o.bytes() + (uint64_t)nq * hd * 2 + (uint64_t)H * 8;
      if (xq_o_on(e))
        return wst_gemv_hier_xq(L.o.qw, L.o.si, L.o.sb, e->xq, nullptr, e->x, nq * hd, H, 1);
      return wst_gemv_int4_hier_ex(L.o.qw, L.o.si, L.o.sb, e->attn, nullptr, e->x, nq * hd, H, 1);
    case WSE_STAGE_GATE_UP:
      *bytes = L.gate_up.bytes() + (uint64_t)H * 6 + (uint64_t)I * 2;
      if (xq_on(e))
        return wst_gemv_hier_swiglu_xq(L.gate_up.qw, L.gate_up.si, L.gate_up.sb, e->x,
                                       L.post_norm, eps, e->act, e->xq, H, I);
      return wst_gemv_hier_swiglu(L.gate_up.qw, L.gate_up.si, L.gate_up.sb, e->x, L.post_norm,
                                  eps, e->act, H, I);
    case WSE_STAGE_DOWN:
      *bytes = L.down.bytes() + (uint64_t)I * 2 + (uint64_t)H * 8;
      if (xq_on(e))
        return wst_gemv_hier_xq(L.down.qw, L.down.si, L.down.sb, e->xq, nullptr, e->x, I, H, 1);
      return wst_gemv_int4_hier_ex(L.down.qw, L.down.si, L.down.sb, e->act, nullptr, e->x, I, H,
                                   1);
    case WSE_STAGE_HEAD: {
      *bytes = m.head().bytes() + (uint64_t)H * 8 + (uint64_t)V * 4;
      if (e->rs_k == 0 && !m.head().dense()) {  // the step's form, without the advance
        const Mat &hm = m.head();
        return wst_gemv_hier_rmsnorm_argmax(hm.qw, hm.si, hm.sb, e->x, m.final_norm, eps, e->h,
                                            e->logits, H, V, e->token, nullptr, e->max_seq);
      }
      return head_logits(e, e->x, true);
    }
    default:
      snprintf(g_msg, sizeof(g_msg), "stage %d cannot be timed on its own", stage);
      return WST_ERR_INVALID_ARG;
  }
}

wst_status_t wse_engine_time_stage(wse_engine_t *e, int32_t stage, int32_t reps,
                                   double *us_per_launch, uint64_t *bytes_per_launch) {
  if (!e || !us_per_launch || reps <= 0) return WST_ERR_INVALID_ARG;
  if (e->mode != WSE_STEP_FUSED) {
    snprintf(g_msg, sizeof(g_msg), "stage timing needs a WSE_STEP_FUSED engine");
    return WST_ERR_INVALID_ARG;
  }
  const int per = stage == WSE_STAGE_HEAD ? 1 : e->m->c.n_layers;
  uint64_t bytes = 0, total = 0;
  for (int l = 0; l < per; ++l) {  // warm-up sweep
    TRY(stage_launch(e, stage, l, &bytes));
    total += bytes;
  }
  while (e->events.size() < 2) {
    void *ev = nullptr;
    TRY(wst_event_create(&ev));
    e->events.push_back(ev);
  }
  TRY(wst_event_record(e->events[0]));
  for (int r = 0; r < reps; ++r)
    for (int l = 0; l < per; ++l) TRY(stage_launch(e, stage, l, &bytes));
  TRY(wst_event_record(e->events[1]));
  float ms = 0.0f;
  TRY(wst_event_elapsed_ms(e->events[0], e->events[1], &ms));
  *us_per_launch = (double)ms * 1e3 / ((double)reps * per);
  if (bytes_per_launch) *bytes_per_launch = total / (uint64_t)per;
  return WST_OK;
}

wst_status_t wse_engine_token(wse_engine_t *e, int32_t *out) {
  if (!e || !out) return WST_ERR_INVALID_ARG;
  return wst_memcpy_d2h(out, e->token, 4);
}

wst_status_t wse_engine_set_token(wse_engine_t *e, int32_t token) {
  if (!e) return WST_ERR_INVALID_ARG;
  return wst_memcpy_h2d(e->token, &token, 4);
}

wst_status_t wse_engine_logits(wse_engine_t *e, float *out) {
  if (!e || !out) return WST_ERR_INVALID_ARG;
  return wst_memcpy_d2h(out, e->logits, (size_t)e->m->c.vocab * 4);
}

// Engine::cross_entropy (engine.rs:585-618): windows of `window` tokens, each
// from an empty cache; position i predicts token i+1 (i < window-1), its
// -log softmax accumulated on the device by wst_nll. Only the two floats come
// back, once per window.
wst_status_t wse_engine_cross_entropy(wse_engine_t *e, const int32_t *tokens, int64_t n_tokens,
                                      int32_t window, int32_t max_windows, double *nll_sum,
                                      int64_t *positions) {
  if (!e || !nll_sum || !positions || n_tokens < 0 || max_windows < 0 ||
      (n_tokens > 0 && !tokens))
    return WST_ERR_INVALID_ARG;
  if (window < 2) {
    snprintf(g_msg, sizeof(g_msg), "window must be at least 2 tokens");
    return WST_ERR_SHAPE;
  }
  if (window > e->max_seq) {
    snprintf(g_msg, sizeof(g_msg), "window %d exceeds the %d token cache; raise --ctx", window,
             e->max_seq);
    return WST_ERR_SHAPE;
  }
  const int32_t vocab = e->m->c.vocab;
  for (int64_t i = 0; i < n_tokens; ++i)
    if (tokens[i] < 0 || tokens[i] >= vocab) {
      snprintf(g_msg, sizeof(g_msg), "token %d at %lld is outside the vocabulary", tokens[i],
               (long long)i);
      return WST_ERR_INVALID_ARG;
    }
  if (!e->nll_acc) TRY(e->arena.alloc(&e->nll_acc, 8, true));
  TRY(wst_memset(e->nll_acc, 0, 8));
  int64_t n = n_tokens / window;
  if (n > max_windows) n = max_windows;
  for (int64_t w = 0; w < n; ++w) {
    TRY(wse_engine_reset(e));
    const int32_t *chunk = tokens + w * window;
    for (int i = 0; i < window - 1; ++i) {
      TRY(wse_engine_forward(e, chunk[i]));
      TRY(wst_nll(e->logits, chunk[i + 1], e->nll_acc, vocab));
    }
  }
  float got[2];
  TRY(wst_memcpy_d2h(got, e->nll_acc, 8));
  *nll_sum = (double)got[0];
  *positions = (int64_t)got[1];
  return WST_OK;
}

uint64_t wse_engine_step_bytes(const wse_engine_t *e) {
  if (!e) return 0;
  const wse_config_t &c = e->m->c;
  const uint64_t seq = (uint64_t)(e->pos + 1 < e->max_seq ? e->pos + 1 : e->max_seq);
  const uint64_t kv = (uint64_t)c.n_layers * 2 * (uint64_t)c.n_kv * (uint64_t)c.head_dim * 2 * seq;
  return wse_model_weight_bytes(e->m) + kv;
}

// ---------------------------------------------------------------- prefill

// Engine::chunk_width (engine.rs:682-698): the chunk kernels' width, or
// WHETSTONE_CHUNK_WIDTH=k (an integer >= 1) clamped to it.
static int configured_chunk_width() {
  static int w = 0;
  if (w == 0) {
    const int mx = wst_chunk_max_tokens();
    w = mx;
    if (const char *s = getenv("WHETSTONE_CHUNK_WIDTH")) {
      char *end = nullptr;
      errno = 0;
      const unsigned long long k = strtoull(s, &end, 10);
      if (*s >= '0' && *s <= '9' && end && *end == '\0' && errno == 0 && k >= 1)
        w = k < (unsigned long long)mx ? (int)k : mx;
    }
  }
  return w;
}

static wst_status_t ensure_chunk(wse_engine *e) {
  if (e->chunk_width) return WST_OK;
  const wse_config_t &c = e->m->c;
  const size_t w = (size_t)configured_chunk_width();
  const size_t H = (size_t)c.hidden, hd = (size_t)c.head_dim, I = (size_t)c.inter;
  const size_t nqkv = (size_t)(c.n_q + 2 * c.n_kv) * hd;
  Arena &a = e->arena;
  TRY(a.alloc(&e->c_tokens, w * 4, true));
  TRY(a.alloc(&e->c_x, w * H * 4, true));
  TRY(a.alloc(&e->c_h, w * H * 2, true));
  TRY(a.alloc(&e->c_qkv, w * nqkv * 4, true));
  TRY(a.alloc(&e->c_attn, w * (size_t)c.n_q * hd * 2, true));
  TRY(a.alloc(&e->c_act, w * I * 2, true));
  e->chunk_width = (int)w;
  return WST_OK;
}

// The chunk head's outputs: n x vocab f32 logits and n picks.
static wst_status_t ensure_chunk_head(wse_engine *e) {
  if (e->c_logits) return WST_OK;
  const size_t w = (size_t)e->chunk_width, V = (size_t)e->m->c.vocab;
  TRY(e->arena.alloc(&e->c_logits, w * V * 4, false));
  TRY(e->arena.alloc(&e->c_picks, w * 4, true));
  return WST_OK;
}

struct ChunkBufs {
  void *tokens, *x, *h, *qkv, *attn, *act;
};

// Engine::forward_chunk_ex (engine.rs:748-844). With want_logits the final
// norm and the head (a plain chunk GEMM: no rescore) run for every row of the
// last chunk, the chunk argmax leaves each of those rows' greedy pick, and the
// last row's logits and pick are copied to the single-token buffers (logits,
// token cursor).
//
// n tokens in chunks of `width`: with n > width the chunks go through each
// layer together, one launch per op for all of them (the batched prefill).
// plan_n is the token count the GEMMs' tiling and split-K plan is made for:
// n (plan_n = 0) lets a launch over many chunks drop the split-K that one
// chunk's few tiles need; plan_n = width keeps one chunk's plan, so that every
// token gets the bits the chunk-by-chunk pass gives it. A chunk's attention
// reads the cache only up to its own last position, so the later chunks' K/V
// rows already in the cache are never read.
static wst_status_t chunk_pass(wse_engine *e, const int32_t *ids, int n, bool want_logits,
                               int width, int plan_n, const ChunkBufs &b) {
  const wse_model &m = *e->m;
  const wse_config_t &c = m.c;
  const int H = c.hidden, hd = c.head_dim, nq = c.n_q, nkv = c.n_kv, I = c.inter, V = c.vocab;
  const int nqkv = (nq + 2 * nkv) * hd;
  const float eps = c.eps, scale = (float)(1.0 / sqrt((double)hd));
  if (e->pos + n > e->max_seq) {
    snprintf(g_msg, sizeof(g_msg), "forward_chunk: %d tokens at position %d exceeds the %d token cache",
             n, e->pos, e->max_seq);
    return WST_ERR_SHAPE;
  }
  const int pos0 = e->pos;
  const int pn = plan_n > 0 && plan_n < n ? plan_n : n;  // the plan's token count
  TRY(wst_memcpy_h2d(b.tokens, ids, (size_t)n * 4));
  if (m.embed.dense())
    TRY(wst_embed_fp16_chunk(m.embed.w16, b.tokens, b.x, H, V, n));
  else
    TRY(wst_embed_int4_hier_chunk(m.embed.qw, m.embed.si, m.embed.sb, b.tokens, b.x, H, V, n));
  // Fused chunk forms (whetstone_ext.h; bit-identical to the reference's op
  // sequence): qkv GEMM + RoPE/KV append, o GEMM + post-attention norm, gate|up
  // GEMM + SwiGLU, down GEMM + the next norm (the next layer's input norm, or
  // the final norm before the head). Unfused where a fused form does not
  // apply (f16 head path aside, head_dim above 128).
  const bool rope_fused = hd <= 128;
  TRY(wst_rmsnorm_chunk(b.x, m.layers[0].in_norm, b.h, H, n, eps));
  for (int l = 0; l < c.n_layers; ++l) {
    const Layer &L = m.layers[(size_t)l];
    if (rope_fused) {
      TRY(wst_gemm_hier_rope_chunks(L.qkv.qw, L.qkv.si, L.qkv.sb, b.h, L.qkv_bias, b.qkv, H,
                                    e->kc[(size_t)l], e->vc[(size_t)l], e->cos_tab, e->sin_tab,
                                    nq, nkv, hd, pos0, n, e->max_seq, L.q_norm, L.k_norm, eps,
                                    pn));
    } else {
      TRY(wst_gemm_int4_hier_chunks(L.qkv.qw, L.qkv.si, L.qkv.sb, b.h, L.qkv_bias, b.qkv, H, nqkv,
                                    n, 0, pn));
      TRY(wst_rope_cache_chunk(b.qkv, e->kc[(size_t)l], e->vc[(size_t)l], e->cos_tab,
                               e->sin_tab, nq, nkv, hd, pos0, n, e->max_seq, L.q_norm, L.k_norm,
                               eps));
    }
    TRY(wst_attn_chunk(b.qkv, e->kc[(size_t)l], e->vc[(size_t)l], b.attn, nq, nkv, hd, pos0, n,
                       e->max_seq, scale));
    TRY(wst_gemm_hier_norm_chunks(L.o.qw, L.o.si, L.o.sb, b.attn, nullptr, b.x, nq * hd, H, n, 1,
                                  L.post_norm, eps, b.h, pn));
    TRY(wst_gemm_hier_swiglu_chunks(L.gate_up.qw, L.gate_up.si, L.gate_up.sb, b.h, b.act, H, I,
                                    n, pn));
    const bool last = l + 1 == c.n_layers;
    if (!last || want_logits)
      TRY(wst_gemm_hier_norm_chunks(L.down.qw, L.down.si, L.down.sb, b.act, nullptr, b.x, I, H, n,
                                    1, last ? m.final_norm : m.layers[(size_t)l + 1].in_norm, eps,
                                    b.h, pn));
    else
      TRY(wst_gemm_int4_hier_chunks(L.down.qw, L.down.si, L.down.sb, b.act, nullptr, b.x, I, H, n,
                                    1, pn));
  }
  if (want_logits) {
    // the last chunk's rows
    const int r0 = (n - 1) / width * width, nr = n - r0;
    const void *hl = (const char *)b.h + (size_t)r0 * H * 2;
    const Mat &head = m.head();
    TRY(ensure_chunk_head(e));
    if (head.dense())
      TRY(wst_gemm_fp16(head.w16, hl, nullptr, e->c_logits, H, V, nr, 0));
    else
      TRY(wst_gemm_int4_hier(head.qw, head.si, head.sb, hl, nullptr, e->c_logits, H, V, nr, 0));
    TRY(wst_argmax_chunk(e->c_logits, e->c_picks, V, nr));
    TRY(wst_memcpy_d2d(e->logits, (const char *)e->c_logits + (size_t)(nr - 1) * V * 4,
                       (size_t)V * 4));
    TRY(wst_memcpy_d2d(e->token, (const char *)e->c_picks + (size_t)(nr - 1) * 4, 4));
    e->c_ran = true;
  }
  for (int i = 0; i < n; ++i) note(e, ids[i]);
  return wse_engine_set_pos(e, pos0 + n);
}

static wst_status_t forward_chunk(wse_engine *e, const int32_t *ids, int n, bool want_logits) {
  const ChunkBufs b{e->c_tokens, e->c_x, e->c_h, e->c_qkv, e->c_attn, e->c_act};
  return chunk_pass(e, ids, n, want_logits, e->chunk_width, 0, b);
}

// The batched prefill's buffers, grown to n tokens.
static wst_status_t ensure_batch(wse_engine *e, int n) {
  if (e->b_cap >= n) return WST_OK;
  const wse_config_t &c = e->m->c;
  const size_t w = (size_t)n;
  const size_t H = (size_t)c.hidden, hd = (size_t)c.head_dim, I = (size_t)c.inter;
  const size_t nqkv = (size_t)(c.n_q + 2 * c.n_kv) * hd;
  Arena &a = e->arena;
  TRY(a.alloc(&e->b_tokens, w * 4, true));
  TRY(a.alloc(&e->b_x, w * H * 4, true));
  TRY(a.alloc(&e->b_h, w * H * 2, true));
  TRY(a.alloc(&e->b_qkv, w * nqkv * 4, true));
  TRY(a.alloc(&e->b_attn, w * (size_t)c.n_q * hd * 2, true));
  TRY(a.alloc(&e->b_act, w * I * 2, true));
  e->b_cap = n;
  return WST_OK;
}

// The full chunks of a chunked prefill go through each layer together
// (chunk_pass with n > width), planned for the whole launch (1, the default);
// WSE_CHUNK_BATCH=chunk keeps one chunk's plan per launch (bit-identical to
// the chunk-by-chunk pass); WSE_CHUNK_BATCH=0 runs the chunks one by one.
enum BatchMode { BATCH_OFF, BATCH_WHOLE, BATCH_CHUNK_PLAN };
static BatchMode chunk_batch_mode() {
  const char *v = getenv("WSE_CHUNK_BATCH");
  if (!v || !v[0]) return BATCH_WHOLE;
  if (v[0] == '0') return BATCH_OFF;
  return strcmp(v, "chunk") == 0 ? BATCH_CHUNK_PLAN : BATCH_WHOLE;
}

wst_status_t wse_engine_max_seq(const wse_engine_t *e, int32_t *out) {
  if (!e || !out) return WST_ERR_INVALID_ARG;
  *out = e->max_seq;
  return WST_OK;
}

wst_status_t wse_engine_chunk_width(wse_engine_t *e, int32_t *out) {
  if (!e || !out) return WST_ERR_INVALID_ARG;
  *out = configured_chunk_width();
  return WST_OK;
}

wst_status_t wse_engine_forward_chunk(wse_engine_t *e, const int32_t *ids, int32_t n,
                                      int32_t want_logits) {
  if (!e || !ids) return WST_ERR_INVALID_ARG;
  if (n <= 0) {
    snprintf(g_msg, sizeof(g_msg), "forward_chunk: empty chunk");
    return WST_ERR_SHAPE;
  }
  TRY(ensure_chunk(e));
  if (n > e->chunk_width) {
    snprintf(g_msg, sizeof(g_msg), "forward_chunk: %d tokens exceeds the %d token chunk width", n,
             e->chunk_width);
    return WST_ERR_SHAPE;
  }
  return forward_chunk(e, ids, n, want_logits != 0);
}

wst_status_t wse_engine_chunk_picks(wse_engine_t *e, int32_t n, int32_t *out) {
  if (!e || !out || n < 0) return WST_ERR_INVALID_ARG;
  if (!e->c_ran) {
    snprintf(g_msg, sizeof(g_msg), "no chunk pass has run");
    return WST_ERR_SHAPE;
  }
  if (n > e->chunk_width) {
    snprintf(g_msg, sizeof(g_msg), "chunk_picks: %d exceeds the %d token chunk width", n,
             e->chunk_width);
    return WST_ERR_SHAPE;
  }
  if (n == 0) return WST_OK;
  TRY(wst_memcpy_d2h(out, e->c_picks, (size_t)n * 4));
  for (int i = 0; i < n; ++i) out[i] = out[i] < 0 ? 0 : out[i];  // v.max(0)
  return WST_OK;
}

wst_status_t wse_engine_rewind(wse_engine_t *e, int32_t pos) {
  if (!e || pos < 0) return WST_ERR_INVALID_ARG;
  if (pos > e->pos) {
    snprintf(g_msg, sizeof(g_msg), "rewind: %d is ahead of the current position %d", pos, e->pos);
    return WST_ERR_SHAPE;
  }
  return wse_engine_set_pos(e, pos);
}

wst_status_t wse_engine_prefill(wse_engine_t *e, const int32_t *ids, int32_t n, int32_t chunked) {
  if (!e || !ids || n <= 0) return WST_ERR_INVALID_ARG;
  if (chunked && n > 1) {
    TRY(ensure_chunk(e));
    const int w = e->chunk_width;
    int s = 0;
    const int full = n / w * w;  // the full chunks (a shorter last chunk keeps its own plan)
    const BatchMode mode = chunk_batch_mode();
    if (mode != BATCH_OFF && full >= 2 * w) {
      TRY(ensure_batch(e, full));
      const ChunkBufs b{e->b_tokens, e->b_x, e->b_h, e->b_qkv, e->b_attn, e->b_act};
      TRY(chunk_pass(e, ids, full, full == n, w, mode == BATCH_CHUNK_PLAN ? w : 0, b));
      s = full;
    }
    for (; s < n; s += w) {
      const int k = n - s < w ? n - s : w;
      TRY(forward_chunk(e, ids + s, k, s + k == n));
    }
    return WST_OK;
  }
  for (int i = 0; i < n; ++i) TRY(wse_engine_forward(e, ids[i]));
  return WST_OK;
}

wst_status_t wse_engine_generate(wse_engine_t *e, const int32_t *prompt, int32_t n_prompt,
                                 int32_t n_new, int32_t chunked, int32_t *out, int32_t *n_out) {
  if (!e || !prompt || n_prompt <= 0 || n_new < 0 || (n_new && !out) || !n_out)
    return WST_ERR_INVALID_ARG;
  *n_out = 0;
  TRY(wse_engine_prefill(e, prompt, n_prompt, chunked));
  int32_t next = 0;
  TRY(wse_engine_token(e, &next));
  note(e, next);  // Sampler::Greedy notes its pick (engine.rs:650-656)
  for (int i = 0; i < n_new; ++i) {
    out[i] = next;
    *n_out = i + 1;
    if (i + 1 == n_new || e->pos >= e->max_seq) break;
    TRY(wse_engine_step(e));
    TRY(wse_engine_token(e, &next));
    note(e, next);
  }
  return WST_OK;
}

wst_status_t wse_engine_sample(wse_engine_t *e, const wse_sampling_config_t *cfg, uint64_t step,
                               int32_t *out) {
  if (!e || !out) return WST_ERR_INVALID_ARG;
  int32_t t = 0;
  if (!cfg) {
    TRY(wse_engine_token(e, &t));
  } else {
    std::vector<float> lg((size_t)e->m->c.vocab);
    TRY(wse_engine_logits(e, lg.data()));
    std::vector<int32_t> rc(e->recent.begin(), e->recent.end());
    t = wse_sample_with(lg.data(), e->m->c.vocab, cfg, step, rc.data(), (int32_t)rc.size());
    TRY(wse_engine_set_token(e, t));
  }
  note(e, t);
  *out = t;
  return WST_OK;
}

wst_status_t wse_engine_generate_sampled(wse_engine_t *e, const int32_t *prompt, int32_t n_prompt,
                                         int32_t n_new, int32_t chunked,
                                         const wse_sampling_config_t *cfg, int32_t *out,
                                         int32_t *n_out) {
  if (!e || !prompt || n_new < 0 || (n_new && !out) || !n_out) return WST_ERR_INVALID_ARG;
  *n_out = 0;
  if (n_prompt <= 0) {
    snprintf(g_msg, sizeof(g_msg), "cannot generate from an empty prompt");
    return WST_ERR_SHAPE;
  }
  TRY(wse_engine_prefill(e, prompt, n_prompt, chunked));
  int32_t next = 0;
  TRY(wse_engine_sample(e, cfg, 0, &next));
  for (int32_t st = 0; st < n_new; ++st) {
    out[st] = next;
    *n_out = st + 1;
    if (e->pos >= e->max_seq) break;
    TRY(wse_engine_step(e));
    TRY(wse_engine_sample(e, cfg, (uint64_t)st + 1, &next));
  }
  return WST_OK;
}

}  // extern "C"
