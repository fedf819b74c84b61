// Greedy generation with an n-gram draft, verified by one chunk pass per round
// (crates/whetstone-core/src/speculate.rs). Host C++ over the engine's public
// C ABI only, as the reference's module uses only Engine's public methods.
//
// A round: the token `next` is confirmed (it is the target's own argmax). The
// draft proposes up to width-1 tokens that followed the most recent earlier
// occurrence of the history's tail; [next, drafts...] run through one chunk
// pass, whose per-row greedy picks say how many drafts the target agrees
// with. The cache is rewound to just after the last agreed token, and the pick
// at that row is the next confirmed token. A round with no proposal is one
// ordinary decode step. The emitted stream is the greedy stream whenever the
// chunk pass's picks equal the decode step's argmax at the same positions.
#include <stdio.h>

#include <vector>

#include "engine_internal.hpp"
#include "whetstone_engine.h"

using wse::g_msg;

// propose (speculate.rs:122-150): longest n-gram first, most recent match
// first, at most `want` tokens and never past the end of the history.
static int propose(const int32_t *hist, int len, int ngram_max, int ngram_min, int want,
                   int32_t *out) {
  if (want <= 0) return 0;
  const int n_max = ngram_max < len - 1 ? ngram_max : (len - 1 > 0 ? len - 1 : 0);
  for (int n = n_max; n >= ngram_min && n >= 0; --n) {
    if (len <= n) continue;
    const int32_t *tail = hist + (len - n);
    for (int start = len - n - 1; start >= 0; --start) {
      bool eq = true;
      for (int i = 0; i < n && eq; ++i) eq = hist[start + i] == tail[i];
      if (!eq) continue;
      const int from = start + n;
      const int take = want < len - from ? want : len - from;
      if (take > 0) {
        for (int i = 0; i < take; ++i) out[i] = hist[from + i];
        return take;
      }
    }
  }
  return 0;
}

extern "C" {

int32_t wse_spec_propose(const int32_t *history, int32_t n, int32_t ngram_max, int32_t ngram_min,
                         int32_t want, int32_t *out) {
  if (!history || !out || n < 0 || ngram_max < 0 || ngram_min < 0) return 0;
  return propose(history, n, ngram_max, ngram_min, want, out);
}

wst_status_t wse_speculate_generate(wse_engine_t *e, const int32_t *prompt, int32_t n_prompt,
                                    int32_t max_new, const wse_spec_config_t *cfg,
                                    int32_t *out_tokens, int32_t *n_out, wse_spec_stats_t *stats) {
  if (!e || !prompt || !cfg || !n_out || max_new < 0 || (max_new > 0 && !out_tokens) ||
      cfg->draft < 0 || cfg->ngram_max < 0 || cfg->ngram_min < 0)
    return WST_ERR_INVALID_ARG;
  if (n_prompt <= 0) {
    snprintf(g_msg, sizeof(g_msg), "cannot generate from an empty prompt");
    return WST_ERR_SHAPE;
  }
  *n_out = 0;
  wse_spec_stats_t st{};
  int32_t width = 0;
  TRY(wse_engine_chunk_width(e, &width));
  if (width > (cfg->draft > 1 ? cfg->draft : 1)) width = cfg->draft > 1 ? cfg->draft : 1;
  int32_t max_seq = 0;
  TRY(wse_engine_max_seq(e, &max_seq));

  TRY(wse_engine_prefill(e, prompt, n_prompt, 1));
  std::vector<int32_t> history(prompt, prompt + n_prompt);
  int32_t next = 0;
  TRY(wse_engine_token(e, &next));  // prefill left the argmax in the cursor

  int generated = 0;
  std::vector<int32_t> drafts((size_t)width), inputs((size_t)width), picks((size_t)width);
  while (generated < max_new) {
    out_tokens[generated++] = next;  // confirmed: the target's own argmax
    history.push_back(next);
    if (generated >= max_new || wse_engine_pos(e) >= max_seq) break;

    const int room = max_seq - wse_engine_pos(e);
    const int want = width - 1 < room - 1 ? width - 1 : (room - 1 > 0 ? room - 1 : 0);
    const int nd = propose(history.data(), (int)history.size(), cfg->ngram_max, cfg->ngram_min,
                           want, drafts.data());
    if (nd == 0) {  // nothing to speculate on: one ordinary step
      ++st.rounds;
      ++st.empty_rounds;
      TRY(wse_engine_forward(e, next));
      TRY(wse_engine_token(e, &next));
      continue;
    }
    const int k = 1 + nd;
    inputs[0] = next;
    for (int i = 0; i < nd; ++i) inputs[(size_t)i + 1] = drafts[(size_t)i];
    const int pos0 = wse_engine_pos(e);
    TRY(wse_engine_forward_chunk(e, inputs.data(), k, 1));
    TRY(wse_engine_chunk_picks(e, k, picks.data()));
    ++st.rounds;
    st.proposed += nd;
    // picks[j] is the target's choice after inputs[..=j]: the first
    // disagreement with inputs[j+1] ends the accepted run.
    int m = k - 1;
    for (int j = 0; j < k - 1; ++j)
      if (picks[(size_t)j] != inputs[(size_t)j + 1]) {
        m = j;
        break;
      }
    st.accepted += m;
    // The cache keeps inputs[0..=m]; the rejected tail is overwritten later.
    TRY(wse_engine_rewind(e, pos0 + m + 1));
    wse_engine_unnote(e, k - (m + 1));  // speculate.rs:240: the rejected inputs leave the window
    bool stop = false;
    for (int j = 1; j <= m; ++j) {
      out_tokens[generated++] = inputs[(size_t)j];
      history.push_back(inputs[(size_t)j]);
      if (generated >= max_new) {
        stop = true;
        break;
      }
    }
    if (stop) break;
    next = picks[(size_t)m];
    TRY(wse_engine_set_token(e, next));  // the cursor holds the last row's pick
  }
  *n_out = generated;
  if (stats) *stats = st;
  return WST_OK;
}

}  // extern "C"
