// Types and helpers shared by the engine's translation units (engine.cpp: the
// step and the synthetic model; wstone.cpp: the .wstone reader and loader).
// Host C++ only; the GPU is reached through the C ABI.
#pragma once

#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "whetstone.h"
#include "whetstone_engine.h"
#include "whetstone_ext.h"

#define TRY(expr)                                  \
  do {                                             \
    const wst_status_t _s = (expr);                \
    if (_s != WST_OK) return _s;                   \
  } while (0)

namespace wse {

// Engine-level refusals carry their message here (wse_last_error); kernel
// failures keep theirs in the library's wst_last_error.
extern thread_local char g_msg[512];

wst_status_t shape_error(const char *fmt, const char *what);

// A weight matrix on the device: int4-hier-g32 (qw, si, sb) or, for the
// embedding and the output projection only, dense f16 (w16).
struct Mat {
  void *qw = nullptr, *si = nullptr, *sb = nullptr;
  void *w16 = nullptr;  // f16 [out_f][in_f] when the matrix is stored dense
  int64_t in_f = 0, out_f = 0;
  bool dense() const { return w16 != nullptr; }
  uint64_t bytes() const {
    return dense() ? (uint64_t)out_f * (uint64_t)in_f * 2
                   : (uint64_t)out_f * (uint64_t)(in_f / 2 + in_f / 32 + 4);
  }
};

struct Layer {
  Mat qkv, o, gate_up, down;
  void *qkv_bias = nullptr, *in_norm = nullptr, *post_norm = nullptr;
  void *q_norm = nullptr, *k_norm = nullptr;
};

// Device allocations owned by a model or an engine, freed together.
struct Arena {
  std::vector<void *> ptrs;
  wst_status_t alloc(void **out, size_t bytes, bool zero) {
    *out = nullptr;
    TRY(wst_malloc(out, bytes));
    ptrs.push_back(*out);
    if (zero) TRY(wst_memset(*out, 0, bytes));
    return WST_OK;
  }
  void free_all() {
    for (void *p : ptrs) wst_free(p);
    ptrs.clear();
  }
};

wst_status_t alloc_mat(Arena &a, Mat &m, int64_t in_f, int64_t out_f);
wst_status_t check_config(const wse_config_t *c);

}  // namespace wse

struct wse_model {
  wse_config_t c{};
  wse::Mat embed, lm_head;
  void *final_norm = nullptr;
  void *rescore = nullptr;  // f16 [vocab][hidden]
  std::vector<wse::Layer> layers;
  wse::Arena arena;
  const wse::Mat &head() const { return c.tied ? embed : lm_head; }
};
