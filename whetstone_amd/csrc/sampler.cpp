// Host-side stochastic sampling (crates/whetstone-core/src/engine.rs:969-1114,
// `sample_with`): repetition penalty over the recent window, then greedy when
// the temperature is <= 0, else a pool of the top-k (at most 512) logits,
// temperature, min-p, top-p, and one SplitMix64 draw. Host C++: the reference
// samples on the host too, after a device-to-host copy of the logits.
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <vector>

#include "whetstone_engine.h"

namespace {

constexpr int kNucleusPool = 512;  // NUCLEUS_POOL (engine.rs:969)

// SplitMix64 (engine.rs:1107-1114): the published constants.
uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  uint64_t r = z;
  r = (r ^ (r >> 30)) * 0xBF58476D1CE4E5B9ull;
  r = (r ^ (r >> 27)) * 0x94D049BB133111EBull;
  return r ^ (r >> 31);
}

// Index of the largest logit, NaN-tolerant (engine.rs:1098-1105): Rust's
// `max_by` with partial_cmp and Equal for NaN keeps the later element unless
// the earlier one compares strictly greater, so ties go to the LAST maximum.
int32_t host_argmax(const float *l, int n) {
  int32_t best = 0;
  float bv = l[0];
  for (int i = 1; i < n; ++i)
    if (!(bv > l[i])) {
      best = i;
      bv = l[i];
    }
  return best;
}

}  // namespace

extern "C" uint64_t wse_splitmix64(uint64_t z) { return splitmix64(z); }

extern "C" int32_t wse_sample_with(float *logits, int32_t n, const wse_sampling_config_t *cfg,
                                   uint64_t step, const int32_t *recent, int32_t n_recent) {
  if (!logits || n <= 0 || !cfg) return 0;
  // 1. repetition penalty (CTRL form: divide a positive logit, multiply a
  // negative one), once per occurrence in the last repeat_last_n tokens.
  if (cfg->repeat_penalty != 1.0f && cfg->repeat_last_n > 0 && recent && n_recent > 0) {
    const int w = cfg->repeat_last_n < n_recent ? cfg->repeat_last_n : n_recent;
    for (int j = n_recent - w; j < n_recent; ++j) {
      const int32_t t = recent[j];
      if (t >= 0 && t < n)
        logits[t] = logits[t] > 0.0f ? logits[t] / cfg->repeat_penalty
                                     : logits[t] * cfg->repeat_penalty;
    }
  }
  if (cfg->temperature <= 0.0f) return host_argmax(logits, n);

  // 2. the pool: the k highest logits, sorted descending. Rust's unstable
  // select/sort leaves the order of equal logits unspecified; here it is
  // fixed (lower index first) and a NaN sorts below every number.
  auto key_gt = [&](int32_t a, int32_t b) {
    const float x = logits[a], y = logits[b];
    const bool xn = x != x, yn = y != y;
    if (xn != yn) return yn;  // a number beats NaN
    if (!xn && x != y) return x > y;
    return a < b;
  };
  const int pool = cfg->top_k > 0 ? std::min(cfg->top_k, kNucleusPool) : kNucleusPool;
  const int k = std::min(pool, (int)n);
  std::vector<int32_t> order((size_t)n);
  for (int i = 0; i < n; ++i) order[(size_t)i] = i;
  std::partial_sort(order.begin(), order.begin() + k, order.end(), key_gt);
  order.resize((size_t)k);

  // 3. temperature, in f64 relative to the top candidate
  const double mx = (double)logits[order[0]];
  std::vector<double> probs((size_t)k);
  double total = 0.0;
  for (int i = 0; i < k; ++i) {
    const double p = exp(((double)logits[order[(size_t)i]] - mx) / (double)cfg->temperature);
    total += p;
    probs[(size_t)i] = p;
  }
  // 4. min-p, relative to the leader
  int cut = k;
  if (cfg->min_p > 0.0f) {
    const double floor_ = probs[0] * (double)cfg->min_p;
    cut = k;
    for (int i = 0; i < k; ++i)
      if (probs[(size_t)i] < floor_) {
        cut = i;
        break;
      }
    if (cut < 1) cut = 1;
  }
  // 5. top-p over the normalised pool
  if (cfg->top_p < 1.0f) {
    double acc = 0.0;
    for (int i = 0; i < cut; ++i) {
      acc += probs[(size_t)i] / total;
      if (acc >= (double)cfg->top_p) {
        cut = i + 1;
        break;
      }
    }
  }
  // 6. the draw
  double mass = 0.0;
  for (int i = 0; i < cut; ++i) mass += probs[(size_t)i];
  const double u = (double)splitmix64(cfg->seed ^ (step * 0x9E3779B97F4A7C15ull)) /
                   (double)UINT64_MAX * mass;
  double acc = 0.0;
  for (int i = 0; i < cut; ++i) {
    acc += probs[(size_t)i];
    if (acc >= u) return order[(size_t)i];
  }
  return order[(size_t)(cut > 0 ? cut - 1 : 0)];
}
