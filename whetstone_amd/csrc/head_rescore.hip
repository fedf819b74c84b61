// Top-k head rescore: choose a threshold from a ladder of margins below the
// maximum logit, then recompute every logit above it from an f16 copy of the
// head. reference: crates/whetstone-kernels/cuda/head_rescore.cu.
//
// The ladder (head_rescore.cu:62-180): rung c admits logits with
// max - v <= 2^c/64 (12 rungs, 1/64 .. 32 nats); pick the smallest rung that
// admits >= k, then step down while it admits > cap; thresh = max - 2^pick/64.
//
// gfx950 shape: the max and the counts are grid-wide passes whose cross-block
// combine is done by the last block to finish (device-scope counter, reset by
// that block), so the threshold takes two launches instead of four and no
// memset. Counts are integer atomics: order-independent, deterministic.
#include "common.hpp"

#define RESCORE_RUNGS 12

struct RescoreScratch {
  unsigned int max_counter;
  unsigned int count_counter;
  unsigned int pad[62];
  float maxv;        // fused path: the maximum
  int32_t counts[RESCORE_RUNGS];
  float thresh;      // fused path
  int32_t enabled;   // fused path: counts[pick] <= cap
};

static RescoreScratch *rescore_scratch() {
  return (RescoreScratch *)wst_static_scratch(WST_SCRATCH_RESCORE, sizeof(RescoreScratch));
}

// Pass 1: per-block maxima into partial[]; the last block reduces them into
// *maxv and clears the rung counters.
__global__ __launch_bounds__(256) void head_max_kernel(const float *__restrict__ logits, int n,
                                                       float *__restrict__ partial,
                                                       float *__restrict__ maxv,
                                                       int32_t *__restrict__ counts,
                                                       unsigned int *__restrict__ counter) {
  __shared__ float red[16];
  float m = -INFINITY;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
    m = fmaxf(m, logits[i]);
  m = block_max(m, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
  if (!last_block_done(counter, gridDim.x)) return;
  float b = -INFINITY;
  for (int i = threadIdx.x; i < (int)gridDim.x; i += 256) b = fmaxf(b, partial[i]);
  b = block_max(b, red);
  if (threadIdx.x == 0) *maxv = b;
  if (threadIdx.x < RESCORE_RUNGS) counts[threadIdx.x] = 0;
}

// Pass 2: rung counts; the last block picks the rung and publishes the
// threshold, and resets the compaction count (head_rescore.cu:108-180).
__global__ __launch_bounds__(256) void head_counts_kernel(
    const float *__restrict__ logits, int n, const float *__restrict__ maxv,
    int32_t *__restrict__ counts, unsigned int *__restrict__ counter, int k, int cap,
    float *__restrict__ out_thresh, int32_t *__restrict__ out_count,
    int32_t *__restrict__ enabled) {
  __shared__ int local[RESCORE_RUNGS];
  if (threadIdx.x < RESCORE_RUNGS) local[threadIdx.x] = 0;
  __syncthreads();
  const float smax = *maxv;
  int mine[RESCORE_RUNGS];
#pragma unroll
  for (int c = 0; c < RESCORE_RUNGS; ++c) mine[c] = 0;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const float d = smax - logits[i];
#pragma unroll
    for (int c = 0; c < RESCORE_RUNGS; ++c) mine[c] += (d <= 0.015625f * (float)(1 << c)) ? 1 : 0;
  }
#pragma unroll
  for (int c = 0; c < RESCORE_RUNGS; ++c) {
    const int s = wave_sum_i32(mine[c]);
    if ((threadIdx.x & 63) == 0 && s) atomicAdd(&local[c], s);
  }
  __syncthreads();
  if (threadIdx.x < RESCORE_RUNGS && local[threadIdx.x] != 0)
    atomicAdd(&counts[threadIdx.x], local[threadIdx.x]);
  if (!last_block_done(counter, gridDim.x)) return;
  if (threadIdx.x == 0) {
    int cnt[RESCORE_RUNGS];
    for (int c = 0; c < RESCORE_RUNGS; ++c)
      cnt[c] = __hip_atomic_load(&counts[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int pick = RESCORE_RUNGS - 1;
    for (int c = 0; c < RESCORE_RUNGS; ++c)
      if (cnt[c] >= k) {
        pick = c;
        break;
      }
    while (pick > 0 && cnt[pick] > cap) --pick;
    *out_thresh = smax - 0.015625f * (float)(1 << pick);
    if (out_count) *out_count = 0;
    if (enabled) *enabled = cnt[pick] <= cap ? 1 : 0;
  }
}

extern "C" wst_status_t wst_head_threshold(const void *logits, int32_t n, int32_t k, int32_t cap,
                                           void *scratch, int32_t nblocks, void *out_thresh,
                                           void *out_count) {
  WST_REQUIRE(logits && scratch && out_thresh && out_count, "wst_head_threshold: null pointer");
  WST_REQUIRE(n > 0 && k > 0 && cap >= k && nblocks > 0, "wst_head_threshold: bad shape");
  WST_REQUIRE(nblocks <= 65535, "wst_head_threshold: too many blocks");
  RescoreScratch *rs = rescore_scratch();
  if (!rs) return WST_ERR_OOM;
  // Caller scratch layout (head_rescore.cu:190-193): [nblocks] partial maxima,
  // one max, 12 rung counters.
  float *partial = (float *)scratch;
  float *maxv = partial + nblocks;
  int32_t *counts = (int32_t *)(maxv + 1);
  head_max_kernel<<<nblocks, 256, 0, WST_STREAM>>>((const float *)logits, n, partial, maxv,
                                                   counts, &rs->max_counter);
  head_counts_kernel<<<nblocks, 256, 0, WST_STREAM>>>(
      (const float *)logits, n, maxv, counts, &rs->count_counter, k, cap, (float *)out_thresh,
      (int32_t *)out_count, nullptr);
  WST_TRY_KERNEL("wst_head_threshold");
  return WST_OK;
}

// Compaction (head_rescore.cu:215-224): atomic append of every i with
// logits[i] >= thresh, the first `cap` appended kept.
__global__ __launch_bounds__(256) void head_compact_kernel(const float *__restrict__ logits,
                                                           int n,
                                                           const float *__restrict__ thresh,
                                                           int32_t *__restrict__ count,
                                                           int32_t *__restrict__ out_idx,
                                                           int cap) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  if (logits[i] < *thresh) return;
  const int slot = atomicAdd(count, 1);
  if (slot < cap) out_idx[slot] = i;
}

extern "C" wst_status_t wst_head_compact(const void *logits, int32_t n, const void *thresh,
                                         void *count, void *out_idx, int32_t cap) {
  WST_REQUIRE(logits && thresh && count && out_idx, "wst_head_compact: null pointer");
  WST_REQUIRE(n > 0 && cap > 0, "wst_head_compact: n and cap must be positive");
  head_compact_kernel<<<(n + 255) / 256, 256, 0, WST_STREAM>>>(
      (const float *)logits, n, (const float *)thresh, (int32_t *)count, (int32_t *)out_idx,
      cap);
  WST_TRY_KERNEL("wst_head_compact");
  return WST_OK;
}

// f32 dot of an f16 head row with the f16 activation: one wave per row,
// 16 B per lane per load, v_dot2c_f32_f16 accumulation, DPP reduction.
__device__ __forceinline__ float head_row_dot(const uint16_t *__restrict__ head,
                                              const uint16_t *__restrict__ x, int row,
                                              int hidden, int lane) {
  const uint4 *w = (const uint4 *)(head + (size_t)row * hidden);
  const uint4 *xv = (const uint4 *)x;
  float acc = 0.0f;
  for (int v = lane; v < hidden / 8; v += 64) {
    const uint4 a = w[v], b = xv[v];
    acc = __builtin_amdgcn_fdot2(as_h2(a.x), as_h2(b.x), acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(a.y), as_h2(b.y), acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(a.z), as_h2(b.z), acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(a.w), as_h2(b.w), acc, false);
  }
  return wave_sum(acc);
}

// Rescore (head_rescore.cu:251-284): the selected rows, strided over a fixed
// grid so that every survivor up to `cap` is recomputed whatever the count.
__global__ __launch_bounds__(256) void head_rescore_kernel(
    const uint16_t *__restrict__ head, const uint16_t *__restrict__ x,
    const int32_t *__restrict__ idx, const int32_t *__restrict__ count,
    float *__restrict__ logits, int hidden, int cap) {
  const int n = min(*count, cap);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int j = blockIdx.x * 4 + wave; j < n; j += gridDim.x * 4) {
    const int row = idx[j];
    const float acc = head_row_dot(head, x, row, hidden, lane);
    if (lane == 0) logits[row] = acc;
  }
}

extern "C" wst_status_t wst_head_rescore(const void *head, const void *x, const void *idx,
                                         const void *count, void *logits, int32_t hidden,
                                         int32_t cap, int32_t grid) {
  WST_REQUIRE(head && x && idx && count && logits, "wst_head_rescore: null pointer");
  WST_REQUIRE(hidden > 0 && cap > 0 && grid > 0, "wst_head_rescore: bad shape");
  WST_REQUIRE(hidden % 8 == 0, "wst_head_rescore: hidden must be a multiple of 8");
  int blocks = (grid + 3) / 4;
  if (blocks < 1) blocks = 1;
  head_rescore_kernel<<<blocks, 256, 0, WST_STREAM>>>(
      (const uint16_t *)head, (const uint16_t *)x, (const int32_t *)idx, (const int32_t *)count,
      (float *)logits, hidden, cap);
  WST_TRY_KERNEL("wst_head_rescore");
  return WST_OK;
}

// Fused select + rescore: the block that finds a logit >= thresh recomputes
// it. Every selected row is rescored when the ladder's count fits `cap`.
__global__ __launch_bounds__(256) void head_select_rescore_kernel(
    const uint16_t *__restrict__ head, const uint16_t *__restrict__ x,
    float *__restrict__ logits, int n, int hidden, const RescoreScratch *__restrict__ rs) {
  __shared__ int list[256];
  __shared__ int nlist;
  if (!rs->enabled) return;
  const float th = rs->thresh;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int base = blockIdx.x * 256; base < n; base += gridDim.x * 256) {
    if (threadIdx.x == 0) nlist = 0;
    __syncthreads();
    const int i = base + threadIdx.x;
    if (i < n && !(logits[i] < th)) list[atomicAdd(&nlist, 1)] = i;
    __syncthreads();
    const int cnt = nlist;
    for (int j = wave; j < cnt; j += 4) {
      const int row = list[j];
      const float acc = head_row_dot(head, x, row, hidden, lane);
      if (lane == 0) logits[row] = acc;
    }
    __syncthreads();
  }
}

extern "C" wst_status_t wst_head_rescore_fused(const void *head, const void *x, void *logits,
                                               int32_t n, int32_t hidden, int32_t k, int32_t cap,
                                               void *scratch, int32_t nblocks) {
  WST_REQUIRE(head && x && logits && scratch, "wst_head_rescore_fused: null pointer");
  WST_REQUIRE(n > 0 && hidden > 0 && k > 0 && cap >= k && nblocks > 0 && nblocks <= 65535,
              "wst_head_rescore_fused: bad shape");
  WST_REQUIRE(hidden % 8 == 0, "wst_head_rescore_fused: hidden must be a multiple of 8");
  RescoreScratch *rs = rescore_scratch();
  if (!rs) return WST_ERR_OOM;
  float *partial = (float *)scratch;
  head_max_kernel<<<nblocks, 256, 0, WST_STREAM>>>((const float *)logits, n, partial, &rs->maxv,
                                                   rs->counts, &rs->max_counter);
  head_counts_kernel<<<nblocks, 256, 0, WST_STREAM>>>(
      (const float *)logits, n, &rs->maxv, rs->counts, &rs->count_counter, k, cap, &rs->thresh,
      nullptr, &rs->enabled);
  head_select_rescore_kernel<<<nblocks, 256, 0, WST_STREAM>>>(
      (const uint16_t *)head, (const uint16_t *)x, (float *)logits, n, hidden, rs);
  WST_TRY_KERNEL("wst_head_rescore_fused");
  return WST_OK;
}
