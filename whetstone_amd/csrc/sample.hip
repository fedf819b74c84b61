// Token selection on the device: argmax (greedy) and the NLL accumulator.
// reference: crates/whetstone-kernels/cuda/sample.cu.
//
// The argmax packs (order-preserving value key, complemented index) into one
// u64 and takes the maximum (sample.cu:28-37): ties go to the lowest index and
// the result is deterministic. The cross-block combine is done by the last
// block to finish, which also resets the counter, so a call is one launch and
// a captured graph needs no memset node.
#include "common.hpp"

#define ARGMAX_MAX_BLOCKS 256

struct ArgmaxScratch {
  unsigned long long partial[ARGMAX_MAX_BLOCKS];
  unsigned int counter;
  unsigned int pad[63];
  float2 nll_partial[ARGMAX_MAX_BLOCKS];
  unsigned int nll_counter;
};

__device__ __forceinline__ unsigned long long block_argmax_key(const float *__restrict__ v,
                                                               int n, int row_off) {
  __shared__ unsigned long long wbest[16];
  unsigned long long best = 0ull;
  const int stride = gridDim.x * blockDim.x;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const unsigned long long c = argmax_key(v[(size_t)row_off + i], i);
    best = c > best ? c : best;
  }
  best = wave_max_u64(best);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
  __syncthreads();
  unsigned long long b = wbest[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) b = wbest[w] > b ? wbest[w] : b;
  return b;
}

// `pos`, when non-null, is advanced (saturating at max_seq) by the combining
// block: the fused argmax + position advance of the engine's step.
__global__ __launch_bounds__(256) void argmax_kernel(const float *__restrict__ logits, int n,
                                                     ArgmaxScratch *__restrict__ sc,
                                                     int32_t *__restrict__ out,
                                                     int32_t *__restrict__ pos, int max_seq) {
  const unsigned long long b = block_argmax_key(logits, n, 0);
  if (threadIdx.x == 0) sc->partial[blockIdx.x] = b;
  if (!last_block_done(&sc->counter, gridDim.x)) return;
  // Every thread loads one partial (gridDim <= 256), then a block max.
  __shared__ unsigned long long wb[4];
  unsigned long long best = threadIdx.x < gridDim.x ? sc->partial[threadIdx.x] : 0ull;
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) best = wb[w] > best ? wb[w] : best;
    best = wb[0] > best ? wb[0] : best;
    *out = (int32_t)(~(uint32_t)(best & 0xFFFFFFFFull));
    if (pos) {
      const int p = *pos + 1;
      *pos = p < max_seq ? p : max_seq;
    }
  }
}

static ArgmaxScratch *argmax_scratch() {
  return (ArgmaxScratch *)wst_static_scratch(WST_SCRATCH_ARGMAX, sizeof(ArgmaxScratch));
}

static int argmax_blocks(int n) {
  int b = (n + 1023) / 1024;
  if (b > ARGMAX_MAX_BLOCKS) b = ARGMAX_MAX_BLOCKS;
  if (b < 1) b = 1;
  return b;
}

extern "C" wst_status_t wst_argmax(const void *logits, void *out_idx, int32_t n) {
  WST_REQUIRE(logits && out_idx, "wst_argmax: null pointer");
  WST_REQUIRE(n > 0, "wst_argmax: n must be positive");
  ArgmaxScratch *sc = argmax_scratch();
  if (!sc) return WST_ERR_OOM;
  argmax_kernel<<<argmax_blocks(n), 256, 0, WST_STREAM>>>((const float *)logits, n, sc,
                                                          (int32_t *)out_idx, nullptr, 0);
  WST_TRY_KERNEL("wst_argmax");
  return WST_OK;
}

extern "C" wst_status_t wst_argmax_advance(const void *logits, void *out_idx, int32_t n,
                                           void *pos, int32_t max_seq) {
  WST_REQUIRE(logits && out_idx && pos, "wst_argmax_advance: null pointer");
  WST_REQUIRE(n > 0 && max_seq > 0, "wst_argmax_advance: bad shape");
  ArgmaxScratch *sc = argmax_scratch();
  if (!sc) return WST_ERR_OOM;
  argmax_kernel<<<argmax_blocks(n), 256, 0, WST_STREAM>>>((const float *)logits, n, sc,
                                                          (int32_t *)out_idx, (int32_t *)pos,
                                                          max_seq);
  WST_TRY_KERNEL("wst_argmax_advance");
  return WST_OK;
}

// Row-wise argmax of [n][vocab] (chunk_ops.cu:425-468): one block per row.
__global__ __launch_bounds__(256) void argmax_rows_kernel(const float *__restrict__ logits,
                                                          int vocab, int32_t *__restrict__ out) {
  __shared__ unsigned long long wbest[4];
  const float *row = logits + (size_t)blockIdx.x * vocab;
  unsigned long long best = 0ull;
  for (int i = threadIdx.x; i < vocab; i += 256) {
    const unsigned long long c = argmax_key(row[i], i);
    best = c > best ? c : best;
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = wbest[0];
    for (int w = 1; w < 4; ++w) b = wbest[w] > b ? wbest[w] : b;
    out[blockIdx.x] = (int32_t)(~(uint32_t)(b & 0xFFFFFFFFull));
  }
}

// The same for rows of a multiple of 4 logits on 16-byte boundaries: 1024
// threads a row, 16-byte loads, four in flight per thread (the key maximum
// does not depend on the order: same result). The 256-thread form with one
// 4-byte load per iteration waited out a load per step: 204 us over 256
// rows of 151936 logits (155 MB).
__global__ __launch_bounds__(1024) void argmax_rows4_kernel(const float *__restrict__ logits,
                                                           int vocab, int32_t *__restrict__ out) {
  __shared__ unsigned long long wbest[16];
  const float4 *row = (const float4 *)(logits + (size_t)blockIdx.x * vocab);
  const int n4 = vocab >> 2;
  unsigned long long best = 0ull;
  int i = threadIdx.x;
  for (; i + 3 * 1024 < n4; i += 4 * 1024) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = row[i + u * 1024];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int b = 4 * (i + u * 1024);
      best = u64_max(best, u64_max(u64_max(argmax_key(v[u].x, b), argmax_key(v[u].y, b + 1)),
                                   u64_max(argmax_key(v[u].z, b + 2), argmax_key(v[u].w, b + 3))));
    }
  }
  for (; i < n4; i += 1024) {
    const float4 v = row[i];
    const int b = 4 * i;
    best = u64_max(best, u64_max(u64_max(argmax_key(v.x, b), argmax_key(v.y, b + 1)),
                                 u64_max(argmax_key(v.z, b + 2), argmax_key(v.w, b + 3))));
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = wbest[0];
    for (int w = 1; w < 16; ++w) b = u64_max(b, wbest[w]);
    out[blockIdx.x] = (int32_t)(~(uint32_t)(b & 0xFFFFFFFFull));
  }
}

extern "C" wst_status_t wst_argmax_chunk(const void *logits, void *out, int32_t vocab,
                                         int32_t n) {
  WST_REQUIRE(logits && out, "wst_argmax_chunk: null pointer");
  WST_REQUIRE(vocab > 0 && n > 0, "wst_argmax_chunk: bad shape");
  if (vocab % 4 == 0 && !((uintptr_t)logits & 15u)) {
    argmax_rows4_kernel<<<n, 1024, 0, WST_STREAM>>>((const float *)logits, vocab, (int32_t *)out);
    WST_TRY_KERNEL("wst_argmax_chunk");
    return WST_OK;
  }
  argmax_rows_kernel<<<n, 256, 0, WST_STREAM>>>((const float *)logits, vocab, (int32_t *)out);
  WST_TRY_KERNEL("wst_argmax_chunk");
  return WST_OK;
}

// ------------------------------------------------------------- perplexity

// -log softmax(logits)[target] accumulated into acc[0], count into acc[1]
// (sample.cu:102-180). Online logsumexp per block, last block combines.
__global__ __launch_bounds__(256) void nll_kernel(const float *__restrict__ logits, int n,
                                                  int target, ArgmaxScratch *__restrict__ sc,
                                                  float *__restrict__ acc) {
  __shared__ float sm[4], sl[4];
  float m = -INFINITY, l = 0.0f;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const float v = logits[i];
    const float mn = fmaxf(m, v);
    l = l * __expf(m - mn) + __expf(v - mn);
    m = mn;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float om = __shfl_xor(m, o, 64), ol = __shfl_xor(l, o, 64);
    const float mn = fmaxf(m, om);
    l = (m == -INFINITY ? 0.0f : l * __expf(m - mn)) + (om == -INFINITY ? 0.0f : ol * __expf(om - mn));
    m = mn;
  }
  if ((threadIdx.x & 63) == 0) {
    sm[threadIdx.x >> 6] = m;
    sl[threadIdx.x >> 6] = l;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = sm[0], L = sl[0];
    for (int w = 1; w < 4; ++w) {
      const float mn = fmaxf(M, sm[w]);
      L = (M == -INFINITY ? 0.0f : L * __expf(M - mn)) +
          (sm[w] == -INFINITY ? 0.0f : sl[w] * __expf(sm[w] - mn));
      M = mn;
    }
    sc->nll_partial[blockIdx.x] = make_float2(M, L);
  }
  if (!last_block_done(&sc->nll_counter, gridDim.x)) return;
  if (threadIdx.x == 0) {
    float M = sc->nll_partial[0].x, L = sc->nll_partial[0].y;
    for (unsigned int b = 1; b < gridDim.x; ++b) {
      const float2 p = sc->nll_partial[b];
      const float mn = fmaxf(M, p.x);
      L = (M == -INFINITY ? 0.0f : L * __expf(M - mn)) +
          (p.x == -INFINITY ? 0.0f : p.y * __expf(p.x - mn));
      M = mn;
    }
    acc[0] += logf(L) + M - logits[target];
    acc[1] += 1.0f;
  }
}

extern "C" wst_status_t wst_nll(const void *logits, int32_t target, void *acc, int32_t n) {
  WST_REQUIRE(logits && acc, "wst_nll: null pointer");
  WST_REQUIRE(n > 0, "wst_nll: n must be positive");
  WST_REQUIRE(target >= 0 && target < n, "wst_nll: target outside the vocabulary");
  ArgmaxScratch *sc = argmax_scratch();
  if (!sc) return WST_ERR_OOM;
  nll_kernel<<<argmax_blocks(n), 256, 0, WST_STREAM>>>((const float *)logits, n, target, sc,
                                                       (float *)acc);
  WST_TRY_KERNEL("wst_nll");
  return WST_OK;
}
