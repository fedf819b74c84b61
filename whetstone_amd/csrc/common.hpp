// Internal helpers shared by the HIP sources. Not part of the C ABI.
//
// gfx950 (CDNA4) facts these helpers are written for: wave64, 256 compute
// units in 8 XCDs, 160 KB LDS per CU, DPP lane permutes within 16-lane rows
// plus row broadcasts across a wave.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "whetstone.h"
#include "whetstone_ext.h"

// ------------------------------------------------------- error propagation
//
// Per-thread message, as the reference keeps it (common.cuh:15-26,
// runtime.cu:5-7): a failure is reported through the status code and
// wst_last_error(), never by aborting.
extern thread_local char wst_err_buf[512];

inline void wst_set_error(const char *where, hipError_t e) {
  snprintf(wst_err_buf, sizeof(wst_err_buf), "%s: %s (%s)", where, hipGetErrorString(e),
           hipGetErrorName(e));
}
inline void wst_set_error_msg(const char *msg) {
  snprintf(wst_err_buf, sizeof(wst_err_buf), "%s", msg);
}

#define WST_TRY(expr)                                                          \
  do {                                                                         \
    hipError_t _e = (expr);                                                    \
    if (_e != hipSuccess) {                                                    \
      wst_set_error(#expr, _e);                                                \
      return WST_ERR_CUDA;                                                     \
    }                                                                          \
  } while (0)

// Launch errors only; no device synchronisation (same contract as the
// reference's WST_TRY_KERNEL, common.cuh:39-46).
#define WST_TRY_KERNEL(name)                                                   \
  do {                                                                         \
    hipError_t _e = hipGetLastError();                                         \
    if (_e != hipSuccess) {                                                    \
      wst_set_error(name " (launch)", _e);                                     \
      return WST_ERR_CUDA;                                                     \
    }                                                                          \
  } while (0)

#define WST_REQUIRE(cond, msg)                                                 \
  do {                                                                         \
    if (!(cond)) {                                                             \
      wst_set_error_msg(msg);                                                  \
      return WST_ERR_INVALID_ARG;                                              \
    }                                                                          \
  } while (0)

#define WST_STREAM hipStreamPerThread

// Cached positions per decode-attention slice for a cache of max_seq
// positions and head size hd (64, 128 or 256); defined in attention.hip.
int wst_attn_slice_len(int hd, int max_seq);

// --------------------------------------------------------- device facts

// Compute units of the current device, cached per device ordinal: a property
// query is far more expensive than the kernels it would size.
int wst_cu_count();

// A lazily created, zero-initialised device scratch region, one per (device,
// slot). Created outside graph capture by the first eager call, exactly like
// the reference's argmax scratch (sample.cu:82-88). Returns nullptr on failure
// (message set).
void *wst_static_scratch(int slot, size_t bytes);
enum {
  WST_SCRATCH_ARGMAX = 0,
  WST_SCRATCH_ATTN = 1,
  WST_SCRATCH_RESCORE = 2,
  WST_SCRATCH_NLL = 3,
  WST_SCRATCH_ENGINE = 4,
  WST_SCRATCH_GEMM = 5,  // split-K partial sums of the chunk GEMMs
  WST_SCRATCH_HEADMAX = 6,  // per-block argmax keys of the head GEMV's argmax form
  WST_SCRATCH_SLOTS = 8
};

// ----------------------------------------------------------- f16 helpers

typedef _Float16 wst_h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float h2f(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
// f32 -> f16, round to nearest even. The empty asm pins `f` as an f32 value in
// a VGPR: without it the compiler may fold the operation that produced `f`
// into a mixed-precision op that rounds the exact result straight to f16
// (v_fma_mix*), which differs from "round to f32, then to f16" at ties.
__device__ __forceinline__ uint16_t f2h(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ wst_h2 as_h2(uint32_t u) { return __builtin_bit_cast(wst_h2, u); }

// 16-byte streaming load with the non-temporal hint: data read exactly once
// per call (packed weights) should not evict what is reused (activations).
typedef uint32_t wst_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream16(const void *p) {
  const wst_u32x4 v = __builtin_nontemporal_load((const wst_u32x4 *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ----------------------------------------------------------- reductions
//
// DPP sums. After dpp_sum16 every lane of each 16-lane row holds that row's
// sum; quad_perm handles xor 1 and 2, half-mirror and mirror finish the row.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over each 8-lane half row, in every lane of it.
__device__ __forceinline__ float dpp_sum8(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  return v;
}

__device__ __forceinline__ float dpp_sum16(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return v;
}

// The same four steps as fused DPP maxima, one VALU op each (written out:
// the compiler's form is a DPP move, a canonicalising max and the max). Each
// op reads the previous one's result through DPP, which needs two wait states
// after the write: the s_nop 1 before each.
__device__ __forceinline__ float dpp_max16(float v) {
  asm("s_nop 1\n\tv_max_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\tv_max_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\tv_max_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\tv_max_f32_dpp %0, %0, %0 row_mirror row_mask:0xf bank_mask:0xf"
      : "+v"(v));
  return v;
}

// Cross-row exchange (gfx950 v_permlane16_swap / v_permlane32_swap, plain
// VALU ops). permlane16_swap(a, b) swaps the odd 16-lane rows of a with the
// even rows of b; called with a == b == v it returns, in both lanes of every
// pair (i, i^16), the even row's value in one result and the odd row's in the
// other (permlane32_swap: the same for the two 32-lane halves). Every caller
// combines the two with a commutative operation, so both lanes of a pair
// compute the same bits whichever result holds which row.
struct RowPair {
  float a, b;
};
__device__ __forceinline__ RowPair xrow16(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return {__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
__device__ __forceinline__ RowPair xrow32(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return {__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
__device__ __forceinline__ float xrow16_sum(float v) {
  const RowPair p = xrow16(v);
  return p.a + p.b;
}
__device__ __forceinline__ float xrow32_sum(float v) {
  const RowPair p = xrow32(v);
  return p.a + p.b;
}
// Sum over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48); every
// lane gets the same bits (each step adds a pair, which commutes).
__device__ __forceinline__ float row4_sum(float v) { return xrow32_sum(xrow16_sum(v)); }

// Sum over the 32 lanes of each half wave, returned in every lane of that half.
__device__ __forceinline__ float half_wave_sum(float v) { return xrow16_sum(dpp_sum16(v)); }

// Sum over the whole wave, in every lane.
__device__ __forceinline__ float wave_sum(float v) {
  return xrow32_sum(xrow16_sum(dpp_sum16(v)));
}

__device__ __forceinline__ float wave_max(float v) {
  v = dpp_max16(v);
  RowPair p = xrow16(v);
  v = fmaxf(p.a, p.b);
  p = xrow32(v);
  return fmaxf(p.a, p.b);
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ int wave_sum_i32(int v) {
  v += dpp_i<0xB1>(v);
  v += dpp_i<0x4E>(v);
  v += dpp_i<0x141>(v);
  v += dpp_i<0x140>(v);
  uint32_t u = (uint32_t)v;
  auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  u = (uint32_t)r[0] + (uint32_t)r[1];
  r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return (int)((uint32_t)r[0] + (uint32_t)r[1]);
}

__device__ __forceinline__ unsigned long long u64_max(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
  const int lo = dpp_i<CTRL>((int)(uint32_t)v), hi = dpp_i<CTRL>((int)(uint32_t)(v >> 32));
  return ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo;
}
__device__ __forceinline__ unsigned long long xrow_u64_max(unsigned long long v, bool x32) {
  const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  const auto rl = x32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                      : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  const auto rh = x32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                      : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  return u64_max(((unsigned long long)(uint32_t)rh[0] << 32) | (uint32_t)rl[0],
                 ((unsigned long long)(uint32_t)rh[1] << 32) | (uint32_t)rl[1]);
}

// Maximum over the wave. Within a 16-lane row the quad swaps and mirrors pair
// every lane with one of the other group at each step (a maximum does not
// need the xor pairing a lane-wise sum of vectors would).
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
  v = u64_max(v, dpp_u64<0xB1>(v));
  v = u64_max(v, dpp_u64<0x4E>(v));
  v = u64_max(v, dpp_u64<0x141>(v));
  v = u64_max(v, dpp_u64<0x140>(v));
  v = xrow_u64_max(v, false);
  return xrow_u64_max(v, true);
}

// Block-wide sum for blocks of up to 1024 threads; every thread gets the
// result. `red` holds 16 floats of LDS. Contains barriers.
__device__ __forceinline__ float block_sum(float v, float *red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nw = (blockDim.x + 63) >> 6;
  v = wave_sum(v);
  __syncthreads();  // `red` may still be read from a previous call
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = 0.0f;
  for (int i = 0; i < nw; ++i) s += red[i];  // fixed order: deterministic
  return s;
}

__device__ __forceinline__ float block_max(float v, float *red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nw = (blockDim.x + 63) >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = -INFINITY;
  for (int i = 0; i < nw; ++i) s = fmaxf(s, red[i]);
  return s;
}

// The RMS scale 1/sqrt(mean(x^2) + eps) of x[0..n), for 512-thread blocks:
// thread t accumulates the 8-element blocks t, t+512, ... (each in element
// order) with fmaf, then block_sum adds the threads in a fixed order. The
// RMSNorm kernel and the GEMV's fused RMSNorm prologue both use this order, so
// they produce the same f16 vector.
__device__ __forceinline__ float rms_scale512(const float *__restrict__ x, int n, float eps,
                                              float *red) {
  float acc = 0.0f;
  for (int b = threadIdx.x; 8 * b < n; b += 512)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (8 * b + e < n) acc = fmaf(x[8 * b + e], x[8 * b + e], acc);
  acc = block_sum(acc, red);
  return 1.0f / sqrtf(acc / (float)n + eps);
}

// ------------------------------------------------------------------ RoPE
//
// Half-rotation RoPE (decode.cu:112-178) with an explicit fma shape, so every
// kernel that rotates (rope_cache, the fused attention prologue) rounds
// identically.
__device__ __forceinline__ float rope_lo(float x1, float x2, float c, float s) {
  return fmaf(x1, c, -(x2 * s));
}
__device__ __forceinline__ float rope_hi(float x1, float x2, float c, float s) {
  return fmaf(x2, c, x1 * s);
}

// Per-head QK-RMSNorm (common.cuh:185-202): thread j holds elements j and
// j+half of the head; the block reduces over all hd elements; shared gain
// [hd]. Called by every thread of the block (it contains barriers).
__device__ __forceinline__ void qk_norm(float &x1, float &x2, const uint16_t *__restrict__ g,
                                        int j, int half, int hd, float eps, bool active,
                                        float *red) {
  const float a = active ? fmaf(x1, x1, x2 * x2) : 0.0f;
  const float ss = block_sum(a, red);
  const float s = 1.0f / sqrtf(ss / (float)hd + eps);
  if (active) {
    x1 = x1 * s * h2f(g[j]);
    x2 = x2 * s * h2f(g[j + half]);
  }
}

// qk_norm for a head held by one wave (not a whole block): the same sum, as
// block_sum over a one-wave block returns the wave's sum.
__device__ __forceinline__ void qk_norm_wave(float &x1, float &x2,
                                             const uint16_t *__restrict__ g, int j, int half,
                                             int hd, float eps, bool active) {
  const float ss = wave_sum(active ? fmaf(x1, x1, x2 * x2) : 0.0f);
  const float s = 1.0f / sqrtf(ss / (float)hd + eps);
  if (active) {
    x1 = x1 * s * h2f(g[j]);
    x2 = x2 * s * h2f(g[j + half]);
  }
}

// ------------------------------------------------------ argmax key
//
// Order-preserving key (sample.cu:28-37): value in the high word, complemented
// index in the low word, so the u64 maximum is the largest value and, among
// equal values, the lowest index.
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)k << 32) | (unsigned long long)(~(uint32_t)idx);
}

// "Last block done": every block calls this once after publishing its partial
// result with plain stores. The block that observes count == nblocks-1 returns
// true (in every thread) and owns the final combine; it also resets the
// counter to zero so the next launch (or a graph replay) starts clean.
//
// Visibility: every wave waits for its own stores to complete (s_waitcnt 0;
// a workgroup barrier alone does not wait for global stores), then the
// barrier orders them before thread 0's
// agent-scope acq_rel add (on gfx950 an L2 write-back, the atomic, then an
// L1/L2 invalidate of this CU and XCD), which makes them visible across XCDs
// and, in the last block, invalidates stale lines before the second barrier
// releases the other waves to read. Agent scope only: a system-scope fence
// writes back and invalidates for the host as well, which cost several
// microseconds per launch.
__device__ __forceinline__ bool last_block_done(unsigned int *counter, unsigned int nblocks) {
  __shared__ bool is_last;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned int prev =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (prev == nblocks - 1);
    if (is_last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return is_last;
}
