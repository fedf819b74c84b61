// Device-side fixture generation: seeded N(0, std) weights and the int4-hier-g32
// packer, so 7B-shaped synthetic models are built in HBM in seconds.
//
// The packer restates crates/whetstone-quant/src/hier.rs:113-391 operation for
// operation, in f32 with no contraction (#pragma clang fp contract(off)),
// correctly rounded division and square root (HIP's default), roundf = round
// half away from zero (Rust's f32::round) and Rust's saturating float->int
// casts. It is checked bit-exact against the host restatement in oracle/.
#include "common.hpp"

#define HGROUP 32

// ------------------------------------------------------------------- RNG

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__device__ __forceinline__ uint64_t stream_key(uint64_t seed, uint64_t stream) {
  return splitmix64(seed ^ splitmix64(stream + 0x632BE59BD9B4E019ull));
}

// Sum of twelve 16-bit uniforms (elements 3*index .. 3*index+2 of the
// splitmix64 sequence keyed by (seed, stream)), re-centred; exact in integers,
// one f32 rounding at the end.
__device__ __forceinline__ float fixture_normal(uint64_t key, uint64_t index, float std_) {
#pragma clang fp contract(off)
  int64_t s = 0;
#pragma unroll
  for (uint64_t k = 0; k < 3; ++k) {
    const uint64_t h = splitmix64(key + (index * 3u + k) * 0x9E3779B97F4A7C15ull);
    s += (int64_t)(h & 0xFFFFu) + (int64_t)((h >> 16) & 0xFFFFu) +
         (int64_t)((h >> 32) & 0xFFFFu) + (int64_t)(h >> 48);
  }
  const int32_t n = (int32_t)(s * 2 + 12 - 12 * 65536);
  return __fmul_rn(__fmul_rn((float)n, 7.62939453125e-06f), std_);
}

__global__ void fixture_f32_kernel(float *__restrict__ out, size_t n, uint64_t key,
                                   uint64_t index0, float std_) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = fixture_normal(key, index0 + i, std_);
}

__global__ void fixture_f16_kernel(uint16_t *__restrict__ out, size_t n, uint64_t key,
                                   uint64_t index0, float std_, float offset) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = f2h(__fadd_rn(offset, fixture_normal(key, index0 + i, std_)));
}

static int fill_blocks(size_t n) {
  size_t b = (n + 255) / 256;
  const size_t cap = (size_t)wst_cu_count() * 32;
  return (int)(b < cap ? (b ? b : 1) : cap);
}

static uint64_t host_splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
static uint64_t host_stream_key(uint64_t seed, uint64_t stream) {
  return host_splitmix64(seed ^ host_splitmix64(stream + 0x632BE59BD9B4E019ull));
}

extern "C" wst_status_t wst_fixture_normal_f32(void *out, size_t n, uint64_t seed,
                                               uint64_t stream, uint64_t index0, float std_) {
  WST_REQUIRE(out, "wst_fixture_normal_f32: null pointer");
  if (n == 0) return WST_OK;
  fixture_f32_kernel<<<fill_blocks(n), 256, 0, WST_STREAM>>>(
      (float *)out, n, host_stream_key(seed, stream), index0, std_);
  WST_TRY_KERNEL("wst_fixture_normal_f32");
  return WST_OK;
}

extern "C" wst_status_t wst_fixture_normal_f16(void *out, size_t n, uint64_t seed,
                                               uint64_t stream, uint64_t index0, float std_,
                                               float offset) {
  WST_REQUIRE(out, "wst_fixture_normal_f16: null pointer");
  if (n == 0) return WST_OK;
  fixture_f16_kernel<<<fill_blocks(n), 256, 0, WST_STREAM>>>(
      (uint16_t *)out, n, host_stream_key(seed, stream), index0, std_, offset);
  WST_TRY_KERNEL("wst_fixture_normal_f16");
  return WST_OK;
}

// ----------------------------------------------------------------- packer

__device__ __forceinline__ float rclamp(float v, float lo, float hi) {
  if (v < lo) v = lo;
  if (v > hi) v = hi;
  return v;
}

// Rust `as u32` of a float: NaN -> 0, saturating.
__device__ __forceinline__ uint32_t rust_as_u(float v, float hi) {
  if (v != v) return 0u;
  if (v <= 0.0f) return 0u;
  if (v >= hi) return (uint32_t)hi;
  return (uint32_t)v;
}

// make_qkx2_quants fit of one group of 32 (hier.rs:113-195).
__device__ void fit_group(const float *x, float &out_scale, float &out_min) {
#pragma clang fp contract(off)
  const float QMAX = 15.0f, RMIN = -1.0f, RDELTA = 0.1f;
  float ss = 0.0f;
  for (int i = 0; i < HGROUP; ++i) ss = ss + x[i] * x[i];
  const float av = sqrtf(ss / 32.0f);
  float lo = INFINITY, hi = -INFINITY;
  for (int i = 0; i < HGROUP; ++i) lo = fminf(lo, x[i]);
  lo = fminf(lo, 0.0f);
  for (int i = 0; i < HGROUP; ++i) hi = fmaxf(hi, x[i]);
  const float rng = hi - lo;
  if (!(rng - rng == 0.0f) || rng <= 0.0f) {  // !finite || <= 0
    out_scale = 0.0f;
    out_min = fminf(lo, 0.0f);
    return;
  }
  float w[HGROUP];
  for (int i = 0; i < HGROUP; ++i) w[i] = av + fabsf(x[i]);
  float sum_w = 0.0f, sum_x = 0.0f;
  for (int i = 0; i < HGROUP; ++i) sum_w = sum_w + w[i];
  for (int i = 0; i < HGROUP; ++i) sum_x = sum_x + w[i] * x[i];
  float best_scale = rng / QMAX, best_min = lo, best_err = 0.0f;
  {
    const float s = best_scale;
    for (int i = 0; i < HGROUP; ++i) {
      const float q = rclamp(roundf((x[i] - lo) / s), 0.0f, QMAX);
      const float d = q * s + lo - x[i];
      best_err = best_err + w[i] * d * d;
    }
  }
  for (int step = 0; step <= 20; ++step) {
    const float iscale = (QMAX + RMIN + RDELTA * (float)step) / rng;
    float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
    float lvl[HGROUP];
    for (int i = 0; i < HGROUP; ++i) {
      const float l = rclamp(roundf(iscale * (x[i] - lo)), 0.0f, QMAX);
      lvl[i] = l;
      sum_l = sum_l + w[i] * l;
      sum_l2 = sum_l2 + w[i] * l * l;
      sum_xl = sum_xl + w[i] * l * x[i];
    }
    const float det = sum_w * sum_l2 - sum_l * sum_l;
    if (det <= 0.0f) continue;
    float scale = (sum_w * sum_xl - sum_x * sum_l) / det;
    float mn = (sum_l2 * sum_x - sum_l * sum_xl) / det;
    if (mn > 0.0f) {
      mn = 0.0f;
      scale = (sum_l2 > 0.0f) ? sum_xl / sum_l2 : scale;
    }
    float err = 0.0f;
    for (int i = 0; i < HGROUP; ++i) {
      const float d = scale * lvl[i] + mn - x[i];
      err = err + w[i] * d * d;
    }
    if (err < best_err) {
      best_err = err;
      best_scale = scale;
      best_min = mn;
    }
  }
  out_scale = best_scale;
  out_min = best_min;
}

// hier.rs:219-233
__device__ __forceinline__ uint16_t shared_scale(float v) {
  if (v != v || v <= 0.0f) return 0x3C00u;  // f16 1.0
  const uint16_t h = f2h(v);
  if (h2f(h) > 0.0f) return ((h & 0x7C00u) != 0x7C00u) ? h : (uint16_t)0x7BFFu;
  return 1u;
}

// One block per row. The 32 weights of a group are generated (or read) into
// registers by the thread that owns the group; the per-row maxima are block
// reductions (max is exact in any order).
template <bool GEN>
__global__ __launch_bounds__(256) void pack_hier_kernel(const float *__restrict__ w,
                                                        uint32_t *__restrict__ qw,
                                                        uint8_t *__restrict__ si,
                                                        uint32_t *__restrict__ sb, int in_f,
                                                        int64_t row0, uint64_t key, float std_) {
#pragma clang fp contract(off)
  __shared__ float red[16];
  __shared__ float s_scale[1024], s_min[1024];
  const int G = in_f / HGROUP;
  const int64_t r = blockIdx.x;  // row within this tensor
  float max_scale = 0.0f, max_min = 0.0f;
  for (int g = threadIdx.x; g < G; g += blockDim.x) {
    float x[HGROUP];
    for (int i = 0; i < HGROUP; ++i) {
      const int64_t e = r * in_f + (int64_t)g * HGROUP + i;
      x[i] = GEN ? fixture_normal(key, (uint64_t)e, std_) : w[e];
    }
    float s, m;
    fit_group(x, s, m);
    s_scale[g] = s;
    s_min[g] = m;
    max_scale = fmaxf(max_scale, s);
    max_min = fmaxf(max_min, -m);
  }
  max_scale = block_max(max_scale, red);
  max_min = block_max(max_min, red);
  const uint16_t d = shared_scale(max_scale > 0.0f ? max_scale / 15.0f : 1.0f);
  const bool dm_pos = max_min > 0.0f;
  const uint16_t dm = shared_scale(dm_pos ? max_min / 15.0f : 1.0f);
  const float df = h2f(d), dmf = h2f(dm);
  const int64_t R = row0 + r;
  if (threadIdx.x == 0) sb[R] = (uint32_t)d | ((uint32_t)dm << 16);
  for (int g = threadIdx.x; g < G; g += blockDim.x) {
    const uint32_t ls = rust_as_u(rclamp(roundf(s_scale[g] / df), 1.0f, 15.0f), 255.0f);
    const uint32_t lm =
        dm_pos ? rust_as_u(rclamp(roundf(fmaxf(-s_min[g], 0.0f) / dmf), 0.0f, 15.0f), 255.0f)
               : 0u;
    si[R * G + g] = (uint8_t)(ls | (lm << 4));
    const float s = df * (float)ls;
    const float m = -dmf * (float)lm;
    uint32_t words[4] = {0u, 0u, 0u, 0u};
    for (int i = 0; i < HGROUP; ++i) {
      const int64_t e = r * in_f + (int64_t)g * HGROUP + i;
      const float v = GEN ? fixture_normal(key, (uint64_t)e, std_) : w[e];
      const uint32_t q = rust_as_u(rclamp(roundf((v - m) / s), 0.0f, 15.0f), 4294967295.0f);
      words[i / 8] |= q << (4 * (i % 8));
    }
    uint4 *dst = (uint4 *)(qw + (R * G + g) * 4);
    *dst = make_uint4(words[0], words[1], words[2], words[3]);
  }
}

static wst_status_t pack_check(const void *qw, const void *si, const void *sb, int64_t in_f,
                               int64_t rows) {
  WST_REQUIRE(qw && si && sb, "wst_pack_hier: null pointer");
  WST_REQUIRE(in_f > 0 && in_f % HGROUP == 0 && in_f / HGROUP <= 1024,
              "wst_pack_hier: in_f must be a multiple of 32 and at most 32768");
  WST_REQUIRE(rows >= 0 && rows <= 0x7FFFFFFF, "wst_pack_hier: bad row count");
  return WST_OK;
}

extern "C" wst_status_t wst_fixture_pack_hier(void *qw, void *si, void *sb, int64_t in_f,
                                              int64_t row0, int64_t rows, uint64_t seed,
                                              uint64_t stream, float std_) {
  const wst_status_t st = pack_check(qw, si, sb, in_f, rows);
  if (st != WST_OK) return st;
  if (rows == 0) return WST_OK;
  pack_hier_kernel<true><<<(unsigned)rows, 256, 0, WST_STREAM>>>(
      nullptr, (uint32_t *)qw, (uint8_t *)si, (uint32_t *)sb, (int)in_f, row0,
      host_stream_key(seed, stream), std_);
  WST_TRY_KERNEL("wst_fixture_pack_hier");
  return WST_OK;
}

extern "C" wst_status_t wst_quantize_int4_hier(const void *w, void *qw, void *si, void *sb,
                                               int64_t in_f, int64_t rows) {
  WST_REQUIRE(w, "wst_quantize_int4_hier: null pointer");
  const wst_status_t st = pack_check(qw, si, sb, in_f, rows);
  if (st != WST_OK) return st;
  if (rows == 0) return WST_OK;
  pack_hier_kernel<false><<<(unsigned)rows, 256, 0, WST_STREAM>>>(
      (const float *)w, (uint32_t *)qw, (uint8_t *)si, (uint32_t *)sb, (int)in_f, 0, 0, 0.0f);
  WST_TRY_KERNEL("wst_quantize_int4_hier");
  return WST_OK;
}

// ------------------------------------------------------------- KV context

__global__ void fill_kv_kernel(uint16_t *__restrict__ k, uint16_t *__restrict__ v, int n_kv,
                               int max_seq, int hd, int n, uint64_t key) {
  const size_t total = (size_t)n_kv * 2 * n * hd;
  for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < total;
       e += (size_t)gridDim.x * blockDim.x) {
    const int i = (int)(e % hd);
    const int t = (int)((e / hd) % n);
    const int kv = (int)((e / ((size_t)hd * n)) % 2);
    const int h = (int)(e / ((size_t)hd * n * 2));
    const uint64_t idx = ((((uint64_t)(h * 2 + kv)) << 20) + (uint64_t)t) * (uint64_t)hd + i;
    const uint16_t val = f2h(fixture_normal(key, idx, 1.0f));
    (kv ? v : k)[((size_t)h * max_seq + t) * hd + i] = val;
  }
}

extern "C" wst_status_t wst_fixture_fill_kv(void *k_cache, void *v_cache, int32_t n_kv,
                                            int32_t max_seq, int32_t head_dim, int32_t n,
                                            uint64_t seed, uint64_t stream) {
  WST_REQUIRE(k_cache && v_cache, "wst_fixture_fill_kv: null pointer");
  WST_REQUIRE(n_kv > 0 && max_seq > 0 && head_dim > 0 && n >= 0 && n <= max_seq,
              "wst_fixture_fill_kv: bad shape");
  WST_REQUIRE(n < (1 << 20), "wst_fixture_fill_kv: context too long");
  if (n == 0) return WST_OK;
  const size_t total = (size_t)n_kv * 2 * n * head_dim;
  fill_kv_kernel<<<fill_blocks(total), 256, 0, WST_STREAM>>>(
      (uint16_t *)k_cache, (uint16_t *)v_cache, n_kv, max_seq, head_dim, n,
      host_stream_key(seed, stream));
  WST_TRY_KERNEL("wst_fixture_fill_kv");
  return WST_OK;
}
