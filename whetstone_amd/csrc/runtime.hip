// Device, memory, graphs, events and the bandwidth probe: the non-kernel half
// of the C ABI (reference: crates/whetstone-kernels/cuda/runtime.cu,
// cuda/graph.cu).
#include "common.hpp"

#include <mutex>

thread_local char wst_err_buf[512] = "no error";

extern "C" const char *wst_last_error(void) { return wst_err_buf; }

extern "C" void wst_abi_layout(wst_abi_layout_t *out) {
  if (out == nullptr) return;
  out->device_info_size = (uint32_t)sizeof(wst_device_info_t);
  out->device_info_align = (uint32_t)alignof(wst_device_info_t);
  out->probe_size = (uint32_t)sizeof(wst_probe_t);
  out->probe_align = (uint32_t)alignof(wst_probe_t);
}

// ------------------------------------------------------------- device facts

static constexpr int kMaxDevices = 64;
static int g_cu_count[kMaxDevices];
static void *g_scratch[kMaxDevices][WST_SCRATCH_SLOTS];
static size_t g_scratch_bytes[kMaxDevices][WST_SCRATCH_SLOTS];
static std::mutex g_mu;

static int current_device() {
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= kMaxDevices) return 0;
  return d;
}

int wst_cu_count() {
  const int d = current_device();
  int n = g_cu_count[d];
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess ||
        n <= 0)
      n = 256;
    g_cu_count[d] = n;
  }
  return n;
}

void *wst_static_scratch(int slot, size_t bytes) {
  const int d = current_device();
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[d][slot] != nullptr && g_scratch_bytes[d][slot] >= bytes)
    return g_scratch[d][slot];
  // Growing a slot is only legal outside graph capture; the engine runs an
  // eager warm-up step first, as the reference does (engine.rs:352-367).
  if (g_scratch[d][slot] != nullptr) {
    (void)hipDeviceSynchronize();
    (void)hipFree(g_scratch[d][slot]);
    g_scratch[d][slot] = nullptr;
  }
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    wst_set_error("static scratch hipMalloc", e);
    return nullptr;
  }
  e = hipMemset(p, 0, bytes);
  if (e != hipSuccess) {
    wst_set_error("static scratch hipMemset", e);
    (void)hipFree(p);
    return nullptr;
  }
  g_scratch[d][slot] = p;
  g_scratch_bytes[d][slot] = bytes;
  return p;
}

extern "C" wst_status_t wst_device_count(int32_t *out_count) {
  WST_REQUIRE(out_count != nullptr, "wst_device_count: null out_count");
  int n = 0;
  WST_TRY(hipGetDeviceCount(&n));
  *out_count = n;
  return WST_OK;
}

extern "C" wst_status_t wst_device_set(int32_t ordinal) {
  WST_REQUIRE(ordinal >= 0 && ordinal < kMaxDevices, "wst_device_set: ordinal out of range");
  WST_TRY(hipSetDevice(ordinal));
  return WST_OK;
}

extern "C" wst_status_t wst_device_synchronize(void) {
  WST_TRY(hipDeviceSynchronize());
  return WST_OK;
}

extern "C" wst_status_t wst_device_info(int32_t ordinal, wst_device_info_t *out) {
  WST_REQUIRE(out != nullptr, "wst_device_info: null out");
  hipDeviceProp_t p;
  WST_TRY(hipGetDeviceProperties(&p, ordinal));
  memset(out, 0, sizeof(*out));
  snprintf(out->name, sizeof(out->name), "%s (%s)", p.name, p.gcnArchName);
  out->major = p.major;
  out->minor = p.minor;
  out->sm_count = p.multiProcessorCount;
  out->clock_khz = p.clockRate;
  out->mem_clock_khz = p.memoryClockRate;
  out->mem_bus_width = p.memoryBusWidth;
  out->max_threads_per_block = p.maxThreadsPerBlock;
  out->max_smem_per_block = (int32_t)p.sharedMemPerBlock;
  out->warp_size = p.warpSize;
  out->l2_bytes = p.l2CacheSize;
  out->mem_total = (uint64_t)p.totalGlobalMem;
  out->bandwidth_gbs = 2.0 * (double)p.memoryClockRate * (p.memoryBusWidth / 8.0) / 1.0e6;
  size_t freeb = 0, totalb = 0;
  int cur = 0;
  if (hipGetDevice(&cur) == hipSuccess && cur == ordinal &&
      hipMemGetInfo(&freeb, &totalb) == hipSuccess) {
    out->mem_free = (uint64_t)freeb;
    out->mem_total = (uint64_t)totalb;
  }
  // CDNA equivalents of the reference's capability flags (runtime.cu:63-71).
  const bool cdna = strncmp(p.gcnArchName, "gfx9", 4) == 0;
  out->has_tensor_cores = cdna;  // MFMA
  out->has_imma = cdna;          // int8 MFMA
  out->has_fp8 = strncmp(p.gcnArchName, "gfx950", 6) == 0 ||
                 strncmp(p.gcnArchName, "gfx942", 6) == 0;
  return WST_OK;
}

// ------------------------------------------------------------------ memory

extern "C" wst_status_t wst_malloc(void **out_ptr, size_t bytes) {
  WST_REQUIRE(out_ptr != nullptr, "wst_malloc: null out_ptr");
  *out_ptr = nullptr;
  if (bytes == 0) return WST_OK;
  void *p = nullptr;
  const hipError_t e = hipMalloc(&p, bytes);
  if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) {
    (void)hipGetLastError();
    snprintf(wst_err_buf, sizeof(wst_err_buf), "wst_malloc: out of device memory (%zu bytes)",
             bytes);
    return WST_ERR_OOM;
  }
  if (e != hipSuccess) {
    wst_set_error("hipMalloc", e);
    return WST_ERR_CUDA;
  }
  *out_ptr = p;
  return WST_OK;
}

extern "C" wst_status_t wst_malloc_host(void **out_ptr, size_t bytes) {
  if (out_ptr) *out_ptr = nullptr;
  wst_set_error_msg(
      "wst_malloc_host: host-resident weights are not supported by the MI355X backend "
      "(every weight stays resident in HBM)");
  return WST_ERR_UNSUPPORTED_ARCH;
}

extern "C" int32_t wst_host_alloc_supported(void) { return 0; }

extern "C" wst_status_t wst_free(void *ptr) {
  if (ptr == nullptr) return WST_OK;
  WST_TRY(hipFree(ptr));
  return WST_OK;
}

// Blocking, like the reference's cudaMemset/cudaMemcpy (runtime.cu:157-190).
extern "C" wst_status_t wst_memset(void *dst, int32_t value, size_t bytes) {
  if (bytes == 0) return WST_OK;
  WST_REQUIRE(dst != nullptr, "wst_memset: null dst");
  WST_TRY(hipMemsetAsync(dst, value, bytes, WST_STREAM));
  WST_TRY(hipStreamSynchronize(WST_STREAM));
  return WST_OK;
}

extern "C" wst_status_t wst_memcpy_h2d(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return WST_OK;
  WST_REQUIRE(dst && src, "wst_memcpy_h2d: null pointer");
  WST_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, WST_STREAM));
  WST_TRY(hipStreamSynchronize(WST_STREAM));
  return WST_OK;
}

extern "C" wst_status_t wst_memcpy_d2h(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return WST_OK;
  WST_REQUIRE(dst && src, "wst_memcpy_d2h: null pointer");
  WST_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, WST_STREAM));
  WST_TRY(hipStreamSynchronize(WST_STREAM));
  return WST_OK;
}

extern "C" wst_status_t wst_memcpy_d2d(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return WST_OK;
  WST_REQUIRE(dst && src, "wst_memcpy_d2d: null pointer");
  WST_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, WST_STREAM));
  WST_TRY(hipStreamSynchronize(WST_STREAM));
  return WST_OK;
}

// --------------------------------------------------------------- bandwidth

// Streaming read, 16 B per lane per load, four independent loads in flight per
// lane, grid-stride. The sum is consumed so nothing is optimised away.
__global__ __launch_bounds__(256) void bandwidth_read_kernel(const uint4 *__restrict__ src,
                                                             size_t n4, float *__restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n4; i += 4 * stride) {
    const uint4 a = ld_stream16(src + i);
    const uint4 b = ld_stream16(src + i + stride);
    const uint4 c = ld_stream16(src + i + 2 * stride);
    const uint4 d = ld_stream16(src + i + 3 * stride);
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^
           d.z ^ d.w;
  }
  for (; i < n4; i += stride) {
    const uint4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x12345678u) sink[0] = (float)acc;  // practically never true
}

// One launch of the streaming read over a caller's buffer (sink: 16 bytes),
// on the calling thread's stream: the floor a GEMV of the same bytes is held
// against, timed by the caller with the same weights-cold rotation.
extern "C" wst_status_t wst_stream_read(const void *buf, size_t bytes, void *sink) {
  WST_REQUIRE(buf && sink, "wst_stream_read: null pointer");
  WST_REQUIRE(bytes >= 16 && !((uintptr_t)buf & 15u), "wst_stream_read: bad buffer");
  bandwidth_read_kernel<<<wst_cu_count() * 8, 256, 0, WST_STREAM>>>(
      (const uint4 *)buf, bytes / sizeof(uint4), (float *)sink);
  WST_TRY_KERNEL("wst_stream_read");
  return WST_OK;
}

extern "C" wst_status_t wst_bench_bandwidth(size_t bytes, int32_t reps, double *out_gbs) {
  WST_REQUIRE(out_gbs != nullptr, "wst_bench_bandwidth: null out");
  WST_REQUIRE(reps > 0, "wst_bench_bandwidth: reps must be positive");
  WST_REQUIRE(bytes >= 4096, "wst_bench_bandwidth: buffer too small to measure");
  const size_t n4 = bytes / sizeof(uint4);
  void *buf = nullptr, *sink = nullptr;
  wst_status_t st = wst_malloc(&buf, n4 * sizeof(uint4));
  if (st != WST_OK) return st;
  st = wst_malloc(&sink, 16);
  if (st != WST_OK) {
    wst_free(buf);
    return st;
  }
  hipEvent_t a = nullptr, b = nullptr;
  float ms = 0.0f;
  hipError_t e = hipMemsetAsync(buf, 1, n4 * sizeof(uint4), WST_STREAM);
  const int blocks = wst_cu_count() * 8;
  if (e == hipSuccess) e = hipEventCreate(&a);
  if (e == hipSuccess) e = hipEventCreate(&b);
  if (e == hipSuccess) {
    bandwidth_read_kernel<<<blocks, 256, 0, WST_STREAM>>>((const uint4 *)buf, n4, (float *)sink);
    e = hipEventRecord(a, WST_STREAM);
  }
  if (e == hipSuccess) {
    for (int i = 0; i < reps; ++i)
      bandwidth_read_kernel<<<blocks, 256, 0, WST_STREAM>>>((const uint4 *)buf, n4,
                                                            (float *)sink);
    e = hipEventRecord(b, WST_STREAM);
  }
  if (e == hipSuccess) e = hipEventSynchronize(b);
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
  if (e == hipSuccess) e = hipGetLastError();
  if (a) (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  wst_free(buf);
  wst_free(sink);
  if (e != hipSuccess) {
    wst_set_error("wst_bench_bandwidth", e);
    return WST_ERR_CUDA;
  }
  *out_gbs = (double)n4 * sizeof(uint4) * (double)reps / ((double)ms * 1.0e-3) / 1.0e9;
  return WST_OK;
}

// ------------------------------------------------------------------ graphs

extern "C" wst_status_t wst_graph_capture_begin(void) {
  WST_TRY(hipStreamBeginCapture(WST_STREAM, hipStreamCaptureModeThreadLocal));
  return WST_OK;
}

extern "C" wst_status_t wst_graph_capture_end(void **out_exec) {
  WST_REQUIRE(out_exec, "wst_graph_capture_end: null out pointer");
  *out_exec = nullptr;
  hipGraph_t graph = nullptr;
  WST_TRY(hipStreamEndCapture(WST_STREAM, &graph));
  if (graph == nullptr) {
    wst_set_error_msg("wst_graph_capture_end: capture produced no graph");
    return WST_ERR_CUDA;
  }
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) {
    wst_set_error("hipGraphInstantiate", e);
    return WST_ERR_CUDA;
  }
  *out_exec = (void *)exec;
  return WST_OK;
}

extern "C" wst_status_t wst_graph_launch(void *exec) {
  WST_REQUIRE(exec, "wst_graph_launch: null graph");
  WST_TRY(hipGraphLaunch((hipGraphExec_t)exec, WST_STREAM));
  return WST_OK;
}

extern "C" wst_status_t wst_graph_destroy(void *exec) {
  if (exec == nullptr) return WST_OK;
  WST_TRY(hipGraphExecDestroy((hipGraphExec_t)exec));
  return WST_OK;
}

extern "C" wst_status_t wst_stream_sync(void) {
  WST_TRY(hipStreamSynchronize(WST_STREAM));
  return WST_OK;
}

extern "C" wst_status_t wst_event_create(void **out) {
  WST_REQUIRE(out, "wst_event_create: null out pointer");
  hipEvent_t e = nullptr;
  WST_TRY(hipEventCreate(&e));
  *out = (void *)e;
  return WST_OK;
}

extern "C" wst_status_t wst_event_record(void *ev) {
  WST_REQUIRE(ev, "wst_event_record: null event");
  WST_TRY(hipEventRecord((hipEvent_t)ev, WST_STREAM));
  return WST_OK;
}

extern "C" wst_status_t wst_event_elapsed_ms(void *a, void *b, float *out) {
  WST_REQUIRE(a && b && out, "wst_event_elapsed_ms: null pointer");
  WST_TRY(hipEventSynchronize((hipEvent_t)b));
  WST_TRY(hipEventElapsedTime(out, (hipEvent_t)a, (hipEvent_t)b));
  return WST_OK;
}

extern "C" wst_status_t wst_event_destroy(void *ev) {
  if (ev == nullptr) return WST_OK;
  WST_TRY(hipEventDestroy((hipEvent_t)ev));
  return WST_OK;
}

// ------------------------------------------------------------ position cursor

// reference: decode.cu:210-226. One thread; a graph node, not a host update.
__global__ void advance_pos_kernel(int32_t *pos, int max_seq) {
  if (threadIdx.x != 0) return;
  const int p = *pos + 1;
  *pos = p < max_seq ? p : max_seq;
}

extern "C" wst_status_t wst_advance_pos(void *pos, int32_t max_seq) {
  WST_REQUIRE(pos, "wst_advance_pos: null pointer");
  WST_REQUIRE(max_seq > 0, "wst_advance_pos: empty cache");
  advance_pos_kernel<<<1, 64, 0, WST_STREAM>>>((int32_t *)pos, max_seq);
  WST_TRY_KERNEL("wst_advance_pos");
  return WST_OK;
}
