// Device runtime of libwxx_hip.so: device selection, the single in-order
// stream, a size-bucketed caching allocator, host<->device copies, fills,
// synchronisation, error reporting and event timers.
//
// Replaces the reference's WebGPU device singleton, buffer pool and shared
// command buffer (reference src/wxx/backend/device.py:9-273).  Differences
// that follow from HIP rather than WebGPU:
//  * one hipStream_t carries every launch, so "flush" is implicit and a
//    buffer freed on the host may be reused by the next enqueued kernel
//    (stream order makes that safe); no deferred-destroy list is needed;
//  * the cache is not capped at 4 MiB: blocks are kept per exact size until
//    wxx_empty_cache() or an allocation failure, sized for 288 GB of HBM.
#include "common.h"

#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>
#include <cstring>

namespace {

thread_local char g_err[512] = "";
bool g_init = false;
int g_device = -1;
int g_cus = 0;
hipStream_t g_stream = nullptr;

std::mutex g_mu;
std::unordered_map<size_t, std::vector<void*>> g_free;  // rounded size -> blocks
std::unordered_map<void*, size_t> g_live;               // block -> rounded size
size_t g_bytes_live = 0, g_bytes_cached = 0, g_bytes_peak = 0;
size_t g_n_malloc = 0;

// Pinned staging ring for small host->device uploads, so an upload does not
// have to wait for the stream to drain.
constexpr size_t kStageSlot = 1 << 20;
constexpr int kStageSlots = 16;
char* g_stage = nullptr;
hipEvent_t g_stage_ev[kStageSlots];
bool g_stage_used[kStageSlots];
int g_stage_next = 0;

constexpr int kTimers = 64;
hipEvent_t g_timer[kTimers];

size_t round_size(size_t n) {
  if (n == 0) n = 1;
  if (n <= (1u << 20)) return (n + 511) & ~size_t(511);
  return (n + (size_t(2) << 20) - 1) & ~((size_t(2) << 20) - 1);
}

void release_cached_locked() {
  for (auto& kv : g_free)
    for (void* p : kv.second) (void)hipFree(p);
  g_free.clear();
  g_bytes_cached = 0;
}

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = v;
}

}  // namespace

namespace wxx {

hipStream_t stream() { return g_stream; }
bool initialised() { return g_init; }
int num_cus() { return g_cus; }

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void* scratch_alloc(size_t bytes) {
  size_t r = round_size(bytes);
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_free.find(r);
  void* p = nullptr;
  if (it != g_free.end() && !it->second.empty()) {
    p = it->second.back();
    it->second.pop_back();
    g_bytes_cached -= r;
  } else {
    if (hipMalloc(&p, r) != hipSuccess) {
      (void)hipGetLastError();
      release_cached_locked();
      if (hipMalloc(&p, r) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
      }
    }
    ++g_n_malloc;
  }
  g_live[p] = r;
  g_bytes_live += r;
  if (g_bytes_live > g_bytes_peak) g_bytes_peak = g_bytes_live;
  return p;
}

void scratch_free(void* p) {
  if (!p) return;
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_live.find(p);
  if (it == g_live.end()) return;
  size_t r = it->second;
  g_live.erase(it);
  g_bytes_live -= r;
  g_free[r].push_back(p);
  g_bytes_cached += r;
}

}  // namespace wxx

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

WXX_API const char* wxx_last_error() { return g_err; }

WXX_API int wxx_device_count(int* count) {
  WXX_REQUIRE(count, "count is null");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    *count = 0;
    return wxx::set_error(WXX_E_INIT, "hipGetDeviceCount: %s", hipGetErrorString(e));
  }
  *count = n;
  return WXX_OK;
}

WXX_API int wxx_init(int device) {
  if (g_init) {
    if (device == g_device) return WXX_OK;
    return wxx::set_error(WXX_E_ARG, "already initialised on device %d", g_device);
  }
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
    return wxx::set_error(WXX_E_INIT, "no HIP device available");
  WXX_REQUIRE(device >= 0 && device < n, "device %d out of range [0,%d)", device, n);
  WXX_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  WXX_HIP(hipGetDeviceProperties(&prop, device));
  g_cus = prop.multiProcessorCount;
  // Default priority only: streams of mixed priorities are avoided on purpose.
  WXX_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  WXX_HIP(hipHostMalloc((void**)&g_stage, kStageSlot * kStageSlots, hipHostMallocDefault));
  for (int i = 0; i < kStageSlots; ++i) {
    WXX_HIP(hipEventCreateWithFlags(&g_stage_ev[i], hipEventDisableTiming));
    g_stage_used[i] = false;
  }
  for (int i = 0; i < kTimers; ++i) WXX_HIP(hipEventCreate(&g_timer[i]));
  {
    const int rc = wxx::gemm_noalloc_setup(device);
    if (rc != WXX_OK) return rc;
  }
  g_device = device;
  g_init = true;
  return WXX_OK;
}

WXX_API int wxx_device_info(int* cus, char* name, int name_len, size_t* total_mem) {
  WXX_CHECK_INIT();
  hipDeviceProp_t prop;
  WXX_HIP(hipGetDeviceProperties(&prop, g_device));
  if (cus) *cus = prop.multiProcessorCount;
  if (name && name_len > 0) {
    snprintf(name, name_len, "%s (%s)", prop.name, prop.gcnArchName);
  }
  if (total_mem) *total_mem = prop.totalGlobalMem;
  return WXX_OK;
}

WXX_API void* wxx_alloc(size_t bytes) {
  if (!g_init) {
    wxx::set_error(WXX_E_INIT, "wxx_init() has not been called");
    return nullptr;
  }
  void* p = wxx::scratch_alloc(bytes);
  if (!p) wxx::set_error(WXX_E_OOM, "device allocation of %zu bytes failed", bytes);
  return p;
}

WXX_API int wxx_free(void* p) {
  if (!p) return WXX_OK;
  WXX_CHECK_INIT();
  wxx::scratch_free(p);
  return WXX_OK;
}

WXX_API int wxx_empty_cache() {
  WXX_CHECK_INIT();
  WXX_HIP(hipStreamSynchronize(g_stream));
  std::lock_guard<std::mutex> lk(g_mu);
  release_cached_locked();
  return WXX_OK;
}

WXX_API int wxx_mem_stats(size_t* live, size_t* cached, size_t* peak, size_t* n_malloc) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (live) *live = g_bytes_live;
  if (cached) *cached = g_bytes_cached;
  if (peak) *peak = g_bytes_peak;
  if (n_malloc) *n_malloc = g_n_malloc;
  return WXX_OK;
}

WXX_API int wxx_h2d(void* dst, const void* src, size_t bytes) {
  WXX_CHECK_INIT();
  if (bytes == 0) return WXX_OK;
  WXX_REQUIRE(dst && src, "null pointer in wxx_h2d");
  if (bytes <= kStageSlot) {
    int s = g_stage_next;
    g_stage_next = (g_stage_next + 1) % kStageSlots;
    if (g_stage_used[s]) WXX_HIP(hipEventSynchronize(g_stage_ev[s]));
    char* stage = g_stage + size_t(s) * kStageSlot;
    memcpy(stage, src, bytes);
    WXX_HIP(hipMemcpyAsync(dst, stage, bytes, hipMemcpyHostToDevice, g_stream));
    WXX_HIP(hipEventRecord(g_stage_ev[s], g_stream));
    g_stage_used[s] = true;
    return WXX_OK;
  }
  WXX_HIP(hipStreamSynchronize(g_stream));
  WXX_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return WXX_OK;
}

WXX_API int wxx_d2h(void* dst, const void* src, size_t bytes) {
  WXX_CHECK_INIT();
  if (bytes == 0) return WXX_OK;
  WXX_REQUIRE(dst && src, "null pointer in wxx_d2h");
  WXX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
  WXX_HIP(hipStreamSynchronize(g_stream));
  return WXX_OK;
}

WXX_API int wxx_d2d(void* dst, const void* src, size_t bytes) {
  WXX_CHECK_INIT();
  if (bytes == 0) return WXX_OK;
  WXX_REQUIRE(dst && src, "null pointer in wxx_d2d");
  WXX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
  return WXX_OK;
}

// Fill `n` 32-bit words with `bits` using a kernel (never a memset node, so a
// caller capturing the stream into a graph gets a replay-safe fill).
WXX_API int wxx_fill_u32(void* dst, int64_t n, uint32_t bits) {
  WXX_CHECK_INIT();
  if (n <= 0) return WXX_OK;
  WXX_REQUIRE(dst, "null pointer in wxx_fill_u32");
  hipLaunchKernelGGL(fill_u32_kernel, dim3(wxx::grid_1d(n, 256, 65536)), dim3(256), 0,
                     g_stream, (uint32_t*)dst, n, bits);
  WXX_LAUNCHED();
  return WXX_OK;
}

WXX_API int wxx_sync() {
  WXX_CHECK_INIT();
  WXX_HIP(hipStreamSynchronize(g_stream));
  return WXX_OK;
}

WXX_API void* wxx_stream() { return (void*)g_stream; }

WXX_API int wxx_timer_record(int slot) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(slot >= 0 && slot < kTimers, "timer slot %d out of range", slot);
  WXX_HIP(hipEventRecord(g_timer[slot], g_stream));
  return WXX_OK;
}

WXX_API int wxx_timer_elapsed(int start, int stop, float* ms) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(start >= 0 && start < kTimers && stop >= 0 && stop < kTimers && ms,
              "bad timer arguments");
  WXX_HIP(hipEventSynchronize(g_timer[stop]));
  WXX_HIP(hipEventElapsedTime(ms, g_timer[start], g_timer[stop]));
  return WXX_OK;
}
