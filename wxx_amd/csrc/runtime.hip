// Device runtime of libwxx_hip.so: device selection, the single in-order
// stream, a size-bucketed caching allocator, host<->device copies, fills,
// synchronisation, error reporting, event timers and step graphs (one call
// of a host step function recorded from the stream and replayed with one
// hipGraphLaunch).
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

#include <algorithm>
#include <iterator>
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
using FreeLists = std::unordered_map<size_t, std::vector<void*>>;  // rounded size -> blocks
FreeLists g_free;
std::unordered_map<void*, size_t> g_live;  // block -> rounded size
size_t g_bytes_live = 0, g_bytes_cached = 0, g_bytes_peak = 0;
size_t g_n_malloc = 0;

// A captured step.  Every block the capture allocates belongs to the graph's
// own pool for the graph's lifetime: a replay writes those addresses again,
// so eager work must never be handed one of them.  Blocks the capture frees
// go back to that pool (later captured work may reuse them, in stream order);
// blocks still held by host objects after the capture return to it when
// freed.  Uploads made while capturing are copied into pinned arenas the
// graph owns, so each replay copies the bytes the capture saw.
struct Graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  FreeLists pool;
  std::vector<char*> arenas;
  size_t arena_cap = 0, arena_used = 0;
  int64_t nodes = 0;
};
std::unordered_map<void*, Graph*> g_owner;  // graph-owned block -> graph
Graph* g_capture = nullptr;                 // the graph being captured, if any
constexpr size_t kArenaChunk = size_t(4) << 20;

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

bool capturing() { return g_capture != nullptr; }

void* scratch_alloc(size_t bytes) {
  size_t r = round_size(bytes);
  std::lock_guard<std::mutex> lk(g_mu);
  void* p = nullptr;
  if (g_capture) {
    auto own = g_capture->pool.find(r);
    if (own != g_capture->pool.end() && !own->second.empty()) {
      p = own->second.back();
      own->second.pop_back();
    }
  }
  auto it = g_free.find(r);
  if (p) {
  } else if (it != g_free.end() && !it->second.empty()) {
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
  if (g_capture) g_owner[p] = g_capture;
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
  auto own = g_owner.find(p);
  if (own != g_owner.end()) {
    own->second->pool[r].push_back(p);
    return;
  }
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

#define WXX_NOT_CAPTURING(what)                                                      \
  do {                                                                               \
    if (g_capture)                                                                   \
      return wxx::set_error(WXX_E_CAPTURE, "%s is not allowed while a graph is being " \
                            "captured (it would wait for the device)", what);         \
  } while (0)

WXX_API int wxx_empty_cache() {
  WXX_CHECK_INIT();
  WXX_NOT_CAPTURING("wxx_empty_cache");
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

// An upload recorded into the graph being captured: the bytes are kept in a
// pinned arena of the graph, and the captured copy reads them from there on
// every replay.
static int capture_upload(void* dst, const void* src, size_t bytes) {
  Graph* g = g_capture;
  const size_t need = (bytes + 255) & ~size_t(255);
  if (g->arenas.empty() || g->arena_used + need > g->arena_cap) {
    const size_t cap = std::max(kArenaChunk, need);
    char* chunk = nullptr;
    WXX_HIP(hipHostMalloc((void**)&chunk, cap, hipHostMallocDefault));
    g->arenas.push_back(chunk);
    g->arena_cap = cap;
    g->arena_used = 0;
  }
  char* at = g->arenas.back() + g->arena_used;
  g->arena_used += need;
  memcpy(at, src, bytes);
  WXX_HIP(hipMemcpyAsync(dst, at, bytes, hipMemcpyHostToDevice, g_stream));
  return WXX_OK;
}

WXX_API int wxx_h2d(void* dst, const void* src, size_t bytes) {
  WXX_CHECK_INIT();
  if (bytes == 0) return WXX_OK;
  WXX_REQUIRE(dst && src, "null pointer in wxx_h2d");
  if (g_capture) return capture_upload(dst, src, bytes);
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
  WXX_NOT_CAPTURING("a device-to-host read (wxx_d2h)");
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
  WXX_NOT_CAPTURING("wxx_sync");
  WXX_HIP(hipStreamSynchronize(g_stream));
  return WXX_OK;
}

WXX_API void* wxx_stream() { return (void*)g_stream; }

WXX_API int wxx_timer_record(int slot) {
  WXX_CHECK_INIT();
  WXX_NOT_CAPTURING("wxx_timer_record");
  WXX_REQUIRE(slot >= 0 && slot < kTimers, "timer slot %d out of range", slot);
  WXX_HIP(hipEventRecord(g_timer[slot], g_stream));
  return WXX_OK;
}

WXX_API int wxx_timer_elapsed(int start, int stop, float* ms) {
  WXX_CHECK_INIT();
  WXX_NOT_CAPTURING("wxx_timer_elapsed");
  WXX_REQUIRE(start >= 0 && start < kTimers && stop >= 0 && stop < kTimers && ms,
              "bad timer arguments");
  WXX_HIP(hipEventSynchronize(g_timer[stop]));
  WXX_HIP(hipEventElapsedTime(ms, g_timer[start], g_timer[stop]));
  return WXX_OK;
}

// ---------------------------------------------------------------------------
// Step graphs: one call of a host step function recorded from the library's
// stream and replayed with a single launch.
// ---------------------------------------------------------------------------

static void release_graph(Graph* g) {
  {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto& kv : g->pool)
      for (void* p : kv.second) {
        g_owner.erase(p);
        g_free[kv.first].push_back(p);
        g_bytes_cached += kv.first;
      }
    g->pool.clear();
    // Blocks still held by host objects become ordinary cached blocks when freed.
    for (auto it = g_owner.begin(); it != g_owner.end();)
      it = it->second == g ? g_owner.erase(it) : std::next(it);
  }
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  for (char* a : g->arenas) (void)hipHostFree(a);
  delete g;
}

WXX_API int wxx_graph_begin() {
  WXX_CHECK_INIT();
  if (g_capture) return wxx::set_error(WXX_E_CAPTURE, "a graph is already being captured");
  // Work enqueued before the capture must not end up inside it.
  WXX_HIP(hipStreamSynchronize(g_stream));
  Graph* g = new Graph;
  // The first upload arena is allocated before capturing starts.
  char* chunk = nullptr;
  if (hipHostMalloc((void**)&chunk, kArenaChunk, hipHostMallocDefault) != hipSuccess) {
    delete g;
    return wxx::set_error(WXX_E_OOM, "pinned upload arena for a graph");
  }
  g->arenas.push_back(chunk);
  g->arena_cap = kArenaChunk;
  const hipError_t e = hipStreamBeginCapture(g_stream, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) {
    (void)hipHostFree(chunk);
    delete g;
    return wxx::set_error(WXX_E_HIP, "hipStreamBeginCapture failed: %s", hipGetErrorString(e));
  }
  g_capture = g;
  return WXX_OK;
}

WXX_API int wxx_graph_end(void** graph, int64_t* nodes) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(graph, "null graph handle");
  if (!g_capture) return wxx::set_error(WXX_E_CAPTURE, "no graph is being captured");
  Graph* g = g_capture;
  g_capture = nullptr;
  hipError_t e = hipStreamEndCapture(g_stream, &g->graph);
  if (e == hipSuccess) {
    size_t n = 0;
    e = hipGraphGetNodes(g->graph, nullptr, &n);
    g->nodes = (int64_t)n;
  }
  if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    release_graph(g);
    return wxx::set_error(WXX_E_HIP, "graph capture failed: %s", hipGetErrorString(e));
  }
  *graph = g;
  if (nodes) *nodes = g->nodes;
  return WXX_OK;
}

WXX_API int wxx_graph_abort() {
  WXX_CHECK_INIT();
  if (!g_capture) return WXX_OK;
  Graph* g = g_capture;
  g_capture = nullptr;
  (void)hipStreamEndCapture(g_stream, &g->graph);
  (void)hipGetLastError();
  release_graph(g);
  return WXX_OK;
}

WXX_API int wxx_graph_launch(void* graph) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(graph, "null graph handle");
  WXX_NOT_CAPTURING("wxx_graph_launch");
  Graph* g = (Graph*)graph;
  WXX_HIP(hipGraphLaunch(g->exec, g_stream));
  return WXX_OK;
}

WXX_API int wxx_graph_destroy(void* graph) {
  WXX_CHECK_INIT();
  if (!graph) return WXX_OK;
  WXX_NOT_CAPTURING("wxx_graph_destroy");
  // A replay still in flight reads the pool and arenas being released.
  WXX_HIP(hipStreamSynchronize(g_stream));
  release_graph((Graph*)graph);
  return WXX_OK;
}

WXX_API int wxx_graph_capturing(int* on) {
  WXX_REQUIRE(on, "null pointer");
  *on = g_capture != nullptr;
  return WXX_OK;
}
