// Runtime side of the HIP-on-CPU shim (TEST INFRASTRUCTURE ONLY): device
// memory is host heap memory (so AddressSanitizer checks every kernel
// access), streams and events are synchronous.
#include "hip/hip_runtime.h"

namespace wxx_emu {
thread_local uint3_t tl_thread, tl_block;
dim3 g_block_dim, g_grid_dim;
Launch* g_launch = nullptr;

void run(const std::function<void()>& body, dim3 grid, dim3 block) {
  const int nthreads = (int)(block.x * block.y * block.z);
  if (nthreads > 1024 || nthreads <= 0) {
    fprintf(stderr, "emu: bad block size %d\n", nthreads);
    abort();
  }
  static Launch launch;
  g_launch = &launch;
  g_block_dim = block;
  g_grid_dim = grid;
  const long nblocks = (long)grid.x * grid.y * grid.z;
  Barrier done;
  std::vector<std::thread> pool;
  Barrier start;
  start.reset(nthreads + 1);
  Barrier end;
  end.reset(nthreads + 1);
  long cur = -1;
  bool quit = false;
  auto worker = [&](int tid) {
    for (;;) {
      start.wait();
      if (quit) return;
      tl_thread = uint3_t{(unsigned)(tid % block.x), (unsigned)((tid / block.x) % block.y),
                          (unsigned)(tid / (block.x * block.y))};
      tl_block = uint3_t{(unsigned)(cur % grid.x), (unsigned)((cur / grid.x) % grid.y),
                         (unsigned)(cur / ((long)grid.x * grid.y))};
      body();
      // leaving: drop out of the workgroup and wave barriers
      launch.block.leave();
      launch.wave[tid >> 6].leave();
      end.wait();
    }
  };
  for (int t = 0; t < nthreads; ++t) pool.emplace_back(worker, t);
  for (long b = 0; b < nblocks; ++b) {
    cur = b;
    launch.block.reset(nthreads);
    for (int w = 0; w < 16; ++w) launch.wave[w].reset(std::min(64, std::max(0, nthreads - 64 * w)));
    start.wait();
    end.wait();
  }
  quit = true;
  start.wait();
  for (auto& th : pool) th.join();
}
}  // namespace wxx_emu

static float g_fake_clock = 0.f;
hipError_t hipGetDeviceCount(int* n) { *n = 1; return hipSuccess; }
hipError_t hipSetDevice(int) { return hipSuccess; }
hipError_t hipGetDeviceProperties(hipDeviceProp_t* p, int) {
  std::memset(p, 0, sizeof(*p));
  std::snprintf(p->name, 256, "cpu-emulation");
  std::snprintf(p->gcnArchName, 256, "emu");
  p->multiProcessorCount = 256;
  p->totalGlobalMem = size_t(1) << 34;
  return hipSuccess;
}
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned) { *s = (void*)1; return hipSuccess; }
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipMalloc(void** p, size_t n) { *p = std::malloc(n ? n : 1); return *p ? hipSuccess : hipErrorMemoryAllocation; }
hipError_t hipFree(void* p) { std::free(p); return hipSuccess; }
hipError_t hipHostMalloc(void** p, size_t n, unsigned) { *p = std::malloc(n); return hipSuccess; }
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind) { std::memmove(d, s, n); return hipSuccess; }
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t) {
  if (wxx_emu::capturing())
    wxx_emu::record([d, s, n]() { std::memmove(d, s, n); });
  else
    std::memmove(d, s, n);
  return hipSuccess;
}
hipError_t hipHostFree(void* p) { std::free(p); return hipSuccess; }

namespace {
using Ops = std::vector<std::function<void()>>;
Ops* g_capture_ops = nullptr;
}  // namespace
namespace wxx_emu {
bool capturing() { return g_capture_ops != nullptr; }
void record(std::function<void()> op) { g_capture_ops->push_back(std::move(op)); }
}  // namespace wxx_emu
hipError_t hipStreamBeginCapture(hipStream_t, hipStreamCaptureMode) {
  if (g_capture_ops) return 900;  // already capturing
  g_capture_ops = new Ops;
  return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t, hipGraph_t* g) {
  *g = g_capture_ops;
  g_capture_ops = nullptr;
  return hipSuccess;
}
hipError_t hipGraphGetNodes(hipGraph_t g, hipGraphNode_t*, size_t* n) {
  *n = static_cast<Ops*>(g)->size();
  return hipSuccess;
}
hipError_t hipGraphInstantiate(hipGraphExec_t* e, hipGraph_t g, hipGraphNode_t*, char*, size_t) {
  *e = new Ops(*static_cast<Ops*>(g));
  return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t e, hipStream_t) {
  for (auto& op : *static_cast<Ops*>(e)) op();
  return hipSuccess;
}
hipError_t hipGraphExecDestroy(hipGraphExec_t e) { delete static_cast<Ops*>(e); return hipSuccess; }
hipError_t hipGraphDestroy(hipGraph_t g) { delete static_cast<Ops*>(g); return hipSuccess; }
hipError_t hipEventCreate(hipEvent_t* e) { *e = new float(0.f); return hipSuccess; }
hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) { *e = new float(0.f); return hipSuccess; }
hipError_t hipEventRecord(hipEvent_t e, hipStream_t) { *(float*)e = (g_fake_clock += 1.f); return hipSuccess; }
hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b) { *ms = *(float*)b - *(float*)a; return hipSuccess; }
hipError_t hipGetLastError() { return hipSuccess; }
const char* hipGetErrorString(hipError_t) { return "emulated"; }
