// CPU emulation of the subset of HIP used by wxx_amd/csrc/*.hip.
//
// TEST INFRASTRUCTURE ONLY: it lets the unchanged kernel sources build as
// ordinary C++ (clang++ -fsanitize=address) so that every global-memory
// access of every kernel is bounds-checked on the CPU before a kernel ever
// runs on a GPU.  It is never used by the product library.
//
// Execution model: a launch runs its workgroups one after another; each
// workgroup runs blockDim OS threads.  __syncthreads is a barrier over the
// workgroup's live threads, __shfl_xor / MFMA exchange through a per-wave
// slot array guarded by a barrier over the wave's live lanes.  A thread that
// returns early leaves both barriers (the GPU equivalent: an exited wave no
// longer counts for s_barrier).  __shared__ becomes static storage, which is
// safe because workgroups do not overlap in time.
#pragma once
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>
#include <algorithm>
#include <chrono>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define WXX_WAVES_PER_EU(n)
#define __shared__ static
#define __align__(n) __attribute__((aligned(n)))
#define HIP_SYMBOL(x) ((const void*)&(x))

using std::max;
using std::min;

struct dim3 {
  unsigned x, y, z;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct uint3_t { unsigned x, y, z; };

struct float4 { float x, y, z, w; };
inline float4 make_float4(float a, float b, float c, float d) { return float4{a, b, c, d}; }
struct float2 { float x, y; };
inline float2 make_float2(float a, float b) { return float2{a, b}; }

namespace wxx_emu {
extern thread_local uint3_t tl_thread, tl_block;
extern dim3 g_block_dim, g_grid_dim;

struct Barrier {
  std::mutex mu;
  std::condition_variable cv;
  int expected = 0, arrived = 0;
  unsigned long gen = 0;
  void reset(int n) { std::lock_guard<std::mutex> l(mu); expected = n; arrived = 0; }
  void wait() {
    std::unique_lock<std::mutex> l(mu);
    const unsigned long g = gen;
    if (++arrived >= expected) { arrived = 0; ++gen; cv.notify_all(); return; }
    cv.wait(l, [&] { return gen != g; });
  }
  void leave() {
    std::lock_guard<std::mutex> l(mu);
    --expected;
    if (arrived >= expected && expected >= 0 && arrived > 0) { arrived = 0; ++gen; cv.notify_all(); }
  }
};

struct Launch {
  Barrier block;
  Barrier wave[16];
  uint64_t slot[1024][18];  // per-lane exchange: value + MFMA operands
};
extern Launch* g_launch;

inline int lane() { return (int)(tl_thread.x + g_block_dim.x * (tl_thread.y + g_block_dim.y * tl_thread.z)) & 63; }
inline int flat_tid() { return (int)(tl_thread.x + g_block_dim.x * (tl_thread.y + g_block_dim.y * tl_thread.z)); }
inline int wave_id() { return flat_tid() >> 6; }

void run(const std::function<void()>& body, dim3 grid, dim3 block);
}  // namespace wxx_emu

#define threadIdx (wxx_emu::tl_thread)
#define blockIdx (wxx_emu::tl_block)
#define blockDim (wxx_emu::g_block_dim)
#define gridDim (wxx_emu::g_grid_dim)

inline void __syncthreads() { wxx_emu::g_launch->block.wait(); }

template <typename T>
inline T __shfl_xor(T v, int off, int width = 64) {
  static_assert(sizeof(T) <= 8, "shuffle of a value wider than 8 bytes");
  auto* L = wxx_emu::g_launch;
  const int t = wxx_emu::flat_tid(), w = t >> 6, ln = t & 63;
  uint64_t bits = 0;
  std::memcpy(&bits, &v, sizeof(T));
  L->slot[t][0] = bits;
  L->wave[w].wait();
  const int src = (w << 6) | ((ln ^ off) & (width - 1)) | (ln & ~(width - 1));
  uint64_t got = L->slot[src][0];
  L->wave[w].wait();
  T r;
  std::memcpy(&r, &got, sizeof(T));
  return r;
}

// Wave vote: true on every lane when the predicate holds on any lane.
inline int __any(int pred) {
  auto* L = wxx_emu::g_launch;
  const int t = wxx_emu::flat_tid(), w = t >> 6;
  L->slot[t][0] = pred ? 1 : 0;
  L->wave[w].wait();
  int any = 0;
  for (int i = 0; i < 64; ++i)
    if (((w << 6) | i) < (int)(wxx_emu::g_block_dim.x * wxx_emu::g_block_dim.y * wxx_emu::g_block_dim.z))
      any |= (int)L->slot[(w << 6) | i][0];
  L->wave[w].wait();
  return any;
}

// v_exp_f32
inline float __builtin_amdgcn_exp2f(float x) { return std::exp2(x); }

// Register-allocation hint of the device build; nothing to do on the CPU.
#define WXX_OPAQUE(x) ((void)(x))

// Wave-uniform value: every lane of the emulated wave already holds it.
inline int __builtin_amdgcn_readfirstlane(int v) { return v; }

// global_load_lds: lane L's `size` bytes from src land at lds + offset +
// size * L (lds is wave-uniform).  The copy is done at once, so the wait
// for it is a no-op.
inline void __builtin_amdgcn_global_load_lds(const void* src, void* lds, unsigned size, int offset,
                                             int) {
  std::memcpy(static_cast<char*>(lds) + offset + (size_t)size * wxx_emu::lane(), src, size);
}
inline void __builtin_amdgcn_s_waitcnt(int) {}
// the inline-asm form of a dword global_load_lds (wxx_amd/csrc/common.h)
#define WXX_LDS_DMA_DWORD(src, dst) __builtin_amdgcn_global_load_lds((src), (dst), 4, 0, 0)
#define WXX_LDS_DMA_DWORDX4(src, dst) __builtin_amdgcn_global_load_lds((src), (dst), 16, 0, 0)
#define WXX_S_BARRIER() __syncthreads()

inline float __int_as_float(int v) { float f; std::memcpy(&f, &v, 4); return f; }
inline float __uint_as_float(uint32_t v) { float f; std::memcpy(&f, &v, 4); return f; }
inline int __float_as_int(float f) { int v; std::memcpy(&v, &f, 4); return v; }
inline uint32_t __float_as_uint(float f) { uint32_t v; std::memcpy(&v, &f, 4); return v; }
// Correctly rounded single operations (the host compile does not contract them).
inline float __fmul_rn(float a, float b) { return a * b; }
inline float __fadd_rn(float a, float b) { return a + b; }
inline float rsqrtf(float x) { return 1.0f / std::sqrt(x); }
inline void sincospi(double x, double* s, double* c) {
  *s = std::sin(M_PI * x);
  *c = std::cos(M_PI * x);
}
inline float __expf(float x) { return std::exp(x); }

typedef float wxx_floatx16 __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x2f32: A[i][k] from lane i + 32k, B[k][j] from lane j + 32k,
// D[i][j] in lane j + 32*((i/4)%2), register (i%4) + 4*(i/8).
// Device atomics: blocks run one at a time but their threads run
// concurrently, so these use real host atomics.
template <class T>
inline T atomicAdd(T* p, T v) {
  return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST);
}
inline float atomicAdd(float* p, float v) {
  float old, want;
  __atomic_load(p, &old, __ATOMIC_SEQ_CST);
  do {
    want = old + v;
  } while (!__atomic_compare_exchange(p, &old, &want, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST));
  return old;
}

inline wxx_floatx16 __builtin_amdgcn_mfma_f32_32x32x2f32(float a, float b, wxx_floatx16 c, int, int, int) {
  auto* L = wxx_emu::g_launch;
  const int t = wxx_emu::flat_tid(), w = t >> 6, ln = t & 63;
  uint64_t ab = 0;
  std::memcpy(&ab, &a, 4);
  std::memcpy(reinterpret_cast<char*>(&ab) + 4, &b, 4);
  L->slot[t][1] = ab;
  L->wave[w].wait();
  wxx_floatx16 d = c;
  const int j = ln & 31;
  for (int r = 0; r < 16; ++r) {
    const int i = 8 * (r / 4) + 4 * (ln / 32) + (r % 4);
    float acc = 0.f;
    for (int k = 0; k < 2; ++k) {
      float av, bv;
      uint64_t sa = L->slot[(w << 6) + i + 32 * k][1], sb = L->slot[(w << 6) + j + 32 * k][1];
      std::memcpy(&av, &sa, 4);
      std::memcpy(&bv, reinterpret_cast<char*>(&sb) + 4, 4);
      acc += av * bv;
    }
    d[r] += acc;
  }
  L->wave[w].wait();
  return d;
}

// ---------------------------------------------------------------- runtime API
typedef int hipError_t;
enum { hipSuccess = 0, hipErrorMemoryAllocation = 2 };
typedef void* hipStream_t;
typedef void* hipEvent_t;
enum hipMemcpyKind { hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice,
                     hipMemcpyHostToHost, hipMemcpyDefault };
#define hipStreamNonBlocking 1
#define hipEventDisableTiming 2
#define hipHostMallocDefault 0
struct hipDeviceProp_t { char name[256]; char gcnArchName[256]; int multiProcessorCount; size_t totalGlobalMem; };

hipError_t hipGetDeviceCount(int* n);
hipError_t hipSetDevice(int d);
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
// a __device__ variable is ordinary host storage here: its address is the symbol's
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) {
  *p = const_cast<void*>(sym);
  return hipSuccess;
}
hipError_t hipGetDeviceProperties(hipDeviceProp_t* p, int d);
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned f);
hipError_t hipStreamSynchronize(hipStream_t s);
hipError_t hipMalloc(void** p, size_t n);
hipError_t hipFree(void* p);
hipError_t hipHostMalloc(void** p, size_t n, unsigned f);
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind k);
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t st);
hipError_t hipEventCreate(hipEvent_t* e);
hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned f);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s);
hipError_t hipEventSynchronize(hipEvent_t e);
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b);
hipError_t hipGetLastError();
// Occupancy query: the emulation runs one workgroup at a time.
template <class F>
inline hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int* n, F, int, size_t) {
  *n = 1;
  return hipSuccess;
}
const char* hipGetErrorString(hipError_t e);

// Stream capture: while a capture is open, launches and copies are stored
// (kernel arguments by value) and a graph launch runs them in order.
typedef void* hipGraph_t;
typedef void* hipGraphExec_t;
typedef void* hipGraphNode_t;
enum hipStreamCaptureMode { hipStreamCaptureModeGlobal, hipStreamCaptureModeThreadLocal,
                            hipStreamCaptureModeRelaxed };
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode m);
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t* g);
hipError_t hipGraphGetNodes(hipGraph_t g, hipGraphNode_t* nodes, size_t* n);
hipError_t hipGraphInstantiate(hipGraphExec_t* e, hipGraph_t g, hipGraphNode_t* err_node,
                               char* log, size_t log_size);
hipError_t hipGraphLaunch(hipGraphExec_t e, hipStream_t s);
hipError_t hipGraphExecDestroy(hipGraphExec_t e);
hipError_t hipGraphDestroy(hipGraph_t g);
hipError_t hipHostFree(void* p);
namespace wxx_emu {
bool capturing();
void record(std::function<void()> op);
template <class F>
inline void launch(F f, dim3 grid, dim3 block) {
  if (capturing())
    record([f, grid, block]() { run(f, grid, block); });
  else
    run(f, grid, block);
}
}  // namespace wxx_emu

#define hipLaunchKernelGGL(KERNEL, GRID, BLOCK, SHMEM, STREAM, ...) \
  wxx_emu::launch([=]() { KERNEL(__VA_ARGS__); }, dim3(GRID), dim3(BLOCK))
