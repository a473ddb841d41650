// Shared definitions for the gfx950 kernels of libwxx_hip.so.
//
// Every extern "C" entry point returns 0 on success or a negative WXX_E_*
// code; the message of the last failure is kept per host thread and read
// back with wxx_last_error().  All work is enqueued on the one in-order
// stream owned by the runtime (runtime.hip), which gives the same ordering
// guarantees as the reference's single shared compute pass.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstddef>
#include <cstdio>
#include <cstdarg>
#include <algorithm>

#define WXX_API extern "C" __attribute__((visibility("default")))

// Make a per-lane integer opaque to the optimiser (an empty asm that "may
// change" it), e.g. to stop loop-invariant code motion from hoisting and
// keeping alive every address derived from it.
#ifndef WXX_OPAQUE
#define WXX_OPAQUE(x) asm volatile("" : "+v"(x))
#endif

// A bare workgroup barrier (s_barrier) that is only a compiler memory
// clobber, not a memory fence: __syncthreads() also waits for every
// outstanding global load (vmcnt(0)), which would drain a pipeline of loads
// that a kernel keeps in flight across the barrier on purpose.
#ifndef WXX_S_BARRIER
#define WXX_S_BARRIER() asm volatile("s_barrier" ::: "memory")
#endif

// Occupancy hint: at least n waves per SIMD (the register allocator keeps
// within the matching VGPR budget).
#ifndef WXX_WAVES_PER_EU
#define WXX_WAVES_PER_EU(n) __attribute__((amdgpu_waves_per_eu(n)))
#endif

// One global_load_lds_dword: every lane's 4 bytes at `src` (any address)
// land at the wave-uniform LDS address `lds_dst` + 4 * lane.  Written as
// inline asm so that the compiler does not track it as an LDS store: a
// kernel that keeps several chunks of these in flight waits for them itself
// (s_waitcnt vmcnt, which counts them in issue order) instead of getting the
// full vmcnt(0) the compiler inserts before any LDS read it cannot prove
// disjoint.  M0 carries the LDS address; the kernels that use this helper
// have no other M0 user.
#ifndef WXX_LDS_DMA_DWORD
#define WXX_LDS_DMA_DWORD wxx_lds_dma_dword
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved; see above
__device__ __forceinline__ void wxx_lds_dma_dword(const float* src, float* lds_dst) {
  const unsigned lds = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(__attribute__((address_space(3))) float*)lds_dst);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop
#endif

// The same for global_load_lds_dwordx4: every lane's 16 bytes at `src` land
// at `lds_dst` + 16 * lane.
#ifndef WXX_LDS_DMA_DWORDX4
#define WXX_LDS_DMA_DWORDX4 wxx_lds_dma_dwordx4
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved; see above
__device__ __forceinline__ void wxx_lds_dma_dwordx4(const float* src, float* lds_dst) {
  const unsigned lds = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(__attribute__((address_space(3))) float*)lds_dst);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop
#endif

WXX_API int wxx_fill_u32(void* dst, int64_t n, uint32_t bits);
WXX_API int wxx_h2d(void* dst, const void* src, size_t bytes);
WXX_API void* wxx_alloc(size_t bytes);
WXX_API int wxx_free(void* ptr);

enum {
  WXX_OK = 0,
  WXX_E_HIP = -1,        // a HIP runtime call failed
  WXX_E_ARG = -2,        // invalid argument (null pointer, bad enum, bad size)
  WXX_E_OOM = -3,        // device allocation failed
  WXX_E_INIT = -4,       // runtime not initialised / no device
  WXX_E_RANGE = -5,      // index data out of range (e.g. CCE target >= K)
  WXX_E_UNSUPPORTED = -6, // shape/layout outside what a kernel supports
  WXX_E_CAPTURE = -7      // not allowed while a step graph is being captured
};

namespace wxx {

// Runtime state (runtime.hip).
hipStream_t stream();
bool initialised();
int set_error(int code, const char* fmt, ...);
bool capturing();                    // a step graph is being captured
void* scratch_alloc(size_t bytes);   // stream-ordered temporary from the cache
void scratch_free(void* p);
int num_cus();
// Real FFT and its inverse for n = 2^(logm + 1) above one workgroup's LDS
// (fft_big.hip): four-step transforms over global scratch.
int rfft_four_step(const float* x, float2* X, int64_t rows, int64_t in_len, int logm);
int irfft_four_step(const float2* X, float* x, int64_t rows, int64_t in_len, int logm,
                    int64_t out_len, float post);
// Looks up the device address of the allocation-free GEMM's scratch array on
// `device` (which must be current); called once per device by wxx_init.
int gemm_noalloc_setup(int device);

constexpr int kMaxRank = 6;

struct Shape6 {
  int64_t d[kMaxRank];
};

}  // namespace wxx

#define WXX_CHECK_INIT()                                                   \
  do {                                                                     \
    if (!wxx::initialised())                                               \
      return wxx::set_error(WXX_E_INIT, "wxx_init() has not been called"); \
  } while (0)

#define WXX_HIP(call)                                                      \
  do {                                                                     \
    hipError_t e_ = (call);                                                \
    if (e_ != hipSuccess)                                                  \
      return wxx::set_error(WXX_E_HIP, "%s failed: %s", #call,             \
                            hipGetErrorString(e_));                        \
  } while (0)

#define WXX_REQUIRE(cond, ...)                                             \
  do {                                                                     \
    if (!(cond)) return wxx::set_error(WXX_E_ARG, __VA_ARGS__);            \
  } while (0)

// Check the launch that was just enqueued.
#define WXX_LAUNCHED()                                                     \
  do {                                                                     \
    hipError_t e_ = hipGetLastError();                                     \
    if (e_ != hipSuccess)                                                  \
      return wxx::set_error(WXX_E_HIP, "kernel launch failed: %s",         \
                            hipGetErrorString(e_));                        \
  } while (0)

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
namespace wxx {

__device__ __forceinline__ float warp_sum(float v) {
  // 64-wide wavefront butterfly; __shfl_xor lowers to ds_swizzle/DPP moves.
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float warp_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Block-wide sum of one value per thread; every thread gets the result.
// `red` must hold at least blockDim.x / 64 floats.
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  v = warp_sum(v);
  __syncthreads();  // protect `red` from a previous use
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  v = warp_max(v);
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = red[0];
  for (int i = 1; i < nw; ++i) t = fmaxf(t, red[i]);
  return t;
}

// Dropout's keep decision for element `idx` (its flat index, truncated to 32
// bits) under `seed` (reference shaders/layers/dropout.wgsl:14-36): with
// h(x) = ((x>>16)^x)*0x45d9f3b twice then (x>>16)^x, the element is kept when
// f32(h(idx ^ seed) >> 8) * 2^-24 >= p.
__device__ __forceinline__ uint32_t drop_hash(uint32_t x) {
  x = ((x >> 16) ^ x) * 0x45d9f3bu;
  x = ((x >> 16) ^ x) * 0x45d9f3bu;
  x = (x >> 16) ^ x;
  return x;
}

__device__ __forceinline__ bool dropout_keep(uint32_t idx, uint32_t seed, float p) {
  return (float)(drop_hash(idx ^ seed) >> 8) * (1.0f / 16777216.0f) >= p;
}

inline unsigned int grid_1d(int64_t n, int block, int64_t cap = 1 << 20) {
  int64_t g = (n + block - 1) / block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned int)g;
}

}  // namespace wxx
