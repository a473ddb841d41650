// Reductions over an (outer, reduce, inner) view of a contiguous f32 tensor:
// sum / mean / sum-of-squares, max / min with u32 argument, and the
// max/min backward scatter.
//
// Reference semantics (src/wxx/shaders/helpers/reduce.wgsl:15-66,
// reduce_minmax.wgsl:24-72, maxmin_backward.wgsl:15-38; host side
// src/wxx/functional/reductions.py:27-306):
//  * mean divides the fp32 sum by f32(reduce);
//  * max/min start from -1e38 / +1e38 with index 0, replace only on a
//    strictly better value, and resolve ties the way the reference's
//    256-lane strided scan + halving tree does.  That tree keeps the lower
//    slot unless the upper one is strictly better, so among positions that
//    reach the best value the winner minimises
//        (bitrev8(r mod 256), r div 256)
//    lexicographically.  We encode that order in a 64-bit key and reduce
//    (value, key) pairs with an associative comparator, so any launch shape
//    returns the reference's index bit-exactly.
//
// MI355X design: the reference uses one 256-thread workgroup per output and
// a 65 535-workgroup cap.  Here a row reduction (inner == 1) gives each
// (row, split) pair to one 64-lane wave with float4 loads and a DPP/shuffle
// reduction; column reductions (inner > 1) give each thread one output
// column so consecutive lanes read consecutive addresses.  When there are
// too few outputs to fill 256 CUs the reduce axis is split and a second,
// deterministic pass adds the partials in split order (no float atomics).
#include "common.h"

namespace {

using wxx::warp_sum;

constexpr int kBlock = 256;

template <int MODE>
__device__ __forceinline__ float red_term(float v) {
  return MODE == 2 ? v * v : v;
}

// --- rows: inner == 1 ------------------------------------------------------
// One wave per (row, split).  Partial sums go to part[row * splits + split],
// or straight to out[row] (scaled) when splits == 1.
template <int MODE, bool VEC>
__global__ __launch_bounds__(kBlock) void reduce_rows_kernel(
    const float* __restrict__ x, float* __restrict__ dst, int64_t outer, int64_t R,
    int splits, int64_t seg, float scale, int final_write) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = ((int64_t)blockIdx.x * kBlock + threadIdx.x) >> 6;
  const int64_t total = outer * splits;
  if (wave >= total) return;
  const int64_t row = wave / splits;
  const int split = (int)(wave - row * splits);
  const int64_t r0 = (int64_t)split * seg;
  int64_t r1 = r0 + seg;
  if (r1 > R) r1 = R;
  const float* p = x + row * R;
  float acc = 0.f;
  if (VEC) {
    // r0 and R are multiples of 4 here (checked on the host).
    const float4* p4 = reinterpret_cast<const float4*>(p + r0);
    const int64_t n4 = (r1 - r0) >> 2;
    for (int64_t i = lane; i < n4; i += 64) {
      float4 v = p4[i];
      acc += red_term<MODE>(v.x) + red_term<MODE>(v.y) + red_term<MODE>(v.z) +
             red_term<MODE>(v.w);
    }
  } else {
    for (int64_t r = r0 + lane; r < r1; r += 64) acc += red_term<MODE>(p[r]);
  }
  acc = warp_sum(acc);
  if (lane == 0) {
    if (final_write)
      dst[row] = acc * scale;
    else
      dst[wave] = acc;
  }
}

// --- columns: inner > 1 ----------------------------------------------------
// Thread per (outer, inner) output and split of the reduce axis.
template <int MODE>
__global__ __launch_bounds__(kBlock) void reduce_cols_kernel(
    const float* __restrict__ x, float* __restrict__ dst, int64_t outer, int64_t R,
    int64_t inner, int splits, int64_t seg, float scale, int final_write) {
  const int64_t nout = outer * inner;
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int split = blockIdx.y;
  if (t >= nout) return;
  const int64_t o = t / inner;
  const int64_t i = t - o * inner;
  const int64_t r0 = (int64_t)split * seg;
  int64_t r1 = r0 + seg;
  if (r1 > R) r1 = R;
  const float* p = x + o * R * inner + i;
  float acc = 0.f;
  int64_t r = r0;
  // Four independent accumulators keep several loads in flight.
  float a1 = 0.f, a2 = 0.f, a3 = 0.f;
  for (; r + 3 < r1; r += 4) {
    acc += red_term<MODE>(p[r * inner]);
    a1 += red_term<MODE>(p[(r + 1) * inner]);
    a2 += red_term<MODE>(p[(r + 2) * inner]);
    a3 += red_term<MODE>(p[(r + 3) * inner]);
  }
  for (; r < r1; ++r) acc += red_term<MODE>(p[r * inner]);
  acc = (acc + a1) + (a2 + a3);
  if (final_write)
    dst[t] = acc * scale;
  else
    dst[(int64_t)split * nout + t] = acc;
}

// Sum `splits` partials per output in a fixed order (deterministic).
// layout 0: part[out * splits + s], one thread per output;
// layout 1: part[s * nout + out], 64 outputs per workgroup: lane c of wave w
// adds splits w, w + 4, ... (consecutive lanes read consecutive outputs) and
// the four wave sums are added in wave order.
__global__ __launch_bounds__(kBlock) void reduce_finalize_kernel(
    const float* __restrict__ part, float* __restrict__ out, int64_t nout, int splits,
    int layout, float scale) {
  if (layout == 0) {
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= nout) return;
    float acc = 0.f;
    const float* p = part + t * splits;
    for (int s = 0; s < splits; ++s) acc += p[s];
    out[t] = acc * scale;
    return;
  }
  __shared__ float sw[4][64];
  const int c = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * 64 + c;
  float acc = 0.f;
  if (t < nout)
    for (int s = w; s < splits; s += 4) acc += part[(int64_t)s * nout + t];
  sw[w][c] = acc;
  __syncthreads();
  if (w == 0 && t < nout) out[t] = (((sw[0][c] + sw[1][c]) + sw[2][c]) + sw[3][c]) * scale;
}

// --- max / min with argument -------------------------------------------------
__device__ __forceinline__ uint32_t bitrev8(uint32_t v) {
  return __builtin_bitreverse32(v) >> 24;
}

// key 0 is reserved for the initial (-1e38 / +1e38, index 0) candidate so
// that a value equal to the initial one never displaces it (strict compare).
__device__ __forceinline__ uint64_t arg_key(int64_t r) {
  return ((((uint64_t)bitrev8((uint32_t)(r & 255))) << 40) | (uint64_t)(r >> 8)) + 1;
}

template <int OP>  // 0 = max, 1 = min
__device__ __forceinline__ bool better(float v, uint64_t k, float bv, uint64_t bk) {
  if (OP == 0) {
    if (v > bv) return true;
  } else {
    if (v < bv) return true;
  }
  return v == bv && k < bk;
}

template <int OP>
__device__ __forceinline__ void wave_arg_reduce(float& v, uint64_t& k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    float ov = __shfl_xor(v, off, 64);
    uint32_t klo = __shfl_xor((uint32_t)k, off, 64);
    uint32_t khi = __shfl_xor((uint32_t)(k >> 32), off, 64);
    uint64_t ok = ((uint64_t)khi << 32) | klo;
    if (better<OP>(ov, ok, v, k)) {
      v = ov;
      k = ok;
    }
  }
}

__device__ __forceinline__ uint32_t key_to_index(uint64_t k) {
  if (k == 0) return 0u;
  k -= 1;
  uint32_t t = bitrev8((uint32_t)(k >> 40));
  uint64_t hi = k & ((uint64_t(1) << 40) - 1);
  return (uint32_t)((hi << 8) | t);
}

// One wave per output; lanes stride the reduce axis.
template <int OP>
__global__ __launch_bounds__(kBlock) void minmax_kernel(
    const float* __restrict__ x, float* __restrict__ vals, uint32_t* __restrict__ idx,
    int64_t outer, int64_t R, int64_t inner) {
  const int lane = threadIdx.x & 63;
  const int64_t w = ((int64_t)blockIdx.x * kBlock + threadIdx.x) >> 6;
  const int64_t nout = outer * inner;
  if (w >= nout) return;
  const int64_t o = w / inner;
  const int64_t i = w - o * inner;
  const float* p = x + o * R * inner + i;
  float bv = OP == 0 ? -1e38f : 1e38f;
  uint64_t bk = 0;
  for (int64_t r = lane; r < R; r += 64) {
    float v = p[r * inner];
    uint64_t k = arg_key(r);
    if (better<OP>(v, k, bv, bk)) {
      bv = v;
      bk = k;
    }
  }
  wave_arg_reduce<OP>(bv, bk);
  if (lane == 0) {
    vals[w] = bv;
    idx[w] = key_to_index(bk);
  }
}

__global__ __launch_bounds__(kBlock) void maxmin_backward_kernel(
    const float* __restrict__ g, const uint32_t* __restrict__ ind, float* __restrict__ out,
    int64_t R, int64_t inner, int64_t numel) {
  int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (; t < numel; t += stride) {
    const int64_t o = t / (R * inner);
    const int64_t rem = t - o * R * inner;
    const int64_t r = rem / inner;
    const int64_t i = rem - r * inner;
    const int64_t oi = o * inner + i;
    out[t] = ((int64_t)ind[oi] == r) ? g[oi] : 0.f;
  }
}

template <int MODE>
int launch_reduce(const float* x, float* out, int64_t outer, int64_t R, int64_t inner) {
  hipStream_t s = wxx::stream();
  const float scale = MODE == 1 ? 1.0f / (float)R : 1.0f;
  const int64_t nout = outer * inner;
  const int64_t target = (int64_t)wxx::num_cus() * 16;  // waves (rows) or blocks (cols)
  if (inner == 1) {
    int splits = 1;
    if (outer < target) {
      int64_t want = (target + outer - 1) / outer;
      int64_t max_by_len = (R + 4095) / 4096;  // >= 4096 elements per split
      splits = (int)std::max<int64_t>(1, std::min(want, max_by_len));
    }
    int64_t seg = (R + splits - 1) / splits;
    seg = (seg + 3) & ~int64_t(3);
    const bool vec = (R % 4 == 0) && ((uintptr_t)x % 16 == 0);
    float* dst = out;
    float* part = nullptr;
    if (splits > 1) {
      part = (float*)wxx::scratch_alloc(sizeof(float) * outer * splits);
      if (!part) return wxx::set_error(WXX_E_OOM, "reduce partials");
      dst = part;
    }
    const int64_t waves = outer * splits;
    dim3 grid((unsigned)((waves * 64 + kBlock - 1) / kBlock));
    if (vec)
      hipLaunchKernelGGL((reduce_rows_kernel<MODE, true>), grid, dim3(kBlock), 0, s, x, dst,
                         outer, R, splits, seg, scale, splits == 1);
    else
      hipLaunchKernelGGL((reduce_rows_kernel<MODE, false>), grid, dim3(kBlock), 0, s, x, dst,
                         outer, R, splits, seg, scale, splits == 1);
    WXX_LAUNCHED();
    if (splits > 1) {
      hipLaunchKernelGGL(reduce_finalize_kernel, dim3(wxx::grid_1d(nout, kBlock)), dim3(kBlock),
                         0, s, part, out, nout, splits, 0, scale);
      WXX_LAUNCHED();
      wxx::scratch_free(part);
    }
    return WXX_OK;
  }
  const int64_t blocks = (nout + kBlock - 1) / kBlock;
  int splits = 1;
  if (blocks < target) {
    int64_t want = (target + blocks - 1) / blocks;
    int64_t max_by_len = (R + 63) / 64;
    splits = (int)std::max<int64_t>(1, std::min<int64_t>(std::min(want, max_by_len), 1024));
  }
  int64_t seg = (R + splits - 1) / splits;
  float* dst = out;
  float* part = nullptr;
  if (splits > 1) {
    part = (float*)wxx::scratch_alloc(sizeof(float) * nout * splits);
    if (!part) return wxx::set_error(WXX_E_OOM, "reduce partials");
    dst = part;
  }
  hipLaunchKernelGGL((reduce_cols_kernel<MODE>), dim3((unsigned)blocks, splits), dim3(kBlock), 0,
                     s, x, dst, outer, R, inner, splits, seg, scale, splits == 1);
  WXX_LAUNCHED();
  if (splits > 1) {
    hipLaunchKernelGGL(reduce_finalize_kernel, dim3((unsigned)((nout + 63) / 64)), dim3(kBlock),
                       0, s, part, out, nout, splits, 1, scale);
    WXX_LAUNCHED();
    wxx::scratch_free(part);
  }
  return WXX_OK;
}

}  // namespace

// mode: 0 = sum, 1 = mean, 2 = sum of squares.
// Replaces functional.sum / mean / sumsq (reference
// src/wxx/functional/reductions.py:27-197).
WXX_API int wxx_reduce(const float* x, float* out, int64_t outer, int64_t reduce,
                       int64_t inner, int mode) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(outer >= 0 && reduce >= 1 && inner >= 1, "bad reduce dims");
  WXX_REQUIRE(x && out, "null pointer");
  if (outer == 0) return WXX_OK;
  switch (mode) {
    case 0: return launch_reduce<0>(x, out, outer, reduce, inner);
    case 1: return launch_reduce<1>(x, out, outer, reduce, inner);
    case 2: return launch_reduce<2>(x, out, outer, reduce, inner);
    default: return wxx::set_error(WXX_E_ARG, "bad reduce mode %d", mode);
  }
}

// op: 0 = max, 1 = min.  Replaces functional.max / min (reference
// src/wxx/functional/reductions.py:241-312).
WXX_API int wxx_reduce_minmax(const float* x, float* vals, uint32_t* idx, int64_t outer,
                              int64_t reduce, int64_t inner, int op) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && vals && idx, "null pointer");
  WXX_REQUIRE(outer >= 0 && reduce >= 1 && inner >= 1, "bad reduce dims");
  WXX_REQUIRE(reduce < (int64_t(1) << 32), "reduce axis too long for u32 indices");
  const int64_t nout = outer * inner;
  if (nout == 0) return WXX_OK;
  dim3 grid((unsigned)((nout * 64 + kBlock - 1) / kBlock));
  if (op == 0)
    hipLaunchKernelGGL(minmax_kernel<0>, grid, dim3(kBlock), 0, wxx::stream(), x, vals, idx,
                       outer, reduce, inner);
  else if (op == 1)
    hipLaunchKernelGGL(minmax_kernel<1>, grid, dim3(kBlock), 0, wxx::stream(), x, vals, idx,
                       outer, reduce, inner);
  else
    return wxx::set_error(WXX_E_ARG, "bad minmax op %d", op);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.maxmin_backward (reference
// src/wxx/functional/reductions.py:200-237).
WXX_API int wxx_maxmin_backward(const float* g, const uint32_t* idx, float* out, int64_t outer,
                                int64_t reduce, int64_t inner) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(g && idx && out, "null pointer");
  const int64_t numel = outer * reduce * inner;
  if (numel == 0) return WXX_OK;
  hipLaunchKernelGGL(maxmin_backward_kernel, dim3(wxx::grid_1d(numel, kBlock, 65536)),
                     dim3(kBlock), 0, wxx::stream(), g, idx, out, reduce, inner, numel);
  WXX_LAUNCHED();
  return WXX_OK;
}
