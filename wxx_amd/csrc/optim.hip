// Optimizer and gradient-norm kernels.
//
// Reference semantics:
//  * AdamW (src/wxx/shaders/optimizers/adamw.wgsl:35-56, host
//    src/wxx/functional/layers.py:21-68, src/wxx/nn/optimizer.py:59-84):
//      m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g g
//      p = p - lr (m/bc1 / (sqrt(v/bc2) + eps) + wd p)
//    with bc1 = 1 - b1^t, bc2 = 1 - b2^t computed on the host.
//  * clip_grad_norm_ (src/wxx/nn/utils.py:62-103): total = sum over grads of
//    sum(g^2); norm = sqrt(total); if max/(norm+1e-6) < 1 every grad is
//    multiplied by that coefficient.
//
// MI355X design: the reference issues one AdamW launch and one sumsq launch
// (plus an accumulate launch) per parameter tensor — about 150 of each for
// GPT-2 small.  The multi-tensor entry points take the whole parameter list:
// a descriptor table (uploaded through the pinned staging ring) maps each
// 4096-element chunk to its tensor, so one launch updates every parameter
// and one launch (+ one deterministic final pass) reduces every gradient.
#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kChunk = kBlock * 16;  // elements per block in multi-tensor kernels

struct AdamHyper {
  float lr, b1, b2, eps, wd, bc1, bc2;
};

__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v,
                                          const AdamHyper& h) {
  m = h.b1 * m + (1.0f - h.b1) * g;
  v = h.b2 * v + (1.0f - h.b2) * g * g;
  const float mh = m / h.bc1;
  const float vh = v / h.bc2;
  p = p - h.lr * (mh / (sqrtf(vh) + h.eps) + h.wd * p);
}

__global__ __launch_bounds__(kBlock) void adamw_kernel(float* __restrict__ p,
                                                       const float* __restrict__ g,
                                                       float* __restrict__ m,
                                                       float* __restrict__ v, int64_t n,
                                                       AdamHyper h) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    float pp = p[i], mm = m[i], vv = v[i];
    adam_elem(pp, g[i], mm, vv, h);
    p[i] = pp;
    m[i] = mm;
    v[i] = vv;
  }
}

struct TensorDesc {
  float* p;
  const float* g;
  float* m;
  float* v;
  int64_t n;
  int64_t first_block;
};

__device__ __forceinline__ int find_tensor(const TensorDesc* d, int nt, int64_t block) {
  int lo = 0, hi = nt - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (d[mid].first_block <= block)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// `hd`, when set, is a device copy of the hyperparameters that replaces `h`
// (a step graph's replays update it between launches).
__global__ __launch_bounds__(kBlock) void adamw_multi_kernel(const TensorDesc* __restrict__ d,
                                                             int nt, AdamHyper h,
                                                             const AdamHyper* __restrict__ hd) {
  if (hd) h = *hd;
  const int ti = find_tensor(d, nt, blockIdx.x);
  const TensorDesc td = d[ti];
  const int64_t base = (blockIdx.x - td.first_block) * (int64_t)kChunk;
  const int64_t end = min(base + (int64_t)kChunk, td.n);
  const bool vec = ((((uintptr_t)td.p) | ((uintptr_t)td.g) | ((uintptr_t)td.m) |
                     ((uintptr_t)td.v)) & 15) == 0;
  if (vec && end - base == kChunk) {
#pragma unroll
    for (int k = 0; k < kChunk / (4 * kBlock); ++k) {
      const int64_t i = base + ((int64_t)k * kBlock + threadIdx.x) * 4;
      float4 p4 = *reinterpret_cast<float4*>(td.p + i);
      const float4 g4 = *reinterpret_cast<const float4*>(td.g + i);
      float4 m4 = *reinterpret_cast<float4*>(td.m + i);
      float4 v4 = *reinterpret_cast<float4*>(td.v + i);
      adam_elem(p4.x, g4.x, m4.x, v4.x, h);
      adam_elem(p4.y, g4.y, m4.y, v4.y, h);
      adam_elem(p4.z, g4.z, m4.z, v4.z, h);
      adam_elem(p4.w, g4.w, m4.w, v4.w, h);
      *reinterpret_cast<float4*>(td.p + i) = p4;
      *reinterpret_cast<float4*>(td.m + i) = m4;
      *reinterpret_cast<float4*>(td.v + i) = v4;
    }
  } else {
    for (int64_t i = base + threadIdx.x; i < end; i += kBlock) {
      float pp = td.p[i], mm = td.m[i], vv = td.v[i];
      adam_elem(pp, td.g[i], mm, vv, h);
      td.p[i] = pp;
      td.m[i] = mm;
      td.v[i] = vv;
    }
  }
}

// Per-block partial sum of squares; partial index = block id.
__global__ __launch_bounds__(kBlock) void sumsq_multi_kernel(const TensorDesc* __restrict__ d,
                                                             int nt, float* __restrict__ part) {
  __shared__ float red[4];
  const int ti = find_tensor(d, nt, blockIdx.x);
  const TensorDesc td = d[ti];
  const int64_t base = (blockIdx.x - td.first_block) * (int64_t)kChunk;
  const int64_t end = min(base + (int64_t)kChunk, td.n);
  float acc = 0.f;
  for (int64_t i = base + threadIdx.x; i < end; i += kBlock) {
    const float x = td.g[i];
    acc += x * x;
  }
  acc = wxx::block_sum(acc, red);
  if (threadIdx.x == 0) part[blockIdx.x] = acc;
}

// One workgroup adds the partials in a fixed order: deterministic total.
__global__ __launch_bounds__(kBlock) void sum_partials_kernel(const float* __restrict__ part,
                                                              int64_t n, float* __restrict__ out) {
  __shared__ float red[4];
  float acc = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += kBlock) acc += part[i];
  acc = wxx::block_sum(acc, red);
  if (threadIdx.x == 0) out[0] = acc;
}

// The clip coefficient from the device sum of squares, with the host's
// float64 arithmetic: norm = sqrt(s), c = max_norm / (norm + 1e-6), applied
// (rounded to f32) only when c < 1.  Both operations are correctly rounded, so
// the coefficient equals the one the host computes from the same sum.
__device__ __forceinline__ float clip_coef(const float* sumsq, double max_norm, bool* apply) {
  const double norm = sqrt((double)sumsq[0]);
  const double c = max_norm / (norm + 1e-6);
  *apply = c < 1.0;
  return (float)c;
}

__global__ __launch_bounds__(kBlock) void scale_multi_kernel(const TensorDesc* __restrict__ d,
                                                             int nt, float c,
                                                             const float* __restrict__ sumsq,
                                                             double max_norm) {
  if (sumsq) {
    bool apply;
    c = clip_coef(sumsq, max_norm, &apply);
    if (!apply) return;
  }
  const int ti = find_tensor(d, nt, blockIdx.x);
  const TensorDesc td = d[ti];
  const int64_t base = (blockIdx.x - td.first_block) * (int64_t)kChunk;
  const int64_t end = min(base + (int64_t)kChunk, td.n);
  for (int64_t i = base + threadIdx.x; i < end; i += kBlock) td.p[i] *= c;
}

// Build and upload the descriptor table; returns total blocks.
int upload_table(void* const* p, void* const* g, void* const* m, void* const* v,
                 const int64_t* n, int nt, TensorDesc** dev, int64_t* blocks) {
  TensorDesc* host = new TensorDesc[nt];
  int64_t b = 0;
  for (int i = 0; i < nt; ++i) {
    host[i].p = (float*)(p ? p[i] : nullptr);
    host[i].g = (const float*)(g ? g[i] : nullptr);
    host[i].m = (float*)(m ? m[i] : nullptr);
    host[i].v = (float*)(v ? v[i] : nullptr);
    host[i].n = n[i];
    host[i].first_block = b;
    b += (n[i] + kChunk - 1) / kChunk;
  }
  *blocks = b;
  *dev = (TensorDesc*)wxx::scratch_alloc(sizeof(TensorDesc) * nt);
  if (!*dev) {
    delete[] host;
    return wxx::set_error(WXX_E_OOM, "descriptor table");
  }
  const int rc = wxx_h2d(*dev, host, sizeof(TensorDesc) * nt);
  delete[] host;
  return rc;
}

}  // namespace

// Replaces functional.adamw (reference src/wxx/functional/layers.py:21-68).
WXX_API int wxx_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr,
                      float beta1, float beta2, float eps, float weight_decay, float bc1,
                      float bc2) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(p && g && m && v, "null pointer");
  if (n <= 0) return WXX_OK;
  AdamHyper h{lr, beta1, beta2, eps, weight_decay, bc1, bc2};
  hipLaunchKernelGGL(adamw_kernel, dim3(wxx::grid_1d(n, kBlock, 16384)), dim3(kBlock), 0,
                     wxx::stream(), p, g, m, v, n, h);
  WXX_LAUNCHED();
  return WXX_OK;
}

// One launch for a whole parameter list (no reference counterpart: replaces
// the per-parameter loop of AdamW.step, reference src/wxx/nn/optimizer.py:69-84).
// p/g/m/v/n are host arrays of `count` device pointers / element counts.
WXX_API int wxx_adamw_multi(void* const* p, void* const* g, void* const* m, void* const* v,
                            const int64_t* n, int count, float lr, float beta1, float beta2,
                            float eps, float weight_decay, float bc1, float bc2) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(p && g && m && v && n && count >= 0, "null pointer");
  if (count == 0) return WXX_OK;
  TensorDesc* d = nullptr;
  int64_t blocks = 0;
  int rc = upload_table(p, g, m, v, n, count, &d, &blocks);
  if (rc) return rc;
  AdamHyper h{lr, beta1, beta2, eps, weight_decay, bc1, bc2};
  if (blocks > 0)
    hipLaunchKernelGGL(adamw_multi_kernel, dim3((unsigned)blocks), dim3(kBlock), 0,
                       wxx::stream(), d, count, h, (const AdamHyper*)nullptr);
  wxx::scratch_free(d);
  WXX_LAUNCHED();
  return WXX_OK;
}

// wxx_adamw_multi with the hyperparameters read on the device from `hyper`
// (7 floats: lr, beta1, beta2, eps, weight_decay, bc1, bc2) when the kernel
// runs, so a recorded step graph picks up each step's learning rate and bias
// corrections.  No reference counterpart (the reference has no graphs).
WXX_API int wxx_adamw_multi_dev(void* const* p, void* const* g, void* const* m, void* const* v,
                                const int64_t* n, int count, const float* hyper) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(p && g && m && v && n && hyper && count >= 0, "null pointer");
  if (count == 0) return WXX_OK;
  TensorDesc* d = nullptr;
  int64_t blocks = 0;
  int rc = upload_table(p, g, m, v, n, count, &d, &blocks);
  if (rc) return rc;
  AdamHyper h{};
  if (blocks > 0)
    hipLaunchKernelGGL(adamw_multi_kernel, dim3((unsigned)blocks), dim3(kBlock), 0,
                       wxx::stream(), d, count, h, (const AdamHyper*)hyper);
  wxx::scratch_free(d);
  WXX_LAUNCHED();
  return WXX_OK;
}

// out[0] = sum over the `count` tensors of sum(x^2) (device scalar).  Replaces
// the sumsq + accumulate loop of clip_grad_norm_ (reference src/wxx/nn/utils.py:82-93).
WXX_API int wxx_sumsq_multi(void* const* x, const int64_t* n, int count, float* out) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && n && out && count >= 0, "null pointer");
  if (count == 0) return wxx_fill_u32(out, 1, 0u);
  TensorDesc* d = nullptr;
  int64_t blocks = 0;
  int rc = upload_table(nullptr, x, nullptr, nullptr, n, count, &d, &blocks);
  if (rc) return rc;
  float* part = (float*)wxx::scratch_alloc(sizeof(float) * std::max<int64_t>(1, blocks));
  if (!part) {
    wxx::scratch_free(d);
    return wxx::set_error(WXX_E_OOM, "sumsq partials");
  }
  hipStream_t s = wxx::stream();
  if (blocks > 0)
    hipLaunchKernelGGL(sumsq_multi_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, s, d, count,
                       part);
  hipLaunchKernelGGL(sum_partials_kernel, dim3(1), dim3(kBlock), 0, s, part, blocks, out);
  wxx::scratch_free(part);
  wxx::scratch_free(d);
  WXX_LAUNCHED();
  return WXX_OK;
}

// x_i *= c for every tensor (the rescale of clip_grad_norm_, reference
// src/wxx/nn/utils.py:97-101).  The caller passes each storage once.
WXX_API int wxx_scale_multi(void* const* x, const int64_t* n, int count, float c) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && n && count >= 0, "null pointer");
  if (count == 0) return WXX_OK;
  TensorDesc* d = nullptr;
  int64_t blocks = 0;
  int rc = upload_table(x, nullptr, nullptr, nullptr, n, count, &d, &blocks);
  if (rc) return rc;
  if (blocks > 0)
    hipLaunchKernelGGL(scale_multi_kernel, dim3((unsigned)blocks), dim3(kBlock), 0,
                       wxx::stream(), d, count, c, (const float*)nullptr, 0.0);
  wxx::scratch_free(d);
  WXX_LAUNCHED();
  return WXX_OK;
}

__global__ void clip_norm_kernel(const float* __restrict__ sumsq, float* __restrict__ norm) {
  if (threadIdx.x == 0) norm[0] = (float)sqrt((double)sumsq[0]);
}

// The rescale of clip_grad_norm_ (reference src/wxx/nn/utils.py:95-101) with
// the coefficient decided on the device from `sumsq` (wxx_sumsq_multi's
// output), so no readback sits between the norm and the rescale; `norm`
// (optional) receives sqrt(sumsq) rounded to f32.
WXX_API int wxx_clip_scale_multi(void* const* x, const int64_t* n, int count,
                                 const float* sumsq, double max_norm, float* norm) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && n && sumsq && count >= 0, "null pointer");
  if (norm)
    hipLaunchKernelGGL(clip_norm_kernel, dim3(1), dim3(64), 0, wxx::stream(), sumsq, norm);
  if (count == 0) {
    WXX_LAUNCHED();
    return WXX_OK;
  }
  TensorDesc* d = nullptr;
  int64_t blocks = 0;
  int rc = upload_table(x, nullptr, nullptr, nullptr, n, count, &d, &blocks);
  if (rc) return rc;
  if (blocks > 0)
    hipLaunchKernelGGL(scale_multi_kernel, dim3((unsigned)blocks), dim3(kBlock), 0,
                       wxx::stream(), d, count, 0.f, sumsq, max_norm);
  wxx::scratch_free(d);
  WXX_LAUNCHED();
  return WXX_OK;
}
