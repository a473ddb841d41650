// BatchNorm over NCHW f32 tensors: per-channel statistics across (B, H, W),
// running-statistic EMA, normalisation, and the backward pair.
//
// Reference semantics (src/wxx/shaders/layers/batchnorm.wgsl:30-111,
// batchnormdx.wgsl:24-50, batchnormdg.wgsl:22-74; host
// src/wxx/functional/normalization.py:148-305):
//  * training: mu = S/M, var = max(0, Q/M - mu^2), inv = rsqrt(var + eps)
//    (no zero-variance special case), running_mean = (1-m) rm + m mu,
//    running_var = (1-m) rv + m var * M/(M-1) (var itself when M == 1);
//  * eval: inv = rsqrt(running_var + eps), y uses the running mean;
//  * dgamma = sum dy xhat, dbeta = sum dy;
//    dx = (g inv / M) (M dy - dbeta - xhat dgamma).
//
// MI355X design: the reference gives each channel one 256-thread workgroup
// (64-512 workgroups for ResNet18, a quarter of the chip).  Here the
// per-channel sums run as a (channel, split) grid of partial reductions,
// a per-channel finalize adds the partials in split order (deterministic),
// and the normalisation is a separate fully parallel elementwise pass.
#include "common.h"

namespace {

constexpr int kBlock = 256;

// One running-statistic update, r <- (1 - m) r + m v, written once so every
// kernel rounds it the same way.
__device__ __forceinline__ float bn_ema(float r, float m, float v) {
  return (1.f - m) * r + m * v;
}

// The normalised, scaled and shifted value (v - mu) inv g + b, with its
// rounding fixed (one product, then one fused multiply-add) so that the
// backward of the ReLU variant recomputes it bit for bit.
__device__ __forceinline__ float bn_affine(float v, float mu, float is, float g, float b) {
  return __builtin_fmaf((v - mu) * is, g, b);
}

// part[(c * splits + s) * 2 + {0,1}] = sums over this split of (a, b), where
// (a, b) = (x, x^2) for statistics or (dy * xhat, dy) for the gradient.
template <bool GRAD>
__global__ __launch_bounds__(kBlock) void bn_partial_kernel(
    const float* __restrict__ x, const float* __restrict__ dy, const float* __restrict__ mean,
    const float* __restrict__ inv, float* __restrict__ part, int64_t B, int64_t Cc, int64_t HW,
    int splits) {
  __shared__ float red[4];
  const int64_t c = blockIdx.x;
  const int s = blockIdx.y;
  const int64_t M = B * HW;
  const int64_t seg = (M + splits - 1) / splits;
  const int64_t m0 = s * seg;
  const int64_t m1 = m0 + seg < M ? m0 + seg : M;
  float mu = 0.f, is = 0.f;
  if (GRAD) {
    mu = mean[c];
    is = inv[c];
  }
  float a = 0.f, b = 0.f;
  for (int64_t m = m0 + threadIdx.x; m < m1; m += kBlock) {
    const int64_t bb = m / HW, sp = m - bb * HW;
    const int64_t idx = (bb * Cc + c) * HW + sp;
    const float v = x[idx];
    if (GRAD) {
      const float d = dy[idx];
      a += d * (v - mu) * is;
      b += d;
    } else {
      a += v;
      b += v * v;
    }
  }
  a = wxx::block_sum(a, red);
  b = wxx::block_sum(b, red);
  if (threadIdx.x == 0) {
    part[(c * splits + s) * 2 + 0] = a;
    part[(c * splits + s) * 2 + 1] = b;
  }
}

__global__ __launch_bounds__(kBlock) void bn_finalize_kernel(
    const float* __restrict__ part, float* __restrict__ running_mean,
    float* __restrict__ running_var, float* __restrict__ saved_mean, float* __restrict__ inv_std,
    int64_t Cc, int64_t M, int splits, float eps, float momentum, int training) {
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (c >= Cc) return;
  if (!training) {
    saved_mean[c] = running_mean[c];
    inv_std[c] = rsqrtf(running_var[c] + eps);
    return;
  }
  float S = 0.f, Q = 0.f;
  for (int s = 0; s < splits; ++s) {
    S += part[(c * splits + s) * 2 + 0];
    Q += part[(c * splits + s) * 2 + 1];
  }
  const float mf = (float)M;
  const float mu = S / mf;
  const float var = fmaxf(0.f, Q / mf - mu * mu);
  saved_mean[c] = mu;
  inv_std[c] = rsqrtf(var + eps);
  running_mean[c] = bn_ema(running_mean[c], momentum, mu);
  const float unbiased = M > 1 ? var * (mf / (mf - 1.f)) : var;
  running_var[c] = bn_ema(running_var[c], momentum, unbiased);
}

__global__ __launch_bounds__(kBlock) void bn_grad_finalize_kernel(const float* __restrict__ part,
                                                                  float* __restrict__ dg,
                                                                  float* __restrict__ db,
                                                                  int64_t Cc, int splits) {
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (c >= Cc) return;
  float a = 0.f, b = 0.f;
  for (int s = 0; s < splits; ++s) {
    a += part[(c * splits + s) * 2 + 0];
    b += part[(c * splits + s) * 2 + 1];
  }
  dg[c] = a;
  db[c] = b;
}

__global__ __launch_bounds__(kBlock) void bn_apply_kernel(
    const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ b,
    const float* __restrict__ mean, const float* __restrict__ inv, float* __restrict__ y,
    int64_t n, int64_t Cc, int64_t HW) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    const int64_t c = (i / HW) % Cc;
    y[i] = bn_affine(x[i], mean[c], inv[c], g[c], b[c]);
  }
}

__global__ __launch_bounds__(kBlock) void bn_dx_kernel(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ g,
    const float* __restrict__ dg, const float* __restrict__ db, const float* __restrict__ mean,
    const float* __restrict__ inv, float* __restrict__ dx, int64_t n, int64_t Cc, int64_t HW,
    float mf) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    const int64_t c = (i / HW) % Cc;
    const float is = inv[c];
    const float xh = (x[i] - mean[c]) * is;
    dx[i] = (g[c] * is / mf) * (mf * dy[i] - db[c] - xh * dg[c]);
  }
}

// Channels of at most kFusedMaxM elements (ResNet18's BatchNorms at batch
// 128 on 32x32 images but the stem's) run as one workgroup of up to 1024
// threads per channel that holds the channel in registers (E elements per
// thread, all loads issued at once), takes the statistics and writes the
// output in one launch: more launches cost more in latency than their extra
// parallelism gains on these sizes.  Same formulas, the sums in another
// (fixed) order.  (At 32768 elements, 32 per thread, the ReLU backward ran
// out of registers and one workgroup per channel left most CUs idle: 136 us
// against ~10 us for the two-launch split path.)
constexpr int64_t kFusedMaxM = 8192;

__device__ __forceinline__ int64_t bn_index(int m, int HW, int Cc, int c) {
  const int bb = m / HW, sp = m - bb * HW;
  return ((int64_t)bb * Cc + c) * HW + sp;
}

// RES / RELU: the residual block's tail that follows a BatchNorm in
// ResNet, y = relu(bn(x) + r), in the same launch; `updates` applies the
// running-statistic update that many times (the reference's blocks evaluate
// their first BatchNorm twice per forward).
template <int E, bool RES, bool RELU>
__global__ __launch_bounds__(1024) void bn_fused_fwd_kernel(
    const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ b,
    const float* __restrict__ r, float* __restrict__ running_mean,
    float* __restrict__ running_var, float* __restrict__ y, float* __restrict__ saved_mean,
    float* __restrict__ inv_std, int B, int Cc, int HW, float eps, float momentum, int updates) {
  __shared__ float red[16];
  const int c = blockIdx.x, T = blockDim.x;
  const int M = B * HW;
  float v[E];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int m = threadIdx.x + e * T;
    v[e] = m < M ? x[bn_index(m, HW, Cc, c)] : 0.f;
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    s1 += v[e];
    s2 += v[e] * v[e];
  }
  const float S = wxx::block_sum(s1, red);
  const float Q = wxx::block_sum(s2, red);
  const float mf = (float)M;
  const float mu = S / mf;
  const float var = fmaxf(0.f, Q / mf - mu * mu);
  const float is = rsqrtf(var + eps);
  if (threadIdx.x == 0) {
    saved_mean[c] = mu;
    inv_std[c] = is;
    const float unbiased = M > 1 ? var * (mf / (mf - 1.f)) : var;
    float rm = running_mean[c], rv = running_var[c];
    for (int u = 0; u < updates; ++u) {
      rm = bn_ema(rm, momentum, mu);
      rv = bn_ema(rv, momentum, unbiased);
    }
    running_mean[c] = rm;
    running_var[c] = rv;
  }
  const float gc = g[c], bc = b[c];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int m = threadIdx.x + e * T;
    if (m < M) {
      const int64_t i = bn_index(m, HW, Cc, c);
      float t = bn_affine(v[e], mu, is, gc, bc);
      if (RES) t += r[i];
      if (RELU) t = fmaxf(0.f, t);
      y[i] = t;
    }
  }
}

// dgamma, dbeta and dx of one channel per workgroup (sizes as above).  With
// RELU the incoming gradient is first masked by relu' of the forward's
// pre-activation, recomputed from x (and r) exactly as the forward rounded
// it; with RES the masked gradient is also the residual's (dr).
template <int E, bool RES, bool RELU>
__global__ __launch_bounds__(1024) void bn_fused_bwd_kernel(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ g,
    const float* __restrict__ b, const float* __restrict__ r, const float* __restrict__ mean,
    const float* __restrict__ inv, float* __restrict__ dg, float* __restrict__ db,
    float* __restrict__ dx, float* __restrict__ dr, int B, int Cc, int HW) {
  __shared__ float red[16];
  const int c = blockIdx.x, T = blockDim.x;
  const int M = B * HW;
  const float mu = mean[c], is = inv[c];
  const float gc = g[c];
  float d[E], xh[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int m = threadIdx.x + e * T;
    const bool in = m < M;
    const int64_t i = in ? bn_index(m, HW, Cc, c) : 0;
    d[e] = in ? dy[i] : 0.f;
    const float xv = in ? x[i] : 0.f;
    xh[e] = in ? (xv - mu) * is : 0.f;
    if (RELU && in) {
      float t = bn_affine(xv, mu, is, gc, b[c]);
      if (RES) t += r[i];
      d[e] = d[e] * (t > 0.f ? 1.f : 0.f);  // relu' times the gradient, as the unary backward
    }
    if (RES && in) dr[i] = d[e];
  }
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    s1 += d[e] * xh[e];
    s2 += d[e];
  }
  const float A = wxx::block_sum(s1, red);
  const float Bs = wxx::block_sum(s2, red);
  if (threadIdx.x == 0) {
    dg[c] = A;
    db[c] = Bs;
  }
  const float mf = (float)M;
  const float k = gc * is / mf;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int m = threadIdx.x + e * T;
    if (m < M) dx[bn_index(m, HW, Cc, c)] = k * (mf * d[e] - Bs - xh[e] * A);
  }
}

// Larger channels (training): a (channel, split) grid of partial sums, then
// a second launch over the same grid in which every workgroup adds its
// channel's partials itself (all in the same fixed order, so they agree bit
// for bit), the channel's first workgroup stores the statistics, and each
// normalises its own split: two launches at the whole chip's width where one
// workgroup per channel would leave most CUs idle (ResNet18's stem: 64
// channels of 32768) and run out of registers.

// The channel's two sums from its partials: lane l of wave 0 adds splits l,
// l + 64, ... in order, then a butterfly over the wave; every thread gets
// the result.
__device__ __forceinline__ float2 bn_channel_sums(const float* __restrict__ part, int64_t c,
                                                  int splits, float* red) {
  if (threadIdx.x < 64) {
    float a = 0.f, b = 0.f;
    for (int s = threadIdx.x; s < splits; s += 64) {
      a += part[(c * splits + s) * 2 + 0];
      b += part[(c * splits + s) * 2 + 1];
    }
    a = wxx::warp_sum(a);
    b = wxx::warp_sum(b);
    if (threadIdx.x == 0) {
      red[0] = a;
      red[1] = b;
    }
  }
  __syncthreads();
  return make_float2(red[0], red[1]);
}

__device__ __forceinline__ void bn_split_range(int64_t M, int splits, int s, int64_t& m0,
                                               int64_t& m1) {
  const int64_t seg = (M + splits - 1) / splits;
  m0 = s * seg;
  m1 = m0 + seg < M ? m0 + seg : M;
}

template <bool RES, bool RELU>
__global__ __launch_bounds__(kBlock) void bn_split_apply_kernel(
    const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ b,
    const float* __restrict__ r, const float* __restrict__ part, float* __restrict__ running_mean,
    float* __restrict__ running_var, float* __restrict__ y, float* __restrict__ saved_mean,
    float* __restrict__ inv_std, int64_t B, int64_t Cc, int64_t HW, int splits, float eps,
    float momentum, int updates) {
  __shared__ float red[2];
  const int64_t c = blockIdx.x;
  const int s = blockIdx.y;
  const float2 t = bn_channel_sums(part, c, splits, red);
  const int64_t M = B * HW;
  const float mf = (float)M;
  const float mu = t.x / mf;
  const float var = fmaxf(0.f, t.y / mf - mu * mu);
  const float is = rsqrtf(var + eps);
  if (s == 0 && threadIdx.x == 0) {
    saved_mean[c] = mu;
    inv_std[c] = is;
    const float unbiased = M > 1 ? var * (mf / (mf - 1.f)) : var;
    float rm = running_mean[c], rv = running_var[c];
    for (int u = 0; u < updates; ++u) {
      rm = bn_ema(rm, momentum, mu);
      rv = bn_ema(rv, momentum, unbiased);
    }
    running_mean[c] = rm;
    running_var[c] = rv;
  }
  const float gc = g[c], bc = b[c];
  int64_t m0, m1;
  bn_split_range(M, splits, s, m0, m1);
  for (int64_t m = m0 + threadIdx.x; m < m1; m += kBlock) {
    const int64_t bb = m / HW, sp = m - bb * HW;
    const int64_t idx = (bb * Cc + c) * HW + sp;
    float v = bn_affine(x[idx], mu, is, gc, bc);
    if (RES) v += r[idx];
    if (RELU) v = fmaxf(0.f, v);
    y[idx] = v;
  }
}

// The gradient's partial sums (dy xhat, dy), dy masked by relu' of the
// recomputed pre-activation for RELU.
template <bool RES, bool RELU>
__global__ __launch_bounds__(kBlock) void bn_split_grad_partial_kernel(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ g,
    const float* __restrict__ b, const float* __restrict__ r, const float* __restrict__ mean,
    const float* __restrict__ inv, float* __restrict__ part, int64_t B, int64_t Cc, int64_t HW,
    int splits) {
  __shared__ float red[4];
  const int64_t c = blockIdx.x;
  const int s = blockIdx.y;
  const int64_t M = B * HW;
  const float mu = mean[c], is = inv[c];
  const float gc = g[c], bc = RELU ? b[c] : 0.f;
  int64_t m0, m1;
  bn_split_range(M, splits, s, m0, m1);
  float a = 0.f, sd = 0.f;
  for (int64_t m = m0 + threadIdx.x; m < m1; m += kBlock) {
    const int64_t bb = m / HW, sp = m - bb * HW;
    const int64_t idx = (bb * Cc + c) * HW + sp;
    const float xv = x[idx];
    float d = dy[idx];
    if (RELU) {
      float t = bn_affine(xv, mu, is, gc, bc);
      if (RES) t += r[idx];
      d = d * (t > 0.f ? 1.f : 0.f);
    }
    a += d * ((xv - mu) * is);
    sd += d;
  }
  a = wxx::block_sum(a, red);
  sd = wxx::block_sum(sd, red);
  if (threadIdx.x == 0) {
    part[(c * splits + s) * 2 + 0] = a;
    part[(c * splits + s) * 2 + 1] = sd;
  }
}

template <bool RES, bool RELU>
__global__ __launch_bounds__(kBlock) void bn_split_dx_kernel(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ g,
    const float* __restrict__ b, const float* __restrict__ r, const float* __restrict__ mean,
    const float* __restrict__ inv, const float* __restrict__ part, float* __restrict__ dg,
    float* __restrict__ db, float* __restrict__ dx, float* __restrict__ dr, int64_t B, int64_t Cc,
    int64_t HW, int splits) {
  __shared__ float red[2];
  const int64_t c = blockIdx.x;
  const int s = blockIdx.y;
  const float2 t = bn_channel_sums(part, c, splits, red);
  const float A = t.x, Bs = t.y;
  if (s == 0 && threadIdx.x == 0) {
    dg[c] = A;
    db[c] = Bs;
  }
  const int64_t M = B * HW;
  const float mf = (float)M;
  const float mu = mean[c], is = inv[c];
  const float gc = g[c], bc = RELU ? b[c] : 0.f;
  const float k = gc * is / mf;
  int64_t m0, m1;
  bn_split_range(M, splits, s, m0, m1);
  for (int64_t m = m0 + threadIdx.x; m < m1; m += kBlock) {
    const int64_t bb = m / HW, sp = m - bb * HW;
    const int64_t idx = (bb * Cc + c) * HW + sp;
    const float xv = x[idx];
    float d = dy[idx];
    if (RELU) {
      float tt = bn_affine(xv, mu, is, gc, bc);
      if (RES) tt += r[idx];
      d = d * (tt > 0.f ? 1.f : 0.f);
    }
    if (RES) dr[idx] = d;
    dx[idx] = k * (mf * d - Bs - ((xv - mu) * is) * A);
  }
}

// Threads per channel (a multiple of 64, at most 1024) and elements per
// thread E for a channel of M <= kFusedMaxM elements.
struct FusedGeo {
  int threads, E;
};
FusedGeo fused_geo(int64_t M) {
  int E = 1;
  while ((int64_t)E * 1024 < M) E *= 2;
  const int64_t t = (M + E - 1) / E;
  return {(int)std::min<int64_t>(1024, (t + 63) / 64 * 64), E};
}

// Whether a training forward / a backward runs as one fused launch.
bool fused_ok(int64_t B, int64_t C, int64_t HW) {
  const int64_t M = B * HW;
  return M > 0 && M <= kFusedMaxM && C <= 0x7fffffff && B * C * HW < (int64_t(1) << 31);
}

template <bool RES, bool RELU>
int launch_fused_fwd(const float* x, const float* gamma, const float* beta, const float* r,
                     float* running_mean, float* running_var, float* y, float* saved_mean,
                     float* inv_std, int64_t B, int64_t C, int64_t HW, float eps, float momentum,
                     int updates) {
  const FusedGeo fg = fused_geo(B * HW);
  const dim3 grid((unsigned)C), block((unsigned)fg.threads);
  hipStream_t s = wxx::stream();
#define WXX_BN_FWD(EE)                                                                        \
  hipLaunchKernelGGL((bn_fused_fwd_kernel<EE, RES, RELU>), grid, block, 0, s, x, gamma, beta, r, \
                     running_mean, running_var, y, saved_mean, inv_std, (int)B, (int)C, (int)HW, \
                     eps, momentum, updates)
  switch (fg.E) {
    case 1: WXX_BN_FWD(1); break;
    case 2: WXX_BN_FWD(2); break;
    case 4: WXX_BN_FWD(4); break;
    case 8: WXX_BN_FWD(8); break;
    case 16: WXX_BN_FWD(16); break;
    default: WXX_BN_FWD(32); break;
  }
#undef WXX_BN_FWD
  WXX_LAUNCHED();
  return WXX_OK;
}

template <bool RES, bool RELU>
int launch_fused_bwd(const float* dy, const float* x, const float* gamma, const float* beta,
                     const float* r, const float* saved_mean, const float* inv_std, float* dgamma,
                     float* dbeta, float* dx, float* dr, int64_t B, int64_t C, int64_t HW) {
  const FusedGeo fg = fused_geo(B * HW);
  const dim3 grid((unsigned)C), block((unsigned)fg.threads);
  hipStream_t s = wxx::stream();
#define WXX_BN_BWD(EE)                                                                          \
  hipLaunchKernelGGL((bn_fused_bwd_kernel<EE, RES, RELU>), grid, block, 0, s, dy, x, gamma, beta, \
                     r, saved_mean, inv_std, dgamma, dbeta, dx, dr, (int)B, (int)C, (int)HW)
  switch (fg.E) {
    case 1: WXX_BN_BWD(1); break;
    case 2: WXX_BN_BWD(2); break;
    case 4: WXX_BN_BWD(4); break;
    case 8: WXX_BN_BWD(8); break;
    case 16: WXX_BN_BWD(16); break;
    default: WXX_BN_BWD(32); break;
  }
#undef WXX_BN_BWD
  WXX_LAUNCHED();
  return WXX_OK;
}

int pick_splits(int64_t Cc, int64_t M) {
  const int64_t target = (int64_t)wxx::num_cus() * 8;
  int64_t s = (target + Cc - 1) / Cc;
  s = std::min<int64_t>(s, std::max<int64_t>(1, M / 1024));
  return (int)std::max<int64_t>(1, std::min<int64_t>(s, 1024));
}

// Training forward / backward of channels above kFusedMaxM: two launches
// each (partial sums, then sums + elementwise pass).
bool split_ok(int64_t B, int64_t C, int64_t HW) {
  return B * HW > 0 && C <= 0x7fffffff && B * C * HW < (int64_t(1) << 31);
}

template <bool RES, bool RELU>
int launch_split_fwd(const float* x, const float* gamma, const float* beta, const float* r,
                     float* running_mean, float* running_var, float* y, float* saved_mean,
                     float* inv_std, int64_t B, int64_t C, int64_t HW, float eps, float momentum,
                     int updates) {
  hipStream_t s = wxx::stream();
  const int splits = pick_splits(C, B * HW);
  float* part = (float*)wxx::scratch_alloc(sizeof(float) * 2 * C * splits);
  if (!part) return wxx::set_error(WXX_E_OOM, "batchnorm partials");
  const dim3 grid((unsigned)C, splits);
  hipLaunchKernelGGL(bn_partial_kernel<false>, grid, dim3(kBlock), 0, s, x, nullptr, nullptr,
                     nullptr, part, B, C, HW, splits);
  hipLaunchKernelGGL((bn_split_apply_kernel<RES, RELU>), grid, dim3(kBlock), 0, s, x, gamma, beta,
                     r, part, running_mean, running_var, y, saved_mean, inv_std, B, C, HW, splits,
                     eps, momentum, updates);
  wxx::scratch_free(part);
  WXX_LAUNCHED();
  return WXX_OK;
}

template <bool RES, bool RELU>
int launch_split_bwd(const float* dy, const float* x, const float* gamma, const float* beta,
                     const float* r, const float* saved_mean, const float* inv_std, float* dgamma,
                     float* dbeta, float* dx, float* dr, int64_t B, int64_t C, int64_t HW) {
  hipStream_t s = wxx::stream();
  const int splits = pick_splits(C, B * HW);
  float* part = (float*)wxx::scratch_alloc(sizeof(float) * 2 * C * splits);
  if (!part) return wxx::set_error(WXX_E_OOM, "batchnorm partials");
  const dim3 grid((unsigned)C, splits);
  hipLaunchKernelGGL((bn_split_grad_partial_kernel<RES, RELU>), grid, dim3(kBlock), 0, s, dy, x,
                     gamma, beta, r, saved_mean, inv_std, part, B, C, HW, splits);
  hipLaunchKernelGGL((bn_split_dx_kernel<RES, RELU>), grid, dim3(kBlock), 0, s, dy, x, gamma, beta,
                     r, saved_mean, inv_std, part, dgamma, dbeta, dx, dr, B, C, HW, splits);
  wxx::scratch_free(part);
  WXX_LAUNCHED();
  return WXX_OK;
}

}  // namespace

// Replaces functional.batchnorm (reference src/wxx/functional/normalization.py:148-206).
WXX_API int wxx_batchnorm(const float* x, const float* gamma, const float* beta,
                          float* running_mean, float* running_var, float* y, float* saved_mean,
                          float* inv_std, int64_t B, int64_t C, int64_t HW, float eps,
                          float momentum, int training) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && gamma && beta && running_mean && running_var && y && saved_mean && inv_std,
              "null pointer");
  WXX_REQUIRE(B >= 0 && C >= 1 && HW >= 0, "bad batchnorm dims");
  hipStream_t s = wxx::stream();
  const int64_t M = B * HW;
  if (training && fused_ok(B, C, HW)) {
    return launch_fused_fwd<false, false>(x, gamma, beta, nullptr, running_mean, running_var, y,
                                          saved_mean, inv_std, B, C, HW, eps, momentum, 1);
  }
  if (training && split_ok(B, C, HW)) {
    return launch_split_fwd<false, false>(x, gamma, beta, nullptr, running_mean, running_var, y,
                                          saved_mean, inv_std, B, C, HW, eps, momentum, 1);
  }
  int splits = 1;
  float* part = nullptr;
  if (training) {
    splits = pick_splits(C, M);
    part = (float*)wxx::scratch_alloc(sizeof(float) * 2 * C * splits);
    if (!part) return wxx::set_error(WXX_E_OOM, "batchnorm partials");
    hipLaunchKernelGGL(bn_partial_kernel<false>, dim3((unsigned)C, splits), dim3(kBlock), 0, s, x,
                       nullptr, nullptr, nullptr, part, B, C, HW, splits);
    WXX_LAUNCHED();
  }
  hipLaunchKernelGGL(bn_finalize_kernel, dim3(wxx::grid_1d(C, kBlock)), dim3(kBlock), 0, s, part,
                     running_mean, running_var, saved_mean, inv_std, C, M, splits, eps, momentum,
                     training);
  WXX_LAUNCHED();
  if (part) wxx::scratch_free(part);
  const int64_t n = M * C;
  if (n > 0) {
    hipLaunchKernelGGL(bn_apply_kernel, dim3(wxx::grid_1d(n, kBlock, 16384)), dim3(kBlock), 0, s,
                       x, gamma, beta, saved_mean, inv_std, y, n, C, HW);
    WXX_LAUNCHED();
  }
  return WXX_OK;
}

// Replaces functional.batchnormdg (reference normalization.py:260-305).
WXX_API int wxx_batchnormdg(const float* dy, const float* x, const float* saved_mean,
                            const float* inv_std, float* dgamma, float* dbeta, int64_t B,
                            int64_t C, int64_t HW) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && x && saved_mean && inv_std && dgamma && dbeta, "null pointer");
  WXX_REQUIRE(B >= 0 && C >= 1 && HW >= 0, "bad batchnorm dims");
  hipStream_t s = wxx::stream();
  const int64_t M = B * HW;
  const int splits = pick_splits(C, M);
  float* part = (float*)wxx::scratch_alloc(sizeof(float) * 2 * C * splits);
  if (!part) return wxx::set_error(WXX_E_OOM, "batchnorm partials");
  hipLaunchKernelGGL(bn_partial_kernel<true>, dim3((unsigned)C, splits), dim3(kBlock), 0, s, x, dy,
                     saved_mean, inv_std, part, B, C, HW, splits);
  WXX_LAUNCHED();
  hipLaunchKernelGGL(bn_grad_finalize_kernel, dim3(wxx::grid_1d(C, kBlock)), dim3(kBlock), 0, s,
                     part, dgamma, dbeta, C, splits);
  WXX_LAUNCHED();
  wxx::scratch_free(part);
  return WXX_OK;
}

// Replaces functional.batchnormdx (reference normalization.py:209-257).
WXX_API int wxx_batchnormdx(const float* dy, const float* x, const float* gamma,
                            const float* dgamma, const float* dbeta, const float* saved_mean,
                            const float* inv_std, float* dx, int64_t B, int64_t C, int64_t HW) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && x && gamma && dgamma && dbeta && saved_mean && inv_std && dx, "null pointer");
  const int64_t n = B * C * HW;
  if (n <= 0) return WXX_OK;
  hipLaunchKernelGGL(bn_dx_kernel, dim3(wxx::grid_1d(n, kBlock, 16384)), dim3(kBlock), 0,
                     wxx::stream(), dy, x, gamma, dgamma, dbeta, saved_mean, inv_std, dx, n, C,
                     HW, (float)(B * HW));
  WXX_LAUNCHED();
  return WXX_OK;
}

// functional.batchnormdg followed by functional.batchnormdx (reference
// normalization.py:209-305) in one call: the autograd backward of batchnorm.
WXX_API int wxx_batchnorm_backward(const float* dy, const float* x, const float* gamma,
                                   const float* saved_mean, const float* inv_std, float* dgamma,
                                   float* dbeta, float* dx, int64_t B, int64_t C, int64_t HW) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && x && gamma && saved_mean && inv_std && dgamma && dbeta && dx, "null pointer");
  WXX_REQUIRE(B >= 0 && C >= 1 && HW >= 0, "bad batchnorm dims");
  if (fused_ok(B, C, HW)) {
    return launch_fused_bwd<false, false>(dy, x, gamma, nullptr, nullptr, saved_mean, inv_std,
                                          dgamma, dbeta, dx, nullptr, B, C, HW);
  }
  if (split_ok(B, C, HW)) {
    return launch_split_bwd<false, false>(dy, x, gamma, nullptr, nullptr, saved_mean, inv_std,
                                          dgamma, dbeta, dx, nullptr, B, C, HW);
  }
  int rc = wxx_batchnormdg(dy, x, saved_mean, inv_std, dgamma, dbeta, B, C, HW);
  if (rc) return rc;
  return wxx_batchnormdx(dy, x, gamma, dgamma, dbeta, saved_mean, inv_std, dx, B, C, HW);
}

// functional.batchnorm in training (reference normalization.py:148-206)
// followed by the residual add and ReLU of ResNet's blocks (reference
// src/wxx/nn/resnet.py:31-37, 65-66): y = relu(bn(x) + residual), residual
// optional, ReLU optional, the running statistics updated `updates` times (1
// or 2); one launch for channels of at most kFusedMaxM elements, two above.
WXX_API int wxx_batchnorm_act(const float* x, const float* gamma, const float* beta,
                              const float* residual, float* running_mean, float* running_var,
                              float* y, float* saved_mean, float* inv_std, int64_t B, int64_t C,
                              int64_t HW, float eps, float momentum, int updates, int relu) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && gamma && beta && running_mean && running_var && y && saved_mean && inv_std,
              "null pointer");
  WXX_REQUIRE(B >= 0 && C >= 1 && HW >= 0, "bad batchnorm dims");
  WXX_REQUIRE(updates == 1 || updates == 2, "updates must be 1 or 2, got %d", updates);
  if (!split_ok(B, C, HW))
    return wxx::set_error(WXX_E_UNSUPPORTED,
                          "batchnorm_act needs 1 <= B*HW and B*C*HW < 2^31, got B*HW = %lld, "
                          "B*C*HW = %lld", (long long)(B * HW), (long long)(B * C * HW));
  const bool one = fused_ok(B, C, HW);
#define WXX_BN_ACT(RES, RELU)                                                                  \
  (one ? launch_fused_fwd<RES, RELU>(x, gamma, beta, residual, running_mean, running_var, y,     \
                                     saved_mean, inv_std, B, C, HW, eps, momentum, updates)     \
       : launch_split_fwd<RES, RELU>(x, gamma, beta, residual, running_mean, running_var, y,     \
                                     saved_mean, inv_std, B, C, HW, eps, momentum, updates))
  if (residual) return relu ? WXX_BN_ACT(true, true) : WXX_BN_ACT(true, false);
  return relu ? WXX_BN_ACT(false, true) : WXX_BN_ACT(false, false);
#undef WXX_BN_ACT
}

// The backward of wxx_batchnorm_act (autograd's batchnorm backward,
// reference normalization.py:209-305, after the ReLU's and the add's,
// autograd/pointwise.py): dgamma, dbeta, dx, and the residual's gradient
// (dresidual, needed exactly when the forward had a residual).
WXX_API int wxx_batchnorm_act_backward(const float* dy, const float* x, const float* gamma,
                                       const float* beta, const float* residual,
                                       const float* saved_mean, const float* inv_std,
                                       float* dgamma, float* dbeta, float* dx, float* dresidual,
                                       int64_t B, int64_t C, int64_t HW, int relu) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && x && gamma && beta && saved_mean && inv_std && dgamma && dbeta && dx,
              "null pointer");
  WXX_REQUIRE(!residual == !dresidual, "residual and dresidual go together");
  WXX_REQUIRE(B >= 0 && C >= 1 && HW >= 0, "bad batchnorm dims");
  if (!split_ok(B, C, HW))
    return wxx::set_error(WXX_E_UNSUPPORTED,
                          "batchnorm_act needs 1 <= B*HW and B*C*HW < 2^31, got B*HW = %lld, "
                          "B*C*HW = %lld", (long long)(B * HW), (long long)(B * C * HW));
  const bool one = fused_ok(B, C, HW);
#define WXX_BN_ACT_BWD(RES, RELU)                                                              \
  (one ? launch_fused_bwd<RES, RELU>(dy, x, gamma, beta, residual, saved_mean, inv_std, dgamma, \
                                     dbeta, dx, dresidual, B, C, HW)                           \
       : launch_split_bwd<RES, RELU>(dy, x, gamma, beta, residual, saved_mean, inv_std, dgamma, \
                                     dbeta, dx, dresidual, B, C, HW))
  if (residual) return relu ? WXX_BN_ACT_BWD(true, true) : WXX_BN_ACT_BWD(true, false);
  return relu ? WXX_BN_ACT_BWD(false, true) : WXX_BN_ACT_BWD(false, false);
#undef WXX_BN_ACT_BWD
}
