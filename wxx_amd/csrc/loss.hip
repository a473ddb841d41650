// Fused softmax cross-entropy: per-row loss and dlogits in one kernel.
//
// Reference semantics (src/wxx/shaders/loss/cceloss.wgsl:21-85, host
// src/wxx/functional/loss.py:20-101):
//   m = max(-1e38, max_j z_j), s = sum_j exp(z_j - m),
//   loss = (log(s) + m) - z[t],  dz_j = exp(z_j - m) / s - [j == t].
// Targets >= K are rejected: the reference reads every target back to the
// host before launching; here the kernel flags an out-of-range target in a
// device word and the host reads that one word back.
//
// MI355X design: the reference runs one 256-thread workgroup per row with
// three passes over the row (max, sum, write).  Here the row is held in
// VGPRs of one wave / workgroup (up to 65 536 columns with 1024-lane
// workgroups, e.g. GPT-2's 50 304-token vocabulary), so the logits are read
// from HBM once and dlogits written once.
#include "rows.h"

namespace {

template <int TPR, int NCH, bool VEC>
__global__ __launch_bounds__(TPR >= 256 ? TPR : 256) void cce_rows_kernel(
    const float* __restrict__ z, const uint32_t* __restrict__ targets, float* __restrict__ loss,
    float* __restrict__ dz, int64_t rows, int K, int* __restrict__ bad) {
  __shared__ float red[16];
  constexpr int RPB = TPR >= 256 ? 1 : 256 / TPR;
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  if (TPR == 64 && row >= rows) return;
  const float* zr = z + row * K;
  const uint32_t tgt = targets[row];
  const bool ok = tgt < (uint32_t)K;
  if (!ok && t == 0) bad[0] = 1;
  wxx::RowRegs<TPR, NCH, VEC> v;
  v.load(zr, K, t, -INFINITY);
  float m = -1e38f;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) m = fmaxf(m, v.v[e]);
  m = wxx::RowReduce<TPR>::max(m, red);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) {
    const float ev = v.valid(e, t, K) ? expf(v.v[e] - m) : 0.f;
    v.v[e] = ev;
    s += ev;
  }
  s = wxx::RowReduce<TPR>::sum(s, red);
  if (t == 0) loss[row] = ok ? (logf(s) + m) - zr[tgt] : __int_as_float(0x7fc00000);
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) {
    const int col = wxx::RowRegs<TPR, NCH, VEC>::col(e, t);
    v.v[e] = v.v[e] / s - (col == (int)tgt ? 1.f : 0.f);
  }
  v.store(dz + row * K, K, t);
}

// Forward half of the deferred-gradient cross-entropy: per row the loss and
// the (max, exp-sum) pair, computed exactly as cce_rows_kernel does, without
// writing dlogits.  stats[2 row] = m, stats[2 row + 1] = s.
template <int TPR, int NCH, bool VEC>
__global__ __launch_bounds__(TPR >= 256 ? TPR : 256) void cce_stats_kernel(
    const float* __restrict__ z, const uint32_t* __restrict__ targets, float* __restrict__ loss,
    float* __restrict__ stats, int64_t rows, int K, int* __restrict__ bad) {
  __shared__ float red[16];
  constexpr int RPB = TPR >= 256 ? 1 : 256 / TPR;
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  if (TPR == 64 && row >= rows) return;
  const float* zr = z + row * K;
  const uint32_t tgt = targets[row];
  const bool ok = tgt < (uint32_t)K;
  if (!ok && t == 0) bad[0] = 1;
  wxx::RowRegs<TPR, NCH, VEC> v;
  v.load(zr, K, t, -INFINITY);
  float m = -1e38f;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) m = fmaxf(m, v.v[e]);
  m = wxx::RowReduce<TPR>::max(m, red);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) s += v.valid(e, t, K) ? expf(v.v[e] - m) : 0.f;
  s = wxx::RowReduce<TPR>::sum(s, red);
  if (t == 0) {
    loss[row] = ok ? (logf(s) + m) - zr[tgt] : __int_as_float(0x7fc00000);
    stats[2 * row] = m;
    stats[2 * row + 1] = s;
  }
}

// Backward half: dz = (exp(z - m) / s - [j == t]) * g[row * g_stride], the
// values of cce_rows_kernel's dlogits times the upstream gradient as a
// separate multiply (the same two roundings).
template <int TPR, int NCH, bool VEC>
__global__ __launch_bounds__(TPR >= 256 ? TPR : 256) void cce_backward_kernel(
    const float* __restrict__ z, const uint32_t* __restrict__ targets,
    const float* __restrict__ stats, const float* __restrict__ g, int64_t g_stride,
    float* __restrict__ dz, int64_t rows, int K) {
  constexpr int RPB = TPR >= 256 ? 1 : 256 / TPR;
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  if (row >= rows) return;
  const uint32_t tgt = targets[row];
  const float m = stats[2 * row], s = stats[2 * row + 1], gr = g[row * g_stride];
  wxx::RowRegs<TPR, NCH, VEC> v;
  v.load(z + row * K, K, t, -INFINITY);
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) {
    const int col = wxx::RowRegs<TPR, NCH, VEC>::col(e, t);
    const float ev = v.valid(e, t, K) ? expf(v.v[e] - m) : 0.f;
    v.v[e] = __fmul_rn(ev / s - (col == (int)tgt ? 1.f : 0.f), gr);
  }
  v.store(dz + row * K, K, t);
}

// Rows longer than 65536: online (max, sum) pass, then the write pass.
__global__ __launch_bounds__(256) void cce_rows_looped_kernel(
    const float* __restrict__ z, const uint32_t* __restrict__ targets, float* __restrict__ loss,
    float* __restrict__ dz, int64_t K, int* __restrict__ bad) {
  __shared__ float sm[4], ss[4];
  const int64_t row = blockIdx.x;
  const float* zr = z + row * K;
  const uint32_t tgt = targets[row];
  const bool ok = (int64_t)tgt < K;
  if (!ok && threadIdx.x == 0) bad[0] = 1;
  float m = -1e38f, s = 0.f;
  for (int64_t c = threadIdx.x; c < K; c += 256) {
    const float x = zr[c];
    if (x > m) {
      s = s * expf(m - x) + 1.f;
      m = x;
    } else {
      s += expf(x - m);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float om = __shfl_xor(m, off, 64), os = __shfl_xor(s, off, 64);
    const float nm = fmaxf(m, om);
    s = s * expf(m - nm) + os * expf(om - nm);
    m = nm;
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) {
    sm[w] = m;
    ss[w] = s;
  }
  __syncthreads();
  float M = sm[0];
  for (int i = 1; i < 4; ++i) M = fmaxf(M, sm[i]);
  float S = 0.f;
  for (int i = 0; i < 4; ++i) S += ss[i] * expf(sm[i] - M);
  if (threadIdx.x == 0) loss[row] = ok ? (logf(S) + M) - zr[tgt] : __int_as_float(0x7fc00000);
  float* dr = dz + row * K;
  for (int64_t c = threadIdx.x; c < K; c += 256)
    dr[c] = expf(zr[c] - M) / S - (c == (int64_t)tgt ? 1.f : 0.f);
}

}  // namespace

// Replaces functional.cceloss (reference src/wxx/functional/loss.py:20-101).
// `bad` (device int, may be null) is set to 1 when a target is >= K; the
// caller zeroes it first and reads it back.
WXX_API int wxx_cceloss(const float* z, const uint32_t* targets, float* loss, float* dz,
                        int64_t B, int64_t K, int* bad) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(z && targets && loss && dz && bad, "null pointer");
  WXX_REQUIRE(B >= 1 && K >= 1, "cceloss expects non-empty logits");
  hipStream_t s = wxx::stream();
  const bool vec = (K % 4 == 0) && ((uintptr_t)z % 16 == 0) && ((uintptr_t)dz % 16 == 0);
  if (wxx::wide_row_plan(K) == 0) {
    hipLaunchKernelGGL(cce_rows_looped_kernel, dim3((unsigned)B), dim3(256), 0, s, z, targets,
                       loss, dz, K, bad);
  } else {
    int rc = wxx::wide_row_dispatch(K, vec, [&](auto tpr, auto nch, auto v) {
      constexpr int TPR = decltype(tpr)::value;
      hipLaunchKernelGGL((cce_rows_kernel<TPR, decltype(nch)::value, decltype(v)::value>),
                         wxx::row_grid(TPR, B), dim3(TPR >= 256 ? TPR : 256), 0, s, z, targets,
                         loss, dz, B, (int)K, bad);
      return 0;
    });
    if (rc) return rc;
  }
  WXX_LAUNCHED();
  return WXX_OK;
}

// Deferred-gradient cross-entropy (no single reference counterpart: the
// loss and dlogits of functional.cceloss, reference functional/loss.py:20-101,
// with the dlogits produced in the backward, already multiplied by the
// upstream gradient, autograd/layers.py:6-20).  stats receives 2 floats per
// row.  Rows of K <= 65536 only (larger rows use wxx_cceloss).
WXX_API int wxx_cceloss_stats(const float* z, const uint32_t* targets, float* loss, float* stats,
                              int64_t B, int64_t K, int* bad) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(z && targets && loss && stats && bad, "null pointer");
  WXX_REQUIRE(B >= 1 && K >= 1, "cceloss expects non-empty logits");
  if (wxx::wide_row_plan(K) == 0)
    return wxx::set_error(WXX_E_UNSUPPORTED, "deferred cceloss rows of %lld", (long long)K);
  hipStream_t s = wxx::stream();
  const bool vec = (K % 4 == 0) && ((uintptr_t)z % 16 == 0);
  int rc = wxx::wide_row_dispatch(K, vec, [&](auto tpr, auto nch, auto v) {
    constexpr int TPR = decltype(tpr)::value;
    hipLaunchKernelGGL((cce_stats_kernel<TPR, decltype(nch)::value, decltype(v)::value>),
                       wxx::row_grid(TPR, B), dim3(TPR >= 256 ? TPR : 256), 0, s, z, targets,
                       loss, stats, B, (int)K, bad);
    return 0;
  });
  if (rc) return rc;
  WXX_LAUNCHED();
  return WXX_OK;
}

// dz = (softmax(z) - onehot(targets)) * g[row * g_stride] from the stats of
// wxx_cceloss_stats.
WXX_API int wxx_cceloss_backward(const float* z, const uint32_t* targets, const float* stats,
                                 const float* g, int64_t g_stride, float* dz, int64_t B,
                                 int64_t K) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(z && targets && stats && g && dz, "null pointer");
  WXX_REQUIRE(B >= 1 && K >= 1 && g_stride >= 0, "bad cceloss backward dims");
  if (wxx::wide_row_plan(K) == 0)
    return wxx::set_error(WXX_E_UNSUPPORTED, "deferred cceloss rows of %lld", (long long)K);
  hipStream_t s = wxx::stream();
  const bool vec = (K % 4 == 0) && ((uintptr_t)z % 16 == 0) && ((uintptr_t)dz % 16 == 0);
  int rc = wxx::wide_row_dispatch(K, vec, [&](auto tpr, auto nch, auto v) {
    constexpr int TPR = decltype(tpr)::value;
    hipLaunchKernelGGL((cce_backward_kernel<TPR, decltype(nch)::value, decltype(v)::value>),
                       wxx::row_grid(TPR, B), dim3(TPR >= 256 ? TPR : 256), 0, s, z, targets,
                       stats, g, g_stride, dz, B, (int)K);
    return 0;
  });
  if (rc) return rc;
  WXX_LAUNCHED();
  return WXX_OK;
}
