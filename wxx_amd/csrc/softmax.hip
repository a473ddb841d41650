// Softmax along one axis of a contiguous f32 tensor viewed as
// (outer, C, inner).
//
// Reference semantics (src/wxx/shaders/activations/softmax.wgsl:25-77,
// host src/wxx/functional/activations.py:126-173): m = max(-1e38, max_c x),
// s = sum_c exp(x - m), y = exp(x - m) * (1 / s).
//
// MI355X design: the reference runs one thread per row with three serial,
// uncoalesced passes.  Here a row (inner == 1) lives in VGPRs of one wave
// (C <= 2048) or one workgroup (C <= 16384): one HBM read, one HBM write,
// wave-shuffle reductions.  Longer rows use an online (max, sum) pass and a
// write pass.  inner > 1 gives each thread one column so lanes read
// consecutive addresses.
#include "rows.h"

namespace {

// PRE: the row is first mapped x -> x * scale + mask row (row % mask_rows),
// mask rows mask_ld floats apart (the
// attention score scaling and additive mask), with the two roundings of the
// separate multiply and add kept (no fused multiply-add).
//
// CAUSAL (with PRE; mask_rows = the diagonal's period S): the mask is GPT-2's
// causal mask, 0 on and below the diagonal and -1e9 above it, so row
// i = row % S reads only columns j <= i (x * scale + 0 there) and the others
// are probability exactly 0 (exp(-1e9 - m) underflows), as in the masked
// computation.  CAUSAL 1 writes those zeros; CAUSAL 2 leaves them unwritten
// for consumers that read only the lower triangle.
template <int TPR, int NCH, bool VEC, bool PRE = false, int CAUSAL = 0>
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* __restrict__ x,
                                                            float* __restrict__ y, int64_t rows,
                                                            int C,
                                                            const float* __restrict__ mask = nullptr,
                                                            int64_t mask_rows = 1,
                                                            int64_t mask_ld = 0,
                                                            float scale = 1.f) {
  __shared__ float red[4];
  constexpr int RPB = 256 / TPR;
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  if (TPR == 64 && row >= rows) return;
  const float* xr = x + row * C;
  wxx::RowRegs<TPR, NCH, VEC> r;
  const int lim = CAUSAL ? (int)min<int64_t>(C, row % mask_rows + 1) : C;
  if (CAUSAL)
    r.load_lim(xr, lim, t, -INFINITY);
  else
    r.load(xr, C, t, -INFINITY);
  if (PRE && CAUSAL) {
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e)
      if (r.valid(e, t, lim)) r.v[e] = __fadd_rn(__fmul_rn(r.v[e], scale), 0.f);
  } else if (PRE) {
    wxx::RowRegs<TPR, NCH, VEC> mk;
    if (mask) mk.load(mask + (row % mask_rows) * mask_ld, C, t, 0.f);
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e)
      if (r.valid(e, t, C))
        r.v[e] = __fadd_rn(__fmul_rn(r.v[e], scale), mask ? mk.v[e] : 0.f);
  }
  float m = -1e38f;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) m = fmaxf(m, r.v[e]);
  m = wxx::RowReduce<TPR>::max(m, red);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) {
    float ev = r.valid(e, t, C) ? expf(r.v[e] - m) : 0.f;
    r.v[e] = ev;
    s += ev;
  }
  s = wxx::RowReduce<TPR>::sum(s, red);
  const float inv = 1.0f / s;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) r.v[e] *= inv;
  if (CAUSAL == 2)
    r.store_lim(y + row * C, lim, t);
  else
    r.store(y + row * C, C, t);
}

// Rows longer than 16384: online max/sum in one pass, then a write pass.
__global__ __launch_bounds__(256) void softmax_rows_looped_kernel(const float* __restrict__ x,
                                                                   float* __restrict__ y,
                                                                   int64_t C) {
  __shared__ float sm[4], ss[4];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * C;
  float m = -1e38f, s = 0.f;
  for (int64_t c = threadIdx.x; c < C; c += 256) {
    float v = xr[c];
    if (v > m) {
      s = s * expf(m - v) + 1.f;
      m = v;
    } else {
      s += expf(v - m);
    }
  }
  // Combine (m, s) pairs: first within the wave, then across the 4 waves.
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    float om = __shfl_xor(m, off, 64), os = __shfl_xor(s, off, 64);
    float nm = fmaxf(m, om);
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
  const float inv = 1.0f / S;
  float* yr = y + row * C;
  for (int64_t c = threadIdx.x; c < C; c += 256) yr[c] = expf(xr[c] - M) * inv;
}

// inner > 1: thread per (outer, inner) column, three passes over C.
__global__ __launch_bounds__(256) void softmax_cols_kernel(const float* __restrict__ x,
                                                            float* __restrict__ y, int64_t outer,
                                                            int64_t C, int64_t inner) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= outer * inner) return;
  const int64_t o = t / inner, i = t - o * inner;
  const float* p = x + o * C * inner + i;
  float* q = y + o * C * inner + i;
  float m = -1e38f;
  for (int64_t c = 0; c < C; ++c) m = fmaxf(m, p[c * inner]);
  float s = 0.f;
  for (int64_t c = 0; c < C; ++c) s += expf(p[c * inner] - m);
  const float inv = 1.0f / s;
  for (int64_t c = 0; c < C; ++c) q[c * inner] = expf(p[c * inner] - m) * inv;
}

// dx = y * (g - sum(g * y)) per row: one read of y and g, one write.
// SCALED: dx is further multiplied by `scale` (the gradient through the
// score scaling), as a separate rounding.
// CAUSAL (rows of period diag): y is zero above the diagonal, so row
// i = row % diag reads y and g for columns j <= i only (the dot product is
// the same: the other terms are exact zeros); CAUSAL 1 writes dx = 0 above
// the diagonal, CAUSAL 2 leaves it unwritten.
template <int TPR, int NCH, bool VEC, bool SCALED = false, int CAUSAL = 0>
__global__ __launch_bounds__(256) void softmax_bwd_rows_kernel(const float* __restrict__ y,
                                                                const float* __restrict__ g,
                                                                float* __restrict__ dx,
                                                                int64_t rows, int C,
                                                                float scale = 1.f,
                                                                int64_t diag = 1) {
  __shared__ float red[4];
  constexpr int RPB = 256 / TPR;
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  if (TPR == 64 && row >= rows) return;
  wxx::RowRegs<TPR, NCH, VEC> vy, vg;
  const int lim = CAUSAL ? (int)min<int64_t>(C, row % diag + 1) : C;
  if (CAUSAL) {
    vy.load_lim(y + row * C, lim, t, 0.f);
    vg.load_lim(g + row * C, lim, t, 0.f);
  } else {
    vy.load(y + row * C, C, t, 0.f);
    vg.load(g + row * C, C, t, 0.f);
  }
  float dot = 0.f;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) dot += vg.v[e] * vy.v[e];
  dot = wxx::RowReduce<TPR>::sum(dot, red);
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) {
    vy.v[e] = vy.v[e] * (vg.v[e] - dot);
    if (SCALED) vy.v[e] = __fmul_rn(vy.v[e], scale);
  }
  if (CAUSAL == 2)
    vy.store_lim(dx + row * C, lim, t);
  else
    vy.store(dx + row * C, C, t);
}

__global__ __launch_bounds__(256) void softmax_bwd_cols_kernel(const float* __restrict__ y,
                                                                const float* __restrict__ g,
                                                                float* __restrict__ dx,
                                                                int64_t outer, int64_t C,
                                                                int64_t inner) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= outer * inner) return;
  const int64_t o = t / inner, i = t - o * inner;
  const int64_t base = o * C * inner + i;
  float dot = 0.f;
  for (int64_t c = 0; c < C; ++c) dot += g[base + c * inner] * y[base + c * inner];
  for (int64_t c = 0; c < C; ++c)
    dx[base + c * inner] = y[base + c * inner] * (g[base + c * inner] - dot);
}

}  // namespace

// Softmax backward dx = y * (g - sum_c g y) along C.  Replaces the composite
// multiply / sum / unsqueeze / subtract / multiply chain of reference
// src/wxx/autograd/reductions.py:25-35.
WXX_API int wxx_softmax_backward(const float* y, const float* g, float* dx, int64_t outer,
                                 int64_t C, int64_t inner) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(y && g && dx, "null pointer");
  WXX_REQUIRE(outer >= 0 && C >= 1 && inner >= 1, "bad softmax dims");
  if (outer == 0) return WXX_OK;
  hipStream_t s = wxx::stream();
  if (inner == 1 && wxx::row_plan(C) != 0) {
    const bool vec = (C % 4 == 0) && ((((uintptr_t)y) | ((uintptr_t)g) | ((uintptr_t)dx)) % 16 == 0);
    int rc = wxx::row_dispatch(C, vec, [&](auto tpr, auto nch, auto v) {
      hipLaunchKernelGGL((softmax_bwd_rows_kernel<decltype(tpr)::value, decltype(nch)::value,
                                                  decltype(v)::value>),
                         wxx::row_grid(decltype(tpr)::value, outer), dim3(256), 0, s, y, g, dx,
                         outer, (int)C);
      return 0;
    });
    if (rc) return rc;
  } else {
    hipLaunchKernelGGL(softmax_bwd_cols_kernel, dim3(wxx::grid_1d(outer * inner, 256)), dim3(256),
                       0, s, y, g, dx, outer, C, inner);
  }
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.softmax (reference src/wxx/functional/activations.py:126-173).
WXX_API int wxx_softmax(const float* x, float* y, int64_t outer, int64_t C, int64_t inner) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && y, "null pointer");
  WXX_REQUIRE(outer >= 0 && C >= 1 && inner >= 1, "bad softmax dims");
  if (outer == 0) return WXX_OK;
  hipStream_t s = wxx::stream();
  if (inner == 1) {
    const bool vec = (C % 4 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0);
    if (wxx::row_plan(C) == 0) {
      hipLaunchKernelGGL(softmax_rows_looped_kernel, dim3((unsigned)outer), dim3(256), 0, s, x,
                         y, C);
    } else {
      int rc = wxx::row_dispatch(C, vec, [&](auto tpr, auto nch, auto v) {
        hipLaunchKernelGGL((softmax_rows_kernel<decltype(tpr)::value, decltype(nch)::value,
                                                decltype(v)::value>),
                           wxx::row_grid(decltype(tpr)::value, outer), dim3(256), 0, s, x, y,
                           outer, (int)C);
        return 0;
      });
      if (rc) return rc;
    }
    WXX_LAUNCHED();
    return WXX_OK;
  }
  hipLaunchKernelGGL(softmax_cols_kernel, dim3(wxx::grid_1d(outer * inner, 256)), dim3(256), 0,
                     s, x, y, outer, C, inner);
  WXX_LAUNCHED();
  return WXX_OK;
}

// y = softmax along rows of (x * scale + mask[row % mask_rows]); mask may be
// null, its rows are mask_ld floats apart.  The score path of MultiHeadAttention (reference
// src/wxx/nn/module.py:478-483: matmul * (1/sqrt(d_head)), + mask, softmax)
// in one pass over the scores instead of three.  Rows of C <= 16384 only.
WXX_API int wxx_softmax_scale_mask(const float* x, const float* mask, float* y, int64_t rows,
                                   int64_t C, int64_t mask_rows, int64_t mask_ld, float scale) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && y, "null pointer");
  WXX_REQUIRE(rows >= 0 && C >= 1 && (!mask || (mask_rows >= 1 && mask_ld >= C)),
              "bad softmax dims");
  if (wxx::row_plan(C) == 0)
    return wxx::set_error(WXX_E_UNSUPPORTED, "fused softmax rows of %lld", (long long)C);
  if (rows == 0) return WXX_OK;
  hipStream_t s = wxx::stream();
  const bool vec = (C % 4 == 0) && (mask_ld % 4 == 0) &&
                   ((((uintptr_t)x) | ((uintptr_t)y) | ((uintptr_t)mask)) % 16 == 0);
  int rc = wxx::row_dispatch(C, vec, [&](auto tpr, auto nch, auto v) {
    hipLaunchKernelGGL((softmax_rows_kernel<decltype(tpr)::value, decltype(nch)::value,
                                            decltype(v)::value, true>),
                       wxx::row_grid(decltype(tpr)::value, rows), dim3(256), 0, s, x, y, rows,
                       (int)C, mask, mask ? mask_rows : 1, mask ? mask_ld : 0, scale);
    return 0;
  });
  if (rc) return rc;
  WXX_LAUNCHED();
  return WXX_OK;
}

// dx = scale * (y * (g - sum(g * y))) along rows: the softmax gradient of
// wxx_softmax_scale_mask (the mask adds nothing to the gradient).  Rows of
// C <= 16384 only.
WXX_API int wxx_softmax_backward_scale(const float* y, const float* g, float* dx, int64_t rows,
                                       int64_t C, float scale) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(y && g && dx, "null pointer");
  WXX_REQUIRE(rows >= 0 && C >= 1, "bad softmax dims");
  if (wxx::row_plan(C) == 0)
    return wxx::set_error(WXX_E_UNSUPPORTED, "fused softmax rows of %lld", (long long)C);
  if (rows == 0) return WXX_OK;
  hipStream_t s = wxx::stream();
  const bool vec = (C % 4 == 0) && ((((uintptr_t)y) | ((uintptr_t)g) | ((uintptr_t)dx)) % 16 == 0);
  int rc = wxx::row_dispatch(C, vec, [&](auto tpr, auto nch, auto v) {
    hipLaunchKernelGGL((softmax_bwd_rows_kernel<decltype(tpr)::value, decltype(nch)::value,
                                                decltype(v)::value, true>),
                       wxx::row_grid(decltype(tpr)::value, rows), dim3(256), 0, s, y, g, dx, rows,
                       (int)C, scale);
    return 0;
  });
  if (rc) return rc;
  WXX_LAUNCHED();
  return WXX_OK;
}

// Causal attention softmax (no counterpart in the reference: its masked
// path with GPT-2's causal mask, -1e9 above the diagonal and 0 on and below
// it, nn/gpt.py:75-96 + nn/module.py:478-483).  Rows of x are rows of
// (S x C) score blocks; row i = row % S reads x[.. j <= i] only and gives
// y = softmax(x * scale + 0) there and exactly 0 above the diagonal, the
// same numbers as wxx_softmax_scale_mask with that mask.  skip = 1 leaves
// the zeros above the diagonal unwritten (for consumers that read only the
// lower triangle).
WXX_API int wxx_softmax_causal(const float* x, float* y, int64_t rows, int64_t C, int64_t S,
                               float scale, int skip) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && y, "null pointer");
  WXX_REQUIRE(rows >= 0 && C >= 1 && S >= 1, "bad softmax dims");
  if (wxx::row_plan(C) == 0)
    return wxx::set_error(WXX_E_UNSUPPORTED, "fused softmax rows of %lld", (long long)C);
  if (rows == 0) return WXX_OK;
  hipStream_t s = wxx::stream();
  const bool vec = (C % 4 == 0) && ((((uintptr_t)x) | ((uintptr_t)y)) % 16 == 0);
  int rc = wxx::row_dispatch(C, vec, [&](auto tpr, auto nch, auto v) {
    constexpr int TPR = decltype(tpr)::value, NCH = decltype(nch)::value;
    constexpr bool V = decltype(v)::value;
    if (skip)
      hipLaunchKernelGGL((softmax_rows_kernel<TPR, NCH, V, true, 2>), wxx::row_grid(TPR, rows),
                         dim3(256), 0, s, x, y, rows, (int)C, nullptr, S, 0, scale);
    else
      hipLaunchKernelGGL((softmax_rows_kernel<TPR, NCH, V, true, 1>), wxx::row_grid(TPR, rows),
                         dim3(256), 0, s, x, y, rows, (int)C, nullptr, S, 0, scale);
    return 0;
  });
  if (rc) return rc;
  WXX_LAUNCHED();
  return WXX_OK;
}

// Gradient of wxx_softmax_causal: dx = scale * (y * (g - sum_j<=i g y)) on
// and below the diagonal (row i = row % S), 0 above it (left unwritten when
// skip = 1); y and g are read on and below the diagonal only.
WXX_API int wxx_softmax_backward_causal(const float* y, const float* g, float* dx, int64_t rows,
                                        int64_t C, int64_t S, float scale, int skip) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(y && g && dx, "null pointer");
  WXX_REQUIRE(rows >= 0 && C >= 1 && S >= 1, "bad softmax dims");
  if (wxx::row_plan(C) == 0)
    return wxx::set_error(WXX_E_UNSUPPORTED, "fused softmax rows of %lld", (long long)C);
  if (rows == 0) return WXX_OK;
  hipStream_t s = wxx::stream();
  const bool vec = (C % 4 == 0) && ((((uintptr_t)y) | ((uintptr_t)g) | ((uintptr_t)dx)) % 16 == 0);
  int rc = wxx::row_dispatch(C, vec, [&](auto tpr, auto nch, auto v) {
    constexpr int TPR = decltype(tpr)::value, NCH = decltype(nch)::value;
    constexpr bool V = decltype(v)::value;
    if (skip)
      hipLaunchKernelGGL((softmax_bwd_rows_kernel<TPR, NCH, V, true, 2>),
                         wxx::row_grid(TPR, rows), dim3(256), 0, s, y, g, dx, rows, (int)C, scale,
                         S);
    else
      hipLaunchKernelGGL((softmax_bwd_rows_kernel<TPR, NCH, V, true, 1>),
                         wxx::row_grid(TPR, rows), dim3(256), 0, s, y, g, dx, rows, (int)C, scale,
                         S);
    return 0;
  });
  if (rc) return rc;
  WXX_LAUNCHED();
  return WXX_OK;
}
