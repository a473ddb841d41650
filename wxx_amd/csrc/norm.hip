// LayerNorm ("meanvarnorm") and RMSNorm, forward and backward, over an
// (outer, reduce, inner) view of a contiguous f32 tensor; gamma/beta are
// indexed by the reduce coordinate.
//
// Reference semantics:
//  * LayerNorm forward (src/wxx/shaders/layers/meanvarnorm.wgsl:29-111,
//    host src/wxx/functional/normalization.py:82-145): single pass
//    mu = S/n, var = max(0, Q/n - mu^2), inv_std = var > 0 ? rsqrt(var+eps)
//    : 0, y = (x - mu) * inv_std * g + b; eps = 1e-5; saves mu and inv_std.
//  * LayerNorm dx (meanvarnormdx.wgsl:21-90): c1 = mean(g dy),
//    c2 = mean(g dy xhat), dx = inv_std (g dy - c1 - xhat c2).
//  * LayerNorm dgamma/dbeta (meanvarnormdg.wgsl:21-70): sums of dy*xhat and
//    dy over every (outer, inner) position.
//  * RMSNorm forward (rmsnorm.wgsl:17-81, normalization.py:24-79):
//    r = ms > 0 ? rsqrt(ms + 1e-6) : 0, y = x r g; saves r.
//  * RMSNorm dx (rmsnormdx.wgsl:17-71): c = r^2/n * sum(g dy x),
//    dx = r (g dy - x c).  RMSNorm dgamma (rmsnormdg.wgsl:15-56): sum dy x r.
//
// The reference launches rows on workgroup_id.y capped at 65 535 with no
// row loop, so rows >= 65 535 of the forward passes and of LayerNorm dx are
// never written (they read back as zeros from a fresh buffer).  `row_cap`
// reproduces that on request (0 = compute every row, the default).
//
// MI355X design: one wave (R <= 2048) or one workgroup (R <= 16384) per row,
// the row held in VGPRs so x is read from HBM once; gamma/dbeta reductions
// use a column-parallel partial pass plus a deterministic split-order sum
// instead of the reference's one-workgroup-per-feature serial loop.
#include "rows.h"

namespace {

constexpr int kBlock = 256;

// MODE 0 = LayerNorm, 1 = RMSNorm.
template <int MODE, int TPR, int NCH, bool VEC>
__global__ __launch_bounds__(256) void norm_fwd_rows_kernel(
    const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ b,
    float* __restrict__ y, float* __restrict__ mean, float* __restrict__ inv, int64_t rows,
    int R, float eps, int64_t row_cap) {
  __shared__ float red[4];
  constexpr int RPB = 256 / TPR;
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  if (TPR == 64 && row >= rows) return;
  wxx::RowRegs<TPR, NCH, VEC> v;
  v.load(x + row * R, R, t, 0.f);
  float s = 0.f, q = 0.f;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) {
    if (MODE == 0) s += v.v[e];
    q += v.v[e] * v.v[e];
  }
  const float n = (float)R;
  float mu = 0.f, istd;
  if (MODE == 0) {
    s = wxx::RowReduce<TPR>::sum(s, red);
    q = wxx::RowReduce<TPR>::sum(q, red);
    mu = s / n;
    const float var = fmaxf(0.f, q / n - mu * mu);
    istd = var > 0.f ? rsqrtf(var + eps) : 0.f;
  } else {
    q = wxx::RowReduce<TPR>::sum(q, red);
    const float ms = q / n;
    istd = ms > 0.f ? rsqrtf(ms + eps) : 0.f;
  }
  const bool capped = row_cap > 0 && row >= row_cap;
  wxx::RowRegs<TPR, NCH, VEC> gg;
  gg.load(g, R, t, 0.f);
  if (MODE == 0) {
    wxx::RowRegs<TPR, NCH, VEC> bb;
    bb.load(b, R, t, 0.f);
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e)
      v.v[e] = capped ? 0.f : (v.v[e] - mu) * istd * gg.v[e] + bb.v[e];
  } else {
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e) v.v[e] = capped ? 0.f : v.v[e] * istd * gg.v[e];
  }
  v.store(y + row * R, R, t);
  if (t == 0) {
    if (MODE == 0) mean[row] = capped ? 0.f : mu;
    inv[row] = capped ? 0.f : istd;
  }
}

template <int MODE, int TPR, int NCH, bool VEC>
__global__ __launch_bounds__(256) void norm_dx_rows_kernel(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ g,
    const float* __restrict__ mean, const float* __restrict__ inv, float* __restrict__ dx,
    int64_t rows, int R, int64_t row_cap) {
  __shared__ float red[4];
  constexpr int RPB = 256 / TPR;
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  if (TPR == 64 && row >= rows) return;
  wxx::RowRegs<TPR, NCH, VEC> vd, vx, gg;
  vd.load(dy + row * R, R, t, 0.f);
  vx.load(x + row * R, R, t, 0.f);
  gg.load(g, R, t, 0.f);
  const float istd = inv[row];
  const float n = (float)R;
  if (MODE == 0) {
    const float mu = mean[row];
    float c1 = 0.f, c2 = 0.f;
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e) {
      const float db = vd.v[e] * gg.v[e];
      vd.v[e] = db;
      vx.v[e] = (vx.v[e] - mu) * istd;  // xhat
      c1 += db;
      c2 += db * vx.v[e];
    }
    c1 = wxx::RowReduce<TPR>::sum(c1, red) / n;
    c2 = wxx::RowReduce<TPR>::sum(c2, red) / n;
    const bool capped = row_cap > 0 && row >= row_cap;
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e)
      vd.v[e] = capped ? 0.f : istd * (vd.v[e] - c1 - vx.v[e] * c2);
  } else {
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e) {
      const float db = vd.v[e] * gg.v[e];
      vd.v[e] = db;
      acc += db * vx.v[e];
    }
    acc = wxx::RowReduce<TPR>::sum(acc, red);
    const float c = (istd * istd / n) * acc;
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e) vd.v[e] = istd * (vd.v[e] - vx.v[e] * c);
  }
  vd.store(dx + row * R, R, t);
}

// ---- generic (outer, R, inner) column kernels: thread per (o, i) ----------
template <int MODE>
__global__ __launch_bounds__(kBlock) void norm_fwd_cols_kernel(
    const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ b,
    float* __restrict__ y, float* __restrict__ mean, float* __restrict__ inv, int64_t outer,
    int64_t R, int64_t inner, float eps, int64_t row_cap) {
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (t >= outer * inner) return;
  const int64_t o = t / inner, i = t - o * inner;
  const float* p = x + o * R * inner + i;
  float* q = y + o * R * inner + i;
  float s = 0.f, ss = 0.f;
  for (int64_t r = 0; r < R; ++r) {
    const float v = p[r * inner];
    s += v;
    ss += v * v;
  }
  const float n = (float)R;
  float mu = 0.f, istd;
  if (MODE == 0) {
    mu = s / n;
    const float var = fmaxf(0.f, ss / n - mu * mu);
    istd = var > 0.f ? rsqrtf(var + eps) : 0.f;
  } else {
    const float ms = ss / n;
    istd = ms > 0.f ? rsqrtf(ms + eps) : 0.f;
  }
  const bool capped = row_cap > 0 && o >= row_cap;
  for (int64_t r = 0; r < R; ++r) {
    const float v = p[r * inner];
    float out = MODE == 0 ? (v - mu) * istd * g[r] + b[r] : v * istd * g[r];
    q[r * inner] = capped ? 0.f : out;
  }
  if (MODE == 0) mean[t] = capped ? 0.f : mu;
  inv[t] = capped ? 0.f : istd;
}

template <int MODE>
__global__ __launch_bounds__(kBlock) void norm_dx_cols_kernel(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ g,
    const float* __restrict__ mean, const float* __restrict__ inv, float* __restrict__ dx,
    int64_t outer, int64_t R, int64_t inner, int64_t row_cap) {
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (t >= outer * inner) return;
  const int64_t o = t / inner, i = t - o * inner;
  const int64_t base = o * R * inner + i;
  const float istd = inv[t];
  const float n = (float)R;
  if (MODE == 0) {
    const float mu = mean[t];
    float c1 = 0.f, c2 = 0.f;
    for (int64_t r = 0; r < R; ++r) {
      const float db = dy[base + r * inner] * g[r];
      c1 += db;
      c2 += db * (x[base + r * inner] - mu) * istd;
    }
    c1 /= n;
    c2 /= n;
    const bool capped = row_cap > 0 && o >= row_cap;
    for (int64_t r = 0; r < R; ++r) {
      const float db = dy[base + r * inner] * g[r];
      const float xh = (x[base + r * inner] - mu) * istd;
      dx[base + r * inner] = capped ? 0.f : istd * (db - c1 - xh * c2);
    }
  } else {
    float acc = 0.f;
    for (int64_t r = 0; r < R; ++r) acc += dy[base + r * inner] * g[r] * x[base + r * inner];
    const float c = (istd * istd / n) * acc;
    for (int64_t r = 0; r < R; ++r) {
      const float db = dy[base + r * inner] * g[r];
      dx[base + r * inner] = istd * (db - x[base + r * inner] * c);
    }
  }
}

// ---- dgamma / dbeta: partial column sums + split-order finalize ----------
// Thread per (feature r, split); the split walks its share of the
// (outer, inner) positions.  part layout: [split][2][R] (dgamma then dbeta).
template <int MODE>
__global__ __launch_bounds__(kBlock) void norm_dg_partial_kernel(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ inv, float* __restrict__ part, int64_t outer, int64_t R,
    int64_t inner, int64_t seg) {
  const int64_t r = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int split = blockIdx.y;
  if (r >= R) return;
  const int64_t p0 = (int64_t)split * seg;
  int64_t p1 = p0 + seg;
  const int64_t npos = outer * inner;
  if (p1 > npos) p1 = npos;
  float dg = 0.f, db = 0.f;
  if (inner == 1) {
    for (int64_t o = p0; o < p1; ++o) {
      const float d = dy[o * R + r];
      const float xv = x[o * R + r];
      if (MODE == 0) {
        dg += d * (xv - mean[o]) * inv[o];
        db += d;
      } else {
        dg += d * xv * inv[o];
      }
    }
  } else {
    for (int64_t p = p0; p < p1; ++p) {
      const int64_t o = p / inner, i = p - o * inner;
      const int64_t idx = o * R * inner + r * inner + i;
      const float d = dy[idx];
      if (MODE == 0) {
        dg += d * (x[idx] - mean[p]) * inv[p];
        db += d;
      } else {
        dg += d * x[idx] * inv[p];
      }
    }
  }
  part[((int64_t)split * 2 + 0) * R + r] = dg;
  if (MODE == 0) part[((int64_t)split * 2 + 1) * R + r] = db;
}

// 64 features per workgroup: lane c of wave w adds splits w, w + 4, ... of
// feature r (consecutive lanes read consecutive features), then the four
// wave sums are added in wave order (a fixed order: deterministic).
template <int MODE>
__global__ __launch_bounds__(kBlock) void norm_dg_finalize_kernel(const float* __restrict__ part,
                                                                  float* __restrict__ dgamma,
                                                                  float* __restrict__ dbeta,
                                                                  int64_t R, int splits) {
  __shared__ float sg[4][64], sb[4][64];
  const int c = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.x * 64 + c;
  float dg = 0.f, db = 0.f;
  if (r < R) {
    for (int s = w; s < splits; s += 4) {
      dg += part[((int64_t)s * 2 + 0) * R + r];
      if (MODE == 0) db += part[((int64_t)s * 2 + 1) * R + r];
    }
  }
  sg[w][c] = dg;
  sb[w][c] = db;
  __syncthreads();
  if (w == 0 && r < R) {
    dgamma[r] = ((sg[0][c] + sg[1][c]) + sg[2][c]) + sg[3][c];
    if (MODE == 0) dbeta[r] = ((sb[0][c] + sb[1][c]) + sb[2][c]) + sb[3][c];
  }
}

// Middle level for many splits: workgroup (f, gi) adds splits
// [gi * chunk, (gi + 1) * chunk) of 64 features in the finalize kernel's
// order and writes one partial in the same layout, so the finalize kernel
// then adds ceil(splits / chunk) partials instead of every split.
template <int MODE>
__global__ __launch_bounds__(kBlock) void norm_dg_combine_kernel(const float* __restrict__ part,
                                                                 float* __restrict__ out,
                                                                 int64_t R, int splits, int chunk) {
  __shared__ float sg[4][64], sb[4][64];
  const int c = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.x * 64 + c;
  const int s0 = blockIdx.y * chunk, s1 = min(splits, s0 + chunk);
  float dg = 0.f, db = 0.f;
  if (r < R) {
    for (int s = s0 + w; s < s1; s += 4) {
      dg += part[((int64_t)s * 2 + 0) * R + r];
      if (MODE == 0) db += part[((int64_t)s * 2 + 1) * R + r];
    }
  }
  sg[w][c] = dg;
  sb[w][c] = db;
  __syncthreads();
  if (w == 0 && r < R) {
    out[((int64_t)blockIdx.y * 2 + 0) * R + r] = ((sg[0][c] + sg[1][c]) + sg[2][c]) + sg[3][c];
    if (MODE == 0)
      out[((int64_t)blockIdx.y * 2 + 1) * R + r] = ((sb[0][c] + sb[1][c]) + sb[2][c]) + sb[3][c];
  }
}

template <int MODE>
int launch_fwd(const float* x, const float* g, const float* b, float* y, float* mean,
               float* inv, int64_t outer, int64_t R, int64_t inner, float eps,
               int64_t row_cap) {
  hipStream_t s = wxx::stream();
  if (inner == 1 && wxx::row_plan(R) != 0) {
    const bool vec = (R % 4 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0) &&
                     ((uintptr_t)g % 16 == 0) && (MODE == 1 || (uintptr_t)b % 16 == 0);
    int rc = wxx::row_dispatch(R, vec, [&](auto tpr, auto nch, auto v) {
      hipLaunchKernelGGL((norm_fwd_rows_kernel<MODE, decltype(tpr)::value, decltype(nch)::value,
                                               decltype(v)::value>),
                         wxx::row_grid(decltype(tpr)::value, outer), dim3(256), 0, s, x, g, b, y,
                         mean, inv, outer, (int)R, eps, row_cap);
      return 0;
    });
    if (rc) return rc;
  } else {
    hipLaunchKernelGGL(norm_fwd_cols_kernel<MODE>, dim3(wxx::grid_1d(outer * inner, kBlock)),
                       dim3(kBlock), 0, s, x, g, b, y, mean, inv, outer, R, inner, eps, row_cap);
  }
  WXX_LAUNCHED();
  return WXX_OK;
}

template <int MODE>
int launch_dx(const float* dy, const float* x, const float* g, const float* mean,
              const float* inv, float* dx, int64_t outer, int64_t R, int64_t inner,
              int64_t row_cap) {
  hipStream_t s = wxx::stream();
  if (inner == 1 && wxx::row_plan(R) != 0) {
    const bool vec = (R % 4 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)dy % 16 == 0) &&
                     ((uintptr_t)dx % 16 == 0) && ((uintptr_t)g % 16 == 0);
    int rc = wxx::row_dispatch(R, vec, [&](auto tpr, auto nch, auto v) {
      hipLaunchKernelGGL((norm_dx_rows_kernel<MODE, decltype(tpr)::value, decltype(nch)::value,
                                              decltype(v)::value>),
                         wxx::row_grid(decltype(tpr)::value, outer), dim3(256), 0, s, dy, x, g,
                         mean, inv, dx, outer, (int)R, row_cap);
      return 0;
    });
    if (rc) return rc;
  } else {
    hipLaunchKernelGGL(norm_dx_cols_kernel<MODE>, dim3(wxx::grid_1d(outer * inner, kBlock)),
                       dim3(kBlock), 0, s, dy, x, g, mean, inv, dx, outer, R, inner, row_cap);
  }
  WXX_LAUNCHED();
  return WXX_OK;
}

template <int MODE>
int launch_dg(const float* dy, const float* x, const float* mean, const float* inv,
              float* dgamma, float* dbeta, int64_t outer, int64_t R, int64_t inner) {
  hipStream_t s = wxx::stream();
  const int64_t npos = outer * inner;
  const int64_t colblocks = (R + kBlock - 1) / kBlock;
  const int64_t target = (int64_t)wxx::num_cus() * 8;
  int64_t splits = std::max<int64_t>(1, (target + colblocks - 1) / colblocks);
  splits = std::min<int64_t>(splits, std::max<int64_t>(1, npos / 16));
  splits = std::min<int64_t>(splits, 4096);
  const int64_t seg = (npos + splits - 1) / splits;
  float* part = (float*)wxx::scratch_alloc(sizeof(float) * 2 * R * splits);
  if (!part) return wxx::set_error(WXX_E_OOM, "norm dg partials");
  hipLaunchKernelGGL(norm_dg_partial_kernel<MODE>, dim3((unsigned)colblocks, (unsigned)splits),
                     dim3(kBlock), 0, s, dy, x, mean, inv, part, outer, R, inner, seg);
  WXX_LAUNCHED();
  const float* fin = part;
  int64_t nfin = splits;
  float* part2 = nullptr;
  constexpr int64_t kChunk = 32;
  if (splits > 2 * kChunk) {
    nfin = (splits + kChunk - 1) / kChunk;
    part2 = (float*)wxx::scratch_alloc(sizeof(float) * 2 * R * nfin);
    if (!part2) {
      wxx::scratch_free(part);
      return wxx::set_error(WXX_E_OOM, "norm dg partials");
    }
    hipLaunchKernelGGL(norm_dg_combine_kernel<MODE>, dim3((unsigned)((R + 63) / 64), (unsigned)nfin),
                       dim3(kBlock), 0, s, (const float*)part, part2, R, (int)splits, (int)kChunk);
    WXX_LAUNCHED();
    fin = part2;
  }
  hipLaunchKernelGGL(norm_dg_finalize_kernel<MODE>, dim3((unsigned)((R + 63) / 64)), dim3(kBlock),
                     0, s, fin, dgamma, dbeta, R, (int)nfin);
  WXX_LAUNCHED();
  wxx::scratch_free(part);
  if (part2) wxx::scratch_free(part2);
  return WXX_OK;
}

}  // namespace

// Replaces functional.meanvarnorm (reference src/wxx/functional/normalization.py:82-145).
WXX_API int wxx_meanvarnorm(const float* x, const float* gamma, const float* beta, float* y,
                            float* mean, float* inv_std, int64_t outer, int64_t reduce,
                            int64_t inner, float eps, int64_t row_cap) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && gamma && beta && y && mean && inv_std, "null pointer");
  WXX_REQUIRE(outer >= 0 && reduce >= 1 && inner >= 1, "bad dims");
  if (outer == 0) return WXX_OK;
  return launch_fwd<0>(x, gamma, beta, y, mean, inv_std, outer, reduce, inner, eps, row_cap);
}

// Replaces functional.meanvarnormdx (reference normalization.py:308-359).
WXX_API int wxx_meanvarnormdx(const float* dy, const float* x, const float* gamma,
                              const float* mean, const float* inv_std, float* dx, int64_t outer,
                              int64_t reduce, int64_t inner, int64_t row_cap) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && x && gamma && mean && inv_std && dx, "null pointer");
  WXX_REQUIRE(outer >= 0 && reduce >= 1 && inner >= 1, "bad dims");
  if (outer == 0) return WXX_OK;
  return launch_dx<0>(dy, x, gamma, mean, inv_std, dx, outer, reduce, inner, row_cap);
}

// Replaces functional.meanvarnormdg (reference normalization.py:362-412).
WXX_API int wxx_meanvarnormdg(const float* dy, const float* x, const float* mean,
                              const float* inv_std, float* dgamma, float* dbeta, int64_t outer,
                              int64_t reduce, int64_t inner) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && x && mean && inv_std && dgamma && dbeta, "null pointer");
  WXX_REQUIRE(outer >= 0 && reduce >= 1 && inner >= 1, "bad dims");
  if (outer * inner == 0) {
    int rc = wxx_fill_u32(dgamma, reduce, 0u);
    return rc ? rc : wxx_fill_u32(dbeta, reduce, 0u);
  }
  return launch_dg<0>(dy, x, mean, inv_std, dgamma, dbeta, outer, reduce, inner);
}

// Replaces functional.rmsnorm (reference normalization.py:24-79).
WXX_API int wxx_rmsnorm(const float* x, const float* gamma, float* y, float* inv_rms,
                        int64_t outer, int64_t reduce, int64_t inner, float eps,
                        int64_t row_cap) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && gamma && y && inv_rms, "null pointer");
  WXX_REQUIRE(outer >= 0 && reduce >= 1 && inner >= 1, "bad dims");
  if (outer == 0) return WXX_OK;
  return launch_fwd<1>(x, gamma, nullptr, y, nullptr, inv_rms, outer, reduce, inner, eps,
                       row_cap);
}

// Replaces functional.rmsnormdx (reference normalization.py:415-463).
WXX_API int wxx_rmsnormdx(const float* dy, const float* x, const float* gamma,
                          const float* inv_rms, float* dx, int64_t outer, int64_t reduce,
                          int64_t inner) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && x && gamma && inv_rms && dx, "null pointer");
  WXX_REQUIRE(outer >= 0 && reduce >= 1 && inner >= 1, "bad dims");
  if (outer == 0) return WXX_OK;
  return launch_dx<1>(dy, x, gamma, nullptr, inv_rms, dx, outer, reduce, inner, 0);
}

// Replaces functional.rmsnormdg (reference normalization.py:466-513).
WXX_API int wxx_rmsnormdg(const float* dy, const float* x, const float* inv_rms,
                          float* dgamma, int64_t outer, int64_t reduce, int64_t inner) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && x && inv_rms && dgamma, "null pointer");
  WXX_REQUIRE(outer >= 0 && reduce >= 1 && inner >= 1, "bad dims");
  if (outer * inner == 0) return wxx_fill_u32(dgamma, reduce, 0u);
  return launch_dg<1>(dy, x, nullptr, inv_rms, dgamma, nullptr, outer, reduce, inner);
}
