// Real FFT / inverse real FFT for lengths n = 2M beyond what one workgroup's
// LDS holds (M > 16384 complex points, n > 32768), as a four-step transform.
//
// Reference: src/wxx/functional/fft.py:484-645, whose multi-pass path takes
// any power-of-two n (one launch per radix-2 stage over the whole row).
//
// With M = M1 * M2, k = k1 + M1 k2 and j = j2 + M2 j1, the length-M DFT is
//     Z[j2 + M2 j1] = sum_k1 W_M1^{j1 k1} ( W_M^{j2 k1} sum_k2 z[k1 + M1 k2] W_M2^{j2 k2} ):
//   A. for every k1, a length-M2 DFT over k2 of the column z[k1 + M1 k2],
//      each output multiplied by W_M^{j2 k1}, stored as Y[k1][j2];
//   C. for every j2, a length-M1 DFT over k1 of Y[.][j2], stored at j2 + M2 j1.
// M1 and M2 are at most 8192, so each small transform lives in one
// workgroup's LDS: a radix-2 Stockham sweep, every pass reading its points
// into registers, a barrier, and writing them back in the next pass's order
// (natural order at the end, no bit reversal).  The real <-> complex step on
// top (z[m] = x[2m] + i x[2m+1] and the even/odd untangle of bins k and M - k)
// runs as its own pass.  Rows are processed in groups that keep the two
// complex scratch arrays within 256 MiB.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxLogL = 13;  // LDS holds 2^13 complex points (64 KiB)

__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}

// exp(sign * 2 pi i * num / den) with the angle reduced exactly first: num
// and den are integers (den a power of two), so num mod den is exact and the
// single rounding left is that of sincospi.
__device__ __forceinline__ float2 root(int64_t num, int64_t den, float sign) {
  const int64_t r = num & (den - 1);
  double s, c;
  sincospi(2.0 * (double)r / (double)den, &s, &c);
  return make_float2((float)c, sign * (float)s);
}

// Input of a step-A transform: column k1 of row r, point k2.
struct RealColumn {  // z[k] = x[2k] + i x[2k+1] of a real row, zero past in_len
  const float* x;
  int64_t row_stride, in_len;
  __device__ float2 load(int64_t r, int64_t k) const {
    const float* p = x + r * row_stride;
    const int64_t t = 2 * k;
    return make_float2(t < in_len ? p[t] : 0.f, t + 1 < in_len ? p[t + 1] : 0.f);
  }
};
struct ComplexColumn {
  const float2* z;
  int64_t row_stride;
  __device__ float2 load(int64_t r, int64_t k) const { return z[r * row_stride + k]; }
};

// One length-L (L = 2^logl) complex DFT per workgroup, in LDS.  Workgroup w
// handles row r = w / per_row and transform s = w % per_row; its point e is
// read at src(r, s * in_s + e * in_e) and its output point j written to
// dst[r * M + s * out_s + j * out_e], multiplied by root(j s * twk, M) when
// twk != 0 (the four-step twiddle W_M^{j2 k1}).
template <class Src>
__global__ __launch_bounds__(kThreads) void dft_lds_kernel(Src src, float2* __restrict__ dst,
                                                           int logl, int64_t per_row,
                                                           int64_t in_s, int64_t in_e,
                                                           int64_t out_s, int64_t out_e,
                                                           int64_t M, int64_t twk, float sign) {
  __shared__ float2 a[1 << kMaxLogL];
  const int64_t L = int64_t(1) << logl;
  const int64_t r = blockIdx.x / per_row, s = blockIdx.x % per_row;
  for (int64_t e = threadIdx.x; e < L; e += kThreads) a[e] = src.load(r, s * in_s + e * in_e);
  __syncthreads();
  const int64_t half = L >> 1;
  for (int p = 0; p < logl; ++p) {
    const int64_t ns = int64_t(1) << p;
    // each thread keeps at most L / 2 / 256 butterflies (16 at L = 8192);
    // fixed trip counts keep them in registers
    constexpr int kMaxB = (1 << kMaxLogL) / 2 / kThreads;
    float2 lo[kMaxB], hi[kMaxB];
#pragma unroll
    for (int c = 0; c < kMaxB; ++c) {
      const int64_t i = threadIdx.x + (int64_t)c * kThreads;
      if (i < half) {
        const int64_t k = i & (ns - 1);
        const float2 w = root(k, 2 * ns, sign);
        const float2 u = a[i], v = cmul(w, a[i + half]);
        lo[c] = make_float2(u.x + v.x, u.y + v.y);
        hi[c] = make_float2(u.x - v.x, u.y - v.y);
      }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kMaxB; ++c) {
      const int64_t i = threadIdx.x + (int64_t)c * kThreads;
      if (i < half) {
        const int64_t k = i & (ns - 1);
        const int64_t o = (i - k) * 2 + k;
        a[o] = lo[c];
        a[o + ns] = hi[c];
      }
    }
    __syncthreads();
  }
  float2* d = dst + r * M + s * out_s;
  for (int64_t j = threadIdx.x; j < L; j += kThreads) {
    float2 v = a[j];
    if (twk) v = cmul(v, root(j * s * twk, M, sign));
    d[j * out_e] = v;
  }
}

// Forward untangle: Z (rows x M, the DFT of z) -> X (rows x (M + 1)):
// X[k] = (Z[k] + conj Z[M-k]) / 2 - i W_n^k (Z[k] - conj Z[M-k]) / 2, Z[M] = Z[0].
__global__ __launch_bounds__(kThreads) void untangle_kernel(const float2* __restrict__ Z,
                                                            float2* __restrict__ X, int64_t rows,
                                                            int64_t M) {
  const int64_t per = M + 1, n = rows * per;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / per, k = i - r * per;
    const float2 a = Z[r * M + (k == M ? 0 : k)];
    const float2 b = Z[r * M + (k == 0 ? 0 : M - k)];
    const float2 e = make_float2(0.5f * (a.x + b.x), 0.5f * (a.y - b.y));
    const float2 o = make_float2(0.5f * (a.y + b.y), -0.5f * (a.x - b.x));  // (a - conj b) / 2i
    const float2 w = root(k, 2 * M, -1.f);
    const float2 wo = cmul(w, o);
    X[i] = make_float2(e.x + wo.x, e.y + wo.y);
  }
}

// Inverse untangle: one-sided X (rows x in_len, zero past in_len) -> Z (rows
// x M) with Z[k] = E[k] + i O[k], E = (X[k] + conj X[M-k]) / 2,
// O = (X[k] - conj X[M-k]) W_n^{-k} / 2; the imaginary parts of bins 0 and M
// do not reach the real output and are dropped.
__global__ __launch_bounds__(kThreads) void untangle_inv_kernel(const float2* __restrict__ X,
                                                                float2* __restrict__ Z,
                                                                int64_t rows, int64_t in_len,
                                                                int64_t M) {
  const int64_t n = rows * M;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / M, k = i - r * M;
    const float2* xr = X + r * in_len;
    float2 a = k < in_len ? xr[k] : make_float2(0.f, 0.f);
    float2 b = (M - k) < in_len ? xr[M - k] : make_float2(0.f, 0.f);
    if (k == 0) {
      a.y = 0.f;
      b.y = 0.f;
    }
    const float2 e = make_float2(0.5f * (a.x + b.x), 0.5f * (a.y - b.y));
    const float2 d = make_float2(0.5f * (a.x - b.x), 0.5f * (a.y + b.y));
    const float2 o = cmul(d, root(k, 2 * M, 1.f));
    Z[i] = make_float2(e.x - o.y, e.y + o.x);
  }
}

// z (rows x M complex: M times the samples, x[2m] + i x[2m+1], of the
// unnormalised inverse DFT of the untangled spectrum, whose halves already
// carry the 1/2 of the untangle) -> the first out_len real samples of each
// row, each times scale = 1/M and then times post (two roundings, as a
// separate scaling pass would give).
__global__ __launch_bounds__(kThreads) void unpack_real_kernel(const float2* __restrict__ z,
                                                               float* __restrict__ x, int64_t rows,
                                                               int64_t M, int64_t out_len,
                                                               float scale, float post) {
  const int64_t n = rows * out_len;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / out_len, t = i - r * out_len;
    const float2 v = z[r * M + (t >> 1)];
    float s = ((t & 1) ? v.y : v.x) * scale;
    if (post != 1.f) s *= post;
    x[i] = s;
  }
}

inline unsigned grid(int64_t n) { return wxx::grid_1d(n, kThreads, 65536); }

// the two factors of 2^logm, each at most 2^kMaxLogL
inline void split(int logm, int* l1, int* l2) {
  *l1 = logm / 2;
  *l2 = logm - *l1;
}

// rows per group so that two rows x M complex arrays stay within 256 MiB
inline int64_t group_rows(int64_t rows, int64_t M) {
  const int64_t per = std::max<int64_t>(1, (int64_t(256) << 20) / (16 * M));
  return std::min(rows, per);
}

template <class Src>
int four_step(Src src, float2* y, float2* out, int64_t rows, int logm, float sign) {
  int l1, l2;
  split(logm, &l1, &l2);
  const int64_t M = int64_t(1) << logm, M1 = int64_t(1) << l1, M2 = int64_t(1) << l2;
  hipStream_t st = wxx::stream();
  // A: M1 columns (stride M1) of M2 points -> Y[k1][j2] * W_M^{j2 k1}
  hipLaunchKernelGGL((dft_lds_kernel<Src>), dim3((unsigned)(rows * M1)), dim3(kThreads), 0, st,
                     src, y, l2, M1, int64_t(1), M1, M2, int64_t(1), M, int64_t(1), sign);
  // C: M2 columns (stride M2) of Y, M1 points each -> out[j2 + M2 j1]
  hipLaunchKernelGGL((dft_lds_kernel<ComplexColumn>), dim3((unsigned)(rows * M2)),
                     dim3(kThreads), 0, st, ComplexColumn{y, M}, out, l1, M2, int64_t(1), M2,
                     int64_t(1), M2, M, int64_t(0), sign);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return wxx::set_error(WXX_E_HIP, "four-step FFT: %s", hipGetErrorString(e));
  return WXX_OK;
}

}  // namespace

namespace wxx {

int rfft_four_step(const float* x, float2* X, int64_t rows, int64_t in_len, int logm) {
  if (logm > 2 * kMaxLogL)
    return set_error(WXX_E_UNSUPPORTED, "rfft length 2^%d above 2^%d", logm + 1,
                     2 * kMaxLogL + 1);
  const int64_t M = int64_t(1) << logm;
  const int64_t g = group_rows(rows, M);
  float2* y = (float2*)scratch_alloc(sizeof(float2) * g * M);
  float2* z = (float2*)scratch_alloc(sizeof(float2) * g * M);
  int rc = (y && z) ? WXX_OK : set_error(WXX_E_OOM, "four-step FFT scratch");
  for (int64_t r0 = 0; rc == WXX_OK && r0 < rows; r0 += g) {
    const int64_t nr = std::min(g, rows - r0);
    rc = four_step(RealColumn{x + r0 * in_len, in_len, in_len}, y, z, nr, logm, -1.f);
    if (rc == WXX_OK) {
      hipLaunchKernelGGL(untangle_kernel, dim3(grid(nr * (M + 1))), dim3(kThreads), 0, stream(),
                         (const float2*)z, X + r0 * (M + 1), nr, M);
      WXX_LAUNCHED();
    }
  }
  scratch_free(y);
  scratch_free(z);
  return rc;
}

int irfft_four_step(const float2* X, float* x, int64_t rows, int64_t in_len, int logm,
                    int64_t out_len, float post) {
  if (logm > 2 * kMaxLogL)
    return set_error(WXX_E_UNSUPPORTED, "irfft length 2^%d above 2^%d", logm + 1,
                     2 * kMaxLogL + 1);
  const int64_t M = int64_t(1) << logm;
  const int64_t g = group_rows(rows, M);
  float2* y = (float2*)scratch_alloc(sizeof(float2) * g * M);
  float2* z = (float2*)scratch_alloc(sizeof(float2) * g * M);
  int rc = (y && z) ? WXX_OK : set_error(WXX_E_OOM, "four-step FFT scratch");
  // the untangled spectrum is built in z, transformed through y back into z
  const float scale = 1.0f / (float)M;
  for (int64_t r0 = 0; rc == WXX_OK && r0 < rows; r0 += g) {
    const int64_t nr = std::min(g, rows - r0);
    hipLaunchKernelGGL(untangle_inv_kernel, dim3(grid(nr * M)), dim3(kThreads), 0, stream(),
                       X + r0 * in_len, z, nr, in_len, M);
    rc = four_step(ComplexColumn{z, M}, y, z, nr, logm, 1.f);
    if (rc == WXX_OK) {
      hipLaunchKernelGGL(unpack_real_kernel, dim3(grid(nr * out_len)), dim3(kThreads), 0,
                         stream(), (const float2*)z, x + r0 * out_len, nr, M, out_len, scale,
                         post);
      WXX_LAUNCHED();
    }
  }
  scratch_free(y);
  scratch_free(z);
  return rc;
}

}  // namespace wxx
