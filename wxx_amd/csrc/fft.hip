// Real FFT / inverse real FFT along the last dimension, and the complex
// support kernels (multiply, add, conjugate, pad) of the spectral path.
//
// Reference: src/wxx/functional/fft.py:386-645 (rfft / irfft hosts) with
// shaders/helpers/fft_wg_real.wgsl, fft_wg_inverse.wgsl (n <= 1024, one
// workgroup per row) and fft_bitrev_real / fft_stage / fft_copy_out /
// fft_bitrev_complex / ifft_write_real (n > 1024: 1 + log2(n) + 1 launches,
// each a full HBM pass); complex helpers fft.py:168-383.
//
// MI355X design.  A length-n real transform is computed as one length
// M = n/2 complex transform of z[m] = x[2m] + i x[2m+1] followed by the
// standard even/odd untangling X[k] = E[k] + W_n^k O[k] (and the mirror image
// of that for the inverse).  Longer rows take the four-step path of
// fft_big.hip.  For n <= 32768 the M complex points of a row
// (64 KiB at n = 16384) stay in LDS for the whole transform: one workgroup
// per row reads the input from HBM once and writes the spectrum once.
// Inside the workgroup the transform is a Stockham auto-sort FFT: every pass
// loads 16 points per thread from LDS, applies the pass twiddles, does a
// radix-16 (or radix-2/4/8 first pass) DFT in registers and writes the points
// back in their next-pass order, so no bit reversal pass is needed.  The
// first pass reads straight from HBM and, for the inverse, the last pass
// writes straight to HBM (its output order is already natural).
//
// Twiddles come from a per-size table built once on the host in double
// precision.  Pass p stores W_{Ns R}^{r k} at [(r-1) * Ns + k], so for a
// fixed r consecutive lanes (consecutive k) load consecutive entries; the
// untangling twiddles W_n^k, k <= M, follow.
#include "common.h"
#include "nd.h"

#include <cmath>
#include <map>
#include <mutex>
#include <vector>

namespace {

// ---- plan --------------------------------------------------------------
// log2(M) bits are split into passes: the first pass takes log2(M) mod 4
// bits (4 when that is 0), every later pass 4 bits (radix 16).
struct Plan {
  int logm;
  __host__ __device__ constexpr int m() const { return 1 << logm; }
  __host__ __device__ constexpr int ebits() const { return logm < 4 ? logm : 4; }
  __host__ __device__ constexpr int first() const {
    return logm % 4 == 0 ? ebits() : logm % 4;
  }
  __host__ __device__ constexpr int npass() const {
    return logm == 0 ? 1 : (logm - first()) / 4 + 1;
  }
  __host__ __device__ constexpr int bits(int p) const { return p == 0 ? first() : 4; }
  __host__ __device__ constexpr int ns_bits(int p) const {
    return p == 0 ? 0 : first() + 4 * (p - 1);
  }
  // Twiddle entries stored for the passes before p (pass tables back to back).
  __host__ __device__ constexpr int offset(int p) const {
    int o = 0;
    for (int q = 0; q < p; ++q) o += (1 << ns_bits(q)) * ((1 << bits(q)) - 1);
    return o;
  }
  __host__ __device__ constexpr int table_size() const { return offset(npass()) + m() + 1; }
};

constexpr int kMaxLogM = 14;  // n <= 32768 stays resident in LDS

template <int LOGM>
struct Geo {
  static constexpr Plan plan{LOGM};
  static constexpr int M = 1 << LOGM;
  static constexpr int E = 1 << plan.ebits();   // points per thread
  static constexpr int T = M / E;               // threads per row
  static constexpr int NT = T < 256 ? 256 : T;  // threads per block
  static constexpr int RPB = NT / T;            // rows per block
  static constexpr int PM = M + (M >> 4);       // padded LDS row (one pad slot per 16)
};

__device__ __forceinline__ int lds_pad(int i) { return i + (i >> 4); }

__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}

// a * b with the rounding fixed as written: re = fma(a.x, b.x, -(a.y b.y)),
// im = fma(a.x, b.y, a.y b.x).  The elementwise complex product and the
// spectrum products fused into the transforms both use it, so a fused
// product rounds exactly as the separate one does.
__device__ __forceinline__ float2 cmul_op(float2 a, float2 b) {
  return make_float2(fmaf(a.x, b.x, -(a.y * b.y)), fmaf(a.x, b.y, a.y * b.x));
}

// Spectrum operands multiplied into a transform's input bins (irfft) or
// output bins (rfft): bin j of row r becomes v * h[r mod hrows][j]
// (conjugated when conj_h, skipped when h is null) * (w, 0) (when weighted),
// products in that order.  The real bin weight w is w_edge at the DC and
// Nyquist bins (j == 0, j == nyq) and w_mid between them, the form of the
// rfft / irfft adjoints' weights: two scalars instead of a table, so no load
// has to wait behind a row prefetch.  h rows have the spectrum's bins per row.
struct SpecMul {
  const float2* h;
  int64_t hrows;
  int conj_h;
  int weighted;
  float w_edge, w_mid;
  int nyq;
};

// OPS (fixed at compile time, so no bin's loads sit behind a branch of its
// own): bit 0 the h factor (hr: this row's h row), bit 1 the bin weight.
constexpr int kOpH = 1, kOpW = 2;
template <int OPS>
__device__ __forceinline__ float2 spec_mul(float2 v, const SpecMul& m,
                                           const float2* __restrict__ hr, int64_t j) {
  if constexpr ((OPS & kOpH) != 0) {
    float2 b = hr[j];
    if (m.conj_h) b.y = -b.y;
    v = cmul_op(v, b);
  }
  if constexpr ((OPS & kOpW) != 0)
    v = cmul_op(v, make_float2(j == 0 || j == m.nyq ? m.w_edge : m.w_mid, 0.f));
  return v;
}

// cos(pi m / 8), m in [0, 16)
__device__ constexpr float kCosPi8[16] = {
    1.0f,  0.92387953251128674f,  0.70710678118654752f,  0.38268343236508977f,
    0.0f,  -0.38268343236508977f, -0.70710678118654752f, -0.92387953251128674f,
    -1.0f, -0.92387953251128674f, -0.70710678118654752f, -0.38268343236508977f,
    0.0f,  0.38268343236508977f,  0.70710678118654752f,  0.92387953251128674f};

// v * exp(-i pi m / 8) (forward) or v * exp(+i pi m / 8) (inverse); m is a
// compile-time constant after unrolling, so the branches fold away.
template <bool INV>
__device__ __forceinline__ float2 rot(float2 v, int m) {
  m &= 15;
  if (m == 0) return v;
  if (m == 8) return make_float2(-v.x, -v.y);
  if (m == 4) return INV ? make_float2(-v.y, v.x) : make_float2(v.y, -v.x);
  if (m == 12) return INV ? make_float2(v.y, -v.x) : make_float2(-v.y, v.x);
  const float c = kCosPi8[m];
  const float s = INV ? kCosPi8[(m + 12) & 15] : -kCosPi8[(m + 12) & 15];
  return make_float2(v.x * c - v.y * s, v.x * s + v.y * c);
}

// In-register radix-2 decimation-in-frequency DFT of R <= 16 points; the
// result is in bit-reversed order: X[k] = u[bitrev(k)].
template <int R, bool INV>
__device__ __forceinline__ void dft(float2* u) {
  static_assert(R <= 16, "radix above 16 needs finer rotation constants");
#pragma unroll
  for (int s = R / 2; s >= 1; s >>= 1) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (j & s) continue;
      const float2 a = u[j], b = u[j + s];
      u[j] = make_float2(a.x + b.x, a.y + b.y);
      u[j + s] = rot<INV>(make_float2(a.x - b.x, a.y - b.y), (j & (s - 1)) * (8 / s));
    }
  }
}

__host__ __device__ constexpr int bitrev(int x, int bits) {
  int r = 0;
  for (int i = 0; i < bits; ++i) {
    r = (r << 1) | (x & 1);
    x >>= 1;
  }
  return r;
}

// Twiddle + DFT of pass P on the E register points (E/R groups of R).
template <int LOGM, int P, bool INV>
__device__ __forceinline__ void pass_math(float2* v, int t, const float2* __restrict__ tw) {
  using G = Geo<LOGM>;
  constexpr Plan pl{LOGM};
  constexpr int R = 1 << pl.bits(P), NS = 1 << pl.ns_bits(P);
  constexpr int OFF = pl.offset(P);
#pragma unroll
  for (int q = 0; q < G::E / R; ++q) {
    float2* u = v + q * R;
    if constexpr (NS > 1) {
      const int k = (t + q * G::T) & (NS - 1);
#pragma unroll
      for (int r = 1; r < R; ++r) {
        float2 w = tw[OFF + (r - 1) * NS + k];
        if (INV) w.y = -w.y;
        u[r] = cmul(u[r], w);
      }
    }
    dft<R, INV>(u);
  }
}

// Output of an inverse transform's real row (the row pointer is passed
// alongside): samples [0, lim) of the row, each scaled by scale and then by post (two roundings,
// the same values a separate scaling pass would give).  mode 0: the whole row
// (lim = 2M, float2 stores); 1: an even lim (float2 stores below lim); 2: an
// odd lim (scalar stores below lim).
struct RowOut {
  int64_t lim;
  float scale, post;
  int mode;
  int lim32, half;  // lim and lim / 2 as 32-bit ints for the store guards
};

// Stores the real pair z (samples 2j, 2j + 1) of row o; CROP is o.mode,
// fixed at compile time so the uncropped kernel keeps plain float2 stores.
template <int CROP>
__device__ __forceinline__ void row_store(const RowOut& o, float* __restrict__ p, int j,
                                          float2 z) {
  z = make_float2((z.x * o.scale) * o.post, (z.y * o.scale) * o.post);
  if (CROP == 0) {
    reinterpret_cast<float2*>(p)[j] = z;
  } else if (CROP == 1) {
    if (j < o.half) reinterpret_cast<float2*>(p)[j] = z;  // half = lim / 2
  } else {
    const int i = 2 * j;
    if (i < o.lim32) p[i] = z.x;
    if (i + 1 < o.lim32) p[i + 1] = z.y;
  }
}

// The last Stockham pass stores point (q, k) of thread t at sample pair
// j = u + k * GR with u = t + q * T in [0, GR).  An even crop keeps pairs
// j < half: every k below half / GR, and u < half % GR at k = half / GR, so
// the guards are uniform branches plus one lane compare per q.
template <int CROP, int Q, int R, int BITS, int T, int GR>
__device__ __forceinline__ void last_pass_store(const RowOut& o, float* __restrict__ p,
                                                const float2* v, int t) {
  if constexpr (CROP == 1) {
    const int kfull = o.half / GR, rem = o.half % GR;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int u = t + q * T;
      const bool tail = u < rem;
#pragma unroll
      for (int k = 0; k < R; ++k)
        if (k < kfull || (k == kfull && tail))
          row_store<0>(o, p, u + k * GR, v[q * R + bitrev(k, BITS)]);
    }
  } else {
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int k = 0; k < R; ++k)
        row_store<CROP>(o, p, t + q * T + k * GR, v[q * R + bitrev(k, BITS)]);
  }
}

// Passes P.. of the transform.  On entry v holds pass P's input points
// (P == 0: loaded by the caller).  On exit the transform is in buf in natural
// order (TO_GLOBAL false) or stored to the row o (TO_GLOBAL true).
template <int LOGM, int P, bool INV, bool TO_GLOBAL, int CROP = 0>
__device__ __forceinline__ void run_passes(float2* v, float2* buf, int t,
                                           const float2* __restrict__ tw, const RowOut& o,
                                           float* __restrict__ orow, bool live) {
  using G = Geo<LOGM>;
  constexpr Plan pl{LOGM};
  constexpr int BITS = pl.bits(P), R = 1 << BITS, NSB = pl.ns_bits(P), NS = 1 << NSB;
  constexpr int GR = G::M / R;  // groups per pass
  if constexpr (P > 0) {
#pragma unroll
    for (int q = 0; q < G::E / R; ++q)
#pragma unroll
      for (int r = 0; r < R; ++r) v[q * R + r] = buf[lds_pad(t + q * G::T + r * GR)];
  }
  pass_math<LOGM, P, INV>(v, t, tw);
  constexpr bool LAST = P + 1 == pl.npass();
  if constexpr (LAST && TO_GLOBAL) {
    // Last pass: NS == GR, so the output position of (group g, k) is g + k*GR.
    if (live) last_pass_store<CROP, G::E / R, R, BITS, G::T, GR>(o, orow, v, t);
  } else {
    if constexpr (P > 0) __syncthreads();  // every thread has read its pass input
#pragma unroll
    for (int q = 0; q < G::E / R; ++q) {
      const int g = t + q * G::T;
      const int base = ((g >> NSB) << (NSB + BITS)) + (g & (NS - 1));
#pragma unroll
      for (int k = 0; k < R; ++k) buf[lds_pad(base + k * NS)] = v[q * R + bitrev(k, BITS)];
    }
    __syncthreads();
    if constexpr (!LAST)
      run_passes<LOGM, P + 1, INV, TO_GLOBAL, CROP>(v, buf, t, tw, o, orow, live);
  }
}

// x: rows x in_len f32 (zero-padded / truncated to n = 2M); X: rows x (M+1) c64.
// MUL: output bins multiplied by sm's operands (spec_mul).
template <int LOGM, bool VEC, bool MUL>
__global__ __launch_bounds__(Geo<LOGM>::NT) void rfft_kernel(const float* __restrict__ x,
                                                             float2* __restrict__ X,
                                                             const float2* __restrict__ tw,
                                                             int64_t rows, int64_t in_len,
                                                             SpecMul sm) {
  using G = Geo<LOGM>;
  constexpr Plan pl{LOGM};
  __shared__ float2 lds[G::RPB * G::PM];
  const int t = threadIdx.x % G::T;
  const int rb = threadIdx.x / G::T;
  const int64_t row = (int64_t)blockIdx.x * G::RPB + rb;
  const bool live = row < rows;
  float2* buf = lds + rb * G::PM;
  const float* xr = x + (live ? row : 0) * in_len;

  float2 v[G::E];
  constexpr int R0 = 1 << pl.bits(0);
#pragma unroll
  for (int q = 0; q < G::E / R0; ++q)
#pragma unroll
    for (int r = 0; r < R0; ++r) {
      const int64_t j2 = 2 * (int64_t)(t + q * G::T + r * (G::M / R0));
      float2 z = make_float2(0.f, 0.f);
      if (live) {
        if (VEC) {
          if (j2 < in_len) z = *reinterpret_cast<const float2*>(xr + j2);
        } else {
          if (j2 < in_len) z.x = xr[j2];
          if (j2 + 1 < in_len) z.y = xr[j2 + 1];
        }
      }
      v[q * R0 + r] = z;
    }
  run_passes<LOGM, 0, false, false>(v, buf, t, tw, RowOut{}, nullptr, live);

  if (!live) return;
  const float2* wu = tw + pl.offset(pl.npass());
  float2* Xr = X + row * (G::M + 1);
  for (int k = t; k <= G::M; k += G::T) {
    const float2 a = buf[lds_pad(k & (G::M - 1))];
    const float2 b = buf[lds_pad((G::M - k) & (G::M - 1))];
    const float2 e = make_float2(0.5f * (a.x + b.x), 0.5f * (a.y - b.y));
    const float2 o = make_float2(0.5f * (a.y + b.y), 0.5f * (b.x - a.x));
    const float2 w = wu[k];
    const float2 z = make_float2(e.x + (w.x * o.x - w.y * o.y), e.y + (w.x * o.y + w.y * o.x));
    Xr[k] = MUL ? spec_mul<kOpW>(z, sm, nullptr, k) : z;
  }
}

// X: rows x in_len c64 one-sided spectrum; x: rows x n f32 (n = 2M).
// MUL: the spec_mul operand mask applied to the input bins as they load (0: none).
template <int LOGM, int CROP, int MUL>
__global__ __launch_bounds__(Geo<LOGM>::NT) void irfft_kernel(const float2* __restrict__ X,
                                                              float* __restrict__ x,
                                                              const float2* __restrict__ tw,
                                                              int64_t rows, int64_t in_len,
                                                              RowOut ro, SpecMul sm) {
  using G = Geo<LOGM>;
  constexpr Plan pl{LOGM};
  __shared__ float2 lds[G::RPB * G::PM];
  const int t = threadIdx.x % G::T;
  const int rb = threadIdx.x / G::T;
  const int64_t row = (int64_t)blockIdx.x * G::RPB + rb;
  const bool live = row < rows;
  float2* buf = lds + rb * G::PM;
  const float2* Xr = X + (live ? row : 0) * in_len;
  const float2* wu = tw + pl.offset(pl.npass());
  const float2* hr = (MUL & kOpH) ? sm.h + ((live ? row : 0) % sm.hrows) * in_len : nullptr;

  // Pack the Hermitian spectrum into Z = E + i O (E, O: spectra of the even
  // and odd samples).  Bins at or above in_len are zero; the imaginary parts
  // of the DC and Nyquist bins do not contribute to a real signal.
  float2 v[G::E];
  constexpr int R0 = 1 << pl.bits(0);
#pragma unroll
  for (int q = 0; q < G::E / R0; ++q)
#pragma unroll
    for (int r = 0; r < R0; ++r) {
      const int j = t + q * G::T + r * (G::M / R0);
      const int jj = G::M - j;
      float2 a = make_float2(0.f, 0.f), b = make_float2(0.f, 0.f);
      if (live) {
        if (j < in_len) a = MUL ? spec_mul<MUL>(Xr[j], sm, hr, j) : Xr[j];
        if (jj < in_len) b = MUL ? spec_mul<MUL>(Xr[jj], sm, hr, jj) : Xr[jj];
      }
      if (j == 0) a.y = 0.f;
      if (jj == G::M) b.y = 0.f;
      const float2 e = make_float2(0.5f * (a.x + b.x), 0.5f * (a.y - b.y));
      const float2 d = make_float2(0.5f * (a.x - b.x), 0.5f * (a.y + b.y));
      const float2 w = wu[j];  // o = d * conj(w)
      const float2 o = make_float2(d.x * w.x + d.y * w.y, d.y * w.x - d.x * w.y);
      v[q * R0 + r] = make_float2(e.x - o.y, e.y + o.x);
    }
  run_passes<LOGM, 0, true, true, CROP>(v, buf, t, tw, ro, x + (live ? row : 0) * ro.lim, live);
}

// ---- rows of M >= 2048 complex points: persistent workgroups -----------------
// One workgroup of T = M / 32 threads owns one row at a time and walks rows
// blockIdx.x, blockIdx.x + gridDim.x, ...  Each thread holds 32 points; the
// log2(M) bits are split into ceil(log2(M) / 5) Stockham passes of 3..5 bits
// (M = 8192: radix 32, 16, 16, i.e. two LDS exchanges instead of three).
// Workgroups stay resident (two per CU at M = 8192) and drift out of step,
// so one workgroup's HBM loads overlap another's LDS passes.  Each
// thread's twiddles depend only on its lane, so the powers of two of every
// pass twiddle are loaded once per workgroup and the other powers are formed
// by at most four complex products.  The rfft untangling step handles bins
// k and M - k together (one LDS pair read per two output bins).
// Points per thread of the persistent kernels for a row of 2^logm complex
// points: 16 up to 2^13 points (128 VGPRs, so a CU holds as many rows as its
// LDS does, with 4 waves per SIMD to overlap HBM and VALU work), 32 above
// (radix up to 32; 16 points would spill at 2^14).
constexpr int big_ept(int logm) { return logm <= 13 ? 16 : 32; }

template <int LOGM>
struct Big {
  static constexpr int M = 1 << LOGM;
  static constexpr int E = big_ept(LOGM);
  static constexpr int LE = E == 16 ? 4 : 5;  // log2(E): the largest pass radix
  static constexpr int T = M / E;
  static constexpr int NP = (LOGM + LE - 1) / LE;
  static constexpr int PM = M + (M >> 5);  // one pad slot per 32 points
  __host__ __device__ static constexpr int bits(int p) {
    return LOGM / NP + (p < LOGM % NP ? 1 : 0);
  }
  __host__ __device__ static constexpr int nsb(int p) {
    int s = 0;
    for (int q = 0; q < p; ++q) s += bits(q);
    return s;
  }
  // pass twiddle tables back to back, then the untangling twiddles W_{2M}^k
  __host__ __device__ static constexpr int off(int p) {
    int o = 0;
    for (int q = 0; q < p; ++q) o += (1 << nsb(q)) * ((1 << bits(q)) - 1);
    return o;
  }
  __host__ __device__ static constexpr int table_size() { return off(NP) + M + 1; }
  // twiddle-base registers per thread: (E / R) groups x bits for passes >= 1
  __host__ __device__ static constexpr int tbo(int p) {
    int o = 0;
    for (int q = 1; q < p; ++q) o += (E >> bits(q)) * bits(q);
    return o;
  }
  static constexpr int NTB = tbo(NP) > 0 ? tbo(NP) : 1;
  static constexpr int MIN_BLOCKS = (160 * 1024) / (PM * 8) < 1 ? 1 : (160 * 1024) / (PM * 8);
  // __launch_bounds__'s second argument is waves per SIMD: MIN_BLOCKS
  // resident workgroups of T / 64 waves over the CU's 4 SIMDs
  static constexpr int MIN_WAVES = MIN_BLOCKS * (T / 64) / 4 < 1 ? 1 : MIN_BLOCKS * (T / 64) / 4;
};

__device__ __forceinline__ int bpad(int i) { return i + (i >> 5); }
// bpad(x + c) == bpad(x) + bpad_c(c) for every LDS index the persistent
// kernels form (c a multiple of 32, or a Stockham write offset k * NS below
// the next pass's group size); keeping bpad(x) per row and the constant part
// separate lets the constant fold into the ds instruction's offset field.
__host__ __device__ constexpr int bpad_c(int c) { return c + (c >> 5); }

// cos(pi m / 16), m in [0, 32)
__device__ constexpr float kCosPi16[32] = {
    1.0f,
    0.98078528040323044913f,
    0.92387953251128675613f,
    0.83146961230254523708f,
    0.70710678118654752440f,
    0.55557023301960222474f,
    0.38268343236508977173f,
    0.19509032201612826785f,
    0.0f,
    -0.19509032201612826785f,
    -0.38268343236508977173f,
    -0.55557023301960222474f,
    -0.70710678118654752440f,
    -0.83146961230254523708f,
    -0.92387953251128675613f,
    -0.98078528040323044913f,
    -1.0f,
    -0.98078528040323044913f,
    -0.92387953251128675613f,
    -0.83146961230254523708f,
    -0.70710678118654752440f,
    -0.55557023301960222474f,
    -0.38268343236508977173f,
    -0.19509032201612826785f,
    0.0f,
    0.19509032201612826785f,
    0.38268343236508977173f,
    0.55557023301960222474f,
    0.70710678118654752440f,
    0.83146961230254523708f,
    0.92387953251128675613f,
    0.98078528040323044913f};

// v * exp(-i pi m / 16) (forward) or v * exp(+i pi m / 16) (inverse).
template <bool INV>
__device__ __forceinline__ float2 rot32(float2 v, int m) {
  m &= 31;
  if (m == 0) return v;
  if (m == 16) return make_float2(-v.x, -v.y);
  if (m == 8) return INV ? make_float2(-v.y, v.x) : make_float2(v.y, -v.x);
  if (m == 24) return INV ? make_float2(v.y, -v.x) : make_float2(-v.y, v.x);
  const float c = kCosPi16[m];
  const float s = INV ? kCosPi16[(m + 24) & 31] : -kCosPi16[(m + 24) & 31];
  return make_float2(v.x * c - v.y * s, v.x * s + v.y * c);
}

// W_{2M}^k of the untangling table at a lane-independent offset k (a multiple
// of T, constant after unrolling).  With 16 points per thread T = M / 16, so
// W_{2M}^k = exp(-i pi (k / T) / 16) comes from the rotation constants instead
// of a global load: the persistent kernels keep a row prefetch in flight
// across the untangle, and an in-order vmcnt wait for a table load would wait
// for that prefetch too.
template <int E, int T>
__device__ __forceinline__ float2 untangle_tw(const float2* __restrict__ wu, int k) {
  if constexpr (E == 16) {
    const int m = k / T;
    return make_float2(kCosPi16[m & 31], -kCosPi16[(m + 24) & 31]);
  } else {
    return wu[k];
  }
}

// In-register radix-2 decimation-in-frequency DFT of R <= 32 points; output
// in bit-reversed order.
template <int R, bool INV>
__device__ __forceinline__ void dft32(float2* u) {
  static_assert(R <= 32, "radix above 32 needs finer rotation constants");
#pragma unroll
  for (int s = R / 2; s >= 1; s >>= 1) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (j & s) continue;
      const float2 a = u[j], b = u[j + s];
      u[j] = make_float2(a.x + b.x, a.y + b.y);
      u[j + s] = rot32<INV>(make_float2(a.x - b.x, a.y - b.y), (j & (s - 1)) * (16 / s));
    }
  }
}

// u[r] *= w^r for r in [1, R), from base[i] = w^(2^i): w^r is the product of
// the bases of r's set bits (at most log2(R) - 1 products deep).
template <int R>
__device__ __forceinline__ void twiddle_powers(float2* u, const float2* base) {
  float2 w[R];
#pragma unroll
  for (int r = 1; r < R; ++r) {
    const int hb = 31 - __builtin_clz(r);  // constant after unrolling
    w[r] = (r == (1 << hb)) ? base[hb] : cmul(w[r - (1 << hb)], base[hb]);
    u[r] = cmul(u[r], w[r]);
  }
}

// Twiddle bases of passes >= 1 for this thread (conjugated for the inverse).
template <int LOGM, int P, bool INV>
__device__ __forceinline__ void load_tw_bases(float2* twb, int t, const float2* __restrict__ tw) {
  using G = Big<LOGM>;
  if constexpr (P < G::NP) {
    constexpr int BITS = G::bits(P), R = 1 << BITS, NS = 1 << G::nsb(P), Q = G::E / R;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int k = (t + q * G::T) & (NS - 1);
#pragma unroll
      for (int i = 0; i < BITS; ++i) {
        float2 w = tw[G::off(P) + ((1 << i) - 1) * NS + k];
        if (INV) w.y = -w.y;
        twb[G::tbo(P) + q * BITS + i] = w;
      }
    }
    load_tw_bases<LOGM, P + 1, INV>(twb, t, tw);
  }
}

// Passes P.. of one row (see run_passes for the Stockham indexing).  v holds
// pass P's input (P == 0: loaded by the caller).  SYNC0: barrier before pass
// 0 writes LDS (other threads may still read the row buffer).
template <int LOGM, int P, bool INV, bool TO_GLOBAL, bool SYNC0, int CROP = 0>
__device__ __forceinline__ void big_passes(float2* v, float2* buf, int t, const float2* twb,
                                           const RowOut& o, float* __restrict__ orow) {
  using G = Big<LOGM>;
  constexpr int BITS = G::bits(P), R = 1 << BITS, NSB = G::nsb(P), NS = 1 << NSB;
  constexpr int GR = G::M / R, Q = G::E / R;
  if constexpr (P > 0) {
    const int tb = bpad(t);
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int r = 0; r < R; ++r) v[q * R + r] = buf[tb + bpad_c(q * G::T + r * GR)];
  }
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    if constexpr (NS > 1) twiddle_powers<R>(v + q * R, twb + G::tbo(P) + q * BITS);
    dft32<R, INV>(v + q * R);
  }
  constexpr bool LAST = P + 1 == G::NP;
  if constexpr (LAST && TO_GLOBAL) {
    last_pass_store<CROP, Q, R, BITS, G::T, GR>(o, orow, v, t);
  } else {
    if constexpr (P > 0 || SYNC0) __syncthreads();
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int g = t + q * G::T;
      const int base = bpad(((g >> NSB) << (NSB + BITS)) + (g & (NS - 1)));
#pragma unroll
      for (int k = 0; k < R; ++k) buf[base + bpad_c(k * NS)] = v[q * R + bitrev(k, BITS)];
    }
    __syncthreads();
    if constexpr (!LAST)
      big_passes<LOGM, P + 1, INV, TO_GLOBAL, SYNC0, CROP>(v, buf, t, twb, o, orow);
  }
}

// Pass-0 input of one rfft row: z[m] = x[2m] + i x[2m+1], m = t + r T, zero
// beyond in_len.
template <int LOGM, bool VEC, bool FULL>
__device__ __forceinline__ void rfft_big_load(float2* v, const float* __restrict__ xr, int t,
                                              int64_t in_len) {
  using G = Big<LOGM>;
  constexpr int R0 = 1 << G::bits(0), GR0 = G::M / R0, Q0 = G::E / R0;
#pragma unroll
  for (int q = 0; q < Q0; ++q)
#pragma unroll
    for (int r = 0; r < R0; ++r) {
      const int64_t j2 = 2 * (int64_t)(t + q * G::T + r * GR0);
      float2 z = make_float2(0.f, 0.f);
      if (VEC && FULL) {  // the row covers every sample: no guards
        z = *reinterpret_cast<const float2*>(xr + j2);
      } else if (VEC) {
        if (j2 < in_len) z = *reinterpret_cast<const float2*>(xr + j2);
      } else {
        if (j2 < in_len) z.x = xr[j2];
        if (j2 + 1 < in_len) z.y = xr[j2 + 1];
      }
      v[q * R0 + r] = z;
    }
}

template <int LOGM, bool VEC, bool MUL>
__global__ __launch_bounds__(Big<LOGM>::T, Big<LOGM>::MIN_WAVES) void rfft_big_kernel(
    const float* __restrict__ x, float2* __restrict__ X, const float2* __restrict__ tw,
    int64_t rows, int64_t in_len, SpecMul sm) {
  using G = Big<LOGM>;
  __shared__ float2 buf[G::PM];
  float2 twb[G::NTB];
  load_tw_bases<LOGM, 1, false>(twb, threadIdx.x, tw);
  const float2* wu = tw + G::off(G::NP);
  const float2 wt = wu[threadIdx.x];  // W_{2M}^t

  float2 v[G::E];
  const bool full = in_len >= 2 * G::M;
  if ((int64_t)blockIdx.x < rows) {
    if (full)
      rfft_big_load<LOGM, VEC, true>(v, x + blockIdx.x * in_len, threadIdx.x, in_len);
    else
      rfft_big_load<LOGM, VEC, false>(v, x + blockIdx.x * in_len, threadIdx.x, in_len);
  }
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    // Hide the lane index from loop-invariant code motion: every LDS address
    // below is a function of t, and hoisting them all out of the row loop
    // would hold ~200 VGPRs; recomputed per row they fold into base + offset.
    int t = threadIdx.x;
    WXX_OPAQUE(t);
    big_passes<LOGM, 0, false, false, true>(v, buf, t, twb, RowOut{}, nullptr);
    // The transform is in LDS and v is free: start loading this workgroup's
    // next row now, so its HBM latency overlaps the untangle and the stores
    // below instead of following them.
    const int64_t next = row + gridDim.x;
    if (next < rows) {
      if (full)
        rfft_big_load<LOGM, VEC, true>(v, x + next * in_len, t, in_len);
      else
        rfft_big_load<LOGM, VEC, false>(v, x + next * in_len, t, in_len);
    }
    // untangle: bins k and M - k from Z[k], Z[M - k].  wt is hidden per row
    // like t: its products with the constant twiddles are loop invariant, and
    // hoisted they would hold 2 E VGPRs across the row loop.
    float2 wtr = wt;
    WXX_OPAQUE(wtr.x);
    WXX_OPAQUE(wtr.y);
    float2* Xr = X + row * (G::M + 1);
    const int tb = bpad(t), nb = -t + ((-t) >> 5);  // bpad(t), and bpad(a - t) - bpad_c(a)
#pragma unroll
    for (int i = 0; i <= G::E / 2; ++i) {
      const int k = t + i * G::T;
      if (k > G::M / 2) break;
      const float2 a = buf[tb + bpad_c(i * G::T)];
      const float2 b = buf[k == 0 ? 0 : nb + bpad_c(G::M - i * G::T)];  // bin (M - k) mod M
      const float2 e = make_float2(0.5f * (a.x + b.x), 0.5f * (a.y - b.y));
      const float2 o = make_float2(0.5f * (a.y + b.y), 0.5f * (b.x - a.x));
      const float2 w = cmul(wtr, untangle_tw<G::E, G::T>(wu, i * G::T));
      const float2 wo = cmul(w, o);
      const float2 lo = make_float2(e.x + wo.x, e.y + wo.y);
      const float2 hi = make_float2(e.x - wo.x, wo.y - e.y);
      Xr[k] = MUL ? spec_mul<kOpW>(lo, sm, nullptr, k) : lo;
      if (k != G::M / 2) Xr[G::M - k] = MUL ? spec_mul<kOpW>(hi, sm, nullptr, G::M - k) : hi;
    }
    __syncthreads();  // the row buffer is free for the next row
  }
}

// Offset (beyond the lane index t) of the position held in register e for
// pass 0: e = q R0 + r holds point t + q T + r (M / R0).
template <int LOGM>
__host__ __device__ constexpr int big_pos0(int e) {
  using G = Big<LOGM>;
  constexpr int R0 = 1 << G::bits(0);
  return (e / R0) * G::T + (e % R0) * (G::M / R0);
}

// Spectrum bins of one irfft row at this thread's pass-0 positions.
template <int LOGM, bool FULL, int MUL>
__device__ __forceinline__ void irfft_big_load(float2* a, const float2* __restrict__ Xr, int t,
                                               int64_t in_len, const SpecMul& sm,
                                               const float2* __restrict__ hr) {
  using G = Big<LOGM>;
#pragma unroll
  for (int e = 0; e < G::E; ++e) {
    const int j = t + big_pos0<LOGM>(e);
    a[e] = (FULL || j < in_len) ? (MUL ? spec_mul<MUL>(Xr[j], sm, hr, j) : Xr[j])
                                : make_float2(0.f, 0.f);  // FULL: in_len >= M
  }
}

template <int LOGM, int CROP, int MUL>
__global__ __launch_bounds__(Big<LOGM>::T, Big<LOGM>::MIN_WAVES) void irfft_big_kernel(
    const float2* __restrict__ X, float* __restrict__ x, const float2* __restrict__ tw,
    int64_t rows, int64_t in_len, RowOut ro, SpecMul sm) {
  using G = Big<LOGM>;
  __shared__ float2 buf[G::PM];
  float2 twb[G::NTB];
  load_tw_bases<LOGM, 1, true>(twb, threadIdx.x, tw);
  const float2* wu = tw + G::off(G::NP);
  const float2 wt = wu[threadIdx.x];

  float2 v[G::E];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    int t = threadIdx.x;  // t and wt opaque per row, as in rfft_big_kernel
    WXX_OPAQUE(t);
    float2 wtr = wt;
    WXX_OPAQUE(wtr.x);
    WXX_OPAQUE(wtr.y);
    const float2* Xr = X + row * in_len;
    const float2* hr = (MUL & kOpH) ? sm.h + (row % sm.hrows) * in_len : nullptr;
    if (in_len >= G::M)
      irfft_big_load<LOGM, true, MUL>(v, Xr, t, in_len, sm, hr);
    else
      irfft_big_load<LOGM, false, MUL>(v, Xr, t, in_len, sm, hr);
    const float2 nyq = G::M < in_len ? (MUL ? spec_mul<MUL>(Xr[G::M], sm, hr, G::M) : Xr[G::M])
                                     : make_float2(0.f, 0.f);
    // exchange the bins through LDS to pair j with M - j
    const int tb = bpad(t), nb = -t + ((-t) >> 5);  // bpad(t), and bpad(a - t) - bpad_c(a)
#pragma unroll
    for (int e = 0; e < G::E; ++e) buf[tb + bpad_c(big_pos0<LOGM>(e))] = v[e];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < G::E; ++e) {
      const int j = t + big_pos0<LOGM>(e);
      float2 a = v[e];
      // select the LDS index, then the value (a select between &nyq and the
      // LDS slot would become a generic pointer and flat loads)
      float2 b = buf[j == 0 ? 0 : nb + bpad_c(G::M - big_pos0<LOGM>(e))];
      if (j == 0) b = nyq;
      if (j == 0) {
        a.y = 0.f;
        b.y = 0.f;
      }
      const float2 ee = make_float2(0.5f * (a.x + b.x), 0.5f * (a.y - b.y));
      const float2 d = make_float2(0.5f * (a.x - b.x), 0.5f * (a.y + b.y));
      // o = d * conj(w); the constant twiddles only at n = 16384, where they
      // fit the VGPR budget (the shorter rows' kernels would spill)
      const float2 w = LOGM == 13 ? cmul(wtr, untangle_tw<G::E, G::T>(wu, big_pos0<LOGM>(e)))
                                  : cmul(wt, wu[big_pos0<LOGM>(e)]);
      const float2 o = make_float2(d.x * w.x + d.y * w.y, d.y * w.x - d.x * w.y);
      v[e] = make_float2(ee.x - o.y, ee.y + o.x);
    }
    // SYNC0: every thread has read its pair partner before pass 0 overwrites LDS
    big_passes<LOGM, 0, true, true, true, CROP>(v, buf, t, twb, ro, x + row * ro.lim);
    __syncthreads();  // last pass reads of this row are done
  }
}

// n == 1: X[row] = x[row, 0] (or 0 for an empty row).
__global__ __launch_bounds__(256) void rfft1_kernel(const float* __restrict__ x,
                                                    float2* __restrict__ X, int64_t rows,
                                                    int64_t in_len) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r < rows) X[r] = make_float2(in_len > 0 ? x[r * in_len] : 0.f, 0.f);
}

// ---- twiddle tables (built once per size, kept for the process) -----------
std::mutex g_tw_mu;
std::map<int, float2*> g_tw;

const float2* twiddles(int logm) {
  std::lock_guard<std::mutex> lock(g_tw_mu);
  auto it = g_tw.find(logm);
  if (it != g_tw.end()) return it->second;
  const Plan pl{logm};
  const int64_t M = pl.m();
  std::vector<float2> h(pl.table_size());
  const double two_pi = 6.283185307179586476925286766559;
  for (int p = 0; p < pl.npass(); ++p) {
    const int64_t R = 1 << pl.bits(p), NS = 1 << pl.ns_bits(p);
    for (int64_t r = 1; r < R; ++r)
      for (int64_t k = 0; k < NS; ++k) {
        const double a = -two_pi * (double)(r * k) / (double)(NS * R);
        h[pl.offset(p) + (r - 1) * NS + k] = make_float2((float)std::cos(a), (float)std::sin(a));
      }
  }
  for (int64_t k = 0; k <= M; ++k) {
    const double a = -two_pi * (double)k / (double)(2 * M);
    h[pl.offset(pl.npass()) + k] = make_float2((float)std::cos(a), (float)std::sin(a));
  }
  void* d = wxx_alloc(h.size() * sizeof(float2));
  if (!d) return nullptr;
  if (wxx_h2d(d, h.data(), h.size() * sizeof(float2)) != WXX_OK) {
    wxx_free(d);
    return nullptr;
  }
  g_tw[logm] = static_cast<float2*>(d);
  return static_cast<float2*>(d);
}

template <int LOGM>
const float2* big_twiddles() {
  using G = Big<LOGM>;
  std::lock_guard<std::mutex> lock(g_tw_mu);
  const int key = 0x100 | LOGM;
  auto it = g_tw.find(key);
  if (it != g_tw.end()) return it->second;
  std::vector<float2> h(G::table_size());
  const double two_pi = 6.283185307179586476925286766559;
  for (int p = 0; p < G::NP; ++p) {
    const int64_t R = 1 << G::bits(p), NS = 1 << G::nsb(p);
    for (int64_t r = 1; r < R; ++r)
      for (int64_t k = 0; k < NS; ++k) {
        const double a = -two_pi * (double)(r * k) / (double)(NS * R);
        h[G::off(p) + (r - 1) * NS + k] = make_float2((float)std::cos(a), (float)std::sin(a));
      }
  }
  for (int64_t k = 0; k <= G::M; ++k) {
    const double a = -two_pi * (double)k / (double)(2 * G::M);
    h[G::off(G::NP) + k] = make_float2((float)std::cos(a), (float)std::sin(a));
  }
  void* d = wxx_alloc(h.size() * sizeof(float2));
  if (!d) return nullptr;
  if (wxx_h2d(d, h.data(), h.size() * sizeof(float2)) != WXX_OK) {
    wxx_free(d);
    return nullptr;
  }
  g_tw[key] = static_cast<float2*>(d);
  return static_cast<float2*>(d);
}

// Persistent grid: as many workgroups as fit on the device at once.
template <typename K>
unsigned persistent_grid(K kernel, int threads, int64_t rows) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const int64_t cus = wxx::num_cus() > 0 ? wxx::num_cus() : 256;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(rows, per_cu * cus));
}

constexpr int kBigMinLogM = 11;

int log2_exact(int64_t n) {
  int l = 0;
  while ((int64_t(1) << l) < n) ++l;
  return (int64_t(1) << l) == n ? l : -1;
}

// sm null: the plain transform; else the MUL instantiation with *sm.
template <int LOGM, bool VEC, bool MUL>
void launch_rfft_k(const float* x, float2* X, const float2* tw, int64_t rows, int64_t in_len,
                   const SpecMul& sm) {
  if constexpr (LOGM >= kBigMinLogM) {
    const float2* btw = big_twiddles<LOGM>();
    if (!btw) {
      wxx::set_error(WXX_E_OOM, "rfft twiddle table allocation failed");
      return;
    }
    constexpr int T = Big<LOGM>::T;
    const unsigned g = persistent_grid(rfft_big_kernel<LOGM, VEC, MUL>, T, rows);
    hipLaunchKernelGGL((rfft_big_kernel<LOGM, VEC, MUL>), dim3(g), dim3(T), 0, wxx::stream(), x,
                       X, btw, rows, in_len, sm);
  } else {
    using G = Geo<LOGM>;
    const dim3 grid((unsigned)((rows + G::RPB - 1) / G::RPB));
    hipLaunchKernelGGL((rfft_kernel<LOGM, VEC, MUL>), grid, dim3(G::NT), 0, wxx::stream(), x, X,
                       tw, rows, in_len, sm);
  }
}

template <int LOGM>
void launch_rfft(const float* x, float2* X, const float2* tw, int64_t rows, int64_t in_len,
                 bool vec, const SpecMul* sm) {
  const SpecMul none{};
  if (sm) {
    if (vec)
      launch_rfft_k<LOGM, true, true>(x, X, tw, rows, in_len, *sm);
    else
      launch_rfft_k<LOGM, false, true>(x, X, tw, rows, in_len, *sm);
  } else if (vec) {
    launch_rfft_k<LOGM, true, false>(x, X, tw, rows, in_len, none);
  } else {
    launch_rfft_k<LOGM, false, false>(x, X, tw, rows, in_len, none);
  }
}

template <int LOGM, int CROP, int MUL>
void launch_irfft_mode(const float2* X, float* x, const float2* tw, int64_t rows, int64_t in_len,
                       RowOut ro, const SpecMul& sm) {
  ro.scale = 1.0f / (float)(1 << LOGM);
  if constexpr (LOGM >= kBigMinLogM) {
    const float2* btw = big_twiddles<LOGM>();
    if (!btw) {
      wxx::set_error(WXX_E_OOM, "irfft twiddle table allocation failed");
      return;
    }
    constexpr int T = Big<LOGM>::T;
    const unsigned g = persistent_grid(irfft_big_kernel<LOGM, CROP, MUL>, T, rows);
    hipLaunchKernelGGL((irfft_big_kernel<LOGM, CROP, MUL>), dim3(g), dim3(T), 0, wxx::stream(), X,
                       x, btw, rows, in_len, ro, sm);
    return;
  }
  using G = Geo<LOGM>;
  const dim3 grid((unsigned)((rows + G::RPB - 1) / G::RPB));
  hipLaunchKernelGGL((irfft_kernel<LOGM, CROP, MUL>), grid, dim3(G::NT), 0, wxx::stream(), X, x,
                     tw, rows, in_len, ro, sm);
}

template <int LOGM, int MUL>
void launch_irfft_m(const float2* X, float* x, const float2* tw, int64_t rows, int64_t in_len,
                    const RowOut& ro, const SpecMul& sm) {
  if (ro.mode == 0)
    launch_irfft_mode<LOGM, 0, MUL>(X, x, tw, rows, in_len, ro, sm);
  else if (ro.mode == 1)
    launch_irfft_mode<LOGM, 1, MUL>(X, x, tw, rows, in_len, ro, sm);
  else
    launch_irfft_mode<LOGM, 2, MUL>(X, x, tw, rows, in_len, ro, sm);
}

template <int LOGM>
void launch_irfft(const float2* X, float* x, const float2* tw, int64_t rows, int64_t in_len,
                  const RowOut& ro, const SpecMul* sm) {
  const int ops = sm ? (sm->h ? kOpH : 0) | (sm->weighted ? kOpW : 0) : 0;
  if (ops == kOpH)
    launch_irfft_m<LOGM, kOpH>(X, x, tw, rows, in_len, ro, *sm);
  else if (ops == kOpW)
    launch_irfft_m<LOGM, kOpW>(X, x, tw, rows, in_len, ro, *sm);
  else if (ops == (kOpH | kOpW))
    launch_irfft_m<LOGM, kOpH | kOpW>(X, x, tw, rows, in_len, ro, *sm);
  else
    launch_irfft_m<LOGM, 0>(X, x, tw, rows, in_len, ro, SpecMul{});
}

template <int L = 0>
void dispatch_rfft(int logm, const float* x, float2* X, const float2* tw, int64_t rows,
                   int64_t in_len, bool vec, const SpecMul* sm = nullptr) {
  if constexpr (L <= kMaxLogM) {
    if (logm == L) return launch_rfft<L>(x, X, tw, rows, in_len, vec, sm);
    dispatch_rfft<L + 1>(logm, x, X, tw, rows, in_len, vec, sm);
  }
}

template <int L = 0>
void dispatch_irfft(int logm, const float2* X, float* x, const float2* tw, int64_t rows,
                    int64_t in_len, const RowOut& ro, const SpecMul* sm = nullptr) {
  if constexpr (L <= kMaxLogM) {
    if (logm == L) return launch_irfft<L>(X, x, tw, rows, in_len, ro, sm);
    dispatch_irfft<L + 1>(logm, X, x, tw, rows, in_len, ro, sm);
  }
}

// ---- complex elementwise --------------------------------------------------
// op 0: out = a * b, op 1: out = a + b; conj flags conjugate an operand.
__device__ __forceinline__ float2 complex_op(float2 u, float2 w, int op, int conj_a,
                                             int conj_b) {
  if (conj_a) u.y = -u.y;
  if (conj_b) w.y = -w.y;
  return op == 0 ? cmul_op(u, w) : make_float2(u.x + w.x, u.y + w.y);
}

template <bool WIDE>
__global__ __launch_bounds__(256) void complex_binary_kernel(float2* __restrict__ out,
                                                             const float2* __restrict__ a,
                                                             const float2* __restrict__ b,
                                                             wxx::ND nd, int64_t n, int op,
                                                             int conj_a, int conj_b) {
  const int64_t step = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += step) {
    int64_t off[3];
    if (WIDE)
      wxx::offsets64<3>(nd, i, off);
    else
      wxx::offsets<3>(nd, i, off);
    out[off[0]] = complex_op(a[off[1]], b[off[2]], op, conj_a, conj_b);
  }
}

// a and out contiguous over all n elements, b contiguous too (BROW false) or
// one row of `cols` elements repeated for every row (BROW true: a spectrum
// times a filter or a weight vector broadcast over its rows): two elements
// per thread through 16-byte loads and stores, four pairs in flight per
// thread, 32-bit index arithmetic (2 n < 2^31).
template <bool BROW>
__global__ __launch_bounds__(256) void complex_binary_pairs_kernel(
    float4* __restrict__ out, const float4* __restrict__ a, const float2* __restrict__ b,
    int n2, int cols, int op, int conj_a, int conj_b) {
  const int step = gridDim.x * 256;
  for (int t0 = blockIdx.x * 256 + threadIdx.x; t0 < n2; t0 += 4 * step) {
    float4 av[4], bv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = t0 + u * step;
      if (t < n2) {
        av[u] = a[t];
        if (!BROW) {
          bv[u] = reinterpret_cast<const float4*>(b)[t];
        } else {
          const int c = (2 * t) % cols;  // the pair's first column; the second may wrap
          const float2 b0 = b[c], b1 = b[c + 1 == cols ? 0 : c + 1];
          bv[u] = make_float4(b0.x, b0.y, b1.x, b1.y);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = t0 + u * step;
      if (t < n2) {
        const float2 r0 = complex_op(make_float2(av[u].x, av[u].y), make_float2(bv[u].x, bv[u].y),
                                     op, conj_a, conj_b);
        const float2 r1 = complex_op(make_float2(av[u].z, av[u].w), make_float2(bv[u].z, bv[u].w),
                                     op, conj_a, conj_b);
        out[t] = make_float4(r0.x, r0.y, r1.x, r1.y);
      }
    }
  }
}

// Rank <= 2 after collapsing (rows x columns, e.g. a (B, D, F) spectrum times
// a (D, F) filter): rows on grid y, columns on grid x, no index division.
__global__ __launch_bounds__(256) void complex_binary_rows_kernel(
    float2* __restrict__ out, const float2* __restrict__ a, const float2* __restrict__ b,
    wxx::ND nd, int64_t rows, int64_t cols, int op, int conj_a, int conj_b) {
  const int r0 = nd.rank == 2 ? 0 : -1;  // stride slot of the row dimension
  const int c0 = nd.rank - 1;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const int64_t ro = r0 < 0 ? 0 : r * nd.stride[0][r0];
    const int64_t ra = r0 < 0 ? 0 : r * nd.stride[1][r0];
    const int64_t rb = r0 < 0 ? 0 : r * nd.stride[2][r0];
    for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < cols;
         c += (int64_t)gridDim.x * 256)
      out[ro + c * nd.stride[0][c0]] = complex_op(a[ra + c * nd.stride[1][c0]],
                                                  b[rb + c * nd.stride[2][c0]], op, conj_a, conj_b);
  }
}

__global__ __launch_bounds__(256) void complex_conj_kernel(float2* __restrict__ dst,
                                                           const float2* __restrict__ src,
                                                           wxx::ND nd, int64_t n) {
  const int64_t step = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += step) {
    int64_t off[2];
    wxx::offsets64<2>(nd, i, off);
    const float2 u = src[off[1]];
    dst[off[0]] = make_float2(u.x, -u.y);
  }
}

// out[i] = sum over b < batch of a[b n + i] * (conj) c[b n + i]: the product
// of a spectrum gradient with a batch of spectra summed over the batch (the
// adjoint of a filter broadcast over the batch), one output per thread.  Each
// part is summed in the column-sum order of the reduction kernels: rows
// r = 4 q + s into four partial sums s (the rows past the last multiple of
// four into the first), then (s0 + s1) + (s2 + s3), so the fused sum equals
// the product followed by that reduction.
__global__ __launch_bounds__(256) void complex_mul_batch_sum_kernel(
    float2* __restrict__ out, const float2* __restrict__ a, const float2* __restrict__ c,
    int64_t batch, int64_t n, int conj_c) {
  const int64_t step = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += step) {
    float2 s[4] = {make_float2(0.f, 0.f), make_float2(0.f, 0.f), make_float2(0.f, 0.f),
                   make_float2(0.f, 0.f)};
    int64_t b = 0;
    for (; b + 3 < batch; b += 4) {
      float2 p[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float2 w = c[(b + u) * n + i];
        if (conj_c) w.y = -w.y;
        p[u] = cmul_op(a[(b + u) * n + i], w);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u] = make_float2(s[u].x + p[u].x, s[u].y + p[u].y);
    }
    for (; b < batch; ++b) {
      float2 w = c[b * n + i];
      if (conj_c) w.y = -w.y;
      const float2 p = cmul_op(a[b * n + i], w);
      s[0] = make_float2(s[0].x + p.x, s[0].y + p.y);
    }
    out[i] = make_float2((s[0].x + s[1].x) + (s[2].x + s[3].x),
                         (s[0].y + s[1].y) + (s[2].y + s[3].y));
  }
}

__global__ __launch_bounds__(256) void complex_pad_kernel(const float2* __restrict__ src,
                                                          float2* __restrict__ dst,
                                                          int64_t batch, int64_t in_len,
                                                          int64_t out_len) {
  const int64_t n = batch * out_len;
  const int64_t step = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += step) {
    const int64_t r = i / out_len, c = i - r * out_len;
    dst[i] = c < in_len ? src[r * in_len + c] : make_float2(0.f, 0.f);
  }
}

}  // namespace

// Replaces functional.rfft (fft.py:484-563): rows x in_len f32 -> rows x
// (n/2+1) c64, zero-padding or truncating each row to the power of two n.
WXX_API int wxx_rfft(const float* x, void* X, int64_t rows, int64_t in_len, int64_t n) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && X, "null pointer");
  WXX_REQUIRE(rows >= 0 && in_len >= 0, "bad rfft dims");
  const int logn = log2_exact(n);
  WXX_REQUIRE(logn >= 0, "FFT length must be a positive power of two, got %lld", (long long)n);
  if (rows == 0) return WXX_OK;
  float2* Xc = static_cast<float2*>(X);
  if (logn - 1 > kMaxLogM) return wxx::rfft_four_step(x, Xc, rows, in_len, logn - 1);
  if (n == 1) {
    hipLaunchKernelGGL(rfft1_kernel, dim3(wxx::grid_1d(rows, 256)), dim3(256), 0, wxx::stream(),
                       x, Xc, rows, in_len);
  } else {
    const float2* tw = twiddles(logn - 1);
    if (!tw) return wxx::set_error(WXX_E_OOM, "rfft twiddle table allocation failed");
    const bool vec = in_len % 2 == 0 && (uintptr_t)x % 8 == 0;
    dispatch_rfft(logn - 1, x, Xc, tw, rows, in_len, vec);
  }
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.irfft (fft.py:566-645): rows x in_len c64 one-sided
// spectrum -> rows x out_len f32, the first out_len of the n samples of each
// row (n a power of two >= 2), each multiplied by post_scale after the 1/n
// normalisation.  out_len < n fuses the crop irfft(...)[..., :L] of the Hyena
// long convolution (nn/hyena.py:208-216); post_scale fuses the factor n of the
// rfft backward (autograd/utils.py:549-718).
WXX_API int wxx_irfft_crop(const void* X, float* x, int64_t rows, int64_t in_len, int64_t n,
                           int64_t out_len, float post_scale) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && X, "null pointer");
  WXX_REQUIRE(rows >= 0 && in_len >= 0, "bad irfft dims");
  const int logn = log2_exact(n);
  WXX_REQUIRE(logn >= 1, "irfft length must be a power of two >= 2, got %lld", (long long)n);
  WXX_REQUIRE(out_len >= 1 && out_len <= n, "irfft output length %lld not in [1, %lld]",
              (long long)out_len, (long long)n);
  if (rows == 0) return WXX_OK;
  if (logn - 1 > kMaxLogM)
    return wxx::irfft_four_step(static_cast<const float2*>(X), x, rows, in_len, logn - 1,
                                out_len, post_scale);
  const float2* tw = twiddles(logn - 1);
  if (!tw) return wxx::set_error(WXX_E_OOM, "irfft twiddle table allocation failed");
  RowOut ro{};
  ro.lim = out_len;
  ro.lim32 = (int)out_len;
  ro.half = (int)(out_len / 2);
  ro.post = post_scale;
  ro.mode = out_len == n ? 0 : (out_len % 2 == 0 ? 1 : 2);
  dispatch_irfft(logn - 1, static_cast<const float2*>(X), x, tw, rows, in_len, ro);
  WXX_LAUNCHED();
  return WXX_OK;
}

// functional.irfft without a crop: rows x n.
WXX_API int wxx_irfft(const void* X, float* x, int64_t rows, int64_t in_len, int64_t n) {
  return wxx_irfft_crop(X, x, rows, in_len, n, n, 1.0f);
}

// rfft with each output bin k multiplied by the real weight w_k = w_edge at
// k = 0 and k = n/2, w_mid between: the spectrum product of the irfft
// backward (reference autograd/utils.py:549-718, complex_mul of rfft(g) with
// the bin weights) fused into the transform's store.  The product rounds as
// wxx_complex_binary's does with the weight vector (w_k, 0), so the result is
// the bit pattern of wxx_rfft followed by that product.
WXX_API int wxx_rfft_mul(const float* x, void* X, int64_t rows, int64_t in_len, int64_t n,
                         float w_edge, float w_mid) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && X, "null pointer");
  WXX_REQUIRE(rows >= 0 && in_len >= 0, "bad rfft dims");
  const int logn = log2_exact(n);
  WXX_REQUIRE(logn >= 1 && logn - 1 <= kMaxLogM,
              "fused spectrum product needs a power-of-two n in [2, %d], got %lld",
              2 << kMaxLogM, (long long)n);
  if (rows == 0) return WXX_OK;
  const float2* tw = twiddles(logn - 1);
  if (!tw) return wxx::set_error(WXX_E_OOM, "rfft twiddle table allocation failed");
  const SpecMul sm{nullptr, 1, 0, 1, w_edge, w_mid, (int)(n / 2)};
  const bool vec = in_len % 2 == 0 && (uintptr_t)x % 8 == 0;
  dispatch_rfft(logn - 1, x, static_cast<float2*>(X), tw, rows, in_len, vec, &sm);
  WXX_LAUNCHED();
  return WXX_OK;
}

// wxx_irfft_crop of the product X * h * w, formed as the bins load: row r of
// X (in_len bins) times row r mod hrows of h (conjugated when conj_h; null h
// skips it) times, when weighted, the real bin weight (w_edge at bins 0 and
// n/2, w_mid between; in_len must then be n/2 + 1), products in that order
// and rounded as wxx_complex_binary's with the weight vector (w_k, 0).  Fuses the Hyena long convolution's
// spectrum product into its inverse transform (reference nn/hyena.py:208-216:
// irfft(rfft(x) * rfft(h))) and the filter product and bin weights of its
// backward into the rfft adjoint (autograd/utils.py:549-718).
WXX_API int wxx_irfft_mul(const void* X, const void* h, float* x, int64_t rows, int64_t in_len,
                          int64_t hrows, int conj_h, int weighted, float w_edge, float w_mid,
                          int64_t n, int64_t out_len, float post_scale) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && X, "null pointer");
  WXX_REQUIRE(rows >= 0 && in_len >= 0, "bad irfft dims");
  WXX_REQUIRE(!h || hrows >= 1, "operand rows must be >= 1, got %lld", (long long)hrows);
  const int logn = log2_exact(n);
  WXX_REQUIRE(logn >= 1 && logn - 1 <= kMaxLogM,
              "fused spectrum product needs a power-of-two n in [2, %d], got %lld",
              2 << kMaxLogM, (long long)n);
  WXX_REQUIRE(out_len >= 1 && out_len <= n, "irfft output length %lld not in [1, %lld]",
              (long long)out_len, (long long)n);
  WXX_REQUIRE(!weighted || in_len == n / 2 + 1,
              "bin weights need the n/2 + 1 = %lld bins of the spectrum, got %lld",
              (long long)(n / 2 + 1), (long long)in_len);
  if (rows == 0) return WXX_OK;
  const float2* tw = twiddles(logn - 1);
  if (!tw) return wxx::set_error(WXX_E_OOM, "irfft twiddle table allocation failed");
  RowOut ro{};
  ro.lim = out_len;
  ro.lim32 = (int)out_len;
  ro.half = (int)(out_len / 2);
  ro.post = post_scale;
  ro.mode = out_len == n ? 0 : (out_len % 2 == 0 ? 1 : 2);
  const SpecMul sm{static_cast<const float2*>(h), h ? hrows : 1, conj_h ? 1 : 0,
                   weighted ? 1 : 0, w_edge, w_mid, (int)(n / 2)};
  dispatch_irfft(logn - 1, static_cast<const float2*>(X), x, tw, rows, in_len, ro, &sm);
  WXX_LAUNCHED();
  return WXX_OK;
}

// out[i] = sum over b < batch of a[b n + i] * c[b n + i] (c conjugated when
// conj_c): the broadcast operand's gradient of complex_mul (reference
// autograd/utils.py:549-718, the product g * conj(a) summed to the filter's
// shape) in one pass, with the products and the summation order of
// wxx_complex_binary followed by wxx_reduce over the batch.
WXX_API int wxx_complex_mul_batch_sum(void* out, const void* a, const void* c, int64_t batch,
                                      int64_t n, int conj_c) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(out && a && c, "null pointer");
  WXX_REQUIRE(batch >= 1 && n >= 0, "bad batch-sum dims");
  if (n == 0) return WXX_OK;
  hipLaunchKernelGGL(complex_mul_batch_sum_kernel, dim3(wxx::grid_1d(n, 256, 16384)), dim3(256),
                     0, wxx::stream(), static_cast<float2*>(out), static_cast<const float2*>(a),
                     static_cast<const float2*>(c), batch, n, conj_c ? 1 : 0);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.complex_mul (fft.py:168-213, op 0, conj flags) and
// complex_add_inplace (fft.py:216-245, op 1; here out-of-place or with
// out == a).  Strides count complex elements; 0 = broadcast.
WXX_API int wxx_complex_binary(void* out, const void* a, const void* b, int rank,
                               const int64_t* shape, const int64_t* s_out, const int64_t* s_a,
                               const int64_t* s_b, int op, int conj_a, int conj_b) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(out && a && b && shape && s_out && s_a && s_b, "null pointer");
  WXX_REQUIRE(rank >= 0 && rank <= wxx::kMaxRank, "rank %d unsupported", rank);
  WXX_REQUIRE(op == 0 || op == 1, "bad complex op %d", op);
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) n *= shape[d];
  if (n == 0) return WXX_OK;
  const int64_t* ss[3] = {s_out, s_a, s_b};
  const wxx::ND nd = wxx::collapse(rank, shape, ss, 3);
  float2* o = static_cast<float2*>(out);
  const float2* pa = static_cast<const float2*>(a);
  const float2* pb = static_cast<const float2*>(b);
  const int ca = conj_a ? 1 : 0, cb = conj_b ? 1 : 0;
  if (nd.rank <= 2) {
    const int64_t cols = nd.shape[nd.rank - 1], rows = n / cols;
    // out and a one contiguous run of n, b the same run or one row broadcast
    const int c0 = nd.rank - 1;
    const bool flat_oa = nd.stride[0][c0] == 1 && nd.stride[1][c0] == 1 &&
                         (nd.rank == 1 || (nd.stride[0][0] == cols && nd.stride[1][0] == cols));
    const bool b_flat = nd.stride[2][c0] == 1 && (nd.rank == 1 || nd.stride[2][0] == cols);
    const bool b_row = nd.stride[2][c0] == 1 && nd.rank == 2 && nd.stride[2][0] == 0;
    const bool b_one = nd.stride[2][c0] == 0 && (nd.rank == 1 || nd.stride[2][0] == 0);
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (flat_oa && n % 2 == 0 && n < (int64_t(1) << 30) && al16(o) && al16(pa) &&
        ((b_flat && al16(pb)) || b_row || b_one)) {
      const int64_t n2 = n / 2;
      const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>((n2 + 1023) / 1024, 16384)));
      if (b_flat)
        hipLaunchKernelGGL(complex_binary_pairs_kernel<false>, grid, dim3(256), 0, wxx::stream(),
                           reinterpret_cast<float4*>(o), reinterpret_cast<const float4*>(pa), pb,
                           (int)n2, 1, op, ca, cb);
      else
        hipLaunchKernelGGL(complex_binary_pairs_kernel<true>, grid, dim3(256), 0, wxx::stream(),
                           reinterpret_cast<float4*>(o), reinterpret_cast<const float4*>(pa), pb,
                           (int)n2, b_one ? 1 : (int)cols, op, ca, cb);
      WXX_LAUNCHED();
      return WXX_OK;
    }
    const int64_t gy = std::min<int64_t>(rows, 65535);
    const int64_t gx = std::min<int64_t>((cols + 255) / 256, std::max<int64_t>(64, 16384 / gy));
    const dim3 grid((unsigned)gx, (unsigned)gy);
    hipLaunchKernelGGL(complex_binary_rows_kernel, grid, dim3(256), 0, wxx::stream(), o, pa, pb,
                       nd, rows, cols, op, ca, cb);
  } else if (n < (int64_t(1) << 31)) {
    hipLaunchKernelGGL(complex_binary_kernel<false>, dim3(wxx::grid_1d(n, 256, 16384)), dim3(256),
                       0, wxx::stream(), o, pa, pb, nd, n, op, ca, cb);
  } else {
    hipLaunchKernelGGL(complex_binary_kernel<true>, dim3(wxx::grid_1d(n, 256, 16384)), dim3(256),
                       0, wxx::stream(), o, pa, pb, nd, n, op, ca, cb);
  }
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.complex_conj (fft.py:248-292).
WXX_API int wxx_complex_conj(void* dst, const void* src, int rank, const int64_t* shape,
                             const int64_t* s_dst, const int64_t* s_src) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dst && src && shape && s_dst && s_src, "null pointer");
  WXX_REQUIRE(rank >= 0 && rank <= wxx::kMaxRank, "rank %d unsupported", rank);
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) n *= shape[d];
  if (n == 0) return WXX_OK;
  const int64_t* ss[2] = {s_dst, s_src};
  const wxx::ND nd = wxx::collapse(rank, shape, ss, 2);
  hipLaunchKernelGGL(complex_conj_kernel, dim3(wxx::grid_1d(n, 256, 16384)), dim3(256), 0,
                     wxx::stream(), static_cast<float2*>(dst), static_cast<const float2*>(src),
                     nd, n);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.complex_pad (fft.py:345-383): batch x in_len ->
// batch x out_len, zero-padded or truncated.
WXX_API int wxx_complex_pad(const void* src, void* dst, int64_t batch, int64_t in_len,
                            int64_t out_len) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(src && dst, "null pointer");
  WXX_REQUIRE(batch >= 0 && in_len >= 0 && out_len >= 0, "bad complex_pad dims");
  if (batch == 0 || out_len == 0) return WXX_OK;
  hipLaunchKernelGGL(complex_pad_kernel, dim3(wxx::grid_1d(batch * out_len, 256, 16384)),
                     dim3(256), 0, wxx::stream(), static_cast<const float2*>(src),
                     static_cast<float2*>(dst), batch, in_len, out_len);
  WXX_LAUNCHED();
  return WXX_OK;
}
