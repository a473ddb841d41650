// Elementwise and layout kernels: broadcast binary ops (out-of-place and in
// place), scalar ops, unary math / activation (+ local derivative) ops,
// clamp, equality, masked fill, the fused mul backward, strided gather
// ("contiguous"), strided assign / fill, scatter_zeros and unfold backward.
//
// Reference kernels and hosts:
//   pointwise/pointwise.wgsl:19-61, pointwise/_pointwise.wgsl:17-60,
//   pointwise/scalarpointwise.wgsl:17-72, pointwise/{abs,exp,log,negate,
//   rsqrt,sign,sqrt,square}.wgsl, activations/{relu,gelu,sigmoid,selu,sin,
//   cos}*.wgsl, helpers/{clamp,clampbackwards,equal,maskedfill,mul_backward,
//   contiguous,assign,scatter_zeros,unfolddx}.wgsl; hosts in
//   src/wxx/functional/pointwise.py, activations.py and utils.py.
//
// MI355X design: the reference decomposes every linear index with a div/mod
// per dimension.  Here the host first coalesces dimensions that are
// contiguous in every operand and drops size-1 dimensions, so the common
// cases (same-shape contiguous tensors, row/column broadcast, a permuted
// view) run as rank-1/2/3 loops; rank-1 unit-stride operands use float4
// accesses.  Index arithmetic is 32-bit whenever the tensor has fewer than
// 2^31 elements.
#include "common.h"
#include "nd.h"

#include <cmath>
#include <type_traits>

namespace {

constexpr int kBlock = 256;
using wxx::ND;
using wxx::collapse;
using wxx::offsets;
using wxx::offsets64;

// ---- binary ----------------------------------------------------------------
__device__ __forceinline__ float binop(int op, float a, float b) {
  switch (op) {
    case 1: return a - b;
    case 2: return a * b;
    case 3: return a / b;
    default: return a + b;
  }
}

// operands: 0 = out, 1 = a, 2 = b
template <bool BIG>
__global__ __launch_bounds__(kBlock) void binary_kernel(float* __restrict__ out,
                                                        const float* __restrict__ a,
                                                        const float* __restrict__ b, ND nd,
                                                        int64_t n, int op) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    int64_t off[3];
    if (BIG)
      offsets64<3>(nd, i, off);
    else
      offsets<3>(nd, i, off);
    out[off[0]] = binop(op, a[off[1]], b[off[2]]);
  }
}

__global__ __launch_bounds__(kBlock) void binary_flat4_kernel(float4* __restrict__ out,
                                                              const float4* __restrict__ a,
                                                              const float4* __restrict__ b,
                                                              int64_t n4, int op) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n4; i += step) {
    float4 x = a[i], y = b[i];
    out[i] = make_float4(binop(op, x.x, y.x), binop(op, x.y, y.y), binop(op, x.z, y.z),
                         binop(op, x.w, y.w));
  }
}

// Rank 2 (rows x cols) with unit column stride in every operand (b's row
// stride may be 0: a row broadcast): V consecutive columns per thread item
// through V-wide accesses (the host picks the widest that every row base
// allows), four items in flight per thread, 32-bit index arithmetic.
template <int V>
__global__ __launch_bounds__(kBlock) void binary_rows_kernel(float* __restrict__ out,
                                                             const float* __restrict__ a,
                                                             const float* __restrict__ b, int rows,
                                                             int cols, int so, int sa, int sb,
                                                             int op) {
  using T = typename std::conditional<V == 4, float4, typename std::conditional<V == 2, float2,
                                                                                float>::type>::type;
  const int cg = cols / V;  // items per row
  const int total = rows * cg, step = gridDim.x * kBlock;
  for (int t0 = blockIdx.x * kBlock + threadIdx.x; t0 < total; t0 += 4 * step) {
    T x[4], y[4];
    int oo[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = t0 + u * step;
      if (t < total) {
        const int r = t / cg, c = (t - r * cg) * V;
        x[u] = *reinterpret_cast<const T*>(a + r * sa + c);
        y[u] = *reinterpret_cast<const T*>(b + r * sb + c);
        oo[u] = r * so + c;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (t0 + u * step < total) {
        if constexpr (V == 4)
          *reinterpret_cast<float4*>(out + oo[u]) =
              make_float4(binop(op, x[u].x, y[u].x), binop(op, x[u].y, y[u].y),
                          binop(op, x[u].z, y[u].z), binop(op, x[u].w, y[u].w));
        else if constexpr (V == 2)
          *reinterpret_cast<float2*>(out + oo[u]) =
              make_float2(binop(op, x[u].x, y[u].x), binop(op, x[u].y, y[u].y));
        else
          out[oo[u]] = binop(op, x[u], y[u]);
      }
    }
  }
}

// (batch, M, N) with out and one operand row-major (unit stride along N) and
// the other column-major (unit stride along M, a transposed view): 64 x 64
// tiles, the column-major operand read along M into LDS and read back along N,
// so every global access runs along an operand's unit stride.  tr = 1: a is
// the column-major operand, 2: b.
__global__ __launch_bounds__(kBlock) void binary_transposed_kernel(
    float* __restrict__ out, const float* __restrict__ a, const float* __restrict__ b, int M,
    int N, int tiles_n, int64_t so0, int64_t so1, int64_t sa0, int64_t sa1, int64_t sa2,
    int64_t sb0, int64_t sb1, int64_t sb2, int tr, int op) {
  __shared__ float t[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
  const int m0 = tm * 64, n0 = tn * 64;
  const int64_t bt = blockIdx.y;
  const float* T = tr == 1 ? a + bt * sa0 : b + bt * sb0;  // column-major: unit stride along M
  const int64_t tsn = tr == 1 ? sa2 : sb2;
  const float* R = tr == 1 ? b + bt * sb0 : a + bt * sa0;  // row-major: unit stride along N
  const int64_t rsm = tr == 1 ? sb1 : sa1;
  // Indices past the edge are clamped into the tensor rather than guarded, so
  // every load is unconditional and all of a thread's loads (both operands)
  // issue before the first wait; a guarded load sits behind a branch of its
  // own and waits alone.  Clamped values reach no stored output.
  float tl[16], rv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int n = min(n0 + ty + 4 * i, N - 1), m = min(m0 + tx, M - 1);
    tl[i] = T[(int64_t)n * tsn + m];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int m = min(m0 + ty + 4 * i, M - 1), n = min(n0 + tx, N - 1);
    rv[i] = R[(int64_t)m * rsm + n];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) t[ty + 4 * i][tx] = tl[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = ty + 4 * i;
    const int m = m0 + r, n = n0 + tx;
    if (m < M && n < N) {
      const float tv = t[tx][r];
      out[bt * so0 + (int64_t)m * so1 + n] =
          tr == 1 ? binop(op, tv, rv[i]) : binop(op, rv[i], tv);
    }
  }
}

// ---- scalar / unary ----------------------------------------------------------
__device__ __forceinline__ float scalar_op(int op, float x, float c, int rev) {
  switch (op) {
    case 0: return x + c;
    case 1: return rev ? c - x : x - c;
    case 2: return x * c;
    case 3: {
      if (rev) return powf(c, x);
      if (x < 0.f) {
        if (c == truncf(c)) {
          const float mag = powf(-x, c);
          const bool odd = fmodf(fabsf(c) * 0.5f, 1.0f) > 0.25f;
          return odd ? -mag : mag;
        }
        return __int_as_float(0x7fc00000);
      }
      return powf(x, c);
    }
    case 4: return rev ? c / x : x / c;
    default: return x;
  }
}

enum Unary {
  U_RELU = 0, U_RELU_BWD, U_GELU, U_GELU_BWD, U_SIGMOID, U_SIGMOID_BWD, U_SELU, U_SELU_BWD,
  U_SIN, U_SIN_BWD, U_COS, U_COS_BWD, U_ABS, U_EXP, U_LOG, U_NEG, U_RSQRT, U_SIGN, U_SQRT,
  U_SQUARE, U_COUNT
};

constexpr float kSqrt2OverPi = 0.7978845608f;
constexpr float kGeluC = 0.044715f;
constexpr float kGeluDC = 0.134145f;
constexpr float kSeluAlpha = 1.6732632423543772848170429916717f;
constexpr float kSeluScale = 1.0507009873554804934193349852946f;

__device__ __forceinline__ float unary_op(int op, float x) {
  switch (op) {
    case U_RELU: return fmaxf(0.f, x);
    case U_RELU_BWD: return x > 0.f ? 1.f : 0.f;
    case U_GELU: {
      if (x > 10.f) return x;
      if (x < -10.f) return 0.f;
      const float u = kSqrt2OverPi * (x + kGeluC * x * x * x);
      return 0.5f * x * (1.f + tanhf(u));
    }
    case U_GELU_BWD: {
      if (x > 10.f) return 1.f;
      if (x < -10.f) return 0.f;
      const float u = kSqrt2OverPi * (x + kGeluC * x * x * x);
      const float t = tanhf(u);
      const float du = kSqrt2OverPi * (1.f + kGeluDC * x * x);
      return 0.5f * (1.f + t) + 0.5f * x * (1.f - t * t) * du;
    }
    case U_SIGMOID: {
      const float xc = fminf(fmaxf(x, -88.f), 88.f);
      return 1.f / (1.f + expf(-xc));
    }
    case U_SIGMOID_BWD: return x * (1.f - x);
    case U_SELU: return x > 0.f ? kSeluScale * x : kSeluScale * kSeluAlpha * (expf(x) - 1.f);
    case U_SELU_BWD: return x > 0.f ? kSeluScale : kSeluScale * kSeluAlpha * expf(x);
    case U_SIN: return sinf(x);
    case U_SIN_BWD: return cosf(x);
    case U_COS: return cosf(x);
    case U_COS_BWD: return -sinf(x);
    case U_ABS: return fabsf(x);
    case U_EXP: return expf(x);
    case U_LOG: return logf(x);
    case U_NEG: return -x;
    case U_RSQRT: return rsqrtf(x);
    case U_SIGN: return x > 0.f ? 1.f : (x < 0.f ? -1.f : 0.f);
    case U_SQRT: return sqrtf(x);
    case U_SQUARE: return x * x;
    default: return x;
  }
}

template <int OP>
__global__ __launch_bounds__(kBlock) void unary_kernel(const float* __restrict__ x,
                                                       float* __restrict__ y, int64_t n,
                                                       int vec) {
  const int64_t n4 = vec ? n >> 2 : 0;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4* y4 = reinterpret_cast<float4*>(y);
  for (int64_t i = t; i < n4; i += step) {
    float4 v = x4[i];
    y4[i] = make_float4(unary_op(OP, v.x), unary_op(OP, v.y), unary_op(OP, v.z),
                        unary_op(OP, v.w));
  }
  for (int64_t i = (n4 << 2) + t; i < n; i += step) y[i] = unary_op(OP, x[i]);
}

// out = f'(x) * g with f' given by a derivative op code (bit-identical to
// computing the derivative tensor and multiplying it by g).
template <int OP>
__global__ __launch_bounds__(kBlock) void unary_bwd_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ g,
                                                           float* __restrict__ y, int64_t n,
                                                           int vec) {
  const int64_t n4 = vec ? n >> 2 : 0;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  const float4* g4 = reinterpret_cast<const float4*>(g);
  float4* y4 = reinterpret_cast<float4*>(y);
  for (int64_t i = t; i < n4; i += step) {
    const float4 v = x4[i], w = g4[i];
    y4[i] = make_float4(unary_op(OP, v.x) * w.x, unary_op(OP, v.y) * w.y,
                        unary_op(OP, v.z) * w.z, unary_op(OP, v.w) * w.w);
  }
  for (int64_t i = (n4 << 2) + t; i < n; i += step) y[i] = unary_op(OP, x[i]) * g[i];
}

// SwiGLU's gate h = (sigmoid(a) a) b in one pass instead of the sigmoid,
// a s and g b kernels, every operation rounded as those kernels round it:
// contraction is off in these helpers (__fmul_rn / __fadd_rn are plain
// operators here, which the compiler may fuse into an fma), as it is across
// the separate kernels.
__device__ __forceinline__ float swiglu_h(float a, float b) {
#pragma clang fp contract(off)
  const float s = unary_op(U_SIGMOID, a);
  return (s * a) * b;
}

// Its backward from dh: with s and g = s a recomputed, db = dh g, dg = dh b,
// da = dg s + sigmoid'(s) (dg a) -- the products and the sum of the mul,
// mul and sigmoid backwards and the gradient accumulation they replace.
__device__ __forceinline__ void swiglu_dab(float dh, float a, float b, float& da, float& db) {
#pragma clang fp contract(off)
  const float s = unary_op(U_SIGMOID, a);
  const float g = s * a;
  db = dh * g;
  const float dg = dh * b;
  const float ds = dg * a;
  const float t1 = dg * s, t2 = unary_op(U_SIGMOID_BWD, s) * ds;
  da = t1 + t2;
}

__global__ __launch_bounds__(kBlock) void swiglu_gate_kernel(const float* __restrict__ a,
                                                             const float* __restrict__ b,
                                                             float* __restrict__ h, int64_t n,
                                                             int vec) {
  const int64_t n4 = vec ? n >> 2 : 0;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  for (int64_t i = t; i < n4; i += step) {
    const float4 x = reinterpret_cast<const float4*>(a)[i];
    const float4 y = reinterpret_cast<const float4*>(b)[i];
    reinterpret_cast<float4*>(h)[i] = make_float4(swiglu_h(x.x, y.x), swiglu_h(x.y, y.y),
                                                  swiglu_h(x.z, y.z), swiglu_h(x.w, y.w));
  }
  for (int64_t i = (n4 << 2) + t; i < n; i += step) h[i] = swiglu_h(a[i], b[i]);
}

__global__ __launch_bounds__(kBlock) void swiglu_gate_bwd_kernel(
    const float* __restrict__ dh, const float* __restrict__ a, const float* __restrict__ b,
    float* __restrict__ da, float* __restrict__ db, int64_t n, int vec) {
  const int64_t n4 = vec ? n >> 2 : 0;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  for (int64_t i = t; i < n4; i += step) {
    const float4 g = reinterpret_cast<const float4*>(dh)[i];
    const float4 x = reinterpret_cast<const float4*>(a)[i];
    const float4 y = reinterpret_cast<const float4*>(b)[i];
    float4 ra, rb;
    swiglu_dab(g.x, x.x, y.x, ra.x, rb.x);
    swiglu_dab(g.y, x.y, y.y, ra.y, rb.y);
    swiglu_dab(g.z, x.z, y.z, ra.z, rb.z);
    swiglu_dab(g.w, x.w, y.w, ra.w, rb.w);
    reinterpret_cast<float4*>(da)[i] = ra;
    reinterpret_cast<float4*>(db)[i] = rb;
  }
  for (int64_t i = (n4 << 2) + t; i < n; i += step) swiglu_dab(dh[i], a[i], b[i], da[i], db[i]);
}

// dst[i] = src[offset(i)] * scale for a dense dst over `shape` (broadcast read).
__global__ __launch_bounds__(kBlock) void broadcast_scale_kernel(float* __restrict__ dst,
                                                                 const float* __restrict__ src,
                                                                 ND nd, int64_t n, float scale) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    int64_t off[2];
    offsets64<2>(nd, i, off);
    dst[off[0]] = src[off[1]] * scale;
  }
}

__global__ __launch_bounds__(kBlock) void scalar_kernel(const float* __restrict__ x,
                                                        float* __restrict__ y, int64_t n, int op,
                                                        float c, int rev, int vec) {
  const int64_t n4 = vec ? n >> 2 : 0;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4* y4 = reinterpret_cast<float4*>(y);
  for (int64_t i = t; i < n4; i += step) {
    float4 v = x4[i];
    y4[i] = make_float4(scalar_op(op, v.x, c, rev), scalar_op(op, v.y, c, rev),
                        scalar_op(op, v.z, c, rev), scalar_op(op, v.w, c, rev));
  }
  for (int64_t i = (n4 << 2) + t; i < n; i += step) y[i] = scalar_op(op, x[i], c, rev);
}

// mode 0: clamp; 1: clamp backward mask; 2: masked fill (x != 0 ? x : lo)
__global__ __launch_bounds__(kBlock) void clamp_kernel(const float* __restrict__ x,
                                                       float* __restrict__ y, int64_t n, float lo,
                                                       float hi, int mode) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    const float v = x[i];
    float r;
    if (mode == 0)
      r = fminf(fmaxf(v, lo), hi);
    else if (mode == 1)
      r = (v >= lo && v <= hi) ? 1.f : 0.f;
    else
      r = v != 0.f ? v : lo;
    y[i] = r;
  }
}

// mode 0: f32 == f32, 1: u32 == u32, 2: f32 == scalar bits, 3: u32 == scalar
__global__ __launch_bounds__(kBlock) void equal_kernel(const uint32_t* __restrict__ a,
                                                       const uint32_t* __restrict__ b,
                                                       float* __restrict__ out, int64_t n,
                                                       int mode, uint32_t number) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    const uint32_t x = a[i];
    bool eq;
    switch (mode) {
      case 0: eq = __uint_as_float(x) == __uint_as_float(b[i]); break;
      case 1: eq = x == b[i]; break;
      case 2: eq = __uint_as_float(x) == __uint_as_float(number); break;
      default: eq = x == number; break;
    }
    out[i] = eq ? 1.f : 0.f;
  }
}

__global__ __launch_bounds__(kBlock) void mul_backward_kernel(const float* __restrict__ g,
                                                              const float* __restrict__ a,
                                                              const float* __restrict__ b,
                                                              float* __restrict__ da,
                                                              float* __restrict__ db, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    const float gv = g[i];
    da[i] = gv * b[i];
    db[i] = gv * a[i];
  }
}

__global__ __launch_bounds__(kBlock) void mul_backward4_kernel(const float4* __restrict__ g,
                                                               const float4* __restrict__ a,
                                                               const float4* __restrict__ b,
                                                               float4* __restrict__ da,
                                                               float4* __restrict__ db,
                                                               int64_t n4) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n4; i += step) {
    const float4 gv = g[i], av = a[i], bv = b[i];
    da[i] = make_float4(gv.x * bv.x, gv.y * bv.y, gv.z * bv.z, gv.w * bv.w);
    db[i] = make_float4(gv.x * av.x, gv.y * av.y, gv.z * av.z, gv.w * av.w);
  }
}

// ---- layout -------------------------------------------------------------------
// dst (operand 0) and src (operand 1) both strided; element type T.
template <typename T, bool BIG>
__global__ __launch_bounds__(kBlock) void copy_strided_kernel(T* __restrict__ dst,
                                                              const T* __restrict__ src, ND nd,
                                                              int64_t n) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    int64_t off[2];
    if (BIG)
      offsets64<2>(nd, i, off);
    else
      offsets<2>(nd, i, off);
    dst[off[0]] = src[off[1]];
  }
}

// 16 bytes moved as one element by copy_strided_kernel (dwordx4 accesses).
struct alignas(16) Quad {
  uint32_t x, y, z, w;
};

template <typename T>
__global__ __launch_bounds__(kBlock) void fill_strided_kernel(T* __restrict__ dst, ND nd,
                                                              int64_t n, T v) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    int64_t off[1];
    offsets64<1>(nd, i, off);
    dst[off[0]] = v;
  }
}

// Tiled transpose of the two innermost collapsed dims (the source is unit
// stride along rows, the destination along columns): read 64x64 tiles
// coalesced, write coalesced through LDS.
template <typename T>
__global__ __launch_bounds__(kBlock) void transpose_tile_kernel(T* __restrict__ dst,
                                                                const T* __restrict__ src,
                                                                int64_t batch, int64_t rows,
                                                                int64_t cols, int64_t sb,
                                                                int64_t sr, int64_t sc,
                                                                int64_t db, int64_t dr) {
  // dst[b*db + r*dr + c] = src[b*sb + r*sr + c*sc], with sr == 1 expected
  // (fast read along r).  Tile: 64 (r) x 64 (c).
  __shared__ T tile[64][65];
  const int64_t b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
  // edge indices clamped into the tensor instead of guarded: every load is
  // unconditional and all 16 issue before the first wait (a guarded load sits
  // behind a branch of its own and waits alone); clamped values reach no store
  T tl[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t c = min(c0 + ty + 4 * i, cols - 1), r = min(r0 + tx, rows - 1);
    tl[i] = src[b * sb + r * sr + c * sc];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) tile[ty + 4 * i][tx] = tl[i];
  __syncthreads();
  for (int k = ty; k < 64; k += 4) {
    const int64_t r = r0 + k, c = c0 + tx;
    if (r < rows && c < cols) dst[b * db + r * dr + c] = tile[tx][k];
  }
}

__global__ __launch_bounds__(kBlock) void scatter_zeros_kernel(float* __restrict__ out,
                                                               const float* __restrict__ grad,
                                                               ND nd, int64_t n, int dim,
                                                               int64_t start, int64_t length) {
  // nd.shape = output shape (uncollapsed), nd.stride[0] = grad strides.
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    int64_t rem = i, off = 0;
    bool in = true;
    for (int d = nd.rank - 1; d >= 0; --d) {
      const int64_t sz = nd.shape[d];
      const int64_t q = rem / sz;
      int64_t c = rem - q * sz;
      rem = q;
      if (d == dim) {
        if (c < start || c >= start + length) {
          in = false;
        } else {
          c -= start;
        }
      }
      off += c * nd.stride[0][d];
    }
    float v = 0.f;
    if (in) v = grad[off];
    out[i] = v;
  }
}

__global__ __launch_bounds__(kBlock) void unfolddx_kernel(const float* __restrict__ dy,
                                                          float* __restrict__ dx, int64_t prefix,
                                                          int64_t length, int64_t suffix,
                                                          int64_t windows, int64_t size,
                                                          int64_t stepw) {
  const int64_t total = prefix * length * suffix;
  int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t gstep = (int64_t)gridDim.x * kBlock;
  for (; idx < total; idx += gstep) {
    const int64_t s = idx % suffix;
    const int64_t nn = (idx / suffix) % length;
    const int64_t p = idx / (suffix * length);
    float acc = 0.f;
    for (int64_t w = 0; w < size; ++w) {
      if (nn >= w) {
        const int64_t pos = nn - w;
        if (pos % stepw == 0) {
          const int64_t l = pos / stepw;
          if (l < windows) acc += dy[((p * windows + l) * suffix + s) * size + w];
        }
      }
    }
    dx[idx] = acc;
  }
}

inline unsigned grid_for(int64_t n) { return wxx::grid_1d(n, kBlock, 16384); }

bool fits32(const ND& nd, int64_t n) {
  if (n >= (int64_t(1) << 31)) return false;
  for (int d = 0; d < nd.rank; ++d)
    if (nd.shape[d] >= (int64_t(1) << 31)) return false;
  return true;
}

// Rank 2 or 3 (batch, M, N) with out row-major along N (unit stride), one of
// a / b row-major along N and the other with unit stride along M: returns
// 1 (a column-major) or 2 (b column-major), else 0.  Batches fit grid y and
// M, N fit 32 bits.
int transposed_pair(const ND& nd) {
  if (nd.rank != 2 && nd.rank != 3) return 0;
  const int r3 = nd.rank == 3;
  const int im = r3, in = r3 + 1;
  if (nd.shape[im] < 2 || nd.shape[in] < 2 || nd.shape[im] >= (int64_t(1) << 31) ||
      nd.shape[in] >= (int64_t(1) << 31) || (r3 && nd.shape[0] > 65535))
    return 0;
  if (nd.stride[0][in] != 1) return 0;
  const bool a_row = nd.stride[1][in] == 1, b_row = nd.stride[2][in] == 1;
  const bool a_col = nd.stride[1][im] == 1, b_col = nd.stride[2][im] == 1;
  if (b_row && a_col && !a_row) return 1;
  if (a_row && b_col && !b_row) return 2;
  return 0;
}

// Every offset r * row_stride + c of a rank-2 view stays below 2^31.
bool rows_fit32(const ND& nd) {
  for (int k = 0; k < 3; ++k) {
    const int64_t st = nd.stride[k][0];
    if (st < 0 || (nd.shape[0] - 1) * st + nd.shape[1] >= (int64_t(1) << 31)) return false;
  }
  return true;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

// out = a op b with broadcasting; a/b/out strides in elements over the
// output shape (0 for broadcast dims).  op: 0 add, 1 sub, 2 mul, 3 div.
// Replaces functional.pointwise (reference src/wxx/functional/pointwise.py:29-98)
// and, with out == a, functional._pointwise (pointwise.py:231-289).
WXX_API int wxx_pointwise(float* out, const float* a, const float* b, int rank,
                          const int64_t* shape, const int64_t* s_out, const int64_t* s_a,
                          const int64_t* s_b, int op) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(out && a && b && shape && s_out && s_a && s_b, "null pointer");
  WXX_REQUIRE(rank >= 0 && rank <= wxx::kMaxRank, "rank %d unsupported", rank);
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) n *= shape[d];
  if (n == 0) return WXX_OK;
  const int64_t* ss[3] = {s_out, s_a, s_b};
  ND nd = collapse(rank, shape, ss, 3);
  hipStream_t s = wxx::stream();
  if (nd.rank == 1 && nd.stride[0][0] == 1 && nd.stride[1][0] == 1 && nd.stride[2][0] == 1 &&
      n % 4 == 0 && ((uintptr_t)out | (uintptr_t)a | (uintptr_t)b) % 16 == 0) {
    hipLaunchKernelGGL(binary_flat4_kernel, dim3(grid_for(n / 4)), dim3(kBlock), 0, s,
                       (float4*)out, (const float4*)a, (const float4*)b, n / 4, op);
  } else if (transposed_pair(nd) != 0) {
    // one operand a transposed view of the others' layout
    const int tr = transposed_pair(nd);
    const int r3 = nd.rank == 3;
    const int64_t B = r3 ? nd.shape[0] : 1, M = nd.shape[r3], N = nd.shape[r3 + 1];
    const int tiles_n = (int)((N + 63) / 64);
    const dim3 grid((unsigned)(((M + 63) / 64) * tiles_n), (unsigned)B);
    hipLaunchKernelGGL(binary_transposed_kernel, grid, dim3(kBlock), 0, s, out, a, b, (int)M,
                       (int)N, tiles_n, r3 ? nd.stride[0][0] : 0, nd.stride[0][r3],
                       r3 ? nd.stride[1][0] : 0, nd.stride[1][r3], nd.stride[1][r3 + 1],
                       r3 ? nd.stride[2][0] : 0, nd.stride[2][r3], nd.stride[2][r3 + 1], tr, op);
  } else if (nd.rank == 2 && nd.stride[0][1] == 1 && nd.stride[1][1] == 1 &&
             nd.stride[2][1] == 1 && fits32(nd, n) && rows_fit32(nd)) {
    // rows of unit stride (a strided view's rows, a row broadcast): the
    // widest access every row base and the row length allow
    const int rows = (int)nd.shape[0], cols = (int)nd.shape[1];
    const int64_t so = nd.stride[0][0], sa = nd.stride[1][0], sb = nd.stride[2][0];
    auto fits = [&](int v) {
      const uintptr_t bytes = 4 * (uintptr_t)v;
      return cols % v == 0 && so % v == 0 && sa % v == 0 && sb % v == 0 &&
             ((uintptr_t)out | (uintptr_t)a | (uintptr_t)b) % bytes == 0;
    };
    if (fits(4))
      hipLaunchKernelGGL(binary_rows_kernel<4>, dim3(grid_for(n / 16)), dim3(kBlock), 0, s, out,
                         a, b, rows, cols, (int)so, (int)sa, (int)sb, op);
    else if (fits(2))
      hipLaunchKernelGGL(binary_rows_kernel<2>, dim3(grid_for(n / 8)), dim3(kBlock), 0, s, out,
                         a, b, rows, cols, (int)so, (int)sa, (int)sb, op);
    else
      hipLaunchKernelGGL(binary_rows_kernel<1>, dim3(grid_for(n / 4)), dim3(kBlock), 0, s, out,
                         a, b, rows, cols, (int)so, (int)sa, (int)sb, op);
  } else if (fits32(nd, n)) {
    hipLaunchKernelGGL(binary_kernel<false>, dim3(grid_for(n)), dim3(kBlock), 0, s, out, a, b,
                       nd, n, op);
  } else {
    hipLaunchKernelGGL(binary_kernel<true>, dim3(grid_for(n)), dim3(kBlock), 0, s, out, a, b, nd,
                       n, op);
  }
  WXX_LAUNCHED();
  return WXX_OK;
}

// y = x op c (or c op x when reverse); op: 0 add, 1 sub, 2 mul, 3 pow, 4 div.
// Replaces functional.scalarpointwise (reference pointwise.py:101-146).
WXX_API int wxx_scalarpointwise(const float* x, float* y, int64_t n, int op, float c,
                                int reverse) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && y, "null pointer");
  WXX_REQUIRE(op >= 0 && op <= 4, "bad scalar op %d", op);
  if (n <= 0) return WXX_OK;
  const int vec = ((uintptr_t)x | (uintptr_t)y) % 16 == 0;
  hipLaunchKernelGGL(scalar_kernel, dim3(grid_for((n + 3) / 4)), dim3(kBlock), 0, wxx::stream(),
                     x, y, n, op, c, reverse, vec);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Unary op on a contiguous tensor; op numbering in the Unary enum above
// (relu, relu', gelu, gelu', sigmoid, sigmoid'(from y), selu, selu', sin,
// sin', cos, cos', abs, exp, log, neg, rsqrt, sign, sqrt, square).
// Replaces the _unary_op family (reference src/wxx/backend/dispatch.py:59-89,
// functional/activations.py:22-124, functional/pointwise.py:293-354).
WXX_API int wxx_unary(const float* x, float* y, int64_t n, int op) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && y, "null pointer");
  WXX_REQUIRE(op >= 0 && op < U_COUNT, "bad unary op %d", op);
  if (n <= 0) return WXX_OK;
  const int vec = ((uintptr_t)x | (uintptr_t)y) % 16 == 0;
  dim3 grid(grid_for((n + 3) / 4));
  hipStream_t s = wxx::stream();
#define WXX_UCASE(OP) \
  case OP: hipLaunchKernelGGL(unary_kernel<OP>, grid, dim3(kBlock), 0, s, x, y, n, vec); break;
  switch (op) {
    WXX_UCASE(U_RELU) WXX_UCASE(U_RELU_BWD) WXX_UCASE(U_GELU) WXX_UCASE(U_GELU_BWD)
    WXX_UCASE(U_SIGMOID) WXX_UCASE(U_SIGMOID_BWD) WXX_UCASE(U_SELU) WXX_UCASE(U_SELU_BWD)
    WXX_UCASE(U_SIN) WXX_UCASE(U_SIN_BWD) WXX_UCASE(U_COS) WXX_UCASE(U_COS_BWD)
    WXX_UCASE(U_ABS) WXX_UCASE(U_EXP) WXX_UCASE(U_LOG) WXX_UCASE(U_NEG) WXX_UCASE(U_RSQRT)
    WXX_UCASE(U_SIGN) WXX_UCASE(U_SQRT) WXX_UCASE(U_SQUARE)
    default: break;
  }
#undef WXX_UCASE
  WXX_LAUNCHED();
  return WXX_OK;
}

// Fused local derivative times gradient: out = f'(x) * g, where op is the
// derivative's Unary code (relu', gelu', sigmoid' (from y), selu', sin',
// cos').  Replaces the derivative kernel + pointwise multiply pair that the
// reference's activation backwards issue (reference
// src/wxx/autograd/pointwise.py:291-388).
WXX_API int wxx_unary_backward(const float* x, const float* g, float* y, int64_t n, int op) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && g && y, "null pointer");
  WXX_REQUIRE(op >= 0 && op < U_COUNT, "bad unary op %d", op);
  if (n <= 0) return WXX_OK;
  const int vec = ((uintptr_t)x | (uintptr_t)g | (uintptr_t)y) % 16 == 0;
  dim3 grid(grid_for((n + 3) / 4));
  hipStream_t s = wxx::stream();
#define WXX_UBCASE(OP) \
  case OP: hipLaunchKernelGGL(unary_bwd_kernel<OP>, grid, dim3(kBlock), 0, s, x, g, y, n, vec); break;
  switch (op) {
    WXX_UBCASE(U_RELU_BWD) WXX_UBCASE(U_GELU_BWD) WXX_UBCASE(U_SIGMOID_BWD)
    WXX_UBCASE(U_SELU_BWD) WXX_UBCASE(U_SIN_BWD) WXX_UBCASE(U_COS_BWD)
    default: return wxx::set_error(WXX_E_ARG, "op %d is not a derivative op", op);
  }
#undef WXX_UBCASE
  WXX_LAUNCHED();
  return WXX_OK;
}

// dst (dense over `shape`) = src read through s_src (0 = broadcast) * scale.
// Replaces the ones_like * grad products of sum/mean backward (reference
// src/wxx/autograd/reductions.py:38-95).
WXX_API int wxx_broadcast_scale(float* dst, const float* src, int rank, const int64_t* shape,
                                const int64_t* s_src, float scale) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dst && src && shape && s_src, "null pointer");
  WXX_REQUIRE(rank >= 0 && rank <= wxx::kMaxRank, "rank %d unsupported", rank);
  int64_t n = 1;
  int64_t dense[wxx::kMaxRank];
  for (int d = rank - 1; d >= 0; --d) {
    dense[d] = n;
    n *= shape[d];
  }
  if (n == 0) return WXX_OK;
  const int64_t* ss[2] = {dense, s_src};
  ND nd = collapse(rank, shape, ss, 2);
  hipLaunchKernelGGL(broadcast_scale_kernel, dim3(grid_for(n)), dim3(kBlock), 0, wxx::stream(),
                     dst, src, nd, n, scale);
  WXX_LAUNCHED();
  return WXX_OK;
}

// mode 0: clamp (reference helpers/clamp.wgsl); 1: clamp backward mask
// (clampbackwards.wgsl); 2: masked fill with `lo` (maskedfill.wgsl).
WXX_API int wxx_clamp(const float* x, float* y, int64_t n, float lo, float hi, int mode) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && y, "null pointer");
  WXX_REQUIRE(mode >= 0 && mode <= 2, "bad clamp mode %d", mode);
  if (n <= 0) return WXX_OK;
  hipLaunchKernelGGL(clamp_kernel, dim3(grid_for(n)), dim3(kBlock), 0, wxx::stream(), x, y, n,
                     lo, hi, mode);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.equal / equal_number (reference functional/utils.py:502-556).
WXX_API int wxx_equal(const void* a, const void* b, float* out, int64_t n, int mode,
                      uint32_t number) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(a && out && (mode >= 2 || b), "null pointer");
  WXX_REQUIRE(mode >= 0 && mode <= 3, "bad equal mode %d", mode);
  if (n <= 0) return WXX_OK;
  hipLaunchKernelGGL(equal_kernel, dim3(grid_for(n)), dim3(kBlock), 0, wxx::stream(),
                     (const uint32_t*)a, (const uint32_t*)(b ? b : a), out, n, mode, number);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.mul_backward (reference pointwise.py:460-502).
WXX_API int wxx_mul_backward(const float* g, const float* a, const float* b, float* da,
                             float* db, int64_t n) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(g && a && b && da && db, "null pointer");
  if (n <= 0) return WXX_OK;
  if (n % 4 == 0 && ((uintptr_t)g | (uintptr_t)a | (uintptr_t)b | (uintptr_t)da | (uintptr_t)db) %
                            16 == 0)
    hipLaunchKernelGGL(mul_backward4_kernel, dim3(grid_for(n / 4)), dim3(kBlock), 0,
                       wxx::stream(), (const float4*)g, (const float4*)a, (const float4*)b,
                       (float4*)da, (float4*)db, n / 4);
  else
    hipLaunchKernelGGL(mul_backward_kernel, dim3(grid_for(n)), dim3(kBlock), 0, wxx::stream(), g,
                       a, b, da, db, n);
  WXX_LAUNCHED();
  return WXX_OK;
}

// dst (strided view) <- src (strided view), element size 4 or 8 bytes.
// With s_dst row-major this is functional.contiguous (reference
// functional/utils.py:316-369, fft.py:295-342); otherwise functional.assign
// from a tensor (utils.py:29-101).
WXX_API int wxx_copy_strided(void* dst, const void* src, int itemsize, int rank,
                             const int64_t* shape, const int64_t* s_dst, const int64_t* s_src) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dst && src && shape && s_dst && s_src, "null pointer");
  WXX_REQUIRE(itemsize == 4 || itemsize == 8, "itemsize %d unsupported", itemsize);
  WXX_REQUIRE(rank >= 0 && rank <= wxx::kMaxRank, "rank %d unsupported", rank);
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) n *= shape[d];
  if (n == 0) return WXX_OK;
  const int64_t* ss[2] = {s_dst, s_src};
  ND nd = collapse(rank, shape, ss, 2);
  hipStream_t s = wxx::stream();
  // Transpose-shaped copy: destination unit stride along the innermost dim,
  // source unit stride along the next one -> LDS-tiled transpose (the
  // destination may be a strided view, e.g. a slice being assigned).
  if (nd.rank >= 2 && nd.rank <= 3 && nd.stride[0][nd.rank - 1] == 1 &&
      nd.stride[1][nd.rank - 2] == 1 && nd.stride[1][nd.rank - 1] != 1) {
    const int64_t rows = nd.shape[nd.rank - 2], cols = nd.shape[nd.rank - 1];
    const int64_t batch = nd.rank == 3 ? nd.shape[0] : 1;
    const int64_t sb = nd.rank == 3 ? nd.stride[1][0] : 0;
    const int64_t db = nd.rank == 3 ? nd.stride[0][0] : 0, dr = nd.stride[0][nd.rank - 2];
    if (batch <= 65535 && (rows + 63) / 64 <= 65535) {
      dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64), (unsigned)batch);
      if (itemsize == 4)
        hipLaunchKernelGGL(transpose_tile_kernel<uint32_t>, grid, dim3(kBlock), 0, s,
                           (uint32_t*)dst, (const uint32_t*)src, batch, rows, cols, sb,
                           nd.stride[1][nd.rank - 2], nd.stride[1][nd.rank - 1], db, dr);
      else
        hipLaunchKernelGGL(transpose_tile_kernel<uint64_t>, grid, dim3(kBlock), 0, s,
                           (uint64_t*)dst, (const uint64_t*)src, batch, rows, cols, sb,
                           nd.stride[1][nd.rank - 2], nd.stride[1][nd.rank - 1], db, dr);
      WXX_LAUNCHED();
      return WXX_OK;
    }
  }
  // Both views unit stride along the innermost dim, whose length and every
  // outer stride are multiples of 4, on 16-byte aligned bases (e.g. the
  // attention head split / merge permutes, 64 contiguous floats per head):
  // copy 16-byte quads, a quarter of the index arithmetic per byte.
  if (itemsize == 4 && nd.stride[0][nd.rank - 1] == 1 && nd.stride[1][nd.rank - 1] == 1 &&
      nd.shape[nd.rank - 1] % 4 == 0 && ((uintptr_t)dst & 15) == 0 &&
      ((uintptr_t)src & 15) == 0) {
    bool quads = true;
    for (int d = 0; d + 1 < nd.rank; ++d)
      quads = quads && nd.stride[0][d] % 4 == 0 && nd.stride[1][d] % 4 == 0;
    if (quads) {
      ND q = nd;
      q.shape[q.rank - 1] /= 4;
      for (int d = 0; d + 1 < q.rank; ++d) {
        q.stride[0][d] /= 4;
        q.stride[1][d] /= 4;
      }
      const int64_t nq = n / 4;
      if (!fits32(q, nq))
        hipLaunchKernelGGL((copy_strided_kernel<Quad, true>), dim3(grid_for(nq)), dim3(kBlock), 0,
                           s, (Quad*)dst, (const Quad*)src, q, nq);
      else
        hipLaunchKernelGGL((copy_strided_kernel<Quad, false>), dim3(grid_for(nq)), dim3(kBlock),
                           0, s, (Quad*)dst, (const Quad*)src, q, nq);
      WXX_LAUNCHED();
      return WXX_OK;
    }
  }
  const bool big = !fits32(nd, n);
  if (itemsize == 4) {
    if (big)
      hipLaunchKernelGGL((copy_strided_kernel<uint32_t, true>), dim3(grid_for(n)), dim3(kBlock),
                         0, s, (uint32_t*)dst, (const uint32_t*)src, nd, n);
    else
      hipLaunchKernelGGL((copy_strided_kernel<uint32_t, false>), dim3(grid_for(n)), dim3(kBlock),
                         0, s, (uint32_t*)dst, (const uint32_t*)src, nd, n);
  } else {
    if (big)
      hipLaunchKernelGGL((copy_strided_kernel<uint64_t, true>), dim3(grid_for(n)), dim3(kBlock),
                         0, s, (uint64_t*)dst, (const uint64_t*)src, nd, n);
    else
      hipLaunchKernelGGL((copy_strided_kernel<uint64_t, false>), dim3(grid_for(n)), dim3(kBlock),
                         0, s, (uint64_t*)dst, (const uint64_t*)src, nd, n);
  }
  WXX_LAUNCHED();
  return WXX_OK;
}

// Fill a strided view with a 32-bit pattern (functional.assign with a
// scalar, reference functional/utils.py:29-101).
WXX_API int wxx_fill_strided(void* dst, int rank, const int64_t* shape, const int64_t* s_dst,
                             uint32_t bits) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dst && shape && s_dst, "null pointer");
  WXX_REQUIRE(rank >= 0 && rank <= wxx::kMaxRank, "rank %d unsupported", rank);
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) n *= shape[d];
  if (n == 0) return WXX_OK;
  const int64_t* ss[1] = {s_dst};
  ND nd = collapse(rank, shape, ss, 1);
  if (nd.rank == 1 && nd.stride[0][0] == 1) return wxx_fill_u32(dst, n, bits);
  hipLaunchKernelGGL(fill_strided_kernel<uint32_t>, dim3(grid_for(n)), dim3(kBlock), 0,
                     wxx::stream(), (uint32_t*)dst, nd, n, bits);
  WXX_LAUNCHED();
  return WXX_OK;
}

// out (dense, shape `shape`) = zeros with `grad` (strided) placed at
// [start, start+length) along `dim`.  Replaces functional.scatter_zeros
// (reference functional/utils.py:760-827).
WXX_API int wxx_scatter_zeros(float* out, const float* grad, int rank, const int64_t* shape,
                              const int64_t* s_grad, int dim, int64_t start, int64_t length) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(out && grad && shape && s_grad, "null pointer");
  WXX_REQUIRE(rank >= 1 && rank <= wxx::kMaxRank && dim >= 0 && dim < rank, "bad rank/dim");
  ND nd;
  nd.rank = rank;
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) {
    nd.shape[d] = shape[d];
    nd.stride[0][d] = s_grad[d];
    n *= shape[d];
  }
  if (n == 0) return WXX_OK;
  hipLaunchKernelGGL(scatter_zeros_kernel, dim3(grid_for(n)), dim3(kBlock), 0, wxx::stream(), out,
                     grad, nd, n, dim, start, length);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.unfolddx (reference functional/utils.py:239-287).
WXX_API int wxx_unfolddx(const float* dy, float* dx, int64_t prefix, int64_t length,
                         int64_t suffix, int64_t windows, int64_t size, int64_t step) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && dx, "null pointer");
  WXX_REQUIRE(size >= 1 && step >= 1 && suffix >= 1, "bad unfold parameters");
  const int64_t n = prefix * length * suffix;
  if (n <= 0) return WXX_OK;
  hipLaunchKernelGGL(unfolddx_kernel, dim3(grid_for(n)), dim3(kBlock), 0, wxx::stream(), dy, dx,
                     prefix, length, suffix, windows, size, step);
  WXX_LAUNCHED();
  return WXX_OK;
}

// SwiGLU's gate silu(a) * b (reference src/wxx/nn/module.py:551-552, with
// Tensor.silu = sigmoid(x) * x at Tensor.py:724-727) in one pass.
WXX_API int wxx_swiglu_gate(const float* a, const float* b, float* h, int64_t n) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(a && b && h, "null pointer");
  if (n <= 0) return WXX_OK;
  const int vec = ((uintptr_t)a | (uintptr_t)b | (uintptr_t)h) % 16 == 0;
  hipLaunchKernelGGL(swiglu_gate_kernel, dim3(grid_for((n + 3) / 4)), dim3(kBlock), 0,
                     wxx::stream(), a, b, h, n, vec);
  WXX_LAUNCHED();
  return WXX_OK;
}

// The backward of wxx_swiglu_gate: da and db from dh, a and b (the composed
// ops' backwards, autograd/pointwise.py mul and sigmoid, in one pass).
WXX_API int wxx_swiglu_gate_backward(const float* dh, const float* a, const float* b, float* da,
                                     float* db, int64_t n) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dh && a && b && da && db, "null pointer");
  if (n <= 0) return WXX_OK;
  const int vec =
      ((uintptr_t)dh | (uintptr_t)a | (uintptr_t)b | (uintptr_t)da | (uintptr_t)db) % 16 == 0;
  hipLaunchKernelGGL(swiglu_gate_bwd_kernel, dim3(grid_for((n + 3) / 4)), dim3(kBlock), 0,
                     wxx::stream(), dh, a, b, da, db, n, vec);
  WXX_LAUNCHED();
  return WXX_OK;
}
