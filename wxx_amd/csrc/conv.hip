// 2-D convolution (NCHW, f32) forward / input-gradient / weight-gradient as
// implicit GEMMs on the fp32 matrix cores, plus deterministic split-K.
//
// Reference semantics (src/wxx/shaders/layers/conv2d.wgsl:33-111,
// conv2ddx.wgsl:33-118, conv2ddw.wgsl + conv2ddw_reduce.wgsl; hosts
// src/wxx/functional/convolution.py:658-908):
//   Ho = (H + 2 ph - dh (KH - 1) - 1) / sh + 1  (same for Wo)
//   Y[b,co,oh,ow]  = bias[co] + sum_{ci,kh,kw} X[b,ci,oh sh - ph + kh dh, ow sw - pw + kw dw]
//                                              * W[co,ci,kh,kw]     (zero outside X)
//   dX[b,ci,ih,iw] = sum_{co,kh,kw} dY[b,co,oh,ow] W[co,ci,kh,kw]
//                    over oh = (ih + ph - kh dh) / sh when that divides exactly and is in range
//   dW[co,ci,kh,kw]= sum_{b,oh,ow} dY[b,co,oh,ow] X[b,ci,oh sh - ph + kh dh, ...]
//
// MI355X design.  Each mode is one GEMM  Out[i][j] = sum_k P[i][k] Q[k][j]
// where j is the output's contiguous axis, so the MFMA's output lanes (which
// run along j) store coalesced NCHW rows:
//   forward: i = co, j = (b, oh, ow), k = (ci, kh, kw); P = W, Q = im2col(X)
//   dX:      i = ci, j = (b, ih, iw), k = (co, kh, kw); P = W (ci-strided), Q = gather(dY)
//   dW:      i = co, j = (ci, kh, kw), k = (b, oh, ow); P = dY, Q = im2col(X)^T
// Q is gathered on the fly into k-major LDS tiles (never materialised in
// HBM).  Each lane owns one column j for the whole K loop, so its (b, oh, ow)
// or (ci, kh, kw) decomposition is computed once; the k decomposition is
// wave-uniform and runs on the scalar unit.  Tiles are BI x BJ (64 or 128)
// with 4 waves of v_mfma_f32_32x32x2f32 and register-staged double buffering.
// When the tile grid is too small to fill 256 CUs (ResNet's deep layers, and
// every dW whose K = B Ho Wo is long) the K range is split: each split writes
// a partial tile and a second pass adds the partials in split order, so the
// result does not depend on scheduling (no float atomics).
#include "common.h"

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

enum { kFwd = 0, kDx = 1, kDw = 2 };

struct ConvArgs {
  const float* P;
  const float* Q;
  const float* bias;
  float* out;  // final tensor (splits == 1) or partials [splits][I][J]
  int B, Cin, H, W, Cout, KH, KW, Ho, Wo, sh, sw, ph, pw, dh, dw;
  int I, J, K;
  int kps;  // K elements per split (multiple of the K chunk)
  int splits;
  int tiles_i, tiles_j;
};

constexpr int BK = 16;
constexpr int kPad = 4;

template <int MODE, int BI, int BJ>
__global__ __launch_bounds__(256) void conv_mfma_kernel(ConvArgs a) {
  constexpr int WI = BI / 2, WJ = BJ / 2;  // 2 x 2 waves
  constexpr int TM = WI / 32, TN = WJ / 32;
  constexpr int LP = BI + kPad, LQ = BJ + kPad;
  constexpr int PPT = BI * BK / 256;  // P elements per thread per chunk
  constexpr int QPT = BJ * BK / 256;  // Q elements per thread per chunk
  constexpr int P_TPR = BK / PPT;     // threads per P row
  static_assert(PPT >= 1 && QPT >= 1 && BK % PPT == 0, "tile shape");

  __shared__ __attribute__((aligned(16))) float Ps[2][BK * LP];
  __shared__ __attribute__((aligned(16))) float Qs[2][BK * LQ];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wi = wave >> 1, wj = wave & 1;

  // tile ids: consecutive blocks walk j first (neighbouring j tiles share P)
  const int tile = blockIdx.x;
  const int ti = tile / a.tiles_j, tj = tile % a.tiles_j;
  const int i0 = ti * BI, j0 = tj * BJ;
  const int z = blockIdx.y;
  const int kbeg = z * a.kps;
  const int kend = min(a.K, kbeg + a.kps);

  const int KK = a.KH * a.KW;
  const int HW = a.H * a.W, HoWo = a.Ho * a.Wo;

  // ---- per-thread P row and Q column ------------------------------------
  const int p_i = i0 + tid / P_TPR;
  const int p_k = (tid % P_TPR) * PPT;
  const bool p_ok = p_i < a.I;
  const int q_j = j0 + tid % BJ;
  const int q_k = (tid / BJ) * QPT;  // wave-uniform when BJ >= 64
  const bool q_ok = q_j < a.J;

  // Q column decomposition (constant over K)
  int qb = 0, qy = 0, qx = 0;     // forward / dX: (b, y, x) of column j
  int qci = 0, qkh = 0, qkw = 0;  // dW: (ci, kh, kw) of column j
  if (MODE == kDw) {
    qci = q_j / KK;
    const int r = q_j - qci * KK;
    qkh = r / a.KW;
    qkw = r - qkh * a.KW;
  } else {
    const int S = MODE == kFwd ? HoWo : HW;
    const int SW = MODE == kFwd ? a.Wo : a.W;
    qb = q_j / S;
    const int r = q_j - qb * S;
    qy = r / SW;
    qx = r - qy * SW;
  }

  auto loadP = [&](int k) -> float {
    if (!p_ok || k >= kend) return 0.f;
    if (MODE == kFwd) return a.P[(int64_t)p_i * a.K + k];
    if (MODE == kDx) {
      const int co = k / KK, kk = k - co * KK;
      return a.P[((int64_t)co * a.Cin + p_i) * KK + kk];
    }
    const int b = k / HoWo, pos = k - b * HoWo;
    return a.P[((int64_t)b * a.Cout + p_i) * HoWo + pos];
  };

  auto loadQ = [&](int k) -> float {
    if (!q_ok || k >= kend) return 0.f;
    if (MODE == kFwd) {
      const int ci = k / KK, kk = k - ci * KK;
      const int kh = kk / a.KW, kw = kk - kh * a.KW;
      const int ih = qy * a.sh - a.ph + kh * a.dh;
      const int iw = qx * a.sw - a.pw + kw * a.dw;
      if (ih < 0 || ih >= a.H || iw < 0 || iw >= a.W) return 0.f;
      return a.Q[(((int64_t)qb * a.Cin + ci) * a.H + ih) * a.W + iw];
    }
    if (MODE == kDx) {
      const int co = k / KK, kk = k - co * KK;
      const int kh = kk / a.KW, kw = kk - kh * a.KW;
      const int th = qy + a.ph - kh * a.dh;
      const int tw = qx + a.pw - kw * a.dw;
      if (th < 0 || tw < 0) return 0.f;
      const int oh = th / a.sh, ow = tw / a.sw;
      if (oh * a.sh != th || ow * a.sw != tw || oh >= a.Ho || ow >= a.Wo) return 0.f;
      return a.Q[(((int64_t)qb * a.Cout + co) * a.Ho + oh) * a.Wo + ow];
    }
    const int b = k / HoWo, pos = k - b * HoWo;
    const int oh = pos / a.Wo, ow = pos - oh * a.Wo;
    const int ih = oh * a.sh - a.ph + qkh * a.dh;
    const int iw = ow * a.sw - a.pw + qkw * a.dw;
    if (ih < 0 || ih >= a.H || iw < 0 || iw >= a.W) return 0.f;
    return a.Q[(((int64_t)b * a.Cin + qci) * a.H + ih) * a.W + iw];
  };

  float rp[PPT], rq[QPT];
  auto load_chunk = [&](int k0) {
#pragma unroll
    for (int e = 0; e < PPT; ++e) rp[e] = loadP(k0 + p_k + e);
#pragma unroll
    for (int e = 0; e < QPT; ++e) rq[e] = loadQ(k0 + q_k + e);
  };
  auto store_chunk = [&](int buf) {
    const int pi = tid / P_TPR, qj = tid % BJ;
#pragma unroll
    for (int e = 0; e < PPT; ++e) Ps[buf][(p_k + e) * LP + pi] = rp[e];
#pragma unroll
    for (int e = 0; e < QPT; ++e) Qs[buf][(q_k + e) * LQ + qj] = rq[e];
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int x = 0; x < TM; ++x)
#pragma unroll
    for (int y = 0; y < TN; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[x][y][r] = 0.f;

  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int pa = wi * WI + l32;
  const int qa = wj * WJ + l32;

  const int nk = (kend - kbeg + BK - 1) / BK;
  load_chunk(kbeg);
  store_chunk(0);
  __syncthreads();
  for (int c = 0; c < nk; ++c) {
    const int cur = c & 1;
    if (c + 1 < nk) load_chunk(kbeg + (c + 1) * BK);
    const float* ps = Ps[cur];
    const float* qs = Qs[cur];
#pragma unroll
    for (int s = 0; s < BK / 2; ++s) {
      const int kk = s + half * (BK / 2);
      float af[TM], bf[TN];
#pragma unroll
      for (int x = 0; x < TM; ++x) af[x] = ps[kk * LP + pa + 32 * x];
#pragma unroll
      for (int y = 0; y < TN; ++y) bf[y] = qs[kk * LQ + qa + 32 * y];
#pragma unroll
      for (int x = 0; x < TM; ++x)
#pragma unroll
        for (int y = 0; y < TN; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[x], bf[y], acc[x][y], 0, 0, 0);
    }
    if (c + 1 < nk) store_chunk(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: D[i][j] of a 32x32 tile is in lane j + 32 ((i/4)%2),
  //      register (i%4) + 4 (i/8) ------------------------------------------
#pragma unroll
  for (int y = 0; y < TN; ++y) {
    const int j = j0 + wj * WJ + 32 * y + l32;
    if (j >= a.J) continue;
    int64_t base = 0, istride = 0;
    if (a.splits > 1) {
      base = (int64_t)z * a.I * a.J + j;
      istride = a.J;
    } else if (MODE == kDw) {
      base = j;
      istride = a.J;
    } else {
      const int S = MODE == kFwd ? HoWo : HW;
      const int C = MODE == kFwd ? a.Cout : a.Cin;
      const int b = j / S, pos = j - b * S;
      base = (int64_t)b * C * S + pos;
      istride = S;
    }
#pragma unroll
    for (int x = 0; x < TM; ++x) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + wi * WI + 32 * x + 8 * (r >> 2) + 4 * half + (r & 3);
        if (i < a.I) {
          float v = acc[x][y][r];
          if (MODE != kDw && a.splits == 1 && a.bias) v += a.bias[i];
          a.out[base + (int64_t)i * istride] = v;
        }
      }
    }
  }
}

// Adds the split partials in split order and writes the final layout.
template <int MODE>
__global__ __launch_bounds__(256) void conv_splitk_reduce_kernel(ConvArgs a,
                                                                  const float* __restrict__ part,
                                                                  float* __restrict__ out) {
  const int64_t n = (int64_t)a.I * a.J;
  const int HoWo = a.Ho * a.Wo, HW = a.H * a.W;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * 256) {
    const int i = (int)(e / a.J), j = (int)(e - (int64_t)i * a.J);
    float v = 0.f;
    for (int s = 0; s < a.splits; ++s) v += part[(int64_t)s * n + e];
    if (MODE == kDw) {
      out[e] = v;
    } else {
      const int S = MODE == kFwd ? HoWo : HW;
      const int C = MODE == kFwd ? a.Cout : a.Cin;
      const int b = j / S, pos = j - b * S;
      if (a.bias) v += a.bias[i];
      out[((int64_t)b * C + i) * S + pos] = v;
    }
  }
}

template <int MODE, int BI, int BJ>
int launch(ConvArgs& a, float* final_out) {
  a.tiles_i = (a.I + BI - 1) / BI;
  a.tiles_j = (a.J + BJ - 1) / BJ;
  const int64_t tiles = (int64_t)a.tiles_i * a.tiles_j;
  const int64_t cus = wxx::num_cus() > 0 ? wxx::num_cus() : 256;
  // Split K when the tile grid leaves CUs idle; keep >= 8 chunks per split.
  int splits = 1;
  if (tiles < 2 * cus) {
    const int64_t want = (2 * cus + tiles - 1) / tiles;
    const int64_t maxs = std::max<int64_t>(1, a.K / (8 * BK));
    splits = (int)std::min<int64_t>(std::min<int64_t>(want, maxs), 64);
  }
  int kps = (a.K + splits - 1) / splits;
  kps = (kps + BK - 1) / BK * BK;
  splits = (a.K + kps - 1) / kps;
  if (splits < 1) splits = 1;
  a.kps = splits > 1 ? kps : std::max(a.K, 1);
  a.splits = splits;
  hipStream_t s = wxx::stream();
  float* part = nullptr;
  if (splits > 1) {
    part = (float*)wxx::scratch_alloc(sizeof(float) * (size_t)splits * a.I * a.J);
    if (!part) return wxx::set_error(WXX_E_OOM, "conv split-K partials");
    a.out = part;
  } else {
    a.out = final_out;
  }
  hipLaunchKernelGGL((conv_mfma_kernel<MODE, BI, BJ>), dim3((unsigned)tiles, (unsigned)splits),
                     dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && splits > 1) {
    const int64_t n = (int64_t)a.I * a.J;
    hipLaunchKernelGGL((conv_splitk_reduce_kernel<MODE>), dim3(wxx::grid_1d(n, 256, 8192)),
                       dim3(256), 0, s, a, (const float*)part, final_out);
    e = hipGetLastError();
  }
  if (part) wxx::scratch_free(part);
  if (e != hipSuccess) return wxx::set_error(WXX_E_HIP, "conv launch: %s", hipGetErrorString(e));
  return WXX_OK;
}

template <int MODE>
int dispatch(ConvArgs& a, float* final_out) {
  const bool bi = a.I >= 128, bj = a.J >= 128;
  if (bi && bj) return launch<MODE, 128, 128>(a, final_out);
  if (bj) return launch<MODE, 64, 128>(a, final_out);
  if (bi) return launch<MODE, 128, 64>(a, final_out);
  return launch<MODE, 64, 64>(a, final_out);
}

// Shapes of a convolution with input (B, Cin, H, W), weight (Cout, Cin, KH, KW)
// and output (B, Cout, Ho, Wo).  Ho / Wo < 0 means the conv2d formula; a
// transposed convolution passes its own input size there (with its output
// padding that size need not follow from the formula).
int setup(ConvArgs& a, int64_t B, int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t KH,
          int64_t KW, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
          int64_t Ho = -1, int64_t Wo = -1) {
  WXX_REQUIRE(B >= 0 && Cin >= 1 && H >= 1 && W >= 1 && Cout >= 1 && KH >= 1 && KW >= 1,
              "conv2d: bad shape");
  WXX_REQUIRE(sh >= 1 && sw >= 1 && dh >= 1 && dw >= 1 && ph >= 0 && pw >= 0,
              "conv2d: stride/dilation must be >= 1 and padding >= 0");
  if (Ho < 0) {
    WXX_REQUIRE(H + 2 * ph - dh * (KH - 1) - 1 >= 0 && W + 2 * pw - dw * (KW - 1) - 1 >= 0,
                "conv2d: kernel larger than the padded input");
    Ho = (H + 2 * ph - dh * (KH - 1) - 1) / sh + 1;
    Wo = (W + 2 * pw - dw * (KW - 1) - 1) / sw + 1;
  }
  WXX_REQUIRE(Ho >= 1 && Wo >= 1, "conv2d: empty output");
  const int64_t lim = (int64_t(1) << 31) - 1;
  WXX_REQUIRE(B * Cin * H * W < lim && B * Cout * Ho * Wo < lim && Cout * Cin * KH * KW < lim,
              "conv2d: tensor too large for 32-bit indexing");
  a.B = (int)B;
  a.Cin = (int)Cin;
  a.H = (int)H;
  a.W = (int)W;
  a.Cout = (int)Cout;
  a.KH = (int)KH;
  a.KW = (int)KW;
  a.Ho = (int)Ho;
  a.Wo = (int)Wo;
  a.sh = (int)sh;
  a.sw = (int)sw;
  a.ph = (int)ph;
  a.pw = (int)pw;
  a.dh = (int)dh;
  a.dw = (int)dw;
  a.bias = nullptr;
  return WXX_OK;
}

}  // namespace

// Replaces functional.conv2d (reference src/wxx/functional/convolution.py:658-729).
WXX_API int wxx_conv2d(const float* X, const float* Wt, const float* bias, float* Y, int64_t B,
                       int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t KH, int64_t KW,
                       int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(X && Wt && Y, "null pointer");
  ConvArgs a;
  int rc = setup(a, B, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, dh, dw);
  if (rc) return rc;
  if (B == 0) return WXX_OK;
  a.P = Wt;
  a.Q = X;
  a.bias = bias;
  a.I = a.Cout;
  a.J = a.B * a.Ho * a.Wo;
  a.K = a.Cin * a.KH * a.KW;
  return dispatch<kFwd>(a, Y);
}

// Replaces functional.conv2ddx (reference src/wxx/functional/convolution.py:732-793).
WXX_API int wxx_conv2ddx(const float* dY, const float* Wt, float* dX, int64_t B, int64_t Cin,
                         int64_t H, int64_t W, int64_t Cout, int64_t KH, int64_t KW, int64_t sh,
                         int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dY && Wt && dX, "null pointer");
  ConvArgs a;
  int rc = setup(a, B, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, dh, dw);
  if (rc) return rc;
  if (B == 0) return WXX_OK;
  a.P = Wt;
  a.Q = dY;
  a.I = a.Cin;
  a.J = a.B * a.H * a.W;
  a.K = a.Cout * a.KH * a.KW;
  return dispatch<kDx>(a, dX);
}

// Replaces functional.conv2ddw + conv2ddw_reduce (reference
// src/wxx/functional/convolution.py:796-908).
WXX_API int wxx_conv2ddw(const float* dY, const float* X, float* dW, int64_t B, int64_t Cin,
                         int64_t H, int64_t W, int64_t Cout, int64_t KH, int64_t KW, int64_t sh,
                         int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dY && X && dW, "null pointer");
  ConvArgs a;
  int rc = setup(a, B, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, dh, dw);
  if (rc) return rc;
  if (B == 0) return wxx_fill_u32(dW, Cout * Cin * KH * KW, 0u);
  a.P = dY;
  a.Q = X;
  a.I = a.Cout;
  a.J = a.Cin * a.KH * a.KW;
  a.K = a.B * a.Ho * a.Wo;
  return dispatch<kDw>(a, dW);
}

// Transposed convolution: X (B, Cin, H, W), W (Cin, Cout, KH, KW), output
// (B, Cout, Hout, Wout).  It is the input gradient of the convolution that maps
// (B, Cout, Hout, Wout) to (B, Cin, H, W) with the same weight, so it runs on
// the dX gather with that convolution's shapes (and a bias epilogue).

// Replaces functional.conv2dtranspose (reference
// src/wxx/functional/convolution.py:911-1000); bias may be null.
WXX_API int wxx_conv2dtranspose(const float* X, const float* Wt, const float* bias, float* Y,
                                int64_t B, int64_t Cin, int64_t H, int64_t W, int64_t Cout,
                                int64_t KH, int64_t KW, int64_t sh, int64_t sw, int64_t ph,
                                int64_t pw, int64_t dh, int64_t dw, int64_t Hout, int64_t Wout) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(X && Wt && Y, "null pointer");
  ConvArgs a;
  int rc = setup(a, B, Cout, Hout, Wout, Cin, KH, KW, sh, sw, ph, pw, dh, dw, H, W);
  if (rc) return rc;
  if (B == 0) return WXX_OK;
  a.P = Wt;
  a.Q = X;
  a.bias = bias;
  a.I = a.Cin;
  a.J = a.B * a.H * a.W;
  a.K = a.Cout * a.KH * a.KW;
  return dispatch<kDx>(a, Y);
}

// Replaces functional.conv2dtranspose_dx (reference
// src/wxx/functional/convolution.py:1003-1064): dX (B, Cin, H, W) from
// dY (B, Cout, Hout, Wout), a plain convolution of dY with the weight.
WXX_API int wxx_conv2dtranspose_dx(const float* dY, const float* Wt, float* dX, int64_t B,
                                   int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t KH,
                                   int64_t KW, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                                   int64_t dh, int64_t dw, int64_t Hout, int64_t Wout) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dY && Wt && dX, "null pointer");
  ConvArgs a;
  int rc = setup(a, B, Cout, Hout, Wout, Cin, KH, KW, sh, sw, ph, pw, dh, dw, H, W);
  if (rc) return rc;
  if (B == 0) return WXX_OK;
  a.P = Wt;
  a.Q = dY;
  a.I = a.Cout;
  a.J = a.B * a.Ho * a.Wo;
  a.K = a.Cin * a.KH * a.KW;
  return dispatch<kFwd>(a, dX);
}

// Replaces functional.conv2dtranspose_dw (reference
// src/wxx/functional/convolution.py:1067-1185): dW (Cin, Cout, KH, KW) from
// dY (B, Cout, Hout, Wout) and X (B, Cin, H, W).
WXX_API int wxx_conv2dtranspose_dw(const float* dY, const float* X, float* dW, int64_t B,
                                   int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t KH,
                                   int64_t KW, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                                   int64_t dh, int64_t dw, int64_t Hout, int64_t Wout) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dY && X && dW, "null pointer");
  ConvArgs a;
  int rc = setup(a, B, Cout, Hout, Wout, Cin, KH, KW, sh, sw, ph, pw, dh, dw, H, W);
  if (rc) return rc;
  if (B == 0) return wxx_fill_u32(dW, Cout * Cin * KH * KW, 0u);
  a.P = X;
  a.Q = dY;
  a.I = a.Cout;
  a.J = a.Cin * a.KH * a.KW;
  a.K = a.B * a.Ho * a.Wo;
  return dispatch<kDw>(a, dW);
}
