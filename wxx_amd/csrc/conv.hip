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
// wave-uniform and runs on the scalar unit.  Tiles are BI x BJ with 4 waves
// of v_mfma_f32_32x32x2f32, gathered straight into a 3-stage LDS ring.
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

// ---------------------------------------------------------------------------
// The implicit-GEMM tile kernel.
//
// Out[i][j] = sum_k P[i][k] Q[k][j] over one K range (a split), for a BI x BJ
// output tile with 4 waves of v_mfma_f32_32x32x2f32 (each wave a BI/2 x BJ/2
// quarter).  Both operand tiles are gathered straight into LDS with
// global_load_lds_dword: one wave instruction takes one 4-byte word per lane
// from any 64 addresses and writes them as 64 consecutive LDS words, so a
// tile row k (BI or BJ words, k-major layout) is BI/64 or BJ/64
// instructions, no VGPR holds the data on its way and no ds_write runs.
// Elements outside the tensor (padding, ragged tile edges, the end of the K
// range) are taken from a word of zeros.  A ring of three LDS stages keeps
// two chunks of loads in flight while the matrix cores work on the third: at
// chunk c a wave waits until only its loads of chunk c + 1 are outstanding
// (s_waitcnt vmcnt, loads complete in order), one barrier makes every wave's
// part of chunk c visible and frees the stage of chunk c - 1, which then
// receives chunk c + 2.
//
// The k index of a row decomposes as k = (t0 R1 + t1) R2 + t2 with
// (t0, t1, t2) = (ci, kh, kw) for the forward, (co, kh, kw) for dX and
// (b, oh, ow) for dW.  A wave loads 8 consecutive rows per chunk, so it
// carries the decomposition of its first row on the scalar unit and steps it
// (by 1 per row, by BK per chunk) with carries instead of dividing.
constexpr int BK = 32;
constexpr int kStages = 3;
constexpr int kRowsPerWave = BK / 4;

__device__ const float g_conv_zero[4] = {0.f, 0.f, 0.f, 0.f};

// (t0, t1, t2) digits of k in radices (R1, R2) and the step arithmetic.
struct KDigits {
  int t0, t1, t2;
};

__device__ __forceinline__ void kd_step1(KDigits& d, int R1, int R2) {
  if (++d.t2 == R2) {
    d.t2 = 0;
    if (++d.t1 == R1) {
      d.t1 = 0;
      ++d.t0;
    }
  }
}

// d += n where n = (n0 R1 + n1) R2 + n2 with n1 < R1, n2 < R2.
__device__ __forceinline__ void kd_add(KDigits& d, int n0, int n1, int n2, int R1, int R2) {
  d.t2 += n2;
  int c = 0;
  if (d.t2 >= R2) {
    d.t2 -= R2;
    c = 1;
  }
  d.t1 += n1 + c;
  c = 0;
  if (d.t1 >= R1) {
    d.t1 -= R1;
    c = 1;
  }
  d.t0 += n0 + c;
}

template <int MODE, int BI, int BJ>
__global__ __launch_bounds__(256) void conv_lds_kernel(ConvArgs a) {
  constexpr int WI = BI / 2, WJ = BJ / 2;
  constexpr int TM = WI / 32, TN = WJ / 32;
  constexpr int LP = BI + 2, LQ = BJ + 2;  // rows k and k + 16 land 32 banks apart
  constexpr int HP = BI / 64, HQ = BJ / 64;  // instructions per tile row
  // separate objects per stage, so the compiler can tell the loads into one
  // stage from the reads of another
  __shared__ float P0[BK * LP], P1[BK * LP], P2[BK * LP];
  __shared__ float Q0[BK * LQ], Q1[BK * LQ], Q2[BK * LQ];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wi = wave >> 1, wj = wave & 1;

  const int tile = blockIdx.x;
  const int ti = tile / a.tiles_j, tj = tile - (tile / a.tiles_j) * a.tiles_j;
  const int i0 = ti * BI, j0 = tj * BJ;
  const int z = blockIdx.y;
  const int kbeg = z * a.kps;
  const int kend = min(a.K, kbeg + a.kps);
  const int nk = (kend - kbeg + BK - 1) / BK;

  const int HW = a.H * a.W, HoWo = a.Ho * a.Wo, KK = a.KH * a.KW;
  // radices of k's digits
  const int R1 = MODE == kDw ? a.Ho : a.KH;
  const int R2 = MODE == kDw ? a.Wo : a.KW;
  const int R12 = R1 * R2;
  const float* __restrict__ zero = g_conv_zero;

  // ---- per-lane column data (constant over K) ------------------------------
  // P: lane's row i of each instruction half; Q: lane's column j.
  int p_i[HP];
  int64_t p_off[HP];
#pragma unroll
  for (int h = 0; h < HP; ++h) {
    p_i[h] = i0 + 64 * h + lane;
    const int64_t stride = MODE == kFwd ? a.K : (MODE == kDx ? KK : HoWo);
    p_off[h] = (int64_t)p_i[h] * stride;
  }
  // Q column: forward (b, oh, ow) -> base offset and input corner;
  //           dX (b, y, x) of dX;  dW (ci, kh, kw).
  int q_ok[HQ], q_b[HQ], q_y[HQ], q_x[HQ];
  int64_t q_off[HQ];
#pragma unroll
  for (int h = 0; h < HQ; ++h) {
    const int j = j0 + 64 * h + lane;
    q_ok[h] = j < a.J;
    const int jj = q_ok[h] ? j : 0;
    if (MODE == kDw) {
      const int ci = jj / KK, kk = jj - (jj / KK) * KK;
      const int kh = kk / a.KW, kw = kk - (kk / a.KW) * a.KW;
      q_b[h] = 0;
      q_y[h] = kh * a.dh;  // added to the row's oh sh - ph
      q_x[h] = kw * a.dw;
      q_off[h] = (int64_t)ci * HW;
    } else {
      const int S = MODE == kFwd ? HoWo : HW;
      const int SW = MODE == kFwd ? a.Wo : a.W;
      const int b = jj / S, r = jj - (jj / S) * S;
      const int y = r / SW, x = r - (r / SW) * SW;
      q_b[h] = b;
      if (MODE == kFwd) {
        q_y[h] = y * a.sh - a.ph;
        q_x[h] = x * a.sw - a.pw;
        q_off[h] = (int64_t)b * a.Cin * HW;
      } else {
        q_y[h] = y + a.ph;
        q_x[h] = x + a.pw;
        q_off[h] = (int64_t)b * a.Cout * HoWo;
      }
    }
  }

  // ---- the wave's first row of the first chunk, as digits ------------------
  KDigits base;
  {
    const int k = kbeg + kRowsPerWave * wave;
    base.t0 = k / R12;
    const int r = k - base.t0 * R12;
    base.t1 = r / R2;
    base.t2 = r - base.t1 * R2;
  }
  // BK as digits, for the per-chunk advance
  const int n0 = BK / R12, n1 = (BK - n0 * R12) / R2, n2 = BK - n0 * R12 - n1 * R2;

  auto issue = [&](int c, float* ps, float* qs) __attribute__((always_inline)) {
    KDigits d = base;
    const int krow0 = kbeg + c * BK + kRowsPerWave * wave;
#pragma unroll
    for (int m = 0; m < kRowsPerWave; ++m) {
      const int k = krow0 + m;
      const bool kin = k < kend;
      const int row = kRowsPerWave * wave + m;
      // P row k
#pragma unroll
      for (int h = 0; h < HP; ++h) {
        const float* src = zero;
        if (kin && p_i[h] < a.I) {
          int64_t off;
          if (MODE == kFwd) off = k;
          else if (MODE == kDx) off = (int64_t)d.t0 * a.Cin * KK + d.t1 * a.KW + d.t2;
          else off = (int64_t)d.t0 * a.Cout * HoWo + d.t1 * a.Wo + d.t2;
          src = a.P + p_off[h] + off;
        }
        WXX_LDS_DMA_DWORD(src, ps + row * LP + 64 * h);
      }
      // Q row k
#pragma unroll
      for (int h = 0; h < HQ; ++h) {
        const float* src = zero;
        if (kin && q_ok[h]) {
          if (MODE == kFwd) {
            const int iy = q_y[h] + d.t1 * a.dh, ix = q_x[h] + d.t2 * a.dw;
            if ((unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W)
              src = a.Q + q_off[h] + (int64_t)d.t0 * HW + iy * a.W + ix;
          } else if (MODE == kDx) {
            const int th = q_y[h] - d.t1 * a.dh, tw = q_x[h] - d.t2 * a.dw;
            if (th >= 0 && tw >= 0) {
              const int oh = th / a.sh, ow = tw / a.sw;
              if (oh * a.sh == th && ow * a.sw == tw && oh < a.Ho && ow < a.Wo)
                src = a.Q + q_off[h] + (int64_t)d.t0 * HoWo + oh * a.Wo + ow;
            }
          } else {
            const int iy = d.t1 * a.sh - a.ph + q_y[h], ix = d.t2 * a.sw - a.pw + q_x[h];
            if ((unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W)
              src = a.Q + (int64_t)d.t0 * a.Cin * HW + q_off[h] + iy * a.W + ix;
          }
        }
        WXX_LDS_DMA_DWORD(src, qs + row * LQ + 64 * h);
      }
      kd_step1(d, R1, R2);
    }
    kd_add(base, n0, n1, n2, R1, R2);
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

  auto compute = [&](const float* ps, const float* qs) __attribute__((always_inline)) {
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
  };

  // s_waitcnt with vmcnt = n (expcnt and lgkmcnt left alone): on gfx9 the
  // vmcnt field is bits 0-3 and 14-15
  constexpr int kPerChunk = kRowsPerWave * (HP + HQ);  // loads per wave per chunk
  static_assert(kPerChunk < 64, "vmcnt holds at most 63");
  constexpr int kWaitOne = 0x0F70 | (kPerChunk & 15) | ((kPerChunk >> 4) << 14);

  // Three stages: chunk c lives in stage c % 3.  The loop is unrolled by 3
  // so that every stage is a named LDS object.
  auto step = [&](int c, float* ps, float* qs, float* ps2, float* qs2)
      __attribute__((always_inline)) {
    if (c + 1 < nk)
      __builtin_amdgcn_s_waitcnt(kWaitOne);
    else
      __builtin_amdgcn_s_waitcnt(0x0F70);
    // a bare barrier: __syncthreads() is also a release fence, which would
    // wait for every outstanding load (vmcnt(0)) and serialise the ring.
    // Each wave's words of chunk c are in LDS by the wait above; its reads
    // of chunk c - 1 have all returned (the MFMAs consumed them).
    WXX_S_BARRIER();
    if (c + 2 < nk) issue(c + 2, ps2, qs2);
    compute(ps, qs);
  };
  if (nk > 0) issue(0, P0, Q0);
  if (nk > 1) issue(1, P1, Q1);
  for (int c = 0; c < nk; c += 3) {
    step(c, P0, Q0, P2, Q2);
    if (c + 1 < nk) step(c + 1, P1, Q1, P0, Q0);
    if (c + 2 < nk) step(c + 2, P2, Q2, P1, Q1);
  }

  // ---- epilogue: D[i][j] of a 32x32 tile is in lane j + 32 ((i/4)%2),
  //      register (i%4) + 4 (i/8) ------------------------------------------
#pragma unroll
  for (int y = 0; y < TN; ++y) {
    const int j = j0 + wj * WJ + 32 * y + l32;
    if (j >= a.J) continue;
    int64_t obase = 0, istride = 0;
    if (a.splits > 1) {
      obase = (int64_t)z * a.I * a.J + j;
      istride = a.J;
    } else if (MODE == kDw) {
      obase = j;
      istride = a.J;
    } else {
      const int S = MODE == kFwd ? HoWo : HW;
      const int C = MODE == kFwd ? a.Cout : a.Cin;
      const int b = j / S, pos = j - b * S;
      obase = (int64_t)b * C * S + pos;
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
          a.out[obase + (int64_t)i * istride] = v;
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
  // Split K when the tile grid leaves CUs idle; keep >= 4 chunks per split.
  int splits = 1;
  if (tiles < 2 * cus) {
    const int64_t want = (2 * cus + tiles - 1) / tiles;
    const int64_t maxs = std::max<int64_t>(1, a.K / (4 * BK));
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
  hipLaunchKernelGGL((conv_lds_kernel<MODE, BI, BJ>), dim3((unsigned)tiles, (unsigned)splits),
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
