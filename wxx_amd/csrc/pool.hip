// Pooling (max / average / adaptive average over NCHW, 1-D as H = 1) and the
// depthwise causal 1-D convolution of Hyena, forward and backward.
//
// Reference semantics:
//  * maxpool2d (src/wxx/shaders/layers/maxpool2d.wgsl:28-70, host
//    src/wxx/functional/convolution.py:60-125): window max starting from
//    -1e38 with index 0xFFFFFFFF, strict '>' in (kh, kw) order, padded cells
//    skipped; the index is the flat input index b*C*H*W + c*H*W + ih*W + iw.
//  * maxpool2ddx (maxpool2ddx.wgsl): each input cell sums dY over the output
//    windows that can contain it (ho, wo ascending) whose index equals it.
//  * avgpool2d (avgpool2d.wgsl): mean over in-range cells
//    (count_include_pad = False), 0 for an empty window; optional max index.
//  * avgpool2ddx (avgpool2ddx.wgsl): sum of dY / valid_count over the windows
//    that can contain the cell.
//  * adaptive_avgpool2d / dx (adaptive_avgpool2d.wgsl, adaptive_avgpool2ddx.wgsl):
//    window [floor(o in / out), ceil((o+1) in / out)), and the backward over
//    o in [floor(i out / in), floor(((i+1) out - 1) / in)].
//  * maxpool1d / avgpool1d (+dx) are the 2-D kernels with H = 1.
//  * causal_conv1d (helpers/causal_conv1d.wgsl): y[b,d,n] = bias[d] +
//    sum_k w[d,k] x[b,d,n-k] over n >= k, x a strided view;
//    backward (causal_conv1d_backward.wgsl): dx[b,d,n] = sum_k w[d,k]
//    dy[b,d,n+k] (n+k < L); dw[d,k] = sum_{b, n>=k} dy[b,d,n] x[b,d,n-k];
//    db[d] = sum_{b,n} dy[b,d,n].
//
// MI355X design: the pools are one thread per output (or per input cell for
// the backward, a gather with no atomics, so results are deterministic),
// 32-bit index math.  The causal conv works on 64-channel x 64-position
// tiles staged through LDS, so a transposed input view is read coalesced and
// the output written coalesced; its weight / bias gradients take all KS + 1
// sums in one pass over dy and x per tile, then add the per-workgroup
// partials in a fixed order (the reference gives each (d, k) one thread that
// walks B*L elements serially).
#include "common.h"

namespace {

constexpr int kBlock = 256;

struct PoolArgs {
  int B, C, H, W, Ho, Wo, KH, KW, sh, sw, ph, pw;
};

template <bool AVG>
__global__ __launch_bounds__(kBlock) void pool2d_kernel(const float* __restrict__ x,
                                                         float* __restrict__ y,
                                                         uint32_t* __restrict__ idx, PoolArgs a,
                                                         int64_t total) {
  for (int64_t o = (int64_t)blockIdx.x * kBlock + threadIdx.x; o < total;
       o += (int64_t)gridDim.x * kBlock) {
    int64_t rem = o;
    const int wo = (int)(rem % a.Wo);
    rem /= a.Wo;
    const int ho = (int)(rem % a.Ho);
    rem /= a.Ho;
    const int64_t bc = rem;  // b * C + c
    const int64_t base = bc * a.H * a.W;
    const int h0 = ho * a.sh - a.ph, w0 = wo * a.sw - a.pw;
    float best = -1e38f, sum = 0.f, cnt = 0.f;
    uint32_t bi = 0xFFFFFFFFu;
    for (int kh = 0; kh < a.KH; ++kh) {
      const int ih = h0 + kh;
      if (ih < 0 || ih >= a.H) continue;
      for (int kw = 0; kw < a.KW; ++kw) {
        const int iw = w0 + kw;
        if (iw < 0 || iw >= a.W) continue;
        const int64_t in = base + (int64_t)ih * a.W + iw;
        const float v = x[in];
        if (AVG) {
          sum += v;
          cnt += 1.f;
        }
        if (v > best) {
          best = v;
          bi = (uint32_t)in;
        }
      }
    }
    y[o] = AVG ? (cnt > 0.f ? sum / cnt : 0.f) : best;
    if (idx) idx[o] = bi;
  }
}

// Output rows [lo, hi] whose windows may contain input coordinate i
// (the reference's signed-division bounds, truncating like WGSL i32 '/').
__device__ __forceinline__ void out_range(int i, int p, int k, int s, int n_out, int& lo, int& hi) {
  const int ip = i + p;
  lo = max(0, (ip - k + s) / s);
  hi = min(n_out - 1, ip / s);
}

template <bool AVG>
__global__ __launch_bounds__(kBlock) void pool2d_dx_kernel(const float* __restrict__ dy,
                                                            const uint32_t* __restrict__ idx,
                                                            float* __restrict__ dx, PoolArgs a,
                                                            int64_t total) {
  for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * kBlock) {
    int64_t rem = e;
    const int iw = (int)(rem % a.W);
    rem /= a.W;
    const int ih = (int)(rem % a.H);
    rem /= a.H;
    const int64_t bc = rem;
    int hlo, hhi, wlo, whi;
    out_range(ih, a.ph, a.KH, a.sh, a.Ho, hlo, hhi);
    out_range(iw, a.pw, a.KW, a.sw, a.Wo, wlo, whi);
    float acc = 0.f;
    if (hlo <= hhi && wlo <= whi) {
      const int64_t obase = bc * a.Ho * a.Wo;
      for (int ho = hlo; ho <= hhi; ++ho) {
        const int hs = ho * a.sh - a.ph;
        for (int wo = wlo; wo <= whi; ++wo) {
          const int64_t o = obase + (int64_t)ho * a.Wo + wo;
          if (AVG) {
            const int ws = wo * a.sw - a.pw;
            const int vh = min(a.H, hs + a.KH) - max(0, hs);
            const int vw = min(a.W, ws + a.KW) - max(0, ws);
            const float cnt = (float)(vh * vw);
            if (cnt > 0.f) acc += dy[o] / cnt;
          } else if (idx[o] == (uint32_t)e) {
            acc += dy[o];
          }
        }
      }
    }
    dx[e] = acc;
  }
}

__global__ __launch_bounds__(kBlock) void adaptive_avg_kernel(const float* __restrict__ x,
                                                               float* __restrict__ y, int H, int W,
                                                               int Ho, int Wo, int64_t total) {
  for (int64_t o = (int64_t)blockIdx.x * kBlock + threadIdx.x; o < total;
       o += (int64_t)gridDim.x * kBlock) {
    const int ow = (int)(o % Wo);
    const int64_t t0 = o / Wo;
    const int oh = (int)(t0 % Ho);
    const int64_t bc = t0 / Ho;
    const int hs = (oh * H) / Ho, he = ((oh + 1) * H + Ho - 1) / Ho;
    const int ws = (ow * W) / Wo, we = ((ow + 1) * W + Wo - 1) / Wo;
    const float* xb = x + bc * H * W;
    float acc = 0.f;
    for (int h = hs; h < he; ++h)
      for (int w = ws; w < we; ++w) acc += xb[h * W + w];
    y[o] = acc / (float)((he - hs) * (we - ws));
  }
}

__global__ __launch_bounds__(kBlock) void adaptive_avg_dx_kernel(const float* __restrict__ dy,
                                                                  float* __restrict__ dx, int H,
                                                                  int W, int Ho, int Wo,
                                                                  int64_t total) {
  for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * kBlock) {
    const int iw = (int)(e % W);
    const int64_t t0 = e / W;
    const int ih = (int)(t0 % H);
    const int64_t bc = t0 / H;
    const int ohs = (ih * Ho) / H, ohe = ((ih + 1) * Ho - 1) / H;
    const int ows = (iw * Wo) / W, owe = ((iw + 1) * Wo - 1) / W;
    const float* gb = dy + bc * Ho * Wo;
    float acc = 0.f;
    for (int oh = ohs; oh <= ohe; ++oh) {
      const int hs = (oh * H) / Ho, he = ((oh + 1) * H + Ho - 1) / Ho;
      for (int ow = ows; ow <= owe; ++ow) {
        const int ws = (ow * W) / Wo, we = ((ow + 1) * W + Wo - 1) / Wo;
        const float cnt = (float)((he - hs) * (we - ws));
        acc += gb[oh * Wo + ow] / cnt;
      }
    }
    dx[e] = acc;
  }
}

// ---- depthwise causal conv1d ------------------------------------------------

struct View3 {
  int64_t off, sb, sc, sl;
};

__global__ __launch_bounds__(kBlock) void causal_conv1d_kernel(const float* __restrict__ x,
                                                                View3 v,
                                                                const float* __restrict__ w,
                                                                const float* __restrict__ bias,
                                                                float* __restrict__ y, int D,
                                                                int L, int KS, int64_t total) {
  for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * kBlock) {
    const int n = (int)(e % L);
    const int64_t r = e / L;
    const int d = (int)(r % D);
    const int64_t b = r / D;
    float acc = bias[d];
    const float* xr = x + v.off + b * v.sb + d * v.sc;
    for (int k = 0; k < KS; ++k)
      if (n >= k) acc = fmaf(w[d * KS + k], xr[(int64_t)(n - k) * v.sl], acc);
    y[e] = acc;
  }
}

__global__ __launch_bounds__(kBlock) void causal_conv1d_dx_kernel(const float* __restrict__ dy,
                                                                   const float* __restrict__ w,
                                                                   float* __restrict__ dx, int D,
                                                                   int L, int KS, int64_t total) {
  for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * kBlock) {
    const int n = (int)(e % L);
    const int d = (int)((e / L) % D);
    float acc = 0.f;
    for (int k = 0; k < KS; ++k)
      if (n + k < L) acc = fmaf(w[d * KS + k], dy[e + k], acc);
    dx[e] = acc;
  }
}

// One workgroup per (d, k) weight (k == KS is the bias): a block-wide sum
// over (b, n), b-major then n, combined by a fixed tree (deterministic).
__global__ __launch_bounds__(kBlock) void causal_conv1d_dw_kernel(const float* __restrict__ dy,
                                                                   const float* __restrict__ x,
                                                                   View3 v, float* __restrict__ dw,
                                                                   float* __restrict__ db, int B,
                                                                   int D, int L, int KS) {
  __shared__ float red[kBlock / 64];
  const int d = blockIdx.x / (KS + 1);
  const int k = blockIdx.x % (KS + 1);
  float acc = 0.f;
  for (int b = 0; b < B; ++b) {
    const float* g = dy + ((int64_t)b * D + d) * L;
    if (k == KS) {
      for (int n = threadIdx.x; n < L; n += kBlock) acc += g[n];
    } else {
      const float* xr = x + v.off + b * v.sb + d * v.sc;
      for (int n = k + threadIdx.x; n < L; n += kBlock)
        acc = fmaf(g[n], xr[(int64_t)(n - k) * v.sl], acc);
    }
  }
  acc = wxx::block_sum(acc, red);
  if (threadIdx.x == 0) {
    if (k == KS)
      db[d] = acc;
    else
      dw[d * KS + k] = acc;
  }
}

// ---- tiled causal conv: 64 channels x 64 positions of one batch row per
// workgroup, the x window (64 + KS - 1 positions) staged in LDS with loads
// that run along whichever of the view's channel / position axes is unit
// stride (Hyena passes transposed (B, L, D) projections, channel-contiguous).
constexpr int kCT = 64;        // channels and positions per tile
constexpr int kCMaxKS = 8;     // kernel sizes handled by the tiled kernels
constexpr int kCW = kCT + kCMaxKS + 1;  // LDS row pitch, odd: a column read is conflict-free

// Stages x[b, d0 + dd, n0 - (KS - 1) + nn] (zero outside the tensor and for
// n < 0) into xs[dd][nn], dd < 64, nn < 64 + KS - 1.  The window is walked as
// a fixed 64 x kCX grid (columns >= 64 + KS - 1 skipped) so the loop has a
// constant trip count: every load is issued before the first LDS store.
constexpr int kCX = kCT + kCMaxKS;                        // window columns walked
constexpr int kStage = (kCT * kCX + kBlock - 1) / kBlock;  // loads per thread

__device__ __forceinline__ void conv_stage_x(float (*xs)[kCW], const float* __restrict__ x,
                                             const View3& v, int64_t b, int d0, int n0, int D,
                                             int L, int KS) {
  const int W = kCT + KS - 1;
  const float* xb = x + v.off + b * v.sb;
  const bool chan_fast = v.sc == 1 && v.sl != 1;  // lanes along channels when those are unit stride
  float r[kStage];
#pragma unroll
  for (int it = 0; it < kStage; ++it) {
    const int i = threadIdx.x + it * kBlock;
    const int dd = chan_fast ? i % kCT : i / kCX, nn = chan_fast ? i / kCT : i % kCX;
    const int d = d0 + dd, n = n0 - (KS - 1) + nn;
    r[it] = (i < kCT * kCX && nn < W && d < D && n >= 0 && n < L)
                ? xb[(int64_t)d * v.sc + (int64_t)n * v.sl]
                : 0.f;
  }
#pragma unroll
  for (int it = 0; it < kStage; ++it) {
    const int i = threadIdx.x + it * kBlock;
    const int dd = chan_fast ? i % kCT : i / kCX, nn = chan_fast ? i / kCT : i % kCX;
    if (i < kCT * kCX && nn < W) xs[dd][nn] = r[it];
  }
}

// y[b, d, n] for one (b, 64-channel, 64-position) tile; grid (L tiles, D tiles, B).
__global__ __launch_bounds__(kBlock) void causal_conv1d_tiled_kernel(
    const float* __restrict__ x, View3 v, const float* __restrict__ w,
    const float* __restrict__ bias, float* __restrict__ y, int D, int L, int KS) {
  __shared__ float xs[kCT][kCW];
  // the tile's weights and biases, staged with the window: a channel index
  // formed from threadIdx.x is not known to be wave-uniform, so reading them
  // from global memory in the loop below would be one vector load (and one
  // wait behind the streaming loads) per tap and channel
  __shared__ float ws[kCT][kCMaxKS + 1];  // [dd][k], k == kCMaxKS: bias
  const int n0 = blockIdx.x * kCT, d0 = blockIdx.y * kCT;
  const int64_t b = blockIdx.z;
  float wr[(kCT * (kCMaxKS + 1) + kBlock - 1) / kBlock];
#pragma unroll
  for (int it = 0; it < (kCT * (kCMaxKS + 1) + kBlock - 1) / kBlock; ++it) {
    const int i = threadIdx.x + it * kBlock;
    const int c = i / (kCMaxKS + 1), k = i % (kCMaxKS + 1);
    const bool in = i < kCT * (kCMaxKS + 1) && d0 + c < D && (k < KS || k == kCMaxKS);
    wr[it] = in ? (k == kCMaxKS ? bias[d0 + c] : w[(d0 + c) * KS + k]) : 0.f;
  }
  conv_stage_x(xs, x, v, b, d0, n0, D, L, KS);
#pragma unroll
  for (int it = 0; it < (kCT * (kCMaxKS + 1) + kBlock - 1) / kBlock; ++it) {
    const int i = threadIdx.x + it * kBlock;
    if (i < kCT * (kCMaxKS + 1)) ws[i / (kCMaxKS + 1)][i % (kCMaxKS + 1)] = wr[it];
  }
  __syncthreads();
  const int nn = threadIdx.x % kCT;
  const int n = n0 + nn;
  if (n >= L) return;
#pragma unroll 4
  for (int dd = threadIdx.x / kCT; dd < kCT; dd += kBlock / kCT) {
    const int d = d0 + dd;
    if (d >= D) break;
    float acc = ws[dd][kCMaxKS];
    for (int k = 0; k < KS; ++k)  // same order and terms as the untiled kernel
      if (n >= k) acc = fmaf(ws[dd][k], xs[dd][nn + KS - 1 - k], acc);
    y[(b * D + d) * (int64_t)L + n] = acc;
  }
}

// dx[b, d, n] = sum_k w[d, k] dy[b, d, n + k]: one row chunk of 4 * 256
// positions per workgroup, grid (chunks, rows).
__global__ __launch_bounds__(kBlock) void causal_conv1d_dx_rows_kernel(
    const float* __restrict__ dy, const float* __restrict__ w, float* __restrict__ dx, int D,
    int L, int KS, int64_t rows) {
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const int d = (int)(r % D);
    const float* g = dy + r * L;
    float* o = dx + r * L;
    for (int i = 0; i < 4; ++i) {
      const int n = (blockIdx.x * 4 + i) * kBlock + threadIdx.x;
      if (n >= L) break;
      float acc = 0.f;
      if (KS <= kCMaxKS) {
#pragma unroll
        for (int k = 0; k < kCMaxKS; ++k)  // unrolled: the tap loads issue together
          if (k < KS && n + k < L) acc = fmaf(w[d * KS + k], g[n + k], acc);
      } else {
        for (int k = 0; k < KS; ++k)
          if (n + k < L) acc = fmaf(w[d * KS + k], g[n + k], acc);
      }
      o[n] = acc;
    }
  }
}

// The same dx with four consecutive positions per thread (L a multiple of 4,
// 16-byte aligned rows, KS <= kCMaxKS): the inputs dy[n .. n + 3 + KS - 1]
// come through two or three 16-byte loads issued together, then the four
// sums run the row kernel's FMA sequence (acc from 0, taps in order, taps
// past the row skipped), so the values are the same bits.  Grid
// (ceil(L / (4 kBlock)), rows).
__global__ __launch_bounds__(kBlock) void causal_conv1d_dx_vec_kernel(
    const float* __restrict__ dy, const float* __restrict__ w, float* __restrict__ dx, int D,
    int L, int KS, int64_t rows) {
  const int L4 = L / 4;
  const int q = blockIdx.x * kBlock + threadIdx.x;  // float4 index within the row
  if (q >= L4) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const int d = (int)(r % D);
    const float4* g4 = reinterpret_cast<const float4*>(dy + r * L);
    float gv[12];
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
      if ((u < 2 || KS > 5) && q + u < L4) t = g4[q + u];
      gv[4 * u] = t.x;
      gv[4 * u + 1] = t.y;
      gv[4 * u + 2] = t.z;
      gv[4 * u + 3] = t.w;
    }
    float out[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = 4 * q + i;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < kCMaxKS; ++k)
        if (k < KS && n + k < L) acc = fmaf(w[d * KS + k], gv[i + k], acc);
      out[i] = acc;
    }
    reinterpret_cast<float4*>(dx + r * L)[q] = make_float4(out[0], out[1], out[2], out[3]);
  }
}

// Weight / bias gradient partials: workgroup (s, t) sums the (b, position)
// tiles s, s + S, s + 2S, ... of channel tile t in one pass over dy and x,
// all KS + 1 sums at once (k == KS: the bias).  Lane = channel, the four
// waves take 16 positions each; the waves' sums are added in wave order.
// part[s][d][k], reduced over s in order by causal_conv1d_dw_finalize_kernel.
__global__ __launch_bounds__(kBlock) void causal_conv1d_dw_tiled_kernel(
    const float* __restrict__ dy, const float* __restrict__ x, View3 v,
    float* __restrict__ part, int B, int D, int L, int KS) {
  __shared__ float xs[kCT][kCW];
  __shared__ float gs[kCT][kCT + 1];
  // the waves' final sums reuse the x tile's LDS (35 KB a workgroup, so the
  // four per CU the launch sizes for are resident together)
  static_assert((kBlock / kCT) * kCT * (kCMaxKS + 1) <= kCT * kCW, "sums exceed the x tile");
  auto red = reinterpret_cast<float(*)[kCT][kCMaxKS + 1]>(&xs[0][0]);
  const int d0 = blockIdx.y * kCT;
  const int ntl = (L + kCT - 1) / kCT;
  const int64_t tiles = (int64_t)B * ntl;
  const int dd = threadIdx.x % kCT, wv = threadIdx.x / kCT;
  float acc[kCMaxKS + 1];
#pragma unroll
  for (int k = 0; k <= kCMaxKS; ++k) acc[k] = 0.f;
  for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const int64_t b = tile / ntl;
    const int n0 = (int)(tile % ntl) * kCT;
    __syncthreads();  // previous tile's LDS reads are done
    float rg[kCT * kCT / kBlock];
#pragma unroll
    for (int it = 0; it < kCT * kCT / kBlock; ++it) {
      const int i = threadIdx.x + it * kBlock;
      const int nn = i % kCT, c = i / kCT;
      const int d = d0 + c, n = n0 + nn;
      rg[it] = (d < D && n < L) ? dy[(b * D + d) * (int64_t)L + n] : 0.f;
    }
    conv_stage_x(xs, x, v, b, d0, n0, D, L, KS);
#pragma unroll
    for (int it = 0; it < kCT * kCT / kBlock; ++it) {
      const int i = threadIdx.x + it * kBlock;
      gs[i / kCT][i % kCT] = rg[it];
    }
    __syncthreads();
    for (int j = 0; j < kCT / 4; ++j) {
      const int nn = wv * (kCT / 4) + j;
      const float g = gs[dd][nn];
      const int n = n0 + nn;
#pragma unroll
      for (int k = 0; k < kCMaxKS; ++k)
        if (k < KS && n >= k) acc[k] = fmaf(g, xs[dd][nn + KS - 1 - k], acc[k]);
      acc[kCMaxKS] += g;
    }
  }
  __syncthreads();  // the last tile's reads of xs are done
#pragma unroll
  for (int k = 0; k <= kCMaxKS; ++k) red[wv][dd][k] = acc[k];
  __syncthreads();
  for (int i = threadIdx.x; i < kCT * (KS + 1); i += kBlock) {
    const int c = i / (KS + 1), k = i % (KS + 1);
    const int kk = k == KS ? kCMaxKS : k;
    if (d0 + c < D) {
      float t = red[0][c][kk];
      for (int q = 1; q < kBlock / kCT; ++q) t += red[q][c][kk];
      part[((int64_t)blockIdx.x * D + d0 + c) * (KS + 1) + k] = t;
    }
  }
}

// dw[d, k] (k < KS) and db[d] (k == KS): one wave per output; lane l adds
// splits l, l + 64, ... and the lanes are combined by a fixed butterfly, so
// the order is the same on every run.
__global__ __launch_bounds__(kBlock) void causal_conv1d_dw_finalize_kernel(
    const float* __restrict__ part, float* __restrict__ dw, float* __restrict__ db, int D,
    int KS, int splits) {
  const int i = blockIdx.x * (kBlock / 64) + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (i >= D * (KS + 1)) return;
  float t = 0.f;
  for (int s = lane; s < splits; s += 64) t += part[(int64_t)s * D * (KS + 1) + i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off, 64);
  if (lane == 0) {
    const int d = i / (KS + 1), k = i % (KS + 1);
    if (k == KS)
      db[d] = t;
    else
      dw[d * KS + k] = t;
  }
}

int pool_setup(PoolArgs& a, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW,
               int64_t sh, int64_t sw, int64_t ph, int64_t pw) {
  WXX_REQUIRE(B >= 0 && C >= 0 && H >= 1 && W >= 1 && KH >= 1 && KW >= 1 && sh >= 1 && sw >= 1 &&
                  ph >= 0 && pw >= 0,
              "pool: bad shape / kernel / stride / padding");
  const int64_t Ho = (H + 2 * ph - KH) / sh + 1, Wo = (W + 2 * pw - KW) / sw + 1;
  WXX_REQUIRE(H + 2 * ph - KH >= 0 && W + 2 * pw - KW >= 0 && Ho >= 1 && Wo >= 1,
              "pooling produces an empty output");
  WXX_REQUIRE(B * C * H * W < (int64_t(1) << 32) - 1, "pool input too large for u32 indices");
  a = PoolArgs{(int)B, (int)C, (int)H, (int)W, (int)Ho, (int)Wo, (int)KH, (int)KW,
               (int)sh,  (int)sw, (int)ph, (int)pw};
  return WXX_OK;
}

}  // namespace

// Replaces functional.maxpool2d (avg = 0) and avgpool2d (avg = 1)
// (reference src/wxx/functional/convolution.py:60-192); maxpool1d / avgpool1d
// (:195-321) call it with H = 1.  idx may be null (no indices requested).
WXX_API int wxx_pool2d(const float* x, float* y, uint32_t* idx, int64_t B, int64_t C, int64_t H,
                       int64_t W, int64_t KH, int64_t KW, int64_t sh, int64_t sw, int64_t ph,
                       int64_t pw, int avg) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && y, "null pointer");
  PoolArgs a;
  int rc = pool_setup(a, B, C, H, W, KH, KW, sh, sw, ph, pw);
  if (rc) return rc;
  const int64_t total = B * C * (int64_t)a.Ho * a.Wo;
  if (total == 0) return WXX_OK;
  const dim3 g(wxx::grid_1d(total, kBlock, 65536));
  if (avg)
    hipLaunchKernelGGL(pool2d_kernel<true>, g, dim3(kBlock), 0, wxx::stream(), x, y, idx, a, total);
  else
    hipLaunchKernelGGL(pool2d_kernel<false>, g, dim3(kBlock), 0, wxx::stream(), x, y, idx, a,
                       total);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.maxpool2ddx (avg = 0, idx required) and avgpool2ddx
// (avg = 1) (reference src/wxx/functional/convolution.py:425-476, 601-653);
// maxpool1ddx / avgpool1ddx (:324-422) call it with H = 1.
WXX_API int wxx_pool2d_backward(const float* dy, const uint32_t* idx, float* dx, int64_t B,
                                int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW,
                                int64_t sh, int64_t sw, int64_t ph, int64_t pw, int avg) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && dx && (avg || idx), "null pointer");
  PoolArgs a;
  int rc = pool_setup(a, B, C, H, W, KH, KW, sh, sw, ph, pw);
  if (rc) return rc;
  const int64_t total = B * C * H * W;
  if (total == 0) return WXX_OK;
  const dim3 g(wxx::grid_1d(total, kBlock, 65536));
  if (avg)
    hipLaunchKernelGGL(pool2d_dx_kernel<true>, g, dim3(kBlock), 0, wxx::stream(), dy, idx, dx, a,
                       total);
  else
    hipLaunchKernelGGL(pool2d_dx_kernel<false>, g, dim3(kBlock), 0, wxx::stream(), dy, idx, dx,
                       a, total);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.adaptive_avgpool2d (reference
// src/wxx/functional/convolution.py:490-543).
WXX_API int wxx_adaptive_avgpool2d(const float* x, float* y, int64_t B, int64_t C, int64_t H,
                                   int64_t W, int64_t Ho, int64_t Wo) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && y, "null pointer");
  WXX_REQUIRE(B >= 0 && C >= 0 && H >= 1 && W >= 1 && Ho >= 1 && Wo >= 1,
              "adaptive_avgpool2d: bad shape");
  WXX_REQUIRE((Ho + 1) * H < (int64_t(1) << 31) && (Wo + 1) * W < (int64_t(1) << 31),
              "adaptive_avgpool2d: sizes too large");
  const int64_t total = B * C * Ho * Wo;
  if (total == 0) return WXX_OK;
  hipLaunchKernelGGL(adaptive_avg_kernel, dim3(wxx::grid_1d(total, kBlock, 65536)), dim3(kBlock),
                     0, wxx::stream(), x, y, (int)H, (int)W, (int)Ho, (int)Wo, total);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.adaptive_avgpool2ddx (reference
// src/wxx/functional/convolution.py:546-598).
WXX_API int wxx_adaptive_avgpool2ddx(const float* dy, float* dx, int64_t B, int64_t C, int64_t H,
                                     int64_t W, int64_t Ho, int64_t Wo) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && dx, "null pointer");
  WXX_REQUIRE(B >= 0 && C >= 0 && H >= 1 && W >= 1 && Ho >= 1 && Wo >= 1,
              "adaptive_avgpool2ddx: bad shape");
  WXX_REQUIRE((Ho + 1) * H < (int64_t(1) << 31) && (Wo + 1) * W < (int64_t(1) << 31),
              "adaptive_avgpool2ddx: sizes too large");
  const int64_t total = B * C * H * W;
  if (total == 0) return WXX_OK;
  hipLaunchKernelGGL(adaptive_avg_dx_kernel, dim3(wxx::grid_1d(total, kBlock, 65536)),
                     dim3(kBlock), 0, wxx::stream(), dy, dx, (int)H, (int)W, (int)Ho, (int)Wo,
                     total);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.causal_conv1d (reference
// src/wxx/functional/convolution.py:1188-1257); x is a strided (B, D, L) view
// given by its element offset and strides.
WXX_API int wxx_causal_conv1d(const float* x, int64_t x_off, int64_t sb, int64_t sc, int64_t sl,
                              const float* w, const float* bias, float* y, int64_t B, int64_t D,
                              int64_t L, int64_t KS) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && w && bias && y, "null pointer");
  WXX_REQUIRE(B >= 0 && D >= 1 && L >= 1 && KS >= 1 && D * KS < (int64_t(1) << 31) &&
                  L < (int64_t(1) << 31),
              "causal_conv1d: bad shape");
  const int64_t total = B * D * L;
  if (total == 0) return WXX_OK;
  View3 v{x_off, sb, sc, sl};
  if (KS <= kCMaxKS && B <= 65535 && D <= 65535 * kCT) {
    const dim3 grid((unsigned)((L + kCT - 1) / kCT), (unsigned)((D + kCT - 1) / kCT), (unsigned)B);
    hipLaunchKernelGGL(causal_conv1d_tiled_kernel, grid, dim3(kBlock), 0, wxx::stream(), x, v, w,
                       bias, y, (int)D, (int)L, (int)KS);
  } else {
    hipLaunchKernelGGL(causal_conv1d_kernel, dim3(wxx::grid_1d(total, kBlock, 65536)),
                       dim3(kBlock), 0, wxx::stream(), x, v, w, bias, y, (int)D, (int)L, (int)KS,
                       total);
  }
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.causal_conv1d_backward (reference
// src/wxx/functional/convolution.py:1260-1351).  dy is contiguous (B, D, L);
// dw / db may be null when the weight gradient is not needed.
WXX_API int wxx_causal_conv1d_backward(const float* dy, const float* x, int64_t x_off, int64_t sb,
                                       int64_t sc, int64_t sl, const float* w, float* dx,
                                       float* dw, float* db, int64_t B, int64_t D, int64_t L,
                                       int64_t KS) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(dy && x && w && dx, "null pointer");
  WXX_REQUIRE((dw == nullptr) == (db == nullptr), "dw and db must both be given or both null");
  WXX_REQUIRE(B >= 0 && D >= 1 && L >= 1 && KS >= 1 && D * (KS + 1) < (int64_t(1) << 31) &&
                  L < (int64_t(1) << 31) && B < (int64_t(1) << 31),
              "causal_conv1d_backward: bad shape");
  const int64_t total = B * D * L;
  hipStream_t s = wxx::stream();
  if (total > 0) {
    const int64_t rows = B * D;
    const dim3 grid((unsigned)((L + 4 * kBlock - 1) / (4 * kBlock)),
                    (unsigned)std::min<int64_t>(rows, 65535));
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (KS <= kCMaxKS && L % 4 == 0 && al16(dy) && al16(dx))
      hipLaunchKernelGGL(causal_conv1d_dx_vec_kernel, grid, dim3(kBlock), 0, s, dy, w, dx,
                         (int)D, (int)L, (int)KS, rows);
    else
      hipLaunchKernelGGL(causal_conv1d_dx_rows_kernel, grid, dim3(kBlock), 0, s, dy, w, dx,
                         (int)D, (int)L, (int)KS, rows);
  }
  if (dw) {
    View3 v{x_off, sb, sc, sl};
    const int64_t dtiles = (D + kCT - 1) / kCT;
    const int64_t tiles = B * ((L + kCT - 1) / kCT);
    if (KS <= kCMaxKS && tiles > 0 && dtiles <= 65535) {
      // about four workgroups per CU, at least 4 (b, position) tiles each
      const int64_t cus = wxx::num_cus() > 0 ? wxx::num_cus() : 256;
      int64_t splits = std::max<int64_t>(1, (4 * cus + dtiles - 1) / dtiles);
      splits = std::min<int64_t>(splits, std::max<int64_t>(1, tiles / 4));
      float* part = (float*)wxx::scratch_alloc(sizeof(float) * (size_t)(splits * D * (KS + 1)));
      if (!part) return wxx::set_error(WXX_E_OOM, "causal_conv1d dw partials");
      hipLaunchKernelGGL(causal_conv1d_dw_tiled_kernel, dim3((unsigned)splits, (unsigned)dtiles),
                         dim3(kBlock), 0, s, dy, x, v, part, (int)B, (int)D, (int)L, (int)KS);
      hipLaunchKernelGGL(causal_conv1d_dw_finalize_kernel,
                         dim3((unsigned)((D * (KS + 1) + kBlock / 64 - 1) / (kBlock / 64))),
                         dim3(kBlock), 0,
                         s, (const float*)part, dw, db, (int)D, (int)KS, (int)splits);
      wxx::scratch_free(part);
    } else {
      hipLaunchKernelGGL(causal_conv1d_dw_kernel, dim3((unsigned)(D * (KS + 1))), dim3(kBlock), 0,
                         s, dy, x, v, dw, db, (int)B, (int)D, (int)L, (int)KS);
    }
  }
  WXX_LAUNCHED();
  return WXX_OK;
}
