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
// Neither operand is materialised in HBM: both are gathered on the fly into
// LDS tiles, each in the layout (k-major or row-major, conv_addr.h) that
// reads its tensor with fewer cache lines for the launch's shape.  Tiles are
// 64 x 64 with 4 waves of v_mfma_f32_32x32x2f32; every load is a fixed
// per-slot offset plus a wave-uniform offset per chunk, four chunks of loads
// are in flight in registers and two LDS stages alternate.  When the tile
// grid is too small for 256 CUs (ResNet's deep layers, and every dW whose
// K = B Ho Wo is long) the K range is split where a cost model says it pays:
// each split writes a partial tile and a second pass adds the partials in a
// fixed order, so the result does not depend on scheduling (no float
// atomics).
#include "common.h"

#define WXX_HD __host__ __device__ __forceinline__
#include "conv_addr.h"

#include <map>
#include <mutex>
#include <tuple>

// The source of every zero operand element (padding, stride gaps, ragged
// tiles).  The kernels receive its address as an argument, so nothing in
// device code names it: external linkage and `used` keep it in the code
// object for hipGetSymbolAddress.  Nothing writes it.
__device__ __attribute__((used)) float wxx_conv_zero_word[4];

namespace {

using namespace wxx_conv;

typedef float floatx16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// The implicit-GEMM tile kernel.
//
// Out[i][j] = sum_k P[i][k] Q[k][j] over one K range (a split), for a 64 x 64
// output tile with 4 waves of v_mfma_f32_32x32x2f32 (each wave a 32 x 32
// quarter).  Each operand tile reaches LDS in the layout chosen on the host
// (KX or XK, conv_addr.h) through ordinary global loads into registers and
// ds_write: one-float global_load_lds DMA instructions, which a gather needs,
// retire too slowly to feed the matrix cores.  Elements outside the tensor
// (padding, stride gaps, ragged tile edges, the end of the K range) are
// loaded from a word of zeros.
//
// BK = 36 for 3x3 forward / dX chunks (four whole input channels of taps, so
// every load keeps fixed taps), 32 otherwise.
constexpr int kLQ = kTile + 2;  // KX row stride: rows k and k + 16 land 32 banks apart
constexpr int kDepth = 4;       // chunks of loads in flight per wave


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

template <int BK, bool XK>
struct OpWords {
  static constexpr int kWords = XK ? Xk<BK>::kWords : BK * kLQ;
  static constexpr int kPerWave = XK ? Xk<BK>::kPerWave : BK / 4;  // loads per wave per chunk
};

// SLOTS: every operand is a set of slots (a fixed offset per load plus a
// wave-uniform offset per chunk; case 1 or 2 of conv_addr.h, and always the
// forward's P).  Otherwise (case 0: a kernel whose tap count does not divide
// the chunk) the non-slot operands are KX rows whose k digits are stepped on
// the scalar unit per row.
//
// KS: groups of 4 waves per workgroup that share the tile and split its K
// range chunk by chunk (group g takes chunks g, g + KS, ...; a group past
// the end multiplies a chunk of zeros, so every group passes the same
// barriers), each with its own LDS stages; at the end the groups' sums are
// added in group order.  KS = 2 gives a launch of at most one workgroup per
// CU two waves per SIMD, so one wave's loads and barrier waits overlap the
// other's matrix work.
template <int MODE, int BK, bool PXK, bool QXK, bool SLOTS, int KS>
__global__ __launch_bounds__(256 * KS, 2) void conv_lds_kernel(ConvArgs a) {
  using OP = OpWords<BK, PXK>;
  using OQ = OpWords<BK, QXK>;
  constexpr int kRowsPerWave = BK / 4;
  constexpr bool PS = SLOTS || MODE == kFwd;  // P as slots
  constexpr bool QS = SLOTS;                  // Q as slots
  static_assert(PS || !PXK, "an XK operand is always slots");
  static_assert(QS || !QXK, "an XK operand is always slots");
  // separate objects per stage, so the compiler can tell the writes into one
  // stage from the reads of the other
  __shared__ float P0s[KS][OP::kWords], P1s[KS][OP::kWords];
  __shared__ float Q0s[KS][OQ::kWords], Q1s[KS][OQ::kWords];
  __shared__ float xch[KS > 1 ? 16 * 256 : 1];  // the other groups' sums
  __shared__ SlotX xtab[2][kTile];
  __shared__ SlotC ctab[2][BK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);  // wave of its group
  const int grp = KS > 1 ? __builtin_amdgcn_readfirstlane(tid >> 8) : 0;
  const int wi = wave >> 1, wj = wave & 1;
  float* const P0 = P0s[grp];
  float* const P1 = P1s[grp];
  float* const Q0 = Q0s[grp];
  float* const Q1 = Q1s[grp];

  const int tile = blockIdx.x;
  const int ti = tile / a.tiles_j, tj = tile - (tile / a.tiles_j) * a.tiles_j;
  const int i0 = ti * kTile, j0 = tj * kTile;
  const int z = blockIdx.y;
  const int kbeg = z * a.kps;
  const int kend = min(a.K, kbeg + a.kps);
  const int nk = (kend - kbeg + BK - 1) / BK;
  const int nks = (nk + KS - 1) / KS;  // steps: chunks per group
  const int kg = kbeg + grp * BK;      // this group's first chunk

  const int R1 = conv_r1(MODE, a), R2 = conv_r2(MODE, a);
  const int R12 = R1 * R2;
  const float* __restrict__ zero = a.zero;

  // ---- slots: row entries of the tile and column entries of a chunk, then
  //      each of the wave's loads from one of each -----------------------------
  if (grp == 0 && wave == 0) {
    xtab[0][lane] = slot_x<MODE, true>(a, i0 + lane);
    xtab[1][lane] = slot_x<MODE, false>(a, j0 + lane);
  } else if (grp == 0 && wave == 1 && lane < BK) {
    ctab[0][lane] = slot_c<MODE, true>(a, lane, BK);
    ctab[1][lane] = slot_c<MODE, false>(a, lane, BK);
  }
  __syncthreads();
  XkSlot psl[PS ? OP::kPerWave : 1], qsl[QS ? OQ::kPerWave : 1];
  auto make = [&](int op, bool xk, int n) __attribute__((always_inline)) {
    int xl, c;
    if (xk) {
      const int w = 64 * (wave + 4 * n) + lane;
      xl = w / (BK + 1);
      c = w - xl * (BK + 1);
    } else {
      xl = lane;
      c = kRowsPerWave * wave + n;
    }
    XkSlot sl;
    sl.off = sl.iy = 0;
    sl.c = kDeadSlot;
    if (xl < kTile && c < BK)
      sl = op == 0 ? slot_make<MODE, true>(a, xtab[0][xl], ctab[0][c], c)
                   : slot_make<MODE, false>(a, xtab[1][xl], ctab[1][c], c);
    return sl;
  };
  if constexpr (PS) {
#pragma unroll
    for (int n = 0; n < OP::kPerWave; ++n) psl[n] = make(0, PXK, n);
  }
  if constexpr (QS) {
#pragma unroll
    for (int n = 0; n < OQ::kPerWave; ++n) qsl[n] = make(1, QXK, n);
  }
  XkUniform xu = xk_uniform(MODE, a, kg);

  // ---- case 0: KX rows with scalar digits -----------------------------------
  const KxCol pcol = kx_col<MODE, true>(a, i0 + lane);
  const KxCol qcol = kx_col<MODE, false>(a, j0 + lane);
  const bool dx_strided = MODE == kDx && (a.sh != 1 || a.sw != 1);
  KDigits base;
  int n0 = 0, n1 = 0, n2 = 0;
  if constexpr (!PS || !QS) {
    const int k = kg + kRowsPerWave * wave;
    base.t0 = fdiv(k, a.dR12);
    const int r = k - base.t0 * R12;
    base.t1 = fdiv(r, a.dR2);
    base.t2 = r - base.t1 * R2;
    // BK as digits, for the per-chunk advance
    n0 = BK / R12;
    n1 = (BK - n0 * R12) / R2;
    n2 = BK - n0 * R12 - n1 * R2;
  }

  // Every source is the operand's base plus a wave-uniform chunk / row offset
  // plus the load's fixed offset, or the zero word.  One chunk of loads is in
  // flight in registers: the n-th load of a wave goes to its LDS word (see
  // commit).
  float pr[kDepth][OP::kPerWave], qr[kDepth][OQ::kPerWave];
  auto issue = [&](int c, float* prs, float* qrs) __attribute__((always_inline)) {
    const int kbase = kbeg + (c * KS + grp) * BK;
    const int rem = kend - kbase;
    const int lim = rem >= BK ? kDeadSlot : rem;  // only a split's last chunk is partial
    if constexpr (PS) {
      const float* pb = a.P + xk_uoff<MODE, true>(a, xu, kbase);
#pragma unroll
      for (int n = 0; n < OP::kPerWave; ++n)
        prs[n] = *(xk_valid<MODE, true>(a, psl[n], xu, lim) ? pb + psl[n].off : zero);
    }
    if constexpr (QS) {
      const float* qb = a.Q + xk_uoff<MODE, false>(a, xu, kbase);
#pragma unroll
      for (int n = 0; n < OQ::kPerWave; ++n)
        qrs[n] = *(xk_valid<MODE, false>(a, qsl[n], xu, lim) ? qb + qsl[n].off : zero);
    }
    if constexpr (!PS || !QS) {
      KDigits d = base;
#pragma unroll
      for (int m = 0; m < kRowsPerWave; ++m) {
        const int k = kbase + kRowsPerWave * wave + m;
        const bool kin = k < kend;
        if constexpr (!PS) {
          const float* rb = a.P + kx_uoff<MODE, true>(a, k, d.t0, d.t1, d.t2);
          prs[m] = *(kin && pcol.ok ? rb + pcol.lo : zero);
        }
        if constexpr (!QS) {
          const float* src = zero;
          if (dx_strided) {
            int off = 0;
            if (kin && kx_src_strided(a, qcol, d.t0, d.t1, d.t2, off)) src = a.Q + off;
          } else {
            const float* rb = a.Q + kx_uoff<MODE, false>(a, k, d.t0, d.t1, d.t2);
            if (kin && kx_valid<MODE, false>(a, qcol, d.t1, d.t2)) src = rb + qcol.lo;
          }
          qrs[m] = *src;
        }
        kd_step1(d, R1, R2);
      }
#pragma unroll
      for (int g = 0; g < KS; ++g) kd_add(base, n0, n1, n2, R1, R2);
    }
    if constexpr (PS || QS) {
#pragma unroll
      for (int g = 0; g < KS; ++g) xk_advance(MODE, a, xu, BK);
    }
  };

  floatx16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;

  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int pa = wi * 32 + l32;
  const int qa = wj * 32 + l32;

  auto compute = [&](const float* ps, const float* qs) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < BK / 2; ++s) {
      const int kk = s + half * (BK / 2);
      const float af = PXK ? ps[pa * (BK + 1) + kk] : ps[kk * kLQ + pa];
      const float bf = QXK ? qs[qa * (BK + 1) + kk] : qs[kk * kLQ + qa];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af, bf, acc, 0, 0, 0);
    }
  };

  // the registers of one issue() into a stage: the same LDS words the loads'
  // slots (XK) or rows (KX) name
  auto commit = [&](const float* prs, const float* qrs, float* ps, float* qs)
      __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < OP::kPerWave; ++n)
      ps[(PXK ? 64 * (wave + 4 * n) : (kRowsPerWave * wave + n) * kLQ) + lane] = prs[n];
#pragma unroll
    for (int n = 0; n < OQ::kPerWave; ++n)
      qs[(QXK ? 64 * (wave + 4 * n) : (kRowsPerWave * wave + n) * kLQ) + lane] = qrs[n];
  };

  // Two LDS stages (chunk c in stage c % 2) and kDepth chunks of loads in
  // flight in registers (chunk c in register set c % kDepth).  Step c:
  //   wait for this wave's LDS writes, barrier: stage c % 2 (written at step
  //   c - 1) is complete and everyone has finished reading the other stage;
  //   issue chunk c + kDepth into the register set chunk c has left;
  //   multiply chunk c; write chunk c + 1 from its registers into the other
  //   stage (the compiler's vmcnt wait covers only those loads).
  // The barrier is bare (s_barrier after an lgkmcnt wait): __syncthreads()
  // would also wait for every outstanding load and drain the pipeline.
  constexpr int kLgkmOnly = 0xC07F;  // s_waitcnt lgkmcnt(0), vmcnt and expcnt at their maxima
  auto step = [&](int c, int rs, int rs1, float* ps, float* qs, float* ps1, float* qs1)
      __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(kLgkmOnly);
    WXX_S_BARRIER();
    if (c + kDepth < nks) issue(c + kDepth, pr[rs], qr[rs]);
    compute(ps, qs);
    if (c + 1 < nks) commit(pr[rs1], qr[rs1], ps1, qs1);
  };
#pragma unroll
  for (int c = 0; c < kDepth; ++c)
    if (c < nks) issue(c, pr[c], qr[c]);
  if (nks > 0) commit(pr[0], qr[0], P0, Q0);
  static_assert(kDepth == 4, "the step loop below is unrolled for 4 register sets");
  for (int c = 0; c < nks; c += 4) {
    step(c, 0, 1, P0, Q0, P1, Q1);
    if (c + 1 < nks) step(c + 1, 1, 2, P1, Q1, P0, Q0);
    if (c + 2 < nks) step(c + 2, 2, 3, P0, Q0, P1, Q1);
    if (c + 3 < nks) step(c + 3, 3, 0, P1, Q1, P0, Q0);
  }
  if constexpr (KS > 1) {
    // group 1 hands its sums to group 0 (the same lane and register of the
    // same wave of the tile), which adds them after its own
    static_assert(KS == 2, "the groups' sums are exchanged pairwise");
    if (grp == 1) {
#pragma unroll
      for (int r = 0; r < 16; ++r) xch[r * 256 + wave * 64 + lane] = acc[r];
    }
    __syncthreads();
    if (grp == 1) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] += xch[r * 256 + wave * 64 + lane];
  }

  // ---- epilogue: D[i][j] of a 32x32 tile is in lane j + 32 ((i/4)%2),
  //      register (i%4) + 4 (i/8) ------------------------------------------
  const int j = j0 + wj * 32 + l32;
  if (j >= a.J) return;
  const int HoWo = a.Ho * a.Wo, HW = a.H * a.W;
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
  for (int r = 0; r < 16; ++r) {
    const int i = i0 + wi * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
    if (i < a.I) {
      float v = acc[r];
      if (MODE != kDw && a.splits == 1 && a.bias) v += a.bias[i];
      a.out[obase + (int64_t)i * istride] = v;
    }
  }
}

// Adds the split partials in a fixed order and writes the final layout.  A
// workgroup takes 64 consecutive elements; wave w sums splits w, w + 4, ...
// in order, and the four sums are added in wave order.
template <int MODE>
__global__ __launch_bounds__(256) void conv_splitk_reduce_kernel(ConvArgs a,
                                                                  const float* __restrict__ part,
                                                                  float* __restrict__ out) {
  __shared__ float red[4][64];
  const int64_t n = (int64_t)a.I * a.J;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t e = (int64_t)blockIdx.x * 64 + lane;
  float v = 0.f;
  if (e < n) {
#pragma unroll 4
    for (int s = w; s < a.splits; s += 4) v += part[(int64_t)s * n + e];
  }
  red[w][lane] = v;
  __syncthreads();
  if (w != 0 || e >= n) return;
  v = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
  const int i = (int)(e / a.J), j = (int)(e - (int64_t)i * a.J);
  if (MODE == kDw) {
    out[e] = v;
  } else {
    const int S = MODE == kFwd ? a.Ho * a.Wo : a.H * a.W;
    const int C = MODE == kFwd ? a.Cout : a.Cin;
    const int b = j / S, pos = j - b * S;
    if (a.bias) v += a.bias[i];
    out[((int64_t)b * C + i) * S + pos] = v;
  }
}

template <int MODE, int BK, bool PXK, bool QXK, bool SLOTS>
int launch(ConvArgs& a, float* final_out) {
  a.tiles_i = (a.I + kTile - 1) / kTile;
  a.tiles_j = (a.J + kTile - 1) / kTile;
  const int64_t tiles = (int64_t)a.tiles_i * a.tiles_j;
  const int64_t cus = wxx::num_cus() > 0 ? wxx::num_cus() : 256;
  // K splits from a cost model fitted to measured launches on MI355X: a
  // launch costs ~5 us of fixed latency (dispatch, prologue, first loads,
  // store drain), a chunk ~0.7 us for one workgroup per CU (more workgroups
  // per CU share its matrix cores), and a split adds the reduce pass (~3 us
  // plus the partials written and read back at ~3 TB/s).
  int splits = 1;
  {
    const int64_t chunks = (a.K + BK - 1) / BK;
    // a 36-deep chunk (four channels of 3x3 taps) measured ~1.2 us at one
    // workgroup per CU (ResNet18 layer1: 16 chunks in 25 us unsplit, 21 us
    // on 2 splits)
    const double per_chunk = BK == 36 ? 1.2 : 0.7;
    double best = 1e30;
    for (int sp = 1; sp <= 64 && sp <= chunks; ++sp) {
      const int64_t per = (chunks + sp - 1) / sp;
      const double load = std::max(1.0, (double)(tiles * sp) / (double)cus);
      double t = 5.0 + per_chunk * (double)per * load;
      if (sp > 1) t += 3.0 + (double)sp * a.I * a.J * 8.0 / 3.0e6;
      if (t < best - 1e-9) {
        best = t;
        splits = sp;
      }
    }
  }
  // Two groups of waves per workgroup when the launch leaves CUs without a
  // second workgroup and each workgroup has a long K range (measured on
  // MI355X: ResNet18's layer1 forward 25.1 -> 23.8 us, the stem's weight
  // gradient 28.1 -> 26.1 us; short ranges lose to the groups' exchange).
  const int64_t chunks_per_split = ((a.K + splits - 1) / splits + BK - 1) / BK;
  const int ks = tiles * splits <= cus && chunks_per_split >= 8 ? 2 : 1;
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
  const dim3 grid((unsigned)tiles, (unsigned)splits);
  if (ks == 2)
    hipLaunchKernelGGL((conv_lds_kernel<MODE, BK, PXK, QXK, SLOTS, 2>), grid, dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((conv_lds_kernel<MODE, BK, PXK, QXK, SLOTS, 1>), grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && splits > 1) {
    const int64_t n = (int64_t)a.I * a.J;
    hipLaunchKernelGGL((conv_splitk_reduce_kernel<MODE>), dim3((unsigned)((n + 63) / 64)),
                       dim3(256), 0, s, a, (const float*)part, final_out);
    e = hipGetLastError();
  }
  if (part) wxx::scratch_free(part);
  if (e != hipSuccess) return wxx::set_error(WXX_E_HIP, "conv launch: %s", hipGetErrorString(e));
  return WXX_OK;
}

// Which layout each operand takes for a shape: the one whose wave loads
// touch fewer 128-byte lines over one chunk of a middle tile.  Cached per
// shape (the count costs ~1 ms of host time).
template <int MODE, int BK>
std::pair<bool, bool> choose_layouts(const ConvArgs& a) {
  using Key = std::tuple<int, int, int, int, int, int, int, int, int, int, int, int, int, int, int,
                         int, int>;
  static std::mutex mu;
  static std::map<Key, std::pair<bool, bool>> cache;
  const Key key{MODE, BK, a.B, a.Cin, a.H, a.W, a.Cout, a.KH, a.KW, a.Ho, a.Wo, a.sh, a.sw, a.ph,
                a.pw, a.dh, a.dw};
  {
    std::lock_guard<std::mutex> g(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  ConvArgs t = a;
  t.tiles_i = (a.I + kTile - 1) / kTile;
  t.tiles_j = (a.J + kTile - 1) / kTile;
  const int i0 = (t.tiles_i / 2) * kTile, j0 = (t.tiles_j / 2) * kTile;
  const int kbase = (a.K / 2) / BK * BK;
  bool pxk = false, qxk = false;
  if (MODE == kFwd || a.kcase != 0)
    pxk = conv_lines<MODE, true, BK>(t, true, i0, kbase) <
          conv_lines<MODE, true, BK>(t, false, i0, kbase);
  if (a.kcase != 0)
    qxk = conv_lines<MODE, false, BK>(t, true, j0, kbase) <
          conv_lines<MODE, false, BK>(t, false, j0, kbase);
  std::lock_guard<std::mutex> g(mu);
  cache[key] = {pxk, qxk};
  return {pxk, qxk};
}

template <int MODE, int BK>
int dispatch_bk(ConvArgs& a, float* final_out) {
  if (a.kcase == 0) {
    // forward: W as row-major slots, im2col rows with scalar digits; dX / dW:
    // both operands as rows
    if constexpr (MODE == kFwd) return launch<MODE, BK, true, false, false>(a, final_out);
    return launch<MODE, BK, false, false, false>(a, final_out);
  }
  const std::pair<bool, bool> l = choose_layouts<MODE, BK>(a);
  if (l.first && l.second) return launch<MODE, BK, true, true, true>(a, final_out);
  if (l.first) return launch<MODE, BK, true, false, true>(a, final_out);
  if (l.second) return launch<MODE, BK, false, true, true>(a, final_out);
  return launch<MODE, BK, false, false, true>(a, final_out);
}

// Device address of wxx_conv_zero_word (looked up once per device).
const float* zero_word() {
  static const float* ptr[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  if (!ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(wxx_conv_zero_word)) != hipSuccess) return nullptr;
    ptr[dev] = (const float*)p;
  }
  return ptr[dev];
}

// Copies between a weight-shaped tensor [outer][KH][KW] and its window of
// taps [outer][KHe][KWe] starting at (kh0, kw0): into the window
// (expand == 0), or back out of it with zeros at the other taps.
__global__ __launch_bounds__(256) void conv_tap_window_kernel(const float* __restrict__ src,
                                                              float* __restrict__ dst,
                                                              int64_t outer, int KH, int KW,
                                                              int kh0, int kw0, int KHe, int KWe,
                                                              int expand) {
  // one element per thread, 32-bit index arithmetic (weights are < 2^31
  // elements, checked by setup())
  const int n = (int)(outer * (expand ? KH * KW : KHe * KWe));
  const int e = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (e >= n) return;
  if (expand) {
    const int o = e / (KH * KW);
    const int t = e - o * KH * KW, kh = t / KW - kh0, kw = t % KW - kw0;
    dst[e] = kh >= 0 && kh < KHe && kw >= 0 && kw < KWe ? src[(o * KHe + kh) * KWe + kw] : 0.f;
  } else {
    const int o = e / (KHe * KWe);
    const int t = e - o * KHe * KWe, kh = t / KWe + kh0, kw = t % KWe + kw0;
    dst[e] = src[(o * KH + kh) * KW + kw];
  }
}

// [lo, hi): the taps along one axis that read at least one input element for
// some output position (input index o s - p + k d in [0, n_in) for some o in
// [0, n_out)); the taps outside only ever read padding.
void live_taps(int K, int n_in, int n_out, int s, int p, int d, int& lo, int& hi) {
  lo = K;
  hi = 0;
  for (int k = 0; k < K; ++k) {
    const int c = k * d - p;  // input index of output 0
    const int o = c >= 0 ? 0 : (-c + s - 1) / s;
    if (o < n_out && o * s + c < n_in) {
      lo = std::min(lo, k);
      hi = k + 1;
    }
  }
}

template <int MODE>
int dispatch_all_taps(ConvArgs& a, float* final_out);

// A convolution whose kernel reaches past the input on every output (ResNet's
// 3x3 convolutions on 1 x 1 and 2 x 2 maps) runs on its live taps only: the
// others multiply nothing but padding, so dropping them leaves every sum's
// terms the same but for zeros.  The weight window is copied out for the
// forward / dX (the padding shrinks by the dropped leading taps), and the
// weight gradient of the window is expanded back with zeros at the dead taps.
template <int MODE>
int dispatch(ConvArgs& a, float* final_out) {
  int kh0, kh1, kw0, kw1;
  live_taps(a.KH, a.H, a.Ho, a.sh, a.ph, a.dh, kh0, kh1);
  live_taps(a.KW, a.W, a.Wo, a.sw, a.pw, a.dw, kw0, kw1);
  // Worth the window's copy when at most a third of the taps live (a half
  // for dX, whose strided gathers gain more): measured on MI355X, ResNet18's
  // 3x3 convolutions on 1 x 1 maps (1 of 9 taps) forward 20.1 -> 14.3 us and
  // dX 21.6 -> 16.0 us; its stride-2 2 x 2 -> 1 x 1 one (4 of 9) dX 32.5 ->
  // 25.2 us but forward 15.3 -> 17.4 us.
  const int live = (kh1 - kh0) * (kw1 - kw0);
  const bool prune = kh1 > kh0 && kw1 > kw0 && kh0 * a.dh <= a.ph && kw0 * a.dw <= a.pw &&
                     (MODE == kDx ? 2 * live <= a.KH * a.KW : 3 * live <= a.KH * a.KW);
  if (!prune) return dispatch_all_taps<MODE>(a, final_out);
  const int KHe = kh1 - kh0, KWe = kw1 - kw0;
  const int64_t outer = (int64_t)a.Cout * a.Cin;
  const int64_t nwin = outer * KHe * KWe;
  float* win = (float*)wxx::scratch_alloc(sizeof(float) * (size_t)nwin);
  if (!win) return wxx::set_error(WXX_E_OOM, "conv weight window");
  ConvArgs b = a;
  b.KH = KHe;
  b.KW = KWe;
  b.ph = a.ph - kh0 * a.dh;
  b.pw = a.pw - kw0 * a.dw;
  hipStream_t s = wxx::stream();
  int rc = WXX_OK;
  if (MODE != kDw) {
    hipLaunchKernelGGL(conv_tap_window_kernel, dim3(wxx::grid_1d(nwin, 256, int64_t(1) << 23)),
                       dim3(256), 0, s, a.P, win, outer, a.KH, a.KW, kh0, kw0, KHe, KWe, 0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) rc = wxx::set_error(WXX_E_HIP, "conv weight window: %s", hipGetErrorString(e));
    b.P = win;
    b.K = (MODE == kFwd ? a.Cin : a.Cout) * KHe * KWe;
    if (rc == WXX_OK) rc = dispatch_all_taps<MODE>(b, final_out);
  } else {
    b.J = a.Cin * KHe * KWe;
    rc = dispatch_all_taps<MODE>(b, win);
    if (rc == WXX_OK) {
      const int64_t n = outer * a.KH * a.KW;
      hipLaunchKernelGGL(conv_tap_window_kernel, dim3(wxx::grid_1d(n, 256, int64_t(1) << 23)),
                         dim3(256), 0, s, win, final_out, outer, a.KH, a.KW, kh0, kw0, KHe, KWe,
                         1);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) rc = wxx::set_error(WXX_E_HIP, "conv weight window: %s", hipGetErrorString(e));
    }
  }
  wxx::scratch_free(win);
  return rc;
}

template <int MODE>
int dispatch_all_taps(ConvArgs& a, float* final_out) {
  const int R2 = conv_r2(MODE, a), R12 = conv_r1(MODE, a) * R2;
  // chunks of whole input channels of 3x3 taps for the forward and dX
  const int bk = (MODE != kDw && R12 == 9) ? 36 : 32;
  a.kcase = bk % R12 == 0 ? 1 : (MODE == kDw && R12 % bk == 0 && bk % R2 == 0) ? 2 : 0;
  a.zero = zero_word();
  if (!a.zero) return wxx::set_error(WXX_E_HIP, "conv: zero word address");
  conv_prepare(MODE, a);
  if constexpr (MODE != kDw) {
    if (bk == 36) return dispatch_bk<MODE, 36>(a, final_out);
  }
  return dispatch_bk<MODE, 32>(a, final_out);
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
