// Fused multi-head attention, forward and backward, on fp32 MFMA.
//
// Reference semantics (src/wxx/nn/module.py:460-495, MultiHeadAttention):
// per batch b and head h, with q, k, v the (S, d) slices of the three
// projections,
//   probs = softmax(q k^T * (1 / sqrt(d)) + mask),  out = dropout(probs) v,
// where mask is GPT-2's causal mask (-1e9 above the diagonal, so those
// probabilities are exactly 0) or absent, and dropout keeps element
// (b * H + h, i, j) of the (B * H, S, S) probabilities by the hash of its
// flat index (shaders/layers/dropout.wgsl:14-36) and scales kept values by
// 1 / (1 - p).  The reference materialises the scores and probabilities and
// permutes the heads apart and back together (module.py:462-495).
//
// MI355X design: nothing of size S x S reaches HBM.  The projections are
// read and the output written in their (B, S, H, d) layout directly (no
// head permutes).  Each workgroup owns 128 rows (4 waves x 32) and streams
// the other side through LDS in blocks of 64; every product is a
// v_mfma_f32_32x32x2f32 chain:
//  * forward: S^T = K Q^T with the wave's 32 queries in the lanes (each lane
//    holds 16 of a 32-key column; its partner lane j ^ 32 the other 16), so
//    the online softmax needs one cross-lane max / sum per tile and the
//    probabilities already sit in the B-operand layout of O^T += V^T P^T;
//    the row's log-sum-exp is kept for the backward;
//  * backward, dQ: recomputes P^T and dP^T = V dO^T per key tile with the
//    queries in the lanes, dS^T = P^T (dP^T - D), dQ^T += K^T dS^T, where
//    D = rowsum(dO o O) is formed from registers and stored for dK / dV;
//  * backward, dK / dV: keys in the lanes, S = Q K^T and dP = dO V^T per
//    query tile, dV^T += dO^T P and dK^T += Q^T dS.
// Each workgroup's K loop is deterministic (no atomics), so results do not
// vary from run to run.  In causal mode tiles wholly above the diagonal are
// skipped and the heaviest row blocks are dispatched first.
#include "common.h"

#include <cmath>
#include <initializer_list>

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kWaveRows = 32;                // rows a wave owns
constexpr int kGroupRows = 4 * kWaveRows;    // rows a workgroup owns
constexpr int kBlock = 64;                   // rows of the other side per LDS block

struct AttnArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* o;
  const float* dout;
  float* out;
  float* dq;
  float* dk;
  float* dv;
  float* lse;           // forward: written
  const float* lse_in;  // backward: read
  float* dvec;
  int64_t S, H, ld;  // ld = H * d: row stride of every (B, S, H, d) operand
  int64_t BH;        // batch * heads
  float scale, p_drop, drop_scale;
  uint32_t seed;
  const uint32_t* seed_dev;
  int causal;
};

// Row of a 32 x 32 MFMA output held by register r of a lane in half h.
__device__ __forceinline__ int tile_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

__device__ __forceinline__ floatx16 mfma(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

// acc += A B^T over d for one 32 x 32 tile: lane (j, h) supplies row j of
// `lds` (pitch P, rows r0..r0+31) as A and the register row `reg` as B.
template <int HD, int P>
__device__ __forceinline__ floatx16 dot_tile(const float* lds, int r0, const float4 (&reg)[HD / 8],
                                             int j, int h) {
  floatx16 acc = {};
#pragma unroll
  for (int g = 0; g < HD / 8; ++g) {
    const float4 a = ld4(&lds[(r0 + j) * P + 8 * g + 4 * h]);
    acc = mfma(a.x, reg[g].x, acc);
    acc = mfma(a.y, reg[g].y, acc);
    acc = mfma(a.z, reg[g].z, acc);
    acc = mfma(a.w, reg[g].w, acc);
  }
  return acc;
}

// acc[blk] += T^T-tile x vals over the 32 rows of a tile: A comes from the
// transposed LDS copy `lds_t` (pitch P, column c0 = first row of the tile),
// B from the 16 per-register values `vals` (rows tile_row(r, h)).
template <int HD, int P>
__device__ __forceinline__ void accum_tile(floatx16 (&acc)[HD / 32], const float* lds_t, int c0,
                                           const float (&vals)[16], int j, int h) {
#pragma unroll
  for (int blk = 0; blk < HD / 32; ++blk) {
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const float4 a = ld4(&lds_t[(32 * blk + j) * P + c0 + 8 * rg + 4 * h]);
      acc[blk] = mfma(a.x, vals[4 * rg + 0], acc[blk]);
      acc[blk] = mfma(a.y, vals[4 * rg + 1], acc[blk]);
      acc[blk] = mfma(a.z, vals[4 * rg + 2], acc[blk]);
      acc[blk] = mfma(a.w, vals[4 * rg + 3], acc[blk]);
    }
  }
}

// A row of a (B, S, H, d) operand in MFMA register order: reg[g] holds
// d = 8 g + 4 h .. 8 g + 4 h + 3 of row `row` (zeros past the end).
template <int HD>
__device__ __forceinline__ void load_row(float4 (&reg)[HD / 8], const float* base, int64_t row,
                                         int64_t S, int64_t ld, int h) {
  // rows past the end read the last row (in bounds, no branch) and become 0
  const float* src = base + (row < S ? row : S - 1) * ld + 4 * h;
  const float keep = row < S ? 1.f : 0.f;
#pragma unroll
  for (int g = 0; g < HD / 8; ++g) {
    const float4 v = ld4(src + 8 * g);
    reg[g] = make_float4(v.x * keep, v.y * keep, v.z * keep, v.w * keep);
  }
}

// Store a (d x 32) accumulator transposed back to rows: lane (j, h) writes
// row `row`, d = 32 blk + tile_row(r, h), times `mul`.
template <int HD>
__device__ __forceinline__ void store_row(float* base, int64_t row, int64_t ld,
                                          const floatx16 (&acc)[HD / 32], float mul, int h) {
#pragma unroll
  for (int blk = 0; blk < HD / 32; ++blk)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg)
      st4(base + row * ld + 32 * blk + 8 * rg + 4 * h,
          make_float4(acc[blk][4 * rg] * mul, acc[blk][4 * rg + 1] * mul,
                      acc[blk][4 * rg + 2] * mul, acc[blk][4 * rg + 3] * mul));
}

// Stage rows [r0, r0 + 64) of up to two (B, S, H, d) operands in LDS: thread
// t takes row t % 64 and d quads 4 (t / 64) + 16 p.  `rows` keeps the row
// layout (pitch HD + 4), `cols` the transposed one (pitch 64 + 4); either may
// be null.  Loads go to registers first so the next block's HBM reads
// overlap the current block's products.
template <int HD>
struct Stage {
  static constexpr int kPasses = HD / 16;
  float4 a[kPasses], b[kPasses];

  // Rows past the end load the last row (in bounds, no branch); the kernels
  // mask every product that involves them.
  __device__ __forceinline__ void load(const float* pa, const float* pb, int64_t r0, int64_t S,
                                       int64_t ld, int tid) {
    const int64_t row = r0 + (tid & 63);
    const int64_t off = (row < S ? row : S - 1) * ld + 4 * (tid >> 6);
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      a[p] = ld4(pa + off + 16 * p);
      b[p] = ld4(pb + off + 16 * p);
    }
  }
};

template <int HD>
__device__ __forceinline__ void put_rows(float* lds, const float4 (&v)[HD / 16], int tid) {
  constexpr int P = HD + 4;
  const int row = tid & 63, d0 = 4 * (tid >> 6);
#pragma unroll
  for (int p = 0; p < HD / 16; ++p) st4(&lds[row * P + 16 * p + d0], v[p]);
}

template <int HD>
__device__ __forceinline__ void put_cols(float* lds, const float4 (&v)[HD / 16], int tid) {
  constexpr int P = kBlock + 4;
  const int row = tid & 63, d0 = 4 * (tid >> 6);
#pragma unroll
  for (int p = 0; p < HD / 16; ++p) {
    const int d = 16 * p + d0;
    lds[(d + 0) * P + row] = v[p].x;
    lds[(d + 1) * P + row] = v[p].y;
    lds[(d + 2) * P + row] = v[p].z;
    lds[(d + 3) * P + row] = v[p].w;
  }
}

__device__ __forceinline__ uint32_t seed_of(const AttnArgs& a) {
  return a.seed_dev ? *a.seed_dev : a.seed;
}

// Workgroup -> (row block, batch-head).  The grid is one-dimensional and
// ordered by work: in causal mode the row blocks that see the most of the
// other side (the last query blocks, the first key blocks) come first, all
// batch-heads of one block level next to each other.  Workgroups are dealt
// to the 8 XCDs round robin, so every XCD gets an equal share of every level
// (with a 2-D grid of 8 row blocks, one XCD would get every heaviest block).
struct RowBlock {
  int block;
  int64_t bh;
};
__device__ __forceinline__ RowBlock row_block(const AttnArgs& a, int nblocks, bool queries) {
  const int64_t i = blockIdx.x;
  const int level = (int)(i / a.BH);
  const int64_t bh = i - (int64_t)level * a.BH;
  const int block = a.causal && queries ? nblocks - 1 - level : level;
  return RowBlock{block, bh};
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// 2^x on the exponent unit (v_exp_f32): the softmax weights are formed as
// 2^(s * scale * log2(e) - m), one fused multiply-add and one exp per score.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Offsets i (0..31) of a 32-row tile at `t0` that a row at `row` may see:
// i in [lo, hi].  Keys (or queries) past the end are never visible; in causal
// mode a query sees keys at or before it.
struct Window {
  int lo, hi;
};
__device__ __forceinline__ Window keys_visible(int64_t t0, int64_t row, int64_t S, int causal) {
  int64_t hi = S - 1 - t0;
  if (causal && row - t0 < hi) hi = row - t0;
  return Window{0, (int)(hi < -1 ? -1 : hi > 31 ? 31 : hi)};
}
__device__ __forceinline__ Window queries_visible(int64_t t0, int64_t key, int64_t S, int causal) {
  const int64_t hi = S - 1 - t0;
  int64_t lo = causal ? key - t0 : 0;
  if (key >= S) lo = 32;
  return Window{(int)(lo < 0 ? 0 : lo > 32 ? 32 : lo), (int)(hi > 31 ? 31 : hi)};
}
__device__ __forceinline__ bool inside(Window w, int i) { return i >= w.lo && i <= w.hi; }

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <int HD, bool DROP>
__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(AttnArgs a) {
  constexpr int KP = HD + 4, TP = kBlock + 4;
  __shared__ __align__(16) float k_lds[kBlock * KP];
  __shared__ __align__(16) float vt_lds[HD * TP];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, j = lane & 31, h = lane >> 5;
  const int64_t S = a.S, ld = a.ld;
  const int nqb = (int)((S + kGroupRows - 1) / kGroupRows);
  const RowBlock rb = row_block(a, nqb, true);
  const int qb = rb.block;
  const int64_t bh = rb.bh, bb = bh / a.H;
  const int64_t base = bb * S * ld + (bh - bb * a.H) * HD;
  const int64_t q0 = (int64_t)qb * kGroupRows + w * kWaveRows, qj = q0 + j;
  const uint32_t seed = DROP ? seed_of(a) : 0u;

  float4 qreg[HD / 8];
  load_row<HD>(qreg, a.q + base, qj, S, ld, h);
  floatx16 acc[HD / 32];
#pragma unroll
  for (int blk = 0; blk < HD / 32; ++blk) acc[blk] = floatx16{};
  // m: the reference point of the weights, in units of log2 (scores times
  // scale * log2(e)); it is raised only when a score exceeds it by more than
  // 8 (a factor 256), so the accumulators are rescaled rarely.  The result,
  // acc / l with both taken against the same m, is the softmax either way.
  const float c2 = a.scale * kLog2e;
  float m = -INFINITY, l = 0.f;
  const uint32_t drop_row = DROP ? (uint32_t)((bh * S + qj) * S) : 0u;

  const int64_t q_stop = (int64_t)(qb + 1) * kGroupRows;
  const int64_t k_end = a.causal && q_stop < S ? q_stop : S;
  const int nkb = (int)((k_end + kBlock - 1) / kBlock);
  Stage<HD> st;
  st.load(a.k + base, a.v + base, 0, S, ld, tid);
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();  // every wave is done with the previous block
    put_rows<HD>(k_lds, st.a, tid);
    put_cols<HD>(vt_lds, st.b, tid);
    __syncthreads();
    if (kb + 1 < nkb) st.load(a.k + base, a.v + base, (int64_t)(kb + 1) * kBlock, S, ld, tid);
#pragma unroll
    for (int t = 0; t < kBlock / 32; ++t) {
      const int64_t kt = (int64_t)kb * kBlock + 32 * t;
      if (kt >= k_end || (a.causal && kt > q0 + kWaveRows - 1)) break;  // wave-uniform
      const floatx16 s = dot_tile<HD, KP>(k_lds, 32 * t, qreg, j, h);
      // a tile wholly visible to every row of the wave needs no mask
      const bool full = kt + 31 < S && (!a.causal || kt + 31 <= q0);
      const Window win = keys_visible(kt, qj, S, a.causal);
      float smax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        smax = fmaxf(smax, full || inside(win, tile_row(r, h)) ? s[r] : -INFINITY);
      smax = fmaxf(smax, __shfl_xor(smax, 32, 64));
      const float tmax = smax * c2;  // finite: every row sees key 0 of its first tile
      const bool grow = tmax > m + 8.f;
      if (__any(grow)) {
        const float mn = grow ? tmax : m;
        const float alpha = exp2_fast(m - mn);
        l *= alpha;
#pragma unroll
        for (int blk = 0; blk < HD / 32; ++blk) acc[blk] *= alpha;
        m = mn;
      }
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = exp2_fast(fmaf(s[r], c2, -m));
        const float pr = full || inside(win, tile_row(r, h)) ? e : 0.f;
        l += pr;
        p[r] = pr;
        if (DROP)
          p[r] = wxx::dropout_keep(drop_row + (uint32_t)(kt + tile_row(r, h)), seed, a.p_drop)
                     ? pr * a.drop_scale
                     : 0.f;
      }
      accum_tile<HD, TP>(acc, vt_lds, 32 * t, p, j, h);
    }
  }
  const float lt = l + __shfl_xor(l, 32, 64);
  if (qj < S) {
    store_row<HD>(a.out + base, qj, ld, acc, 1.f / lt, h);
    if (h == 0) a.lse[bh * S + qj] = (m + log2f(lt)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// backward: dQ (and D = rowsum(dO o O))
// ---------------------------------------------------------------------------
template <int HD, bool DROP>
__global__ __launch_bounds__(kThreads) void attn_bwd_dq_kernel(AttnArgs a) {
  constexpr int KP = HD + 4, TP = kBlock + 4;
  __shared__ __align__(16) float k_lds[kBlock * KP];
  __shared__ __align__(16) float kt_lds[HD * TP];
  __shared__ __align__(16) float v_lds[kBlock * KP];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, j = lane & 31, h = lane >> 5;
  const int64_t S = a.S, ld = a.ld;
  const int nqb = (int)((S + kGroupRows - 1) / kGroupRows);
  const RowBlock rb = row_block(a, nqb, true);
  const int qb = rb.block;
  const int64_t bh = rb.bh, bb = bh / a.H;
  const int64_t base = bb * S * ld + (bh - bb * a.H) * HD;
  const int64_t q0 = (int64_t)qb * kGroupRows + w * kWaveRows, qj = q0 + j;
  const uint32_t seed = DROP ? seed_of(a) : 0u;

  float4 qreg[HD / 8], doreg[HD / 8];
  load_row<HD>(qreg, a.q + base, qj, S, ld, h);
  load_row<HD>(doreg, a.dout + base, qj, S, ld, h);
  float dpart = 0.f;
  {
    float4 oreg[HD / 8];
    load_row<HD>(oreg, a.o + base, qj, S, ld, h);
#pragma unroll
    for (int g = 0; g < HD / 8; ++g)
      dpart += doreg[g].x * oreg[g].x + doreg[g].y * oreg[g].y + doreg[g].z * oreg[g].z +
               doreg[g].w * oreg[g].w;
  }
  const float dq_row = dpart + __shfl_xor(dpart, 32, 64);
  const bool valid = qj < S;
  if (valid && h == 0) a.dvec[bh * S + qj] = dq_row;
  // the row's weights are 2^(s * c2 - lse * log2(e))
  const float c2 = a.scale * kLog2e;
  const float lse2 = valid ? a.lse_in[bh * S + qj] * kLog2e : 0.f;
  const uint32_t drop_row = DROP ? (uint32_t)((bh * S + qj) * S) : 0u;
  floatx16 acc[HD / 32];
#pragma unroll
  for (int blk = 0; blk < HD / 32; ++blk) acc[blk] = floatx16{};

  const int64_t q_stop = (int64_t)(qb + 1) * kGroupRows;
  const int64_t k_end = a.causal && q_stop < S ? q_stop : S;
  const int nkb = (int)((k_end + kBlock - 1) / kBlock);
  Stage<HD> st;
  st.load(a.k + base, a.v + base, 0, S, ld, tid);
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();
    put_rows<HD>(k_lds, st.a, tid);
    put_cols<HD>(kt_lds, st.a, tid);
    put_rows<HD>(v_lds, st.b, tid);
    __syncthreads();
    if (kb + 1 < nkb) st.load(a.k + base, a.v + base, (int64_t)(kb + 1) * kBlock, S, ld, tid);
#pragma unroll
    for (int t = 0; t < kBlock / 32; ++t) {
      const int64_t kt = (int64_t)kb * kBlock + 32 * t;
      if (kt >= k_end || (a.causal && kt > q0 + kWaveRows - 1)) break;
      const floatx16 s = dot_tile<HD, KP>(k_lds, 32 * t, qreg, j, h);
      const floatx16 dp = dot_tile<HD, KP>(v_lds, 32 * t, doreg, j, h);
      const bool full = kt + 31 < S && (!a.causal || kt + 31 <= q0) && q0 + 31 < S;
      const Window win = keys_visible(kt, qj, S, a.causal);
      float ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = exp2_fast(fmaf(s[r], c2, -lse2));
        const float p = full || (valid && inside(win, tile_row(r, h))) ? e : 0.f;
        float dpr = dp[r];
        if (DROP)
          dpr = wxx::dropout_keep(drop_row + (uint32_t)(kt + tile_row(r, h)), seed, a.p_drop)
                    ? dpr * a.drop_scale
                    : 0.f;
        ds[r] = p * (dpr - dq_row);
      }
      accum_tile<HD, TP>(acc, kt_lds, 32 * t, ds, j, h);
    }
  }
  if (valid) store_row<HD>(a.dq + base, qj, ld, acc, a.scale, h);
}

// ---------------------------------------------------------------------------
// backward: dK, dV
// ---------------------------------------------------------------------------
// Two waves per SIMD where the registers allow it without spilling (the
// dropout variant at d = 64 would spill, d = 128 does not fit).
template <int HD, bool DROP>
__global__ __launch_bounds__(kThreads) WXX_WAVES_PER_EU(HD == 32 || (HD == 64 && !DROP) ? 2 : 1)
void attn_bwd_dkdv_kernel(AttnArgs a) {
  constexpr int KP = HD + 4, TP = kBlock + 4;
  __shared__ __align__(16) float q_lds[kBlock * KP];
  __shared__ __align__(16) float qt_lds[HD * TP];
  __shared__ __align__(16) float do_lds[kBlock * KP];
  __shared__ __align__(16) float dot_lds[HD * TP];
  __shared__ float lse_lds[kBlock], d_lds[kBlock];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, j = lane & 31, h = lane >> 5;
  const int64_t S = a.S, ld = a.ld;
  const RowBlock rb = row_block(a, (int)((S + kGroupRows - 1) / kGroupRows), false);
  const int64_t bh = rb.bh, bb = bh / a.H;
  const int64_t base = bb * S * ld + (bh - bb * a.H) * HD;
  // key blocks in order: in causal mode the first ones see the most queries
  const int64_t kg0 = (int64_t)rb.block * kGroupRows;
  const int64_t k0 = kg0 + w * kWaveRows, kj = k0 + j;
  const uint32_t seed = DROP ? seed_of(a) : 0u;

  float4 kreg[HD / 8], vreg[HD / 8];
  load_row<HD>(kreg, a.k + base, kj, S, ld, h);
  load_row<HD>(vreg, a.v + base, kj, S, ld, h);
  floatx16 dk[HD / 32], dv[HD / 32];
#pragma unroll
  for (int blk = 0; blk < HD / 32; ++blk) dk[blk] = dv[blk] = floatx16{};

  const float c2 = a.scale * kLog2e;
  const int64_t q_begin = a.causal ? kg0 : 0;  // kg0 is a multiple of kBlock
  const int nqb = (int)((S - q_begin + kBlock - 1) / kBlock);
  Stage<HD> st;
  float lse_st = 0.f, d_st = 0.f;
  auto load_block = [&](int64_t r0) __attribute__((always_inline)) {
    st.load(a.q + base, a.dout + base, r0, S, ld, tid);
    if (tid < kBlock) {
      const int64_t row = r0 + tid;
      lse_st = row < S ? a.lse_in[bh * S + row] * kLog2e : 0.f;
      d_st = row < S ? a.dvec[bh * S + row] : 0.f;
    }
  };
  if (nqb > 0) load_block(q_begin);
  for (int qbk = 0; qbk < nqb; ++qbk) {
    const int64_t r0 = q_begin + (int64_t)qbk * kBlock;
    __syncthreads();
    put_rows<HD>(q_lds, st.a, tid);
    put_cols<HD>(qt_lds, st.a, tid);
    put_rows<HD>(do_lds, st.b, tid);
    put_cols<HD>(dot_lds, st.b, tid);
    if (tid < kBlock) {
      lse_lds[tid] = lse_st;
      d_lds[tid] = d_st;
    }
    __syncthreads();
    if (qbk + 1 < nqb) load_block(r0 + kBlock);
#pragma unroll
    for (int t = 0; t < kBlock / 32; ++t) {
      const int64_t qt = r0 + 32 * t;
      if (qt >= S) break;                                             // wave-uniform
      if (a.causal && qt + kWaveRows - 1 < k0) continue;              // wholly above
      const floatx16 s = dot_tile<HD, KP>(q_lds, 32 * t, kreg, j, h);
      const floatx16 dp = dot_tile<HD, KP>(do_lds, 32 * t, vreg, j, h);
      // every (query, key) pair of the tile visible: no mask
      const bool full = qt + 31 < S && k0 + 31 < S && (!a.causal || qt >= k0 + 31);
      const Window win = queries_visible(qt, kj, S, a.causal);
      float pd[16], ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * t + tile_row(r, h);
        const float e = exp2_fast(fmaf(s[r], c2, -lse_lds[i]));
        const float p = full || inside(win, tile_row(r, h)) ? e : 0.f;
        float dpr = dp[r], pk = p;
        if (DROP) {
          const uint32_t idx = (uint32_t)((bh * S + r0 + i) * S + kj);
          const bool keep = wxx::dropout_keep(idx, seed, a.p_drop);
          pk = keep ? p * a.drop_scale : 0.f;
          dpr = keep ? dpr * a.drop_scale : 0.f;
        }
        pd[r] = pk;
        ds[r] = p * (dpr - d_lds[i]);
      }
      accum_tile<HD, TP>(dv, dot_lds, 32 * t, pd, j, h);
      accum_tile<HD, TP>(dk, qt_lds, 32 * t, ds, j, h);
    }
  }
  if (kj < S) {
    store_row<HD>(a.dk + base, kj, ld, dk, a.scale, h);
    store_row<HD>(a.dv + base, kj, ld, dv, 1.f, h);
  }
}

template <int HD, bool DROP>
int launch_fwd(const AttnArgs& a, int64_t batch_heads) {
  const dim3 grid((unsigned)((a.S + kGroupRows - 1) / kGroupRows * batch_heads));
  hipLaunchKernelGGL((attn_fwd_kernel<HD, DROP>), grid, dim3(kThreads), 0, wxx::stream(), a);
  WXX_LAUNCHED();
  return WXX_OK;
}

template <int HD, bool DROP>
int launch_bwd(const AttnArgs& a, int64_t batch_heads) {
  const dim3 grid((unsigned)((a.S + kGroupRows - 1) / kGroupRows * batch_heads));
  hipLaunchKernelGGL((attn_bwd_dq_kernel<HD, DROP>), grid, dim3(kThreads), 0, wxx::stream(), a);
  hipLaunchKernelGGL((attn_bwd_dkdv_kernel<HD, DROP>), grid, dim3(kThreads), 0, wxx::stream(), a);
  WXX_LAUNCHED();
  return WXX_OK;
}

template <bool BWD>
int dispatch(const AttnArgs& a, int64_t batch_heads, int64_t hd, bool drop) {
#define WXX_ATTN_CASE(HDV)                                                           \
  if (hd == HDV) {                                                                   \
    if (BWD) return drop ? launch_bwd<HDV, true>(a, batch_heads)                     \
                         : launch_bwd<HDV, false>(a, batch_heads);                   \
    return drop ? launch_fwd<HDV, true>(a, batch_heads) : launch_fwd<HDV, false>(a, batch_heads); \
  }
  WXX_ATTN_CASE(32)
  WXX_ATTN_CASE(64)
  WXX_ATTN_CASE(128)
#undef WXX_ATTN_CASE
  return wxx::set_error(WXX_E_UNSUPPORTED, "attention head size %lld (32, 64 or 128 supported)",
                        (long long)hd);
}

int check_common(int64_t batch, int64_t seq, int64_t heads, int64_t hd, float p_drop,
                 std::initializer_list<const void*> ptrs) {
  WXX_REQUIRE(batch >= 0 && seq >= 0 && heads > 0, "bad attention shape");
  WXX_REQUIRE((seq + 127) / 128 * batch * heads < (int64_t(1) << 31),
              "too many attention row blocks");
  WXX_REQUIRE(p_drop >= 0.f && p_drop < 1.f, "dropout probability %g outside [0, 1)", p_drop);
  for (const void* p : ptrs) {
    WXX_REQUIRE(p, "null pointer");
    WXX_REQUIRE(((uintptr_t)p & 15) == 0, "attention operands must be 16-byte aligned");
  }
  (void)hd;
  return WXX_OK;
}

}  // namespace

// softmax(q k^T * scale [+ causal mask]) with dropout, times v, for (B, S, H, d)
// operands (reference nn/module.py:460-495); lse gets each row's log-sum-exp
// of the scaled, masked scores (B * H * S floats) for the backward.
WXX_API int wxx_attention_fwd(const float* q, const float* k, const float* v, float* out,
                              float* lse, int64_t batch, int64_t seq, int64_t heads,
                              int64_t head_dim, int causal, float scale, float p_drop,
                              float drop_scale, uint32_t seed, const uint32_t* seed_dev) {
  WXX_CHECK_INIT();
  int rc = check_common(batch, seq, heads, head_dim, p_drop, {q, k, v, out, lse});
  if (rc) return rc;
  if (batch == 0 || seq == 0) return WXX_OK;
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.lse = lse;
  a.S = seq;
  a.H = heads;
  a.ld = heads * head_dim;
  a.scale = scale;
  a.p_drop = p_drop;
  a.drop_scale = drop_scale;
  a.seed = seed;
  a.seed_dev = seed_dev;
  a.causal = causal ? 1 : 0;
  a.BH = batch * heads;
  return dispatch<false>(a, batch * heads, head_dim, p_drop > 0.f);
}

// Gradients of wxx_attention_fwd with respect to q, k and v, from the forward's
// output and log-sum-exp (same shape, scale, mask and dropout arguments).
WXX_API int wxx_attention_bwd(const float* q, const float* k, const float* v, const float* out,
                              const float* dout, const float* lse, float* dq, float* dk,
                              float* dv, int64_t batch, int64_t seq, int64_t heads,
                              int64_t head_dim, int causal, float scale, float p_drop,
                              float drop_scale, uint32_t seed, const uint32_t* seed_dev) {
  WXX_CHECK_INIT();
  int rc = check_common(batch, seq, heads, head_dim, p_drop, {q, k, v, out, dout, lse, dq, dk, dv});
  if (rc) return rc;
  if (batch == 0 || seq == 0) return WXX_OK;
  float* dvec = (float*)wxx::scratch_alloc(sizeof(float) * (size_t)(batch * heads * seq));
  if (!dvec) return wxx::set_error(WXX_E_OOM, "attention backward row sums");
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = out;
  a.dout = dout;
  a.lse_in = lse;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.dvec = dvec;
  a.S = seq;
  a.H = heads;
  a.ld = heads * head_dim;
  a.scale = scale;
  a.p_drop = p_drop;
  a.drop_scale = drop_scale;
  a.seed = seed;
  a.seed_dev = seed_dev;
  a.causal = causal ? 1 : 0;
  a.BH = batch * heads;
  rc = dispatch<true>(a, batch * heads, head_dim, p_drop > 0.f);
  wxx::scratch_free(dvec);
  return rc;
}
