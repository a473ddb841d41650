// Batched fp32 GEMM with fused bias on the CDNA4 fp32 matrix cores:
//     C[b] = op(A[b]) . op(B[b]) + bias
//
// Reference semantics (src/wxx/shaders/matmul.wgsl:1-151, host
// src/wxx/functional/utils.py:378-499):
//  * A is (M, K) row-major, or (K, M) when transpose_A; B is (K, N), or
//    (N, K) when transpose_B; an unbatched operand has batch stride 0;
//  * bias_mode 0 = none, 1 = (N,), 2 = (M, N) shared by every batch,
//    3 = (batch, M, N);
//  * every output element is sum_k A[i,k] B[k,j] accumulated in fp32.
//
// MI355X design (not a translation of the reference's 16x16-thread,
// 4x4-register scalar tile):
//  * 256-thread workgroups (4 wavefronts) own a BM x BN tile; each wave owns
//    a WM x WN sub-tile computed with v_mfma_f32_32x32x2f32 (64 FLOP/clk per
//    SIMD, the fp32 matrix peak of 157.3 TFLOP/s at 256 CUs);
//  * A and B tiles are staged k-major in LDS ([BK][BM] and [BK][BN]); the
//    global loads of chunk k+1 are in flight in registers while the MFMAs of
//    chunk k run, and the LDS tile is double buffered (one barrier per
//    chunk) or, for the 32-deep chunk variant, single (two barriers, half
//    the LDS);
//  * within an MFMA the two K lanes (lane / 32) take k and k + BK/2 of the
//    chunk, so a lane's A/B fragment is one conflict-free ds_read_b32;
//  * tile ids are remapped so that consecutive tiles land on the same XCD
//    (each of the 8 XCDs has its own L2) and walked in GROUP_M row groups;
//  * interior tiles run a loop body with no bounds checks, float4 global
//    loads when the operands are 16-byte aligned and scalar loads otherwise
//    (chosen once per workgroup, so the loop carries no branches); edge
//    tiles and a ragged last K chunk use guarded scalar loads;
//  * long K over few output tiles is split across workgroups (grid z) into
//    partials that a second pass adds in split order, so results do not
//    depend on timing.
#include "common.h"

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const float* A;
  const float* B;
  const float* bias;
  float* C;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t sA, sB, sC, sBias;
  int64_t bias_rows;  // mode 2: rows of the bias matrix (row index taken modulo)
  int bias_mode;
  int tiles_m, tiles_n;
  int64_t nbatch;  // batches in the launch (grid x = nbatch * tiles)
  int vec_ok;  // all leading dims, batch strides and base pointers allow float4
  int64_t kps;  // K elements per split (TileId::split); the whole K when not split
  int64_t sZ;   // element stride between split partial outputs (0 when not split)
  // Causal attention structure (square in the triangular dimension, entries
  // above the diagonal exactly zero or not needed): 0 none; 1 output tiles
  // wholly above the diagonal are written as zeros without computing; 2 op(A)
  // is lower triangular, so row tile m0 stops K at m0 + BM; 3 op(A) is upper
  // triangular (a transposed lower-triangular matrix), so K starts at m0;
  // 4 as 1 but the tiles above the diagonal are not written at all.
  int tri;
  // Modes 2 and 3 give row tile m a K range of m + 1 (mode 2) or T - m (mode
  // 3) of the T row tiles' chunks, so when pair_m = T > 0 the grid covers
  // pairs of row tiles and the workgroup of pair p runs tiles p and T - 1 - p:
  // every workgroup then has the same T + 1 chunks of work.
  int pair_m;
  // Host side only (no kernel reads them): a caller-provided buffer for the
  // split-K partials, used instead of an allocation when ws != nullptr, and
  // its capacity in floats.
  float* ws;
  int64_t ws_floats;
};

constexpr int kGroupM = 8;
constexpr int kPad = 4;

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB>
struct GemmCfg {
  static constexpr int kThreads = 256;
  static constexpr int kWavesM = BM / WM;
  static constexpr int kWavesN = BN / WN;
  static_assert(kWavesM * kWavesN == 4, "4 waves per workgroup");
  static constexpr int TM = WM / 32;
  static constexpr int TN = WN / 32;
  static constexpr int LDA_S = BM + kPad;  // LDS row stride (floats) of the A tile
  static constexpr int LDB_S = BN + kPad;
  // global -> register loads, in float4 units per thread
  static constexpr int PA = (BM * BK) / (4 * kThreads);
  static constexpr int PB = (BN * BK) / (4 * kThreads);
  static_assert(PA >= 1 && PB >= 1, "tile too small for 256 threads");
};

// Output tile of this workgroup.  blockIdx.x runs over (batch, tile) pairs.
// Workgroups are dealt to the 8 XCDs round-robin by id, so id -> (id % 8) *
// (total / 8) + id / 8 gives each XCD a contiguous run of pairs: all tiles of
// a batch (which share that batch's operands) and neighbouring tiles of one
// GEMM hit one L2.  Within a batch, tiles are walked in GROUP_M row groups.
struct TileId {
  int64_t batch;
  int tile_m, tile_n;
  int split;  // K range (kps elements from split * kps)
};
__device__ __forceinline__ TileId tile_id(const GemmArgs& g) {
  // Tiles are remapped so that each XCD (workgroups reach the 8 XCDs
  // round-robin in dispatch order) takes a contiguous run of them; the K
  // split is the grid's z.  (Folding the split into the run measured slower:
  // 1024^3 on 2 splits 30.0 against 27.5 us.)
  const int ntiles = g.tiles_m * g.tiles_n;
  const int64_t total = (int64_t)ntiles * g.nbatch;
  int64_t lin = blockIdx.x;
  if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
  TileId t;
  t.split = (int)blockIdx.z;
  t.batch = lin / ntiles;
  const int bid = (int)(lin - t.batch * ntiles);
  const int group_size = kGroupM * g.tiles_n;
  const int group = bid / group_size;
  const int first_m = group * kGroupM;
  const int gm = min(g.tiles_m - first_m, kGroupM);
  t.tile_m = first_m + (bid % group_size) % gm;
  t.tile_n = (bid % group_size) / gm;
  return t;
}

// Writes a wave's TM x TN 32x32 MFMA accumulators (rows from row0, columns
// from col0) with the bias; rows and columns outside M x N are skipped.
// D[i][j] of a 32x32 tile sits in lane j + 32*((i/4)%2), register
// (i%4) + 4*(i/8).
template <int TM, int TN>
__device__ __forceinline__ void store_acc(const GemmArgs& g, float* __restrict__ C,
                                          const floatx16 (&acc)[TM][TN], int64_t row0,
                                          int64_t col0, int l32, int half, int64_t batch) {
  const float* __restrict__ bias = g.bias;
#pragma unroll
  for (int a = 0; a < TM; ++a) {
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const int64_t col = col0 + 32 * b + l32;
      if (col >= g.N) continue;
      float bias1 = 0.f;
      if (g.bias_mode == 1) bias1 = bias[col];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = row0 + 32 * a + 8 * (r >> 2) + 4 * half + (r & 3);
        if (row < g.M) {
          float v = acc[a][b][r];
          if (g.bias_mode == 1)
            v += bias1;
          else if (g.bias_mode == 2)
            v += bias[(row % g.bias_rows) * g.N + col];
          else if (g.bias_mode == 3)
            v += bias[batch * g.sBias + row * g.N + col];
          C[row * g.ldc + col] = v;
        }
      }
    }
  }
}

// NBUF = 2: double-buffered LDS tiles, one barrier per K chunk; NBUF = 1: one
// LDS tile (half the LDS, so more workgroups per CU), two barriers per chunk.
// TRI: the triangular (causal attention) modes are compiled in; the plain
// instantiations carry none of their code.
// One output tile of gemm_f32_mfma_kernel (the workgroup's, or each of its
// pair of row tiles in the paired triangular modes).
template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, int NBUF, bool TRI>
__device__ __forceinline__ void gemm_mfma_tile(const GemmArgs& g, const TileId tid_) {
  using Cfg = GemmCfg<BM, BN, BK, WM, WN, TA, TB>;
  constexpr int TM = Cfg::TM, TN = Cfg::TN;
  constexpr int LDA_S = Cfg::LDA_S, LDB_S = Cfg::LDB_S;
  constexpr int PA = Cfg::PA, PB = Cfg::PB;

  __shared__ __attribute__((aligned(16))) float As[NBUF][BK * LDA_S];
  __shared__ __attribute__((aligned(16))) float Bs[NBUF][BK * LDB_S];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / Cfg::kWavesN;
  const int wn = wave % Cfg::kWavesN;

  const int64_t batch = tid_.batch;
  const int tile_m = tid_.tile_m, tile_n = tid_.tile_n;

  const float* __restrict__ A = g.A + batch * g.sA;
  const float* __restrict__ B = g.B + batch * g.sB;
  float* __restrict__ C = g.C + batch * g.sC + (int64_t)tid_.split * g.sZ;

  const int64_t m0 = (int64_t)tile_m * BM;
  const int64_t n0 = (int64_t)tile_n * BN;
  const int64_t M = g.M, N = g.N;
  // this workgroup's K range [kbeg, K): the whole K, or one split of it
  int64_t kbeg = (int64_t)tid_.split * g.kps;
  int64_t K = min(g.K, kbeg + g.kps);
  // The skipped products are those of exact zeros, so the sums are unchanged.
  if constexpr (TRI) {
    if (g.tri == 1 && n0 >= m0 + BM) K = kbeg;  // every (i, j) of the tile has j > i
    if (g.tri == 4 && n0 >= m0 + BM) return;     // same tiles, left unwritten
    if (g.tri == 2) K = min(K, m0 + BM);         // A[i][k] == 0 for k > i
    if (g.tri == 3) kbeg = max(kbeg, (m0 / BK) * BK);  // op(A)[i][k] == 0 for k < i
  }
  const bool interior = (m0 + BM <= M) && (n0 + BN <= N);

  float4 ra[PA], rb[PB];

  // ---- global -> registers for the K chunk starting at k0 ---------------
  // mode (a compile-time choice of the caller): 0 = guarded scalar loads;
  // the chunk lies inside M, N and K, so no per-element guard is needed,
  // with 1 = float4 loads (aligned operands) or 2 = scalar loads.
  auto load_chunk = [&](int64_t k0, auto mode_tag) {
    constexpr int mode = decltype(mode_tag)::value;
#pragma unroll
    for (int p = 0; p < PA; ++p) {
      const int f = p * 256 + tid;  // float4 index within the A tile
      int64_t i, k;
      if (!TA) {
        constexpr int KV = BK / 4;
        i = m0 + f / KV;
        k = k0 + (f % KV) * 4;
        const float* src = A + i * g.lda + k;
        if (mode == 1) {
          ra[p] = *reinterpret_cast<const float4*>(src);
        } else if (mode == 2) {
          ra[p] = make_float4(src[0], src[1], src[2], src[3]);
        } else {
          float v[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] = (i < M && k + c < K) ? src[c] : 0.f;
          ra[p] = make_float4(v[0], v[1], v[2], v[3]);
        }
      } else {
        constexpr int IV = BM / 4;
        i = m0 + (f % IV) * 4;
        k = k0 + f / IV;
        const float* src = A + k * g.lda + i;
        if (mode == 1) {
          ra[p] = *reinterpret_cast<const float4*>(src);
        } else if (mode == 2) {
          ra[p] = make_float4(src[0], src[1], src[2], src[3]);
        } else {
          float v[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] = (k < K && i + c < M) ? src[c] : 0.f;
          ra[p] = make_float4(v[0], v[1], v[2], v[3]);
        }
      }
    }
#pragma unroll
    for (int p = 0; p < PB; ++p) {
      const int f = p * 256 + tid;
      int64_t j, k;
      if (!TB) {
        constexpr int JV = BN / 4;
        j = n0 + (f % JV) * 4;
        k = k0 + f / JV;
        const float* src = B + k * g.ldb + j;
        if (mode == 1) {
          rb[p] = *reinterpret_cast<const float4*>(src);
        } else if (mode == 2) {
          rb[p] = make_float4(src[0], src[1], src[2], src[3]);
        } else {
          float v[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] = (k < K && j + c < N) ? src[c] : 0.f;
          rb[p] = make_float4(v[0], v[1], v[2], v[3]);
        }
      } else {
        constexpr int KV = BK / 4;
        j = n0 + f / KV;
        k = k0 + (f % KV) * 4;
        const float* src = B + j * g.ldb + k;
        if (mode == 1) {
          rb[p] = *reinterpret_cast<const float4*>(src);
        } else if (mode == 2) {
          rb[p] = make_float4(src[0], src[1], src[2], src[3]);
        } else {
          float v[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] = (j < N && k + c < K) ? src[c] : 0.f;
          rb[p] = make_float4(v[0], v[1], v[2], v[3]);
        }
      }
    }
  };

  // ---- registers -> LDS (k-major tiles) ----------------------------------
  auto store_chunk = [&](int buf) {
    float* as = As[buf];
    float* bs = Bs[buf];
#pragma unroll
    for (int p = 0; p < PA; ++p) {
      const int f = p * 256 + tid;
      if (!TA) {
        constexpr int KV = BK / 4;
        const int i = f / KV, k = (f % KV) * 4;
        as[(k + 0) * LDA_S + i] = ra[p].x;
        as[(k + 1) * LDA_S + i] = ra[p].y;
        as[(k + 2) * LDA_S + i] = ra[p].z;
        as[(k + 3) * LDA_S + i] = ra[p].w;
      } else {
        constexpr int IV = BM / 4;
        const int i = (f % IV) * 4, k = f / IV;
        *reinterpret_cast<float4*>(&as[k * LDA_S + i]) = ra[p];
      }
    }
#pragma unroll
    for (int p = 0; p < PB; ++p) {
      const int f = p * 256 + tid;
      if (!TB) {
        constexpr int JV = BN / 4;
        const int j = (f % JV) * 4, k = f / JV;
        *reinterpret_cast<float4*>(&bs[k * LDB_S + j]) = rb[p];
      } else {
        constexpr int KV = BK / 4;
        const int j = f / KV, k = (f % KV) * 4;
        bs[(k + 0) * LDB_S + j] = rb[p].x;
        bs[(k + 1) * LDB_S + j] = rb[p].y;
        bs[(k + 2) * LDB_S + j] = rb[p].z;
        bs[(k + 3) * LDB_S + j] = rb[p].w;
      }
    }
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  const int half = lane >> 5;  // which K lane of the MFMA this lane feeds
  const int l32 = lane & 31;
  const int a_off = wm * WM + l32;
  const int b_off = wn * WN + l32;

  auto compute_chunk = [&](int buf) {
    const float* as = As[buf];
    const float* bs = Bs[buf];
#pragma unroll
    for (int s = 0; s < BK / 2; ++s) {
      const int kk = s + half * (BK / 2);
      float af[TM], bf[TN];
#pragma unroll
      for (int a = 0; a < TM; ++a) af[a] = as[kk * LDA_S + a_off + 32 * a];
#pragma unroll
      for (int b = 0; b < TN; ++b) bf[b] = bs[kk * LDB_S + b_off + 32 * b];
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a], bf[b], acc[a][b], 0, 0, 0);
    }
  };

  // K chunks [kbeg, K) of BK.  Interior tiles load every chunk but a ragged
  // last one without guards (float4 when the operands allow it, else
  // scalar); edge tiles always use guarded loads.  The choice is made once
  // per workgroup, so each loop body is branch-free.
  const int64_t nk = (K - kbeg + BK - 1) / BK;
  auto main_loop = [&](auto mode_tag) {
    constexpr int LM = decltype(mode_tag)::value;  // load mode of the full chunks
    const int64_t nfast = LM != 0 ? (K - kbeg) / BK : 0;  // chunks loadable without guards
    auto load = [&](int64_t kc) {
      const int64_t k0 = kbeg + kc * BK;
      if (LM != 0 && kc < nfast)
        load_chunk(k0, std::integral_constant<int, LM>{});
      else
        load_chunk(k0, std::integral_constant<int, 0>{});
      // Triangular op(A): in chunks that cross the diagonal band the entries
      // on the zero side are set to 0 as loaded, so the product never depends
      // on what that triangle holds (it may be left unwritten).
      if (TRI && ((g.tri == 2 && k0 + BK - 1 > m0) || (g.tri == 3 && k0 < m0 + BM - 1))) {
#pragma unroll
        for (int p = 0; p < PA; ++p) {
          const int f = p * 256 + tid;  // the index mapping of load_chunk
          float e[4] = {ra[p].x, ra[p].y, ra[p].z, ra[p].w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            int64_t i, k;
            if (!TA) {
              i = m0 + f / (BK / 4);
              k = k0 + (f % (BK / 4)) * 4 + c;
            } else {
              i = m0 + (f % (BM / 4)) * 4 + c;
              k = k0 + f / (BM / 4);
            }
            if (g.tri == 2 ? k > i : k < i) e[c] = 0.f;
          }
          ra[p] = make_float4(e[0], e[1], e[2], e[3]);
        }
      }
    };
    load(0);
    store_chunk(0);
    __syncthreads();
    for (int64_t kc = 0; kc < nk; ++kc) {
      const int cur = NBUF == 2 ? (int)(kc & 1) : 0;
      if (kc + 1 < nk) load(kc + 1);
      compute_chunk(cur);
      if (kc + 1 < nk) {
        if (NBUF == 1) __syncthreads();  // every wave is done reading the tile
        store_chunk(NBUF == 2 ? cur ^ 1 : 0);
      }
      __syncthreads();
    }
  };
  if (interior && g.vec_ok)
    main_loop(std::integral_constant<int, 1>{});
  else if (interior)
    main_loop(std::integral_constant<int, 2>{});
  else
    main_loop(std::integral_constant<int, 0>{});

  store_acc<TM, TN>(g, C, acc, m0 + wm * WM, n0 + wn * WN, l32, half, batch);
}

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, int NBUF, bool TRI = false>
__global__ __launch_bounds__(256) void gemm_f32_mfma_kernel(GemmArgs g) {
  TileId t = tile_id(g);
  if constexpr (TRI) {
    if (g.pair_m > 0) {
      // tile_id ran over pairs: row tiles t.tile_m and pair_m - 1 - t.tile_m
      const int partner = g.pair_m - 1 - t.tile_m;
      gemm_mfma_tile<BM, BN, BK, WM, WN, TA, TB, NBUF, TRI>(g, t);
      if (partner != t.tile_m) {
        __syncthreads();  // every wave is done with the LDS tiles
        t.tile_m = partner;
        gemm_mfma_tile<BM, BN, BK, WM, WN, TA, TB, NBUF, TRI>(g, t);
      }
      return;
    }
  }
  gemm_mfma_tile<BM, BN, BK, WM, WN, TA, TB, NBUF, TRI>(g, t);
}

// ---- direct-to-LDS variant: 128 x BN tiles (BN 128 or 192), 32-deep K chunks
// For launches whose tiles are all interior (M a multiple of 128, N of BN,
// every K range a multiple of 32, operands float4-aligned).  Each chunk's operand
// tiles go from global memory straight into LDS (global_load_lds_dwordx4:
// one wave instruction fills 1 KiB, lane L's 16 bytes at byte 16 L), so no
// registers stage them and no ds_write runs; two LDS buffers (separate
// objects, so the compiler can tell the loads into one from the reads of the
// other), one barrier per chunk.  Which global quad a lane fetches sets the
// LDS layout:
//  * k-contiguous operand (A when !TA, B when TB): row x of the tile holds
//    its 32 k as 8 quads, quad q in slot q ^ ((x >> 1) & 7), so the 16 lanes
//    of a ds_read_b128 phase (16 rows, one quad each) hit distinct banks;
//  * m/n-contiguous operand (A when TA, B when !TB): row k holds the tile's
//    128 m (BN n) in order; a region's 256 floats are the next 256 of that
//    row-major k x BN tile, whichever rows they fall in.
// BN = 192 serves outputs of N = 768 (GPT-2's d_model): 8192 x 768 is 256
// tiles, one per CU, where 128 x 128 tiles would leave half the CUs a second
// tile.  Its 80 KiB of LDS would let two workgroups share a CU, so it is
// launched with 4 KiB of dynamic LDS more, which keeps one per CU.
// Step s = 4t + r of a chunk feeds the MFMA's K lanes k = 8t + r (lanes
// 0-31) and k = 8t + 4 + r (lanes 32-63), so a k-contiguous fragment is one
// ds_read_b128 per 4 steps.
template <bool TA, bool TB, int BN, int NB = 2, int BM = 128>
__global__ __launch_bounds__(256, 2) void gemm_f32_dtl_kernel(GemmArgs g) {
  static_assert(BN == 64 || BN == 128 || BN == 192, "direct-to-LDS tiles are 64/128 x 64/128/192");
  static_assert(BM == 128 || (BM == 64 && BN == 64), "64-row tiles are 64 x 64");
  static_assert(NB == 2 || NB == 3, "two or three LDS buffers");
  constexpr int BK = 32, WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
  constexpr int RA = BM * BK / 256 / 4;  // 1 KiB regions of the A tile per wave
  constexpr int RB = BN * BK / 256 / 4;  // 1 KiB regions of the B tile per wave
  __shared__ __attribute__((aligned(16))) float As0[BM * BK];
  __shared__ __attribute__((aligned(16))) float As1[BM * BK];
  __shared__ __attribute__((aligned(16))) float Bs0[BN * BK];
  __shared__ __attribute__((aligned(16))) float Bs1[BN * BK];
  __shared__ __attribute__((aligned(16))) float As2[NB == 3 ? BM * BK : 4];
  __shared__ __attribute__((aligned(16))) float Bs2[NB == 3 ? BN * BK : 4];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;  // 2 x 2 waves of 64 x WN
  const int half = lane >> 5, l32 = lane & 31;

  const TileId tid_ = tile_id(g);
  const int64_t batch = tid_.batch;
  const int64_t m0 = (int64_t)tid_.tile_m * BM, n0 = (int64_t)tid_.tile_n * BN;
  const float* __restrict__ A = g.A + batch * g.sA;
  const float* __restrict__ B = g.B + batch * g.sB;
  float* __restrict__ C = g.C + batch * g.sC + (int64_t)tid_.split * g.sZ;
  const int64_t kbeg = (int64_t)tid_.split * g.kps;
  const int64_t nk = (min(g.K, kbeg + g.kps) - kbeg) / BK;

  // The lane's global source for each of the wave's instructions per
  // operand tile (instruction j fills the tile's 1 KiB region R = 4 wave + j
  // of A, R = RB wave + j of B) at the first chunk, and the advance per chunk.
  // pb has a fixed size (RB <= 6 entries used): with the template-dependent
  // size RB, the host pass of this compiler silently emits no launch stub for
  // the kernel, whose lambdas capture the array.
  const float* pa[4];
  const float* pb[6];
  static_assert(RA <= 4 && RB <= 6, "A / B regions per wave");
  constexpr int kRowLanes = BM / 4;  // m-contiguous A: lanes per k row of a region
#pragma unroll
  for (int j = 0; j < RA; ++j) {
    const int R = RA * wave + j;
    const int r = 8 * R + (lane >> 3);                // k-contiguous: tile row
    const int q = (lane & 7) ^ ((r >> 1) & 7);        // logical quad of slot lane & 7
    const int kr = (256 / BM) * R + lane / kRowLanes;  // m-contiguous: k row
    pa[j] = TA ? A + (kbeg + kr) * g.lda + m0 + 4 * (lane % kRowLanes)
               : A + (m0 + r) * g.lda + kbeg + 4 * q;
  }
#pragma unroll
  for (int j = 0; j < RB; ++j) {
    const int R = RB * wave + j;
    const int r = 8 * R + (lane >> 3);
    const int q = (lane & 7) ^ ((r >> 1) & 7);
    const int f = 256 * R + 4 * lane;                 // n-contiguous: float f of the tile
    pb[j] = TB ? B + (n0 + r) * g.ldb + kbeg + 4 * q
               : B + (kbeg + f / BN) * g.ldb + n0 + f % BN;
  }
  const int64_t a_step = TA ? BK * g.lda : BK;
  const int64_t b_step = TB ? BK : BK * g.ldb;

  // Two buffers: the compiler-tracked DMA builtin (it waits for all of a
  // chunk's loads before the barrier anyway).  Three buffers: the same
  // instruction as inline asm, which the compiler does not track, so that
  // one chunk's loads stay in flight across the barrier (the tracked form
  // gets a vmcnt(0) before every LDS read it cannot prove disjoint).
  auto issue = [&](int64_t kc, auto buf_tag) {
    constexpr int bt = decltype(buf_tag)::value;
    float* as = bt == 2 ? As2 : (bt == 1 ? As1 : As0);
    float* bs = bt == 2 ? Bs2 : (bt == 1 ? Bs1 : Bs0);
#pragma unroll
    for (int j = 0; j < RA; ++j) {
      if constexpr (NB == 3)
        WXX_LDS_DMA_DWORDX4(pa[j] + kc * a_step, as + (RA * wave + j) * 256);
      else
        __builtin_amdgcn_global_load_lds(pa[j] + kc * a_step, as + (RA * wave + j) * 256, 16, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      if constexpr (NB == 3)
        WXX_LDS_DMA_DWORDX4(pb[j] + kc * b_step, bs + (RB * wave + j) * 256);
      else
        __builtin_amdgcn_global_load_lds(pb[j] + kc * b_step, bs + (RB * wave + j) * 256, 16, 0, 0);
    }
  };

  // fragment addresses (floats): k-contiguous row x = w * 64 + l32 (+ 32 a)
  // reads logical quad 2t + half, i.e. slot (2t + half) ^ ((l32 >> 1) & 7);
  // m/n-contiguous reads (k, y) at k * 128 + y with k = 8t + 4 half + r.
  const int sw = (l32 >> 1) & 7;
  int qoff[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) qoff[t] = 4 * (((2 * t) ^ (sw & 6)) | ((half ^ sw) & 1));
  const int xa = (wm * WM + l32) * BK, xb = (wn * WN + l32) * BK;
  const int ya = 4 * half * BM + wm * WM + l32, yb = 4 * half * BN + wn * WN + l32;

  floatx16 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  auto compute = [&](auto buf_tag) {
    constexpr int bt = decltype(buf_tag)::value;
    const float* as = bt == 2 ? As2 : (bt == 1 ? As1 : As0);
    const float* bs = bt == 2 ? Bs2 : (bt == 1 ? Bs1 : Bs0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float av[TM][4], bv[TN][4];
#pragma unroll
      for (int a = 0; a < TM; ++a) {
        if (!TA) {
          const float4 v = *reinterpret_cast<const float4*>(&as[xa + 32 * BK * a + qoff[t]]);
          av[a][0] = v.x, av[a][1] = v.y, av[a][2] = v.z, av[a][3] = v.w;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) av[a][r] = as[(8 * t + r) * BM + ya + 32 * a];
        }
      }
#pragma unroll
      for (int b = 0; b < TN; ++b) {
        if (TB) {
          const float4 v = *reinterpret_cast<const float4*>(&bs[xb + 32 * BK * b + qoff[t]]);
          bv[b][0] = v.x, bv[b][1] = v.y, bv[b][2] = v.z, bv[b][3] = v.w;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) bv[b][r] = bs[(8 * t + r) * BN + yb + 32 * b];
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
          for (int b = 0; b < TN; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a][r], bv[b][r], acc[a][b], 0, 0, 0);
    }
  };
  // every wave's loads of a chunk have landed before the barrier that
  // publishes it (0x0F70: s_waitcnt vmcnt(0), the other counters left alone)
  auto landed = [&]() {
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
  };

  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  using B2 = std::integral_constant<int, 2>;
  if constexpr (NB == 3) {
    // chunk c in buffer c % 3: at step c a wave waits until only its loads
    // of chunk c + 1 are outstanding (loads complete in order), a bare
    // barrier publishes chunk c and frees the buffer of chunk c - 1, which
    // then receives chunk c + 2
    constexpr int kPer = RA + RB;  // loads per wave per chunk
    constexpr int kWaitNext = 0x0F70 | (kPer & 15) | ((kPer >> 4) << 14);
    auto step = [&](int64_t kc, auto cur, auto nxt2) {
      if (kc + 1 < nk)
        __builtin_amdgcn_s_waitcnt(kWaitNext);
      else
        __builtin_amdgcn_s_waitcnt(0x0F70);
      WXX_S_BARRIER();
      if (kc + 2 < nk) issue(kc + 2, nxt2);
      compute(cur);
    };
    if (nk > 0) issue(0, B0{});
    if (nk > 1) issue(1, B1{});
    for (int64_t kc = 0; kc < nk; kc += 3) {
      step(kc, B0{}, B2{});
      if (kc + 1 < nk) step(kc + 1, B1{}, B0{});
      if (kc + 2 < nk) step(kc + 2, B2{}, B1{});
    }
  } else if (nk > 0) {
    issue(0, B0{});
    landed();
    for (int64_t kc = 0; kc < nk; kc += 2) {
      if (kc + 1 < nk) issue(kc + 1, B1{});
      compute(B0{});
      landed();  // chunk kc + 1 is in buffer 1; every wave is done with buffer 0
      if (kc + 1 < nk) {
        if (kc + 2 < nk) issue(kc + 2, B0{});
        compute(B1{});
        landed();
      }
    }
  }
  store_acc<TM, TN>(g, C, acc, m0 + wm * WM, n0 + wn * WN, l32, half, batch);
}

template <int BM, int BN, int BK, int WM, int WN, int NBUF, bool TRI = false, bool DTL = false>
int launch_tiles(GemmArgs& g, int64_t batch, bool ta, bool tb, int splits);

// Adds the split-K partials part[z][b][M][N] in split order (deterministic)
// and applies the bias: C = sum_z part[z] + bias.
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(GemmArgs g,
                                                                  const float* __restrict__ part,
                                                                  int splits, int64_t batch) {
  const int64_t mn = g.M * g.N, n = mn * batch;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * 256) {
    float v = 0.f;
    for (int z = 0; z < splits; ++z) v += part[(int64_t)z * n + e];
    const int64_t b = e / mn, r = e - b * mn;
    const int64_t row = r / g.N, col = r - row * g.N;
    if (g.bias_mode == 1)
      v += g.bias[col];
    else if (g.bias_mode == 2)
      v += g.bias[(row % g.bias_rows) * g.N + col];
    else if (g.bias_mode == 3)
      v += g.bias[b * g.sBias + r];
    g.C[b * g.sC + row * g.ldc + col] = v;
  }
}

// The same for a contiguous C (ldc == N) with N % 4 == 0, 16-byte aligned
// partials and C, and fewer than 2^31 elements: four columns per item,
// four items per thread with every split's loads issued before the sums,
// 32-bit row arithmetic once per item.
__global__ __launch_bounds__(256) void gemm_splitk_reduce4_kernel(GemmArgs g,
                                                                   const float4* __restrict__ part,
                                                                   int splits, int64_t batch) {
  const int n4 = (int)(g.M * g.N * batch / 4), mn4 = (int)(g.M * g.N / 4), N4 = (int)(g.N / 4);
  const int step = gridDim.x * 256;
  for (int e0 = blockIdx.x * 256 + threadIdx.x; e0 < n4; e0 += 4 * step) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (e0 + u * step < n4) v[u] = part[e0 + u * step];
    for (int z = 1; z < splits; ++z) {
      float4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (e0 + u * step < n4) q[u] = part[(int64_t)z * n4 + e0 + u * step];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        v[u].x += q[u].x;
        v[u].y += q[u].y;
        v[u].z += q[u].z;
        v[u].w += q[u].w;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = e0 + u * step;
      if (e >= n4) continue;
      const int b = e / mn4, r4 = e - b * mn4;
      const int row = r4 / N4, col = 4 * (r4 - row * N4);
      const float* bias = nullptr;
      if (g.bias_mode == 1)
        bias = g.bias + col;
      else if (g.bias_mode == 2)
        bias = g.bias + (int64_t)(row % g.bias_rows) * g.N + col;
      else if (g.bias_mode == 3)
        bias = g.bias + (int64_t)b * g.sBias + (int64_t)row * g.N + col;
      float4 w = v[u];
      if (bias) {
        w.x += bias[0];
        w.y += bias[1];
        w.z += bias[2];
        w.w += bias[3];
      }
      *(float4*)(g.C + (int64_t)b * g.sC + (int64_t)row * g.N + col) = w;
    }
  }
}

template <int BM, int BN, int BK, int WM, int WN, int NBUF = 2, bool TRI = false,
          bool DTL = false>
int launch_cfg(GemmArgs& g, int64_t batch, bool ta, bool tb, int splits = 1) {
  g.tiles_m = (int)((g.M + BM - 1) / BM);
  g.tiles_n = (int)((g.N + BN - 1) / BN);
  g.pair_m = 0;
  if (TRI && (g.tri == 2 || g.tri == 3) && splits <= 1 && g.tiles_m > 1) {
    g.pair_m = g.tiles_m;
    g.tiles_m = (g.tiles_m + 1) / 2;
  }
  // K == 0 has nothing to split (and no K range to size splits from)
  if (splits <= 1 || g.K == 0) {
    g.kps = g.K > 0 ? g.K : 1;
    g.sZ = 0;
    return launch_tiles<BM, BN, BK, WM, WN, NBUF, TRI, DTL>(g, batch, ta, tb, 1);
  }
  // Split K: partial products go to a scratch buffer (bias off), then one
  // pass adds them in split order and applies the bias.
  int64_t kps = (g.K + splits - 1) / splits;
  kps = (kps + BK - 1) / BK * BK;
  splits = (int)((g.K + kps - 1) / kps);
  GemmArgs p = g;
  const int64_t n = g.M * g.N * batch;
  float* part;
  if (g.ws) {
    // every split writes every element of its partial (splits were
    // recounted above so none has an empty K range): nothing to clear
    if (n * splits > g.ws_floats)
      return wxx::set_error(WXX_E_RANGE,
                            "GEMM split-K partials need %lld floats (%lld x %d splits); the "
                            "allocation-free scratch holds %lld",
                            (long long)(n * splits), (long long)n, splits,
                            (long long)g.ws_floats);
    part = g.ws;
  } else {
    part = (float*)wxx::scratch_alloc(sizeof(float) * (size_t)n * splits);
    if (!part) return wxx::set_error(WXX_E_OOM, "GEMM split-K partials");
  }
  p.C = part;
  p.ldc = g.N;
  p.sC = g.M * g.N;
  p.sZ = n;
  p.kps = kps;
  p.bias_mode = 0;
  int rc = launch_tiles<BM, BN, BK, WM, WN, NBUF, TRI, DTL>(p, batch, ta, tb, splits);
  if (rc == WXX_OK) {
    const bool vec4 = g.ldc == g.N && g.N % 4 == 0 && n < (int64_t(1) << 31) &&
                      (batch == 1 || g.sC % 4 == 0) && (g.bias_mode != 3 || g.sBias % 4 == 0) &&
                      ((uintptr_t)g.C & 15) == 0 && ((uintptr_t)part & 15) == 0;
    if (vec4)
      hipLaunchKernelGGL(gemm_splitk_reduce4_kernel, dim3(wxx::grid_1d(n / 16, 256, 8192)),
                         dim3(256), 0, wxx::stream(), g, (const float4*)part, splits, batch);
    else
      hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3(wxx::grid_1d(n, 256, 8192)), dim3(256),
                         0, wxx::stream(), g, (const float*)part, splits, batch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) rc = wxx::set_error(WXX_E_HIP, "split-K reduce: %s", hipGetErrorString(e));
  }
  if (!g.ws) wxx::scratch_free(part);
  return rc;
}

template <int BM, int BN, int BK, int WM, int WN, int NBUF, bool TRI, bool DTL>
int launch_tiles(GemmArgs& g, int64_t batch, bool ta, bool tb, int splits) {
  g.nbatch = batch;
  dim3 grid((unsigned)((int64_t)g.tiles_m * g.tiles_n * batch), 1, (unsigned)splits);
  hipStream_t s = wxx::stream();
  if constexpr (DTL) {
    static_assert((BM == 128 && (BN == 64 || BN == 128 || BN == 192) || BM == 64 && BN == 64) &&
                      BK == 32,
                  "direct-to-LDS tiles are 128 x 64/128/192 or 64 x 64, x 32");
    // 128 x 192: 4 KiB of dynamic LDS on top of the tiles' 80 KiB, so that
    // one workgroup occupies a CU (the grids it is chosen for are <= 1 per CU)
    const unsigned dyn = BN == 192 ? 4096u : 0u;
    constexpr int NB = NBUF == 3 ? 3 : 2;
    if (!ta && !tb)
      hipLaunchKernelGGL((gemm_f32_dtl_kernel<false, false, BN, NB, BM>), grid, dim3(256), dyn, s, g);
    else if (!ta && tb)
      hipLaunchKernelGGL((gemm_f32_dtl_kernel<false, true, BN, NB, BM>), grid, dim3(256), dyn, s, g);
    else if (ta && !tb)
      hipLaunchKernelGGL((gemm_f32_dtl_kernel<true, false, BN, NB, BM>), grid, dim3(256), dyn, s, g);
    else
      hipLaunchKernelGGL((gemm_f32_dtl_kernel<true, true, BN, NB, BM>), grid, dim3(256), dyn, s, g);
  } else {
    if (!ta && !tb)
      hipLaunchKernelGGL((gemm_f32_mfma_kernel<BM, BN, BK, WM, WN, false, false, NBUF, TRI>),
                         grid, dim3(256), 0, s, g);
    else if (!ta && tb)
      hipLaunchKernelGGL((gemm_f32_mfma_kernel<BM, BN, BK, WM, WN, false, true, NBUF, TRI>),
                         grid, dim3(256), 0, s, g);
    else if (ta && !tb)
      hipLaunchKernelGGL((gemm_f32_mfma_kernel<BM, BN, BK, WM, WN, true, false, NBUF, TRI>),
                         grid, dim3(256), 0, s, g);
    else
      hipLaunchKernelGGL((gemm_f32_mfma_kernel<BM, BN, BK, WM, WN, true, true, NBUF, TRI>),
                         grid, dim3(256), 0, s, g);
  }
  WXX_LAUNCHED();
  return WXX_OK;
}

inline bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// Replaces functional.matmul_add (reference src/wxx/functional/utils.py:378-499).
// Strides are in elements; sA / sB == 0 marks an unbatched operand.
// tile: 0 = choose automatically, 1 = 64x64, 2 = 128x128, 3 = 256x128; 4-10 select
// alternative tile / K-chunk / buffering shapes of the same kernel; 11 / 12 / 13 the
// direct-to-LDS 128x128 / 128x192 / 128x64 kernel, 14 its 128x64 tiles with
// three LDS buffers, 15 its 64x64 tiles with three buffers.  With an
// explicit tile code, bits 8-15 give the number of K splits (0 or 1: none).
namespace {
int matmul_impl(const float* A, const float* B, const float* bias, float* C, int64_t M, int64_t N,
                int64_t K, int64_t batch, int64_t sA, int64_t sB, int64_t sBias, int bias_mode,
                int transpose_A, int transpose_B, int tile, int tri, float* ws = nullptr,
                int64_t ws_floats = 0);
}  // namespace

WXX_API int wxx_matmul_add(const float* A, const float* B, const float* bias, float* C,
                           int64_t M, int64_t N, int64_t K, int64_t batch, int64_t sA,
                           int64_t sB, int64_t sBias, int bias_mode, int transpose_A,
                           int transpose_B, int tile) {
  return matmul_impl(A, B, bias, C, M, N, K, batch, sA, sB, sBias, bias_mode, transpose_A,
                     transpose_B, tile, 0);
}

// Causal-attention products (no counterpart in the reference: the same
// C = op(A) op(B) as wxx_matmul_add without bias, for operands whose
// entries above the diagonal are exactly zero, or outputs whose entries
// above the diagonal are not needed).  tri 1: C is square (M == N) and its
// tiles wholly above the diagonal are set to 0 instead of computed (the
// scores Q K^T and dO V^T of masked attention); tri 2: op(A) is square lower
// triangular (M == K), e.g. the probabilities P in P V; tri 3: op(A) is
// square upper triangular, e.g. P^T in P^T dO; tri 4: as 1, but the tiles
// wholly above the diagonal are left unwritten (for consumers that read only
// the lower triangle).  The products skipped are those of exact zeros, so
// the results equal wxx_matmul_add's.
WXX_API int wxx_matmul_tri(const float* A, const float* B, float* C, int64_t M, int64_t N,
                           int64_t K, int64_t batch, int64_t sA, int64_t sB, int transpose_A,
                           int transpose_B, int tri) {
  WXX_REQUIRE(tri >= 1 && tri <= 4, "bad tri mode %d", tri);
  WXX_REQUIRE((tri == 1 || tri == 4) ? M == N : M == K,
              "tri mode %d needs a square triangular operand", tri);
  return matmul_impl(A, B, nullptr, C, M, N, K, batch, sA, sB, 0, 0, transpose_A, transpose_B, 0,
                     tri);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of wxx_matmul_add, for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops): its only
// temporary, the split-K partials, lives in this fixed array instead of the
// caching allocator.  Every GPU that loads the library holds its own copy
// (64 MiB) until the process ends.  In host code `scratch` names a host-side
// stand-in, never the device memory: the device address is looked up once
// per device with hipGetSymbolAddress (wxx::gemm_noalloc_setup, run by
// wxx_init with that device current) and only that address is used.
constexpr int64_t kNoAllocScratchFloats = int64_t(16) << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
float* g_scratch_dev[kMaxDevices] = {};
}  // namespace

namespace wxx {
int gemm_noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices)
    return set_error(WXX_E_ARG, "device %d beyond the %d the library tracks", device,
                     kMaxDevices);
  if (g_scratch_dev[device]) return WXX_OK;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return set_error(WXX_E_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  g_scratch_dev[device] = (float*)p;
  return WXX_OK;
}
}  // namespace wxx

// Same arguments, kernels and results as wxx_matmul_add (bit for bit: the
// tile and split choice is the same), but allocates nothing: a call whose
// split-K partials would exceed the scratch (16 Mi floats) fails with
// WXX_E_RANGE before anything is enqueued.  All calls on a GPU share its one
// scratch array: calls that overlap on one GPU (other streams or processes
// running the library's stream concurrently) race.  The partials of each
// split are written in full before they are read, so nothing in the scratch
// has to start at zero and a call never depends on an earlier call's
// contents.
WXX_API int wxx_matmul_add_noalloc(const float* A, const float* B, const float* bias, float* C,
                                   int64_t M, int64_t N, int64_t K, int64_t batch, int64_t sA,
                                   int64_t sB, int64_t sBias, int bias_mode, int transpose_A,
                                   int transpose_B, int tile) {
  WXX_CHECK_INIT();
  int dev = -1;
  WXX_HIP(hipGetDevice(&dev));
  float* ws = (dev >= 0 && dev < kMaxDevices) ? g_scratch_dev[dev] : nullptr;
  if (!ws)
    return wxx::set_error(WXX_E_INIT, "no allocation-free scratch on device %d (wxx_init "
                          "sets it up)", dev);
  return matmul_impl(A, B, bias, C, M, N, K, batch, sA, sB, sBias, bias_mode, transpose_A,
                     transpose_B, tile, 0, ws, kNoAllocScratchFloats);
}

namespace {
int matmul_impl(const float* A, const float* B, const float* bias, float* C, int64_t M, int64_t N,
                int64_t K, int64_t batch, int64_t sA, int64_t sB, int64_t sBias, int bias_mode,
                int transpose_A, int transpose_B, int tile, int tri, float* ws,
                int64_t ws_floats) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(A && B && C, "null pointer");
  WXX_REQUIRE(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "negative GEMM dims");
  WXX_REQUIRE(bias_mode >= 0 && bias_mode <= 3, "bad bias_mode %d", bias_mode);
  WXX_REQUIRE(bias_mode == 0 || bias, "bias pointer is null for bias_mode %d", bias_mode);
  WXX_REQUIRE(batch <= 65535, "batch %lld exceeds 65535", (long long)batch);
  if (M == 0 || N == 0 || batch == 0) return WXX_OK;

  GemmArgs g;
  g.A = A;
  g.B = B;
  g.bias = bias;
  g.C = C;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = transpose_A ? M : K;
  g.ldb = transpose_B ? K : N;
  g.ldc = N;
  g.sA = sA;
  g.sB = sB;
  g.sC = M * N;
  g.sBias = sBias;
  g.bias_mode = bias_mode;
  g.bias_rows = M;
  g.tri = tri;
  g.pair_m = 0;
  g.ws = ws;
  g.ws_floats = ws_floats;
  int64_t nb = batch;
  // Fold the batch into M when B is shared and A's rows are contiguous across
  // batches: one larger GEMM fills the GPU better than `batch` small ones.
  // (A per-batch bias folds into an (M*batch, N) bias only when its batches
  // are packed back to back.)
  if (batch > 1 && sB == 0 && !transpose_A && sA == M * K && tri == 0 &&
      (bias_mode != 3 || sBias == M * N)) {
    g.M = M * batch;
    g.sA = 0;
    g.sC = 0;
    if (bias_mode == 3) {
      g.bias_mode = 2;
      g.bias_rows = M * batch;
    }
    nb = 1;
  }
  g.vec_ok = (g.lda % 4 == 0) && (g.ldb % 4 == 0) && (g.sA % 4 == 0) && (g.sB % 4 == 0) &&
             al16(A) && al16(B);
  // every tile interior and every K range whole chunks: the direct-to-LDS kernel applies
  const bool dtl_ok = g.vec_ok && g.M % 128 == 0 && g.N % 128 == 0 && K > 0 && K % 32 == 0 &&
                      tri == 0;
  const bool dtl192_ok = g.vec_ok && g.M % 128 == 0 && g.N % 192 == 0 && K > 0 && K % 32 == 0 &&
                         tri == 0;
  const bool dtl64_ok = g.vec_ok && g.M % 128 == 0 && g.N % 64 == 0 && K > 0 && K % 32 == 0 &&
                        tri == 0;
  const bool dtl6464_ok = g.vec_ok && g.M % 64 == 0 && g.N % 64 == 0 && K > 0 && K % 32 == 0 &&
                          tri == 0;

  if (K == 0) {
    // Empty contraction: C = bias (or 0).  Reuse the kernel with K = 0: the
    // k-loop is skipped and the epilogue writes the bias.
  }
  int splits = (tile >> 8) & 0xff;
  tile &= 0xff;
  WXX_REQUIRE(splits <= 64, "bad split count %d", splits);
  splits = std::max(splits, 1);
  if (K == 0) splits = 1;
  if (tile == 0) {
    // Measured on MI355X (fp32 GEMM shapes of GPT-2 small and BASELINE
    // config 2): the direct-to-LDS 128x128 tiles are the fastest wherever
    // they apply and balance; otherwise 128x128 tiles once they cover the CUs
    // twice (128x64 below that when K is short);
    // the 32-deep single-buffered variant wins for long K; 64x64 tiles win
    // for thin operands (attention's N = 64 / K = 64 products) and when the
    // grid would otherwise leave CUs idle; K is split only when the output
    // tiles cannot cover the CUs twice and every split keeps >= 1024 of K.
    const int64_t cus = wxx::num_cus() > 0 ? wxx::num_cus() : 256;
    const int64_t t128 = ((g.M + 127) / 128) * ((g.N + 127) / 128) * nb;
    const int64_t t64 = ((g.M + 63) / 64) * ((g.N + 63) / 64) * nb;
    const int64_t kmax = std::max<int64_t>(g.K / 1024, 1);
    // Direct-to-LDS 128 x 128 tiles when every tile is interior and the
    // tiles, times at most 16 K splits of >= 512, keep the CUs evenly busy:
    // s splits of t tiles give t*s units, of which a CU runs
    // ceil(t*s / cus), so the balance is t*s / (ceil(t*s / cus) * cus).  With
    // s > 1 the partials' extra pass moves (s + 1) * M * N * 4 bytes at
    // ~5 TB/s next to 2 * M * N * K flops at ~130 TFLOP/s, a relative cost of
    // (s + 1) * 52 / K.  Below an efficiency of 0.8 the smaller tiles below
    // do better.
    // (Not for K <= 128 or thin M / N: the register-staged 64 x 64 / 128 x 64
    // tiles below are faster there, e.g. attention's 96 x 1024 x 1024 x 64
    // scores at 191 us against 237 us on 128 x 128 direct-to-LDS tiles.)
    const bool thin = g.M <= 64 || g.N <= 64 || g.K <= 128;
    // (Up to 64 splits where K allows: a few output tiles over a very long K,
    // Hyena's 256 x 256 weight gradients over K = 65536, take 64 splits of
    // 1024 on 4 tiles instead of 32 splits on 16 register-staged 64 x 64
    // tiles.)
    const int64_t smax =
        dtl_ok && !thin ? std::min<int64_t>(64, std::max<int64_t>(g.K / 512, 1)) : 0;
    double best = 0.0;
    int best_splits = 1;
    for (int64_t sp = 1; sp <= smax; ++sp) {
      const int64_t units = t128 * sp;
      const double bal = (double)units / (double)(((units + cus - 1) / cus) * cus) /
                         (sp > 1 ? 1.0 + (double)(sp + 1) * 52.0 / (double)g.K : 1.0);
      if (bal > best + 1e-9) {
        best = bal;
        best_splits = (int)sp;
      }
    }
    // 128 x 192 direct-to-LDS tiles, unsplit, when they make one round of at
    // most one tile per CU that balances better (8192 x 768: 256 tiles, where
    // 128 x 128 makes 384, or needs split-K partials to balance), and only
    // where they measured faster on MI355X (GPT-2 small): K >= 16384, where
    // the 128 x 128 alternative adds 16 splits' partials (8192x768x50304:
    // 4.99 against 5.19 ms).  Below that the 128 x 64 tiles (three per CU)
    // are faster, also for a k-contiguous B (8192x768x3072: 303 against 310
    // us, 8192x768x2304: 230 against 239 us; at K = 768 100-101 against
    // 107-108 us).
    const int64_t t192 = dtl192_ok && !thin && g.K >= 16384
                             ? (g.M / 128) * (g.N / 192) * nb
                             : 0;
    const double bal192 = (double)t192 / (double)cus;
    // 128 x 64 direct-to-LDS tiles, unsplit, for grids of 1-4 rounds over the
    // CUs that they balance better than the 128 x 128 ones (measured on
    // MI355X: 8192x768x768 93 / 90 us against 106 / 107 us on the 128 x 64
    // register-staged tiles, B n- / k-contiguous; 8192x768x3072 310 us
    // against 317 us on two K splits of 128 x 128).  Not for thin operands:
    // attention's N = 64 products keep the tiles their causal variants
    // reproduce bit for bit.
    const int64_t t64d = dtl64_ok && !thin ? (g.M / 128) * (g.N / 64) * nb : 0;
    const double bal64 =
        t64d > 0 ? (double)t64d / (double)(((t64d + cus - 1) / cus) * cus) : 0.0;
    // 128 x 64 direct-to-LDS tiles split in K when they number fewer than
    // the CUs, by the same balance and partial-pass cost (1024^3: 128 tiles
    // x 2 splits, 25.3 + 3 us against 35.1 us on unsplit 64 x 64 tiles).
    int s64 = 0;
    double bal64s = 0.0;
    if (t64d > 0 && t64d < cus) {
      for (int sp = 2; sp <= 4; ++sp) {
        if (g.K / sp < 256) break;
        const int64_t units = t64d * sp;
        const double bal = (double)units / (double)(((units + cus - 1) / cus) * cus) /
                           (1.0 + (double)(sp + 1) * 52.0 / (double)g.K);
        if (bal > bal64s + 1e-9) {
          bal64s = bal;
          s64 = sp;
        }
      }
    }
    // 64 x 64 direct-to-LDS tiles (three buffers) where the 128 x 64 ones
    // make less than one round: up to 8 power-of-two K splits of >= 256
    // within one round, by the same balance (measured on MI355X: 1024^3 on
    // 256 unsplit tiles 24.6 against 29.8 us on two K splits of 128 x 64;
    // 1024 x 1024 x 2048 44.0 against 48.4 us; 512 x 512 x 4096 as 64 tiles
    // x 4 splits 28.6 against 43.2 us).
    const int64_t t6464 = dtl6464_ok && !thin ? (g.M / 64) * (g.N / 64) * nb : 0;
    int s6464 = 0;
    double bal6464 = 0.0;
    if (t6464 > 0 && t64d < cus) {
      for (int sp = 1; sp <= 8; sp *= 2) {
        if (sp > 1 && g.K / sp < 256) break;
        const int64_t units = t6464 * sp;
        if (units > cus) break;
        const double bal = (double)units / (double)cus /
                           (sp > 1 ? 1.0 + (double)(sp + 1) * 52.0 / (double)g.K : 1.0);
        if (bal > bal6464 + 1e-9) {
          bal6464 = bal;
          s6464 = sp;
        }
      }
    }
    if (t192 > 0 && t192 <= cus && bal192 >= 0.9 && bal192 > best) {
      tile = 12;
      splits = 1;
    } else if (t64d >= cus && t64d <= 4 * cus && bal64 >= 0.95 && bal64 > best) {
      tile = 13;
      splits = 1;
    } else if (t64d > 4 * cus && g.K <= 1024 && bal64 >= 0.95 && best < 0.95) {
      // many rounds of short-K products that 128 x 128 tiles balance
      // poorly (GPT-2 small's q/k/v projection, 8192 x 2304 x 768: 4.5
      // rounds of 128 x 128, 237 against 255 us on 128 x 64 tiles)
      tile = 13;
      splits = 1;
    } else if (s6464 > 0 && bal6464 >= 0.8 && bal6464 >= bal64s && bal6464 > best &&
               g.K / s6464 <= 2048) {
      // (only for short K per unit: over long K ranges the 128 x 128 tiles'
      // higher arithmetic intensity wins, e.g. 256 x 1024 x 65536 at 309 us
      // on 16 tiles x 16 splits against 352 us on 64 x 64 tiles x 4 splits)
      tile = 15;
      splits = s6464;
    } else if (s64 > 0 && bal64s >= 0.8 && bal64s > best) {
      // three buffers: one round of one workgroup per CU has nothing else
      // to hide its load latency behind (1024^3: 29.5 against 30.2 us)
      tile = 14;
      splits = s64;
    } else if (dtl_ok && t128 * smax >= cus && best >= 0.8) {
      tile = 11;
      splits = best_splits;
    } else if (g.M <= 64 || g.N <= 64 || g.K <= 128) {
      // N = 64 over long M (attention's P V, dS K, P^T dO): 128 x 64 tiles
      tile = (g.N <= 64 && g.M >= 128 && g.K > 128) ? (transpose_A ? 10 : 9) : 1;
      if (nb == 1 && kmax == 1 && g.K >= 256 && 4 * t64 <= cus) {
        // An unbatched product over at most a quarter of the CUs' worth of
        // 64 x 64 tiles with K in [256, 2048) is latency-bound (one
        // workgroup takes about 1.4 us per 16-deep K step): 64 x 64 tiles
        // and up to 8 power-of-two splits of >= 64 of K, as below (measured
        // on MI355X, ResNet18's classifier 128 x 10 x 512: 11.1 us against
        // 44.7 us on one 128 x 64 tile; at K = 128 splitting measured
        // slower).  Batched N <= 64 products (attention's) keep the tiles
        // whose causal variants reproduce them bit for bit.
        tile = 1;
        int s = 1;
        while (s < 8 && t64 * s * 2 <= cus && g.K / (s * 2) >= 64) s *= 2;
        splits = s;
      } else if (tile == 1 && t64 < 2 * cus) {
        // few thin tiles over a long K (Hyena's filter-network weight
        // gradients, 17 x 64 and 64 x 256 over K = 8192): splits of >= 256
        splits = (int)std::min<int64_t>((8 * cus + t64 - 1) / t64,
                                        std::max<int64_t>(g.K / 256, 1));
      }
    } else if (t128 >= cus) {
      tile = g.K >= 4096 ? 4 : 2;
      if (t128 < 2 * cus && g.K >= 2048) {
        tile = 2;
        splits = 2;
      } else if (t128 < 2 * cus) {
        tile = 9;  // short K: 128 x 64 tiles give the grid twice the workgroups
      }
    } else if (2 * t128 >= cus && g.K >= 4096) {
      tile = 4;
      splits = (int)std::min<int64_t>((4 * cus + t128 - 1) / t128, kmax);
    } else if (!dtl_ok && t128 * 64 <= 4 * cus && g.K >= 32768) {
      // a few output tiles over a very long K that the direct-to-LDS tiles
      // cannot take (Hyena's SwiGLU weight gradients, 256 x 682 and 682 x
      // 256 over K = 65536): 128 x 128 tiles, about 3 units per CU, measured
      // 262 us against 286 us on 64 x 64 tiles with 32 splits
      tile = 4;
      splits = (int)std::min<int64_t>(std::min<int64_t>(64, (3 * cus + t128 - 1) / t128), kmax);
    } else {
      tile = 1;
      if (t64 < 2 * cus) splits = (int)std::min<int64_t>((8 * cus + t64 - 1) / t64, kmax);
      // Short K (< 2048) over at most a quarter of the CUs' worth of tiles:
      // these launches are latency-bound (about 1 us per 16-deep K step), so
      // up to 8 power-of-two splits of >= 64 of K that keep the grid within
      // one round of the CUs.  Measured on MI355X (config-1 shapes, split
      // against unsplit): 256x256x512 (A^T) 11.1 / 20.8 us, 256x1024x512
      // 13.4 / 21.1 us, 512x256x1024 13.3 / 32.6 us, 512x256x256 9.8 / 11.1
      // us; 512x1024x256 (128 tiles) is fastest unsplit.
      if (kmax == 1 && 4 * t64 <= cus) {
        int s = 1;
        while (s < 8 && t64 * s * 2 <= cus && g.K / (s * 2) >= 64) s *= 2;
        splits = s;
      }
    }
    splits = std::max(1, std::min(splits, tile == 4 || tile == 11 ? 64 : 32));
  }
  if (tri) {
    // triangular modes: one K range per row tile (no split), on the tile
    // shapes that carry the triangular code.  Modes 2 and 3 run paired row
    // tiles on 64 x 64 tiles: at GPT-2 small's attention (96 x 1024 x 64,
    // K = 1024) that is 768 workgroups of equal work, 3 per CU, and measured
    // 96 / 110 us (modes 2 / 3) against 130 / 125 us for paired 128 x 64
    // tiles (384 workgroups) and 142 / 131 us for unpaired ones, which take
    // as long as the full-K product: the CUs given the long-K row tiles set
    // the time.
    const int t = (g.N <= 64 && g.M >= 128 && tri != 2 && tri != 3) ? (transpose_A ? 10 : 9) : 1;
    // The K chunk depth sets which k pairs each MFMA adds, so mode 3 keeps the
    // 32-deep chunks of tile 10, which the untriangular product of that shape
    // runs on: the skipped chunks are exact zeros, and the sums stay equal bit
    // for bit to the plain masked computation's.
    if (tri == 3 && g.N <= 64 && g.M >= 128 && g.K > 128 && transpose_A)
      return launch_cfg<64, 64, 32, 32, 32, 2, true>(g, nb, transpose_A, transpose_B, 1);
    if (t == 1) return launch_cfg<64, 64, 16, 32, 32, 2, true>(g, nb, transpose_A, transpose_B, 1);
    if (t == 9) return launch_cfg<128, 64, 16, 64, 32, 2, true>(g, nb, transpose_A, transpose_B, 1);
    return launch_cfg<128, 64, 32, 64, 32, 1, true>(g, nb, transpose_A, transpose_B, 1);
  }
  switch (tile) {
    case 1: return launch_cfg<64, 64, 16, 32, 32>(g, nb, transpose_A, transpose_B, splits);
    case 2: return launch_cfg<128, 128, 16, 64, 64>(g, nb, transpose_A, transpose_B, splits);
    case 3: return launch_cfg<256, 128, 16, 128, 64>(g, nb, transpose_A, transpose_B, splits);
    // alternative shapes of the same kernel (K chunk 32, single LDS buffer)
    case 4: return launch_cfg<128, 128, 32, 64, 64, 1>(g, nb, transpose_A, transpose_B, splits);
    case 5: return launch_cfg<256, 128, 32, 128, 64, 1>(g, nb, transpose_A, transpose_B, splits);
    case 6: return launch_cfg<128, 128, 32, 64, 64, 2>(g, nb, transpose_A, transpose_B, splits);
    case 7: return launch_cfg<256, 128, 32, 128, 64, 2>(g, nb, transpose_A, transpose_B, splits);
    case 8: return launch_cfg<128, 256, 16, 64, 128>(g, nb, transpose_A, transpose_B, splits);
    case 9: return launch_cfg<128, 64, 16, 64, 32>(g, nb, transpose_A, transpose_B, splits);
    case 10: return launch_cfg<128, 64, 32, 64, 32, 1>(g, nb, transpose_A, transpose_B, splits);
    case 11:
      WXX_REQUIRE(dtl_ok, "tile 11 needs M, N multiples of 128, K a multiple of 32 and "
                  "16-byte aligned operands");
      return launch_cfg<128, 128, 32, 64, 64, 2, false, true>(g, nb, transpose_A, transpose_B,
                                                              splits);
    case 12:
      WXX_REQUIRE(dtl192_ok, "tile 12 needs M a multiple of 128, N of 192, K of 32 and "
                  "16-byte aligned operands");
      return launch_cfg<128, 192, 32, 64, 96, 2, false, true>(g, nb, transpose_A, transpose_B,
                                                              splits);
    case 13:
      WXX_REQUIRE(dtl64_ok, "tile 13 needs M a multiple of 128, N of 64, K of 32 and "
                  "16-byte aligned operands");
      return launch_cfg<128, 64, 32, 64, 32, 2, false, true>(g, nb, transpose_A, transpose_B,
                                                             splits);
    case 14:
      WXX_REQUIRE(dtl64_ok, "tile 14 needs M a multiple of 128, N of 64, K of 32 and "
                  "16-byte aligned operands");
      return launch_cfg<128, 64, 32, 64, 32, 3, false, true>(g, nb, transpose_A, transpose_B,
                                                             splits);
    case 15:
      WXX_REQUIRE(dtl6464_ok, "tile 15 needs M, N multiples of 64, K of 32 and 16-byte aligned "
                  "operands");
      return launch_cfg<64, 64, 32, 32, 32, 3, false, true>(g, nb, transpose_A, transpose_B,
                                                            splits);
    default: return wxx::set_error(WXX_E_ARG, "bad tile %d", tile);
  }
}
}  // namespace
