// Embedding gather / scatter-add, dropout, and Hyena's decay window.
//
// Reference semantics:
//  * embed (src/wxx/shaders/layers/embed.wgsl:22-36, host
//    src/wxx/functional/layers.py:161-206): out[t, d] = W[id[t], d].
//  * embeddx (embeddx.wgsl:22-47, layers.py:209-254): grad[v, d] =
//    sum over tokens t with id[t] == v of g[t, d]; ids >= vocab are skipped.
//    The reference adds with a float compare-and-swap loop, so its order of
//    addition (and result) varies from run to run.
//  * dropout / dropoutdx (dropout.wgsl:14-36, dropoutdx.wgsl): with
//    h(x) = ((x>>16)^x)*0x45d9f3b twice then (x>>16)^x, element i is kept when
//    f32(h(i ^ seed) >> 8) * 2^-24 >= p, and kept values are scaled by
//    1/(1-p).  Reproduced bit-exactly.
//  * decay_window (decay_window.wgsl:22-33): W[d, t] = exp(-|r_d| t);
//    backward (decay_window_backward.wgsl:24-46): dr_d = sum_t g[d,t] W[d,t]
//    (-sign(r_d) t), written into the `stage` row of a zeroed (rows, channels).
//
// MI355X design: the embedding backward is deterministic and made of plain
// kernels only (so it can be recorded into a step graph: no library sort, no
// memset nodes).  Ids are histogrammed, the histogram is scanned into per-row
// segment offsets, each segment is filled with its tokens in token order by
// one thread per vocabulary row, and each vocabulary row is produced by one
// pass that adds its tokens' gradient rows in token order and writes zeros
// for unused rows (no separate zero-fill launch).
#include "common.h"

#include <cstring>

namespace {

constexpr int kBlock = 256;

// ---- embedding -------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void embed_kernel(const uint32_t* __restrict__ ids,
                                                       const float* __restrict__ W,
                                                       float* __restrict__ out, int64_t ntok,
                                                       int64_t D, int64_t V, int vec) {
  // one thread per 4 (vec) or 1 output element(s), grid-stride
  const int64_t per = vec ? D / 4 : D;
  const int64_t total = ntok * per;
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < total; i += step) {
    const int64_t t = i / per, d = i - t * per;
    const uint32_t id = ids[t];
    if (vec) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (id < (uint64_t)V) v = reinterpret_cast<const float4*>(W + (int64_t)id * D)[d];
      reinterpret_cast<float4*>(out + t * D)[d] = v;
    } else {
      out[t * D + d] = id < (uint64_t)V ? W[(int64_t)id * D + d] : 0.f;
    }
  }
}

// counts[v] = number of tokens with id v (ids >= V are not counted).  The
// atomics only count, so the result does not depend on their order.
__global__ __launch_bounds__(kBlock) void embed_hist_kernel(const uint32_t* __restrict__ ids,
                                                            uint32_t* __restrict__ counts,
                                                            int64_t ntok, int64_t V) {
  int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; t < ntok; t += step) {
    const uint32_t id = ids[t];
    if (id < (uint64_t)V) atomicAdd(&counts[id], 1u);
  }
}

// out = exclusive prefix sum of in[0, n), by one workgroup: each thread sums a
// contiguous run, the run totals are scanned in LDS, then each run is written.
constexpr int kScanBlock = 1024;
__global__ __launch_bounds__(kScanBlock) void exclusive_scan_u32_kernel(
    const uint32_t* __restrict__ in, uint32_t* __restrict__ out, int64_t n) {
  __shared__ uint32_t part[kScanBlock];
  const int tid = threadIdx.x;
  const int64_t per = (n + kScanBlock - 1) / kScanBlock;
  const int64_t lo = min((int64_t)tid * per, n), hi = min(lo + per, n);
  uint32_t run = 0;
  for (int64_t i = lo; i < hi; ++i) run += in[i];
  part[tid] = run;
  __syncthreads();
  for (int off = 1; off < kScanBlock; off <<= 1) {
    const uint32_t add = tid >= off ? part[tid - off] : 0u;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  run = tid ? part[tid - 1] : 0u;
  for (int64_t i = lo; i < hi; ++i) {
    const uint32_t c = in[i];
    out[i] = run;
    run += c;
  }
}

// sorted_tok[offsets[v] ...] = the tokens whose id is v, in token order: one
// thread per id walks the ids (staged through LDS, read by every lane at the
// same address) and appends each match, so each segment is stable without a
// sort.  Work is V x ntok compares, V / 64 waves each reading ntok ids.
constexpr int kPlaceChunk = 4096;
__global__ __launch_bounds__(kBlock) void embed_place_kernel(const uint32_t* __restrict__ ids,
                                                             const uint32_t* __restrict__ offsets,
                                                             uint32_t* __restrict__ sorted_tok,
                                                             int64_t ntok, int64_t V) {
  __shared__ uint32_t sid[kPlaceChunk];
  const int64_t v = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  uint32_t pos = v < V ? offsets[v] : 0u;
  for (int64_t base = 0; base < ntok; base += kPlaceChunk) {
    const int len = (int)min((int64_t)kPlaceChunk, ntok - base);
    __syncthreads();
    for (int i = threadIdx.x; i < len; i += kBlock) sid[i] = ids[base + i];
    __syncthreads();
    if (v < V) {
      for (int i = 0; i < len; ++i)
        if (sid[i] == (uint32_t)v) sorted_tok[pos++] = (uint32_t)(base + i);
    }
  }
}

// The same placement with the token list cut into nseg segments of seglen
// tokens, so that V x nseg threads share the V x ntok compares: count each
// (segment, id), turn the counts into each segment's write offset per id
// (an exclusive scan over segments from offsets[v]), then place each
// segment's tokens in token order.  The result equals embed_place_kernel's.
__global__ __launch_bounds__(kBlock) void embed_seg_count_kernel(const uint32_t* __restrict__ ids,
                                                                 uint32_t* __restrict__ cnt,
                                                                 int64_t ntok, int64_t V,
                                                                 int seglen) {
  __shared__ uint32_t sid[kPlaceChunk];
  const int64_t v = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t base = (int64_t)blockIdx.y * seglen;
  const int len = (int)min((int64_t)seglen, ntok - base);
  for (int i = threadIdx.x; i < len; i += kBlock) sid[i] = ids[base + i];
  __syncthreads();
  if (v >= V) return;
  uint32_t c = 0;
  for (int i = 0; i < len; ++i) c += sid[i] == (uint32_t)v;
  cnt[(int64_t)blockIdx.y * V + v] = c;
}

__global__ __launch_bounds__(kBlock) void embed_seg_base_kernel(const uint32_t* __restrict__ offsets,
                                                                uint32_t* __restrict__ cnt,
                                                                int64_t V, int nseg) {
  const int64_t v = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (v >= V) return;
  uint32_t acc = offsets[v];
  // eight segments' counts loaded before any is overwritten (one round trip
  // per eight instead of per segment)
  constexpr int kU = 8;
  for (int sg0 = 0; sg0 < nseg; sg0 += kU) {
    uint32_t c[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) c[u] = sg0 + u < nseg ? cnt[(int64_t)(sg0 + u) * V + v] : 0u;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (sg0 + u < nseg) cnt[(int64_t)(sg0 + u) * V + v] = acc;
      acc += c[u];
    }
  }
}

__global__ __launch_bounds__(kBlock) void embed_seg_place_kernel(const uint32_t* __restrict__ ids,
                                                                 const uint32_t* __restrict__ segbase,
                                                                 uint32_t* __restrict__ sorted_tok,
                                                                 int64_t ntok, int64_t V, int seglen) {
  __shared__ uint32_t sid[kPlaceChunk];
  const int64_t v = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t base = (int64_t)blockIdx.y * seglen;
  const int len = (int)min((int64_t)seglen, ntok - base);
  for (int i = threadIdx.x; i < len; i += kBlock) sid[i] = ids[base + i];
  __syncthreads();
  if (v >= V) return;
  uint32_t pos = segbase[(int64_t)blockIdx.y * V + v];
  for (int i = 0; i < len; ++i)
    if (sid[i] == (uint32_t)v) sorted_tok[pos++] = (uint32_t)(base + i);
}

// grad[v, :] = sum over the v-segment of the sorted token list, in token order.
__global__ __launch_bounds__(kBlock) void embed_segsum_kernel(
    const float* __restrict__ g, const uint32_t* __restrict__ sorted_tok,
    const uint32_t* __restrict__ offsets, const uint32_t* __restrict__ counts,
    float* __restrict__ grad, int64_t D, int64_t V, int vec) {
  const int64_t v = blockIdx.x;
  if (v >= V) return;
  const uint32_t start = offsets[v], n = counts[v];
  if (vec) {
    const int64_t D4 = D / 4;
    for (int64_t d = (int64_t)blockIdx.y * kBlock + threadIdx.x; d < D4;
         d += (int64_t)gridDim.y * kBlock) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      for (uint32_t k = 0; k < n; ++k) {
        const float4 x = reinterpret_cast<const float4*>(g + (int64_t)sorted_tok[start + k] * D)[d];
        acc.x += x.x;
        acc.y += x.y;
        acc.z += x.z;
        acc.w += x.w;
      }
      reinterpret_cast<float4*>(grad + v * D)[d] = acc;
    }
  } else {
    for (int64_t d = (int64_t)blockIdx.y * kBlock + threadIdx.x; d < D;
         d += (int64_t)gridDim.y * kBlock) {
      float acc = 0.f;
      for (uint32_t k = 0; k < n; ++k) acc += g[(int64_t)sorted_tok[start + k] * D + d];
      grad[v * D + d] = acc;
    }
  }
}

// ---- dropout -----------------------------------------------------------------

// `seed_dev`, when set, holds the seed on the device (a step graph's replays
// write a fresh one before each launch) and replaces `seed`.
__global__ __launch_bounds__(kBlock) void dropout_kernel(const float* __restrict__ x,
                                                         float* __restrict__ y, int64_t n,
                                                         uint32_t seed, float p, float scale,
                                                         const uint32_t* __restrict__ seed_dev) {
  if (seed_dev) seed = *seed_dev;
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += step) {
    y[i] = wxx::dropout_keep((uint32_t)i, seed, p) ? x[i] * scale : 0.f;
  }
}

// ---- Hyena decay window ------------------------------------------------------
__global__ __launch_bounds__(kBlock) void decay_window_kernel(const float* __restrict__ decay,
                                                              float* __restrict__ w,
                                                              int64_t channels, int64_t length,
                                                              int64_t stage) {
  const int64_t total = channels * length;
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * kBlock;
  for (; i < total; i += step) {
    const int64_t d = i / length, t = i - d * length;
    const float r = decay[stage * channels + d];
    w[i] = expf(-fabsf(r) * (float)t);
  }
}

// One workgroup per channel: reduce over t (the reference loops serially).
__global__ __launch_bounds__(kBlock) void decay_window_bwd_kernel(const float* __restrict__ g,
                                                                  const float* __restrict__ decay,
                                                                  float* __restrict__ out,
                                                                  int64_t rows, int64_t channels,
                                                                  int64_t length, int64_t stage) {
  __shared__ float red[4];
  const int64_t d = blockIdx.x;
  const float r = decay[stage * channels + d];
  const float sgn = r > 0.f ? 1.f : (r < 0.f ? -1.f : 0.f);
  float acc = 0.f;
  for (int64_t t = threadIdx.x; t < length; t += kBlock) {
    const float w = expf(-fabsf(r) * (float)t);
    acc += g[d * length + t] * w * (-sgn * (float)t);
  }
  acc = wxx::block_sum(acc, red);
  if (threadIdx.x == 0) {
    for (int64_t row = 0; row < rows; ++row) out[row * channels + d] = row == stage ? acc : 0.f;
  }
}

}  // namespace

// Replaces functional.embed (reference src/wxx/functional/layers.py:161-206).
// Ids >= V produce zero rows (the reference leaves that read unchecked).
WXX_API int wxx_embed(const uint32_t* ids, const float* W, float* out, int64_t ntok, int64_t D,
                      int64_t V) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(ids && W && out, "null pointer");
  if (ntok <= 0 || D <= 0) return WXX_OK;
  const int vec = (D % 4 == 0) && ((((uintptr_t)W) | ((uintptr_t)out)) % 16 == 0);
  const int64_t work = ntok * (vec ? D / 4 : D);
  hipLaunchKernelGGL(embed_kernel, dim3(wxx::grid_1d(work, kBlock, 16384)), dim3(kBlock), 0,
                     wxx::stream(), ids, W, out, ntok, D, V, vec);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.embeddx (reference src/wxx/functional/layers.py:209-254),
// deterministic: each row sums its tokens' gradients in token order.
WXX_API int wxx_embeddx(const float* g, const uint32_t* ids, float* grad, int64_t ntok,
                        int64_t D, int64_t V) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(g && ids && grad, "null pointer");
  WXX_REQUIRE(ntok < (int64_t(1) << 31) && V < (int64_t(1) << 31), "too many tokens / rows");
  if (V <= 0 || D <= 0) return WXX_OK;
  if (ntok <= 0) return wxx_fill_u32(grad, V * D, 0u);
  hipStream_t s = wxx::stream();
  const size_t n = (size_t)ntok;
  uint32_t* buf = (uint32_t*)wxx::scratch_alloc(sizeof(uint32_t) * (n + 2 * (size_t)V));
  if (!buf) return wxx::set_error(WXX_E_OOM, "embeddx scratch");
  uint32_t* sorted_tok = buf;
  uint32_t* counts = sorted_tok + n;
  uint32_t* offsets = counts + V;
  int rc = wxx_fill_u32(counts, V, 0u);
  if (rc) {
    wxx::scratch_free(buf);
    return rc;
  }
  hipLaunchKernelGGL(embed_hist_kernel, dim3(wxx::grid_1d(ntok, kBlock, 16384)), dim3(kBlock), 0,
                     s, ids, counts, ntok, V);
  hipLaunchKernelGGL(exclusive_scan_u32_kernel, dim3(1), dim3(kScanBlock), 0, s, counts, offsets,
                     V);
  // Segments: enough (segment, id) threads to fill the chip (~64k), each
  // segment at most kPlaceChunk tokens (one LDS stage) and, below that, at
  // least 256 tokens (GPT-2 config 1's 512 tokens: 2 segments, not 64 / 512
  // whose serial bases cost 16-29 us).
  int64_t nseg = std::max<int64_t>((ntok + kPlaceChunk - 1) / kPlaceChunk, (65536 + V - 1) / V);
  nseg = std::min<int64_t>(nseg, std::max<int64_t>((ntok + kPlaceChunk - 1) / kPlaceChunk,
                                                   ntok / 256));
  nseg = std::min<int64_t>(std::min<int64_t>(nseg, ntok), 65535);
  const int seglen = (int)((ntok + nseg - 1) / nseg);
  nseg = (ntok + seglen - 1) / seglen;
  uint32_t* segcnt = nullptr;
  if (nseg > 1) segcnt = (uint32_t*)wxx::scratch_alloc(sizeof(uint32_t) * (size_t)(nseg * V));
  const dim3 vblocks((unsigned)((V + kBlock - 1) / kBlock));
  if (segcnt) {
    const dim3 grid2(vblocks.x, (unsigned)nseg);
    hipLaunchKernelGGL(embed_seg_count_kernel, grid2, dim3(kBlock), 0, s, ids, segcnt, ntok, V,
                       seglen);
    hipLaunchKernelGGL(embed_seg_base_kernel, vblocks, dim3(kBlock), 0, s, offsets, segcnt, V,
                       (int)nseg);
    hipLaunchKernelGGL(embed_seg_place_kernel, grid2, dim3(kBlock), 0, s, ids, segcnt, sorted_tok,
                       ntok, V, seglen);
  } else {
    hipLaunchKernelGGL(embed_place_kernel, vblocks, dim3(kBlock), 0, s, ids, offsets, sorted_tok,
                       ntok, V);
  }
  WXX_LAUNCHED();
  const int vec = (D % 4 == 0) && ((((uintptr_t)g) | ((uintptr_t)grad)) % 16 == 0);
  const int64_t dwork = vec ? D / 4 : D;
  const unsigned gy = (unsigned)std::min<int64_t>((dwork + kBlock - 1) / kBlock, 65535);
  hipLaunchKernelGGL(embed_segsum_kernel, dim3((unsigned)V, gy), dim3(kBlock), 0, s, g,
                     sorted_tok, offsets, counts, grad, D, V, vec);
  WXX_LAUNCHED();
  if (segcnt) wxx::scratch_free(segcnt);
  wxx::scratch_free(buf);
  return WXX_OK;
}

// Replaces functional.dropout / dropoutdx (reference layers.py:73-158): the
// same kernel serves both (dropoutdx applies the mask to the gradient).
WXX_API int wxx_dropout(const float* x, float* y, int64_t n, uint32_t seed, float p,
                        float scale) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && y, "null pointer");
  if (n <= 0) return WXX_OK;
  hipLaunchKernelGGL(dropout_kernel, dim3(wxx::grid_1d(n, kBlock, 16384)), dim3(kBlock), 0,
                     wxx::stream(), x, y, n, seed, p, scale, (const uint32_t*)nullptr);
  WXX_LAUNCHED();
  return WXX_OK;
}

// wxx_dropout with the seed read on the device from `seed` when the kernel
// runs (for recorded step graphs; no reference counterpart).
WXX_API int wxx_dropout_dev(const float* x, float* y, int64_t n, const uint32_t* seed, float p,
                            float scale) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(x && y && seed, "null pointer");
  if (n <= 0) return WXX_OK;
  hipLaunchKernelGGL(dropout_kernel, dim3(wxx::grid_1d(n, kBlock, 16384)), dim3(kBlock), 0,
                     wxx::stream(), x, y, n, 0u, p, scale, seed);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.decay_window (reference src/wxx/functional/pointwise.py:357-404).
WXX_API int wxx_decay_window(const float* decay, float* w, int64_t rows, int64_t channels,
                             int64_t length, int64_t stage) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(decay && w, "null pointer");
  WXX_REQUIRE(stage >= 0 && stage < rows, "stage out of range");
  if (channels * length <= 0) return WXX_OK;
  hipLaunchKernelGGL(decay_window_kernel, dim3(wxx::grid_1d(channels * length, kBlock, 16384)),
                     dim3(kBlock), 0, wxx::stream(), decay, w, channels, length, stage);
  WXX_LAUNCHED();
  return WXX_OK;
}

// Replaces functional.decay_window_backward (reference pointwise.py:407-457).
WXX_API int wxx_decay_window_backward(const float* g, const float* decay, float* out,
                                      int64_t rows, int64_t channels, int64_t length,
                                      int64_t stage) {
  WXX_CHECK_INIT();
  WXX_REQUIRE(g && decay && out, "null pointer");
  WXX_REQUIRE(stage >= 0 && stage < rows, "stage out of range");
  if (channels <= 0) return WXX_OK;
  WXX_REQUIRE(channels <= 0x7fffffff, "too many channels");
  hipLaunchKernelGGL(decay_window_bwd_kernel, dim3((unsigned)channels), dim3(kBlock), 0,
                     wxx::stream(), g, decay, out, rows, channels, length, stage);
  WXX_LAUNCHED();
  return WXX_OK;
}
