// Strided N-d addressing shared by the elementwise and complex kernels: the
// host collapses dimensions that are contiguous in every operand (and drops
// size-1 dimensions) so kernels loop over as few dimensions as possible.
#pragma once

#include "common.h"

namespace wxx {

constexpr int kMaxOps = 3;

struct ND {
  int rank;
  int64_t shape[wxx::kMaxRank];
  int64_t stride[kMaxOps][wxx::kMaxRank];
};

// Merge dimensions that are contiguous in every operand, drop size-1 dims.
inline ND collapse(int rank, const int64_t* shape, const int64_t* const* strides, int nops) {
  ND r;
  r.rank = 0;
  for (int d = 0; d < rank; ++d) {
    if (shape[d] == 1) continue;
    if (r.rank > 0) {
      const int p = r.rank - 1;
      bool merge = true;
      for (int o = 0; o < nops; ++o)
        if (r.stride[o][p] != strides[o][d] * shape[d]) merge = false;
      if (merge) {
        r.shape[p] *= shape[d];
        for (int o = 0; o < nops; ++o) r.stride[o][p] = strides[o][d];
        continue;
      }
    }
    r.shape[r.rank] = shape[d];
    for (int o = 0; o < nops; ++o) r.stride[o][r.rank] = strides[o][d];
    ++r.rank;
  }
  if (r.rank == 0) {
    r.rank = 1;
    r.shape[0] = 1;
    for (int o = 0; o < nops; ++o) r.stride[o][0] = 0;
  }
  return r;
}

template <int NOPS>
__device__ __forceinline__ void offsets(const ND& nd, int64_t idx, int64_t* off) {
#pragma unroll
  for (int o = 0; o < NOPS; ++o) off[o] = 0;
  if (nd.rank == 1) {
#pragma unroll
    for (int o = 0; o < NOPS; ++o) off[o] = idx * nd.stride[o][0];
    return;
  }
  // 32-bit decomposition when possible (AMD has no hardware 64-bit divide).
  uint32_t rem = (uint32_t)idx;
  for (int d = nd.rank - 1; d >= 0; --d) {
    const uint32_t n = (uint32_t)nd.shape[d];
    const uint32_t q = rem / n;
    const uint32_t c = rem - q * n;
    rem = q;
#pragma unroll
    for (int o = 0; o < NOPS; ++o) off[o] += (int64_t)c * nd.stride[o][d];
  }
}

template <int NOPS>
__device__ __forceinline__ void offsets64(const ND& nd, int64_t idx, int64_t* off) {
#pragma unroll
  for (int o = 0; o < NOPS; ++o) off[o] = 0;
  for (int d = nd.rank - 1; d >= 0; --d) {
    const int64_t n = nd.shape[d];
    const int64_t q = idx / n;
    const int64_t c = idx - q * n;
    idx = q;
#pragma unroll
    for (int o = 0; o < NOPS; ++o) off[o] += c * nd.stride[o][d];
  }
}

}  // namespace wxx
