// Register-resident row helpers for row-wise kernels (softmax, LayerNorm,
// RMSNorm, cross-entropy).  A row of C floats is spread over TPR lanes
// (64 = one wavefront per row, 256 = one workgroup per row) in NCH chunks,
// loaded once from HBM with float4 accesses when the row length allows, and
// kept in VGPRs until the output is written: each row costs exactly one HBM
// read and one HBM write.
#pragma once
#include "common.h"
#include <type_traits>

namespace wxx {

template <int TPR>
struct RowReduce {
  // `red` is LDS scratch of at least TPR / 64 floats (TPR >= 256 only).
  __device__ static float sum(float v, float* red) {
    if (TPR == 64) return warp_sum(v);
    return block_sum(v, red);
  }
  __device__ static float max(float v, float* red) {
    if (TPR == 64) return warp_max(v);
    return block_max(v, red);
  }
};

// Element e (0 <= e < NCH*4) held by lane t maps to a column index:
//  VEC:  ((e / 4) * TPR + t) * 4 + e % 4   (float4 per chunk, coalesced)
//  !VEC: ((e / 4) * 4 + e % 4) * TPR + t   (scalar, coalesced)
template <int TPR, int NCH, bool VEC>
struct RowRegs {
  float v[NCH * 4];

  __device__ __forceinline__ static int col(int e, int t) {
    return VEC ? (((e >> 2) * TPR + t) << 2) + (e & 3) : e * TPR + t;
  }

  __device__ __forceinline__ void load(const float* __restrict__ row, int C, int t, float pad) {
    if (VEC) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int base = (c * TPR + t) * 4;
        if (base < C) {
          float4 q = *reinterpret_cast<const float4*>(row + base);
          v[c * 4 + 0] = q.x;
          v[c * 4 + 1] = q.y;
          v[c * 4 + 2] = q.z;
          v[c * 4 + 3] = q.w;
        } else {
          v[c * 4 + 0] = v[c * 4 + 1] = v[c * 4 + 2] = v[c * 4 + 3] = pad;
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < NCH * 4; ++e) {
        const int j = e * TPR + t;
        v[e] = j < C ? row[j] : pad;
      }
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ row, int C, int t) const {
    if (VEC) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int base = (c * TPR + t) * 4;
        if (base < C) {
          float4 q = make_float4(v[c * 4 + 0], v[c * 4 + 1], v[c * 4 + 2], v[c * 4 + 3]);
          *reinterpret_cast<float4*>(row + base) = q;
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < NCH * 4; ++e) {
        const int j = e * TPR + t;
        if (j < C) row[j] = v[e];
      }
    }
  }

  __device__ __forceinline__ bool valid(int e, int t, int C) const { return col(e, t) < C; }

  // The first lim columns of the row (lim <= C), pad beyond: the lower
  // triangle of a causal attention row.
  __device__ __forceinline__ void load_lim(const float* __restrict__ row, int lim, int t,
                                           float pad) {
    if (VEC) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int base = (c * TPR + t) * 4;
        if (base + 4 <= lim) {
          float4 q = *reinterpret_cast<const float4*>(row + base);
          v[c * 4 + 0] = q.x;
          v[c * 4 + 1] = q.y;
          v[c * 4 + 2] = q.z;
          v[c * 4 + 3] = q.w;
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) v[c * 4 + k] = base + k < lim ? row[base + k] : pad;
        }
      }
    } else {
      load(row, lim, t, pad);
    }
  }

  // Stores the first lim columns only.
  __device__ __forceinline__ void store_lim(float* __restrict__ row, int lim, int t) const {
    if (VEC) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int base = (c * TPR + t) * 4;
        if (base + 4 <= lim) {
          *reinterpret_cast<float4*>(row + base) =
              make_float4(v[c * 4 + 0], v[c * 4 + 1], v[c * 4 + 2], v[c * 4 + 3]);
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if (base + k < lim) row[base + k] = v[c * 4 + k];
        }
      }
    } else {
      store(row, lim, t);
    }
  }
};

// Pick (TPR, NCH) for a row length: one wave per row up to 2048 columns,
// one 256-lane workgroup per row up to 16384 columns, otherwise 0 (looped
// kernel).  Returned as TPR * 100 + NCH.
inline int row_plan(int64_t C) {
  if (C <= 64 * 4 * 1) return 64 * 100 + 1;
  if (C <= 64 * 4 * 2) return 64 * 100 + 2;
  if (C <= 64 * 4 * 4) return 64 * 100 + 4;
  if (C <= 64 * 4 * 8) return 64 * 100 + 8;
  if (C <= 256 * 4 * 4) return 256 * 100 + 4;
  if (C <= 256 * 4 * 8) return 256 * 100 + 8;
  if (C <= 256 * 4 * 16) return 256 * 100 + 16;
  return 0;
}

}  // namespace wxx

namespace wxx {

template <int V>
using ic = std::integral_constant<int, V>;

// Call f(ic<TPR>, ic<NCH>, std::bool_constant<VEC>) for the plan of C.
// Rows per 256-thread block = 256 / TPR.  Returns f's status.
template <typename F>
int row_dispatch(int64_t C, bool vec, F&& f) {
  const int plan = row_plan(C);
#define WXX_RD_CASE(TPR, NCH)                                                  \
  case TPR * 100 + NCH:                                                        \
    return vec ? f(ic<TPR>{}, ic<NCH>{}, std::true_type{})                     \
               : f(ic<TPR>{}, ic<NCH>{}, std::false_type{});
  switch (plan) {
    WXX_RD_CASE(64, 1)
    WXX_RD_CASE(64, 2)
    WXX_RD_CASE(64, 4)
    WXX_RD_CASE(64, 8)
    WXX_RD_CASE(256, 4)
    WXX_RD_CASE(256, 8)
    WXX_RD_CASE(256, 16)
    default:
      return set_error(WXX_E_UNSUPPORTED, "no row plan for length %lld", (long long)C);
  }
#undef WXX_RD_CASE
}

// Wide-row plan for kernels that can use 1024-lane workgroups (up to 65536
// columns in registers): TPR * 100 + NCH, or 0 for the looped kernel.
inline int wide_row_plan(int64_t C) {
  const int p = row_plan(C);
  if (p) return p;
  if (C <= 1024 * 4 * 8) return 1024 * 100 + 8;
  if (C <= 1024 * 4 * 16) return 1024 * 100 + 16;
  return 0;
}

template <typename F>
int wide_row_dispatch(int64_t C, bool vec, F&& f) {
  const int plan = wide_row_plan(C);
  if (plan / 100 != 1024) return row_dispatch(C, vec, f);
  if (plan % 100 == 8)
    return vec ? f(ic<1024>{}, ic<8>{}, std::true_type{}) : f(ic<1024>{}, ic<8>{}, std::false_type{});
  return vec ? f(ic<1024>{}, ic<16>{}, std::true_type{}) : f(ic<1024>{}, ic<16>{}, std::false_type{});
}

inline dim3 row_grid(int tpr, int64_t rows) {
  const int64_t rpb = tpr >= 256 ? 1 : 256 / tpr;
  return dim3((unsigned)((rows + rpb - 1) / rpb));
}

}  // namespace wxx
