// CPU stand-in for rocprim::exclusive_scan (TEST INFRASTRUCTURE ONLY).
#pragma once
#include <cstddef>
namespace rocprim {
template <typename T>
struct plus { T operator()(const T& a, const T& b) const { return a + b; } };
template <typename In, typename Out, typename T, typename Op>
inline hipError_t exclusive_scan(void* tmp, size_t& bytes, In in, Out out, T init, size_t n,
                                 Op op, hipStream_t) {
  if (!tmp) { bytes = 16; return hipSuccess; }
  T acc = init;
  for (size_t i = 0; i < n; ++i) { T x = in[i]; out[i] = acc; acc = op(acc, x); }
  return hipSuccess;
}
}  // namespace rocprim
