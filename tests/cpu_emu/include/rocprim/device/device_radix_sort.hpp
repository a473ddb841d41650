// CPU stand-in for rocprim::radix_sort_pairs (TEST INFRASTRUCTURE ONLY):
// a stable sort of (key, value) pairs by key, used by the ASan emulation.
#pragma once
#include <algorithm>
#include <cstddef>
#include <numeric>
#include <vector>
namespace rocprim {
template <typename K, typename V>
inline hipError_t radix_sort_pairs(void* tmp, size_t& bytes, const K* keys_in, K* keys_out,
                                   const V* vals_in, V* vals_out, size_t n, unsigned, unsigned,
                                   hipStream_t) {
  if (!tmp) { bytes = 16; return hipSuccess; }
  std::vector<size_t> order(n);
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) { return keys_in[a] < keys_in[b]; });
  std::vector<K> k(n);
  std::vector<V> v(n);
  for (size_t i = 0; i < n; ++i) { k[i] = keys_in[order[i]]; v[i] = vals_in[order[i]]; }
  std::copy(k.begin(), k.end(), keys_out);
  std::copy(v.begin(), v.end(), vals_out);
  return hipSuccess;
}
}  // namespace rocprim
