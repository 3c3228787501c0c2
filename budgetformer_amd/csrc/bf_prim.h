// Device-wide radix sort, scan, select and reduce over rocPRIM, the primitives
// the index and graph builders use between their own kernels.
//
// rocPRIM is called twice per operation: with temp == nullptr to size the
// temporary storage, then to run. It sizes the storage for the kernel
// configuration it picks from the template types, the count type included, so
// the query and the run must see the same types: every wrapper here takes the
// count as int64_t and passes it on converted the same way in both calls
// (32-bit for the sorts and select, whose callers check n < 2^31; size_t for
// the scans and the reduce, as rocPRIM declares them).
#pragma once

#include <cstdint>
#include <cstring>

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_reduce.hpp>
#include <rocprim/device/device_scan.hpp>
#include <rocprim/device/device_select.hpp>

namespace bf {
namespace prim {

// rocPRIM sorts up to 1M keys of more than 2 bytes by a block sort plus
// log2(n / block) merge passes, each a dependent launch over all keys. The
// sorts here cover only the few id bits they need (17-27 bits: three or four
// 8-bit digit passes), so past one block's worth the onesweep radix sort is
// the shorter route: on gfx950 a 0.82M-key sort of 18 bits takes 86 us as
// block sort + 10 merge passes and 63 us as onesweep (histogram + 3 digit
// passes). Merge sort is kept for sizes where its few passes are cheaper than
// onesweep's fixed launches. (The per-step reverse-index sort uses this
// build's own radix sort, bf_sort.h; these wrappers serve the once-per-graph
// COO -> CSR, coalesce and generator sorts.)
constexpr size_t kMergeSortLimit = size_t(1) << 16;
using radix_config = rocprim::radix_sort_config<rocprim::default_config, rocprim::default_config,
                                                rocprim::default_config, kMergeSortLimit>;

// Sorts keys by bits [begin_bit, end_bit) (stable).
template <typename K>
inline hipError_t sort_keys(void* temp, size_t& bytes, const K* in, K* out, int64_t n, int begin_bit, int end_bit,
                            hipStream_t st) {
  return rocprim::radix_sort_keys<radix_config>(temp, bytes, in, out, uint32_t(n), unsigned(begin_bit),
                                                unsigned(end_bit), st);
}

// Sorts (key, value) pairs by the keys' bits [begin_bit, end_bit) (stable).
template <typename K, typename V>
inline hipError_t sort_pairs(void* temp, size_t& bytes, const K* keys_in, K* keys_out, const V* vals_in, V* vals_out,
                             int64_t n, int begin_bit, int end_bit, hipStream_t st) {
  return rocprim::radix_sort_pairs<radix_config>(temp, bytes, keys_in, keys_out, vals_in, vals_out, uint32_t(n),
                                                 unsigned(begin_bit), unsigned(end_bit), st);
}

template <typename In, typename Out>
inline hipError_t inclusive_sum(void* temp, size_t& bytes, const In* in, Out* out, int64_t n, hipStream_t st) {
  return rocprim::inclusive_scan(temp, bytes, in, out, size_t(n), rocprim::plus<Out>(), st);
}

template <typename In, typename Out, typename Op>
inline hipError_t inclusive_scan(void* temp, size_t& bytes, const In* in, Out* out, Op op, int64_t n,
                                 hipStream_t st) {
  return rocprim::inclusive_scan(temp, bytes, in, out, size_t(n), op, st);
}

template <typename In, typename Out>
inline hipError_t exclusive_sum(void* temp, size_t& bytes, const In* in, Out* out, int64_t n, hipStream_t st) {
  return rocprim::exclusive_scan(temp, bytes, in, out, Out(0), size_t(n), rocprim::plus<Out>(), st);
}

// out[0, *count) = the in[i] whose flag is nonzero, in order.
template <typename T, typename F, typename C>
inline hipError_t select_flagged(void* temp, size_t& bytes, const T* in, const F* flags, T* out, C* count, int64_t n,
                                 hipStream_t st) {
  return rocprim::select(temp, bytes, in, flags, out, count, uint32_t(n), st);
}

// *out = sum of in[0, n).
template <typename T>
inline hipError_t reduce_sum(void* temp, size_t& bytes, const T* in, T* out, int64_t n, hipStream_t st) {
  return rocprim::reduce(temp, bytes, in, out, T(0), size_t(n), rocprim::plus<T>(), st);
}

}  // namespace prim
}  // namespace bf
