// Synthetic power-law (Chung-Lu) graphs generated on the device, so benchmark
// shapes up to 1.6B edges never pass through host memory.
//
// Expected degree of node i is proportional to (i + i0)^(-1/(exponent-1)),
// rescaled to sum to 2*pairs and capped at max_degree. Endpoints are drawn by
// inverse-CDF binary search over the prefix sums of the weights (Philox4x32-10
// keyed by the seed, counter = draw index), self pairs dropped, unordered pairs
// deduplicated by radix sort, trimmed to exactly `pairs` by a hash order, then
// symmetrised into a coalesced CSR (int64 rowptr, int32 col).
//
// The weights' sum and prefix sums are taken in 64-bit fixed point: integer
// sums do not depend on the order a parallel scan adds them in (a
// floating-point look-back scan rounds differently from run to run), so a
// seed always gives the same graph.
#include "bf_common.h"
#include "bf_prim.h"

namespace bf {
namespace {

constexpr int kThreads = 256;
constexpr uint64_t kNone = ~uint64_t(0);

inline unsigned blocks_for(int64_t n) { return unsigned(ceil_div(n, kThreads)); }
inline size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

int bits_for(uint64_t maxval) {
  int b = 1;
  while (b < 64 && (uint64_t(1) << b) <= maxval) ++b;
  return b;
}

// Fixed-point scales: raw weights (each at most i0^(-1/(exponent-1)) <= 1) in units of 2^-36, so that the
// sum of up to 2^31 of them stays below 2^63; scaled weights (expected degrees, summing to 2*pairs < 2^31)
// in units of 2^-24.
constexpr double kRawScale = 68719476736.0;     // 2^36
constexpr double kCdfScale = 16777216.0;        // 2^24

__global__ void weights_kernel(int64_t n, double i0, double expo, uint64_t* __restrict__ w) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n) w[i] = uint64_t(llrint(pow(double(i) + i0, -1.0 / (expo - 1.0)) * kRawScale));
}

__global__ void scale_cap_kernel(int64_t n, const uint64_t* __restrict__ raw_sum, double target, double cap,
                                 uint64_t* __restrict__ w) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  double x = double(w[i]) * (target / double(*raw_sum));
  if (cap > 0.0 && x > cap) x = cap;
  w[i] = uint64_t(llrint(x * kCdfScale));
}

__device__ __forceinline__ int64_t inverse_cdf(const uint64_t* __restrict__ cdf, int64_t n, uint64_t x) {
  int64_t lo = 0, hi = n - 1;  // first i with cdf[i] > x
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (cdf[mid] > x) hi = mid; else lo = mid + 1;
  }
  return lo;
}

__device__ __forceinline__ double u53(uint32_t a, uint32_t b) {
  return (double(a >> 5) * 67108864.0 + double(b >> 6)) * (1.0 / 9007199254740992.0);
}

__global__ void draw_pairs_kernel(const uint64_t* __restrict__ cdf, int64_t n, int64_t draws, uint64_t seed,
                                  uint64_t counter_base, uint64_t* __restrict__ keys) {
  const int64_t j = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (j >= draws) return;
  const uint64_t c = counter_base + uint64_t(j);
  const U32x4 r = philox4x32_10(U32x4{uint32_t(c), uint32_t(c >> 32), 0x5eed5eedu, 0u}, uint32_t(seed),
                                uint32_t(seed >> 32));
  const double total = double(cdf[n - 1]);
  // u in [0, 1): the point lies below the total (u * total rounds to at most total - 1 below 2^53)
  const int64_t a = inverse_cdf(cdf, n, uint64_t(u53(r.x, r.y) * total));
  const int64_t b = inverse_cdf(cdf, n, uint64_t(u53(r.z, r.w) * total));
  if (a == b) {
    keys[j] = kNone;
    return;
  }
  const uint64_t lo = uint64_t(a < b ? a : b), hi = uint64_t(a < b ? b : a);
  keys[j] = lo * uint64_t(n) + hi;
}

__global__ void unique_flag_kernel(const uint64_t* __restrict__ keys, int64_t m, int32_t* __restrict__ flags) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i < m) flags[i] = (keys[i] != kNone && (i == 0 || keys[i] != keys[i - 1])) ? 1 : 0;
}

__global__ void hash_keys_kernel(const uint64_t* __restrict__ keys, int64_t m, uint64_t seed,
                                 uint64_t* __restrict__ h) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= m) return;
  const uint64_t k = keys[i];
  const U32x4 r = philox4x32_10(U32x4{uint32_t(k), uint32_t(k >> 32), 0x7a11u, 0u}, uint32_t(seed ^ 0x9e37u),
                                uint32_t(seed >> 32));
  h[i] = (uint64_t(r.x) << 32) | r.y;
}

__global__ void symmetrize_kernel(const uint64_t* __restrict__ pairs, int64_t m, uint64_t n,
                                  uint64_t* __restrict__ dir) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= m) return;
  const uint64_t lo = pairs[i] / n, hi = pairs[i] % n;
  dir[2 * i] = lo * n + hi;
  dir[2 * i + 1] = hi * n + lo;
}

__global__ void csr_col_kernel(const uint64_t* __restrict__ keys, int64_t m, uint64_t n, int32_t* __restrict__ col) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i < m) col[i] = int32_t(keys[i] % n);
}

__global__ void csr_rowptr_kernel(const uint64_t* __restrict__ keys, int64_t m, uint64_t n,
                                  int64_t* __restrict__ rowptr) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i > m) return;
  const int64_t r_here = i < m ? int64_t(keys[i] / n) : int64_t(n);
  const int64_t r_prev = i > 0 ? int64_t(keys[i - 1] / n) : -1;
  fill_gap(r_prev, r_here, i, [&](int64_t r, int64_t v) { rowptr[r] = v; });
}

}  // namespace
}  // namespace bf

using namespace bf;

// Scratch: 4 uint64 slabs of `draws` keys + cdf (N doubles) + sort/scan temp.
extern "C" int bf_chung_lu_workspace_size(int64_t num_nodes, int64_t pairs, size_t* bytes) {
  BF_CHECK_ARG(bytes && num_nodes > 1 && pairs > 0, "chung_lu_workspace_size: bad arguments");
  const int64_t draws = pairs + pairs / 4 + 1024;
  const int64_t slab_n = 2 * pairs > draws ? 2 * pairs : draws;
  size_t sort_bytes = 0, sort2_bytes = 0, scan_bytes = 0, red_bytes = 0, sel_bytes = 0;
  const hipStream_t none = nullptr;
  (void)prim::select_flagged(nullptr, sel_bytes, static_cast<const uint64_t*>(nullptr),
                             static_cast<const int32_t*>(nullptr), static_cast<uint64_t*>(nullptr),
                             static_cast<int*>(nullptr), draws, none);
  (void)prim::sort_keys(nullptr, sort_bytes, static_cast<const uint64_t*>(nullptr), static_cast<uint64_t*>(nullptr),
                        slab_n, 0, 64, none);
  (void)prim::sort_pairs(nullptr, sort2_bytes, static_cast<const uint64_t*>(nullptr), static_cast<uint64_t*>(nullptr),
                         static_cast<const uint64_t*>(nullptr), static_cast<uint64_t*>(nullptr), draws, 0, 64, none);
  (void)prim::inclusive_sum(nullptr, scan_bytes, static_cast<const uint64_t*>(nullptr),
                            static_cast<uint64_t*>(nullptr), num_nodes, none);
  (void)prim::reduce_sum(nullptr, red_bytes, static_cast<const uint64_t*>(nullptr), static_cast<uint64_t*>(nullptr),
                         num_nodes, none);
  size_t temp = sort_bytes;
  for (size_t t : {sort2_bytes, scan_bytes, red_bytes, sel_bytes}) temp = t > temp ? t : temp;
  *bytes = 4 * align_up(size_t(slab_n) * 8) + 2 * align_up(size_t(num_nodes) * 8) + align_up(size_t(draws) * 4) +
           align_up(temp) + 1024;
  return BF_OK;
}

extern "C" int bf_chung_lu(int64_t num_nodes, int64_t pairs, double exponent, double i0, double max_degree,
                           uint64_t seed, int64_t* rowptr, int32_t* col, int64_t* num_edges_host, void* workspace,
                           size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(num_nodes > 1 && num_nodes < (int64_t(1) << 31) && pairs > 0, "chung_lu: bad sizes");
  BF_CHECK_ARG(exponent > 1.0 && i0 > 0.0, "chung_lu: exponent must be > 1 and i0 > 0");
  BF_CHECK_ARG(rowptr && col && num_edges_host, "chung_lu: null output");
  BF_CHECK_ARG(2 * pairs < (int64_t(1) << 31), "chung_lu: 2*pairs must fit int32 item counts");
  BF_CHECK_ARG(uint64_t(pairs) <= uint64_t(num_nodes) * uint64_t(num_nodes - 1) / 2, "chung_lu: too many pairs");
  // the raw weights' fixed-point sum (2^-36 units) stays below 2^63: num_nodes times node 0's weight < 2^27
  BF_CHECK_ARG(double(num_nodes) * pow(i0, -1.0 / (exponent - 1.0)) < 134217728.0,
               "chung_lu: weights too large for the fixed-point sum (raise i0 or the exponent)");
  size_t need = 0;
  bf_chung_lu_workspace_size(num_nodes, pairs, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "chung_lu: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  const int64_t draws = pairs + pairs / 4 + 1024;
  const int64_t slab_n = 2 * pairs > draws ? 2 * pairs : draws;
  char* p = static_cast<char*>(workspace);
  auto take = [&](size_t b) { char* q = p; p += align_up(b); return q; };
  auto* keys_a = reinterpret_cast<uint64_t*>(take(size_t(slab_n) * 8));
  auto* keys_b = reinterpret_cast<uint64_t*>(take(size_t(slab_n) * 8));
  auto* keys_c = reinterpret_cast<uint64_t*>(take(size_t(slab_n) * 8));
  auto* keys_d = reinterpret_cast<uint64_t*>(take(size_t(slab_n) * 8));
  auto* cdf = reinterpret_cast<uint64_t*>(take(size_t(num_nodes) * 8));
  auto* dsum = reinterpret_cast<uint64_t*>(take(size_t(num_nodes) * 8));
  auto* flags = reinterpret_cast<int32_t*>(take(size_t(draws) * 4));
  void* temp = p;
  size_t temp_bytes = workspace_bytes - size_t(p - static_cast<char*>(workspace));
  const uint64_t n = uint64_t(num_nodes);
  const int pair_bits = bits_for(n * n);

  // weights -> scaled, capped -> prefix sums
  BF_LAUNCH("weights_kernel", weights_kernel, dim3(blocks_for(num_nodes)), dim3(kThreads), 0, st, num_nodes, i0,
            exponent, dsum);
  BF_CHECK_LAUNCH();
  size_t tb = temp_bytes;
  BF_CHECK_HIP(prim::reduce_sum(temp, tb, static_cast<const uint64_t*>(dsum), cdf, num_nodes, st));
  BF_LAUNCH("scale_cap_kernel", scale_cap_kernel, dim3(blocks_for(num_nodes)), dim3(kThreads), 0, st, num_nodes, cdf,
            double(2 * pairs), max_degree, dsum);
  BF_CHECK_LAUNCH();
  tb = temp_bytes;
  BF_CHECK_HIP(prim::inclusive_sum(temp, tb, static_cast<const uint64_t*>(dsum), cdf, num_nodes, st));

  // draw, sort, count unique; redraw into the tail until enough unique pairs exist
  int64_t have = 0;           // unique keys at the front of keys_a (sorted)
  uint64_t counter = 0;
  for (int round = 0; round < 64 && have < pairs; ++round) {
    const int64_t fresh = draws - have;
    BF_LAUNCH("draw_pairs_kernel", draw_pairs_kernel, dim3(blocks_for(fresh)), dim3(kThreads), 0, st, cdf, num_nodes,
              fresh, seed, counter, keys_a + have);
    BF_CHECK_LAUNCH();
    counter += uint64_t(fresh);
    tb = temp_bytes;
    BF_CHECK_HIP(prim::sort_keys(temp, tb, static_cast<const uint64_t*>(keys_a), keys_b, draws, 0, 64, st));
    BF_LAUNCH("unique_flag_kernel", unique_flag_kernel, dim3(blocks_for(draws)), dim3(kThreads), 0, st, keys_b, draws,
              flags);
    BF_CHECK_LAUNCH();
    int* d_count = reinterpret_cast<int*>(keys_d);
    tb = temp_bytes;
    BF_CHECK_HIP(prim::select_flagged(temp, tb, static_cast<const uint64_t*>(keys_b),
                                      static_cast<const int32_t*>(flags), keys_a, d_count, draws, st));
    int h = 0;
    BF_CHECK_HIP(hipMemcpyAsync(&h, d_count, sizeof(int), hipMemcpyDeviceToHost, st));
    BF_CHECK_HIP(hipStreamSynchronize(st));
    have = h;
  }
  BF_CHECK_ARG(have >= pairs, "chung_lu: could not draw %lld distinct pairs", (long long)pairs);

  // exact trim: order the unique pairs by a keyed hash, keep the first `pairs`, restore key order
  BF_LAUNCH("hash_keys_kernel", hash_keys_kernel, dim3(blocks_for(have)), dim3(kThreads), 0, st, keys_a, have, seed,
            keys_b);
  BF_CHECK_LAUNCH();
  tb = temp_bytes;
  BF_CHECK_HIP(prim::sort_pairs(temp, tb, static_cast<const uint64_t*>(keys_b), keys_c,
                                static_cast<const uint64_t*>(keys_a), keys_d, have, 0, 64, st));
  tb = temp_bytes;
  BF_CHECK_HIP(prim::sort_keys(temp, tb, static_cast<const uint64_t*>(keys_d), keys_a, pairs, 0, pair_bits, st));

  // symmetrise and sort (src, dst)
  BF_LAUNCH("symmetrize_kernel", symmetrize_kernel, dim3(blocks_for(pairs)), dim3(kThreads), 0, st, keys_a, pairs, n,
            keys_b);
  BF_CHECK_LAUNCH();
  const int64_t m = 2 * pairs;
  tb = temp_bytes;
  BF_CHECK_HIP(prim::sort_keys(temp, tb, static_cast<const uint64_t*>(keys_b), keys_c, m, 0, pair_bits, st));
  BF_LAUNCH("csr_col_kernel", csr_col_kernel, dim3(blocks_for(m)), dim3(kThreads), 0, st, keys_c, m, n, col);
  BF_CHECK_LAUNCH();
  BF_LAUNCH("csr_rowptr_kernel", csr_rowptr_kernel, dim3(blocks_for(m + 1)), dim3(kThreads), 0, st, keys_c, m, n,
            rowptr);
  BF_CHECK_LAUNCH();
  BF_CHECK_HIP(hipStreamSynchronize(st));
  *num_edges_host = m;
  return BF_OK;
}
