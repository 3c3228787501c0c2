// Stable LSD radix sort of 64-bit keys by bits [begin_bit, end_bit), written
// for the reverse-index build: a few hundred thousand to a few hundred million
// keys, sorted by 17-27 id bits.
//
// Each digit pass is three launches, reduce-then-scan:
//   count   one workgroup per tile of kThreads * ITEMS keys: the tile's digit
//           histogram in LDS, stored digit-major (counts[d * tiles + t]);
//   scan    one workgroup per digit: exclusive sum over the tiles, in place,
//           and the digit's total;
//   scatter one workgroup per tile: each key's stable rank among the tile's
//           keys of its digit (ballot-matched per wave, waves in order), the
//           tile's keys regrouped by digit in LDS, then written out so that
//           consecutive lanes store consecutive positions of a digit's run.
// No look-back, no global atomics, nothing to clear between calls. Against
// rocPRIM's onesweep sort on the reverse-index keys of the benchmark builds
// (gfx950): 0.82M keys, 18 bits: 39 us (2 passes of 9 bits) vs 76 us; 31M
// keys, 22 bits: 584 us vs 614 us; 32M keys: 625 vs 639 us; 210M keys, 27
// bits: 4.57 ms vs 5.13 ms.
#pragma once

#include <cstdint>

#include "bf_common.h"

namespace bf {
namespace sort {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// The digit width and tile of a sort: 9-bit digits when they save a pass
// (18 and 27 bits), else 8. 9-bit tiles grow with the key count (2048 keys up
// to 4M keys, 4096 up to 32M, then 8192: fewer tiles, a smaller count array,
// longer digit runs per tile to write; at 210M keys the scatter pass takes
// 0.99 ms with 8192-key tiles, 1.03 with 6144 and 1.81 with 12288, whose 256
// VGPRs and 110 KB of LDS leave one wave per SIMD); 8-bit tiles hold 4096.
// Both passes map workgroups to tiles XCD by XCD (xcd_slot), so the tiles
// that share a line of the digit-major count array meet in one L2: the
// scatter pass at 210M keys went from 1.18 to 1.03 ms with it.
struct Plan {
  int radix;
  int items;
  int passes;
  int64_t tiles;
};

#ifndef BF_SORT_ITEMS_LARGE
#define BF_SORT_ITEMS_LARGE 32
#endif
inline Plan make_plan(int64_t n, int bits) {
  Plan p{};
  const int p8 = (bits + 7) / 8, p9 = (bits + 8) / 9;
  p.radix = p9 < p8 ? 9 : 8;
  p.items = p.radix == 8 ? 16 : n <= (int64_t(1) << 22) ? 8 : n <= (int64_t(1) << 25) ? 16 : BF_SORT_ITEMS_LARGE;
  p.passes = bits > 0 ? (bits + p.radix - 1) / p.radix : 0;
  const int64_t tile = int64_t(kThreads) * p.items;
  p.tiles = (n + tile - 1) / tile;
  return p;
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// The keys to sort: cap, or, with a device count, *n_dev - n_sub clamped to [0, cap] (the buffers and
// the grids are sized for cap; the tiles past the count hold nothing).
__device__ __forceinline__ int64_t live_count(int64_t cap, const int64_t* n_dev, int64_t n_sub) {
  if (!n_dev) return cap;
  const int64_t n = *n_dev - n_sub;
  return n < 0 ? 0 : (n > cap ? cap : n);
}

// Workspace of make_plan(n, bits): the second key buffer, the per-tile counts and the digit totals.
inline size_t workspace_bytes(int64_t n, int bits) {
  const Plan p = make_plan(n, bits);
  const size_t digits = size_t(1) << p.radix;
  return align256(size_t(n > 0 ? n : 1) * 8) + align256(size_t(p.tiles > 0 ? p.tiles : 1) * digits * 4) +
         align256(digits * 4);
}

// The most any bit count needs for n keys.
inline size_t workspace_bytes_max(int64_t n) {
  size_t m = 0;
  for (int bits = 1; bits <= 64; ++bits) {
    const size_t b = workspace_bytes(n, bits);
    if (b > m) m = b;
  }
  return m;
}

// block-wide exclusive scan of one value per thread; *total gets the sum
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* tmp, uint32_t* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[w] = x;
  __syncthreads();
  uint32_t wbase = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    const uint32_t t = tmp[i];
    if (i < w) wbase += t;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return wbase + x - v;
}

template <int R, int ITEMS>
__global__ __launch_bounds__(kThreads) void radix_count_kernel(const uint64_t* __restrict__ in, int64_t cap,
                                                               const int64_t* __restrict__ n_dev, int64_t n_sub,
                                                               int shift, uint32_t mask, int64_t tiles,
                                                               uint32_t* __restrict__ counts) {
  constexpr int B = 1 << R;
  constexpr int64_t TILE = int64_t(kThreads) * ITEMS;
  const int64_t n = live_count(cap, n_dev, n_sub);
  __shared__ uint32_t h[B];
  for (int i = threadIdx.x; i < B; i += kThreads) h[i] = 0;
  __syncthreads();
  const int64_t tile = xcd_slot(blockIdx.x, gridDim.x);   // the tiles sharing a counts line on one XCD
  const int64_t t0 = tile * TILE;
  uint64_t key[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int64_t pos = t0 + i * kThreads + threadIdx.x;
    key[i] = pos < n ? in[pos] : 0;
  }
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int64_t pos = t0 + i * kThreads + threadIdx.x;
    if (pos < n) atomicAdd(&h[uint32_t(key[i] >> shift) & mask], 1u);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < B; d += kThreads) counts[int64_t(d) * tiles + tile] = h[d];
}

__global__ __launch_bounds__(kThreads) void radix_scan_kernel(uint32_t* __restrict__ counts, int64_t tiles,
                                                              uint32_t* __restrict__ totals) {
  __shared__ uint32_t tmp[kWaves];
  uint32_t* row = counts + int64_t(blockIdx.x) * tiles;
  uint32_t carry = 0;
  for (int64_t base = 0; base < tiles; base += kThreads * 4) {
    uint32_t v[4], s = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t t = base + threadIdx.x * 4 + u;
      v[u] = t < tiles ? row[t] : 0;
      s += v[u];
    }
    uint32_t tot;
    uint32_t e = block_excl_scan(s, tmp, &tot) + carry;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t t = base + threadIdx.x * 4 + u;
      if (t < tiles) row[t] = e;
      e += v[u];
    }
    carry += tot;
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

// Keys of a tile sit wave-striped: wave w holds positions [w * 64 * ITEMS, (w + 1) * 64 * ITEMS) of the
// tile, item i of lane l at offset i * 64 + l, so ranking items in order and lanes in order within a wave,
// and waves in order, follows the input order (the sort is stable).
template <int R, int ITEMS>
__global__ __launch_bounds__(kThreads) void radix_scatter_kernel(const uint64_t* __restrict__ in,
                                                                 uint64_t* __restrict__ out, int64_t cap,
                                                                 const int64_t* __restrict__ n_dev, int64_t n_sub,
                                                                 int shift, uint32_t mask, int64_t tiles,
                                                                 const uint32_t* __restrict__ prefix,
                                                                 const uint32_t* __restrict__ totals) {
  constexpr int B = 1 << R;
  constexpr int DPT = B / kThreads;       // digits per thread
  constexpr int64_t TILE = int64_t(kThreads) * ITEMS;
  static_assert(B % kThreads == 0, "whole digits per thread");
  const int64_t n = live_count(cap, n_dev, n_sub);
  const int64_t tile = xcd_slot(blockIdx.x, gridDim.x);   // as in radix_count_kernel
  if (tile * TILE >= n) return;   // a tile past the count (uniform over the block)
  __shared__ uint32_t wcnt[kWaves * B];   // per wave: running counts, then exclusive offsets over the waves
  __shared__ uint32_t s_scan[kWaves];
  __shared__ uint32_t dstart[B];          // the tile's first LDS slot of each digit
  __shared__ int32_t gofs[B];             // output position of LDS slot j of digit d: gofs[d] + j
  __shared__ uint64_t skeys[TILE];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < kWaves * B; i += kThreads) wcnt[i] = 0;
  uint32_t tv[DPT], pv[DPT], tsum = 0;
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int d = tid * DPT + j;
    tv[j] = totals[d];
    pv[j] = prefix[int64_t(d) * tiles + tile];
    tsum += tv[j];
  }
  __syncthreads();
  const int64_t t0 = tile * TILE + int64_t(w) * (64 * ITEMS) + lane;
  uint64_t key[ITEMS];
  uint32_t dig[ITEMS], rank[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int64_t pos = t0 + i * 64;
    key[i] = pos < n ? __builtin_nontemporal_load(in + pos) : 0;
  }
  const uint64_t below = (uint64_t(1) << lane) - 1;
  uint32_t* wc = wcnt + w * B;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const bool valid = t0 + i * 64 < n;
    const uint32_t d = uint32_t(key[i] >> shift) & mask;
    dig[i] = d;
    // the lanes holding the same digit: R ballots narrow the valid lanes down
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < R; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const uint32_t before = __popcll(peers & below);
    const uint32_t c = valid ? wc[d] : 0u;
    rank[i] = c + before;
    // the lowest lane of each digit advances its wave's count (one writer per address)
    if (valid && before == 0) wc[d] = c + uint32_t(__popcll(peers));
  }
  __syncthreads();
  uint32_t tot[DPT], lsum = 0;
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int d = tid * DPT + j;
    uint32_t s = 0;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      const uint32_t x = wcnt[ww * B + d];
      wcnt[ww * B + d] = s;
      s += x;
    }
    tot[j] = s;
    lsum += s;
  }
  uint32_t total, gtotal;
  uint32_t ls = block_excl_scan(lsum, s_scan, &total);
  uint32_t gs = block_excl_scan(tsum, s_scan, &gtotal);
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int d = tid * DPT + j;
    dstart[d] = ls;
    gofs[d] = int32_t(gs + pv[j]) - int32_t(ls);
    ls += tot[j];
    gs += tv[j];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (t0 + i * 64 < n) skeys[dstart[dig[i]] + wc[dig[i]] + rank[i]] = key[i];
  __syncthreads();
  const int cnt = int(total);
  for (int j = tid; j < cnt; j += kThreads) {
    const uint64_t k = skeys[j];
    const int64_t o = int64_t(gofs[uint32_t(k >> shift) & mask]) + j;
    if (o >= 0 && o < n) out[o] = k;
  }
}

template <int R, int ITEMS>
int run_passes(const Plan& p, const uint64_t* in, uint64_t* out, uint64_t* alt, int64_t n, const int64_t* n_dev,
               int64_t n_sub, int begin_bit, int end_bit, uint32_t* counts, uint32_t* totals, hipStream_t st) {
  for (int pass = 0; pass < p.passes; ++pass) {
    // the last pass writes `out`: pass k writes out when passes - 1 - k is even, alt otherwise
    const uint64_t* src = pass == 0 ? in : ((p.passes - pass) % 2 == 0 ? out : alt);
    uint64_t* dst = (p.passes - 1 - pass) % 2 == 0 ? out : alt;
    const int shift = begin_bit + pass * R;
    const int bits = end_bit - shift < R ? end_bit - shift : R;
    const uint32_t mask = (1u << bits) - 1;
    BF_LAUNCH("radix_count_kernel", (radix_count_kernel<R, ITEMS>), dim3(unsigned(p.tiles)), dim3(kThreads), 0, st,
              src, n, n_dev, n_sub, shift, mask, p.tiles, counts);
    BF_CHECK_LAUNCH();
    BF_LAUNCH("radix_scan_kernel", radix_scan_kernel, dim3(1u << R), dim3(kThreads), 0, st, counts, p.tiles, totals);
    BF_CHECK_LAUNCH();
    BF_LAUNCH("radix_scatter_kernel", (radix_scatter_kernel<R, ITEMS>), dim3(unsigned(p.tiles)), dim3(kThreads), 0,
              st, src, dst, n, n_dev, n_sub, shift, mask, p.tiles, counts, totals);
    BF_CHECK_LAUNCH();
  }
  return BF_OK;
}

// Sorts in[0, n) by bits [begin_bit, end_bit) into out (stable). in and out
// must not overlap; the workspace holds workspace_bytes(n, end_bit - begin_bit).
// With n_dev the count is *n_dev - n_sub, read on the device (n is then a
// capacity: it sizes the grids; out[count, n) is left as it was).
inline int radix_sort_keys(const uint64_t* in, uint64_t* out, int64_t n, int begin_bit, int end_bit,
                           void* workspace, size_t workspace_bytes_given, hipStream_t st,
                           const int64_t* n_dev = nullptr, int64_t n_sub = 0) {
  BF_CHECK_ARG(n >= 0 && n < (int64_t(1) << 31), "radix_sort: %lld keys (at most 2^31 - 1)", (long long)n);
  BF_CHECK_ARG(begin_bit >= 0 && begin_bit <= end_bit && end_bit <= 64, "radix_sort: bits [%d, %d)", begin_bit,
               end_bit);
  if (n == 0) return BF_OK;
  const int bits = end_bit - begin_bit;
  BF_CHECK_ARG(bits > 0 || !n_dev, "radix_sort: an empty bit range takes a host count");
  if (bits == 0) {
    BF_CHECK_HIP(hipMemcpyAsync(out, in, size_t(n) * 8, hipMemcpyDeviceToDevice, st));
    return BF_OK;
  }
  const Plan p = make_plan(n, bits);
  const size_t need = workspace_bytes(n, bits);
  BF_CHECK_ARG(workspace && workspace_bytes_given >= need, "radix_sort: workspace %zu < %zu bytes",
               workspace_bytes_given, need);
  char* ws = static_cast<char*>(workspace);
  auto* alt = reinterpret_cast<uint64_t*>(ws);
  auto* counts = reinterpret_cast<uint32_t*>(ws + align256(size_t(n) * 8));
  auto* totals = reinterpret_cast<uint32_t*>(ws + align256(size_t(n) * 8) +
                                             align256(size_t(p.tiles) * (size_t(1) << p.radix) * 4));
  if (p.radix == 9)
    return p.items == 8    ? run_passes<9, 8>(p, in, out, alt, n, n_dev, n_sub, begin_bit, end_bit, counts, totals,
                                              st)
           : p.items == 16 ? run_passes<9, 16>(p, in, out, alt, n, n_dev, n_sub, begin_bit, end_bit, counts, totals,
                                               st)
           : p.items == 24 ? run_passes<9, 24>(p, in, out, alt, n, n_dev, n_sub, begin_bit, end_bit, counts, totals,
                                               st)
                           : run_passes<9, 32>(p, in, out, alt, n, n_dev, n_sub, begin_bit, end_bit, counts, totals,
                                               st);
  return run_passes<8, 16>(p, in, out, alt, n, n_dev, n_sub, begin_bit, end_bit, counts, totals, st);
}

}  // namespace sort
}  // namespace bf
