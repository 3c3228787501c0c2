// Edge-index format kernels: query-major table -> attention CSR (with the
// Graphormer global token), reference COO -> CSR, the key-major reverse index
// used by the deterministic dK/dV pass and by the COO adaptor, and split plans
// for rows longer than the attention chunk.
//
// The reverse index of a table is sorted by this build's own radix sort
// (bf_sort.h); the other sorts and the prefix sums use rocPRIM (bf_prim.h).
// Both sorts are stable LSD radix sorts, which makes the reverse index ordered
// by (kv, CSR position) = (src, dst).
#include "bf_common.h"
#include "bf_prim.h"
#include "bf_sort.h"

namespace bf {
namespace {

constexpr int kThreads = 256;

inline unsigned blocks_for(int64_t n) { return unsigned(ceil_div(n, kThreads)); }

inline size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

int bits_for(uint64_t maxval) {
  int b = 1;
  while (b < 64 && (uint64_t(1) << b) <= maxval) ++b;
  return b;
}

size_t scan_temp_bytes_i64(int64_t n) {
  size_t bytes = 0;
  (void)prim::inclusive_sum(nullptr, bytes, static_cast<const int64_t*>(nullptr), static_cast<int64_t*>(nullptr),
                            n > 0 ? n : 1, hipStream_t(nullptr));
  return bytes;
}

// block-wide exclusive scan of one 64-bit value per thread
__device__ __forceinline__ uint64_t block_excl_scan_u64(uint64_t v, uint64_t* tmp /*[kThreads / 64]*/) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint64_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[w] = x;
  __syncthreads();
  uint64_t base = 0;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i)
    if (i < w) base += tmp[i];
  __syncthreads();
  return base + x - v;
}

// ---------------------------------------------------------------- table -> CSR
// Row lengths of a table's attention CSR. With the Graphormer token (token):
// every table row gains kv 0; with a token row (lead = 1) attention row 0 is
// the token row of token_len entries and table row r is attention row r + 1.
__global__ void row_lengths_kernel(const int32_t* __restrict__ row_len, int64_t n_rows, int token, int lead,
                                   int64_t token_len, int64_t* __restrict__ lens, int64_t* __restrict__ qptr) {
  const int64_t n_q = n_rows + lead;
  const int64_t t = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (t == 0) qptr[0] = 0;     // the scan writes qptr[1..n_q]
  if (t >= n_q) return;
  lens[t] = (lead && t == 0) ? token_len : int64_t(row_len[t - lead]) + token;
}

// The same row pointers in two launches, for up to kPtrInBlockMax blocks of
// kPtrRows rows: each block's sum of its rows' lengths, then each block adds
// up the sums before it and scans its own rows (no scan state to clear).
constexpr int kPtrRowsPerThread = 16;
constexpr int64_t kPtrRows = int64_t(kThreads) * kPtrRowsPerThread;
constexpr int64_t kPtrInBlockMax = 1024;

__device__ __forceinline__ int64_t row_length(const int32_t* __restrict__ row_len, int64_t t, int token, int lead,
                                              int64_t token_len) {
  return (lead && t == 0) ? token_len : int64_t(row_len[t - lead]) + token;
}

__device__ __forceinline__ int64_t block_sum_i64(int64_t v, int64_t* tmp /*[kThreads / 64]*/) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if ((threadIdx.x & 63) == 0) tmp[threadIdx.x >> 6] = v;
  __syncthreads();
  int64_t s = 0;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) s += tmp[i];
  __syncthreads();
  return s;
}

__global__ __launch_bounds__(kThreads) void row_block_sums_kernel(const int32_t* __restrict__ row_len,
                                                                  int64_t n_rows, int token, int lead,
                                                                  int64_t token_len, int64_t* __restrict__ bsum) {
  __shared__ int64_t tmp[kThreads / 64];
  const int64_t n_q = n_rows + lead;
  const int64_t t0 = int64_t(blockIdx.x) * kPtrRows + threadIdx.x;
  int64_t s = 0;
#pragma unroll
  for (int u = 0; u < kPtrRowsPerThread; ++u) {
    const int64_t t = t0 + u * kThreads;
    if (t < n_q) s += row_length(row_len, t, token, lead, token_len);
  }
  s = block_sum_i64(s, tmp);
  if (threadIdx.x == 0) bsum[blockIdx.x] = s;
}

// Wave w of block b scans rows b * kPtrRows + w * (kPtrRows / 4) + [0, kPtrRows / 4) in rounds of 64
// (coalesced loads and stores, shuffles only), then adds the earlier waves' and blocks' totals.
__global__ __launch_bounds__(kThreads) void row_ptr_kernel(const int32_t* __restrict__ row_len, int64_t n_rows,
                                                           int token, int lead, int64_t token_len,
                                                           const int64_t* __restrict__ bsum,
                                                           int64_t* __restrict__ qptr) {
  __shared__ int64_t tmp[kThreads / 64];
  __shared__ int64_t wtot[kThreads / 64];
  const int64_t n_q = n_rows + lead;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int64_t before = 0;
  for (int64_t k = threadIdx.x; k < int64_t(blockIdx.x); k += kThreads) before += bsum[k];
  before = block_sum_i64(before, tmp);
  const int64_t t0 = int64_t(blockIdx.x) * kPtrRows + int64_t(w) * (64 * kPtrRowsPerThread) + lane;
  int64_t v[kPtrRowsPerThread];
#pragma unroll
  for (int u = 0; u < kPtrRowsPerThread; ++u) {
    const int64_t t = t0 + u * 64;
    v[u] = t < n_q ? row_length(row_len, t, token, lead, token_len) : 0;
  }
  int64_t run = 0;
#pragma unroll
  for (int u = 0; u < kPtrRowsPerThread; ++u) {
    int64_t x = v[u];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    v[u] = run + x;                                 // inclusive within the wave
    run += __shfl(x, 63, 64);
  }
  if (lane == 0) wtot[w] = run;
  __syncthreads();
  int64_t base = before;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i)
    if (i < w) base += wtot[i];
  if (blockIdx.x == 0 && threadIdx.x == 0) qptr[0] = 0;
#pragma unroll
  for (int u = 0; u < kPtrRowsPerThread; ++u) {
    const int64_t t = t0 + u * 64;
    if (t < n_q) qptr[t + 1] = base + v[u];
  }
}

// Validation of an externally supplied table (bf_check_table): bad[0] counts
// rows whose length lies outside [0, width], bad[1] the ids of a row's first
// min(row_len, width) slots outside [0, id_limit). One thread per table slot
// (grid-stride), one pair of atomics per block.
__global__ __launch_bounds__(kThreads) void check_table_kernel(const int32_t* __restrict__ table,
                                                               const int32_t* __restrict__ row_len, int64_t n_rows,
                                                               int width, int64_t id_limit,
                                                               unsigned long long* __restrict__ bad) {
  __shared__ unsigned long long blk[2];
  if (threadIdx.x < 2) blk[threadIdx.x] = 0;
  __syncthreads();
  unsigned long long bad_len = 0, bad_id = 0;
  const int64_t slots = n_rows * width;
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < slots + n_rows; i += stride) {
    if (i >= slots) {                           // one thread per row checks its length
      const int32_t len = row_len[i - slots];
      bad_len += (len < 0 || len > width) ? 1 : 0;
      continue;
    }
    const int64_t r = i / width;
    const int32_t len = row_len[r];
    if (int64_t(i - r * width) < len) {
      const int32_t id = table[i];
      bad_id += (id < 0 || int64_t(id) >= id_limit) ? 1 : 0;
    }
  }
  if (bad_len) atomicAdd(&blk[0], bad_len);
  if (bad_id) atomicAdd(&blk[1], bad_id);
  __syncthreads();
  if (threadIdx.x < 2 && blk[threadIdx.x]) atomicAdd(&bad[threadIdx.x], blk[threadIdx.x]);
}

// Writes table entry pos (slot `slot` of query row `row`): kv, and when rkey
// is given the entry's reverse-index sort key (id << kshift | row << sbits |
// slot) at kidx: a stable radix sort over the id bits alone then leaves each
// kv's entries in (row, slot) order, which is CSR order. With the Graphormer
// token only the table's own entries get keys (kidx counts them in CSR order):
// the token's entries (kv 0 of every row, the token row) have fixed places in
// the reverse index, written without a sort (TokenLayout below).
__device__ __forceinline__ void put_entry(int32_t* __restrict__ kv, uint64_t* __restrict__ rkey, int64_t pos,
                                          int64_t kidx, int64_t row, int slot, int32_t id, int kshift, int sbits) {
  kv[pos] = id;
  if (rkey) rkey[kidx] = (uint64_t(uint32_t(id)) << kshift) | (uint64_t(row) << sbits) | uint64_t(slot);
}

// One thread per table slot, then (with the Graphormer token) one thread per
// index t < max(n_rows, token_len): with a token row (lead = 1) thread t
// writes the token row's entry for kv t+1 at position t, and every thread
// t < n_rows whose table row is empty writes that row's kv 0 entry (a
// non-empty row's slot-0 thread writes it). Table row r is attention row
// r + lead and, with the token, starts with kv 0 followed by its table row
// shifted by one.
constexpr int kFillPerThread = 4;   // table slots per thread: their loads are issued before any store

__global__ __launch_bounds__(kThreads) void table_fill_kernel(
    const int32_t* __restrict__ table, const int32_t* __restrict__ row_len, int64_t n_rows, int width, int token,
    int lead, int64_t token_len, const int64_t* __restrict__ qptr, int32_t* __restrict__ kv,
    uint64_t* __restrict__ rkey, int kshift, int sbits, int slots32) {
  const int64_t slots = n_rows * width;
  const int64_t extra = token ? (lead && token_len > n_rows ? token_len : n_rows) : 0;
  const int64_t total = slots + extra;
  const int64_t base = int64_t(blockIdx.x) * (kThreads * kFillPerThread) + threadIdx.x;
  int32_t val[kFillPerThread], len[kFillPerThread], col[kFillPerThread];
  int64_t row[kFillPerThread], start[kFillPerThread];
#pragma unroll
  for (int u = 0; u < kFillPerThread; ++u) {
    const int64_t i = base + int64_t(u) * kThreads;
    len[u] = -1;                                  // no table slot: nothing to write
    row[u] = start[u] = 0;
    col[u] = val[u] = 0;
    if (i < slots) {
      // 32-bit division when the slot count allows (the host checks it): a
      // 64-bit divide by a runtime width costs several times more instructions
      const int64_t r = slots32 ? int64_t(uint32_t(i) / uint32_t(width)) : i / width;
      row[u] = r;
      col[u] = int32_t(i - r * width);
      len[u] = row_len[r];
      start[u] = qptr[r + lead];                  // table row r is attention row r + lead
      val[u] = table[i];
    }
  }
#pragma unroll
  for (int u = 0; u < kFillPerThread; ++u) {
    const int64_t i = base + int64_t(u) * kThreads;
    if (i >= slots) {
      if (i >= total) continue;
      const int64_t t = i - slots;
      // the token row's entry for kv t+1 sits at position t: its key carries slot 0
      if (lead && t < token_len) kv[t] = int32_t(t + 1);
      if (t < n_rows && row_len[t] == 0) kv[qptr[t + lead]] = 0;
      continue;
    }
    const int c = col[u];
    if (c >= len[u]) continue;
    const int64_t r = row[u] + lead;
    if (token) {
      if (c == 0) kv[start[u]] = 0;
      // the table's own entries before this one: start - token_len (the token row) - r + lead (one kv 0
      // per attention row from lead on)
      const int64_t kidx = start[u] - lead * token_len - (r - lead) + c;
      put_entry(kv, rkey, start[u] + 1 + c, kidx, r, c + 1, val[u] + 1, kshift, sbits);
    } else {
      put_entry(kv, rkey, start[u] + c, start[u] + c, r, c, val[u], kshift, sbits);
    }
  }
}

// ---------------------------------------------------------------- sorted keys -> row pointers
// ptr[r] = first position i with row(i) >= r, from row ids sorted ascending.
template <typename K>
__global__ void boundaries_kernel(const K* __restrict__ keys, int64_t n, uint64_t divisor, int64_t n_rows,
                                  int64_t* __restrict__ ptr) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i > n) return;
  int64_t r_here = i < n ? int64_t(uint64_t(keys[i]) / divisor) : n_rows;
  int64_t r_prev = i > 0 ? int64_t(uint64_t(keys[i - 1]) / divisor) : -1;
  if (r_here > n_rows) r_here = n_rows;
  if (r_prev > n_rows) r_prev = n_rows;
  fill_gap(r_prev, r_here, i, [&](int64_t r, int64_t v) { ptr[r] = v; });
}

__global__ void coo_keys_kernel(const int64_t* __restrict__ src, const int64_t* __restrict__ dst, int64_t nnz,
                                uint64_t n_kv, uint64_t* __restrict__ keys) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= nnz) return;
  keys[i] = uint64_t(dst[i]) * n_kv + uint64_t(src[i]);
}

__global__ void coo_kv_kernel(const uint64_t* __restrict__ keys, int64_t nnz, uint64_t n_kv,
                              int32_t* __restrict__ kv) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= nnz) return;
  kv[i] = int32_t(keys[i] % n_kv);
}

// ---------------------------------------------------------------- reverse index
// rows[i] = r with ptr[r] <= i < ptr[r+1] (binary search; balanced for any row length).
template <typename R>
__global__ void expand_rows_kernel(const int64_t* __restrict__ ptr, int64_t n_rows, int64_t nnz,
                                   R* __restrict__ rows) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= nnz) return;
  int64_t lo = 0, hi = n_rows;  // invariant: ptr[lo] <= i < ptr[hi]
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (ptr[mid] <= i) lo = mid; else hi = mid;
  }
  rows[i] = R(lo);
}

// Row ids of a CSR's entries in two streaming passes: each non-empty row marks
// its first entry with its id, then an inclusive max-scan fills the rest.
__global__ void row_marks_kernel(const int64_t* __restrict__ ptr, int64_t n_rows, int32_t* __restrict__ marks) {
  const int64_t r = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (r >= n_rows) return;
  const int64_t b = ptr[r];
  if (ptr[r + 1] > b) marks[b] = int32_t(r);
}

// Entry i of row r as (r << 32 | slot), slot = i - ptr[r]: the value the pair sort carries.
__global__ void pack_row_entry_kernel(const int32_t* __restrict__ rows, const int64_t* __restrict__ ptr, int64_t nnz,
                                      uint64_t* __restrict__ vals) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= nnz) return;
  const int32_t r = rows[i];
  vals[i] = (uint64_t(uint32_t(r)) << 32) | uint32_t(i - ptr[r]);
}

__global__ void unpack_row_entry_kernel(const uint64_t* __restrict__ vals, int64_t nnz, int32_t* __restrict__ kq,
                                        int32_t* __restrict__ ks) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= nnz) return;
  const uint64_t x = vals[i];
  kq[i] = int32_t(x >> 32);
  ks[i] = int32_t(uint32_t(x));
}

// The Graphormer token's part of a table's reverse index (tok = 1): kv 0 is
// attended by every attention row from `lead` on, first in the row (c0 = n_q -
// lead entries), and with a token row (lead = 1) kv t+1 (t < token_len) by row
// 0 at position t. Their reverse entries need no sort: kv 0's segment is those
// rows in order, and a token-row entry opens its kv's segment (row 0 comes
// first). The table's own entries, sorted, follow them: sorted key i with id k
// lands at c0 + lead * min(k, token_len) + i, and kv r >= 1 starts at
// c0 + lead * min(r - 1, token_len) + (keys with id < r). The kernels that
// write kv r's start (the sorted keys' boundaries) also write its token-row
// entry there, beside the keys' own entries; kv 0's segment is written apart.
struct TokenLayout {
  int tok;
  int lead;
  int64_t token_len;
  int64_t c0;
  __device__ __forceinline__ int64_t key_slot(int64_t i, int64_t k) const {
    return tok ? c0 + (lead ? (k < token_len ? k : token_len) : 0) + i : i;
  }
  __device__ __forceinline__ int64_t row_base(int64_t r) const {
    if (!tok || r == 0) return 0;
    return c0 + (lead ? (r - 1 < token_len ? r - 1 : token_len) : 0);
  }
  // kv r opens with the token row's entry (CSR position r - 1)
  __device__ __forceinline__ bool token_entry(int64_t r) const { return lead && r >= 1 && r - 1 < token_len; }
};

// A table entry's slot in its query's row, from its key (no read of qptr).
__device__ __forceinline__ int32_t slot_of(uint64_t x, int sbits) {
  return int32_t(x & ((uint64_t(1) << sbits) - 1));
}

constexpr int kUnpackPerThread = 4;  // sorted keys per thread (kThreads apart), loaded before any store

// The table entries that carry a sort key: the index's entries (qptr[n_q], read on the device) less the
// token's own, clamped to the capacity the buffers and grids were sized for.
__device__ __forceinline__ int64_t keyed_entries(const int64_t* __restrict__ nnz_dev, int64_t n_token,
                                                 int64_t cap) {
  const int64_t n = *nnz_dev - n_token;
  return n < 0 ? 0 : (n > cap ? cap : n);
}

// Sorted keys -> kptr (boundaries of the id field), kq, and ks when asked for.
// Blocks from key_blocks on write kv 0's segment with the token instead (what
// token_reverse_kernel writes), saving its launch.
__global__ __launch_bounds__(kThreads) void unpack_rkey_kernel(
    const uint64_t* __restrict__ keys, const int64_t* __restrict__ nnz_dev, int64_t n_token, int64_t key_cap,
    int kshift, int sbits, TokenLayout tl, int64_t n_kv, int64_t* __restrict__ kptr, int32_t* __restrict__ kq,
    int32_t* __restrict__ ks, int64_t key_blocks) {
  if (int64_t(blockIdx.x) >= key_blocks) {
    const int64_t j = (int64_t(blockIdx.x) - key_blocks) * kThreads + threadIdx.x;
    if (j < tl.c0) {
      kq[j] = int32_t(tl.lead + j);
      if (ks) ks[j] = 0;                 // kv 0 opens every row from `lead` on
    }
    return;
  }
  const int64_t n_keys = keyed_entries(nnz_dev, n_token, key_cap);
  const int64_t base = int64_t(blockIdx.x) * (kThreads * kUnpackPerThread) + threadIdx.x;
  uint64_t cur[kUnpackPerThread], prev[kUnpackPerThread];
#pragma unroll
  for (int u = 0; u < kUnpackPerThread; ++u) {
    const int64_t i = base + int64_t(u) * kThreads;
    cur[u] = i < n_keys ? keys[i] : 0;
    prev[u] = (i > 0 && i <= n_keys) ? keys[i - 1] : 0;
  }
#pragma unroll
  for (int u = 0; u < kUnpackPerThread; ++u) {
    const int64_t i = base + int64_t(u) * kThreads;
    if (i > n_keys) break;
    int64_t r_here = i < n_keys ? int64_t(cur[u] >> kshift) : n_kv;
    // with the token the keys' ids start at 1 and kptr[0] = 0 (kv 0's segment opens the index)
    int64_t r_prev = i > 0 ? int64_t(prev[u] >> kshift) : (tl.tok ? 0 : -1);
    if (r_here > n_kv) r_here = n_kv;
    if (r_prev > n_kv) r_prev = n_kv;
    if (i == 0 && tl.tok) kptr[0] = 0;
    fill_gap(r_prev, r_here, i, [&](int64_t r, int64_t v) {
      const int64_t b = tl.row_base(r) + v;
      kptr[r] = b;
      if (r < n_kv && tl.token_entry(r)) {
        kq[b] = 0;
        if (ks) ks[b] = int32_t(r - 1);  // the token row lists kv r at slot r - 1
      }
    });
    if (i == n_keys) break;
    const int64_t o = tl.key_slot(i, int64_t(cur[u] >> kshift));
    kq[o] = int32_t((cur[u] >> sbits) & ((uint64_t(1) << (kshift - sbits)) - 1));
    if (ks) ks[o] = slot_of(cur[u], sbits);
  }
}

// ks from the sorted keys (one thread per key, plus one past the end): with
// the token row, the thread that meets the first key with id >= r (or the
// end) also writes kv r's token-row entry (r <= token_len), at kv r's start.
__global__ void reverse_slots_kernel(const uint64_t* __restrict__ keys, const int64_t* __restrict__ nnz_dev,
                                     int64_t n_token, int64_t key_cap, int kshift, int sbits, TokenLayout tl,
                                     int32_t* __restrict__ ks) {
  const int64_t n_keys = keyed_entries(nnz_dev, n_token, key_cap);
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i > n_keys) return;
  const uint64_t x = i < n_keys ? keys[i] : 0;
  if (tl.lead) {
    const int64_t top = tl.token_len;    // the last kv row with a token-row entry
    int64_t r_here = i < n_keys ? int64_t(x >> kshift) : top;
    int64_t r_prev = i > 0 ? int64_t(keys[i - 1] >> kshift) : 0;
    if (r_here > top) r_here = top;
    if (r_prev > top) r_prev = top;
    fill_gap(r_prev, r_here, i, [&](int64_t r, int64_t v) { ks[tl.row_base(r) + v] = int32_t(r - 1); });
  }
  if (i < n_keys) ks[tl.key_slot(i, int64_t(x >> kshift))] = slot_of(x, sbits);
}

// kv 0's reverse segment with the token (kq and/or ks): thread j < c0 writes the entry of attention row
// lead + j, first in that row (slot 0).
__global__ void token_reverse_kernel(TokenLayout tl, int32_t* __restrict__ kq, int32_t* __restrict__ ks) {
  const int64_t j = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (j < tl.c0) {
    if (kq) kq[j] = int32_t(tl.lead + j);
    if (ks) ks[j] = 0;
  }
}

inline TokenLayout token_layout(int global_token, int64_t token_row, int64_t n_q) {
  TokenLayout tl{0, 0, 0, 0};
  if (!global_token) return tl;
  tl.tok = 1;
  tl.lead = token_row >= 0 ? 1 : 0;
  tl.token_len = tl.lead ? token_row : 0;
  tl.c0 = n_q - tl.lead;
  return tl;
}

inline int launch_token_reverse(const TokenLayout& tl, int32_t* kq, int32_t* ks, hipStream_t st) {
  if (!tl.tok || tl.c0 == 0) return BF_OK;
  BF_LAUNCH("token_reverse_kernel", token_reverse_kernel, dim3(blocks_for(tl.c0)), dim3(kThreads), 0, st, tl, kq,
            ks);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

// Row order, longest first: bucket 255 - min(len, 255). Three launches in
// the radix sort's count / scan / place pattern over blocks of kOrderRows
// rows: each block's bucket counts (bucket-major), an exclusive sum per bucket
// over the blocks (sort::radix_scan_kernel), then each block places its rows
// from its buckets' offsets. No global atomics and nothing to clear. Rows of
// one bucket within a block come out in an arbitrary order: the order only
// decides which group serves which row, never a row's arithmetic.
constexpr int kBuckets = 256;
static_assert(kBuckets == kThreads, "the order kernels keep one bucket per thread");
constexpr int kOrderRowsPerThread = 8;
constexpr int64_t kOrderRows = int64_t(kThreads) * kOrderRowsPerThread;

// A row's split-plan entry: (items << 32) | (1 if it splits), items =
// split_row_items(len) for rows longer than the threshold, else 0. The plan is
// the exclusive sum of these over the rows.
__device__ __forceinline__ uint64_t split_count(int64_t len, int threshold, int item_size) {
  if (len <= threshold) return 0;
  return (uint64_t(split_row_items(len, item_size)) << 32) | 1u;
}

__device__ __forceinline__ int bucket_of(int64_t len) { return 255 - int(len < 255 ? len : 255); }

__global__ __launch_bounds__(kThreads) void order_count_kernel(const int64_t* __restrict__ ptr, int64_t n_rows,
                                                               int64_t blocks, uint32_t* __restrict__ counts) {
  __shared__ uint32_t h[kBuckets];
  h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t r0 = int64_t(blockIdx.x) * kOrderRows + threadIdx.x;
#pragma unroll
  for (int u = 0; u < kOrderRowsPerThread; ++u) {
    const int64_t r = r0 + u * kThreads;
    if (r < n_rows) atomicAdd(&h[bucket_of(ptr[r + 1] - ptr[r])], 1u);
  }
  __syncthreads();
  counts[int64_t(threadIdx.x) * blocks + blockIdx.x] = h[threadIdx.x];
}

// Places block b's rows: slot = (rows of longer buckets) + (rows of this
// bucket in earlier blocks) + rank in the block; with `spans` each slot's row
// as (begin << 32 | length), which the reader then takes from the slot instead
// of a random read of the row pointers; with `packed` the split-plan entry of
// each of the first n_slots slots.
__global__ __launch_bounds__(kThreads) void order_place_kernel(const int64_t* __restrict__ ptr, int64_t n_rows,
                                                               int64_t blocks, const uint32_t* __restrict__ prefix,
                                                               const uint32_t* __restrict__ totals,
                                                               int32_t* __restrict__ order,
                                                               uint64_t* __restrict__ spans, int threshold,
                                                               int item_size, int64_t n_slots,
                                                               uint64_t* __restrict__ packed) {
  __shared__ uint32_t base[kBuckets];
  __shared__ uint32_t cnt[kBuckets];
  __shared__ uint32_t tmp[kThreads / 64];
  const int tid = threadIdx.x;
  uint32_t all;
  const uint32_t before = sort::block_excl_scan(totals[tid], tmp, &all);
  base[tid] = before + prefix[int64_t(tid) * blocks + blockIdx.x];
  cnt[tid] = 0;
  __syncthreads();
  const int64_t r0 = int64_t(blockIdx.x) * kOrderRows + tid;
#pragma unroll
  for (int u = 0; u < kOrderRowsPerThread; ++u) {
    const int64_t r = r0 + u * kThreads;
    if (r >= n_rows) break;
    const int64_t beg = ptr[r], len = ptr[r + 1] - beg;
    const int b = bucket_of(len);
    const uint32_t slot = base[b] + atomicAdd(&cnt[b], 1u);
    order[slot] = int32_t(r);
    if (spans) spans[slot] = (uint64_t(beg) << 32) | uint64_t(len);
    if (packed && slot < n_slots) packed[slot] = split_count(len, threshold, item_size);
  }
}

// The split plan of a CSR whose only row longer than the threshold is row 0,
// cut into n_items items (0: no split row): what split_count / scan /
// split_rows would write, in one pass and with no scan.
__global__ void split_first_row_kernel(int64_t n_rows, int n_items, int32_t* __restrict__ nitems,
                                       int32_t* __restrict__ item_off, int32_t* __restrict__ item_row,
                                       int32_t* __restrict__ heavy_rows, int32_t* __restrict__ counts) {
  const int64_t r = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (r < n_rows) {
    nitems[r] = r == 0 ? n_items : 0;
    item_off[r] = r == 0 ? 0 : n_items;
  }
  if (r < n_items) item_row[r] = 0;
  if (r == 0) {
    if (n_items) heavy_rows[0] = 0;
    counts[0] = n_items;
    counts[1] = n_items ? 1 : 0;
  }
}

struct MaxOp {
  __device__ __forceinline__ int32_t operator()(int32_t a, int32_t b) const { return a > b ? a : b; }
};

size_t row_ids_temp_bytes(int64_t nnz) {
  size_t bytes = 0;
  (void)prim::inclusive_scan(nullptr, bytes, static_cast<const int32_t*>(nullptr), static_cast<int32_t*>(nullptr),
                             MaxOp(), nnz > 0 ? nnz : 1, hipStream_t(nullptr));
  return bytes;
}

// rows[i] for every entry of a CSR (int32); marks and rows may not alias.
int row_ids(const int64_t* ptr, int64_t n_rows, int64_t nnz, int32_t* marks, int32_t* rows, void* temp,
            size_t temp_bytes, hipStream_t st) {
  BF_CHECK_HIP(hipMemsetAsync(marks, 0, size_t(nnz) * sizeof(int32_t), st));
  BF_LAUNCH("row_marks_kernel", row_marks_kernel, dim3(blocks_for(n_rows)), dim3(kThreads), 0, st, ptr, n_rows, marks);
  BF_CHECK_LAUNCH();
  BF_CHECK_HIP(prim::inclusive_scan(temp, temp_bytes, static_cast<const int32_t*>(marks), rows, MaxOp(), nnz, st));
  return BF_OK;
}

// ---------------------------------------------------------------- split plans
// Per row (items << 32 | is_heavy), so that ONE exclusive scan yields both the
// first item and the heavy-list slot of every row.
__global__ void split_count_kernel(const int64_t* __restrict__ ptr, int64_t n_rows, int threshold, int item_size,
                                   uint64_t* __restrict__ packed) {
  const int64_t r = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (r < n_rows) packed[r] = split_count(ptr[r + 1] - ptr[r], threshold, item_size);
}

// nitems, item_off, the heavy-row list (compacted by the scanned flags),
// item_row of each item and the two plan counts, one thread per slot: slot j
// is row j, or with an order row order[j], and then only the split rows'
// entries are written. A row's thread writes the item_row of its first
// kOwnItems items; rows with more (the Graphormer token row and column, hubs)
// are queued in LDS and their remaining items written by the whole block.
// packed_off NULL: the exclusive sums are formed here, each block adding up
// the slots before it (plans of at most kPlanInBlockSlots slots).
constexpr int kOwnItems = 32;
constexpr int64_t kPlanInBlockSlots = 32768;

__global__ __launch_bounds__(kThreads) void split_rows_kernel(
    const uint64_t* __restrict__ packed, const uint64_t* __restrict__ packed_off, const int32_t* __restrict__ order,
    int64_t n_slots, int64_t item_cap, int32_t* __restrict__ nitems, int32_t* __restrict__ item_off,
    int32_t* __restrict__ item_row, int32_t* __restrict__ heavy_rows, int64_t heavy_cap,
    int32_t* __restrict__ counts) {
  __shared__ int64_t long_first[kThreads];
  __shared__ int32_t long_n[kThreads], long_row[kThreads];
  __shared__ int n_long;
  __shared__ uint64_t scan_tmp[kThreads / 64];
  if (threadIdx.x == 0) n_long = 0;
  const int64_t j = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  uint64_t in_block_off = 0;
  if (!packed_off) {
    // With an order the split rows hold its first slots (longest first), so a slot's entry is zero only
    // past the last split row: a thread stops at its first zero. Four loads in flight per step.
    const int64_t lim = int64_t(blockIdx.x) * kThreads;
    uint64_t before = 0;
    for (int64_t k = threadIdx.x; k < lim; k += 4 * kThreads) {
      uint64_t x[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) x[u] = k + u * kThreads < lim ? packed[k + u * kThreads] : 0;
      before += x[0] + x[1] + x[2] + x[3];
      if (order && x[3] == 0) break;
    }
    // the block's total of `before` is the sum over every earlier slot
    const uint64_t lo = block_excl_scan_u64(before, scan_tmp);
    __shared__ uint64_t s_before;
    if (threadIdx.x == kThreads - 1) s_before = lo + before;
    __syncthreads();
    in_block_off = s_before + block_excl_scan_u64(j < n_slots ? packed[j] : 0, scan_tmp);
  }
  __syncthreads();
  if (j < n_slots) {
    const int n = int(packed[j] >> 32);
    const uint64_t off = packed_off ? packed_off[j] : in_block_off;
    const int64_t first_item = int64_t(off >> 32);
    const int64_t slot = int64_t(uint32_t(off));
    if (!order || n > 0) {
      const int32_t r = order ? order[j] : int32_t(j);
      nitems[r] = n;
      item_off[r] = int32_t(first_item);
      if (n > 0 && slot < heavy_cap) heavy_rows[slot] = r;
      for (int64_t i = 0; i < n && i < kOwnItems && first_item + i < item_cap; ++i) item_row[first_item + i] = r;
      if (n > kOwnItems) {
        const int k = atomicAdd(&n_long, 1);
        long_first[k] = first_item;
        long_n[k] = n;
        long_row[k] = r;
      }
    }
    if (j == n_slots - 1) {
      const int64_t items = first_item + n;
      const int64_t heavy = slot + (n > 0 ? 1 : 0);
      counts[0] = int32_t(items < item_cap ? items : item_cap);
      counts[1] = int32_t(heavy < heavy_cap ? heavy : heavy_cap);
    }
  }
  __syncthreads();
  for (int k = 0; k < n_long; ++k) {
    const int64_t first_item = long_first[k];
    for (int64_t j = kOwnItems + threadIdx.x; j < long_n[k] && first_item + j < item_cap; j += kThreads)
      item_row[first_item + j] = long_row[k];
  }
}

}  // namespace
}  // namespace bf

using namespace bf;

extern "C" int bf_scan_workspace_size(int64_t n, size_t* bytes) {
  BF_CHECK_ARG(bytes && n >= 0, "scan_workspace_size: bad arguments");
  *bytes = align_up(size_t(n > 0 ? n : 1) * sizeof(int64_t)) + align_up(scan_temp_bytes_i64(n)) + 256;
  return BF_OK;
}

extern "C" int bf_table_csr_ptr(const int32_t* row_len, int64_t n_rows, int32_t global_token, int64_t token_row,
                                int64_t* qptr, int64_t* nnz_host, void* workspace, size_t workspace_bytes,
                                void* stream) {
  BF_CHECK_ARG(qptr && n_rows >= 0 && (row_len || n_rows == 0), "table_csr_ptr: bad arguments");
  BF_CHECK_ARG(!global_token || token_row < (int64_t(1) << 31) - 1, "table_csr_ptr: token row of %lld entries",
               (long long)token_row);
  const int lead = (global_token && token_row >= 0) ? 1 : 0;
  const int64_t n_q = n_rows + lead;
  size_t need = 0;
  bf_scan_workspace_size(n_q, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "table_csr_ptr: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  if (n_q == 0) BF_CHECK_HIP(hipMemsetAsync(qptr, 0, sizeof(int64_t), st));
  const int64_t ptr_blocks = ceil_div(n_q, kPtrRows);
  if (n_q > 0 && ptr_blocks <= kPtrInBlockMax) {
    auto* bsum = static_cast<int64_t*>(workspace);     // the first ptr_blocks of the n_q slots
    const int64_t token_len = lead ? token_row : int64_t(0);
    BF_LAUNCH("row_block_sums_kernel", row_block_sums_kernel, dim3(unsigned(ptr_blocks)), dim3(kThreads), 0, st,
              row_len, n_rows, int(global_token != 0), lead, token_len, bsum);
    BF_CHECK_LAUNCH();
    BF_LAUNCH("row_ptr_kernel", row_ptr_kernel, dim3(unsigned(ptr_blocks)), dim3(kThreads), 0, st, row_len, n_rows,
              int(global_token != 0), lead, token_len, static_cast<const int64_t*>(bsum), qptr);
    BF_CHECK_LAUNCH();
  } else if (n_q > 0) {
    auto* lens = static_cast<int64_t*>(workspace);
    void* temp = static_cast<char*>(workspace) + align_up(size_t(n_q) * sizeof(int64_t));
    size_t temp_bytes = scan_temp_bytes_i64(n_q);
    BF_LAUNCH("row_lengths_kernel", row_lengths_kernel, dim3(blocks_for(n_q)), dim3(kThreads), 0, st, row_len, n_rows,
              int(global_token != 0), lead, lead ? token_row : int64_t(0), lens, qptr);
    BF_CHECK_LAUNCH();
    BF_CHECK_HIP(prim::inclusive_sum(temp, temp_bytes, static_cast<const int64_t*>(lens), qptr + 1, n_q, st));
  }
  if (!nnz_host) return BF_OK;   // the caller reads qptr[n_q] itself, when it needs it
  int64_t h = 0;
  BF_CHECK_HIP(hipMemcpyAsync(&h, qptr + n_q, sizeof(h), hipMemcpyDeviceToHost, st));
  BF_CHECK_HIP(hipStreamSynchronize(st));
  *nnz_host = h;
  return BF_OK;
}

extern "C" int bf_check_table(const int32_t* table, const int32_t* row_len, int64_t n_rows, int32_t width,
                              int64_t id_limit, int64_t* bad_host, void* workspace, size_t workspace_bytes,
                              void* stream) {
  BF_CHECK_ARG(n_rows >= 0 && width >= 0 && id_limit >= 0, "check_table: bad sizes");
  BF_CHECK_ARG(n_rows == 0 || (table && row_len), "check_table: null tensor");
  BF_CHECK_ARG(workspace && workspace_bytes >= 2 * sizeof(int64_t), "check_table: workspace %zu < 16 bytes",
               workspace_bytes);
  hipStream_t st = as_stream(stream);
  auto* bad = static_cast<unsigned long long*>(workspace);
  BF_CHECK_HIP(hipMemsetAsync(bad, 0, 2 * sizeof(int64_t), st));
  const int64_t work = n_rows * width + n_rows;
  if (work > 0) {
    const int64_t need = ceil_div(work, int64_t(kThreads));
    const int64_t blocks = need < 4096 ? need : 4096;
    BF_LAUNCH("check_table_kernel", check_table_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0, st, table, row_len,
              n_rows, width, id_limit, bad);
    BF_CHECK_LAUNCH();
  }
  int64_t h[2] = {0, 0};
  BF_CHECK_HIP(hipMemcpyAsync(h, bad, sizeof(h), hipMemcpyDeviceToHost, st));
  BF_CHECK_HIP(hipStreamSynchronize(st));
  if (bad_host) {
    bad_host[0] = h[0];
    bad_host[1] = h[1];
  }
  BF_CHECK_ARG(h[0] == 0, "check_table: %lld row lengths outside [0, %d]", (long long)h[0], width);
  BF_CHECK_ARG(h[1] == 0, "check_table: %lld table ids outside [0, %lld)", (long long)h[1], (long long)id_limit);
  return BF_OK;
}

extern "C" int bf_table_to_csr(const int32_t* table, const int32_t* row_len, int64_t n_rows, int32_t width,
                               int32_t global_token, int64_t token_row, const int64_t* qptr, int32_t* kv,
                               uint64_t* rkey, int32_t q_bits, int32_t slot_bits, void* stream) {
  BF_CHECK_ARG(n_rows >= 0 && width >= 0 && qptr, "table_to_csr: bad arguments");
  BF_CHECK_ARG(!global_token || token_row < (int64_t(1) << 31) - 1, "table_to_csr: token row of %lld entries",
               (long long)token_row);
  const int lead = (global_token && token_row >= 0) ? 1 : 0;
  const int64_t token_len = lead ? token_row : 0;
  BF_CHECK_ARG((n_rows == 0 || (table && row_len)) && (kv || (n_rows == 0 && token_len == 0)),
               "table_to_csr: null tensor");
  if (rkey) {
    const int64_t n_q = n_rows + lead;
    BF_CHECK_ARG(q_bits >= bits_for(uint64_t(n_q)) && slot_bits >= bits_for(uint64_t(width)) &&
                     q_bits + slot_bits <= 33,
                 "table_to_csr: key fields (%d query bits, %d slot bits) do not hold %lld queries of width %d "
                 "beside a 31-bit id", q_bits, slot_bits, (long long)n_q, width);
  }
  const int64_t extra = global_token ? (token_len > n_rows ? token_len : n_rows) : 0;
  const int64_t threads = n_rows * width + extra;
  if (threads > 0) {
    BF_LAUNCH("table_fill_kernel", table_fill_kernel, dim3(unsigned(ceil_div(threads, int64_t(kThreads) * kFillPerThread))),
              dim3(kThreads), 0, as_stream(stream),
              table, row_len, n_rows, width, int(global_token != 0), lead, token_len, qptr, kv, rkey,
              q_bits + slot_bits, slot_bits, int(n_rows * width < (int64_t(1) << 32)));
    BF_CHECK_LAUNCH();
  }
  return BF_OK;
}

extern "C" int bf_coo_to_csr_workspace_size(int64_t nnz, int64_t n_q, size_t* bytes) {
  BF_CHECK_ARG(bytes && nnz >= 0 && n_q >= 0, "coo_to_csr_workspace_size: bad arguments");
  size_t sort_bytes = 0;
  (void)prim::sort_keys(nullptr, sort_bytes, static_cast<const uint64_t*>(nullptr), static_cast<uint64_t*>(nullptr),
                        nnz > 0 ? nnz : 1, 0, 64, hipStream_t(nullptr));
  *bytes = 2 * align_up(size_t(nnz > 0 ? nnz : 1) * sizeof(uint64_t)) + align_up(sort_bytes) + 256;
  (void)n_q;
  return BF_OK;
}

extern "C" int bf_coo_to_csr(const int64_t* src, const int64_t* dst, int64_t nnz, int64_t n_q, int64_t n_kv,
                             int64_t* qptr, int32_t* kv, void* workspace, size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(nnz >= 0 && n_q >= 0 && n_kv > 0 && qptr, "coo_to_csr: bad arguments");
  BF_CHECK_ARG(n_kv < (int64_t(1) << 31) && nnz < (int64_t(1) << 31), "coo_to_csr: sizes must fit int32");
  size_t need = 0;
  bf_coo_to_csr_workspace_size(nnz, n_q, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "coo_to_csr: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  if (nnz == 0) {
    BF_CHECK_HIP(hipMemsetAsync(qptr, 0, size_t(n_q + 1) * sizeof(int64_t), st));
    return BF_OK;
  }
  auto* keys_in = static_cast<uint64_t*>(workspace);
  auto* keys_out = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + align_up(size_t(nnz) * 8));
  void* temp = static_cast<char*>(workspace) + 2 * align_up(size_t(nnz) * 8);
  size_t temp_bytes = 0;
  (void)prim::sort_keys(nullptr, temp_bytes, static_cast<const uint64_t*>(keys_in), keys_out, nnz, 0, 64, st);
  BF_LAUNCH("coo_keys_kernel", coo_keys_kernel, dim3(blocks_for(nnz)), dim3(kThreads), 0, st, src, dst, nnz,
                     uint64_t(n_kv), keys_in);
  BF_CHECK_LAUNCH();
  const int end_bit = bits_for(uint64_t(n_q) * uint64_t(n_kv));
  BF_CHECK_HIP(prim::sort_keys(temp, temp_bytes, static_cast<const uint64_t*>(keys_in), keys_out, nnz, 0, end_bit, st));
  BF_LAUNCH("coo_kv_kernel", coo_kv_kernel, dim3(blocks_for(nnz)), dim3(kThreads), 0, st, keys_out, nnz,
                     uint64_t(n_kv), kv);
  BF_CHECK_LAUNCH();
  BF_LAUNCH("boundaries_kernel", boundaries_kernel<uint64_t>, dim3(blocks_for(nnz + 1)), dim3(kThreads), 0, st, keys_out,
                     nnz, uint64_t(n_kv), n_q, qptr);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int bf_reverse_index_workspace_size(int64_t nnz, int64_t n_kv, size_t* bytes) {
  BF_CHECK_ARG(bytes && nnz >= 0 && n_kv >= 0, "reverse_index_workspace_size: bad arguments");
  size_t sort_bytes = 0;
  const int64_t n = nnz > 0 ? nnz : 1;
  (void)prim::sort_pairs(nullptr, sort_bytes, static_cast<const uint32_t*>(nullptr), static_cast<uint32_t*>(nullptr),
                         static_cast<const uint64_t*>(nullptr), static_cast<uint64_t*>(nullptr), n, 0, 32,
                         hipStream_t(nullptr));
  const size_t scan_bytes = row_ids_temp_bytes(nnz);
  // keys_out (4) + marks (4) + rows (4) + packed values in/out (8 + 8) bytes per entry, then temp
  *bytes = 3 * align_up(size_t(n) * 4) + 2 * align_up(size_t(n) * 8) +
           align_up(sort_bytes > scan_bytes ? sort_bytes : scan_bytes) + 256;
  return BF_OK;
}

extern "C" int bf_reverse_index(const int64_t* qptr, const int32_t* kv, int64_t n_q, int64_t n_kv, int64_t nnz,
                                int64_t* kptr, int32_t* kq, int32_t* ks, void* workspace,
                                size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(qptr && kptr && n_q >= 0 && n_kv >= 0 && nnz >= 0, "reverse_index: bad arguments");
  BF_CHECK_ARG(nnz < (int64_t(1) << 31) && n_q < (int64_t(1) << 31), "reverse_index: sizes must fit int32");
  size_t need = 0;
  bf_reverse_index_workspace_size(nnz, n_kv, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "reverse_index: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  if (nnz == 0) {
    BF_CHECK_HIP(hipMemsetAsync(kptr, 0, size_t(n_kv + 1) * sizeof(int64_t), st));
    return BF_OK;
  }
  BF_CHECK_ARG(kv && kq && ks, "reverse_index: null tensor");
  char* p = static_cast<char*>(workspace);
  auto take = [&](size_t b) { char* q = p; p += align_up(b); return q; };
  auto* keys_out = reinterpret_cast<uint32_t*>(take(size_t(nnz) * 4));
  auto* marks = reinterpret_cast<int32_t*>(take(size_t(nnz) * 4));
  auto* rows = reinterpret_cast<int32_t*>(take(size_t(nnz) * 4));
  auto* vals_in = reinterpret_cast<uint64_t*>(take(size_t(nnz) * 8));
  auto* vals_out = reinterpret_cast<uint64_t*>(take(size_t(nnz) * 8));
  void* temp = p;
  const size_t temp_bytes = workspace_bytes - size_t(p - static_cast<char*>(workspace));
  int rc = row_ids(qptr, n_q, nnz, marks, rows, temp, temp_bytes, st);
  if (rc) return rc;
  BF_LAUNCH("pack_row_entry_kernel", pack_row_entry_kernel, dim3(blocks_for(nnz)), dim3(kThreads), 0, st, rows, qptr,
            nnz, vals_in);
  BF_CHECK_LAUNCH();
  const int end_bit = bits_for(uint64_t(n_kv > 0 ? n_kv : 1));
  size_t tb = temp_bytes;
  BF_CHECK_HIP(prim::sort_pairs(temp, tb, reinterpret_cast<const uint32_t*>(kv), keys_out,
                                static_cast<const uint64_t*>(vals_in), vals_out, nnz, 0, end_bit, st));
  BF_LAUNCH("boundaries_kernel", boundaries_kernel<uint32_t>, dim3(blocks_for(nnz + 1)), dim3(kThreads), 0, st, keys_out,
            nnz, uint64_t(1), n_kv, kptr);
  BF_CHECK_LAUNCH();
  BF_LAUNCH("unpack_row_entry_kernel", unpack_row_entry_kernel, dim3(blocks_for(nnz)), dim3(kThreads), 0, st, vals_out,
            nnz, kq, ks);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int bf_reverse_index_packed_workspace_size(int64_t nnz, size_t* bytes) {
  BF_CHECK_ARG(bytes && nnz >= 0, "reverse_index_packed_workspace_size: bad arguments");
  *bytes = sort::workspace_bytes_max(nnz) + 256;
  return BF_OK;
}

extern "C" int bf_reverse_index_packed(const uint64_t* rkey, const int64_t* qptr, int64_t nnz, int64_t n_q,
                                       int64_t n_kv, int32_t q_bits, int32_t slot_bits, int32_t global_token,
                                       int64_t token_row, uint64_t* sorted, int64_t* kptr, int32_t* kq, int32_t* ks,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(kptr && qptr && n_q >= 0 && n_kv >= 0 && nnz >= 0, "reverse_index_packed: bad arguments");
  BF_CHECK_ARG(nnz < (int64_t(1) << 31), "reverse_index_packed: sizes must fit int32");
  const int kshift = q_bits + slot_bits;
  const int id_bits = bits_for(uint64_t(n_kv > 0 ? n_kv : 1));
  BF_CHECK_ARG(q_bits >= bits_for(uint64_t(n_q)) && slot_bits >= 1 && kshift + id_bits <= 64,
               "reverse_index_packed: key fields (%d + %d + %d bits) do not fit", q_bits, slot_bits, id_bits);
  const TokenLayout tl = token_layout(global_token != 0, token_row, n_q);
  BF_CHECK_ARG(!tl.tok || (tl.c0 >= 0 && tl.token_len < n_kv), "reverse_index_packed: token layout does not fit "
               "(%lld queries, token row of %lld entries, %lld kv rows)", (long long)n_q, (long long)tl.token_len,
               (long long)n_kv);
  const int64_t n_token = tl.tok ? tl.c0 + tl.token_len : 0;
  const int64_t n_keys = nnz - n_token;     // a capacity: the count itself is qptr[n_q] - n_token
  BF_CHECK_ARG(n_keys >= 0, "reverse_index_packed: %lld entries cannot hold the token's %lld", (long long)nnz,
               (long long)(tl.c0 + tl.token_len));
  size_t need = 0;
  bf_reverse_index_packed_workspace_size(nnz, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "reverse_index_packed: workspace %zu < %zu bytes",
               workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  if (nnz == 0) {
    BF_CHECK_HIP(hipMemsetAsync(kptr, 0, size_t(n_kv + 1) * sizeof(int64_t), st));
    return BF_OK;
  }
  BF_CHECK_ARG(kq && (n_keys == 0 || (rkey && sorted)), "reverse_index_packed: null tensor");
  if (n_keys > 0) {
    // only the id bits are sorted; the stable passes keep each id's entries in CSR order
    const int rc = sort::radix_sort_keys(rkey, sorted, n_keys, kshift, kshift + id_bits, workspace, workspace_bytes,
                                         st, qptr + n_q, n_token);
    if (rc) return rc;
  }
  const int64_t key_blocks = ceil_div(n_keys + 1, int64_t(kThreads) * kUnpackPerThread);
  const int64_t tok_blocks = tl.tok ? ceil_div(tl.c0, int64_t(kThreads)) : 0;
  BF_LAUNCH("unpack_rkey_kernel", unpack_rkey_kernel, dim3(unsigned(key_blocks + tok_blocks)), dim3(kThreads), 0, st,
            sorted, qptr + n_q, n_token, n_keys, kshift, slot_bits, tl, n_kv, kptr, kq, ks, key_blocks);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int bf_radix_sort_workspace_size(int64_t n, int32_t begin_bit, int32_t end_bit, size_t* bytes) {
  BF_CHECK_ARG(bytes && n >= 0 && begin_bit >= 0 && begin_bit <= end_bit && end_bit <= 64,
               "radix_sort_workspace_size: bad arguments");
  *bytes = sort::workspace_bytes(n, end_bit - begin_bit);
  return BF_OK;
}

extern "C" int bf_radix_sort_keys(const uint64_t* in, uint64_t* out, int64_t n, int32_t begin_bit, int32_t end_bit,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(n == 0 || (in && out && in != out), "radix_sort_keys: bad buffers");
  return sort::radix_sort_keys(in, out, n, begin_bit, end_bit, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int bf_reverse_slots(const uint64_t* sorted, const int64_t* qptr, int64_t nnz, int64_t n_q,
                                int32_t q_bits, int32_t slot_bits, int32_t global_token, int64_t token_row, int32_t* ks,
                                void* stream) {
  BF_CHECK_ARG(qptr && nnz >= 0 && nnz < (int64_t(1) << 31) && n_q >= 0, "reverse_slots: bad arguments");
  BF_CHECK_ARG(q_bits >= bits_for(uint64_t(n_q)) && slot_bits >= 1 && q_bits + slot_bits <= 33,
               "reverse_slots: bad key fields (%d + %d bits)", q_bits, slot_bits);
  const TokenLayout tl = token_layout(global_token != 0, token_row, n_q);
  const int64_t n_token = tl.tok ? tl.c0 + tl.token_len : 0;
  const int64_t n_keys = nnz - n_token;     // a capacity, as in bf_reverse_index_packed
  BF_CHECK_ARG(n_keys >= 0, "reverse_slots: %lld entries cannot hold the token's %lld", (long long)nnz,
               (long long)(tl.c0 + tl.token_len));
  if (nnz == 0) return BF_OK;
  BF_CHECK_ARG(ks && (n_keys == 0 || sorted), "reverse_slots: null tensor");
  hipStream_t st = as_stream(stream);
  if (n_keys > 0 || tl.lead) {
    BF_LAUNCH("reverse_slots_kernel", reverse_slots_kernel, dim3(blocks_for(n_keys + 1)), dim3(kThreads), 0, st,
              sorted, qptr + n_q, n_token, n_keys, q_bits + slot_bits, slot_bits, tl, ks);
    BF_CHECK_LAUNCH();
  }
  return launch_token_reverse(tl, nullptr, ks, st);
}

extern "C" int bf_expand_rows(const int64_t* ptr, int64_t n_rows, int64_t nnz, int64_t* rows, void* stream) {
  BF_CHECK_ARG(ptr && n_rows >= 0 && nnz >= 0 && (rows || nnz == 0), "expand_rows: bad arguments");
  BF_CHECK_ARG(nnz == 0 || n_rows > 0, "expand_rows: entries without rows");
  if (nnz == 0) return BF_OK;
  BF_LAUNCH("expand_rows_kernel", expand_rows_kernel<int64_t>, dim3(blocks_for(nnz)), dim3(kThreads), 0, as_stream(stream),
                     ptr, n_rows, nnz, rows);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int64_t bf_split_item_capacity(int64_t nnz, int32_t threshold, int32_t item_size) {
  if (threshold < 1 || item_size < 1 || nnz < 0) return 0;
  // only rows longer than threshold split: sum ceil(len/item) <= nnz/item + #heavy rows
  return nnz / item_size + nnz / threshold + 1;
}

extern "C" int64_t bf_split_row_items(int64_t len, int32_t item_size) {
  if (len <= 0 || item_size < 1) return 0;
  return split_row_items(len, item_size);
}

extern "C" int64_t bf_split_row_capacity(int64_t nnz, int32_t threshold) {
  if (threshold < 1 || nnz < 0) return 0;
  return nnz / threshold + 1;
}

extern "C" int bf_split_plan_workspace_size(int64_t n_rows, size_t* bytes) {
  BF_CHECK_ARG(bytes && n_rows >= 0, "split_plan_workspace_size: bad arguments");
  size_t temp_bytes = 0;
  (void)prim::exclusive_sum(nullptr, temp_bytes, static_cast<const uint64_t*>(nullptr),
                            static_cast<uint64_t*>(nullptr), n_rows > 0 ? n_rows : 1, hipStream_t(nullptr));
  *bytes = 2 * align_up(size_t(n_rows > 0 ? n_rows : 1) * 8) + align_up(temp_bytes) + 256;
  return BF_OK;
}

extern "C" int bf_split_plan(const int64_t* ptr, int64_t n_rows, int32_t threshold, int32_t item_size,
                             int32_t* nitems, int32_t* item_off, int32_t* item_row, int64_t item_cap,
                             int32_t* heavy_rows, int64_t heavy_cap, int32_t* counts, void* workspace,
                             size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(ptr && n_rows >= 0 && threshold >= 1 && item_size >= 1 && counts, "split_plan: bad arguments");
  BF_CHECK_ARG(item_cap >= 0 && item_cap < (int64_t(1) << 31) && heavy_cap >= 0 && heavy_cap < (int64_t(1) << 31),
               "split_plan: bad capacity");
  BF_CHECK_ARG(n_rows < (int64_t(1) << 31), "split_plan: too many rows");
  hipStream_t st = as_stream(stream);
  if (n_rows == 0) {
    BF_CHECK_HIP(hipMemsetAsync(counts, 0, 2 * sizeof(int32_t), st));
    return BF_OK;
  }
  BF_CHECK_ARG(nitems && item_off && (item_row || item_cap == 0) && (heavy_rows || heavy_cap == 0),
               "split_plan: null tensor");
  size_t need = 0;
  bf_split_plan_workspace_size(n_rows, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "split_plan: workspace %zu < %zu bytes", workspace_bytes, need);
  const size_t slab = align_up(size_t(n_rows) * 8);
  auto* packed = static_cast<uint64_t*>(workspace);
  auto* packed_off = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + slab);
  void* temp = static_cast<char*>(workspace) + 2 * slab;
  size_t temp_bytes = 0;
  (void)prim::exclusive_sum(nullptr, temp_bytes, static_cast<const uint64_t*>(packed), packed_off, n_rows, st);
  BF_LAUNCH("split_count_kernel", split_count_kernel, dim3(blocks_for(n_rows)), dim3(kThreads), 0, st, ptr, n_rows,
            threshold, item_size, packed);
  BF_CHECK_LAUNCH();
  const bool in_block = n_rows <= kPlanInBlockSlots;
  if (!in_block)
    BF_CHECK_HIP(prim::exclusive_sum(temp, temp_bytes, static_cast<const uint64_t*>(packed), packed_off, n_rows,
                                     st));
  BF_LAUNCH("split_rows_kernel", split_rows_kernel, dim3(blocks_for(n_rows)), dim3(kThreads), 0, st, packed,
            in_block ? nullptr : packed_off, static_cast<const int32_t*>(nullptr), n_rows, item_cap, nitems,
            item_off, item_row, heavy_rows, heavy_cap, counts);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int bf_split_plan_first_row(int64_t n_rows, int32_t n_items, int32_t* nitems, int32_t* item_off,
                                       int32_t* item_row, int64_t item_cap, int32_t* heavy_rows, int64_t heavy_cap,
                                       int32_t* counts, void* stream) {
  BF_CHECK_ARG(n_rows >= 0 && n_rows < (int64_t(1) << 31) && n_items >= 0 && counts && (n_items == 0 || n_rows > 0),
               "split_plan_first_row: bad arguments");
  BF_CHECK_ARG(item_cap >= n_items && heavy_cap >= (n_items ? 1 : 0), "split_plan_first_row: capacity too small");
  BF_CHECK_ARG(n_rows == 0 || (nitems && item_off), "split_plan_first_row: null tensor");
  BF_CHECK_ARG(n_items == 0 || (item_row && heavy_rows), "split_plan_first_row: null tensor");
  const int64_t threads = n_rows > 1 ? n_rows : 1;
  BF_LAUNCH("split_first_row_kernel", split_first_row_kernel, dim3(blocks_for(threads)), dim3(kThreads), 0,
            as_stream(stream), n_rows, n_items, nitems, item_off, item_row, heavy_rows, counts);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

// ---------------------------------------------------------------- hop pool and coalesce
namespace bf {
namespace {

// Hop pool flags in pool order (d-major, then walk): entry (d, w) is kept iff
// walks[w, d] >= 0 and (d == 1 or walks[w, d] != walks[w, d-1]).
__global__ void hop_flags_kernel(const int64_t* __restrict__ walks, int64_t n_walks,
                                                             int L, int min_hop, int32_t* __restrict__ flags) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int D = L - min_hop + 1;
  if (i >= n_walks * D) return;
  const int d = min_hop + int(i / n_walks);
  const int64_t w = i % n_walks;
  const int64_t kv = walks[w * (L + 1) + d];
  flags[i] = (kv >= 0 && (d == 1 || kv != walks[w * (L + 1) + d - 1])) ? 1 : 0;
}

__global__ void hop_fill_kernel(const int64_t* __restrict__ walks, int64_t n_walks,
                                                            int L, int min_hop, const int32_t* __restrict__ flags,
                                                            const int64_t* __restrict__ pos,
                                                            int64_t* __restrict__ pool_kv,
                                                            int64_t* __restrict__ pool_q) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int D = L - min_hop + 1;
  if (i >= n_walks * D || !flags[i]) return;
  const int d = min_hop + int(i / n_walks);
  const int64_t w = i % n_walks;
  pool_kv[pos[i]] = walks[w * (L + 1) + d];
  pool_q[pos[i]] = walks[w * (L + 1)];
}

__global__ void i32_to_i64_kernel(const int32_t* __restrict__ a, int64_t n, int64_t* __restrict__ b) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n) b[i] = a[i];
}

__global__ void coalesce_keys_kernel(const int64_t* __restrict__ src, const int64_t* __restrict__ dst, int64_t nnz,
                                     uint64_t n, uint64_t* __restrict__ keys) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i < nnz) keys[i] = uint64_t(src[i]) * n + uint64_t(dst[i]);
}

__global__ void unique_flags_kernel(const uint64_t* __restrict__ keys, int64_t nnz, int64_t* __restrict__ flags) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i < nnz) flags[i] = (i == 0 || keys[i] != keys[i - 1]) ? 1 : 0;
}

__global__ void unique_fill_kernel(const uint64_t* __restrict__ keys, const int64_t* __restrict__ incl, int64_t nnz,
                                   uint64_t n, int64_t* __restrict__ out_src, int64_t* __restrict__ out_dst) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= nnz) return;
  if (i == 0 || keys[i] != keys[i - 1]) {
    const int64_t p = incl[i] - 1;
    out_src[p] = int64_t(keys[i] / n);
    out_dst[p] = int64_t(keys[i] % n);
  }
}

}  // namespace
}  // namespace bf

extern "C" int bf_hop_pool_workspace_size(int64_t n_walks, int32_t walk_length, int32_t min_hop, size_t* bytes) {
  BF_CHECK_ARG(bytes && n_walks >= 0 && walk_length >= 1 && min_hop >= 1, "hop_pool_workspace_size: bad arguments");
  const int64_t m = n_walks * (min_hop <= walk_length ? walk_length - min_hop + 1 : 0);
  size_t scan_bytes = 0;
  (void)prim::exclusive_sum(nullptr, scan_bytes, static_cast<const int64_t*>(nullptr), static_cast<int64_t*>(nullptr),
                            m > 0 ? m : 1, hipStream_t(nullptr));
  *bytes = align_up(size_t(m > 0 ? m : 1) * 4) + 2 * align_up(size_t(m > 0 ? m : 1) * 8) + align_up(scan_bytes) + 256;
  return BF_OK;
}

extern "C" int bf_hop_pool(const int64_t* walks, int64_t n_walks, int32_t walk_length, int32_t min_hop,
                           int64_t* pool_kv, int64_t* pool_q, int64_t* count_host, void* workspace,
                           size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(count_host && n_walks >= 0 && walk_length >= 1 && min_hop >= 1, "hop_pool: bad arguments");
  *count_host = 0;
  if (min_hop > walk_length || n_walks == 0) return BF_OK;
  const int64_t m = n_walks * (walk_length - min_hop + 1);
  BF_CHECK_ARG(m < (int64_t(1) << 31), "hop_pool: %lld candidates exceed int32 scan range", (long long)m);
  BF_CHECK_ARG(walks && pool_kv && pool_q, "hop_pool: null tensor");
  size_t need = 0;
  bf_hop_pool_workspace_size(n_walks, walk_length, min_hop, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "hop_pool: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  auto* flags = static_cast<int32_t*>(workspace);
  auto* flags64 = reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + align_up(size_t(m) * 4));
  auto* pos = reinterpret_cast<int64_t*>(reinterpret_cast<char*>(flags64) + align_up(size_t(m) * 8));
  void* temp = reinterpret_cast<char*>(pos) + align_up(size_t(m) * 8);
  size_t temp_bytes = 0;
  (void)prim::exclusive_sum(nullptr, temp_bytes, static_cast<const int64_t*>(flags64), pos, m, st);
  BF_LAUNCH("hop_flags_kernel", hop_flags_kernel, dim3(blocks_for(m)), dim3(kThreads), 0, st, walks, n_walks,
            walk_length, min_hop, flags);
  BF_CHECK_LAUNCH();
  BF_LAUNCH("i32_to_i64_kernel", i32_to_i64_kernel, dim3(blocks_for(m)), dim3(kThreads), 0, st, flags, m, flags64);
  BF_CHECK_LAUNCH();
  BF_CHECK_HIP(prim::exclusive_sum(temp, temp_bytes, static_cast<const int64_t*>(flags64), pos, m, st));
  BF_LAUNCH("hop_fill_kernel", hop_fill_kernel, dim3(blocks_for(m)), dim3(kThreads), 0, st, walks, n_walks,
            walk_length, min_hop, flags, pos, pool_kv, pool_q);
  BF_CHECK_LAUNCH();
  int64_t last_pos = 0;
  int32_t last_flag = 0;
  BF_CHECK_HIP(hipMemcpyAsync(&last_pos, pos + m - 1, sizeof(last_pos), hipMemcpyDeviceToHost, st));
  BF_CHECK_HIP(hipMemcpyAsync(&last_flag, flags + m - 1, sizeof(last_flag), hipMemcpyDeviceToHost, st));
  BF_CHECK_HIP(hipStreamSynchronize(st));
  *count_host = last_pos + last_flag;
  return BF_OK;
}

extern "C" int bf_coalesce_workspace_size(int64_t nnz, size_t* bytes) {
  BF_CHECK_ARG(bytes && nnz >= 0, "coalesce_workspace_size: bad arguments");
  const int64_t n = nnz > 0 ? nnz : 1;
  size_t sort_bytes = 0, scan_bytes = 0;
  (void)prim::sort_keys(nullptr, sort_bytes, static_cast<const uint64_t*>(nullptr), static_cast<uint64_t*>(nullptr),
                        n, 0, 64, hipStream_t(nullptr));
  (void)prim::inclusive_sum(nullptr, scan_bytes, static_cast<const int64_t*>(nullptr), static_cast<int64_t*>(nullptr),
                            n, hipStream_t(nullptr));
  *bytes = 4 * align_up(size_t(n) * 8) + align_up(sort_bytes > scan_bytes ? sort_bytes : scan_bytes) + 256;
  return BF_OK;
}

extern "C" int bf_coalesce(const int64_t* src, const int64_t* dst, int64_t nnz, int64_t num_nodes, int64_t* out_src,
                           int64_t* out_dst, int64_t* count_host, void* workspace, size_t workspace_bytes,
                           void* stream) {
  BF_CHECK_ARG(count_host && nnz >= 0 && num_nodes > 0, "coalesce: bad arguments");
  BF_CHECK_ARG(nnz < (int64_t(1) << 31) && num_nodes < (int64_t(1) << 32), "coalesce: sizes out of range");
  *count_host = 0;
  if (nnz == 0) return BF_OK;
  BF_CHECK_ARG(src && dst && out_src && out_dst, "coalesce: null tensor");
  size_t need = 0;
  bf_coalesce_workspace_size(nnz, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "coalesce: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  const size_t slab = align_up(size_t(nnz) * 8);
  auto* keys_in = static_cast<uint64_t*>(workspace);
  auto* keys = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + slab);
  auto* flags = reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + 2 * slab);
  auto* incl = reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + 3 * slab);
  void* temp = static_cast<char*>(workspace) + 4 * slab;
  size_t sort_bytes = 0, scan_bytes = 0;
  (void)prim::sort_keys(nullptr, sort_bytes, static_cast<const uint64_t*>(keys_in), keys, nnz, 0, 64, st);
  (void)prim::inclusive_sum(nullptr, scan_bytes, static_cast<const int64_t*>(flags), incl, nnz, st);
  BF_LAUNCH("coalesce_keys_kernel", coalesce_keys_kernel, dim3(blocks_for(nnz)), dim3(kThreads), 0, st, src, dst, nnz,
            uint64_t(num_nodes), keys_in);
  BF_CHECK_LAUNCH();
  const int end_bit = bits_for(uint64_t(num_nodes) * uint64_t(num_nodes));
  BF_CHECK_HIP(prim::sort_keys(temp, sort_bytes, static_cast<const uint64_t*>(keys_in), keys, nnz, 0, end_bit, st));
  BF_LAUNCH("unique_flags_kernel", unique_flags_kernel, dim3(blocks_for(nnz)), dim3(kThreads), 0, st, keys, nnz, flags);
  BF_CHECK_LAUNCH();
  BF_CHECK_HIP(prim::inclusive_sum(temp, scan_bytes, static_cast<const int64_t*>(flags), incl, nnz, st));
  BF_LAUNCH("unique_fill_kernel", unique_fill_kernel, dim3(blocks_for(nnz)), dim3(kThreads), 0, st, keys, incl, nnz,
            uint64_t(num_nodes), out_src, out_dst);
  BF_CHECK_LAUNCH();
  BF_CHECK_HIP(hipMemcpyAsync(count_host, incl + nnz - 1, sizeof(int64_t), hipMemcpyDeviceToHost, st));
  BF_CHECK_HIP(hipStreamSynchronize(st));
  return BF_OK;
}

namespace {
// The order kernels' per-block bucket counts and bucket totals, then (plans
// only) the slots' packed counts, their exclusive sums and the scan's
// temporary storage.
int64_t order_blocks(int64_t n_rows) { return ceil_div(n_rows > 0 ? n_rows : 1, kOrderRows); }

size_t order_counts_bytes(int64_t n_rows) {
  return align_up(size_t(order_blocks(n_rows)) * kBuckets * sizeof(uint32_t)) + align_up(kBuckets * sizeof(uint32_t));
}

size_t plan_slots_scan_bytes(int64_t n_slots) {
  size_t temp_bytes = 0;
  (void)prim::exclusive_sum(nullptr, temp_bytes, static_cast<const uint64_t*>(nullptr),
                            static_cast<uint64_t*>(nullptr), n_slots > 0 ? n_slots : 1, hipStream_t(nullptr));
  return temp_bytes;
}

int launch_row_order(const int64_t* ptr, int64_t n_rows, int32_t* order, uint64_t* spans, void* ws,
                     int threshold, int item_size, int64_t n_slots, uint64_t* packed, hipStream_t st) {
  const int64_t blocks = order_blocks(n_rows);
  auto* counts = static_cast<uint32_t*>(ws);
  auto* totals = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) +
                                             align_up(size_t(blocks) * kBuckets * sizeof(uint32_t)));
  BF_LAUNCH("order_count_kernel", order_count_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0, st, ptr, n_rows,
            blocks, counts);
  BF_CHECK_LAUNCH();
  BF_LAUNCH("radix_scan_kernel", sort::radix_scan_kernel, dim3(kBuckets), dim3(kThreads), 0, st, counts, blocks,
            totals);
  BF_CHECK_LAUNCH();
  BF_LAUNCH("order_place_kernel", order_place_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0, st, ptr, n_rows,
            blocks, counts, totals, order, spans, threshold, item_size, n_slots, packed);
  BF_CHECK_LAUNCH();
  return BF_OK;
}
}  // namespace

extern "C" int bf_row_order_workspace_size(int64_t n_rows, size_t* bytes) {
  BF_CHECK_ARG(bytes && n_rows >= 0, "row_order_workspace_size: bad arguments");
  *bytes = order_counts_bytes(n_rows) + 256;
  return BF_OK;
}

extern "C" int bf_row_order(const int64_t* ptr, int64_t n_rows, int32_t* order, uint64_t* spans, void* workspace,
                            size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(ptr && n_rows >= 0 && n_rows < (int64_t(1) << 31), "row_order: bad arguments");
  if (n_rows == 0) return BF_OK;
  BF_CHECK_ARG(order != nullptr, "row_order: null output");
  size_t need = 0;
  bf_row_order_workspace_size(n_rows, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "row_order: workspace %zu < %zu bytes", workspace_bytes, need);
  return launch_row_order(ptr, n_rows, order, spans, workspace, 0, 1, 0, nullptr, as_stream(stream));
}

extern "C" int bf_row_order_and_plan_workspace_size(int64_t n_rows, int64_t heavy_cap, size_t* bytes) {
  BF_CHECK_ARG(bytes && n_rows >= 0 && heavy_cap >= 0, "row_order_and_plan_workspace_size: bad arguments");
  const int64_t n_slots = heavy_cap < n_rows ? heavy_cap : n_rows;
  const size_t slab = align_up(size_t(n_slots > 0 ? n_slots : 1) * 8);
  *bytes = order_counts_bytes(n_rows) + 2 * slab + align_up(plan_slots_scan_bytes(n_slots)) + 256;
  return BF_OK;
}

extern "C" int bf_row_order_and_plan(const int64_t* ptr, int64_t n_rows, int32_t threshold, int32_t item_size,
                                     int32_t* order, uint64_t* spans, int32_t* nitems, int32_t* item_off,
                                     int32_t* item_row, int64_t item_cap, int32_t* heavy_rows, int64_t heavy_cap,
                                     int32_t* counts, void* workspace, size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(ptr && n_rows >= 0 && n_rows < (int64_t(1) << 31) && counts, "row_order_and_plan: bad arguments");
  BF_CHECK_ARG(threshold >= 1 && threshold < 255 && item_size >= 1,
               "row_order_and_plan: threshold must lie in [1, 254] and item_size be >= 1");
  BF_CHECK_ARG(item_cap >= 0 && item_cap < (int64_t(1) << 31) && heavy_cap >= 1 && heavy_cap < (int64_t(1) << 31),
               "row_order_and_plan: bad capacity");
  hipStream_t st = as_stream(stream);
  if (n_rows == 0) {
    BF_CHECK_HIP(hipMemsetAsync(counts, 0, 2 * sizeof(int32_t), st));
    return BF_OK;
  }
  BF_CHECK_ARG(order && nitems && item_off && (item_row || item_cap == 0) && heavy_rows,
               "row_order_and_plan: null tensor");
  size_t need = 0;
  bf_row_order_and_plan_workspace_size(n_rows, heavy_cap, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "row_order_and_plan: workspace %zu < %zu bytes",
               workspace_bytes, need);
  // Rows longer than the threshold (< 255) have the highest capped lengths, so
  // the order puts them in its first slots, and there are at most heavy_cap of
  // them: the plan needs only the first n_slots slots.
  const int64_t n_slots = heavy_cap < n_rows ? heavy_cap : n_rows;
  const size_t slab = align_up(size_t(n_slots) * 8);
  char* ws = static_cast<char*>(workspace);
  const size_t ob = order_counts_bytes(n_rows);
  auto* packed = reinterpret_cast<uint64_t*>(ws + ob);
  auto* packed_off = reinterpret_cast<uint64_t*>(ws + ob + slab);
  void* temp = ws + ob + 2 * slab;
  size_t temp_bytes = plan_slots_scan_bytes(n_slots);
  const int rc = launch_row_order(ptr, n_rows, order, spans, ws, threshold, item_size, n_slots, packed, st);
  if (rc) return rc;
  // few slots: split_rows_kernel sums the slots before its block itself, with no scan launch
  const bool in_block = n_slots <= kPlanInBlockSlots;
  if (!in_block)
    BF_CHECK_HIP(prim::exclusive_sum(temp, temp_bytes, static_cast<const uint64_t*>(packed), packed_off, n_slots,
                                     st));
  BF_LAUNCH("split_rows_kernel", split_rows_kernel, dim3(blocks_for(n_slots)), dim3(kThreads), 0, st, packed,
            in_block ? nullptr : packed_off, order, n_slots, item_cap, nitems, item_off, item_row, heavy_rows,
            heavy_cap, counts);
  BF_CHECK_LAUNCH();
  return BF_OK;
}
