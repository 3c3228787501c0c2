// Gather-rate calibration: how fast MI355X serves the attention passes' row
// gathers, on each pass's own order of ids, with no arithmetic. No reference
// counterpart. It plays the part a plain copy kernel plays for streaming
// bandwidth: a kernel that only moves the bytes, against which a pass that
// also computes is judged. Random row gathers do not reach the 8 TB/s of a
// stream (a 128-byte line per request, scattered over the DRAM pages), so a
// gathering pass's fraction of HBM peak says little on its own; its time
// against this floor says how much of it is the gathers themselves.
//
// Id e reads row ids[e] & id_mask of up to three tables (rows of 16 to 512
// bytes, 16-byte aligned, the row stride equal to the row size) with 16-byte
// loads by a group of G lanes (the widest row's 16-byte chunks, rounded up to
// a power of two), non-temporal when asked, as the key-major pass gathers
// tables larger than the Infinity Cache. Each lane folds the words it loads
// into one value that is written (to `sink`, atomically) only when it equals
// a constant the fold practically never produces, so the compiler keeps every
// load and the kernel writes nothing.
#include "bf_common.h"

namespace bf {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kSinkMatch = 0x9e3779b9u;
constexpr int64_t kMaxBlocks = int64_t(1) << 16;   // 16.7M lanes: fills the chip, far below 2^32 work-items
constexpr int kUnroll = 4;                          // ids a lane has in flight
typedef unsigned int V4u __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ uint32_t fold_row(const V4u* __restrict__ tab, int64_t row, int chunks, int j, int g) {
  uint32_t acc = 0;
  for (int k = j; k < chunks; k += g) {
    const V4u* p = tab + row * chunks + k;
    const V4u v = NT ? __builtin_nontemporal_load(p) : *p;
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  return acc;
}

// Grid-stride over the ids: a dispatch counts its work-items in 32 bits, so the grid is capped
// (kMaxBlocks) and a lane group takes every (gridDim.x * kThreads / G)-th id, kUnroll at a time; G
// divides kThreads, so a lane keeps its place j in its group.
template <int G, bool NT>
__global__ __launch_bounds__(kThreads) void gather_probe_kernel(const V4u* __restrict__ t0, const V4u* __restrict__ t1,
                                                                const V4u* __restrict__ t2, int c0, int c1, int c2,
                                                                const int32_t* __restrict__ ids, int64_t n,
                                                                uint32_t id_mask, uint32_t* __restrict__ sink) {
  const int j = int(threadIdx.x % G);
  const int64_t stride = int64_t(gridDim.x) * (kThreads / G);
  uint32_t acc = 0;
  for (int64_t e = (int64_t(blockIdx.x) * kThreads + threadIdx.x) / G; e < n; e += kUnroll * stride) {
    // kUnroll ids, then all their rows: the loads of kUnroll ids in flight at once
    int64_t row[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t eu = e + u * stride;
      row[u] = eu < n ? int64_t(uint32_t(ids[eu]) & id_mask) : -1;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (row[u] < 0) continue;
      if (t0) acc ^= fold_row<NT>(t0, row[u], c0, j, G);
      if (t1) acc ^= fold_row<NT>(t1, row[u], c1, j, G);
      if (t2) acc ^= fold_row<NT>(t2, row[u], c2, j, G);
    }
  }
  if (acc == kSinkMatch) atomicXor(sink, acc);
}

// Row streams: id e (row ids[e], or row e when ids is NULL) reads that row of
// r0 and r1 and writes zeros over it in w0 and w1 (non-temporal stores, as the
// passes write their outputs), G lanes of 16 bytes per row: the rows a pass
// reads and writes once each, in its own order, without its gathers or its
// arithmetic. Same grid-stride and sink as the gather probe.
template <int G, bool NT>
__global__ __launch_bounds__(kThreads) void row_stream_probe_kernel(const V4u* __restrict__ r0,
                                                                    const V4u* __restrict__ r1, V4u* __restrict__ w0,
                                                                    V4u* __restrict__ w1, int chunks,
                                                                    const int32_t* __restrict__ ids, int64_t n,
                                                                    uint32_t* __restrict__ sink) {
  const int j = int(threadIdx.x % G);
  const int64_t stride = int64_t(gridDim.x) * (kThreads / G);
  const V4u zero = {0u, 0u, 0u, 0u};
  uint32_t acc = 0;
  for (int64_t e = (int64_t(blockIdx.x) * kThreads + threadIdx.x) / G; e < n; e += kUnroll * stride) {
    int64_t row[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t eu = e + u * stride;
      row[u] = eu < n ? (ids ? int64_t(ids[eu]) : eu) : -1;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (row[u] < 0) continue;
      if (r0) acc ^= fold_row<NT>(r0, row[u], chunks, j, G);
      if (r1) acc ^= fold_row<NT>(r1, row[u], chunks, j, G);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (row[u] < 0) continue;
      for (int k = j; k < chunks; k += G) {
        if (w0) __builtin_nontemporal_store(zero, w0 + row[u] * chunks + k);
        if (w1) __builtin_nontemporal_store(zero, w1 + row[u] * chunks + k);
      }
    }
  }
  if (acc == kSinkMatch) atomicXor(sink, acc);
}

template <int G>
int launch_stream(bool nt, dim3 grid, hipStream_t st, const V4u* r0, const V4u* r1, V4u* w0, V4u* w1, int chunks,
                  const int32_t* ids, int64_t n, uint32_t* sink) {
  if (nt)
    BF_LAUNCH("row_stream_probe_kernel", (row_stream_probe_kernel<G, true>), grid, dim3(kThreads), 0, st, r0, r1, w0,
              w1, chunks, ids, n, sink);
  else
    BF_LAUNCH("row_stream_probe_kernel", (row_stream_probe_kernel<G, false>), grid, dim3(kThreads), 0, st, r0, r1,
              w0, w1, chunks, ids, n, sink);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

template <int G>
int launch_probe(bool nt, dim3 grid, hipStream_t st, const V4u* t0, const V4u* t1, const V4u* t2, int c0, int c1,
                 int c2, const int32_t* ids, int64_t n, uint32_t id_mask, uint32_t* sink) {
  if (nt)
    BF_LAUNCH("gather_probe_kernel", (gather_probe_kernel<G, true>), grid, dim3(kThreads), 0, st, t0, t1, t2, c0, c1,
              c2, ids, n, id_mask, sink);
  else
    BF_LAUNCH("gather_probe_kernel", (gather_probe_kernel<G, false>), grid, dim3(kThreads), 0, st, t0, t1, t2, c0, c1,
              c2, ids, n, id_mask, sink);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

}  // namespace
}  // namespace bf

using namespace bf;

extern "C" int bf_gather_probe(const void* t0, int32_t row_bytes0, const void* t1, int32_t row_bytes1,
                               const void* t2, int32_t row_bytes2, const int32_t* ids, int64_t n_ids,
                               uint32_t id_mask, int32_t nontemporal, uint32_t* sink, void* stream) {
  const void* tabs[3] = {t0, t1, t2};
  const int32_t rb[3] = {row_bytes0, row_bytes1, row_bytes2};
  int widest = 0;
  for (int i = 0; i < 3; ++i) {
    if (!tabs[i]) continue;
    BF_CHECK_ARG(rb[i] >= 16 && rb[i] <= 512 && rb[i] % 16 == 0, "gather_probe: row of %d bytes (16..512, a multiple "
                 "of 16)", rb[i]);
    BF_CHECK_ARG((reinterpret_cast<uintptr_t>(tabs[i]) & 15) == 0, "gather_probe: table %d is not 16-byte aligned", i);
    widest = rb[i] > widest ? rb[i] : widest;
  }
  BF_CHECK_ARG(widest > 0, "gather_probe: no table");
  BF_CHECK_ARG(n_ids >= 0 && (ids || n_ids == 0) && sink, "gather_probe: bad ids or sink");
  if (n_ids == 0) return BF_OK;
  int g = 1;
  while (g * 16 < widest) g <<= 1;
  const int64_t need = ceil_div(n_ids * g, int64_t(kThreads));
  const dim3 grid{unsigned(need < kMaxBlocks ? need : kMaxBlocks)};
  const V4u* p0 = static_cast<const V4u*>(t0);
  const V4u* p1 = static_cast<const V4u*>(t1);
  const V4u* p2 = static_cast<const V4u*>(t2);
  const int c0 = t0 ? row_bytes0 / 16 : 0, c1 = t1 ? row_bytes1 / 16 : 0, c2 = t2 ? row_bytes2 / 16 : 0;
  hipStream_t st = as_stream(stream);
  const bool nt = nontemporal != 0;
  switch (g) {
    case 1: return launch_probe<1>(nt, grid, st, p0, p1, p2, c0, c1, c2, ids, n_ids, id_mask, sink);
    case 2: return launch_probe<2>(nt, grid, st, p0, p1, p2, c0, c1, c2, ids, n_ids, id_mask, sink);
    case 4: return launch_probe<4>(nt, grid, st, p0, p1, p2, c0, c1, c2, ids, n_ids, id_mask, sink);
    case 8: return launch_probe<8>(nt, grid, st, p0, p1, p2, c0, c1, c2, ids, n_ids, id_mask, sink);
    case 16: return launch_probe<16>(nt, grid, st, p0, p1, p2, c0, c1, c2, ids, n_ids, id_mask, sink);
    default: return launch_probe<32>(nt, grid, st, p0, p1, p2, c0, c1, c2, ids, n_ids, id_mask, sink);
  }
}

extern "C" int bf_row_stream_probe(const void* r0, const void* r1, void* w0, void* w1, int32_t row_bytes,
                                   const int32_t* ids, int64_t n_rows, int32_t nontemporal, uint32_t* sink,
                                   void* stream) {
  const void* tabs[4] = {r0, r1, w0, w1};
  bool any = false;
  for (int i = 0; i < 4; ++i) {
    if (!tabs[i]) continue;
    any = true;
    BF_CHECK_ARG((reinterpret_cast<uintptr_t>(tabs[i]) & 15) == 0, "row_stream_probe: table %d is not 16-byte "
                 "aligned", i);
  }
  BF_CHECK_ARG(any, "row_stream_probe: no table");
  BF_CHECK_ARG(row_bytes >= 16 && row_bytes <= 1024 && row_bytes % 16 == 0, "row_stream_probe: row of %d bytes "
               "(16..1024, a multiple of 16)", row_bytes);
  BF_CHECK_ARG(n_rows >= 0 && sink, "row_stream_probe: bad row count or sink");
  if (n_rows == 0) return BF_OK;
  const int chunks = row_bytes / 16;
  int g = 1;
  while (g < chunks) g <<= 1;
  const int64_t need = ceil_div(n_rows * g, int64_t(kThreads));
  const dim3 grid{unsigned(need < kMaxBlocks ? need : kMaxBlocks)};
  const V4u* p0 = static_cast<const V4u*>(r0);
  const V4u* p1 = static_cast<const V4u*>(r1);
  V4u* q0 = static_cast<V4u*>(w0);
  V4u* q1 = static_cast<V4u*>(w1);
  hipStream_t st = as_stream(stream);
  const bool nt = nontemporal != 0;
  switch (g) {
    case 1: return launch_stream<1>(nt, grid, st, p0, p1, q0, q1, chunks, ids, n_rows, sink);
    case 2: return launch_stream<2>(nt, grid, st, p0, p1, q0, q1, chunks, ids, n_rows, sink);
    case 4: return launch_stream<4>(nt, grid, st, p0, p1, q0, q1, chunks, ids, n_rows, sink);
    case 8: return launch_stream<8>(nt, grid, st, p0, p1, q0, q1, chunks, ids, n_rows, sink);
    case 16: return launch_stream<16>(nt, grid, st, p0, p1, q0, q1, chunks, ids, n_rows, sink);
    case 32: return launch_stream<32>(nt, grid, st, p0, p1, q0, q1, chunks, ids, n_rows, sink);
    default: return launch_stream<64>(nt, grid, st, p0, p1, q0, q1, chunks, ids, n_rows, sink);
  }
}
