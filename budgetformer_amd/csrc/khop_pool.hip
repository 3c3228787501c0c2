// Fanout k-hop pool: the "dgl_neighbor" alternative to the random-walk pool
// (compute_khop_pool_dgl_neighbor, gt_sp/utils.py:1281-1384).
//
// Every node starts a frontier entry (origin u, node u). Hop d replaces each
// entry (o, c) by (o, s) for each s in node c's hop-d sample of out-neighbours
// (one sample per node and hop, shared by every entry at that node) and, from
// min_hop on, emits the pool pair (s -> o) for s != o. The host runs the hops:
// per hop one sample kernel, an offsets scan over the frontier, an expand
// kernel and a compaction of the emitted pairs.
//
// The sample: a node whose out-degree is at most the fanout keeps all its
// out-neighbours in CSR order; otherwise Floyd's algorithm draws `fanout`
// distinct indices of [0, deg) from Philox words (counter = (u, offset + hop *
// 2^32 + i / 4), key = seed; word i % 4, mapped to [0, j] by a 32x32 high
// product), kept in ascending index order. DGL's own sampler RNG cannot be
// reproduced outside DGL; the order of the sample does not matter downstream,
// where a pool is ranked per query by the edge key.
#include "bf_common.h"
#include "bf_prim.h"

namespace bf {
namespace {

constexpr int kThreads = 256;
constexpr int kSampleThreads = 64;   // one node per thread; LDS holds each thread's draws

inline unsigned blocks_for(int64_t n) { return unsigned(ceil_div(n, kThreads)); }
inline size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

__global__ __launch_bounds__(kSampleThreads) void fanout_sample_kernel(const int64_t* __restrict__ rowptr,
                                                                       const int32_t* __restrict__ col,
                                                                       int64_t n, int f, uint32_t hop,
                                                                       uint64_t seed, uint64_t offset,
                                                                       int32_t* __restrict__ cnt,
                                                                       int32_t* __restrict__ sel) {
  extern __shared__ int32_t draws[];   // f slots per thread
  const int64_t u = int64_t(blockIdx.x) * kSampleThreads + threadIdx.x;
  if (u >= n) return;
  const int64_t beg = rowptr[u];
  const int64_t deg = rowptr[u + 1] - beg;
  int32_t* out = sel + u * f;
  if (deg <= f) {
    for (int64_t i = 0; i < deg; ++i) out[i] = col[beg + i];
    cnt[u] = int32_t(deg);
    return;
  }
  int32_t* chosen = draws + threadIdx.x * f;
  U32x4 r{0u, 0u, 0u, 0u};
  for (int i = 0; i < f; ++i) {
    if ((i & 3) == 0) {
      const uint64_t b = offset + (uint64_t(hop) << 32) + uint64_t(i >> 2);
      r = philox4x32_10(U32x4{uint32_t(uint64_t(u)), uint32_t(uint64_t(u) >> 32), uint32_t(b), uint32_t(b >> 32)},
                        uint32_t(seed), uint32_t(seed >> 32));
    }
    const uint32_t w = (i & 3) == 0 ? r.x : (i & 3) == 1 ? r.y : (i & 3) == 2 ? r.z : r.w;
    const int64_t j = deg - f + i;
    const int32_t t = int32_t((uint64_t(w) * uint64_t(j + 1)) >> 32);
    bool seen = false;
    for (int m = 0; m < i; ++m) seen |= chosen[m] == t;
    chosen[i] = seen ? int32_t(j) : t;
  }
  for (int a = 1; a < f; ++a) {       // ascending index order
    const int32_t x = chosen[a];
    int b = a - 1;
    while (b >= 0 && chosen[b] > x) {
      chosen[b + 1] = chosen[b];
      --b;
    }
    chosen[b + 1] = x;
  }
  for (int i = 0; i < f; ++i) out[i] = col[beg + chosen[i]];
  cnt[u] = f;
}

// counts[i] = the sample size of frontier entry i's node: cnt[c] (a sample table) or ptr[c+1] - ptr[c]
// (all out-neighbours); counts[n] = 0, so an exclusive scan leaves the total there.
__global__ void frontier_counts_kernel(const int32_t* __restrict__ cur, int64_t n, const int64_t* __restrict__ ptr,
                                       const int32_t* __restrict__ cnt, int64_t* __restrict__ counts) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i > n) return;
  if (i == n) {
    counts[n] = 0;
    return;
  }
  const int64_t c = cur[i];
  counts[i] = cnt ? int64_t(cnt[c]) : ptr[c + 1] - ptr[c];
}

// Entry i writes (origin, s) for each s of its node's sample at offsets[i]: from the table row c * stride
// (stride > 0) or the CSR range ptr[c] .. (stride 0).
__global__ void frontier_expand_kernel(const int32_t* __restrict__ origin, const int32_t* __restrict__ cur,
                                       int64_t n, const int64_t* __restrict__ offsets,
                                       const int64_t* __restrict__ ptr, const int32_t* __restrict__ ids,
                                       int32_t stride, int32_t* __restrict__ new_origin,
                                       int32_t* __restrict__ new_cur) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t c = cur[i];
  const int32_t o = origin[i];
  const int64_t src = stride > 0 ? c * stride : ptr[c];
  const int64_t dst = offsets[i];
  const int64_t m = offsets[i + 1] - dst;
  for (int64_t j = 0; j < m; ++j) {
    new_origin[dst + j] = o;
    new_cur[dst + j] = ids[src + j];
  }
}

// flags[i] = 1 when entry i is an edge (node != origin); flags[n] = 0.
__global__ void frontier_flags_kernel(const int32_t* __restrict__ origin, const int32_t* __restrict__ cur, int64_t n,
                                      int64_t* __restrict__ flags) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i > n) return;
  flags[i] = i < n && cur[i] != origin[i] ? 1 : 0;
}

// The flagged entries, in order, as pool pairs: kv[k] = node, q[k] = origin; count[0] = how many.
__global__ void frontier_emit_kernel(const int32_t* __restrict__ origin, const int32_t* __restrict__ cur, int64_t n,
                                     const int64_t* __restrict__ pos, int64_t* __restrict__ kv,
                                     int64_t* __restrict__ q, int64_t* __restrict__ count) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i > n) return;
  if (i == n) {
    count[0] = pos[n];
    return;
  }
  if (cur[i] != origin[i]) {
    const int64_t k = pos[i];
    kv[k] = cur[i];
    q[k] = origin[i];
  }
}

size_t scan_bytes(int64_t n) {
  size_t bytes = 0;
  (void)prim::exclusive_sum(nullptr, bytes, static_cast<const int64_t*>(nullptr), static_cast<int64_t*>(nullptr),
                            n + 1, hipStream_t(nullptr));
  return bytes;
}

}  // namespace
}  // namespace bf

using namespace bf;

extern "C" int bf_fanout_sample(const int64_t* rowptr, const int32_t* col, int64_t num_nodes, int32_t fanout,
                                int32_t hop, uint64_t seed, uint64_t offset, int32_t* cnt, int32_t* sel,
                                void* stream) {
  BF_CHECK_ARG(rowptr && num_nodes >= 0 && num_nodes < (int64_t(1) << 31), "fanout_sample: bad graph");
  BF_CHECK_ARG(fanout >= 1 && fanout <= BF_MAX_FANOUT, "fanout_sample: fanout %d outside [1, %d]", fanout,
               BF_MAX_FANOUT);
  BF_CHECK_ARG(hop >= 0, "fanout_sample: hop %d < 0", hop);
  if (num_nodes == 0) return BF_OK;
  BF_CHECK_ARG(cnt && sel && col, "fanout_sample: null tensor");
  const size_t lds = size_t(kSampleThreads) * size_t(fanout) * sizeof(int32_t);
  BF_LAUNCH("fanout_sample_kernel", fanout_sample_kernel, dim3(unsigned(ceil_div(num_nodes, int64_t(kSampleThreads)))),
            dim3(kSampleThreads), lds, as_stream(stream), rowptr, col, num_nodes, int(fanout), uint32_t(hop), seed,
            offset, cnt, sel);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int bf_frontier_offsets_workspace_size(int64_t n, size_t* bytes) {
  BF_CHECK_ARG(bytes && n >= 0, "frontier_offsets_workspace_size: bad arguments");
  *bytes = align_up(size_t(n + 1) * sizeof(int64_t)) + align_up(scan_bytes(n)) + 256;
  return BF_OK;
}

extern "C" int bf_frontier_offsets(const int32_t* cur, int64_t n, const int64_t* ptr, const int32_t* cnt,
                                   int64_t* offsets, void* workspace, size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(n >= 0 && offsets && (ptr != nullptr) != (cnt != nullptr) && (cur || n == 0),
               "frontier_offsets: bad arguments (exactly one of ptr and cnt)");
  size_t need = 0;
  bf_frontier_offsets_workspace_size(n, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "frontier_offsets: workspace %zu < %zu bytes",
               workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  int64_t* counts = static_cast<int64_t*>(workspace);
  void* temp = static_cast<char*>(workspace) + align_up(size_t(n + 1) * sizeof(int64_t));
  size_t tb = align_up(scan_bytes(n));
  BF_LAUNCH("frontier_counts_kernel", frontier_counts_kernel, dim3(blocks_for(n + 1)), dim3(kThreads), 0, st, cur, n,
            ptr, cnt, counts);
  BF_CHECK_LAUNCH();
  BF_CHECK_HIP(prim::exclusive_sum(temp, tb, counts, offsets, n + 1, st));
  return BF_OK;
}

extern "C" int bf_frontier_expand(const int32_t* origin, const int32_t* cur, int64_t n, const int64_t* offsets,
                                  const int64_t* ptr, const int32_t* ids, int32_t stride, int32_t* new_origin,
                                  int32_t* new_cur, void* stream) {
  BF_CHECK_ARG(n >= 0 && stride >= 0 && (stride > 0 || ptr), "frontier_expand: bad arguments");
  if (n == 0) return BF_OK;
  BF_CHECK_ARG(origin && cur && offsets && ids && new_origin && new_cur, "frontier_expand: null tensor");
  BF_LAUNCH("frontier_expand_kernel", frontier_expand_kernel, dim3(blocks_for(n)), dim3(kThreads), 0,
            as_stream(stream), origin, cur, n, offsets, ptr, ids, stride, new_origin, new_cur);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int bf_frontier_emit_workspace_size(int64_t n, size_t* bytes) {
  BF_CHECK_ARG(bytes && n >= 0, "frontier_emit_workspace_size: bad arguments");
  *bytes = 2 * align_up(size_t(n + 1) * sizeof(int64_t)) + align_up(scan_bytes(n)) + 256;
  return BF_OK;
}

extern "C" int bf_frontier_emit(const int32_t* origin, const int32_t* cur, int64_t n, int64_t* kv, int64_t* q,
                                int64_t* count, void* workspace, size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(n >= 0 && count && (n == 0 || (origin && cur && kv && q)), "frontier_emit: bad arguments");
  size_t need = 0;
  bf_frontier_emit_workspace_size(n, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "frontier_emit: workspace %zu < %zu bytes", workspace_bytes,
               need);
  hipStream_t st = as_stream(stream);
  const size_t region = align_up(size_t(n + 1) * sizeof(int64_t));
  int64_t* flags = static_cast<int64_t*>(workspace);
  int64_t* pos = reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + region);
  void* temp = static_cast<char*>(workspace) + 2 * region;
  size_t tb = align_up(scan_bytes(n));
  BF_LAUNCH("frontier_flags_kernel", frontier_flags_kernel, dim3(blocks_for(n + 1)), dim3(kThreads), 0, st, origin,
            cur, n, flags);
  BF_CHECK_LAUNCH();
  BF_CHECK_HIP(prim::exclusive_sum(temp, tb, flags, pos, n + 1, st));
  BF_LAUNCH("frontier_emit_kernel", frontier_emit_kernel, dim3(blocks_for(n + 1)), dim3(kThreads), 0, st, origin,
            cur, n, pos, kv, q, count);
  BF_CHECK_LAUNCH();
  return BF_OK;
}
