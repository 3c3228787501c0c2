// Budgeted query-centric edge construction for gfx950.
//
// Reference chain (utils/fullgraph_sp_support.py:2943-3026 _build_merged_edges):
//   real part: per dst, the k_real smallest key(src, dst, seed+17) among the
//              graph edges into dst                          (:1312-1491, :1195-1228)
//   RW part:   uniform walks from every node (torch_cluster / DGL, gt_sp/utils.py:
//              1387-1473), hop pool (kv = walks[w,d], q = walks[w,0]) kept iff
//              d == 1 or the walk moved (gt_sp/utils.py:1232-1248), then per q the
//              k_rw smallest key(kv, q, seed+37)             (:1494-1517)
//   merge:     coalesce (set union, src-major) when both parts are non-empty,
//              pass-through otherwise                          (gt_sp/utils.py:877-887)
//
// MI355X design. Every RW pool entry of query q comes from q's own P walks, so
// the pool is never materialised: one lane runs one walk (coalesced rowptr/col
// gathers, Philox counter RNG or injected uniforms), the P lanes of a query
// stage their P*L candidates in LDS and sort them there with a bitonic
// network. The real-edge top-k scans q's in-neighbour list with a 16-lane
// group (per-lane sorted register lists, then rounds of a group min, in batches
// of the list length), and the same group merges both parts through LDS with a
// rank sort (dedup = first occurrence wins) into a fixed-stride int32 table
// row. Keys are 31-bit: an RW candidate (key << 32 | id) orders by key, and
// equal values are the same pair; a real candidate (key << 32 | position)
// orders by (key, position), the reference's tie-break, and its source comes
// back from the key (the key is a bijection of the source for a fixed query).
// Budgets and walk shapes are unbounded: a merged row of up to 768 ids is
// ranked in LDS, a wider one by a workgroup in its own table slots; up to 8191
// walk candidates per query are sorted in LDS, more are selected by a
// streaming top-k that re-runs the walks (no staging memory either way).
#include "bf_common.h"

namespace bf {
namespace {

constexpr int kThreads = 256;
constexpr uint64_t kNone = ~uint64_t(0);

__device__ __forceinline__ int64_t walk_step(const int64_t* __restrict__ rowptr,
                                             const int32_t* __restrict__ col, int64_t cur, float u) {
  const int64_t beg = rowptr[cur];
  const int64_t deg = rowptr[cur + 1] - beg;
  if (deg <= 0) return cur;                       // dead end: stay
  int64_t idx = int64_t(u * float(deg));          // fp32 multiply (RNE), truncate
  if (idx > deg - 1) idx = deg - 1;
  return col[beg + idx];
}

// Walk records (bf_walk_records): per CSR edge e, 16 bytes {target id, the
// target's degree, the target's row start (low word, high word)}. A walk that
// carries its node's (row start, degree) takes a step with one random 16-byte
// read, the chosen edge's record, where walk_step makes two dependent ones
// (the rowptr pair, then col). The step arithmetic is walk_step's.
struct WalkCursor {
  int64_t cur, beg, deg;
};

__device__ __forceinline__ WalkCursor walk_start(const int64_t* __restrict__ rowptr, int64_t q) {
  const int64_t b = rowptr[q];
  return WalkCursor{q, b, rowptr[q + 1] - b};
}

__device__ __forceinline__ void walk_step_rec(const int4* __restrict__ rec, WalkCursor& w, float u) {
  if (w.deg <= 0) return;                         // dead end: stay
  int64_t idx = int64_t(u * float(w.deg));        // as walk_step
  if (idx > w.deg - 1) idx = w.deg - 1;
  const int4 r = rec[w.beg + idx];
  w.cur = r.x;
  w.deg = r.y;
  w.beg = int64_t((uint64_t(uint32_t(r.w)) << 32) | uint32_t(r.z));
}

__global__ __launch_bounds__(kThreads) void walk_records_kernel(const int64_t* __restrict__ rowptr,
                                                                const int32_t* __restrict__ col, int64_t num_nodes,
                                                                int64_t num_edges, int4* __restrict__ rec) {
  const int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= num_edges) return;
  const int32_t t = col[e];
  int64_t b = 0, d = 0;                           // a target outside the graph reads as a dead end
  if (t >= 0 && t < num_nodes) {
    b = rowptr[t];
    d = rowptr[t + 1] - b;
  }
  rec[e] = make_int4(t, int32_t(d), int32_t(uint32_t(uint64_t(b))), int32_t(uint32_t(uint64_t(b) >> 32)));
}

__global__ __launch_bounds__(kThreads) void random_walk_kernel(
    const int64_t* __restrict__ rowptr, const int32_t* __restrict__ col, int64_t q_lo, int64_t n_walks,
    int P, int L, const float* __restrict__ u, uint64_t seed, uint64_t offset, int64_t* __restrict__ walks) {
  const int64_t wl = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (wl >= n_walks) return;
  const int64_t q = q_lo + wl / P;
  const int64_t w = q * P + (wl % P);
  int64_t cur = q;
  int64_t* row = walks + wl * (L + 1);
  row[0] = cur;
  WalkStream rng{seed, offset, uint64_t(w), {}};
  for (int l = 0; l < L; ++l) {
    const float uu = u ? u[wl * L + l] : rng.at(l);
    cur = walk_step(rowptr, col, cur, uu);
    row[l + 1] = cur;
  }
}

__global__ __launch_bounds__(kThreads) void walk_uniforms_kernel(int64_t q_lo, int64_t n_walks, int P, int L,
                                                                 uint64_t seed, uint64_t offset,
                                                                 float* __restrict__ u) {
  const int64_t wl = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (wl >= n_walks) return;
  const int64_t w = (q_lo + wl / P) * P + (wl % P);
  WalkStream rng{seed, offset, uint64_t(w), {}};
  for (int l = 0; l < L; ++l) u[wl * L + l] = rng.at(l);
}

// Walks from arbitrary start nodes; walk i draws its Philox stream as walk id (id_base + i).
__global__ __launch_bounds__(kThreads) void random_walk_starts_kernel(
    const int64_t* __restrict__ rowptr, const int32_t* __restrict__ col, const int64_t* __restrict__ starts,
    int64_t n_walks, int L, const float* __restrict__ u, uint64_t seed, uint64_t offset, uint64_t id_base,
    int64_t* __restrict__ walks) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n_walks) return;
  int64_t cur = starts[i];
  int64_t* row = walks + i * (L + 1);
  row[0] = cur;
  WalkStream rng{seed, offset, id_base + uint64_t(i), {}};
  for (int l = 0; l < L; ++l) {
    const float uu = u ? u[i * L + l] : rng.at(l);
    cur = walk_step(rowptr, col, cur, uu);
    row[l + 1] = cur;
  }
}

// Query of table row qi: the explicit id list when given (dst-filtered builds),
// else the contiguous range starting at q_lo. -1 marks an id outside the graph.
__device__ __forceinline__ int64_t row_query(const int32_t* __restrict__ qids, int64_t q_lo, int64_t qi,
                                             int64_t num_nodes) {
  if (!qids) return q_lo + qi;
  const int64_t q = qids[qi];
  return (q >= 0 && q < num_nodes) ? q : -1;
}

// Whether x occurs in the ascending list a[lo, hi).
__device__ __forceinline__ bool sorted_contains(const int32_t* __restrict__ a, int64_t lo, int64_t hi, int32_t x) {
  const int64_t end = hi;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (a[mid] < x) lo = mid + 1; else hi = mid;
  }
  return lo < end && a[lo] == x;
}

// ---- 32-bit keys (the RW register ranking and the fused light/heavy kernel).
// For a fixed query q, key(src) = (src*A + base_q) mod 2^31 with A odd is a
// bijection of src < 2^31, so a row's candidates never tie and the KR smallest
// keys alone name the winners: src = ((key - base_q) * A^-1) mod 2^31. A list
// entry is then one 32-bit value, inserted without a branch.
constexpr uint32_t kKeyMul = 1103515245u;
constexpr uint32_t kKeyMulInv = 0xeeb9eb65u;   // kKeyMul * kKeyMulInv == 1 (mod 2^32)
constexpr uint32_t kNoKey = 0xffffffffu;       // above every 31-bit key

__device__ __forceinline__ uint32_t key_base(uint32_t q, uint32_t kc) { return q * 214013u + kc; }
__device__ __forceinline__ uint32_t key_of(uint32_t src, uint32_t base) { return (src * kKeyMul + base) & 0x7fffffffu; }
__device__ __forceinline__ int32_t src_of(uint32_t key, uint32_t base) {
  return int32_t(((key - base) * kKeyMulInv) & 0x7fffffffu);
}

// The walk of lane p of query row qi (walk id q*P + p): step(l), called for
// l = 0, 1, ... in turn, is candidate l, (key << 32 | kv) of the node reached
// at step l, or kNone for a filtered step (a stay after step 0, a query
// outside the graph, or with sub_ptr/sub_src a kv already joined to q by a
// graph edge).
struct RwWalk {
  const int64_t* __restrict__ rowptr;
  const int32_t* __restrict__ col;
  const int4* __restrict__ rec;
  const float* __restrict__ u;
  const int64_t* __restrict__ sub_ptr;
  const int32_t* __restrict__ sub_src;
  int64_t q, cur, wl;
  int L;
  uint32_t kc;
  WalkCursor wc;
  WalkStream rng;

  __device__ __forceinline__ RwWalk(const int64_t* rowptr_, const int32_t* col_, const int4* rec_,
                                    int64_t num_nodes, int64_t q_lo, const int32_t* qids, int64_t qi, int P, int p,
                                    int L_, uint32_t kc_, const float* u_, uint64_t seed, uint64_t offset,
                                    const int64_t* sub_ptr_, const int32_t* sub_src_)
      : rowptr(rowptr_), col(col_), rec(rec_), u(u_), sub_ptr(sub_ptr_), sub_src(sub_src_), L(L_), kc(kc_) {
    q = row_query(qids, q_lo, qi, num_nodes);
    cur = q;
    wl = qi * P + p;
    wc = WalkCursor{q, 0, 0};
    if (rec && q >= 0) wc = walk_start(rowptr, q);
    rng = WalkStream{seed, offset, uint64_t(q * P + p), {}};
  }

  __device__ __forceinline__ uint64_t step(int l) {
    if (q < 0) return kNone;
    const float uu = u ? u[wl * L + l] : rng.at(l);
    int64_t nxt;
    if (rec) {
      walk_step_rec(rec, wc, uu);
      nxt = wc.cur;
    } else {
      nxt = walk_step(rowptr, col, cur, uu);
    }
    bool keep = (l == 0) || (nxt != cur);
    if (keep && sub_ptr) keep = !sorted_contains(sub_src, sub_ptr[q], sub_ptr[q + 1], int32_t(nxt));
    cur = nxt;
    return keep ? (uint64_t(edge_key(uint32_t(nxt), uint32_t(q), kc)) << 32) | uint32_t(nxt) : kNone;
  }

  // The same step as its key alone (kNoKey for a dropped step): for one query the key is a bijection of
  // the source, so ordering keys orders the (key, kv) values above, and src_of recovers kv.
  __device__ __forceinline__ uint32_t step_key(int l) {
    const uint64_t v = step(l);
    return v == kNone ? kNoKey : uint32_t(v >> 32);
  }
};

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t x, int o) {
  const uint32_t lo = __shfl_xor(uint32_t(x), o, 64);
  const uint32_t hi = __shfl_xor(uint32_t(x >> 32), o, 64);
  return (uint64_t(hi) << 32) | lo;
}

// Orders a, b ascending (asc) or descending.
__device__ __forceinline__ void cmp_swap32(uint32_t& a, uint32_t& b, bool asc) {
  const uint32_t lo = min(a, b), hi = max(a, b);
  a = asc ? lo : hi;
  b = asc ? hi : lo;
}


// rw_select for P a power of two <= 64 and L <= R (R a power of two <= 16):
// lane p keeps its walk's candidates in registers x[0, R) (kNone past L), the
// query's element i = p*R + r, and the query's P lanes sort the P*R elements
// ascending with the bitonic network of the LDS kernel below: pairs closer
// than R are compare-exchanged in a lane's registers, pairs R or more apart
// across lanes (xor shuffles within the wave; a query's lanes are an aligned
// group of P), with no LDS and no barrier. Blocks of 256 / P queries.
template <int R>
__global__ __launch_bounds__(kThreads) void rw_select_reg_kernel(
    const int64_t* __restrict__ rowptr, const int32_t* __restrict__ col, const int4* __restrict__ rec,
    int64_t num_nodes, int64_t q_lo, const int32_t* __restrict__ qids, int64_t n_q, int P, int L, int K,
    uint32_t kc, const float* __restrict__ u, uint64_t seed, uint64_t offset, const int64_t* __restrict__ sub_ptr,
    const int32_t* __restrict__ sub_src, int32_t* __restrict__ sel_kv, int32_t* __restrict__ sel_cnt) {
  const int tid = threadIdx.x;
  const int p = tid & (P - 1);
  const int64_t qi = int64_t(blockIdx.x) * (kThreads / P) + tid / P;
  if (qi >= n_q) return;                      // a query's P lanes leave together
  // the candidates as 32-bit keys (src_of names their kv): min / max compare-exchanges and one shuffle
  // per cross-lane step, where (key << 32 | kv) values took 64-bit compares, selects and two shuffles
  uint32_t x[R];
  uint32_t base;
  {
    RwWalk walk(rowptr, col, rec, num_nodes, q_lo, qids, qi, P, p, L, kc, u, seed, offset, sub_ptr, sub_src);
    base = key_base(uint32_t(walk.q), kc);
#pragma unroll
    for (int r = 0; r < R; ++r) x[r] = r < L ? walk.step_key(r) : kNoKey;
  }
  const int M2 = P * R;
  // blocks of up to R elements: in registers
#pragma unroll
  for (int k = 2; k <= R; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if ((r ^ j) > r) cmp_swap32(x[r], x[r ^ j], ((p * R + r) & k) == 0);
      }
    }
  }
  for (int k = 2 * R; k <= M2; k <<= 1) {
    const bool asc = ((p * R) & k) == 0;      // the same for a lane's R elements (k > r)
    for (int j = k >> 1; j >= R; j >>= 1) {
      const int pm = j / R;                   // partner lane p ^ pm holds element i ^ j
      const bool keep_min = ((p & pm) == 0) == asc;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t y = __shfl_xor(x[r], pm, 64);
        x[r] = keep_min ? min(y, x[r]) : max(y, x[r]);
      }
    }
#pragma unroll
    for (int j = R >> 1; j > 0; j >>= 1) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if ((r ^ j) > r) cmp_swap32(x[r], x[r ^ j], asc);
      }
    }
  }
  // the valid candidates are a prefix of the sorted elements
  int cnt = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = p * R + r;
    if (i < K) {
      sel_kv[qi * K + i] = x[r] != kNoKey ? src_of(x[r], base) : -1;
      cnt += x[r] != kNoKey ? 1 : 0;
    }
  }
  for (int i = M2 + p; i < K; i += P) sel_kv[qi * K + i] = -1;
  for (int o = 1; o < P; o <<= 1) cnt += __shfl_xor(cnt, o, 64);
  if (p == 0) sel_cnt[qi] = cnt;
}

// One lane per walk; the P lanes of a query are adjacent. Candidates are staged
// in LDS as (key << 32 | kv) (kNone = filtered step), padded with kNone to M2 =
// the power of two >= P*L, and the query's P lanes sort them ascending with a
// bitonic network (log2(M2) (log2(M2) + 1) / 2 compare-exchange stages, one
// barrier each): the first min(valid, K) slots are the selection, with
// multiplicity (equal values are the same pair). The block holds qpb queries
// (blockDim = qpb * P, sized so the staging fits LDS), so any P*L and K that
// fit it are served. With sub_ptr/sub_src (an in-neighbour CSR with ascending
// rows) a candidate kv that is already a graph edge kv -> q is dropped: the
// probe pools' RW-minus-real subtraction (utils/fullgraph_sp_support.py:
// 1797-1812, 1536-1551).
__global__ __launch_bounds__(kThreads) void rw_select_kernel(
    const int64_t* __restrict__ rowptr, const int32_t* __restrict__ col, const int4* __restrict__ rec,
    int64_t num_nodes, int64_t q_lo,
    const int32_t* __restrict__ qids, int64_t n_q, int P, int L, int K, int M2, int qpb, uint32_t kc,
    const float* __restrict__ u, uint64_t seed, uint64_t offset, const int64_t* __restrict__ sub_ptr,
    const int32_t* __restrict__ sub_src, int32_t* __restrict__ sel_kv, int32_t* __restrict__ sel_cnt) {
  // [qpb][M2 + 1]: the odd row stride puts the rows the queries of a wave read
  // at one time in different LDS banks (a stride of M2 * 8 bytes maps them all
  // to the same bank)
  extern __shared__ uint64_t cand[];
  const int tid = threadIdx.x;
  const int ql = tid / P;
  const int p = tid - ql * P;
  const int M = P * L;
  uint64_t* const c = cand + ql * (M2 + 1);                // this query's slots
  const int64_t qi = int64_t(blockIdx.x) * qpb + ql;
  const bool active = ql < qpb && qi < n_q;
  if (active) {
    uint64_t* const mine = c + p * L;                       // this walk's L candidates
    RwWalk walk(rowptr, col, rec, num_nodes, q_lo, qids, qi, P, p, L, kc, u, seed, offset, sub_ptr, sub_src);
    for (int l = 0; l < L; ++l) mine[l] = walk.step(l);
    for (int i = M + p; i < M2; i += P) c[i] = kNone;       // the padding sorts last
  }
  __syncthreads();
  // bitonic sort of the M2 slots by the query's P lanes; every thread of the block takes part in the
  // barriers (the stage count depends on M2 only)
  for (int k = 2; k <= M2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (active) {
        for (int i = p; i < M2; i += P) {
          const int l = i ^ j;
          if (l > i) {
            const uint64_t x = c[i], y = c[l];
            if ((x > y) == ((i & k) == 0)) {
              c[i] = y;
              c[l] = x;
            }
          }
        }
      }
      __syncthreads();
    }
  }
  if (!active) return;
  // the valid candidates are a prefix of the sorted slots
  for (int r = p; r < K; r += P) {
    const uint64_t v = r < M2 ? c[r] : kNone;
    sel_kv[qi * K + r] = v != kNone ? int32_t(uint32_t(v)) : -1;
  }
  if (p == 0) {
    int lo = 0, hi = K < M2 ? K : M2;       // count of valid slots in [0, min(K, M2)): binary search
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (c[mid] != kNone) lo = mid + 1; else hi = mid;
    }
    sel_cnt[qi] = lo;
  }
}

constexpr int kGroup = 16;                  // lanes per query in the real-edge pass
constexpr int kQPB = kThreads / kGroup;     // queries per block
// Merged rows are listed in LDS, kQPB rows of `cap` = k_real + k_rw ids per
// block plus as many duplicate flags: up to 96 KB, i.e. budgets of up to 768;
// wider rows go to merge_rows_wide_kernel / assemble_rows_wide_kernel.
constexpr size_t kRowLdsBytes = size_t(96) << 10;
constexpr int kMaxRowCap = int(kRowLdsBytes / (2 * sizeof(int32_t) * (kThreads / 16)));
#ifndef BF_SCAN_UNROLL
#define BF_SCAN_UNROLL 8
#endif
constexpr int kScanUnroll = BF_SCAN_UNROLL;  // in-neighbour loads in flight per lane
#ifndef BF_SCAN_X4_UNROLL
#define BF_SCAN_X4_UNROLL 4
#endif
constexpr int kScanX4Unroll = BF_SCAN_X4_UNROLL;  // 16-byte chunks in flight per thread (light rows)


// Folds candidates src[i], src[i+stride], ... (< end) of query q, each as the
// value (key << 32 | position in the row), into the sorted register list lk
// (the KMAX smallest such values >= floor). The value orders by (key,
// position) — the reference's tie-break — and is unique even where the row
// repeats a source (a walk pool is a multiset); the source comes back from the
// key (src_of). U loads are issued before any is used, so a lane keeps U
// gathers in flight instead of one; the slots past end re-read src[end-1] (in
// bounds) and are skipped. The list is the same whatever order the candidates
// arrive in. A selection of more than KMAX winners runs in batches of KMAX,
// each batch's floor one above the last value taken.
template <int U, int KMAX>
__device__ __forceinline__ void scan_topk(const int32_t* __restrict__ src, int64_t row_beg, int64_t i, int64_t end,
                                          int stride, uint32_t q, uint32_t kc, uint64_t floor, uint64_t (&lk)[KMAX]) {
  for (; i < end; i += int64_t(stride) * U) {
    uint32_t s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = i + int64_t(u) * stride;
      s[u] = uint32_t(src[j < end ? j : end - 1]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t c = (uint64_t(edge_key(s[u], q, kc)) << 32) | uint32_t(i + int64_t(u) * stride - row_beg);
      if (i + int64_t(u) * stride < end && c < lk[KMAX - 1] && c >= floor) {
#pragma unroll
        for (int j = KMAX - 1; j > 0; --j) lk[j] = c < lk[j - 1] ? lk[j - 1] : (c < lk[j] ? c : lk[j]);
        lk[0] = c < lk[0] ? c : lk[0];
      }
    }
  }
}

// One round of a block-wide minimum over the heads lk[0] of every thread's
// ascending register list (wave shuffles, then LDS across the 4 waves):
// returns the smallest head, the same in every thread, and shifts it out of
// its holder's list (the lowest thread on a tie; nothing moves when it is
// kNone). Every thread of the block calls it.
template <int KMAX>
__device__ __forceinline__ uint64_t block_pop_min(uint64_t (&lk)[KMAX], uint64_t* wave_min, int* wave_win) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint64_t head = lk[0];
  uint64_t m = head;
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t y = shfl_xor_u64(m, o);
    m = y < m ? y : m;
  }
  const uint64_t bal = __ballot(head == m);
  if (lane == 0) {
    wave_min[wave] = m;
    wave_win[wave] = __ffsll((unsigned long long)bal) - 1;
  }
  __syncthreads();
  uint64_t best = wave_min[0];
  int best_wave = 0;
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) {
    if (wave_min[w] < best) {
      best = wave_min[w];
      best_wave = w;
    }
  }
  const int winner = best_wave * 64 + wave_win[best_wave];
  __syncthreads();
  if (best != kNone && int(threadIdx.x) == winner) {
#pragma unroll
    for (int j = 0; j < KMAX - 1; ++j) lk[j] = lk[j + 1];
    lk[KMAX - 1] = kNone;
  }
  return best;
}

// Top-k_real of one in-neighbour list with a whole workgroup (hubs, and every
// row of a merged row too wide for LDS): every thread keeps a sorted register
// list of its strided share, then rounds of block_pop_min pop the winners in
// key order into out[0, cnt) (written by thread 0), KMAX per batch (a thread's
// list holds only its KMAX smallest, so after KMAX pops the block rescans
// above the last winner). Returns cnt, the same in every thread. Every thread
// of the block must call it.
template <int KMAX>
__device__ __forceinline__ int hub_topk(const int64_t* __restrict__ in_ptr, const int32_t* __restrict__ in_src,
                                        int64_t q, int k_real, uint32_t kc, uint64_t* wave_min, int* wave_win,
                                        int32_t* out) {
  uint64_t lk[KMAX];
  int cnt = 0;
  uint64_t floor = 0;
  while (cnt < k_real) {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) lk[j] = kNone;
    scan_topk<kScanUnroll>(in_src, in_ptr[q], in_ptr[q] + threadIdx.x, in_ptr[q + 1], kThreads, uint32_t(q), kc,
                           floor, lk);
    int popped = 0;
    uint64_t best = kNone;
    while (popped < KMAX && cnt < k_real) {
      best = block_pop_min<KMAX>(lk, wave_min, wave_win);
      if (best == kNone) return cnt;   // the same value in every thread: uniform exit
      if (threadIdx.x == 0) out[cnt] = src_of(uint32_t(best >> 32), key_base(uint32_t(q), kc));
      ++cnt;
      ++popped;
    }
    floor = best + 1;
  }
  return cnt;
}

// Output: hub_sel [n_hubs, k_real] kv ids in key order, hub_cnt.
template <int KMAX>
__global__ __launch_bounds__(kThreads) void real_select_hub_kernel(
    const int64_t* __restrict__ in_ptr, const int32_t* __restrict__ in_src, const int32_t* __restrict__ hubs,
    int k_real, uint32_t kc, int32_t* __restrict__ hub_sel, int32_t* __restrict__ hub_cnt) {
  __shared__ uint64_t wave_min[kThreads / 64];
  __shared__ int wave_win[kThreads / 64];
  const int h = blockIdx.x;
  const int cnt = hub_topk<KMAX>(in_ptr, in_src, hubs[h], k_real, kc, wave_min, wave_win,
                                 hub_sel + int64_t(h) * k_real);
  if (threadIdx.x == 0) hub_cnt[h] = cnt;
}

// Top-k_real of query q's in-neighbour list by one 16-lane group: per-lane
// sorted register lists of its strided share, then rounds of a group minimum,
// KMAX per batch (then a rescan above the last winner); the winners land in
// row[0, n) in key order (lane 0 writes). Returns n, the same in the group's
// lanes.
template <int KMAX>
__device__ __forceinline__ int group_topk(const int64_t* __restrict__ in_ptr, const int32_t* __restrict__ in_src,
                                          int64_t q, int k_real, uint32_t kc, int gl, int32_t* row) {
  uint64_t lk[KMAX];
  const int lane = threadIdx.x & 63;
  const int gbase = lane & ~(kGroup - 1);
  int n = 0;
  uint64_t floor = 0;
  while (n < k_real) {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) lk[j] = kNone;
    scan_topk<kScanUnroll>(in_src, in_ptr[q], in_ptr[q] + gl, in_ptr[q + 1], kGroup, uint32_t(q), kc, floor, lk);
    int popped = 0;
    uint64_t m = kNone;
    while (popped < KMAX && n < k_real) {
      const uint64_t h = lk[0];
      m = h;
      for (int o = 1; o < kGroup; o <<= 1) {
        const uint64_t y = shfl_xor_u64(m, o);
        m = y < m ? y : m;
      }
      if (m == kNone) return n;      // uniform over the group
      const uint64_t bal = __ballot(h == m);
      const uint64_t mine = (bal >> gbase) & ((uint64_t(1) << kGroup) - 1);
      const int winner = __ffsll((unsigned long long)mine) - 1;
      if (gl == winner) {
#pragma unroll
        for (int j = 0; j < KMAX - 1; ++j) lk[j] = lk[j + 1];
        lk[KMAX - 1] = kNone;
      }
      if (gl == 0) row[n] = src_of(uint32_t(m >> 32), key_base(uint32_t(q), kc));
      ++n;
      ++popped;
    }
    floor = m + 1;
  }
  return n;
}

// Writes one table row from the LDS list lst[0, n_tot): with dedup the set of
// values ascending (first occurrence wins), without it the multiset ascending
// (stable), or with key_order the list as it stands (the selection order, i.e.
// ascending key). Every thread of the block calls it (it holds a barrier).
__device__ __forceinline__ void write_row(const int32_t* lst, int32_t* dupf, int gl, bool active, int n_tot, int dedup,
                                          int key_order, int32_t* __restrict__ out, int width,
                                          int32_t* __restrict__ len_out) {
  if (active && dedup) {
    for (int i = gl; i < n_tot; i += kGroup) {
      const int32_t v = lst[i];
      int dup = 0;
      for (int j = 0; j < i; ++j) dup |= lst[j] == v;
      dupf[i] = dup;
    }
  }
  __syncthreads();
  if (!active) return;
  int len = 0;
  for (int i = 0; i < n_tot; ++i) len += dedup ? !dupf[i] : 1;
  for (int i = gl; i < n_tot; i += kGroup) {
    const int32_t v = lst[i];
    int rank = 0;
    if (dedup) {
      if (dupf[i]) continue;
      for (int j = 0; j < n_tot; ++j) rank += !dupf[j] && lst[j] < v;
    } else if (key_order) {
      rank = i;
    } else {
      for (int j = 0; j < n_tot; ++j) {
        const int32_t w = lst[j];
        rank += (w < v) || (w == v && j < i);
      }
    }
    out[rank] = v;
  }
  for (int c = len + gl; c < width; c += kGroup) out[c] = -1;
  if (gl == 0) *len_out = len;
}

// Group-per-query top-k and merge: row li of the launch serves query
// qids[li] (or q_lo + li) and writes table row li.
template <int KMAX>
__global__ __launch_bounds__(kThreads) void real_select_merge_kernel(
    const int64_t* __restrict__ in_ptr, const int32_t* __restrict__ in_src, int64_t num_nodes, int64_t q_lo,
    const int32_t* __restrict__ qids, int64_t n_q, int k_real, uint32_t kc,
    const int32_t* __restrict__ rw_kv, const int32_t* __restrict__ rw_cnt, int k_rw, int dedup, int key_order,
    int32_t* __restrict__ table, int width, int32_t* __restrict__ row_len, const int32_t* __restrict__ hubs,
    const int32_t* __restrict__ hub_sel, const int32_t* __restrict__ hub_cnt, int64_t n_hubs,
    int64_t hub_threshold, int cap) {
  extern __shared__ int32_t row_lds[];         // [kQPB][cap] ids, then [kQPB][cap] duplicate flags
  const int gq = threadIdx.x / kGroup;
  int32_t* const lst = row_lds + gq * cap;
  int32_t* const dupf = row_lds + kQPB * cap + gq * cap;
  const int gl = threadIdx.x % kGroup;
  const int64_t li = int64_t(blockIdx.x) * kQPB + gq;
  const int64_t q = li < n_q ? row_query(qids, q_lo, li, num_nodes) : -1;
  const bool active = li < n_q;
  const int64_t qi = li;
  int n_r = 0, n_w = 0;
  int64_t hub = -1;
  if (q >= 0 && k_real > 0 && n_hubs > 0) {
    if (in_ptr[q + 1] - in_ptr[q] > hub_threshold) {   // selection precomputed by real_select_hub_kernel
      int64_t lo = 0, hi = n_hubs;
      while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (hubs[mid] < q) lo = mid + 1; else hi = mid;
      }
      if (lo < n_hubs && hubs[lo] == q) hub = lo;
    }
  }
  if (hub >= 0) {
    n_r = hub_cnt[hub];
    for (int i = gl; i < n_r; i += kGroup) lst[i] = hub_sel[hub * k_real + i];
  } else if (q >= 0 && k_real > 0) {
    n_r = group_topk<KMAX>(in_ptr, in_src, q, k_real, kc, gl, lst);
  }
  if (active && rw_kv != nullptr && k_rw > 0) {
    n_w = rw_cnt[qi];
    for (int i = gl; i < n_w; i += kGroup) lst[n_r + i] = rw_kv[qi * k_rw + i];
  }
  __syncthreads();
  write_row(lst, dupf, gl, active, n_r + n_w, dedup, key_order, table + (active ? qi : 0) * width, width,
            row_len + (active ? qi : 0));
}

// One candidate of a nested budget probe: per row the first b_r entries of a
// key-ordered real selection and the first b_w of a key-ordered RW selection
// (both from one ranking, so every candidate budget is a prefix), merged as the
// full build merges them (utils/fullgraph_sp_support.py:1824-1879).
__global__ __launch_bounds__(kThreads) void assemble_rows_kernel(
    const int32_t* __restrict__ real_kv, const int32_t* __restrict__ real_cnt, int real_stride, int b_r,
    const int32_t* __restrict__ rw_kv, const int32_t* __restrict__ rw_cnt, int rw_stride, int b_w, int dedup,
    int64_t n, int32_t* __restrict__ table, int width, int32_t* __restrict__ row_len, int cap) {
  extern __shared__ int32_t row_lds[];         // [kQPB][cap] ids, then [kQPB][cap] duplicate flags
  const int gq = threadIdx.x / kGroup;
  int32_t* const lst = row_lds + gq * cap;
  int32_t* const dupf = row_lds + kQPB * cap + gq * cap;
  const int gl = threadIdx.x % kGroup;
  const int64_t qi = int64_t(blockIdx.x) * kQPB + gq;
  const bool active = qi < n;
  int n_r = 0, n_w = 0;
  if (active) {
    if (real_kv && b_r > 0) n_r = min(real_cnt[qi], b_r);
    if (rw_kv && b_w > 0) n_w = min(rw_cnt[qi], b_w);
    for (int i = gl; i < n_r; i += kGroup) lst[i] = real_kv[qi * real_stride + i];
    for (int i = gl; i < n_w; i += kGroup) lst[n_r + i] = rw_kv[qi * rw_stride + i];
  }
  __syncthreads();
  write_row(lst, dupf, gl, active, n_r + n_w, dedup, 0, table + (active ? qi : 0) * width, width,
            row_len + (active ? qi : 0));
}

// ---- Past the LDS staging: one row per workgroup, nothing staged.

// Finishes a merged row that sits in its table slots out[0, n): with dedup
// the set of values ascending, without it the multiset ascending, with
// key_order the list as it stands; slots [len, width) get -1. Returns len, the
// same in every thread. The sort is the all-ascending bitonic network over n
// rounded up to a power of two (each compare-exchange puts the smaller value
// at the lower index; the first step of a merge over blocks of k pairs slot i
// with its mirror k-1-i in the block): the virtual slots past n hold +inf and
// never move, so a comparator reaching past n is skipped and no slot past n is
// read or written. The dedup compaction keeps a value that differs from its
// left neighbour; a round reads its 256 slots before it writes, and a kept
// value lands at or left of where it was read, so no round overwrites a slot
// a later round reads with another value. Every thread of the block calls it,
// with out[0, n) written and visible to the block.
__device__ int wide_row_finish(int32_t* out, int n, int dedup, int key_order, int width, int* wave_cnt) {
  if (!key_order && n > 1) {
    int m2 = 1;
    while (m2 < n) m2 <<= 1;
    for (int k = 2; k <= m2; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int t = threadIdx.x; t < (m2 >> 1); t += kThreads) {
          const int blk = t / j;
          const int off = t - blk * j;
          const int i = blk * 2 * j + off;
          const int l = j == (k >> 1) ? blk * 2 * j + k - 1 - off : i + j;
          if (l < n) {
            const int32_t a = out[i], b = out[l];
            if (b < a) {
              out[i] = b;
              out[l] = a;
            }
          }
        }
        __syncthreads();
      }
    }
  }
  int len = n;
  if (dedup && n > 1) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int base = 0;
    for (int r0 = 0; r0 < n; r0 += kThreads) {
      const int i = r0 + threadIdx.x;
      int32_t v = 0;
      bool keep = false;
      if (i < n) {
        v = out[i];
        keep = i == 0 || out[i - 1] != v;
      }
      const uint64_t bal = __ballot(keep);
      if (lane == 0) wave_cnt[wave] = __popcll(bal);
      __syncthreads();
      int at = base + __popcll(bal & ((uint64_t(1) << lane) - 1));
      int total = 0;
#pragma unroll
      for (int w = 0; w < kThreads / 64; ++w) {
        const int c = wave_cnt[w];
        at += w < wave ? c : 0;
        total += c;
      }
      if (keep) out[at] = v;
      base += total;
      __syncthreads();
    }
    len = base;
  }
  for (int c = len + threadIdx.x; c < width; c += kThreads) out[c] = -1;
  return len;
}

// real_select_merge for budgets whose merged row does not fit the LDS
// staging: a workgroup per row (grid-stride), the real top-k by the whole
// block (hub_topk, for every row: a block per row already), the RW part
// appended, then the row finished in place in its table slots.
template <int KMAX>
__global__ __launch_bounds__(kThreads) void merge_rows_wide_kernel(
    const int64_t* __restrict__ in_ptr, const int32_t* __restrict__ in_src, int64_t num_nodes, int64_t q_lo,
    const int32_t* __restrict__ qids, int64_t n_q, int k_real, uint32_t kc, const int32_t* __restrict__ rw_kv,
    const int32_t* __restrict__ rw_cnt, int k_rw, int dedup, int key_order, int32_t* table, int width,
    int32_t* __restrict__ row_len) {
  __shared__ uint64_t wave_min[kThreads / 64];
  __shared__ int wave_win[kThreads / 64];
  __shared__ int wave_cnt[kThreads / 64];
  for (int64_t li = blockIdx.x; li < n_q; li += gridDim.x) {
    const int64_t q = row_query(qids, q_lo, li, num_nodes);
    int32_t* const out = table + li * width;
    const int n_r = (q >= 0 && k_real > 0) ? hub_topk<KMAX>(in_ptr, in_src, q, k_real, kc, wave_min, wave_win, out)
                                           : 0;
    const int n_w = (rw_kv != nullptr && k_rw > 0) ? min(rw_cnt[li], k_rw) : 0;
    for (int i = threadIdx.x; i < n_w; i += kThreads) out[n_r + i] = rw_kv[li * k_rw + i];
    __syncthreads();
    const int len = wide_row_finish(out, n_r + n_w, dedup, key_order, width, wave_cnt);
    if (threadIdx.x == 0) row_len[li] = len;
  }
}

// assemble_rows for candidates too wide for the LDS staging: a workgroup per
// row (grid-stride) copies the two prefixes into the row's table slots and
// finishes the row there.
__global__ __launch_bounds__(kThreads) void assemble_rows_wide_kernel(
    const int32_t* __restrict__ real_kv, const int32_t* __restrict__ real_cnt, int real_stride, int b_r,
    const int32_t* __restrict__ rw_kv, const int32_t* __restrict__ rw_cnt, int rw_stride, int b_w, int dedup,
    int64_t n, int32_t* table, int width, int32_t* __restrict__ row_len) {
  __shared__ int wave_cnt[kThreads / 64];
  for (int64_t li = blockIdx.x; li < n; li += gridDim.x) {
    int32_t* const out = table + li * width;
    const int n_r = (real_kv && b_r > 0) ? min(real_cnt[li], b_r) : 0;
    const int n_w = (rw_kv && b_w > 0) ? min(rw_cnt[li], b_w) : 0;
    for (int i = threadIdx.x; i < n_r; i += kThreads) out[i] = real_kv[li * real_stride + i];
    for (int i = threadIdx.x; i < n_w; i += kThreads) out[n_r + i] = rw_kv[li * rw_stride + i];
    __syncthreads();
    const int len = wide_row_finish(out, n_r + n_w, dedup, 0, width, wave_cnt);
    if (threadIdx.x == 0) row_len[li] = len;
  }
}

// rw_select for walk shapes whose P*L candidates do not fit one query's LDS
// staging: a workgroup per query (grid-stride), lane p < P runs walk p, and the
// selection streams instead of staging. Each round re-runs the P walks from
// their start (a walk is a pure function of its Philox counters or injected
// uniforms, and of the graph) and every lane keeps the KMAX smallest of its
// candidates at or above `floor` as (key << 32 | p*L + l): values that are
// unique, and that order as the staged (key << 32 | kv) do, since for one
// query the key names the kv. Rounds of block_pop_min then pop up to KMAX
// winners in order (after KMAX pops a lane's list may be spent, so the next
// round rescans above the last winner). A pair drawn by several steps is
// popped once per step: the selection keeps the multiplicity, as the sorting
// kernels do. P*L < 2^32 (checked on the host).
template <int KMAX>
__global__ __launch_bounds__(kThreads) void rw_select_stream_kernel(
    const int64_t* __restrict__ rowptr, const int32_t* __restrict__ col, const int4* __restrict__ rec,
    int64_t num_nodes, int64_t q_lo, const int32_t* __restrict__ qids, int64_t n_q, int P, int L, int K,
    uint32_t kc, const float* __restrict__ u, uint64_t seed, uint64_t offset, const int64_t* __restrict__ sub_ptr,
    const int32_t* __restrict__ sub_src, int32_t* __restrict__ sel_kv, int32_t* __restrict__ sel_cnt) {
  __shared__ uint64_t wave_min[kThreads / 64];
  __shared__ int wave_win[kThreads / 64];
  const int p = threadIdx.x;
  for (int64_t qi = blockIdx.x; qi < n_q; qi += gridDim.x) {
    const int64_t q = row_query(qids, q_lo, qi, num_nodes);
    const uint32_t base = key_base(uint32_t(q), kc);
    int32_t* const out = sel_kv + qi * K;
    int cnt = 0;
    uint64_t floor = 0;
    bool more = q >= 0;                                   // the same in every thread
    while (more && cnt < K) {
      uint64_t lk[KMAX];
#pragma unroll
      for (int j = 0; j < KMAX; ++j) lk[j] = kNone;
      if (p < P) {
        RwWalk walk(rowptr, col, rec, num_nodes, q_lo, qids, qi, P, p, L, kc, u, seed, offset, sub_ptr, sub_src);
        const uint32_t id0 = uint32_t(p) * uint32_t(L);
        for (int l = 0; l < L; ++l) {
          const uint32_t key = walk.step_key(l);
          const uint64_t c = (uint64_t(key) << 32) | (id0 + uint32_t(l));
          if (key != kNoKey && c >= floor && c < lk[KMAX - 1]) {
#pragma unroll
            for (int j = KMAX - 1; j > 0; --j) lk[j] = c < lk[j - 1] ? lk[j - 1] : (c < lk[j] ? c : lk[j]);
            lk[0] = c < lk[0] ? c : lk[0];
          }
        }
      }
      int popped = 0;
      uint64_t best = kNone;
      while (popped < KMAX && cnt < K) {
        best = block_pop_min<KMAX>(lk, wave_min, wave_win);
        if (best == kNone) break;
        if (threadIdx.x == 0) out[cnt] = src_of(uint32_t(best >> 32), base);
        ++cnt;
        ++popped;
      }
      more = best != kNone;
      floor = best + 1;
    }
    for (int i = cnt + threadIdx.x; i < K; i += kThreads) out[i] = -1;
    if (threadIdx.x == 0) sel_cnt[qi] = cnt;
  }
}

// Inserts c into the ascending list lk (the largest value drops out): a
// min/max carry chain, no branch. c == kNoKey leaves lk unchanged.
template <int K>
__device__ __forceinline__ void insert_key(uint32_t (&lk)[K], uint32_t c) {
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const uint32_t lo = lk[j] < c ? lk[j] : c;
    c = lk[j] < c ? c : lk[j];
    lk[j] = lo;
  }
}

// Lane gl of a G-lane group folds row[gl], row[gl+G], ... (< deg) into lk;
// U loads in flight per lane, slots past deg re-read row[deg-1] and are dropped.
template <int U, int K>
__device__ __forceinline__ void scan_keys(const int32_t* __restrict__ row, int32_t deg, int gl, int G, uint32_t base,
                                          uint32_t (&lk)[K]) {
  for (int32_t i = gl; i < deg; i += G * U) {
    uint32_t sv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t j = i + u * G;
      sv[u] = uint32_t(row[j < deg ? j : deg - 1]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) insert_key(lk, i + u * G < deg ? key_of(sv[u], base) : kNoKey);
  }
}

// One thread's scan of src[beg, end) through the aligned 4-entry chunks that
// cover it, with 16-byte loads (src 16-byte aligned), U chunks in flight:
// each load instruction moves 4 entries per lane instead of 1.
template <int U, int K>
__device__ __forceinline__ void scan_keys_x4(const int32_t* __restrict__ src, int64_t beg, int64_t end,
                                             uint32_t base, uint32_t (&lk)[K]) {
  if (end <= beg) return;
  const int4* __restrict__ v4 = reinterpret_cast<const int4*>(src);
  const int64_t c0 = beg >> 2, c_last = (end - 1) >> 2;
  const uint32_t deg = uint32_t(end - beg);
  const int32_t lead = int32_t(beg - c0 * 4);        // entries of chunk c0 before beg
  for (int64_t c = c0; c <= c_last; c += U) {
    int4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = v4[c + u <= c_last ? c + u : c_last];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
      const int32_t rel0 = int32_t(c + u - c0) * 4 - lead;     // row offset of e[0]
#pragma unroll
      for (int t = 0; t < 4; ++t)
        insert_key(lk, uint32_t(rel0 + t) < deg ? key_of(uint32_t(e[t]), base) : kNoKey);
    }
  }
}

// a <- the K smallest of a and b (both ascending), ascending: the
// half-cleaner min(a[j], b[K-1-j]) leaves them as a bitonic sequence, which a
// bitonic merge network sorts. Equal values are both kept.
template <int K>
__device__ __forceinline__ void merge_keys(uint32_t (&a)[K], const uint32_t (&b)[K]) {
  static_assert((K & (K - 1)) == 0, "K must be a power of two");
#pragma unroll
  for (int j = 0; j < K; ++j) a[j] = b[K - 1 - j] < a[j] ? b[K - 1 - j] : a[j];
#pragma unroll
  for (int s = K / 2; s > 0; s >>= 1) {
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if ((i & s) == 0) {
        const uint32_t x = a[i], y = a[i + s];
        a[i] = x < y ? x : y;
        a[i + s] = x < y ? y : x;
      }
    }
  }
}

// Butterfly over the G lanes of an aligned lane group: afterwards every lane
// holds the group's K smallest keys, ascending. Each round pairs lanes whose
// coverage is disjoint, so the multiset is exact.
template <int G, int K>
__device__ __forceinline__ void group_merge_keys(uint32_t (&lk)[K]) {
#pragma unroll
  for (int o = 1; o < G; o <<= 1) {
    uint32_t other[K];
#pragma unroll
    for (int j = 0; j < K; ++j) other[j] = __shfl_xor(lk[j], o, 64);
    merge_keys<K>(lk, other);
  }
}

constexpr int pow2_at_least(int x) { return x <= 1 ? 1 : 2 * pow2_at_least((x + 1) / 2); }

// Ascending bitonic sort of N (a power of two) values in registers.
template <int N>
__device__ __forceinline__ void sort_regs(int32_t (&v)[N]) {
#pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int l = i ^ j;
        if (l > i) {
          const int32_t x = v[i], y = v[l];
          const bool up = (i & k) == 0;
          v[i] = (x < y) == up ? x : y;
          v[l] = (x < y) == up ? y : x;
        }
      }
    }
  }
}

// Row-access flags of emit_row (bits of `vec`): the RW selection's rows and the table's rows are
// 16-byte aligned (k_rw and width multiples of 4 on aligned bases), so they move as 16-byte loads and stores.
constexpr int kVecRw = 4, kVecTable = 2;

// Writes table row qi from the real winners lk[0, k_real) (kNoKey = none) and
// the RW selection rw_kv[qi, 0 .. rw_cnt[qi]): the KR + KW ids, padded to a
// power of two, are sorted by a bitonic network in registers, duplicates
// (with dedup) turned into padding and sorted behind the ids, so that the row
// is the register prefix: stored whole, ascending, -1 past its length. Every
// register index is static, so the row goes out as 16-byte stores (and the
// selection comes in as 16-byte loads) where aligned. Writing the kept ids one
// dword at a time at a running index (each store instruction touching a line
// per lane) left the c4 build's fused kernel far below its memory rate.
template <int KR, int KW>
__device__ __forceinline__ void emit_row(const uint32_t (&lk)[KR], uint32_t base, int k_real,
                                         const int32_t* __restrict__ rw_kv, const int32_t* __restrict__ rw_cnt,
                                         int k_rw, int64_t qi, int dedup, int32_t* __restrict__ table, int width,
                                         int32_t* __restrict__ row_len, int vec) {
  constexpr int NV = pow2_at_least(KR + KW);
  constexpr int32_t kPad = 0x7fffffff;          // sorts after every node id (ids < 2^31 - 1)
  int32_t v[NV];
#pragma unroll
  for (int j = 0; j < KR; ++j) v[j] = (j < k_real && lk[j] != kNoKey) ? src_of(lk[j], base) : kPad;
#pragma unroll
  for (int j = KR; j < NV; ++j) v[j] = kPad;
  if (rw_kv != nullptr && KW > 0) {
    const int n_w = rw_cnt[qi];
    const int32_t* r = rw_kv + qi * k_rw;
    if ((vec & kVecRw) && KW % 4 == 0) {
#pragma unroll
      for (int j = 0; j < KW; j += 4) {
        if (j < k_rw && j < n_w) {              // k_rw is a multiple of 4: the 4 ids are in the row
          const int4 x = *reinterpret_cast<const int4*>(r + j);
          v[KR + j] = x.x;
          v[KR + j + 1] = j + 1 < n_w ? x.y : kPad;
          v[KR + j + 2] = j + 2 < n_w ? x.z : kPad;
          v[KR + j + 3] = j + 3 < n_w ? x.w : kPad;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < KW; ++j) v[KR + j] = (j < n_w && j < k_rw) ? r[j] : kPad;
    }
  }
  sort_regs<NV>(v);
  if (dedup) {
    bool dup[NV];
    dup[0] = false;
#pragma unroll
    for (int j = 1; j < NV; ++j) dup[j] = v[j] != kPad && v[j] == v[j - 1];
#pragma unroll
    for (int j = 1; j < NV; ++j)
      if (dup[j]) v[j] = kPad;
    sort_regs<NV>(v);
  }
  int len = 0;
#pragma unroll
  for (int j = 0; j < NV; ++j) len += v[j] != kPad ? 1 : 0;
  int32_t* out = table + qi * width;              // the row is v[0, min(width, NV)), then -1
  if (vec & kVecTable) {
#pragma unroll
    for (int j = 0; j < NV; j += 4)
      if (j < width)
        *reinterpret_cast<int4*>(out + j) = make_int4(v[j] == kPad ? -1 : v[j], v[j + 1] == kPad ? -1 : v[j + 1],
                                                      v[j + 2] == kPad ? -1 : v[j + 2],
                                                      v[j + 3] == kPad ? -1 : v[j + 3]);
  } else {
#pragma unroll
    for (int j = 0; j < NV; ++j)
      if (j < width) out[j] = v[j] == kPad ? -1 : v[j];
  }
  for (int c = NV; c < width; ++c) out[c] = -1;   // a table wider than the row's parts (no RW selection)
  row_len[qi] = len;
}

// The light/heavy split build in ONE launch, without LDS: blocks
// [0, hub_blocks) take 4 hub rows each (one wave per row), the next blocks 16
// heavy rows each (a 16-lane group per row; hub rows skipped), the rest 256
// light rows each (one per thread, 16-byte loads when in_src is 16-byte
// aligned). A group scans its row into per-lane sorted lists of KR
// (key << 32 | src), merges them by a butterfly, and its first lane writes the
// row. The long hub and heavy work is dispatched first and overlaps the light
// bulk. hubs / heavy: ascending queries of [q_lo, q_lo+n_q) with in-degree
// above hub_threshold / light_max.
constexpr int kHubsPerBlock = kThreads / 64;

template <int KR, int KW>
__global__ __launch_bounds__(kThreads) void real_select_fused_kernel(
    const int64_t* __restrict__ in_ptr, const int32_t* __restrict__ in_src, int64_t q_lo, int64_t n_q,
    int k_real, uint32_t kc, const int32_t* __restrict__ rw_kv, const int32_t* __restrict__ rw_cnt, int k_rw,
    int dedup, int32_t* __restrict__ table, int width, int32_t* __restrict__ row_len,
    const int32_t* __restrict__ hubs, int64_t n_hubs, int64_t hub_threshold, const int32_t* __restrict__ heavy,
    int64_t n_heavy, int64_t light_max, int vec4, int64_t num_nodes) {
  const int64_t b = blockIdx.x;
  const int64_t hub_blocks = ceil_div(n_hubs, int64_t(kHubsPerBlock));
  const int64_t heavy_blocks = ceil_div(n_heavy, int64_t(kQPB));
  uint32_t lk[KR];
#pragma unroll
  for (int j = 0; j < KR; ++j) lk[j] = kNoKey;
  if (b < hub_blocks) {
    const int64_t li = b * kHubsPerBlock + (threadIdx.x >> 6);
    const int64_t q = li < n_hubs ? int64_t(hubs[li]) : -1;
    if (q < q_lo || q >= q_lo + n_q) return;           // uniform over the wave
    const int lane = threadIdx.x & 63;
    const uint32_t base = key_base(uint32_t(q), kc);
    if (k_real > 0) {
      const int64_t beg = in_ptr[q];
      scan_keys<kScanUnroll>(in_src + beg, int32_t(in_ptr[q + 1] - beg), lane, 64, base, lk);
      group_merge_keys<64, KR>(lk);
    }
    if (lane == 0) emit_row<KR, KW>(lk, base, k_real, rw_kv, rw_cnt, k_rw, q - q_lo, dedup, table, width, row_len, vec4);
    return;
  }
  if (b < hub_blocks + heavy_blocks) {
    const int64_t li = (b - hub_blocks) * kQPB + threadIdx.x / kGroup;
    const int gl = threadIdx.x % kGroup;
    const int64_t q = li < n_heavy ? int64_t(heavy[li]) : -1;
    if (q < q_lo || q >= q_lo + n_q) return;           // uniform over the group
    const int64_t beg = in_ptr[q], deg = in_ptr[q + 1] - beg;
    if (deg > hub_threshold) return;                    // a hub: a wave writes its row
    const uint32_t base = key_base(uint32_t(q), kc);
    if (k_real > 0) {
      scan_keys<kScanUnroll>(in_src + beg, int32_t(deg), gl, kGroup, base, lk);
      group_merge_keys<kGroup, KR>(lk);
    }
    if (gl == 0) emit_row<KR, KW>(lk, base, k_real, rw_kv, rw_cnt, k_rw, q - q_lo, dedup, table, width, row_len, vec4);
    return;
  }
  const int64_t qi = (b - hub_blocks - heavy_blocks) * kThreads + threadIdx.x;
  if (qi >= n_q) return;
  const int64_t q = q_lo + qi;
  const uint32_t base = key_base(uint32_t(q), kc);
  if (k_real > 0) {
    const int64_t beg = in_ptr[q], end = in_ptr[q + 1];
    if (end - beg > light_max) return;          // a heavy query: a group writes its row
    // 16-byte chunks read up to 3 entries past `end`: only where they stay inside the array
    if ((vec4 & 1) && ((end - 1) | 3) < in_ptr[num_nodes])
      scan_keys_x4<kScanX4Unroll>(in_src, beg, end, base, lk);
    else
      scan_keys<kScanUnroll>(in_src + beg, int32_t(end - beg), 0, 1, base, lk);
  }
  emit_row<KR, KW>(lk, base, k_real, rw_kv, rw_cnt, k_rw, qi, dedup, table, width, row_len, vec4);
}

// One BFS layer of the probe's reception cone (utils/fullgraph_sp_support.py:
// 2261-2309): reached[s] = 1 for every edge s -> v with frontier[v] set. A
// 16-lane group walks v's in-neighbour row; concurrent stores all write 1.
__global__ __launch_bounds__(kThreads) void mark_in_neighbors_kernel(
    const int64_t* __restrict__ in_ptr, const int32_t* __restrict__ in_src, int64_t num_nodes,
    const uint8_t* __restrict__ frontier, uint8_t* __restrict__ reached) {
  const int64_t v = int64_t(blockIdx.x) * kQPB + threadIdx.x / kGroup;
  const int gl = threadIdx.x % kGroup;
  if (v >= num_nodes || !frontier[v]) return;
  const int64_t beg = in_ptr[v], end = in_ptr[v + 1];
  for (int64_t i = beg + gl; i < end; i += kGroup) {
    const int32_t src = in_src[i];
    if (src >= 0 && src < num_nodes) reached[src] = 1;
  }
}

int check_graph(const int64_t* ptr, const int32_t* idx, int64_t num_nodes, int64_t q_lo, int64_t n_q) {
  BF_CHECK_ARG(ptr != nullptr, "edge build: row pointer is NULL");
  BF_CHECK_ARG(num_nodes >= 0 && num_nodes < (int64_t(1) << 31), "edge build: num_nodes %lld outside int32 ids",
               (long long)num_nodes);
  BF_CHECK_ARG(q_lo >= 0 && n_q >= 0 && q_lo + n_q <= num_nodes, "edge build: query range [%lld,%lld) outside [0,%lld)",
               (long long)q_lo, (long long)(q_lo + n_q), (long long)num_nodes);
  (void)idx;
  return BF_OK;
}

// LDS the RW staging may take per block: past 64 KB a block of few queries would lose more to
// occupancy than it gains; 64 KB holds one query of P*L = 8191 candidates. Larger shapes stream
// (rw_select_stream_kernel).
constexpr size_t kRwLdsBytes = size_t(64) << 10;

// Blocks of the one-row-per-workgroup kernels (grid-stride past it): enough to fill the 256 CUs.
constexpr int64_t kWideGrid = 65536;

// The staging slots per query (a power of two >= P*L) and queries per block of a P, L shape; qpb = 0
// (and M2 = 0) when one query's slots exceed the staging LDS.
inline void rw_shape(int P, int L, int& M2, int& qpb) {
  const int64_t M = int64_t(P) * L;
  int64_t m2 = 1;
  while (m2 < M) m2 <<= 1;
  const int64_t by_lds = int64_t(kRwLdsBytes / ((m2 + 1) * sizeof(uint64_t)));
  const int64_t by_threads = kThreads / P;
  qpb = int(by_lds < by_threads ? by_lds : by_threads);
  M2 = qpb >= 1 ? int(m2) : 0;
}

int launch_rw_select(const int64_t* rowptr, const int32_t* col, const void* walk_rec, int64_t num_nodes,
                     int64_t q_lo, const int32_t* qids, int64_t n_q, int P, int L, int K, uint32_t kc, const float* u,
                     uint64_t seed, uint64_t offset, const int64_t* sub_ptr, const int32_t* sub_src,
                     int32_t* sel_kv, int32_t* sel_cnt, hipStream_t st) {
  int M2 = 0, qpb = 0;
  rw_shape(P, L, M2, qpb);
  BF_CHECK_ARG(int64_t(P) * L < (int64_t(1) << 32), "rw_select: walks_per_node * walk_length = %lld candidates per "
               "query (at most 2^32 - 1)", (long long)(int64_t(P) * L));
  BF_CHECK_ARG((reinterpret_cast<uintptr_t>(walk_rec) & 15) == 0, "rw_select: walk records must be 16-byte aligned");
  if (n_q == 0) return BF_OK;
  const int4* rec = static_cast<const int4*>(walk_rec);
  if (qpb < 1) {
    // past the LDS staging: stream the selection, a workgroup per query
    const dim3 grid(unsigned(n_q < kWideGrid ? n_q : kWideGrid));
#define BF_LAUNCH_RW_STREAM(KM)                                                                                   \
  BF_LAUNCH("rw_select_stream_kernel", rw_select_stream_kernel<KM>, grid, dim3(kThreads), 0, st, rowptr, col, rec,  \
            num_nodes, q_lo, qids, n_q, P, L, K, kc, u, seed, offset, sub_ptr, sub_src, sel_kv, sel_cnt)
    if (K <= 8)
      BF_LAUNCH_RW_STREAM(8);
    else
      BF_LAUNCH_RW_STREAM(32);
#undef BF_LAUNCH_RW_STREAM
    BF_CHECK_LAUNCH();
    return BF_OK;
  }
  int R = 1;
  while (R < L) R <<= 1;
  if (P <= 64 && (P & (P - 1)) == 0 && R <= 16) {
    // register sort: P lanes of R candidates each
    const unsigned grid = unsigned(ceil_div(n_q, int64_t(kThreads / P)));
#define BF_LAUNCH_RW_REG(RR)                                                                                        \
  BF_LAUNCH("rw_select_kernel", rw_select_reg_kernel<RR>, dim3(grid), dim3(kThreads), 0, st, rowptr, col, rec,     \
            num_nodes, q_lo, qids, n_q, P, L, K, kc, u, seed, offset, sub_ptr, sub_src, sel_kv, sel_cnt)
    if (R == 1)
      BF_LAUNCH_RW_REG(1);
    else if (R == 2)
      BF_LAUNCH_RW_REG(2);
    else if (R == 4)
      BF_LAUNCH_RW_REG(4);
    else if (R == 8)
      BF_LAUNCH_RW_REG(8);
    else
      BF_LAUNCH_RW_REG(16);
#undef BF_LAUNCH_RW_REG
    BF_CHECK_LAUNCH();
    return BF_OK;
  }
  const size_t lds = size_t(qpb) * (size_t(M2) + 1) * sizeof(uint64_t);
  BF_LAUNCH("rw_select_kernel", rw_select_kernel, dim3(unsigned(ceil_div(n_q, qpb))), dim3(unsigned(qpb * P)), lds, st,
            rowptr, col, rec, num_nodes, q_lo, qids, n_q, P, L, K, M2, qpb, kc, u, seed, offset, sub_ptr, sub_src,
            sel_kv, sel_cnt);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

// Light/heavy split of a range build: every query of the range goes to the
// thread-per-query kernel, which leaves rows with in-degree > light_max to the
// group kernel over `heavy` (those queries of the range, ascending).
struct LightSplit {
  const int32_t* heavy = nullptr;
  int64_t n_heavy = 0;
  int64_t light_max = -1;     // < 0: no split, the group kernel takes every row
};

int launch_real_merge(const int64_t* in_ptr, const int32_t* in_src, int64_t num_nodes, int64_t q_lo,
                      const int32_t* qids, int64_t n_q, int k_real, uint32_t kc, const int32_t* rw_kv,
                      const int32_t* rw_cnt, int k_rw, int dedup, int key_order, int32_t* table, int width,
                      int32_t* row_len, const int32_t* hubs, int64_t n_hubs, int64_t hub_threshold,
                      int32_t* hub_sel, int32_t* hub_cnt, hipStream_t st, LightSplit split = LightSplit()) {
  const int64_t row_ids = int64_t(k_real) + (rw_kv ? k_rw : 0);
  BF_CHECK_ARG(row_ids < (int64_t(1) << 30), "edge build: budget k_real + k_rw = %lld too large",
               (long long)row_ids);
  if (n_q == 0) return BF_OK;
  const bool light = split.light_max >= 0 && qids == nullptr && !key_order && k_real <= 16 &&
                     (rw_kv == nullptr || k_rw <= 16);
  if (k_real <= 0) n_hubs = 0;
  if (light) {
    const int64_t heavy = k_real > 0 ? split.n_heavy : 0;
    const int64_t blocks = ceil_div(n_hubs, int64_t(kHubsPerBlock)) + ceil_div(heavy, int64_t(kQPB)) +
                           ceil_div(n_q, int64_t(kThreads));
    // bit 0: in_src 16-byte aligned (the light rows' 16-byte chunks); kVecTable, kVecRw: emit_row's rows
    const int vec4 = ((reinterpret_cast<uintptr_t>(in_src) & 15) == 0 ? 1 : 0) |
                     ((reinterpret_cast<uintptr_t>(table) & 15) == 0 && width % 4 == 0 ? kVecTable : 0) |
                     (rw_kv && (reinterpret_cast<uintptr_t>(rw_kv) & 15) == 0 && k_rw % 4 == 0 ? kVecRw : 0);
    const int64_t hub_thr = n_hubs > 0 ? hub_threshold : (int64_t(1) << 62);
    const int64_t light_max = k_real > 0 ? split.light_max : (int64_t(1) << 62);
#define BF_LAUNCH_FUSED(KR, KW)                                                                                     \
  BF_LAUNCH("real_select_fused_kernel", (real_select_fused_kernel<KR, KW>), dim3(unsigned(blocks)), dim3(kThreads), \
            0, st, in_ptr, in_src, q_lo, n_q, k_real, kc, rw_kv, rw_cnt, k_rw, dedup, table, width, row_len, hubs,    \
            n_hubs, hub_thr, split.heavy, heavy, light_max, vec4, num_nodes)
    const int kw = rw_kv ? k_rw : 0;
    const int kr = k_real <= 4 ? 4 : k_real <= 8 ? 8 : 16;
    const int kwp = kw <= 4 ? 4 : kw <= 8 ? 8 : 16;
    if (kr == 4 && kwp == 4)
      BF_LAUNCH_FUSED(4, 4);
    else if (kr == 4 && kwp == 8)
      BF_LAUNCH_FUSED(4, 8);
    else if (kr == 8 && kwp == 4)
      BF_LAUNCH_FUSED(8, 4);
    else if (kr == 8 && kwp == 8)
      BF_LAUNCH_FUSED(8, 8);
    else if (kr == 16 && kwp == 16)
      BF_LAUNCH_FUSED(16, 16);
    else if (kr == 16)
      BF_LAUNCH_FUSED(16, 8);
    else
      BF_LAUNCH_FUSED(8, 16);
#undef BF_LAUNCH_FUSED
    BF_CHECK_LAUNCH();
    return BF_OK;
  }
  if (row_ids > kMaxRowCap) {
    // a merged row wider than the LDS staging: a workgroup per row, finished in its table slots
    BF_LAUNCH("merge_rows_wide_kernel", merge_rows_wide_kernel<32>, dim3(unsigned(n_q < kWideGrid ? n_q : kWideGrid)),
              dim3(kThreads), 0, st, in_ptr, in_src, num_nodes, q_lo, qids, n_q, k_real, kc, rw_kv, rw_cnt, k_rw,
              dedup, key_order, table, width, row_len);
    BF_CHECK_LAUNCH();
    return BF_OK;
  }
  if (n_hubs > 0) {
#define BF_LAUNCH_HUB(KM)                                                                                       \
  BF_LAUNCH("real_select_hub_kernel", real_select_hub_kernel<KM>, dim3(unsigned(n_hubs)), dim3(kThreads), 0, st, \
            in_ptr, in_src, hubs, k_real, kc, hub_sel, hub_cnt)
    if (k_real <= 4)
      BF_LAUNCH_HUB(4);
    else if (k_real <= 8)
      BF_LAUNCH_HUB(8);
    else if (k_real <= 16)
      BF_LAUNCH_HUB(16);
    else
      BF_LAUNCH_HUB(32);
#undef BF_LAUNCH_HUB
    BF_CHECK_LAUNCH();
  }
  const dim3 grid(unsigned(ceil_div(n_q, kQPB)));
  const int cap = k_real + (rw_kv ? k_rw : 0) > 0 ? k_real + (rw_kv ? k_rw : 0) : 1;
  const size_t row_lds = size_t(2) * kQPB * cap * sizeof(int32_t);
#define BF_LAUNCH_MERGE(KM)                                                                                      \
  BF_LAUNCH("real_select_merge_kernel", real_select_merge_kernel<KM>, grid, dim3(kThreads), row_lds, st, in_ptr,   \
            in_src, num_nodes, q_lo, qids, n_q, k_real, kc, rw_kv, rw_cnt, k_rw, dedup, key_order, table, width,  \
            row_len, hubs, hub_sel, hub_cnt, n_hubs, hub_threshold, cap)
  if (k_real <= 4)
    BF_LAUNCH_MERGE(4);
  else if (k_real <= 8)
    BF_LAUNCH_MERGE(8);
  else if (k_real <= 16)
    BF_LAUNCH_MERGE(16);
  else
    BF_LAUNCH_MERGE(32);
#undef BF_LAUNCH_MERGE
  BF_CHECK_LAUNCH();
  return BF_OK;
}

inline size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace
}  // namespace bf

using namespace bf;

extern "C" int bf_random_walk(const int64_t* rowptr, const int32_t* col, int64_t num_nodes, int64_t q_lo,
                              int64_t n_q, int32_t walks_per_node, int32_t walk_length, const float* u,
                              uint64_t philox_seed, uint64_t philox_offset, int64_t* walks, void* stream) {
  int rc = check_graph(rowptr, col, num_nodes, q_lo, n_q);
  if (rc) return rc;
  BF_CHECK_ARG(walks_per_node >= 1 && walk_length >= 1, "random_walk: P=%d L=%d must be >= 1", walks_per_node,
               walk_length);
  BF_CHECK_ARG(walks != nullptr || n_q == 0, "random_walk: walks is NULL");
  const int64_t n_walks = n_q * walks_per_node;
  if (n_walks == 0) return BF_OK;
  BF_LAUNCH("random_walk_kernel", random_walk_kernel, dim3(unsigned(ceil_div(n_walks, kThreads))), dim3(kThreads), 0,
                     as_stream(stream), rowptr, col, q_lo, n_walks, walks_per_node, walk_length, u, philox_seed,
                     philox_offset, walks);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int bf_random_walk_starts(const int64_t* rowptr, const int32_t* col, int64_t num_nodes,
                                    const int64_t* starts, int64_t n_walks, int32_t walk_length, const float* u,
                                    uint64_t philox_seed, uint64_t philox_offset, uint64_t walk_id_base,
                                    int64_t* walks, void* stream) {
  int rc = check_graph(rowptr, col, num_nodes, 0, 0);
  if (rc) return rc;
  BF_CHECK_ARG(n_walks >= 0 && walk_length >= 1, "random_walk_starts: n_walks=%lld L=%d", (long long)n_walks,
               walk_length);
  if (n_walks == 0) return BF_OK;
  BF_CHECK_ARG(starts && walks, "random_walk_starts: null tensor");
  BF_LAUNCH("random_walk_starts_kernel", random_walk_starts_kernel, dim3(unsigned(ceil_div(n_walks, kThreads))),
            dim3(kThreads), 0, as_stream(stream), rowptr, col, starts, n_walks, walk_length, u, philox_seed,
            philox_offset, walk_id_base, walks);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int bf_walk_uniforms(int64_t q_lo, int64_t n_q, int32_t walks_per_node, int32_t walk_length,
                                uint64_t philox_seed, uint64_t philox_offset, float* u, void* stream) {
  BF_CHECK_ARG(q_lo >= 0 && n_q >= 0 && walks_per_node >= 1 && walk_length >= 1, "walk_uniforms: bad arguments");
  const int64_t n_walks = n_q * walks_per_node;
  if (n_walks == 0) return BF_OK;
  BF_CHECK_ARG(u != nullptr, "walk_uniforms: u is NULL");
  BF_LAUNCH("walk_uniforms_kernel", walk_uniforms_kernel, dim3(unsigned(ceil_div(n_walks, kThreads))), dim3(kThreads), 0,
                     as_stream(stream), q_lo, n_walks, walks_per_node, walk_length, philox_seed, philox_offset, u);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int bf_walk_records(const int64_t* rowptr, const int32_t* col, int64_t num_nodes, int64_t num_edges,
                               void* records, void* stream) {
  int rc = check_graph(rowptr, col, num_nodes, 0, 0);
  if (rc) return rc;
  // a degree is at most num_edges: below 2^31 it fits the record's 32-bit field
  BF_CHECK_ARG(num_edges >= 0 && num_edges < (int64_t(1) << 31), "walk_records: %lld edges (the records hold "
               "32-bit degrees: at most 2^31 - 1 edges)", (long long)num_edges);
  if (num_edges == 0) return BF_OK;
  BF_CHECK_ARG(col && records, "walk_records: null tensor");
  BF_CHECK_ARG((reinterpret_cast<uintptr_t>(records) & 15) == 0, "walk_records: records must be 16-byte aligned");
  BF_LAUNCH("walk_records_kernel", walk_records_kernel, dim3(unsigned(ceil_div(num_edges, int64_t(kThreads)))),
            dim3(kThreads), 0, as_stream(stream), rowptr, col, num_nodes, num_edges, static_cast<int4*>(records));
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int bf_rw_select(const int64_t* rowptr, const int32_t* col, const void* walk_rec, int64_t num_nodes,
                            int64_t q_lo,
                            int64_t n_q, int32_t walks_per_node, int32_t walk_length, int32_t k_rw,
                            int64_t key_seed, const float* u, uint64_t philox_seed, uint64_t philox_offset,
                            int32_t* sel_kv, int32_t* sel_cnt, void* stream) {
  int rc = check_graph(rowptr, col, num_nodes, q_lo, n_q);
  if (rc) return rc;
  BF_CHECK_ARG(walks_per_node >= 1 && walks_per_node <= kThreads, "rw_select: walks_per_node %d outside [1,%d]",
               walks_per_node, kThreads);
  BF_CHECK_ARG(walk_length >= 1, "rw_select: walk_length %d < 1", walk_length);
  BF_CHECK_ARG(k_rw >= 1, "rw_select: k_rw %d < 1", k_rw);
  BF_CHECK_ARG((sel_kv && sel_cnt) || n_q == 0, "rw_select: null output");
  return launch_rw_select(rowptr, col, walk_rec, num_nodes, q_lo, nullptr, n_q, walks_per_node, walk_length, k_rw,
                          key_const(key_seed), u, philox_seed, philox_offset, nullptr, nullptr, sel_kv, sel_cnt,
                          as_stream(stream));
}

extern "C" int bf_rw_select_rows(const int64_t* rowptr, const int32_t* col, const void* walk_rec, int64_t num_nodes,
                                 const int32_t* qids,
                                 int64_t n_q, int32_t walks_per_node, int32_t walk_length, int32_t k_rw,
                                 int64_t key_seed, const float* u, uint64_t philox_seed, uint64_t philox_offset,
                                 const int64_t* sub_ptr, const int32_t* sub_src, int32_t* sel_kv, int32_t* sel_cnt,
                                 void* stream) {
  int rc = check_graph(rowptr, col, num_nodes, 0, 0);
  if (rc) return rc;
  BF_CHECK_ARG(n_q >= 0 && (qids || n_q == 0), "rw_select_rows: query id list is NULL");
  BF_CHECK_ARG(walks_per_node >= 1 && walks_per_node <= kThreads, "rw_select_rows: walks_per_node %d outside [1,%d]",
               walks_per_node, kThreads);
  BF_CHECK_ARG(walk_length >= 1, "rw_select_rows: walk_length %d < 1", walk_length);
  BF_CHECK_ARG(k_rw >= 1, "rw_select_rows: k_rw %d < 1", k_rw);
  BF_CHECK_ARG((sub_ptr == nullptr) == (sub_src == nullptr), "rw_select_rows: sub_ptr and sub_src go together");
  BF_CHECK_ARG((sel_kv && sel_cnt) || n_q == 0, "rw_select_rows: null output");
  return launch_rw_select(rowptr, col, walk_rec, num_nodes, 0, qids, n_q, walks_per_node, walk_length, k_rw,
                          key_const(key_seed), u, philox_seed, philox_offset, sub_ptr, sub_src, sel_kv, sel_cnt,
                          as_stream(stream));
}

extern "C" int bf_real_select_merge(const int64_t* in_ptr, const int32_t* in_src, int64_t num_nodes, int64_t q_lo,
                                    int64_t n_q, int32_t k_real, int64_t key_seed, const int32_t* rw_kv,
                                    const int32_t* rw_cnt, int32_t k_rw, int32_t dedup, int32_t* table,
                                    int32_t width, int32_t* row_len, const int32_t* hubs, int64_t n_hubs,
                                    int64_t hub_threshold, int32_t* hub_sel, int32_t* hub_cnt, const int32_t* heavy,
                                    int64_t n_heavy, int64_t light_max, void* stream) {
  int rc = check_graph(in_ptr, in_src, num_nodes, q_lo, n_q);
  if (rc) return rc;
  if (k_real < 0) k_real = 0;
  if (rw_kv == nullptr) k_rw = 0;
  BF_CHECK_ARG(k_rw >= 0, "real_select_merge: k_rw=%d < 0", k_rw);
  BF_CHECK_ARG(k_rw == 0 || rw_cnt != nullptr, "real_select_merge: rw_cnt is NULL");
  BF_CHECK_ARG(width >= k_real + k_rw && width >= 1, "real_select_merge: width %d < k_real + k_rw = %d", width,
               k_real + k_rw);
  BF_CHECK_ARG((table && row_len) || n_q == 0, "real_select_merge: null output");
  BF_CHECK_ARG(n_hubs >= 0 && n_hubs < (int64_t(1) << 31), "real_select_merge: bad hub count");
  BF_CHECK_ARG(n_hubs == 0 || (hubs && hub_sel && hub_cnt && hub_threshold >= 0),
               "real_select_merge: hub arrays missing");
  BF_CHECK_ARG(n_heavy >= 0 && (n_heavy == 0 || heavy), "real_select_merge: heavy list missing");
  LightSplit split;
  split.heavy = heavy;
  split.n_heavy = n_heavy;
  split.light_max = light_max;
  return launch_real_merge(in_ptr, in_src, num_nodes, q_lo, nullptr, n_q, k_real, key_const(key_seed),
                           k_rw ? rw_kv : nullptr, rw_cnt, k_rw, dedup ? 1 : 0, 0, table, width, row_len, hubs, n_hubs,
                           hub_threshold, hub_sel, hub_cnt, as_stream(stream), split);
}

extern "C" int bf_real_select_rows(const int64_t* in_ptr, const int32_t* in_src, int64_t num_nodes,
                                   const int32_t* qids, int64_t n_q, int32_t k_real, int64_t key_seed,
                                   const int32_t* hubs, int64_t n_hubs, int64_t hub_threshold, int32_t* hub_sel,
                                   int32_t* hub_cnt, int32_t* sel_kv, int32_t* sel_cnt, void* stream) {
  int rc = check_graph(in_ptr, in_src, num_nodes, 0, 0);
  if (rc) return rc;
  BF_CHECK_ARG(n_q >= 0 && (qids || n_q == 0), "real_select_rows: query id list is NULL");
  BF_CHECK_ARG(k_real >= 1, "real_select_rows: k_real %d < 1", k_real);
  BF_CHECK_ARG((sel_kv && sel_cnt) || n_q == 0, "real_select_rows: null output");
  BF_CHECK_ARG(n_hubs >= 0 && n_hubs < (int64_t(1) << 31), "real_select_rows: bad hub count");
  BF_CHECK_ARG(n_hubs == 0 || (hubs && hub_sel && hub_cnt && hub_threshold >= 0),
               "real_select_rows: hub arrays missing");
  return launch_real_merge(in_ptr, in_src, num_nodes, 0, qids, n_q, k_real, key_const(key_seed), nullptr, nullptr, 0,
                           0, 1, sel_kv, k_real, sel_cnt, hubs, n_hubs, hub_threshold, hub_sel, hub_cnt,
                           as_stream(stream));
}

extern "C" int bf_assemble_rows(const int32_t* real_kv, const int32_t* real_cnt, int32_t real_stride, int32_t b_real,
                                const int32_t* rw_kv, const int32_t* rw_cnt, int32_t rw_stride, int32_t b_rw,
                                int32_t dedup, int64_t n_rows, int32_t* table, int32_t width, int32_t* row_len,
                                void* stream) {
  BF_CHECK_ARG(n_rows >= 0, "assemble_rows: n_rows < 0");
  if (real_kv == nullptr) b_real = 0;
  if (rw_kv == nullptr) b_rw = 0;
  BF_CHECK_ARG(b_real >= 0 && b_rw >= 0, "assemble_rows: negative budget");
  BF_CHECK_ARG(b_real <= real_stride || real_kv == nullptr, "assemble_rows: b_real %d exceeds the real stride %d",
               b_real, real_stride);
  BF_CHECK_ARG(b_rw <= rw_stride || rw_kv == nullptr, "assemble_rows: b_rw %d exceeds the RW stride %d", b_rw,
               rw_stride);
  BF_CHECK_ARG(int64_t(b_real) + b_rw < (int64_t(1) << 30), "assemble_rows: b_real + b_rw too large");
  BF_CHECK_ARG(width >= b_real + b_rw && width >= 1, "assemble_rows: width %d < %d", width, b_real + b_rw);
  BF_CHECK_ARG((b_real == 0 || real_cnt) && (b_rw == 0 || rw_cnt), "assemble_rows: counts missing");
  BF_CHECK_ARG((table && row_len) || n_rows == 0, "assemble_rows: null output");
  if (n_rows == 0) return BF_OK;
  if (b_real + b_rw > kMaxRowCap) {
    // a row wider than the LDS staging: a workgroup per row, finished in its table slots
    BF_LAUNCH("assemble_rows_wide_kernel", assemble_rows_wide_kernel,
              dim3(unsigned(n_rows < kWideGrid ? n_rows : kWideGrid)), dim3(kThreads), 0, as_stream(stream),
              b_real ? real_kv : nullptr, real_cnt, real_stride, b_real, b_rw ? rw_kv : nullptr, rw_cnt, rw_stride,
              b_rw, dedup ? 1 : 0, n_rows, table, width, row_len);
    BF_CHECK_LAUNCH();
    return BF_OK;
  }
  const int cap = b_real + b_rw > 0 ? b_real + b_rw : 1;
  BF_LAUNCH("assemble_rows_kernel", assemble_rows_kernel, dim3(unsigned(ceil_div(n_rows, kQPB))), dim3(kThreads),
            size_t(2) * kQPB * cap * sizeof(int32_t), as_stream(stream), b_real ? real_kv : nullptr, real_cnt,
            real_stride, b_real, b_rw ? rw_kv : nullptr, rw_cnt, rw_stride, b_rw, dedup ? 1 : 0, n_rows, table, width,
            row_len, cap);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

extern "C" int bf_build_edge_table_workspace_size(int64_t n_q, int32_t k_rw, int64_t n_hubs, int32_t k_real,
                                                  size_t* bytes) {
  BF_CHECK_ARG(bytes && n_q >= 0 && k_rw >= 0 && n_hubs >= 0, "build_edge_table_workspace_size: bad arguments");
  const size_t kr = size_t(k_real > 0 ? k_real : 0);
  *bytes = align_up(size_t(n_q) * size_t(k_rw > 0 ? k_rw : 0) * 4) + align_up(size_t(n_q) * 4) +
           align_up(size_t(n_hubs) * kr * 4) + align_up(size_t(n_hubs) * 4) + 256;
  return BF_OK;
}

extern "C" int bf_build_edge_table(const int64_t* rowptr, const int32_t* col, const void* walk_rec,
                                   const int64_t* in_ptr, const int32_t* in_src, int64_t num_nodes, int64_t num_edges, int64_t q_lo,
                                   int64_t n_q, int32_t walks_per_node, int32_t walk_length, int32_t k_real,
                                   int32_t k_rw, int64_t edge_seed, const float* u, uint64_t philox_seed,
                                   uint64_t philox_offset, const int32_t* hubs, int64_t n_hubs,
                                   int64_t hub_threshold, const int32_t* heavy, int64_t n_heavy,
                                   int64_t light_max, int32_t* table, int32_t* row_len, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  BF_CHECK_ARG(num_edges >= 0, "build_edge_table: num_edges < 0");
  const bool use_rw = k_rw > 0 && walks_per_node > 0 && walk_length > 0 && num_nodes > 0;
  const bool use_real = k_real > 0 && num_edges > 0;
  const int32_t width = (k_real > 0 ? k_real : 0) + (k_rw > 0 ? k_rw : 0);
  BF_CHECK_ARG(width >= 1, "build_edge_table: empty budget (k_real=%d, k_rw=%d)", k_real, k_rw);
  if (!use_real) n_hubs = 0;
  size_t need = 0;
  bf_build_edge_table_workspace_size(n_q, use_rw ? k_rw : 0, n_hubs, k_real, &need);
  BF_CHECK_ARG(workspace && workspace_bytes >= need, "build_edge_table: workspace %zu < %zu bytes",
               workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  char* wp = static_cast<char*>(workspace);
  int32_t* sel_kv = reinterpret_cast<int32_t*>(wp);
  wp += align_up(size_t(n_q) * size_t(use_rw ? k_rw : 0) * 4);
  int32_t* sel_cnt = reinterpret_cast<int32_t*>(wp);
  wp += align_up(size_t(n_q) * 4);
  int32_t* hub_sel = reinterpret_cast<int32_t*>(wp);
  wp += align_up(size_t(n_hubs) * size_t(k_real > 0 ? k_real : 0) * 4);
  int32_t* hub_cnt = reinterpret_cast<int32_t*>(wp);
  if (use_rw) {
    int rc = bf_rw_select(rowptr, col, walk_rec, num_nodes, q_lo, n_q, walks_per_node, walk_length, k_rw,
                          edge_seed + 37, u, philox_seed, philox_offset, sel_kv, sel_cnt, st);
    if (rc) return rc;
  }
  // the reference coalesces only when both parts are globally non-empty
  return bf_real_select_merge(in_ptr, in_src, num_nodes, q_lo, n_q, use_real ? k_real : 0, edge_seed + 17,
                              use_rw ? sel_kv : nullptr, use_rw ? sel_cnt : nullptr, use_rw ? k_rw : 0,
                              (use_real && use_rw) ? 1 : 0, table, width, row_len, hubs, n_hubs, hub_threshold,
                              hub_sel, hub_cnt, heavy, n_heavy, light_max, st);
}

extern "C" int bf_mark_in_neighbors(const int64_t* in_ptr, const int32_t* in_src, int64_t num_nodes,
                                    const uint8_t* frontier, uint8_t* reached, void* stream) {
  int rc = check_graph(in_ptr, in_src, num_nodes, 0, 0);
  if (rc) return rc;
  if (num_nodes == 0) return BF_OK;
  BF_CHECK_ARG(in_src && frontier && reached, "mark_in_neighbors: null tensor");
  BF_LAUNCH("mark_in_neighbors_kernel", mark_in_neighbors_kernel, dim3(unsigned(ceil_div(num_nodes, kQPB))),
            dim3(kThreads), 0, as_stream(stream), in_ptr, in_src, num_nodes, frontier, reached);
  BF_CHECK_LAUNCH();
  return BF_OK;
}
