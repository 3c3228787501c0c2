// Sparse edge attention, forward and backward, for gfx950.
//
// Semantics: models/graphormer_dist_node_level.py:215-263 (GT :215-262, GraphGPS
// models/graphgps_dist_node_level.py:151-177 through the per-edge factor):
//   a = clamp(sum_j k[s,h,j] * q[t,h,j] / sqrt(hn), -c, c) [+ bias[e,h]]
//   p = exp(a)   (no max subtraction; the clamp bounds it when bias is absent)
// with c = 5 on every path but GT's per-head edge lists
// (models/gt_dist_node_level.py:195-218), which clamp the dot product to
// [-5, 5] before the scaling: exp(clamp(x, -5, 5) / sqrt(hn)) is the same
// expression with c = 5 / sqrt(hn).
//   Z[t,h] = sum_e p,  out[t,h,:] = sum_e p * f[e,h] * v[s,h,:] / (Z[t,h] + 1e-6)
//
// Work mapping. A row of D = H*hn activations is split across a group of
// LPR = D/EPL lanes (EPL = elements per 16-byte load: 4 fp32 or 8 bf16), so a
// 64-lane wavefront serves 64/LPR rows at once and every gather of a K/V/Q/dO
// row is one fully coalesced dwordx4 per lane. Per-head dot products reduce
// over LPH = hn/EPL lanes with xor shuffles. Rows (queries in the forward and
// the dq pass, key/value nodes in the dk/dv pass) are walked sequentially by
// their group, several edges per iteration so that their gathers overlap.
// Rows longer than `chunk` (the Graphormer global token row, hub key/value
// nodes) are cut into items by a split plan; items write float partials that
// a reduce sums in item order. Nothing uses atomics: results are deterministic
// run to run. Launches per layer: forward (items + rows), forward reduce,
// dq pass (items + rows), dq reduce, dk/dv pass (items + rows), dk/dv reduce
// (each reduce only when some split row has more than one item).
//
// MFMA is not used: each score is an hn-long dot product of two gathered rows,
// not a dense contraction, and the kernels are bound by gather bandwidth.
#include "bf_common.h"

#include <algorithm>
#include <mutex>

namespace bf {
namespace {

constexpr int kBlock = 256;
// Edges whose gathers are in flight together per group, per pass and element
// type (measured on MI355X: more edges per group cost registers, hence waves).
// Four where they fit the same waves or win anyway: the bf16 dq pass (94
// VGPRs, five waves as with three: c4's dq 2.72 -> 2.61 ms) and the fp32
// forward (66 VGPRs, seven waves instead of eight: c2 131 -> 130 us); three
// elsewhere (the fp32 dq pass at four loses two waves and 7%, the bf16 kv
// pass a wave).
#ifndef BF_UNROLL_FWD_F32
#define BF_UNROLL_FWD_F32 4
#endif
#ifndef BF_UNROLL_FWD_BF16
#define BF_UNROLL_FWD_BF16 3
#endif
#ifndef BF_UNROLL_Q_F32
#define BF_UNROLL_Q_F32 3
#endif
#ifndef BF_UNROLL_Q_BF16
#define BF_UNROLL_Q_BF16 4
#endif
#ifndef BF_UNROLL_KV_F32
#define BF_UNROLL_KV_F32 3
#endif
#ifndef BF_UNROLL_KV_BF16
#define BF_UNROLL_KV_BF16 3
#endif
// The dk/dv pass over cache-resident q and dO tables (the instance that gathers them with normal loads):
// two entries in flight in float32 (c2: 0.196 -> 0.192 ms against three; four 0.202 ms; one, at seven
// waves in 66 VGPRs, 0.196 against 0.189 for two at six); the streaming instance keeps `kv`.
#ifndef BF_UNROLL_KV_CACHED_F32
#define BF_UNROLL_KV_CACHED_F32 2
#endif
// The dk/dv pass with the in-kernel dropout (EX = 1): two entries in flight, whose registers leave room
// for the Philox draw at four waves per SIMD (bf16 four-row instance 121 VGPRs, against 135 and three
// waves with three entries: c4 3.97 -> 3.86 ms).
#ifndef BF_UNROLL_KV_DROPOUT
#define BF_UNROLL_KV_DROPOUT 2
#endif
// The typed-edge (Exphormer) passes: entries in flight of the dk/dv segment and the dq pass (0: the
// untyped pass's setting). Two in the dk/dv segment (bf16 instances 157-171 VGPRs, three waves for most,
// against 181-194 and two): a typed backward over 2.45M queries of 12 entries, 6.90 -> 6.75 ms; the dq
// pass at three or two entries was slower (7.00, 6.92 ms).
#ifndef BF_UNROLL_KV_TYPED
#define BF_UNROLL_KV_TYPED 2
#endif
#ifndef BF_UNROLL_Q_TYPED
#define BF_UNROLL_Q_TYPED 0
#endif
template <typename T> struct Unroll;
template <> struct Unroll<float> {
  static constexpr int fwd = BF_UNROLL_FWD_F32, q = BF_UNROLL_Q_F32, kv = BF_UNROLL_KV_F32,
                       kv_cached = BF_UNROLL_KV_CACHED_F32;
};
template <> struct Unroll<uint16_t> {
  static constexpr int fwd = BF_UNROLL_FWD_BF16, q = BF_UNROLL_Q_BF16, kv = BF_UNROLL_KV_BF16,
                       kv_cached = BF_UNROLL_KV_BF16;
};
template <> struct Unroll<_Float16> {   // the same row bytes and lane mapping as bf16
  static constexpr int fwd = BF_UNROLL_FWD_BF16, q = BF_UNROLL_Q_BF16, kv = BF_UNROLL_KV_BF16,
                       kv_cached = BF_UNROLL_KV_BF16;
};
constexpr float kEps = 1e-6f;
constexpr float kClamp = 5.0f;   // the reference's clamp bound, the default

struct Shape {
  int D;          // H * hn
  int H;
  int lpr_log2;   // lanes per row (power of two)
  int lph_log2;   // lanes per head (power of two)
  int act_lanes;  // D / EPL lanes carry data; the rest of the group idles
  float inv_scale;
  float clamp;    // scores are clamped to [-clamp, clamp] after the 1/sqrt(hn) scaling
};

struct GroupPos {
  int g_lane;
  int head;
  int col0;
  bool act;
  bool lead;      // first lane of its head
};

template <typename T>
__device__ __forceinline__ GroupPos group_pos(const Shape& sh) {
  constexpr int V = Elem<T>::kPerVec;
  GroupPos g;
  g.g_lane = threadIdx.x & ((1 << sh.lpr_log2) - 1);
  g.act = g.g_lane < sh.act_lanes;
  g.head = g.act ? (g.g_lane >> sh.lph_log2) : 0;  // idle lanes never index past H
  g.col0 = g.g_lane * V;
  g.lead = g.act && ((g.g_lane & ((1 << sh.lph_log2) - 1)) == 0);
  return g;
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::Raw load_row_raw(const T* base, int64_t row, int D, const GroupPos& g) {
  return g.act ? Elem<T>::load_raw(base + row * D + g.col0) : Elem<T>::zero_raw();
}

// A pass's own rows (read or written once, in row order) go past the caches:
// the caches then keep the rows the pass gathers at random (c2 query-side
// passes: 5% faster; c5: 4-5%).
template <typename T>
__device__ __forceinline__ typename Elem<T>::Raw load_row_raw_nt(const T* base, int64_t row, int D, const GroupPos& g) {
  return g.act ? Elem<T>::load_raw_nt(base + row * D + g.col0) : Elem<T>::zero_raw();
}

// ------------------------------------------------------------------ per-entry inputs
// Beyond q, k and v an entry may carry an additive bias (after the clamp), a
// factor on its V message (any caller factor), and the GraphGPS attention
// dropout (models/graphgps_dist_node_level.py:166-176), drawn here rather than
// read from a mask: the entry at slot s of query row r (its place in the row's
// ascending kv order) and head h are kept iff u < 1 - rate, u = word h % 4 of
// Philox4x32-10(counter (s, r, offset + h / 4), key seed) mapped to
// (x >> 8) * 2^-24, and a kept entry's V message is scaled by 1 / (1 - rate).
// The three passes evaluate the same bit: the query-major passes know (r, s)
// from the row they walk, the key-major pass from the reverse entry's query
// and slot, so no pass needs an entry's CSR position for it.
// With a keep mask (keepm: byte b of entry e at e * kbytes + b holds heads
// 8b .. 8b + 7, bit h % 8) the forward also stores the bits it draws, and the
// dq pass reads them back instead of drawing them again (EX = 4): the Philox
// rounds cost that pass a wave per SIMD while its rows are in flight. The
// key-major pass, which meets the entries in reverse-index order, keeps drawing.
struct EdgeIn {
  const float* bias;     // float32 [nnz, H] or NULL
  const float* factor;   // float32 [nnz, H] or NULL
  const float* mod;      // typed edges (EX = 3 only): E, float32 [2, H * hn]
  int drop;              // 1: the dropout factor applies
  float keep;            // kept iff u < keep (= 1 - rate)
  float scale;           // factor of a kept entry (1 / (1 - rate); 0 when rate = 1)
  uint32_t seed_lo, seed_hi, off_lo, off_hi;
  uint8_t* keepm;        // NULL, or the keep mask, uint8 [nnz, kbytes] in CSR order
  int kbytes;            // ceil(H / 8)
};

// Keep bits of the entry at slot s of query row r for heads 4*blk .. 4*blk + 3 (bit j: head 4*blk + j),
// one Philox call.
__device__ __forceinline__ uint32_t keep_bits4(const EdgeIn& x, int32_t r, int32_t s, int blk) {
  const uint64_t b = ((uint64_t(x.off_hi) << 32) | x.off_lo) + uint64_t(blk);
  const U32x4 o = philox4x32_10(U32x4{uint32_t(s), uint32_t(r), uint32_t(b), uint32_t(b >> 32)}, x.seed_lo,
                                x.seed_hi);
  return (u24(o.x) < x.keep ? 1u : 0u) | (u24(o.y) < x.keep ? 2u : 0u) | (u24(o.z) < x.keep ? 4u : 0u) |
         (u24(o.w) < x.keep ? 8u : 0u);
}

__device__ __forceinline__ float dropout_factor(const EdgeIn& x, int32_t r, int32_t s, int head) {
  return ((keep_bits4(x, r, s, head >> 2) >> (head & 3)) & 1u) ? x.scale : 0.f;
}

// The keep bits of one iteration's kUnroll entries (query rows rows[u], slots slots[u]), drawn once per
// group: lane j < kUnroll * nb (nb = ceil(H / 4) Philox blocks per entry) draws block j % nb of entry
// j / nb, and every lane then takes its head's bit by a shuffle (iter_factor), instead of each lane
// drawing the block of its own head for every entry (shared). Groups narrower than kUnroll * nb lanes
// draw their own head's bit of every entry here (bit u of task), so the rows and slots are dead after.
template <int kUnroll>
struct IterDrop {
  bool shared;
  uint32_t task;   // shared: this lane's 4 keep bits of its (entry, block); else bit u: entry u, this lane's head
};

template <int kUnroll>
__device__ __forceinline__ IterDrop<kUnroll> iter_drop(const EdgeIn& x, const int32_t (&rows)[kUnroll],
                                                       const int32_t (&slots)[kUnroll], const bool (&ok)[kUnroll],
                                                       const Shape& sh, const GroupPos& g) {
  IterDrop<kUnroll> it{false, 0u};
  if (!x.drop) return it;
  const int nb = (sh.H + 3) >> 2;
  it.shared = kUnroll * nb <= (1 << sh.lpr_log2);
  if (!it.shared) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (ok[u]) it.task |= ((keep_bits4(x, rows[u], slots[u], g.head >> 2) >> (g.head & 3)) & 1u) << u;
    return it;
  }
  const int j = g.g_lane;
  if (j < kUnroll * nb) {
    const int u = j / nb, blk = j - u * nb;
    int32_t r = 0, s = 0;
    bool live = false;
#pragma unroll
    for (int w = 0; w < kUnroll; ++w) {
      if (w == u) {
        r = rows[w];
        s = slots[w];
        live = ok[w];
      }
    }
    if (live) it.task = keep_bits4(x, r, s, blk);
  }
  return it;
}

// V-message factor of entry u of the iteration (CSR position e, which only a caller factor reads) for
// this lane's head: the caller's factor times the dropout factor. Every lane of the group calls it for
// the same u.
template <int kUnroll, int EX>
__device__ __forceinline__ float iter_factor(const EdgeIn& x, const IterDrop<kUnroll>& it, int u, int64_t e,
                                             const Shape& sh, int head) {
  float f = (EX == 2 && x.factor) ? x.factor[e * sh.H + head] : 1.f;
  if (EX == 1 || x.drop) {
    uint32_t keep;
    if (it.shared) {
      const int nb = (sh.H + 3) >> 2;
      keep = (uint32_t(__shfl(int(it.task), u * nb + (head >> 2), 1 << sh.lpr_log2)) >> (head & 3)) & 1u;
    } else {
      keep = (it.task >> u) & 1u;
    }
    f *= keep ? x.scale : 0.f;
  }
  return f;
}

// The dropout factor of head `head` from an entry's keep-mask byte (the byte that holds the head).
__device__ __forceinline__ float mask_factor(const EdgeIn& x, uint32_t byte, int head) {
  return ((byte >> (head & 7)) & 1u) ? x.scale : 0.f;
}

// The V-message factor of a single entry (CSR position e, slot s of query row r) for this lane's head
// (1 without factor and dropout). EX == 4 reads the keep mask the forward wrote.
template <int EX>
__device__ __forceinline__ float edge_factor(const EdgeIn& x, int64_t e, int32_t r, int32_t s, const Shape& sh,
                                             int head) {
  float f = (EX == 2 && x.factor) ? x.factor[e * sh.H + head] : 1.f;
  if (EX == 4)   // one byte per entry (H <= 8)
    f *= mask_factor(x, x.keepm[e], head);
  else if (EX == 1 || x.drop)
    f *= dropout_factor(x, r, s, head);
  return f;
}

// Stores the keep bits of one iteration's entries (CSR positions e0 + u, those below `end`) into the keep
// mask: byte b of an entry holds heads 8b .. 8b + 7, i.e. Philox blocks 2b (low nibble) and 2b + 1 (high).
// With shared draws lane u * nb + blk holds the bits of (entry u, block blk); lane u * kbytes + b fetches
// the two nibbles of its byte by shuffles and stores it (with one byte per entry, lane u stores entry u's).
// Otherwise every lane holds its own head's bit of each entry (bit u), and the writer of each byte collects
// bit u from the first lane of each of its heads. Every lane of the group takes part in the shuffles;
// nothing is drawn again.
// The general instance's form (any head count and group width); the dropout-only instance stores its
// mask a window at a time (keep_window_add).
template <int kUnroll>
__device__ __forceinline__ void store_keep(const EdgeIn& x, const IterDrop<kUnroll>& it, int64_t e0, int64_t end,
                                           const Shape& sh, const GroupPos& g) {
  const int nb = (sh.H + 3) >> 2;
  if (it.shared) {
    const int j = g.g_lane;
    const int u = x.kbytes == 1 ? j : j / x.kbytes, b = j - u * x.kbytes;
    const int src = u * nb + 2 * b;                 // past the group for idle lanes: wraps, unused
    const uint32_t lo = uint32_t(__shfl(int(it.task), src, 1 << sh.lpr_log2));
    const uint32_t hi = uint32_t(__shfl(int(it.task), src + 1, 1 << sh.lpr_log2));
    if (u < kUnroll && e0 + u < end)
      x.keepm[(e0 + u) * x.kbytes + b] = uint8_t((lo & 15u) | (2 * b + 1 < nb ? (hi & 15u) << 4 : 0u));
  } else {
    // narrow groups (fewer lanes than the iteration has bytes, possibly): in rounds of the group's width,
    // lane w = round * lpr + j (w = u * kbytes + b) collects bit u of each head of its byte from the
    // head's first lane; every lane takes part in every round's shuffles
    const int lpr = 1 << sh.lpr_log2;
    const int n = kUnroll * x.kbytes;
    for (int w0 = 0; w0 < n; w0 += lpr) {
      const int w = w0 + g.g_lane;
      const int u = x.kbytes == 1 ? w : w / x.kbytes, b = w - u * x.kbytes;
      uint32_t byte = 0;
#pragma unroll
      for (int h = 0; h < 8; ++h) {
        const int hh = 8 * b + h;
        const uint32_t t = uint32_t(__shfl(int(it.task), hh << sh.lph_log2, lpr));
        if (hh < sh.H) byte |= ((t >> (u & 31)) & 1u) << h;
      }
      if (u < kUnroll && e0 + u < end) x.keepm[(e0 + u) * x.kbytes + b] = uint8_t(byte);
    }
  }
}

// The keep mask of the dropout-only forward (one byte per entry, groups that share an iteration's draws),
// stored a window at a time: lane j of the group owns entry w0 + j of a window of `len` entries (the group's
// width rounded down to whole iterations, so no iteration straddles two windows: for the 2-byte types the
// id chunk of ChunkIds), takes its byte's two nibbles straight from the lanes that drew them (lane
// u * nb + blk holds block blk of entry u), and the window goes out as one store of len consecutive bytes
// once its last iteration is done (or the segment ends). Byte stores per iteration instead left each row's
// bytes to be written a few at a time, the lines partly written and evicted between writes (c4 forward
// 2.13 -> 2.37 ms, windows 2.29 ms). Storing each segment's last window after the walk, so that the groups
// of a wave store together, cost the instance its sixth wave and was slower (2.40 ms). Returns whether the
// window was stored (the caller's window then starts at w0 + len).
// buf: this lane's byte; for the 2-byte types the lane's id register of the chunk, dead once the
// iteration that takes the lane's entry has shuffled it out (the lane's byte arrives in that iteration, and
// the window is stored before the next chunk's ids are loaded), which spares the instance a register.
template <int kUnroll>
__device__ __forceinline__ bool keep_window_add(const EdgeIn& x, const IterDrop<kUnroll>& it, int& buf,
                                                int64_t w0, int len, int64_t e0, int64_t end, const Shape& sh,
                                                const GroupPos& g) {
  const int nb = (sh.H + 3) >> 2;
  const int lpr = 1 << sh.lpr_log2;
  const int u = g.g_lane - int(e0 - w0);          // this lane's entry of the iteration, if 0 <= u < kUnroll
  const int src = (u >= 0 && u < kUnroll ? u : 0) * nb;
  const uint32_t lo = uint32_t(__shfl(int(it.task), src, lpr));
  const uint32_t hi = uint32_t(__shfl(int(it.task), src + 1, lpr));
  if (u >= 0 && u < kUnroll) buf = int((lo & 15u) | (nb > 1 ? (hi & 15u) << 4 : 0u));
  if (e0 + kUnroll >= w0 + len || e0 + kUnroll >= end) {   // the window's last iteration (uniform)
    if (g.g_lane < len && w0 + g.g_lane < end) x.keepm[w0 + g.g_lane] = uint8_t(buf);
    return true;
  }
  return false;
}

// The keep-mask bytes of entries e0 .. e0 + 3 (one byte per entry: H <= 8) of a row ending at `end`, as
// the two aligned dwords that hold them: w0 at e0 & ~3 and, only when the row has entries past it, w1 (no
// load reaches past the row's last byte, so none past the mask). Byte of entry e0 + u: keep_byte(w, o, u).
struct KeepWords {
  uint32_t w0, w1;
  int o;   // e0 & 3
};

__device__ __forceinline__ KeepWords load_keep_words(const uint8_t* __restrict__ keepm, int64_t e0, int64_t end) {
  const int64_t a = e0 >> 2;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(keepm);
  KeepWords k;
  k.o = int(e0 & 3);
  k.w0 = w[a];                                    // bytes 4a .. 4a + 3: e0 is one of them
  k.w1 = 4 * a + 4 < end ? w[a + 1] : 0u;
  return k;
}

__device__ __forceinline__ uint32_t keep_byte(const KeepWords& k, int u) {
  const int sh = 8 * (k.o + u);                   // 0 .. 48
  return (sh < 32 ? (k.w0 >> sh) : (k.w1 >> (sh - 32))) & 0xffu;
}

__device__ __forceinline__ float edge_bias(const EdgeIn& x, int64_t e, const Shape& sh, int head) {
  return x.bias ? x.bias[e * sh.H + head] : 0.f;
}

// ------------------------------------------------------------------ forward
// Entry ids of a row walked kUnroll at a time. bf16: a chunk of them comes in
// one coalesced load, one id per lane of the group, and each iteration takes
// its ids by lane shuffle, so the gathers wait for one id load per chunk
// instead of one per iteration (chunks are a whole number of iterations).
// float32: loaded per iteration (the id register would cost a wave per SIMD).
// A group narrower than kUnroll lanes (bf16 rows of 8 or 16 elements) cannot
// hold one iteration's ids and loads them per iteration as well (len = 0).
template <typename T, int kUnroll>
struct ChunkIds {
  static constexpr bool kChunk = sizeof(T) == 2;
  int lpr, len;
  int64_t c0;
  int ids = 0;
  __device__ __forceinline__ ChunkIds(const Shape& sh, int64_t beg)
      : lpr(1 << sh.lpr_log2),
        len((1 << sh.lpr_log2) >= kUnroll ? ((1 << sh.lpr_log2) / kUnroll) * kUnroll : 0),
        c0(beg - len) {}
  // The ids of entries e0 .. e0 + kUnroll - 1 (0 for those at or past `end`, with ok false), every
  // lane of the group calling it with the same e0. All of an iteration's ids are in registers before
  // any of its row gathers is issued, and the gathers are issued unconditionally (rows past the end
  // read row 0): a gather issued under a branch, or an id load between two gathers, makes the compiler
  // wait for the earlier gathers before the next one is issued, which leaves one row in flight.
  __device__ __forceinline__ void fetch(const int32_t* __restrict__ idx, int64_t e0, int64_t end,
                                        const GroupPos& g, int (&s)[kUnroll], bool (&ok)[kUnroll]) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) ok[u] = e0 + u < end;
    if constexpr (kChunk) {
      if (len > 0) {
        if (e0 - c0 == len) {   // the start of a chunk (uniform over the group): load its ids
          c0 = e0;
          ids = (g.g_lane < len && c0 + g.g_lane < end) ? idx[c0 + g.g_lane] : 0;
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) s[u] = __shfl(ids, int(e0 - c0) + u, lpr);
        return;
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int id = idx[ok[u] ? e0 + u : end - 1];
      s[u] = ok[u] ? id : 0;
    }
  }
};

// Column of this lane's 16 bytes in a gathered row: idle lanes (past D) read the first 16 bytes, so
// that every lane issues the same loads and none reads past the row; their values are never used.
__device__ __forceinline__ int gather_col(const GroupPos& g) { return g.act ? g.col0 : 0; }
// Accumulates sum_e p*f*v (acc) and sum_e p (z) over entries [beg, end) of one row.
// EX: the per-entry inputs compiled in (0 none, 1 dropout only, 2 bias, factor and dropout): each
// instance carries only the code, and the registers, of what it uses.
template <typename T, int EX>
__device__ __forceinline__ void fwd_segment(const T* __restrict__ k, const T* __restrict__ v,
                                            const int32_t* __restrict__ kv, const EdgeIn& ex,
                                            int64_t beg, int64_t end, int32_t row, int64_t row_beg,
                                            const Shape& sh, const GroupPos& g,
                                            const typename Elem<T>::Raw& qr,
                                            float (&acc)[Elem<T>::kPerVec], float& z) {
  constexpr int V = Elem<T>::kPerVec;
  constexpr int kUnroll = Unroll<T>::fwd;
  const int lph = 1 << sh.lph_log2;
  ChunkIds<T, kUnroll> ids(sh, beg);
  int kbuf = 0;                                   // EX == 4, float32: this lane's byte of the keep window
  int64_t kw0 = beg;                              // and the window's start (2-byte types: ids.ids, ids.c0)
  const int col = gather_col(g);
  for (int64_t e0 = beg; e0 < end; e0 += kUnroll) {
    int s[kUnroll];
    bool ok[kUnroll];
    ids.fetch(kv, e0, end, g, s, ok);
    typename Elem<T>::Raw kr[kUnroll], vr[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      kr[u] = Elem<T>::load_raw(k + int64_t(s[u]) * sh.D + col);
      vr[u] = Elem<T>::load_raw(v + int64_t(s[u]) * sh.D + col);
    }
    float d[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) d[u] = Elem<T>::dot(kr[u], qr, 0.f);
    for (int o = 1; o < lph; o <<= 1) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) d[u] += __shfl_xor(d[u], o, 64);
    }
    IterDrop<kUnroll> drop{false, 0u};
    if (EX) {
      int32_t rows[kUnroll], slots[kUnroll];   // the dropout's (query row, slot) of each entry
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        rows[u] = row;
        slots[u] = int32_t(e0 + u - row_beg);
      }
      drop = iter_drop<kUnroll>(ex, rows, slots, ok, sh, g);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (!ok[u]) continue;
      const int64_t e = e0 + u;
      float a = fminf(fmaxf(d[u] * sh.inv_scale, -sh.clamp), sh.clamp);
      if (EX == 2) a += edge_bias(ex, e, sh, g.head);
      const float p = __expf(a);   // a is clamped to [-5, 5] (+ bias): exp2-based form is within 2 ulp
      const float w = EX ? p * iter_factor<kUnroll, EX>(ex, drop, u, e, sh, g.head) : p;
      float vv[V];
      Elem<T>::unpack(vr[u], vv);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = fmaf(w, vv[i], acc[i]);
      z += p;
    }
    // the keep mask, once the iteration's rows are spent (stored earlier, its temporaries would sit beside
    // the V rows still in flight)
    if constexpr (EX == 4) {
      const int klen = ((1 << sh.lpr_log2) / kUnroll) * kUnroll;   // = ids.len for the 2-byte types
      constexpr bool kChunk = ChunkIds<T, kUnroll>::kChunk;
      if (keep_window_add<kUnroll>(ex, drop, kChunk ? ids.ids : kbuf, kChunk ? ids.c0 : kw0, klen, e0, end, sh,
                                   g))
        kw0 += klen;
    }
    if (EX == 2 && ex.drop && ex.keepm) store_keep<kUnroll>(ex, drop, e0, end, sh, g);
  }
}

// ------------------------------------------------------------------ split rows
// A split item: entries [beg, end) of one long row, processed by a whole
// workgroup; each LPR-lane group takes a contiguous sub-range and the groups'
// sums are combined through LDS in group order. Every pass runs as ONE launch
// whose first workgroups take the items (the longest work, dispatched first)
// and whose remaining workgroups take the short rows, so the items overlap the
// row work instead of running as a tail of their own.
struct Items {
  const int64_t* ptr;
  const int32_t* item_off;
  const int32_t* item_row;
  const int32_t* nitems;
  const int32_t* heavy_rows;
  float* partials;  // this plan's records, one per item
  int item_size;
  int stride;       // floats per partial record: 2*D + H
};

struct ItemRange {
  int row;
  int j;          // item index within its row
  bool single;    // the row has one item: the item writes the final result, no record
  int64_t beg;    // this group's sub-range
  int64_t end;
};

__device__ __forceinline__ ItemRange item_group_range(const Items& it, const Shape& sh, int64_t item) {
  ItemRange r;
  r.row = it.item_row[item];
  r.j = int(item - it.item_off[r.row]);
  r.single = it.nitems[r.row] == 1;
  const int64_t rb = it.ptr[r.row], re = it.ptr[r.row + 1];
  // the row's n items are balanced: ceil(len / n) entries each, the last one shorter
  const int64_t size = (re - rb + it.nitems[r.row] - 1) / it.nitems[r.row];
  const int64_t ib = rb + int64_t(r.j) * size;
  const int64_t ie = min(ib + size, re);
  const int gpb = kBlock >> sh.lpr_log2;
  const int grp = threadIdx.x >> sh.lpr_log2;
  const int64_t sub = (size + gpb - 1) / gpb;
  r.beg = min(ib + grp * sub, ie);
  r.end = min(r.beg + sub, ie);
  return r;
}

// Row handled by this lane's group when the row workgroups start at `first_block`.
__device__ __forceinline__ int64_t row_slot(const Shape& sh, unsigned first_block) {
  return int64_t(blockIdx.x - first_block) * (kBlock >> sh.lpr_log2) + (threadIdx.x >> sh.lpr_log2);
}

// Sums `nv` lane vectors of V floats (and, if with_z, one float per head) over
// the groups of the workgroup, in group order. Every thread must call it; the
// result is valid in group 0.
template <int V>
__device__ __forceinline__ void block_combine(float* lds, int stride, const Shape& sh, const GroupPos& g,
                                              float (&a)[V], float (&b)[V], bool with_b, float& z, bool with_z) {
  const int gpb = kBlock >> sh.lpr_log2;
  const int grp = threadIdx.x >> sh.lpr_log2;
  float* rec = lds + grp * stride;
  if (g.act) {
#pragma unroll
    for (int i = 0; i < V; ++i) rec[g.col0 + i] = a[i];
    if (with_b) {
#pragma unroll
      for (int i = 0; i < V; ++i) rec[sh.D + g.col0 + i] = b[i];
    }
    if (with_z && g.lead) rec[2 * sh.D + g.head] = z;
  }
  __syncthreads();
  if (grp == 0 && g.act) {
#pragma unroll
    for (int i = 0; i < V; ++i) a[i] = 0.f;
    if (with_b) {
#pragma unroll
      for (int i = 0; i < V; ++i) b[i] = 0.f;
    }
    z = 0.f;
    for (int gg = 0; gg < gpb; ++gg) {
      const float* r = lds + gg * stride;
#pragma unroll
      for (int i = 0; i < V; ++i) a[i] += r[g.col0 + i];
      if (with_b) {
#pragma unroll
        for (int i = 0; i < V; ++i) b[i] += r[sh.D + g.col0 + i];
      }
      if (with_z) z += r[2 * sh.D + g.head];
    }
  }
}

// Writes group 0's combined record for item `item`.
template <int V>
__device__ __forceinline__ void store_record(const Items& it, int64_t item, const Shape& sh, const GroupPos& g,
                                             const float (&a)[V], const float (&b)[V], bool with_b, float z,
                                             bool with_z) {
  const int grp = threadIdx.x >> sh.lpr_log2;
  if (grp != 0 || !g.act) return;
  float* rec = it.partials + item * it.stride;
#pragma unroll
  for (int i = 0; i < V; ++i) rec[g.col0 + i] = a[i];
  if (with_b) {
#pragma unroll
    for (int i = 0; i < V; ++i) rec[sh.D + g.col0 + i] = b[i];
  }
  if (with_z && g.lead) rec[2 * sh.D + g.head] = z;
}

// Sums the records of split row number `heavy` (one workgroup; groups strided
// over the items with several records in flight each, then combined in group
// order). Returns the row id, or -1 for a row with a single item (finished by
// that item); the sums are valid in group 0. R records in flight per group:
// as many as the reduce kernel's registers allow (the 160 items of the token
// row in one round at D = 128 in the forward).
template <int V, int R = 8>
__device__ __forceinline__ int reduce_row_records(const Items& it, int64_t heavy, float* lds, const Shape& sh,
                                                  const GroupPos& g, float (&a)[V], float (&b)[V], bool with_b,
                                                  float& z, bool with_z) {
  const int row = it.heavy_rows[heavy];
  const int64_t first = it.item_off[row];
  const int n = it.nitems[row];
  if (n == 1) return -1;   // written by its only item (uniform over the workgroup: no barrier skipped unevenly)
  const int gpb = kBlock >> sh.lpr_log2;
  const int grp = threadIdx.x >> sh.lpr_log2;
#pragma unroll
  for (int i = 0; i < V; ++i) a[i] = b[i] = 0.f;
  z = 0.f;
  if (g.act) {
    for (int m0 = grp; m0 < n; m0 += R * gpb) {
      float ra[R][V], rb[R][V], rz[R];
#pragma unroll
      for (int u = 0; u < R; ++u) {
        const int m = m0 + u * gpb;
        const bool ok = m < n;
        const float* rec = it.partials + (first + (ok ? m : 0)) * it.stride;
#pragma unroll
        for (int i = 0; i < V; ++i) ra[u][i] = ok ? rec[g.col0 + i] : 0.f;
        if (with_b) {
#pragma unroll
          for (int i = 0; i < V; ++i) rb[u][i] = ok ? rec[sh.D + g.col0 + i] : 0.f;
        }
        rz[u] = (with_z && ok) ? rec[2 * sh.D + g.head] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < R; ++u) {
#pragma unroll
        for (int i = 0; i < V; ++i) a[i] += ra[u][i];
        if (with_b) {
#pragma unroll
          for (int i = 0; i < V; ++i) b[i] += rb[u][i];
        }
        z += rz[u];
      }
    }
  }
  block_combine<V>(lds, it.stride, sh, g, a, b, with_b, z, with_z);
  return row;
}

// ------------------------------------------------------------------ forward kernels
// out = acc / (Z + eps) and Z of one finished query row.
template <typename T, int V>
__device__ __forceinline__ void store_out(T* __restrict__ out, float* __restrict__ Z, int64_t row, const Shape& sh,
                                          const GroupPos& g, const float (&acc)[V], float z) {
  if (!g.act) return;
  const float den = z + kEps;
  float o[V];
#pragma unroll
  for (int i = 0; i < V; ++i) o[i] = acc[i] / den;
  Elem<T>::store_nt(out + row * sh.D + g.col0, o);
  if (g.lead) Z[row * sh.H + g.head] = z;
}

// Waves per SIMD the compiler must leave room for (amdgpu_waves_per_eu), per instance: 1 leaves the
// allocation free. The float32 plain forward fits eight waves in 62 VGPRs instead of seven in 66 without
// spills (c2 forward 130.9 -> 130.4 us over three A/B pairs).
template <typename T, int EX>
struct FwdWaves {
  static constexpr int kMin = 1;
};
template <>
struct FwdWaves<float, 0> {
  static constexpr int kMin = 8;
};

// Blocks [0, n_items) take the query-side items, the rest one short query row per group.
template <typename T, int EX>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(FwdWaves<T, EX>::kMin))) void attn_fwd_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int64_t* __restrict__ qptr, const int32_t* __restrict__ kv, EdgeIn ex,
    T* __restrict__ out, float* __restrict__ Z, Items it, int n_items_arg, int64_t n_q, Shape sh, int chunk,
    const int32_t* __restrict__ plan_counts) {
  constexpr int V = Elem<T>::kPerVec;
  const GroupPos g = group_pos<T>(sh);
  // blocks [0, n_items_arg) are item slots (the capacity when the counts are on the device; the
  // unused ones exit early, while the items run), the rest one short row per group
  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;
  float z = 0.f;
  if (int(blockIdx.x) < n_items_arg) {
    if (plan_counts && int(blockIdx.x) >= plan_counts[0]) return;
    extern __shared__ float lds[];
    const ItemRange r = item_group_range(it, sh, blockIdx.x);
    float unused[V];
#pragma unroll
    for (int i = 0; i < V; ++i) unused[i] = 0.f;
    const typename Elem<T>::Raw qr = load_row_raw(q, r.row, sh.D, g);
    fwd_segment<T, EX>(k, v, kv, ex, r.beg, r.end, r.row, it.ptr[r.row], sh, g, qr, acc, z);
    block_combine<V>(lds, it.stride, sh, g, acc, unused, false, z, true);
    if (r.single) {
      if ((threadIdx.x >> sh.lpr_log2) == 0) store_out(out, Z, r.row, sh, g, acc, z);
    } else {
      store_record<V>(it, blockIdx.x, sh, g, acc, unused, false, z, true);
    }
    return;
  }
  const int64_t row = row_slot(sh, unsigned(n_items_arg));
  if (row >= n_q) return;
  const int64_t beg = qptr[row], end = qptr[row + 1];
  if (end - beg > chunk) return;  // split row: its items and the reduce write it
  const typename Elem<T>::Raw qr = load_row_raw_nt(q, row, sh.D, g);
  fwd_segment<T, EX>(k, v, kv, ex, beg, end, int32_t(row), beg, sh, g, qr, acc, z);
  store_out(out, Z, row, sh, g, acc, z);
}

template <typename T>
__global__ __launch_bounds__(kBlock) void attn_fwd_reduce_kernel(T* __restrict__ out, float* __restrict__ Z,
                                                                 Items it, Shape sh,
                                                                 const int32_t* __restrict__ plan_counts) {
  constexpr int V = Elem<T>::kPerVec;
  if (plan_counts && int(blockIdx.x) >= plan_counts[1]) return;
  extern __shared__ float lds[];
  const GroupPos g = group_pos<T>(sh);
  float acc[V], unused[V], z;
  const int row = reduce_row_records<V, 80 / V>(it, blockIdx.x, lds, sh, g, acc, unused, false, z, true);
  if (row < 0 || (threadIdx.x >> sh.lpr_log2) != 0) return;
  store_out(out, Z, row, sh, g, acc, z);
}

// ------------------------------------------------------------------ backward, query-major (dq)
// Per query row t and head, with D' = Z + eps, w_e = (dO_t . v_s) / D' and
// m_e = [-5 <= a_pre <= 5] / sqrt(hn) per entry e = (s -> t):
//   Delta  = sum_j dO_j out_j = sum_e p_e f_e w_e       (c below)
//   g_b,e  = (f_e w_e - Delta / D') p_e                  (dbias: the bias is added after the clamp)
//   dq_t   = sum_e g_b,e m_e k_s = A - (Delta / D') B,
//            A = sum_e f_e w_e p_e m_e k_s,  B = sum_e p_e m_e k_s.
// Delta is summed from the entries in the same loop as A and B, in float32,
// instead of being read back from the output tensor: a bfloat16 `out` carries
// its 2^-9 rounding into every g_b, which dominates the rows whose gradient
// nearly cancels (the reference under autocast keeps `out` in float32), and the
// pass no longer reads `out` at all.

// One entry's per-head scalars (every lane of the head holds them).
struct EntryTerms {
  float p;   // exp(clamp(a) [+ bias])
  float f;   // factor or 1
  float w;   // (dO . v) / D'
  float m;   // [inside the clamp] / sqrt(hn)
};

// f: the entry's V-message factor (1 without a factor or dropout).
template <int EX>
__device__ __forceinline__ EntryTerms entry_terms(float d, float wraw, float inv_dprime, const EdgeIn& ex, int64_t e,
                                                  float f, const Shape& sh, const GroupPos& g) {
  EntryTerms t;
  const float apre = d * sh.inv_scale;
  float a = fminf(fmaxf(apre, -sh.clamp), sh.clamp);
  if (EX == 2) a += edge_bias(ex, e, sh, g.head);
  t.p = __expf(a);   // a is clamped to [-5, 5] (+ bias): exp2-based form is within 2 ulp
  t.f = EX ? f : 1.f;
  t.w = wraw * inv_dprime;
  t.m = (apre >= -sh.clamp && apre <= sh.clamp) ? sh.inv_scale : 0.f;
  return t;
}

template <int V>
__device__ __forceinline__ void add_entry(const EntryTerms& t, const float (&kk)[V], float (&A)[V], float (&B)[V],
                                          float& c) {
  const float fwp = t.f * t.w * t.p;
  const float ca = fwp * t.m, cb = t.p * t.m;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    A[i] = fmaf(ca, kk[i], A[i]);
    B[i] = fmaf(cb, kk[i], B[i]);
  }
  c += fwp;
}

// A, B and c over entries [beg, end) of one query row. EX: the per-entry
// inputs compiled in (0 none, 1 dropout only, 2 bias, factor and dropout).
template <typename T, int EX>
__device__ __forceinline__ void dq_segment(const T* __restrict__ k, const T* __restrict__ v,
                                           const int32_t* __restrict__ kv, const EdgeIn& ex,
                                           int64_t beg, int64_t end, int32_t row, int64_t row_beg,
                                           const Shape& sh, const GroupPos& g, float inv_dprime, const typename Elem<T>::Raw& qr,
                                           const typename Elem<T>::Raw& gr,
                                           float (&A)[Elem<T>::kPerVec], float (&B)[Elem<T>::kPerVec], float& c) {
  constexpr int V = Elem<T>::kPerVec;
  constexpr int kUnroll = Unroll<T>::q;
  const int lph = 1 << sh.lph_log2;
  ChunkIds<T, kUnroll> ids(sh, beg);
  const int col = gather_col(g);
  for (int64_t e0 = beg; e0 < end; e0 += kUnroll) {
    int s[kUnroll];
    bool ok[kUnroll];
    ids.fetch(kv, e0, end, g, s, ok);
    typename Elem<T>::Raw kr[kUnroll], vr[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      kr[u] = Elem<T>::load_raw(k + int64_t(s[u]) * sh.D + col);
      vr[u] = Elem<T>::load_raw(v + int64_t(s[u]) * sh.D + col);
    }
    // with a keep mask (EX == 4: one byte per entry) the iteration's bytes in two aligned dwords, loaded
    // after the rows (loads return in order, and the bits are used after the dots)
    KeepWords kw{0u, 0u, 0};
    if constexpr (EX == 4) {
      static_assert(kUnroll <= 4, "an iteration's keep bytes span at most two dwords");
      kw = load_keep_words(ex.keepm, e0, end);
    }
    // otherwise the keep bits depend on the entries' places only: drawn while the rows are in flight (c4's
    // dq pass 2.90 -> 2.72 ms; the forward, one wave per SIMD short of this pass's pressure, keeps its
    // draw after the dots: there the same move costs it its sixth wave and 1%)
    IterDrop<kUnroll> drop{false, 0u};
    if (EX && EX != 4) {
      int32_t rows[kUnroll], slots[kUnroll];   // the dropout's (query row, slot) of each entry
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        rows[u] = row;
        slots[u] = int32_t(e0 + u - row_beg);
      }
      drop = iter_drop<kUnroll>(ex, rows, slots, ok, sh, g);
    }
    float d[kUnroll], w[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      d[u] = Elem<T>::dot(kr[u], qr, 0.f);
      w[u] = Elem<T>::dot(vr[u], gr, 0.f);
    }
    for (int o = 1; o < lph; o <<= 1) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        d[u] += __shfl_xor(d[u], o, 64);
        w[u] += __shfl_xor(w[u], o, 64);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (!ok[u]) continue;
      const float f = EX == 4 ? mask_factor(ex, keep_byte(kw, u), g.head)
                              : (EX ? iter_factor<kUnroll, EX>(ex, drop, u, e0 + u, sh, g.head) : 1.f);
      const EntryTerms t = entry_terms<EX>(d[u], w[u], inv_dprime, ex, e0 + u, f, sh, g);
      float kk[V];
      Elem<T>::unpack(kr[u], kk);
      add_entry<V>(t, kk, A, B, c);
    }
  }
}

// The key-0 entry (CSR position e) of a token-column row. ADD: also added to
// A, B and c like any entry (a short row takes it first, so the sums keep the
// order of the entries); its scalars finish key 0's gradient terms once the
// row's Delta / D' is known (finish_token). A split row's items sum it in
// order with the rest, and the step that finishes the row recomputes these
// scalars without adding them again.
struct TokenEntry {
  float fw;    // f (dO . v_0), before the 1/D'
  float p;
  float f;
  float m;     // [inside the clamp] / sqrt(hn)
};

template <typename T, int EX, bool ADD>
__device__ __forceinline__ TokenEntry token_entry(const T* __restrict__ k, const T* __restrict__ v, const EdgeIn& ex,
                                                  int64_t e, int32_t row, const Shape& sh, const GroupPos& g,
                                                  float inv_dprime,
                                                  const typename Elem<T>::Raw& qr, const typename Elem<T>::Raw& gr,
                                                  float (&A)[Elem<T>::kPerVec], float (&B)[Elem<T>::kPerVec],
                                                  float& c) {
  constexpr int V = Elem<T>::kPerVec;
  const typename Elem<T>::Raw kr = load_row_raw(k, 0, sh.D, g), vr = load_row_raw(v, 0, sh.D, g);
  float d = Elem<T>::dot(kr, qr, 0.f), w = Elem<T>::dot(vr, gr, 0.f);
  for (int o = 1; o < (1 << sh.lph_log2); o <<= 1) {
    d += __shfl_xor(d, o, 64);
    w += __shfl_xor(w, o, 64);
  }
  // key 0 is the first entry of its row: slot 0
  const EntryTerms t =
      entry_terms<EX>(d, w, inv_dprime, ex, e, EX ? edge_factor<EX>(ex, e, row, 0, sh, g.head) : 1.f, sh, g);
  if (ADD) {
    float kk[V];
    Elem<T>::unpack(kr, kk);
    add_entry<V>(t, kk, A, B, c);
  }
  return TokenEntry{t.f * w, t.p, t.f, t.m};
}

// Key 0's terms from this row, dd = Delta / D': fk = g_b m q (its dK term),
// fv = p f dO / D' (its dV term); and its dbias g_b at CSR position e. The
// same expressions the key-major pass evaluates for an entry it gathers.
template <typename T, int EX>
__device__ __forceinline__ void finish_token(const TokenEntry& te, float inv_dprime, float dd,
                                             const typename Elem<T>::Raw& qr, const typename Elem<T>::Raw& gr,
                                             float* __restrict__ dbias, int64_t e, const Shape& sh, const GroupPos& g,
                                             float (&fk)[Elem<T>::kPerVec], float (&fv)[Elem<T>::kPerVec]) {
  constexpr int V = Elem<T>::kPerVec;
  const float gb = fmaf(te.fw, inv_dprime, -dd) * te.p;
  if (EX == 2 && dbias && g.lead) dbias[e * sh.H + g.head] = gb;
  const float gs = gb * te.m;
  const float pf = te.p * te.f * inv_dprime;
  float qq[V], gg[V];
  Elem<T>::unpack(qr, qq);
  Elem<T>::unpack(gr, gg);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    fk[i] = gs * qq[i];
    fv[i] = pf * gg[i];
  }
}

// dq = A - dd B of a finished row and its row stats {1/D', Delta/D'}, which the key-major pass gathers
// (one 8-byte record per query and head, so each reverse entry touches one stats line).
template <typename T, int V>
__device__ __forceinline__ void store_dq(T* __restrict__ dq, float2* __restrict__ rstat, int64_t row, const Shape& sh,
                                         const GroupPos& g, const float (&A)[V], const float (&B)[V], float inv_dprime,
                                         float dd, bool nt) {
  if (!g.act) return;
  float o[V];
#pragma unroll
  for (int i = 0; i < V; ++i) o[i] = fmaf(-dd, B[i], A[i]);
  if (nt)
    Elem<T>::store_nt(dq + row * sh.D + g.col0, o);
  else
    Elem<T>::store(dq + row * sh.D + g.col0, o);
  if (g.lead) rstat[row * sh.H + g.head] = make_float2(inv_dprime, dd);
}

template <typename T>
__device__ __forceinline__ float row_inv_dprime(const float* __restrict__ Z, int64_t row, const Shape& sh,
                                                const GroupPos& g) {
  return 1.0f / ((g.act ? Z[row * sh.H + g.head] : 0.f) + kEps);
}

// Writes one token-column record (2*D floats: key 0's dK terms, then its dV terms).
template <int V>
__device__ __forceinline__ void store_token_record(float* __restrict__ rec, const Shape& sh, const GroupPos& g,
                                                   const float (&fk)[V], const float (&fv)[V]) {
  if (!g.act) return;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    rec[g.col0 + i] = fk[i];
    rec[sh.D + g.col0 + i] = fv[i];
  }
}

// Sums the token-column records [a0, a1) (2*D floats each: key 0's dK terms,
// then its dV terms) into dk, dv. Record m is the dq pass's workgroup m for
// its n_items item workgroups and workgroup m - n_items + item_slots after
// them (the row workgroups follow all item slots).
template <int V>
__device__ __forceinline__ void sum_token_records(const float* __restrict__ rec0, int64_t a0, int64_t a1,
                                                  int64_t n_items, int64_t item_slots, const Shape& sh,
                                                  const GroupPos& g, float (&dk)[V], float (&dv)[V]) {
  if (!g.act) return;
  for (int64_t m = a0; m < a1; ++m) {
    const float* rec = rec0 + (m < n_items ? m : m - n_items + item_slots) * (2 * sh.D);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      dk[i] += rec[g.col0 + i];
      dv[i] += rec[sh.D + g.col0 + i];
    }
  }
}

// Blocks [0, n_items) take the query-side items, the rest one short query row per group.
// With a token column (rows from tok_first on open with key 0) every workgroup also writes one
// record of its rows' key-0 terms; a split row's key-0 terms are finished with the row: by its item
// when the row has one, else by the dq reduce, which writes them into the row's first item's record.
template <typename T, int EX>
__global__ __launch_bounds__(kBlock) void attn_bwd_q_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int64_t* __restrict__ qptr, const int32_t* __restrict__ kv, EdgeIn ex,
    const float* __restrict__ Z, const T* __restrict__ dout,
    T* __restrict__ dq, float* __restrict__ dbias, float2* __restrict__ rstat, Items it, int n_items_arg,
    int64_t n_q, Shape sh, int chunk, float* __restrict__ token_rec, int tok_first,
    const int32_t* __restrict__ plan_counts) {
  constexpr int V = Elem<T>::kPerVec;
  extern __shared__ float lds[];
  const GroupPos g = group_pos<T>(sh);
  const int grp = threadIdx.x >> sh.lpr_log2;
  float A[V], B[V], c = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) A[i] = B[i] = 0.f;
  if (int(blockIdx.x) < n_items_arg) {
    // blocks [0, n_items_arg) are item slots (the capacity when the counts are on the device: an unused
    // slot exits at once and writes no token record)
    if (plan_counts && int(blockIdx.x) >= plan_counts[0]) return;
    const ItemRange r = item_group_range(it, sh, blockIdx.x);
    const typename Elem<T>::Raw qr = load_row_raw(q, r.row, sh.D, g);
    const typename Elem<T>::Raw gr = load_row_raw(dout, r.row, sh.D, g);
    const float inv_dprime = row_inv_dprime<T>(Z, r.row, sh, g);
    const int64_t e_tok = it.ptr[r.row];
    const bool tok_row = token_rec != nullptr && r.row >= tok_first && e_tok < it.ptr[r.row + 1];
    dq_segment<T, EX>(k, v, kv, ex, r.beg, r.end, r.row, e_tok, sh, g, inv_dprime, qr, gr, A, B, c);
    block_combine<V>(lds, it.stride, sh, g, A, B, true, c, true);
    float fk[V], fv[V];
#pragma unroll
    for (int i = 0; i < V; ++i) fk[i] = fv[i] = 0.f;
    if (r.single) {
      if (grp == 0) {
        const float dd = c * inv_dprime;
        if (tok_row) {
          const TokenEntry te = token_entry<T, EX, false>(k, v, ex, e_tok, r.row, sh, g, inv_dprime, qr, gr,
                                                             A, B, c);
          finish_token<T, EX>(te, inv_dprime, dd, qr, gr, dbias, e_tok, sh, g, fk, fv);
        }
        store_dq<T, V>(dq, rstat, r.row, sh, g, A, B, inv_dprime, dd, false);
      }
    } else {
      store_record<V>(it, blockIdx.x, sh, g, A, B, true, c, true);
    }
    if (token_rec && grp == 0) store_token_record<V>(token_rec + int64_t(blockIdx.x) * (2 * sh.D), sh, g, fk, fv);
    return;
  }
  const int64_t row = row_slot(sh, unsigned(n_items_arg));
  int64_t beg = 0, end = 0;
  bool live = row < n_q;
  if (live) {
    beg = qptr[row];
    end = qptr[row + 1];
    live = end - beg <= chunk;    // a split row: its items and the reduce write it
  }
  if (!token_rec && !live) return;
  typename Elem<T>::Raw qr = Elem<T>::zero_raw(), gr = Elem<T>::zero_raw();
  float inv_dprime = 1.f;
  if (live) {
    qr = load_row_raw_nt(q, row, sh.D, g);
    gr = load_row_raw_nt(dout, row, sh.D, g);
    inv_dprime = row_inv_dprime<T>(Z, row, sh, g);
  }
  const bool tok = token_rec != nullptr && live && row >= tok_first && beg < end;
  const int64_t e_tok = beg;
  TokenEntry te{};
  if (tok) {
    te = token_entry<T, EX, true>(k, v, ex, e_tok, int32_t(row), sh, g, inv_dprime, qr, gr, A, B, c);
    ++beg;
  }
  float dd = 0.f;
  if (live) {
    dq_segment<T, EX>(k, v, kv, ex, beg, end, int32_t(row), e_tok, sh, g, inv_dprime, qr, gr, A, B, c);
    dd = c * inv_dprime;
    store_dq<T, V>(dq, rstat, row, sh, g, A, B, inv_dprime, dd, true);
  }
  if (!token_rec) return;
  float fk[V], fv[V];
#pragma unroll
  for (int i = 0; i < V; ++i) fk[i] = fv[i] = 0.f;
  if (tok) finish_token<T, EX>(te, inv_dprime, dd, qr, gr, dbias, e_tok, sh, g, fk, fv);
  // sum the wave's groups (a fixed butterfly), park the wave's sum in LDS, then the waves in order
  for (int o = 1 << sh.lpr_log2; o < 64; o <<= 1) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      fk[i] += __shfl_xor(fk[i], o, 64);
      fv[i] += __shfl_xor(fv[i], o, 64);
    }
  }
  if ((threadIdx.x & 63) < (1u << sh.lpr_log2)) store_token_record<V>(lds + (threadIdx.x >> 6) * (2 * sh.D), sh, g, fk, fv);
  __syncthreads();
  if (threadIdx.x < (1u << sh.lpr_log2) && g.act) {   // the workgroup's record: its waves in order
    float sk[V], sv[V];
#pragma unroll
    for (int i = 0; i < V; ++i) sk[i] = sv[i] = 0.f;
    for (int w = 0; w < kBlock / 64; ++w) {
      const float* slot = lds + w * (2 * sh.D);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        sk[i] += slot[g.col0 + i];
        sv[i] += slot[sh.D + g.col0 + i];
      }
    }
    store_token_record<V>(token_rec + int64_t(blockIdx.x) * (2 * sh.D), sh, g, sk, sv);
  }
}

// One workgroup per query-side split row with more than one item: sums the
// items' records {A, B, c} in item order and finishes the row, writing dq, the
// row stats and, for a token-column row, key 0's terms (and dbias) into the
// record of the row's first item. Runs between the dq pass and the key-major
// pass, which gathers the row stats.
template <typename T>
__global__ __launch_bounds__(kBlock) void attn_bwd_q_reduce_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, EdgeIn ex,
    const float* __restrict__ Z, const T* __restrict__ dout, T* __restrict__ dq,
    float* __restrict__ dbias, float2* __restrict__ rstat, Items it, Shape sh, float* __restrict__ token_rec,
    int tok_first, const int32_t* __restrict__ plan_counts) {
  constexpr int V = Elem<T>::kPerVec;
  if (plan_counts && int(blockIdx.x) >= plan_counts[1]) return;
  extern __shared__ float lds[];
  const GroupPos g = group_pos<T>(sh);
  float A[V], B[V], c;
  const int row = reduce_row_records<V, 40 / V>(it, blockIdx.x, lds, sh, g, A, B, true, c, true);
  if (row < 0 || (threadIdx.x >> sh.lpr_log2) != 0) return;
  const float inv_dprime = row_inv_dprime<T>(Z, row, sh, g);
  const int64_t e_tok = it.ptr[row];
  const bool tok = token_rec != nullptr && row >= tok_first && e_tok < it.ptr[row + 1];
  float fk[V], fv[V];
#pragma unroll
  for (int i = 0; i < V; ++i) fk[i] = fv[i] = 0.f;
  const float dd = c * inv_dprime;
  store_dq<T, V>(dq, rstat, row, sh, g, A, B, inv_dprime, dd, false);
  if (tok) {   // key 0 was summed by item 0; its scalars are recomputed here to finish its terms
    const typename Elem<T>::Raw qr = load_row_raw(q, row, sh.D, g);
    const typename Elem<T>::Raw gr = load_row_raw(dout, row, sh.D, g);
    const TokenEntry te = token_entry<T, 2, false>(k, v, ex, e_tok, row, sh, g, inv_dprime, qr, gr, A, B, c);
    finish_token<T, 2>(te, inv_dprime, dd, qr, gr, dbias, e_tok, sh, g, fk, fv);
    store_token_record<V>(token_rec + int64_t(it.item_off[row]) * (2 * sh.D), sh, g, fk, fv);
  }
}

// ------------------------------------------------------------------ backward, key-major (dk, dv)
// q and dO rows are gathered B times per pass at random points; when the two
// tables exceed the 256 MB Infinity Cache they are read non-temporally, which
// keeps the row stats and the hub K/V rows cached instead (kStreamBytes).
constexpr size_t kStreamBytes = size_t(256) << 20;



template <typename T, bool NT>
__device__ __forceinline__ typename Elem<T>::Raw gather_row(const T* base, int64_t row, int D, int col0) {
  return NT ? Elem<T>::load_raw_nt(base + row * D + col0) : Elem<T>::load_raw(base + row * D + col0);
}

// One reverse entry's terms added to dK and dV of its kv row: d = q_t . k_s and w = dO_t . v_s (summed over
// the head's lanes), rs = the query's {1/D', Delta/D'}, f its V-message factor, e its CSR position (read
// only with EX == 2: bias and dbias).
template <typename T, int EX>
__device__ __forceinline__ void dkv_entry(float d, float w, float2 rs, const typename Elem<T>::Raw& qr,
                                          const typename Elem<T>::Raw& gr, float f, int64_t e, const EdgeIn& ex,
                                          float* __restrict__ dbias, const Shape& sh, const GroupPos& g,
                                          float (&dk)[Elem<T>::kPerVec], float (&dv)[Elem<T>::kPerVec]) {
  constexpr int V = Elem<T>::kPerVec;
  const float apre = d * sh.inv_scale;
  float a = fminf(fmaxf(apre, -sh.clamp), sh.clamp);
  if (EX == 2) a += edge_bias(ex, e, sh, g.head);
  const float p = __expf(a);   // a is clamped to [-5, 5] (+ bias): exp2-based form is within 2 ulp
  const float gb = fmaf(f * w, rs.x, -rs.y) * p;   // rs = {1/D', Delta/D'}
  if (EX == 2 && dbias && g.lead) dbias[e * sh.H + g.head] = gb;
  const float gs = (apre >= -sh.clamp && apre <= sh.clamp) ? gb * sh.inv_scale : 0.f;
  const float pf = p * f * rs.x;
  float qq[V], gg[V];
  Elem<T>::unpack(qr, qq);
  Elem<T>::unpack(gr, gg);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    dv[i] = fmaf(pf, gg[i], dv[i]);
    dk[i] = fmaf(gs, qq[i], dk[i]);
  }
}

// The Graphormer token row's entry of kv row s (1 <= s <= the token row's length): the first of s's
// reverse entries, query 0 at slot s - 1 (CSR position s - 1, since the token row lists kv 1, 2, ...
// in order from position 0). Its q and dO rows and row stats come from the workgroup's LDS copy (tok),
// written once, instead of being gathered again for every kv row; the terms are the ones dkv_segment
// adds for the same entry.
template <typename T, int EX>
__device__ __forceinline__ void dkv_token_entry(const unsigned char* tok, int64_t s, const EdgeIn& ex,
                                                float* __restrict__ dbias, const Shape& sh, const GroupPos& g,
                                                const typename Elem<T>::Raw& krow,
                                                const typename Elem<T>::Raw& vrow,
                                                float (&dk)[Elem<T>::kPerVec], float (&dv)[Elem<T>::kPerVec]) {
  using Raw = typename Elem<T>::Raw;
  const int col = gather_col(g);
  const Raw qr = *reinterpret_cast<const Raw*>(tok + col * sizeof(T));
  const Raw gr = *reinterpret_cast<const Raw*>(tok + (sh.D + col) * sizeof(T));
  const float2 rs = reinterpret_cast<const float2*>(tok + 2 * sh.D * sizeof(T))[g.head];
  float d = Elem<T>::dot(qr, krow, 0.f), w = Elem<T>::dot(gr, vrow, 0.f);
  for (int o = 1; o < (1 << sh.lph_log2); o <<= 1) {
    d += __shfl_xor(d, o, 64);
    w += __shfl_xor(w, o, 64);
  }
  const int64_t e = s - 1;
  const float f = EX ? edge_factor<EX>(ex, e, 0, int32_t(s - 1), sh, g.head) : 1.f;
  dkv_entry<T, EX>(d, w, rs, qr, gr, f, e, ex, dbias, sh, g, dk, dv);
}

// ------------------------------------------------------------------ typed edges (Exphormer)
// models/exphormer_dist_node_level.py:92-117: an edge of type t in {0, 1} scores
//   a = clamp(sum_j k[s,h,j] * q[t,h,j] * E[t,h,j] / sqrt(hn), -5, 5),  E = edge_proj(edge_type_emb(t)),
// with no bias, factor or dropout. The type travels in bit 31 of the entry's id (kv in the query-major
// CSR, kq in the reverse index; ids are below 2^31), so the passes read no per-entry type array and no
// typed copy of K or V exists. dq and dK follow from the same scores with the modulation on the other
// operand, and the gradient of E,
//   dE[t,h,j] = sum over type-t entries of g_a * k[s,h,j] * q[t,h,j] / sqrt(hn),
// is formed by the dq pass per query row (q times its type-t part of dq before the modulation), summed
// per workgroup into one record of 2*D floats and over the records by a reduce in a fixed order.
__device__ __forceinline__ int typed_id(int enc) { return enc & 0x7fffffff; }
__device__ __forceinline__ bool typed_one(int enc) { return enc < 0; }

// This lane's V values of E[t] (float32 [2, D]).
template <int V>
__device__ __forceinline__ void load_mod(const float* __restrict__ mod, int t, const Shape& sh, int col,
                                         float (&e)[V]) {
  const float* p = mod + int64_t(t) * sh.D + col;
#pragma unroll
  for (int i = 0; i < V; ++i) e[i] = p[i];
}

// sum_i a[i] * (one ? b1[i] : b0[i]) in element order (the modulated dot product of one entry).
template <int V>
__device__ __forceinline__ float typed_dot(const float (&a)[V], const float (&b0)[V], const float (&b1)[V], bool one) {
  float d = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) d = fmaf(a[i], one ? b1[i] : b0[i], d);
  return d;
}

// dkv_segment for typed entries: dK accumulates q_t * g_a per type and takes E[0] * dK0 + E[1] * dK1 at
// the end (the modulation is linear, so a split row's items may each apply it to their part).
template <typename T, bool NT>
__device__ __forceinline__ void dkv_segment_typed(const T* __restrict__ q, const T* __restrict__ dout,
                                                  const int32_t* __restrict__ kq, const EdgeIn& ex,
                                                  const float2* __restrict__ rstat, int64_t beg, int64_t end,
                                                  const Shape& sh, const GroupPos& g,
                                                  const typename Elem<T>::Raw& krow,
                                                  const typename Elem<T>::Raw& vrow,
                                                  float (&dk)[Elem<T>::kPerVec], float (&dv)[Elem<T>::kPerVec]) {
  constexpr int V = Elem<T>::kPerVec;
  constexpr int kUnroll = BF_UNROLL_KV_TYPED ? BF_UNROLL_KV_TYPED : Unroll<T>::kv;
  const int lph = 1 << sh.lph_log2;
  const int col = gather_col(g);
  float ke0[V], ke1[V], dk0[V], dk1[V];
  {
    float kk[V], e[V];
    Elem<T>::unpack(krow, kk);
    load_mod<V>(ex.mod, 0, sh, col, e);
#pragma unroll
    for (int i = 0; i < V; ++i) ke0[i] = kk[i] * e[i];
    load_mod<V>(ex.mod, 1, sh, col, e);
#pragma unroll
    for (int i = 0; i < V; ++i) ke1[i] = kk[i] * e[i];
  }
#pragma unroll
  for (int i = 0; i < V; ++i) dk0[i] = dk1[i] = 0.f;
  ChunkIds<T, kUnroll> ids(sh, beg);
  for (int64_t i0 = beg; i0 < end; i0 += kUnroll) {
    int t[kUnroll];
    bool ok[kUnroll], one[kUnroll];
    ids.fetch(kq, i0, end, g, t, ok);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      one[u] = typed_one(t[u]);
      t[u] = typed_id(t[u]);
    }
    typename Elem<T>::Raw qr[kUnroll], gr[kUnroll];
    float2 rs[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      qr[u] = gather_row<T, NT>(q, t[u], sh.D, col);
      gr[u] = gather_row<T, NT>(dout, t[u], sh.D, col);
      rs[u] = rstat[int64_t(t[u]) * sh.H + g.head];
    }
    float d[kUnroll], w[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      float qq[V];
      Elem<T>::unpack(qr[u], qq);
      d[u] = typed_dot<V>(qq, ke0, ke1, one[u]);
      w[u] = Elem<T>::dot(gr[u], vrow, 0.f);
    }
    for (int o = 1; o < lph; o <<= 1) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        d[u] += __shfl_xor(d[u], o, 64);
        w[u] += __shfl_xor(w[u], o, 64);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (!ok[u]) continue;
      const float apre = d[u] * sh.inv_scale;
      const float a = fminf(fmaxf(apre, -sh.clamp), sh.clamp);
      const float p = __expf(a);   // a is clamped to [-5, 5]: exp2-based form is within 2 ulp
      const float gb = fmaf(w[u], rs[u].x, -rs[u].y) * p;   // rs = {1/D', Delta/D'}
      const float gs = (apre >= -sh.clamp && apre <= sh.clamp) ? gb * sh.inv_scale : 0.f;
      const float gs1 = one[u] ? gs : 0.f, gs0 = gs - gs1;
      const float pf = p * rs[u].x;
      float qq[V], gg[V];
      Elem<T>::unpack(qr[u], qq);
      Elem<T>::unpack(gr[u], gg);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        dv[i] = fmaf(pf, gg[i], dv[i]);
        dk0[i] = fmaf(gs0, qq[i], dk0[i]);
        dk1[i] = fmaf(gs1, qq[i], dk1[i]);
      }
    }
  }
  float e0[V], e1[V];
  load_mod<V>(ex.mod, 0, sh, col, e0);
  load_mod<V>(ex.mod, 1, sh, col, e1);
#pragma unroll
  for (int i = 0; i < V; ++i) dk[i] = fmaf(e0[i], dk0[i], fmaf(e1[i], dk1[i], dk[i]));
}

// dK and dV of one kv row over its reverse entries [beg, end); with dbias, each
// entry's g_b = (f w - Delta/D') p at its CSR position (the row stats carry the
// exact Delta/D' the dq pass summed). EX: the per-entry inputs compiled in
// (0 none, 1 dropout only, 2 bias, factor, dropout and dbias, 3 typed edges),
// so the plain pass keeps its register count (fp32: 96 VGPRs, five waves per SIMD).
template <typename T, bool NT, int EX>
__device__ __forceinline__ void dkv_segment(const T* __restrict__ q, const T* __restrict__ dout,
                                            const int32_t* __restrict__ kq, const int32_t* __restrict__ ks,
                                            const int64_t* __restrict__ qptr, const EdgeIn& ex,
                                            float* __restrict__ dbias,
                                            const float2* __restrict__ rstat, int64_t beg,
                                            int64_t end, const Shape& sh, const GroupPos& g,
                                            const typename Elem<T>::Raw& krow,
                                            const typename Elem<T>::Raw& vrow,
                                            float (&dk)[Elem<T>::kPerVec],
                                            float (&dv)[Elem<T>::kPerVec]) {
  if constexpr (EX == 3) {
    dkv_segment_typed<T, NT>(q, dout, kq, ex, rstat, beg, end, sh, g, krow, vrow, dk, dv);
  } else {
    constexpr int kUnroll = EX == 1 ? BF_UNROLL_KV_DROPOUT : (NT ? Unroll<T>::kv : Unroll<T>::kv_cached);
    const int lph = 1 << sh.lph_log2;
    ChunkIds<T, kUnroll> ids(sh, beg);
    const int col = gather_col(g);
    for (int64_t i0 = beg; i0 < end; i0 += kUnroll) {
      int t[kUnroll];
      bool ok[kUnroll];
      ids.fetch(kq, i0, end, g, t, ok);
      // each entry's slot in its query's row: with the query, the dropout's key; with the row's start
      // (gathered only by EX == 2, before the rows, so that it overlaps them), the CSR position that
      // indexes the bias, factor and dbias
      int32_t slot[kUnroll], epos[kUnroll];   // nnz < 2^31
      if (EX) {
  #pragma unroll
        for (int u = 0; u < kUnroll; ++u) slot[u] = ks[ok[u] ? i0 + u : end - 1];
      }
      if (EX == 2) {
  #pragma unroll
        for (int u = 0; u < kUnroll; ++u) epos[u] = slot[u] + int32_t(qptr[t[u]]);
      }
      typename Elem<T>::Raw qr[kUnroll], gr[kUnroll];
      float2 rs[kUnroll];
  #pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        qr[u] = gather_row<T, NT>(q, t[u], sh.D, col);
        gr[u] = gather_row<T, NT>(dout, t[u], sh.D, col);
        rs[u] = rstat[int64_t(t[u]) * sh.H + g.head];
      }
      IterDrop<kUnroll> drop{false, 0u};
      if (EX) drop = iter_drop<kUnroll>(ex, t, slot, ok, sh, g);
      float d[kUnroll], w[kUnroll];
  #pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        d[u] = Elem<T>::dot(qr[u], krow, 0.f);
        w[u] = Elem<T>::dot(gr[u], vrow, 0.f);
      }
      for (int o = 1; o < lph; o <<= 1) {
  #pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          d[u] += __shfl_xor(d[u], o, 64);
          w[u] += __shfl_xor(w[u], o, 64);
        }
      }
  #pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (!ok[u]) continue;
        const int64_t e = EX == 2 ? int64_t(epos[u]) : 0;
        const float f = EX ? iter_factor<kUnroll, EX>(ex, drop, u, e, sh, g.head) : 1.f;
        dkv_entry<T, EX>(d[u], w[u], rs[u], qr[u], gr[u], f, e, ex, dbias, sh, g, dk, dv);
      }
    }
  }
}

// Blocks [0, k_items) take the key-side items, the rest one short key row per
// group, longest rows first. EX: 0 plain, 1 dropout only, 2 bias / factor / dropout / dbias
// (EX > 0 needs ks; EX == 2 also reads qptr).
// As FwdWaves for the dk/dv pass: its float32 plain cached-gather instance fits six waves in 80 VGPRs
// instead of five in 82 without spills (c2 dk/dv pass 0.1929 -> 0.1908 ms over three A/B pairs).
template <typename T, bool NT, int EX>
struct KvWaves {
  static constexpr int kMin = 1;
};
template <>
struct KvWaves<float, false, 0> {
  static constexpr int kMin = 6;
};

template <typename T, bool NT, bool PRE, int EX>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(KvWaves<T, NT, EX>::kMin))) void attn_bwd_kv_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int64_t* __restrict__ kptr, const int32_t* __restrict__ kq,
    const int32_t* __restrict__ ks, const int64_t* __restrict__ qptr, EdgeIn ex, float* __restrict__ dbias,
    const T* __restrict__ dout,
    const float2* __restrict__ rstat, T* __restrict__ dk, T* __restrict__ dv, const int32_t* __restrict__ order,
    const uint64_t* __restrict__ spans, Items kit, int k_items_arg, int64_t n_kv, Shape sh, int chunk,
    int rows_per_group, const float* __restrict__ token_rec, int q_items_arg, int64_t q_row_blocks,
    int tok_row, const int32_t* __restrict__ plan_counts) {
  constexpr int V = Elem<T>::kPerVec;
  extern __shared__ float lds[];
  const GroupPos g = group_pos<T>(sh);
  // Block regions: k_items_arg key-side item slots, then the short key rows. With the counts on the
  // device k_items_arg is a capacity and a slot past the true count exits at once (early in the
  // dispatch, beside the running items).
  const int q_items = plan_counts ? plan_counts[0] : q_items_arg;
  // token-column records: the dq pass's q_items item workgroups, then its q_row_blocks row workgroups
  // (whose records start at slot q_items_arg; sum_token_records maps record m to its slot)
  const int64_t n_token_rec = q_items + q_row_blocks;
  float ak[V], av[V];
  const int b = int(blockIdx.x);
#pragma unroll
  for (int i = 0; i < V; ++i) ak[i] = av[i] = 0.f;
  if (b < k_items_arg) {
    const int64_t item = b;
    if (plan_counts && item >= plan_counts[2]) return;
    const ItemRange r = item_group_range(kit, sh, item);
    if (token_rec && r.row == 0) {
      // key 0's terms were summed per dq-pass workgroup: item j of n takes records [R*j/n, R*(j+1)/n),
      // its groups contiguous shares of them
      const int n0 = kit.nitems[0];
      const int64_t lo = n_token_rec * r.j / n0, hi = n_token_rec * (r.j + 1) / n0;
      const int gpb = kBlock >> sh.lpr_log2;
      const int64_t sub = (hi - lo + gpb - 1) / gpb;
      const int64_t a0 = min(lo + (threadIdx.x >> sh.lpr_log2) * sub, hi), a1 = min(a0 + sub, hi);
      sum_token_records<V>(token_rec, a0, a1, q_items, q_items_arg, sh, g, ak, av);
    } else {
      const typename Elem<T>::Raw kr = load_row_raw(k, r.row, sh.D, g), vr = load_row_raw(v, r.row, sh.D, g);
      dkv_segment<T, NT, EX>(q, dout, kq, ks, qptr, ex, dbias, rstat, r.beg, r.end, sh, g, kr, vr, ak, av);
    }
    float z = 0.f;
    block_combine<V>(lds, kit.stride, sh, g, ak, av, true, z, false);
    if (r.single) {
      if ((threadIdx.x >> sh.lpr_log2) == 0 && g.act) {
        Elem<T>::store(dk + int64_t(r.row) * sh.D + g.col0, ak);
        Elem<T>::store(dv + int64_t(r.row) * sh.D + g.col0, av);
      }
    } else {
      store_record<V>(kit, item, sh, g, ak, av, true, z, false);
    }
    return;
  }
  // With the Graphormer token row (query 0 attends kv 1, 2, ..., tok_len in order) every kv row s in
  // [1, tok_len] opens with query 0's entry: its q and dO rows and row stats are staged in LDS once per
  // workgroup instead of being gathered again for each such row.
  int64_t tok_len = 0;
  const unsigned char* tok = nullptr;
  if (tok_row) {                 // uniform over the launch
    unsigned char* buf = reinterpret_cast<unsigned char*>(lds);
    if (threadIdx.x < (1u << sh.lpr_log2) && g.act) {
      *reinterpret_cast<typename Elem<T>::Raw*>(buf + g.col0 * sizeof(T)) = Elem<T>::load_raw(q + g.col0);
      *reinterpret_cast<typename Elem<T>::Raw*>(buf + (sh.D + g.col0) * sizeof(T)) = Elem<T>::load_raw(dout + g.col0);
      if (g.lead) reinterpret_cast<float2*>(buf + 2 * sh.D * sizeof(T))[g.head] = rstat[g.head];
    }
    tok_len = qptr[1] - qptr[0];
    __syncthreads();
    tok = buf;
  }
  // each group takes rows_per_group consecutive rows of the order (similar lengths)
  const int64_t first = row_slot(sh, unsigned(k_items_arg)) * rows_per_group;
  const int64_t last = first + rows_per_group < n_kv ? first + rows_per_group : n_kv;
  // With several rows per group their slots come in one round of loads: lane i of the group reads
  // slot first + i and each iteration takes its row and span from that lane, so a row's wait for its
  // slot does not follow the previous row's work (the group's lanes loop together, so the source
  // lane is active whenever its readers are). A separate instance (PRE), launched for bf16 only: the
  // registers held across the loop would cost the fp32 kernel a wave (95 -> 100 VGPRs), and the one-row
  // bf16 kernel 6 VGPRs for nothing.
  constexpr bool pre = PRE;
  int32_t pre_row = 0;
  uint64_t pre_span = 0;
  if (pre && g.g_lane < rows_per_group && first + g.g_lane < last) {
    pre_row = order ? order[first + g.g_lane] : int32_t(first + g.g_lane);
    if (spans) pre_span = spans[first + g.g_lane];
  }
  const int lane0 = int(threadIdx.x & 63) - g.g_lane;
  for (int64_t slot = first; slot < last; ++slot) {
    const int src = lane0 + int(slot - first);
    const int64_t row = pre ? int64_t(__shfl(pre_row, src, 64)) : (order ? int64_t(order[slot]) : slot);
    int64_t beg, end;
    if (spans) {                  // the slot's (begin << 32 | length): read in slot order, not at random
      uint64_t sp;
      if (pre) {
        const uint32_t lo = uint32_t(__shfl(int(uint32_t(pre_span)), src, 64));
        const uint32_t hi = uint32_t(__shfl(int(uint32_t(pre_span >> 32)), src, 64));
        sp = (uint64_t(hi) << 32) | lo;
      } else {
        sp = spans[slot];
      }
      beg = int64_t(sp >> 32);
      end = beg + int64_t(sp & 0xffffffffu);
    } else {
      beg = kptr[row];
      end = kptr[row + 1];
    }
    if (end - beg > chunk) continue;
    if (token_rec && row == 0) {  // a short token column: this group sums every record
#pragma unroll
      for (int i = 0; i < V; ++i) ak[i] = av[i] = 0.f;
      sum_token_records<V>(token_rec, 0, n_token_rec, q_items, q_items_arg, sh, g, ak, av);
      if (g.act) {
        Elem<T>::store_nt(dk + g.col0, ak);
        Elem<T>::store_nt(dv + g.col0, av);
      }
      continue;
    }
    if (beg == end) {             // a row no query attends to: zero gradients, no reads, written past the caches
      if (g.act) {
        store_zero16_nt(dk + row * sh.D + g.col0);
        store_zero16_nt(dv + row * sh.D + g.col0);
      }
      continue;
    }
#pragma unroll
    for (int i = 0; i < V; ++i) ak[i] = av[i] = 0.f;
    const typename Elem<T>::Raw kr = load_row_raw(k, row, sh.D, g), vr = load_row_raw(v, row, sh.D, g);
    if (tok && row >= 1 && row <= tok_len) {   // the token row's entry first, from LDS
      dkv_token_entry<T, EX>(tok, row, ex, dbias, sh, g, kr, vr, ak, av);
      ++beg;
    }
    dkv_segment<T, NT, EX>(q, dout, kq, ks, qptr, ex, dbias, rstat, beg, end, sh, g, kr, vr, ak, av);
    if (g.act) {                  // written once, not read again in the pass: past the caches
      Elem<T>::store_nt(dk + row * sh.D + g.col0, ak);
      Elem<T>::store_nt(dv + row * sh.D + g.col0, av);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void attn_bwd_kv_reduce_kernel(T* __restrict__ dk, T* __restrict__ dv,
                                                                    Items it, Shape sh,
                                                                    const int32_t* __restrict__ plan_counts) {
  constexpr int V = Elem<T>::kPerVec;
  if (plan_counts && int(blockIdx.x) >= plan_counts[3]) return;
  extern __shared__ float lds[];
  const GroupPos g = group_pos<T>(sh);
  float ak[V], av[V], z;
  const int row = reduce_row_records<V, 40 / V>(it, blockIdx.x, lds, sh, g, ak, av, true, z, false);
  if (row < 0 || (threadIdx.x >> sh.lpr_log2) != 0 || !g.act) return;
  Elem<T>::store(dk + int64_t(row) * sh.D + g.col0, ak);
  Elem<T>::store(dv + int64_t(row) * sh.D + g.col0, av);
}

// ------------------------------------------------------------------ typed-edge query passes
// One query row per lane group, every row on the row path (a typed index splits no query row: its rows
// are a query's budget plus its expander edges). The forward keeps q * E[0] and q * E[1] for the row.
template <typename T>
__global__ __launch_bounds__(kBlock) void attn_fwd_typed_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, const int64_t* __restrict__ qptr,
    const int32_t* __restrict__ kv, const float* __restrict__ mod, T* __restrict__ out, float* __restrict__ Z,
    int64_t n_q, Shape sh) {
  constexpr int V = Elem<T>::kPerVec;
  constexpr int kUnroll = Unroll<T>::fwd;
  const GroupPos g = group_pos<T>(sh);
  const int64_t row = row_slot(sh, 0);
  if (row >= n_q) return;
  const int64_t beg = qptr[row], end = qptr[row + 1];
  const int col = gather_col(g);
  const int lph = 1 << sh.lph_log2;
  float qe0[V], qe1[V];
  {
    float qq[V], e[V];
    Elem<T>::unpack(load_row_raw_nt(q, row, sh.D, g), qq);
    load_mod<V>(mod, 0, sh, col, e);
#pragma unroll
    for (int i = 0; i < V; ++i) qe0[i] = qq[i] * e[i];
    load_mod<V>(mod, 1, sh, col, e);
#pragma unroll
    for (int i = 0; i < V; ++i) qe1[i] = qq[i] * e[i];
  }
  float acc[V], z = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;
  ChunkIds<T, kUnroll> ids(sh, beg);
  for (int64_t e0 = beg; e0 < end; e0 += kUnroll) {
    int s[kUnroll];
    bool ok[kUnroll], one[kUnroll];
    ids.fetch(kv, e0, end, g, s, ok);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      one[u] = typed_one(s[u]);
      s[u] = typed_id(s[u]);
    }
    typename Elem<T>::Raw kr[kUnroll], vr[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      kr[u] = Elem<T>::load_raw(k + int64_t(s[u]) * sh.D + col);
      vr[u] = Elem<T>::load_raw(v + int64_t(s[u]) * sh.D + col);
    }
    float d[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      float kk[V];
      Elem<T>::unpack(kr[u], kk);
      d[u] = typed_dot<V>(kk, qe0, qe1, one[u]);
    }
    for (int o = 1; o < lph; o <<= 1) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) d[u] += __shfl_xor(d[u], o, 64);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (!ok[u]) continue;
      const float a = fminf(fmaxf(d[u] * sh.inv_scale, -sh.clamp), sh.clamp);
      const float p = __expf(a);
      float vv[V];
      Elem<T>::unpack(vr[u], vv);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = fmaf(p, vv[i], acc[i]);
      z += p;
    }
  }
  store_out(out, Z, row, sh, g, acc, z);
}

// dq of typed rows: per row and type, A_t = sum f w p m k_s and B_t = sum p m k_s over the row's type-t
// entries; S_t = A_t - (Delta / D') B_t is dq's type-t part before the modulation, dq = E[0] S_0 + E[1] S_1,
// and q * S_t is the row's share of dE[t]. Each lane group takes rows_per_group consecutive rows, and
// each workgroup writes one record {dE[0], dE[1]} (2 * D floats) of its rows' shares.
template <typename T>
__global__ __launch_bounds__(kBlock) void attn_bwd_q_typed_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, const int64_t* __restrict__ qptr,
    const int32_t* __restrict__ kv, const float* __restrict__ mod, const float* __restrict__ Z,
    const T* __restrict__ dout, T* __restrict__ dq, float2* __restrict__ rstat, float* __restrict__ mod_rec,
    int64_t n_q, int rows_per_group, Shape sh) {
  constexpr int V = Elem<T>::kPerVec;
  constexpr int kUnroll = BF_UNROLL_Q_TYPED ? BF_UNROLL_Q_TYPED : Unroll<T>::q;
  extern __shared__ float lds[];
  const GroupPos g = group_pos<T>(sh);
  const int col = gather_col(g);
  const int lph = 1 << sh.lph_log2;
  const EdgeIn none{nullptr, nullptr, nullptr, 0, 1.f, 1.f, 0u, 0u, 0u, 0u};
  float e0[V], e1[V], r0[V], r1[V];
  load_mod<V>(mod, 0, sh, col, e0);
  load_mod<V>(mod, 1, sh, col, e1);
#pragma unroll
  for (int i = 0; i < V; ++i) r0[i] = r1[i] = 0.f;
  const int64_t first = row_slot(sh, 0) * rows_per_group;
  const int64_t last = first + rows_per_group < n_q ? first + rows_per_group : n_q;
  for (int64_t row = first; row < last; ++row) {
    const int64_t beg = qptr[row], end = qptr[row + 1];
    const typename Elem<T>::Raw qr = load_row_raw_nt(q, row, sh.D, g);
    const typename Elem<T>::Raw gr = load_row_raw_nt(dout, row, sh.D, g);
    const float inv_dprime = row_inv_dprime<T>(Z, row, sh, g);
    float qq[V], qe0[V], qe1[V], A0[V], B0[V], A1[V], B1[V], c = 0.f;
    Elem<T>::unpack(qr, qq);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      qe0[i] = qq[i] * e0[i];
      qe1[i] = qq[i] * e1[i];
      A0[i] = B0[i] = A1[i] = B1[i] = 0.f;
    }
    ChunkIds<T, kUnroll> ids(sh, beg);
    for (int64_t x0 = beg; x0 < end; x0 += kUnroll) {
      int s[kUnroll];
      bool ok[kUnroll], one[kUnroll];
      ids.fetch(kv, x0, end, g, s, ok);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        one[u] = typed_one(s[u]);
        s[u] = typed_id(s[u]);
      }
      typename Elem<T>::Raw kr[kUnroll], vr[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        kr[u] = Elem<T>::load_raw(k + int64_t(s[u]) * sh.D + col);
        vr[u] = Elem<T>::load_raw(v + int64_t(s[u]) * sh.D + col);
      }
      float d[kUnroll], w[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        float kk[V];
        Elem<T>::unpack(kr[u], kk);
        d[u] = typed_dot<V>(kk, qe0, qe1, one[u]);
        w[u] = Elem<T>::dot(vr[u], gr, 0.f);
      }
      for (int o = 1; o < lph; o <<= 1) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          d[u] += __shfl_xor(d[u], o, 64);
          w[u] += __shfl_xor(w[u], o, 64);
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (!ok[u]) continue;
        const EntryTerms t = entry_terms<0>(d[u], w[u], inv_dprime, none, 0, 1.f, sh, g);
        const float fwp = t.w * t.p;
        const float ca = fwp * t.m, cb = t.p * t.m;
        const float ca1 = one[u] ? ca : 0.f, cb1 = one[u] ? cb : 0.f, ca0 = ca - ca1, cb0 = cb - cb1;
        float kk[V];
        Elem<T>::unpack(kr[u], kk);
#pragma unroll
        for (int i = 0; i < V; ++i) {
          A0[i] = fmaf(ca0, kk[i], A0[i]);
          B0[i] = fmaf(cb0, kk[i], B0[i]);
          A1[i] = fmaf(ca1, kk[i], A1[i]);
          B1[i] = fmaf(cb1, kk[i], B1[i]);
        }
        c += fwp;
      }
    }
    const float dd = c * inv_dprime;
    float o[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float s0 = fmaf(-dd, B0[i], A0[i]), s1 = fmaf(-dd, B1[i], A1[i]);
      o[i] = fmaf(e0[i], s0, e1[i] * s1);
      r0[i] = fmaf(qq[i], s0, r0[i]);
      r1[i] = fmaf(qq[i], s1, r1[i]);
    }
    if (g.act) {
      Elem<T>::store_nt(dq + row * sh.D + g.col0, o);
      if (g.lead) rstat[row * sh.H + g.head] = make_float2(inv_dprime, dd);
    }
  }
  // the workgroup's record: the wave's groups by a fixed butterfly, then its waves in order through LDS
  for (int o = 1 << sh.lpr_log2; o < 64; o <<= 1) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      r0[i] += __shfl_xor(r0[i], o, 64);
      r1[i] += __shfl_xor(r1[i], o, 64);
    }
  }
  if ((threadIdx.x & 63) < (1u << sh.lpr_log2)) store_token_record<V>(lds + (threadIdx.x >> 6) * (2 * sh.D), sh, g, r0, r1);
  __syncthreads();
  if (threadIdx.x < (1u << sh.lpr_log2) && g.act) {
    float s0[V], s1[V];
#pragma unroll
    for (int i = 0; i < V; ++i) s0[i] = s1[i] = 0.f;
    for (int w = 0; w < kBlock / 64; ++w) {
      const float* slot = lds + w * (2 * sh.D);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        s0[i] += slot[g.col0 + i];
        s1[i] += slot[sh.D + g.col0 + i];
      }
    }
    store_token_record<V>(mod_rec + int64_t(blockIdx.x) * (2 * sh.D), sh, g, s0, s1);
  }
}

// out[b][c] = sum of rec[r][c] over records r in [b * per_block, (b + 1) * per_block), in record order
// (cols floats per record): one pass of the fixed-order reduction of the dE records.
__global__ __launch_bounds__(kBlock) void mod_rec_reduce_kernel(const float* __restrict__ rec, int64_t n_rec, int cols,
                                                                int64_t per_block, float* __restrict__ out) {
  const int64_t r0 = int64_t(blockIdx.x) * per_block;
  const int64_t r1 = r0 + per_block < n_rec ? r0 + per_block : n_rec;
  for (int c = threadIdx.x; c < cols; c += kBlock) {
    float s = 0.f;
    for (int64_t r = r0; r < r1; ++r) s += rec[r * cols + c];
    out[int64_t(blockIdx.x) * cols + c] = s;
  }
}

// ------------------------------------------------------------------ host side
int make_shape(int32_t dtype, int32_t H, int32_t hn, Shape& sh) {
  BF_CHECK_ARG(dtype == BF_DTYPE_F32 || dtype == BF_DTYPE_BF16 || dtype == BF_DTYPE_F16,
               "attention: unknown dtype %d", dtype);
  BF_CHECK_ARG(H > 0 && hn > 0, "attention: num_heads=%d head_dim=%d must be positive", H, hn);
  const int V = dtype == BF_DTYPE_F32 ? Elem<float>::kPerVec : Elem<uint16_t>::kPerVec;
  if (hn % V != 0 || !is_pow2(hn / V)) {
    set_error("attention: head_dim %d unsupported for %s (needs head_dim/%d a power of two)", hn,
              dtype == BF_DTYPE_F32 ? "float32" : dtype == BF_DTYPE_BF16 ? "bfloat16" : "float16", V);
    return BF_ERR_UNSUPPORTED;
  }
  const int D = H * hn;
  const int lanes = D / V;
  if (lanes > 64) {
    set_error("attention: row width %d elements exceeds one wavefront (%d lanes x %d)", D, 64, V);
    return BF_ERR_UNSUPPORTED;
  }
  int lpr = 1;
  while (lpr < lanes) lpr <<= 1;
  sh.D = D;
  sh.H = H;
  sh.lpr_log2 = ilog2(lpr);
  sh.lph_log2 = ilog2(hn / V);
  sh.act_lanes = lanes;
  sh.inv_scale = 1.0f / sqrtf(float(hn));
  sh.clamp = kClamp;
  return BF_OK;
}

// The score clamp a call asks for: in (0, 5] (the reference's 5, or GT's per-head-list 5 / sqrt(hn)).
int set_clamp(float score_clamp, Shape& sh) {
  BF_CHECK_ARG(score_clamp > 0.f && score_clamp <= kClamp, "attention: score_clamp %g outside (0, 5]",
               double(score_clamp));
  sh.clamp = score_clamp;
  return BF_OK;
}

int check_index(const bf_attn_index* idx, bool backward) {
  BF_CHECK_ARG(idx != nullptr, "attention: index is NULL");
  BF_CHECK_ARG(idx->n_q >= 0 && idx->n_kv >= 0 && idx->nnz >= 0, "attention: negative sizes");
  BF_CHECK_ARG(idx->n_q < (int64_t(1) << 31) && idx->n_kv < (int64_t(1) << 31) &&
                   idx->nnz < (int64_t(1) << 31),
               "attention: sizes must fit int32 ids");
  BF_CHECK_ARG(idx->chunk >= 1 && idx->item >= 1, "attention: chunk and item must be >= 1");
  BF_CHECK_ARG(idx->qptr && (idx->kv || idx->nnz == 0), "attention: qptr/kv missing");
  BF_CHECK_ARG(idx->q_items >= 0 && idx->q_heavy >= 0, "attention: bad query-side plan counts");
  BF_CHECK_ARG(idx->token_column >= 0 && idx->token_column <= 2, "attention: token_column must be 0, 1 or 2");
  BF_CHECK_ARG(idx->q_items == 0 || (idx->q_nitems && idx->q_item_off && idx->q_item_row && idx->q_heavy_rows),
               "attention: query-side split plan missing");
  if (backward) {
    BF_CHECK_ARG(idx->kptr && (idx->kq || idx->nnz == 0), "attention: reverse index missing");
    BF_CHECK_ARG(idx->k_items >= 0 && idx->k_heavy >= 0, "attention: bad key-side plan counts");
    BF_CHECK_ARG(idx->k_items == 0 || (idx->k_nitems && idx->k_item_off && idx->k_item_row && idx->k_heavy_rows),
                 "attention: key-side split plan missing");
    BF_CHECK_ARG(!idx->k_spans || idx->k_order, "attention: k_spans describe the slots of k_order, which is NULL");
  }
  return BF_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Short kv rows per lane group in the dk/dv pass: 1, or 4 past 16M kv rows,
// where fewer and longer-lived workgroups were measured faster (c5's 111M kv
// rows: 44.9 -> 40.4 ms) while on small tables the extra rows per group cost
// parallelism (c2: 2x slower). The query-side passes keep one row per group:
// four were measured no faster for the dq pass and 4% slower for the forward
// at c5's 27.8M queries. In bf16, where a group's slots are loaded in one
// round, four rows per group also pay from 1M kv rows on (c3's 2.45M: dk/dv
// pass 3.30 -> 3.26 ms; c4's 2.92M: 3.63 -> 3.61 ms; two rows gave the same).
constexpr int64_t kManyRows = int64_t(1) << 24;
constexpr int64_t kManyRowsBf16 = int64_t(1) << 20;
inline int kv_rows_per_group(int64_t n_kv, size_t elem_bytes) {
  return n_kv > (elem_bytes == 2 ? kManyRowsBf16 : kManyRows) ? 4 : 1;
}

inline unsigned grid_for(int64_t rows, const Shape& sh) {
  const int64_t per_block = kBlock >> sh.lpr_log2;
  return unsigned(ceil_div(rows, per_block));
}

inline size_t combine_lds_bytes(const Shape& sh) {
  return size_t(kBlock >> sh.lpr_log2) * size_t(2 * sh.D + sh.H) * sizeof(float);
}

inline Items query_items(const bf_attn_index* idx, const Shape& sh, float* partials) {
  return Items{idx->qptr, idx->q_item_off, idx->q_item_row, idx->q_nitems, idx->q_heavy_rows, partials,
               idx->item, 2 * sh.D + sh.H};
}

// Key-side records follow the query-side ones, so the dk/dv launch can reduce
// the dq split rows while its items write their own records.
inline Items key_items(const bf_attn_index* idx, const Shape& sh, float* partials) {
  return Items{idx->kptr, idx->k_item_off, idx->k_item_row, idx->k_nitems, idx->k_heavy_rows,
               partials + int64_t(idx->q_items) * (2 * sh.D + sh.H), idx->item, 2 * sh.D + sh.H};
}

// The per-entry inputs of a call, with the dropout's Philox key and threshold.
int make_edge_in(const float* bias, const float* factor, const bf_attn_dropout* dropout, int H, EdgeIn& ex) {
  ex = EdgeIn{bias, factor, nullptr, 0, 1.f, 1.f, 0u, 0u, 0u, 0u, nullptr, (H + 7) / 8};
  if (dropout) {
    BF_CHECK_ARG(dropout->rate >= 0.f && dropout->rate <= 1.f, "attention: dropout rate %g outside [0, 1]",
                 double(dropout->rate));
    if (dropout->rate > 0.f) {
      ex.drop = 1;
      ex.keep = 1.f - dropout->rate;
      ex.scale = dropout->rate < 1.f ? 1.f / (1.f - dropout->rate) : 0.f;
      ex.seed_lo = uint32_t(dropout->seed);
      ex.seed_hi = uint32_t(dropout->seed >> 32);
      ex.off_lo = uint32_t(dropout->offset);
      ex.off_hi = uint32_t(dropout->offset >> 32);
      ex.keepm = dropout->keep;
      BF_CHECK_ARG((reinterpret_cast<uintptr_t>(ex.keepm) & 3u) == 0, "attention: the keep mask must be 4-byte aligned");
    }
  }
  return BF_OK;
}

inline bool has_extra(const EdgeIn& ex) { return ex.bias || ex.factor || ex.drop; }

// The per-entry instance a call takes: 0 plain, 1 dropout only, 2 anything with a bias, factor or dbias,
// 4 dropout only with a keep mask (the forward stores the bits it draws, the dq pass reads them; the
// key-major pass takes instance 1 and draws).
inline int edge_mode(const EdgeIn& ex, bool dbias) {
  if (ex.bias || ex.factor || dbias) return 2;
  return ex.drop ? (ex.keepm ? 4 : 1) : 0;
}

template <typename T>
int fwd_impl(const bf_attn_index* idx, const Shape& sh, const void* q, const void* k, const void* v,
             const EdgeIn& ex, void* out, float* Z, float* partials, hipStream_t st) {
  const T* Q = static_cast<const T*>(q);
  const T* K = static_cast<const T*>(k);
  const T* Vv = static_cast<const T*>(v);
  T* O = static_cast<T*>(out);
  const Items it = query_items(idx, sh, partials);
  const int n_items = idx->q_items;
  const int64_t blocks = int64_t(n_items) + grid_for(idx->n_q, sh);
  if (blocks > 0) {
    const size_t lds = n_items > 0 ? combine_lds_bytes(sh) : 0;
#define BF_LAUNCH_FWD(EX)                                                                                        \
  BF_LAUNCH("attn_fwd_kernel", (attn_fwd_kernel<T, EX>), dim3(unsigned(blocks)), dim3(kBlock), lds, st, Q, K, Vv,  \
            idx->qptr, idx->kv, ex, O, Z, it, n_items, idx->n_q, sh, idx->chunk, idx->plan_counts)
    // the dropout-only instance stores the keep mask a window at a time, for one byte per entry (H <= 8)
    // and groups wide enough to share an iteration's draws; other shapes (more heads; H <= 3 with one lane
    // per head) take the general instance, which stores it too
    const bool shared_draws = Unroll<T>::fwd * ((sh.H + 3) >> 2) <= (1 << sh.lpr_log2);
    switch (edge_mode(ex, false)) {
      case 4:
        if (shared_draws && ex.kbytes == 1) {
          BF_LAUNCH_FWD(4);
        } else {
          BF_LAUNCH_FWD(2);
        }
        break;
      case 2: BF_LAUNCH_FWD(2); break;
      case 1: BF_LAUNCH_FWD(1); break;
      default: BF_LAUNCH_FWD(0); break;
    }
#undef BF_LAUNCH_FWD
    BF_CHECK_LAUNCH();
  }
  if (idx->q_heavy > 0) {
    BF_LAUNCH("attn_fwd_reduce_kernel", attn_fwd_reduce_kernel<T>, dim3(unsigned(idx->q_heavy)), dim3(kBlock),
              combine_lds_bytes(sh), st, O, Z, it, sh, idx->plan_counts);
    BF_CHECK_LAUNCH();
  }
  return BF_OK;
}

// The key-major pass and its reduce: the instance for the sizes (rows per group, non-temporal gathers,
// prefetched slots) and the per-entry mode (EX: 0 plain, 1 dropout, 2 bias / factor / dropout / dbias,
// 3 typed edges).
template <typename T>
int kv_pass_impl(const bf_attn_index* idx, const Shape& sh, const T* Q, const T* K, const T* Vv, const EdgeIn& ex,
                 int mode, float* dbias, const T* dO, const float2* rstat, void* dk, void* dv, const Items& kit,
                 const float* token_rec, hipStream_t st) {
  const int rows_per_group = kv_rows_per_group(idx->n_kv, sizeof(T));
  const int64_t kv_blocks = int64_t(idx->k_items) + grid_for(ceil_div(idx->n_kv, rows_per_group), sh);
  if (kv_blocks > 0) {
    // the token row's entries of the short kv rows take query 0's rows and stats from LDS, where a
    // workgroup's copy serves enough rows to pay for its wait (several rows per group: c5 dk/dv pass
    // 45.6 -> 44.6 ms); with one row per group the copy costs more than the gathers it spares (the
    // rows then gather query 0's entry like any other: c2 dk/dv pass 0.199 -> 0.205 ms with the copy)
    const int tok_row = idx->token_column == 1 && idx->n_q > 0 && rows_per_group > 1 ? 1 : 0;
    const size_t tok_lds = tok_row ? size_t(2 * sh.D) * sizeof(T) + size_t(sh.H) * sizeof(float2) : 0;
    const size_t lds = std::max(idx->k_items > 0 ? combine_lds_bytes(sh) : size_t(0), tok_lds);
    const bool stream_rows = size_t(idx->n_q) * size_t(sh.D) * sizeof(T) * 2 > kStreamBytes;
#define BF_LAUNCH_KV1(NT, PRE, EX)                                                                                 \
  BF_LAUNCH("attn_bwd_kv_kernel", (attn_bwd_kv_kernel<T, NT, PRE, EX>), dim3(unsigned(kv_blocks)), dim3(kBlock), lds, st, \
            Q, K, Vv, idx->kptr, idx->kq, idx->ks, idx->qptr, ex, dbias, dO, rstat, static_cast<T*>(dk),            \
            static_cast<T*>(dv), idx->k_order, idx->k_spans, kit, idx->k_items, idx->n_kv, sh, idx->chunk,           \
            rows_per_group, token_rec, idx->q_items, int64_t(grid_for(idx->n_q, sh)), tok_row, idx->plan_counts)
#define BF_LAUNCH_KV(NT, PRE)           \
  do {                                  \
    if (mode == 3)                      \
      BF_LAUNCH_KV1(NT, PRE, 3);        \
    else if (mode == 2)                 \
      BF_LAUNCH_KV1(NT, PRE, 2);        \
    else if (mode == 1)                 \
      BF_LAUNCH_KV1(NT, PRE, 1);        \
    else                                \
      BF_LAUNCH_KV1(NT, PRE, 0);        \
  } while (0)
    if constexpr (sizeof(T) == 2) {
      // the group's slots prefetched (several rows per group)
      const bool pre = rows_per_group > 1 && rows_per_group <= (1 << sh.lpr_log2);
      if (pre && stream_rows)
        BF_LAUNCH_KV(true, true);
      else if (pre)
        BF_LAUNCH_KV(false, true);
      else if (stream_rows)
        BF_LAUNCH_KV(true, false);
      else
        BF_LAUNCH_KV(false, false);
    } else {
      if (stream_rows)
        BF_LAUNCH_KV(true, false);
      else
        BF_LAUNCH_KV(false, false);
    }
#undef BF_LAUNCH_KV
#undef BF_LAUNCH_KV1
    BF_CHECK_LAUNCH();
  }
  if (idx->k_heavy > 0) {
    BF_LAUNCH("attn_bwd_kv_reduce_kernel", attn_bwd_kv_reduce_kernel<T>, dim3(unsigned(idx->k_heavy)), dim3(kBlock),
              combine_lds_bytes(sh), st, static_cast<T*>(dk), static_cast<T*>(dv), kit, sh, idx->plan_counts);
    BF_CHECK_LAUNCH();
  }
  return BF_OK;
}

template <typename T>
int bwd_impl(const bf_attn_index* idx, const Shape& sh, const void* q, const void* k, const void* v,
             const EdgeIn& ex, const float* Z, const void* dout, void* dq, void* dk, void* dv,
             float* dbias, float* rstat_f, float* partials, hipStream_t st) {
  float2* rstat = reinterpret_cast<float2*>(rstat_f);
  const T* Q = static_cast<const T*>(q);
  const T* K = static_cast<const T*>(k);
  const T* Vv = static_cast<const T*>(v);
  const T* dO = static_cast<const T*>(dout);
  const Items qit = query_items(idx, sh, partials);
  const Items kit = key_items(idx, sh, partials);
  const int64_t q_blocks = int64_t(idx->q_items) + grid_for(idx->n_q, sh);
  const int tok_first = idx->token_column == 2 ? 0 : 1;
  // token column: one record of key 0's terms per dq-pass workgroup, after the item records
  float* token_rec = idx->token_column && idx->n_kv > 0 && q_blocks > 0
                         ? partials + (int64_t(idx->q_items) + idx->k_items) * (2 * sh.D + sh.H)
                         : nullptr;
  if (q_blocks > 0) {
    const size_t lds = (idx->q_items > 0 || token_rec) ? combine_lds_bytes(sh) : 0;
#define BF_LAUNCH_Q(EX)                                                                                          \
  BF_LAUNCH("attn_bwd_q_kernel", (attn_bwd_q_kernel<T, EX>), dim3(unsigned(q_blocks)), dim3(kBlock), lds, st, Q, K, \
            Vv, idx->qptr, idx->kv, ex, Z, dO, static_cast<T*>(dq), dbias, rstat, qit, idx->q_items,                \
            idx->n_q, sh, idx->chunk, token_rec, tok_first, idx->plan_counts)
    // the mask is read back where an entry's bits fill one byte (H <= 8); wider rows of heads draw
    switch (edge_mode(ex, dbias != nullptr)) {
      case 4:
        if (ex.kbytes == 1) {
          BF_LAUNCH_Q(4);
        } else {
          BF_LAUNCH_Q(1);
        }
        break;
      case 2: BF_LAUNCH_Q(2); break;
      case 1: BF_LAUNCH_Q(1); break;
      default: BF_LAUNCH_Q(0); break;
    }
#undef BF_LAUNCH_Q
    BF_CHECK_LAUNCH();
  }
  // the query-side split rows finish (dq, row stats) before the key-major pass gathers their stats
  if (idx->q_heavy > 0) {
    BF_LAUNCH("attn_bwd_q_reduce_kernel", attn_bwd_q_reduce_kernel<T>, dim3(unsigned(idx->q_heavy)), dim3(kBlock),
              combine_lds_bytes(sh), st, Q, K, Vv, ex, Z, dO, static_cast<T*>(dq), dbias, rstat, qit, sh,
              token_rec, tok_first, idx->plan_counts);
    BF_CHECK_LAUNCH();
  }
  const int kv_mode = edge_mode(ex, dbias != nullptr);
  BF_CHECK_OK(kv_pass_impl<T>(idx, sh, Q, K, Vv, ex, kv_mode == 4 ? 1 : kv_mode, dbias, dO, rstat, dk, dv, kit,
                               token_rec, st));
  return BF_OK;
}

// ------------------------------------------------------------------ typed edges: host side
// Rows per lane group of the typed dq pass: about 2048 workgroups for large query sets (each writes one
// dE record), at most 16 rows per group.
inline int typed_rows_per_group(int64_t n_q, const Shape& sh) {
  const int64_t gpb = kBlock >> sh.lpr_log2;
  const int64_t r = n_q / (gpb * 2048);
  return int(r < 1 ? 1 : (r > 16 ? 16 : r));
}

inline int64_t typed_q_blocks(int64_t n_q, const Shape& sh) {
  return int64_t(grid_for(ceil_div(n_q, typed_rows_per_group(n_q, sh)), sh));
}

constexpr int64_t kModRecPerBlock = 256;   // dE records summed per workgroup in the first reduce pass

int check_typed(const bf_attn_index* idx, const float* mod) {
  BF_CHECK_ARG(mod != nullptr, "attn typed: type_mod is NULL");
  BF_CHECK_ARG(idx->token_column == 0, "attn typed: a typed index has no token column");
  BF_CHECK_ARG(idx->q_items == 0, "attn typed: a typed index splits no query row (q_items = %d)", idx->q_items);
  return BF_OK;
}

template <typename T>
int fwd_typed_impl(const bf_attn_index* idx, const Shape& sh, const void* q, const void* k, const void* v,
                   const float* mod, void* out, float* Z, hipStream_t st) {
  const unsigned blocks = grid_for(idx->n_q, sh);
  if (blocks == 0) return BF_OK;
  BF_LAUNCH("attn_fwd_typed_kernel", attn_fwd_typed_kernel<T>, dim3(blocks), dim3(kBlock), 0, st,
            static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), idx->qptr, idx->kv, mod,
            static_cast<T*>(out), Z, idx->n_q, sh);
  BF_CHECK_LAUNCH();
  return BF_OK;
}

template <typename T>
int bwd_typed_impl(const bf_attn_index* idx, const Shape& sh, const void* q, const void* k, const void* v,
                   const float* mod, const float* Z, const void* dout, void* dq, void* dk, void* dv, float* dmod,
                   float* rstat_f, float* partials, hipStream_t st) {
  float2* rstat = reinterpret_cast<float2*>(rstat_f);
  const T* Q = static_cast<const T*>(q);
  const T* K = static_cast<const T*>(k);
  const T* Vv = static_cast<const T*>(v);
  const T* dO = static_cast<const T*>(dout);
  const Items kit = key_items(idx, sh, partials);     // the key-side records first (q_items is 0)
  const int64_t n_rec = typed_q_blocks(idx->n_q, sh);
  float* mod_rec = partials + int64_t(idx->k_items) * (2 * sh.D + sh.H);
  float* mod_part = mod_rec + n_rec * (2 * sh.D);
  if (n_rec > 0) {
    BF_LAUNCH("attn_bwd_q_typed_kernel", attn_bwd_q_typed_kernel<T>, dim3(unsigned(n_rec)), dim3(kBlock),
              size_t(kBlock / 64) * size_t(2 * sh.D) * sizeof(float), st, Q, K, Vv, idx->qptr, idx->kv, mod, Z, dO,
              static_cast<T*>(dq), rstat, mod_rec, idx->n_q, typed_rows_per_group(idx->n_q, sh), sh);
    BF_CHECK_LAUNCH();
  }
  EdgeIn ex{nullptr, nullptr, mod, 0, 1.f, 1.f, 0u, 0u, 0u, 0u};
  BF_CHECK_OK(kv_pass_impl<T>(idx, sh, Q, K, Vv, ex, 3, nullptr, dO, rstat, dk, dv, kit, nullptr, st));
  // dE: the records summed in a fixed order, in two passes (an empty query set writes zeros)
  const int cols = 2 * sh.D;
  const int64_t n_part = n_rec > 0 ? ceil_div(n_rec, kModRecPerBlock) : 0;
  if (n_part > 1) {
    BF_LAUNCH("mod_rec_reduce_kernel", mod_rec_reduce_kernel, dim3(unsigned(n_part)), dim3(kBlock), 0, st, mod_rec,
              n_rec, cols, kModRecPerBlock, mod_part);
    BF_CHECK_LAUNCH();
    BF_LAUNCH("mod_rec_reduce_kernel", mod_rec_reduce_kernel, dim3(1), dim3(kBlock), 0, st, mod_part, n_part, cols,
              n_part, dmod);
  } else {
    BF_LAUNCH("mod_rec_reduce_kernel", mod_rec_reduce_kernel, dim3(1), dim3(kBlock), 0, st, mod_rec, n_rec, cols,
              n_rec, dmod);
  }
  BF_CHECK_LAUNCH();
  return BF_OK;
}

}  // namespace
}  // namespace bf

using namespace bf;

extern "C" int64_t bf_attn_partials_floats(const bf_attn_index* idx, int32_t num_heads, int32_t head_dim) {
  if (!idx || num_heads <= 0 || head_dim <= 0) return 0;
  const int64_t items = int64_t(idx->q_items) + idx->k_items;   // query-side records, then key-side
  const int64_t D = int64_t(num_heads) * head_dim;
  int64_t floats = items * (2 * D + num_heads);
  if (idx->token_column) {
    // one 2*D record per dq-pass workgroup; float32 rows take the most lanes per row, hence the most
    // workgroups (bfloat16 rows half as many lanes)
    int64_t lpr = 1;
    while (lpr < (D + 3) / 4 && lpr < 64) lpr <<= 1;
    const int64_t rows_per_block = kBlock / lpr;
    floats += (int64_t(idx->q_items) + ceil_div(idx->n_q, rows_per_block)) * 2 * D;
  }
  return floats;
}

extern "C" int bf_attn_bwd_kv_variant(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim,
                                      int32_t* rows_per_group, int32_t* stream_rows, int32_t* prefetch_slots) {
  Shape sh;
  int rc = make_shape(dtype, num_heads, head_dim, sh);
  if (rc) return rc;
  BF_CHECK_ARG(idx && idx->n_q >= 0 && idx->n_kv >= 0, "attn_bwd_kv_variant: bad index");
  BF_CHECK_ARG(rows_per_group && stream_rows && prefetch_slots, "attn_bwd_kv_variant: null output");
  const size_t s = dtype == BF_DTYPE_F32 ? sizeof(float) : sizeof(uint16_t);   // bf16 and fp16: 2 bytes
  const int rpg = kv_rows_per_group(idx->n_kv, s);
  *rows_per_group = rpg;
  *stream_rows = size_t(idx->n_q) * size_t(sh.D) * s * 2 > kStreamBytes ? 1 : 0;
  *prefetch_slots = (s == 2 && rpg > 1 && rpg <= (1 << sh.lpr_log2)) ? 1 : 0;
  return BF_OK;
}

extern "C" int bf_attn_fwd(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim,
                           float score_clamp, const void* q, const void* k, const void* v, const float* bias,
                           const float* factor, const bf_attn_dropout* dropout, void* out, float* Z,
                           float* partials, void* stream) {
  Shape sh;
  int rc = make_shape(dtype, num_heads, head_dim, sh);
  if (rc || (rc = set_clamp(score_clamp, sh))) return rc;
  if ((rc = check_index(idx, false))) return rc;
  EdgeIn ex;
  if ((rc = make_edge_in(bias, factor, dropout, num_heads, ex))) return rc;
  BF_CHECK_ARG(q && k && v && out && Z, "attn_fwd: null tensor");
  BF_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out),
               "attn_fwd: q/k/v/out must be 16-byte aligned");
  BF_CHECK_ARG(idx->q_items == 0 || partials, "attn_fwd: partials buffer required for split rows");
  if (dtype == BF_DTYPE_F32)
    return fwd_impl<float>(idx, sh, q, k, v, ex, out, Z, partials, as_stream(stream));
  if (dtype == BF_DTYPE_F16)
    return fwd_impl<_Float16>(idx, sh, q, k, v, ex, out, Z, partials, as_stream(stream));
  return fwd_impl<uint16_t>(idx, sh, q, k, v, ex, out, Z, partials, as_stream(stream));
}

extern "C" int bf_attn_bwd(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim,
                           float score_clamp, const void* q, const void* k, const void* v, const float* bias,
                           const float* factor, const bf_attn_dropout* dropout, const float* Z, const void* dout,
                           void* dq, void* dk, void* dv, float* dbias, float* rowstat, float* partials,
                           void* stream) {
  Shape sh;
  int rc = make_shape(dtype, num_heads, head_dim, sh);
  if (rc || (rc = set_clamp(score_clamp, sh))) return rc;
  if ((rc = check_index(idx, true))) return rc;
  EdgeIn ex;
  if ((rc = make_edge_in(bias, factor, dropout, num_heads, ex))) return rc;
  BF_CHECK_ARG(idx->ks || idx->nnz == 0 || (!has_extra(ex) && !dbias),
               "attn_bwd: a bias, factor, dropout or dbias needs the reverse entries' slots (ks)");
  BF_CHECK_ARG(q && k && v && Z && dout && dq && dk && dv && rowstat, "attn_bwd: null tensor");
  BF_CHECK_ARG((reinterpret_cast<uintptr_t>(rowstat) & 7u) == 0, "attn_bwd: rowstat must be 8-byte aligned");
  BF_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(dout) && aligned16(dq) && aligned16(dk) &&
                   aligned16(dv),
               "attn_bwd: tensors must be 16-byte aligned");
  BF_CHECK_ARG((idx->q_items == 0 && idx->k_items == 0 && !idx->token_column) || partials,
               "attn_bwd: partials buffer required for split rows and the token column");
  if (dtype == BF_DTYPE_F32)
    return bwd_impl<float>(idx, sh, q, k, v, ex, Z, dout, dq, dk, dv, dbias, rowstat, partials,
                           as_stream(stream));
  if (dtype == BF_DTYPE_F16)
    return bwd_impl<_Float16>(idx, sh, q, k, v, ex, Z, dout, dq, dk, dv, dbias, rowstat, partials,
                              as_stream(stream));
  return bwd_impl<uint16_t>(idx, sh, q, k, v, ex, Z, dout, dq, dk, dv, dbias, rowstat, partials,
                            as_stream(stream));
}

// ------------------------------------------------------------------ typed edges (Exphormer)
extern "C" int64_t bf_attn_typed_partials_floats(const bf_attn_index* idx, int32_t dtype, int32_t num_heads,
                                                 int32_t head_dim) {
  Shape sh;
  if (!idx || make_shape(dtype, num_heads, head_dim, sh) != BF_OK) return 0;
  const int64_t n_rec = typed_q_blocks(idx->n_q, sh);
  const int64_t n_part = n_rec > 0 ? ceil_div(n_rec, kModRecPerBlock) : 0;
  return int64_t(idx->k_items) * (2 * sh.D + sh.H) + (n_rec + n_part) * (2 * sh.D);
}

extern "C" int bf_attn_fwd_typed(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim,
                                 const void* q, const void* k, const void* v, const float* type_mod, void* out,
                                 float* Z, void* stream) {
  Shape sh;
  int rc = make_shape(dtype, num_heads, head_dim, sh);
  if (rc || (rc = check_index(idx, false)) || (rc = check_typed(idx, type_mod))) return rc;
  BF_CHECK_ARG(q && k && v && out && Z, "attn_fwd_typed: null tensor");
  BF_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) && aligned16(type_mod),
               "attn_fwd_typed: q/k/v/out/type_mod must be 16-byte aligned");
  if (dtype == BF_DTYPE_F32) return fwd_typed_impl<float>(idx, sh, q, k, v, type_mod, out, Z, as_stream(stream));
  if (dtype == BF_DTYPE_F16) return fwd_typed_impl<_Float16>(idx, sh, q, k, v, type_mod, out, Z, as_stream(stream));
  return fwd_typed_impl<uint16_t>(idx, sh, q, k, v, type_mod, out, Z, as_stream(stream));
}

extern "C" int bf_attn_bwd_typed(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim,
                                 const void* q, const void* k, const void* v, const float* type_mod, const float* Z,
                                 const void* dout, void* dq, void* dk, void* dv, float* dtype_mod, float* rowstat,
                                 float* partials, void* stream) {
  Shape sh;
  int rc = make_shape(dtype, num_heads, head_dim, sh);
  if (rc || (rc = check_index(idx, true)) || (rc = check_typed(idx, type_mod))) return rc;
  BF_CHECK_ARG(q && k && v && Z && dout && dq && dk && dv && dtype_mod && rowstat && partials,
               "attn_bwd_typed: null tensor");
  BF_CHECK_ARG((reinterpret_cast<uintptr_t>(rowstat) & 7u) == 0, "attn_bwd_typed: rowstat must be 8-byte aligned");
  BF_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(dout) && aligned16(dq) && aligned16(dk) &&
                   aligned16(dv) && aligned16(type_mod),
               "attn_bwd_typed: tensors must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  if (dtype == BF_DTYPE_F32)
    return bwd_typed_impl<float>(idx, sh, q, k, v, type_mod, Z, dout, dq, dk, dv, dtype_mod, rowstat, partials, st);
  if (dtype == BF_DTYPE_F16)
    return bwd_typed_impl<_Float16>(idx, sh, q, k, v, type_mod, Z, dout, dq, dk, dv, dtype_mod, rowstat, partials,
                                    st);
  return bwd_typed_impl<uint16_t>(idx, sh, q, k, v, type_mod, Z, dout, dq, dk, dv, dtype_mod, rowstat, partials, st);
}

// ------------------------------------------------------------------ allocation-free backward
// bf_attn_bwd's scratch (the row stats and the split partials) for callers that
// cannot allocate: one file-scope device array, BF_ATTN_NOALLOC_SCRATCH_BYTES
// on every GPU the library runs on, held until the process ends. Its address on
// a device is looked up once (hipGetSymbolAddress with that device current) and
// kept; host code never passes the array's own name, which is a host-side
// stand-in. Every call on a GPU shares that GPU's array and finds the previous
// call's contents there; nothing in it needs to start at zero (each pass writes
// every row stat and record before the next pass reads it). Calls that overlap
// on one GPU, on any streams, race on it.
static __device__ __align__(256) unsigned char scratch[BF_ATTN_NOALLOC_SCRATCH_BYTES];

namespace bf {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];   // per device; a plain array: no destructor at exit

int scratch_address(void** out) {
  int dev = 0;
  BF_CHECK_HIP(hipGetDevice(&dev));
  BF_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "attn_bwd_noalloc: device %d beyond the %d the library tracks", dev,
               kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    BF_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    BF_CHECK_ARG(p != nullptr, "attn_bwd_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return BF_OK;
}

}  // namespace
}  // namespace bf

extern "C" int bf_attn_bwd_noalloc(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim,
                                   float score_clamp, const void* q, const void* k, const void* v,
                                   const float* bias, const float* factor, const bf_attn_dropout* dropout,
                                   const float* Z, const void* dout, void* dq, void* dk, void* dv, float* dbias,
                                   void* stream) {
  Shape sh;
  int rc = make_shape(dtype, num_heads, head_dim, sh);
  if (rc || (rc = set_clamp(score_clamp, sh))) return rc;
  if ((rc = check_index(idx, true))) return rc;
  const size_t stat_bytes = (size_t(idx->n_q) * size_t(num_heads) * 2 * sizeof(float) + 255) & ~size_t(255);
  const int64_t part_floats = bf_attn_partials_floats(idx, num_heads, head_dim);
  const size_t need = stat_bytes + size_t(part_floats) * sizeof(float);
  BF_CHECK_ARG(need <= size_t(BF_ATTN_NOALLOC_SCRATCH_BYTES),
               "attn_bwd_noalloc: this index needs %zu bytes of scratch (row stats %zu + partials %zu); the static "
               "array holds %zu (use bf_attn_bwd with caller-provided scratch)",
               need, stat_bytes, size_t(part_floats) * sizeof(float), size_t(BF_ATTN_NOALLOC_SCRATCH_BYTES));
  void* base = nullptr;
  if ((rc = scratch_address(&base))) return rc;
  float* rowstat = static_cast<float*>(base);
  float* partials = reinterpret_cast<float*>(static_cast<unsigned char*>(base) + stat_bytes);
  ProfPause no_timer;   // the timer would create events
  return bf_attn_bwd(idx, dtype, num_heads, head_dim, score_clamp, q, k, v, bias, factor, dropout, Z, dout, dq, dk,
                     dv, dbias, rowstat, partials, stream);
}
