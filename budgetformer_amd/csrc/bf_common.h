// Shared device/host helpers for the BudgetFormer MI355X (gfx950) kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/budgetformer_hip.h"

namespace bf {

// ---------------------------------------------------------------- errors
void set_error(const char* fmt, ...);

#define BF_CHECK_ARG(cond, ...)                         \
  do {                                                  \
    if (!(cond)) {                                      \
      ::bf::set_error(__VA_ARGS__);                     \
      return BF_ERR_INVALID;                            \
    }                                                   \
  } while (0)

#define BF_CHECK_HIP(expr)                                                          \
  do {                                                                              \
    hipError_t _e = (expr);                                                         \
    if (_e != hipSuccess) {                                                         \
      ::bf::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e),        \
                      __FILE__, __LINE__);                                          \
      return BF_ERR_HIP;                                                            \
    }                                                                               \
  } while (0)

#define BF_CHECK_LAUNCH() BF_CHECK_HIP(hipGetLastError())

// Returns the code of a failing library call (its message is already set).
#define BF_CHECK_OK(expr)       \
  do {                          \
    const int _rc = (expr);     \
    if (_rc != BF_OK) return _rc; \
  } while (0)

// Optional per-kernel timing (bf_prof_enable): an event pair around each launch.
bool prof_enabled();
void prof_begin(const char* name, hipStream_t st, int* token);
void prof_end(int token, hipStream_t st);

// Keeps the timer off for the calling thread while in scope (the timer creates
// events and grows host lists, which an allocation-free call must not do).
struct ProfPause {
  ProfPause();
  ~ProfPause();
  bool prev;
};

// Launches a kernel (in a function returning an error code). A dispatch counts
// its work-items per dimension in 32 bits, so a grid of 2^32 or more would be
// cut short without an error: such a launch is refused instead.
#define BF_LAUNCH(name, kern, grid, block, lds, st, ...)                                        \
  do {                                                                                         \
    const dim3 _bf_g = (grid), _bf_b = (block);                                                \
    BF_CHECK_ARG(uint64_t(_bf_g.x) * _bf_b.x <= 0xffffffffull,                                  \
                 "%s: a grid of %llu work-items (a dispatch takes at most 2^32 - 1)", name,     \
                 (unsigned long long)(uint64_t(_bf_g.x) * _bf_b.x));                            \
    int _bf_tok = -1;                                                                          \
    if (::bf::prof_enabled()) ::bf::prof_begin(name, st, &_bf_tok);                            \
    hipLaunchKernelGGL(kern, _bf_g, _bf_b, lds, st, __VA_ARGS__);                              \
    if (_bf_tok >= 0) ::bf::prof_end(_bf_tok, st);                                             \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// The chip's 8 XCDs each have their own L2, and workgroup i of a launch runs on
// XCD i % 8. xcd_slot maps workgroup i of n to a slot such that each XCD takes
// one contiguous run of slots (XCD x: slots [x*q + min(x, r), ...) with n =
// 8q + r, q + 1 of them for x < r, else q), in its own dispatch order; a
// bijection of [0, n). Neighbouring slots then share their L2 lines in one
// L2 instead of eight.
constexpr int kXcds = 8;
__device__ __forceinline__ int64_t xcd_slot(int64_t i, int64_t n) {
  const int64_t q = n / kXcds, r = n % kXcds;
  const int64_t x = i % kXcds, local = i / kXcds;
  return x * q + (x < r ? x : r) + local;
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

// Items a split row of `len` entries is cut into: ceil(len / item_size), at
// most BF_MAX_ITEMS_PER_ROW, except that a row of more than
// BF_MAX_ITEMS_PER_ROW * BF_LONG_ROW_FACTOR items' worth of entries (the
// Graphormer token row of a 100M-node graph) takes ceil(len / (item_size *
// BF_LONG_ROW_FACTOR)) items, so its items still spread over the whole chip.
__host__ __device__ inline int64_t split_row_items(int64_t len, int item_size) {
  int64_t n = ceil_div(len, int64_t(item_size));
  if (n > BF_MAX_ITEMS_PER_ROW) {
    const int64_t big = ceil_div(len, int64_t(item_size) * BF_LONG_ROW_FACTOR);
    n = big > BF_MAX_ITEMS_PER_ROW ? big : BF_MAX_ITEMS_PER_ROW;
  }
  return n;
}

inline int ilog2(int64_t x) {
  int r = 0;
  while ((int64_t(1) << (r + 1)) <= x) ++r;
  return r;
}

// ---------------------------------------------------------------- bf16
// bf16 stored as raw uint16 (upper half of an IEEE float).
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(uint32_t(h) << 16);
}

// Round-to-nearest-even float -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return uint16_t((x >> 16) | 0x40u);
  uint32_t lsb = (x >> 16) & 1u;
  x += 0x7fffu + lsb;
  return uint16_t(x >> 16);
}

// Element traits: each lane moves 16 bytes (one dwordx4) of a row.
template <typename T> struct Elem;

template <> struct Elem<float> {
  static constexpr int kPerVec = 4;
  using Raw = float4;
  __device__ __forceinline__ static Raw load_raw(const float* p) { return *reinterpret_cast<const float4*>(p); }
  __device__ __forceinline__ static Raw load_raw_nt(const float* p) {
    typedef float V4 __attribute__((ext_vector_type(4)));
    const V4 v = __builtin_nontemporal_load(reinterpret_cast<const V4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
  }
  __device__ __forceinline__ static Raw zero_raw() { return make_float4(0.f, 0.f, 0.f, 0.f); }
  __device__ __forceinline__ static void unpack(const Raw& v, float (&o)[4]) {
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  }
  // acc + sum of the four products of a and b, in element order
  __device__ __forceinline__ static float dot(const Raw& a, const Raw& b, float acc) {
    acc = fmaf(a.x, b.x, acc);
    acc = fmaf(a.y, b.y, acc);
    acc = fmaf(a.z, b.z, acc);
    return fmaf(a.w, b.w, acc);
  }
  __device__ __forceinline__ static void load(const float* p, float (&o)[4]) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  }
  __device__ __forceinline__ static void store(float* p, const float (&o)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(o[0], o[1], o[2], o[3]);
  }
  // non-temporal: for rows written once and not read again in the same pass
  __device__ __forceinline__ static void store_nt(float* p, const float (&o)[4]) {
    typedef float V4 __attribute__((ext_vector_type(4)));
    const V4 v = {o[0], o[1], o[2], o[3]};
    __builtin_nontemporal_store(v, reinterpret_cast<V4*>(p));
  }
};

template <> struct Elem<uint16_t> {
  static constexpr int kPerVec = 8;
  using Raw = uint4;
  typedef __bf16 Pair __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static Pair as_pair(uint32_t w) { return __builtin_bit_cast(Pair, w); }
  __device__ __forceinline__ static Raw load_raw(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
  // non-temporal: the line is not kept in the caches (rows gathered once per pass from a table larger than them)
  __device__ __forceinline__ static Raw load_raw_nt(const uint16_t* p) {
    typedef unsigned V4 __attribute__((ext_vector_type(4)));
    const V4 v = __builtin_nontemporal_load(reinterpret_cast<const V4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  }
  __device__ __forceinline__ static Raw zero_raw() { return make_uint4(0u, 0u, 0u, 0u); }
  // acc + sum of the eight products of a and b, straight from the packed pairs
  // (v_dot2 with an fp32 accumulator; bf16 products are exact in fp32)
  __device__ __forceinline__ static float dot(const Raw& a, const Raw& b, float acc) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(as_pair(a.x), as_pair(b.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(as_pair(a.y), as_pair(b.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(as_pair(a.z), as_pair(b.z), acc, false);
    return __builtin_amdgcn_fdot2_f32_bf16(as_pair(a.w), as_pair(b.w), acc, false);
  }
  __device__ __forceinline__ static void unpack(const Raw& v, float (&o)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void load(const uint16_t* p, float (&o)[8]) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void store(uint16_t* p, const float (&o)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = uint32_t(f32_to_bf16(o[2 * i])) | (uint32_t(f32_to_bf16(o[2 * i + 1])) << 16);
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  __device__ __forceinline__ static void store_nt(uint16_t* p, const float (&o)[8]) {
    typedef unsigned V4 __attribute__((ext_vector_type(4)));
    V4 w;
    w.x = uint32_t(f32_to_bf16(o[0])) | (uint32_t(f32_to_bf16(o[1])) << 16);
    w.y = uint32_t(f32_to_bf16(o[2])) | (uint32_t(f32_to_bf16(o[3])) << 16);
    w.z = uint32_t(f32_to_bf16(o[4])) | (uint32_t(f32_to_bf16(o[5])) << 16);
    w.w = uint32_t(f32_to_bf16(o[6])) | (uint32_t(f32_to_bf16(o[7])) << 16);
    __builtin_nontemporal_store(w, reinterpret_cast<V4*>(p));
  }
};

// IEEE fp16 activations (the reference's fp16 autocast: utils/parser_node_level.py:266-272). Products of
// two fp16 values are exact in fp32, so v_dot2_f32_f16 with an fp32 accumulator forms the same sums the
// fp32 path forms; results are rounded to fp16 (round to nearest even) only when stored.
template <> struct Elem<_Float16> {
  static constexpr int kPerVec = 8;
  using Raw = uint4;
  typedef _Float16 Pair __attribute__((ext_vector_type(2)));
  __device__ __forceinline__ static Pair as_pair(uint32_t w) { return __builtin_bit_cast(Pair, w); }
  __device__ __forceinline__ static uint32_t pack(float a, float b) {
    const Pair p = {_Float16(a), _Float16(b)};
    return __builtin_bit_cast(uint32_t, p);
  }
  __device__ __forceinline__ static Raw load_raw(const _Float16* p) { return *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ static Raw load_raw_nt(const _Float16* p) {
    typedef unsigned V4 __attribute__((ext_vector_type(4)));
    const V4 v = __builtin_nontemporal_load(reinterpret_cast<const V4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  }
  __device__ __forceinline__ static Raw zero_raw() { return make_uint4(0u, 0u, 0u, 0u); }
  __device__ __forceinline__ static float dot(const Raw& a, const Raw& b, float acc) {
    acc = __builtin_amdgcn_fdot2(as_pair(a.x), as_pair(b.x), acc, false);
    acc = __builtin_amdgcn_fdot2(as_pair(a.y), as_pair(b.y), acc, false);
    acc = __builtin_amdgcn_fdot2(as_pair(a.z), as_pair(b.z), acc, false);
    return __builtin_amdgcn_fdot2(as_pair(a.w), as_pair(b.w), acc, false);
  }
  __device__ __forceinline__ static void unpack(const Raw& v, float (&o)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const Pair p = as_pair(w[i]);
      o[2 * i] = float(p.x);
      o[2 * i + 1] = float(p.y);
    }
  }
  __device__ __forceinline__ static void load(const _Float16* p, float (&o)[8]) { unpack(load_raw(p), o); }
  __device__ __forceinline__ static void store(_Float16* p, const float (&o)[8]) {
    *reinterpret_cast<uint4*>(p) = make_uint4(pack(o[0], o[1]), pack(o[2], o[3]), pack(o[4], o[5]), pack(o[6], o[7]));
  }
  __device__ __forceinline__ static void store_nt(_Float16* p, const float (&o)[8]) {
    typedef unsigned V4 __attribute__((ext_vector_type(4)));
    V4 w;
    w.x = pack(o[0], o[1]);
    w.y = pack(o[2], o[3]);
    w.z = pack(o[4], o[5]);
    w.w = pack(o[6], o[7]);
    __builtin_nontemporal_store(w, reinterpret_cast<V4*>(p));
  }
};

// 16 zero bytes at p (16-byte aligned) by a non-temporal vector store: rows
// written once and not read again in the pass do not displace cached data.
__device__ __forceinline__ void store_zero16_nt(void* p) {
  typedef unsigned V4 __attribute__((ext_vector_type(4)));
  const V4 z = {0u, 0u, 0u, 0u};
  __builtin_nontemporal_store(z, reinterpret_cast<V4*>(p));
}

// Butterfly sum over aligned groups of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float group_sum(float x, int width) {
  for (int o = 1; o < width; o <<= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// ---------------------------------------------------------------- row pointers from sorted keys
// Kernels that turn sorted row ids into row pointers give each key's thread
// the rows (lo, hi] that start at it: the rows between the previous key's id
// and its own, which have no keys of their own. A gap of up to kGapInline rows
// is written by its own lane; a longer one (a range of ids no entry reaches,
// the tail past the largest id) by every active lane of the wave in turn, so
// one lane never stores millions of pointers alone. write(r, val) stores row
// r's pointer; val is the gap's value (its key's index). Call it from every
// active lane of the wave (lanes without a gap pass hi <= lo).
constexpr int64_t kGapInline = 32;

template <typename F>
__device__ __forceinline__ void fill_gap(int64_t lo, int64_t hi, int64_t val, F&& write) {
  const bool wide = hi - lo > kGapInline;
  if (!wide)
    for (int64_t r = lo + 1; r <= hi; ++r) write(r, val);
  uint64_t pending = __ballot(wide);
  if (pending == 0) return;
  const uint64_t active = __ballot(1);
  const int lane = __lane_id();
  const int64_t rank = __popcll(active & ((uint64_t(1) << lane) - 1));
  const int64_t width = __popcll(active);
  while (pending) {
    const int src = __ffsll((unsigned long long)pending) - 1;
    pending &= pending - 1;
    const int64_t g_lo = __shfl(lo, src), g_hi = __shfl(hi, src), g_val = __shfl(val, src);
    for (int64_t r = g_lo + 1 + rank; r <= g_hi; r += width) write(r, g_val);
  }
}

// ---------------------------------------------------------------- keys
// (src*1103515245 + dst*214013 + c) mod 2^31 with c = seed*2654435761 + 12345,
// computed as the low 31 bits of the uint32-wrapped sum (utils/fullgraph_sp_support.py:984-989).
__host__ __device__ __forceinline__ uint32_t edge_key(uint32_t src, uint32_t dst, uint32_t c) {
  return (src * 1103515245u + dst * 214013u + c) & 0x7fffffffu;
}

inline uint32_t key_const(int64_t seed) {
  return uint32_t(uint64_t(seed) * 2654435761ull + 12345ull);
}

// ---------------------------------------------------------------- Philox4x32-10
// Counter-based RNG of Salmon, Moraes, Dror, Shaw, "Parallel random numbers:
// as easy as 1, 2, 3" (SC'11): 10 rounds of a 4x32 multiply-xor bijection with
// a Weyl-sequence key schedule.
struct U32x4 { uint32_t x, y, z, w; };

__host__ __device__ __forceinline__ void mulhilo32(uint32_t a, uint32_t b, uint32_t& hi, uint32_t& lo) {
  const uint64_t p = uint64_t(a) * uint64_t(b);
  hi = uint32_t(p >> 32);
  lo = uint32_t(p);
}

__host__ __device__ __forceinline__ U32x4 philox4x32_10(U32x4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    uint32_t hi0, lo0, hi1, lo1;
    mulhilo32(0xD2511F53u, c.x, hi0, lo0);
    mulhilo32(0xCD9E8D57u, c.z, hi1, lo1);
    c = U32x4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

// Uniform in [0, 1 - 2^-24]: top 24 bits times 2^-24 (exact in fp32).
__host__ __device__ __forceinline__ float u24(uint32_t x) {
  return float(x >> 8) * (1.0f / 16777216.0f);
}

// Uniform for walk `w`, step `l`: one Philox call serves 4 consecutive steps.
// counter = (w_lo, w_hi, offset_lo + l/4, offset_hi), key = (seed_lo, seed_hi).
__host__ __device__ __forceinline__ float walk_uniform(uint64_t seed, uint64_t offset, uint64_t w, int l) {
  const uint64_t blk = offset + uint64_t(l >> 2);
  U32x4 c{uint32_t(w), uint32_t(w >> 32), uint32_t(blk), uint32_t(blk >> 32)};
  const U32x4 r = philox4x32_10(c, uint32_t(seed), uint32_t(seed >> 32));
  const int j = l & 3;
  const uint32_t x = j == 0 ? r.x : j == 1 ? r.y : j == 2 ? r.z : r.w;
  return u24(x);
}

// walk_uniform for the steps l = 0, 1, 2, ... of one walk in order: one Philox
// call per 4 steps instead of one per step (the same values).
struct WalkStream {
  uint64_t seed, offset, w;
  U32x4 r;
  __device__ __forceinline__ float at(int l) {
    const int j = l & 3;
    if (j == 0) {
      const uint64_t blk = offset + uint64_t(l >> 2);
      r = philox4x32_10(U32x4{uint32_t(w), uint32_t(w >> 32), uint32_t(blk), uint32_t(blk >> 32)}, uint32_t(seed),
                        uint32_t(seed >> 32));
    }
    return u24(j == 0 ? r.x : j == 1 ? r.y : j == 2 ? r.z : r.w);
  }
};

}  // namespace bf
