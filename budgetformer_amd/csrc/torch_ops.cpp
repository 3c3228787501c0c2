// TORCH_LIBRARY(bf, ...) operators over the C ABI (include/budgetformer_hip.h):
// the hot path's entry points as PyTorch operators taking and returning
// at::Tensor, launched on the current HIP stream of the inputs' device. Outputs
// and scratch come from PyTorch's caching allocator (a failed allocation raises
// torch.OutOfMemoryError), argument errors raise ValueError or
// NotImplementedError, HIP errors RuntimeError, as the ctypes bindings do.
// Host code only: every kernel is in libbudgetformer_hip.so.
//
// The attention index (bf_attn_index) travels as 16 optional tensors and 10
// integers, in the order of kIndexTensors and make_index below
// (budgetformer_amd.hip_ops.AttentionIndex.op_args builds them).
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <string>

#include "budgetformer_hip.h"

namespace {

void check_rc(int rc, const char* what) {
  if (rc == BF_OK) return;
  const std::string msg = bf_last_error();
  TORCH_CHECK_VALUE(rc != BF_ERR_INVALID, what, ": ", msg);
  TORCH_CHECK_NOT_IMPLEMENTED(rc != BF_ERR_UNSUPPORTED, what, ": ", msg);
  TORCH_CHECK(false, what, ": ", msg);
}

void* stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void require(const at::Tensor& t, const char* name, at::ScalarType st, const at::Device& dev) {
  TORCH_CHECK_VALUE(t.defined(), name, " is undefined");
  TORCH_CHECK_VALUE(t.device() == dev, name, " is on ", t.device(), ", expected ", dev);
  TORCH_CHECK_VALUE(t.scalar_type() == st, name, " must be ", st, " (got ", t.scalar_type(), ")");
  TORCH_CHECK_VALUE(t.is_contiguous(), name, " must be contiguous");
}

template <typename P>
P* opt_ptr(const std::optional<at::Tensor>& t, const char* name, at::ScalarType st, const at::Device& dev) {
  if (!t.has_value() || !t->defined()) return nullptr;
  require(*t, name, st, dev);
  return static_cast<P*>(t->data_ptr());
}

at::Tensor scratch_bytes(size_t bytes, const at::Device& dev) {
  return at::empty({int64_t(std::max<size_t>(bytes, 1))}, at::TensorOptions().dtype(at::kByte).device(dev));
}

// ---------------------------------------------------------------- attention index
constexpr const char* kIndexTensors[16] = {"qptr",       "kv",         "kptr",         "kq",
                                           "ks",         "q_nitems",   "q_item_off",   "q_item_row",
                                           "q_heavy_rows", "k_nitems", "k_item_off",   "k_item_row",
                                           "k_heavy_rows", "k_order",  "k_spans",      "plan_counts"};
// The 10 integers, in order: n_q, n_kv, nnz, chunk, item, q_items, q_heavy, k_items, k_heavy, token_column.

bf_attn_index make_index(const c10::List<std::optional<at::Tensor>>& t, at::IntArrayRef n, const at::Device& dev) {
  TORCH_CHECK_VALUE(t.size() == 16, "attention index: 16 tensors expected (got ", t.size(), ")");
  TORCH_CHECK_VALUE(n.size() == 10, "attention index: 10 sizes expected (got ", n.size(), ")");
  auto get = [&](int i, at::ScalarType st) -> const void* {
    const std::optional<at::Tensor> o = t.get(i);
    return opt_ptr<const void>(o, kIndexTensors[i], st, dev);
  };
  bf_attn_index x{};
  x.n_q = n[0];
  x.n_kv = n[1];
  x.nnz = n[2];
  x.chunk = int32_t(n[3]);
  x.item = int32_t(n[4]);
  x.q_items = int32_t(n[5]);
  x.q_heavy = int32_t(n[6]);
  x.k_items = int32_t(n[7]);
  x.k_heavy = int32_t(n[8]);
  x.token_column = int32_t(n[9]);
  x.qptr = static_cast<const int64_t*>(get(0, at::kLong));
  x.kv = static_cast<const int32_t*>(get(1, at::kInt));
  x.kptr = static_cast<const int64_t*>(get(2, at::kLong));
  x.kq = static_cast<const int32_t*>(get(3, at::kInt));
  x.ks = static_cast<const int32_t*>(get(4, at::kInt));
  x.q_nitems = static_cast<const int32_t*>(get(5, at::kInt));
  x.q_item_off = static_cast<const int32_t*>(get(6, at::kInt));
  x.q_item_row = static_cast<const int32_t*>(get(7, at::kInt));
  x.q_heavy_rows = static_cast<const int32_t*>(get(8, at::kInt));
  x.k_nitems = static_cast<const int32_t*>(get(9, at::kInt));
  x.k_item_off = static_cast<const int32_t*>(get(10, at::kInt));
  x.k_item_row = static_cast<const int32_t*>(get(11, at::kInt));
  x.k_heavy_rows = static_cast<const int32_t*>(get(12, at::kInt));
  x.k_order = static_cast<const int32_t*>(get(13, at::kInt));
  x.k_spans = static_cast<const uint64_t*>(get(14, at::kLong));
  x.plan_counts = static_cast<const int32_t*>(get(15, at::kInt));
  return x;
}

int32_t dtype_code(const at::Tensor& q) {
  if (q.scalar_type() == at::kFloat) return BF_DTYPE_F32;
  if (q.scalar_type() == at::kHalf) return BF_DTYPE_F16;
  TORCH_CHECK_VALUE(q.scalar_type() == at::kBFloat16,
                    "attention supports float32, bfloat16 and float16 activations (got ", q.scalar_type(), ")");
  return BF_DTYPE_BF16;
}

void check_qkv(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const bf_attn_index& idx) {
  const at::Device dev = q.device();
  for (const auto* p : {&q, &k, &v}) {
    require(*p, p == &q ? "q" : p == &k ? "k" : "v", q.scalar_type(), dev);
    TORCH_CHECK_VALUE(p->dim() == 3, "q, k, v must be [rows, heads, head_dim]");
  }
  TORCH_CHECK_VALUE(k.sizes() == v.sizes() && q.size(1) == k.size(1) && q.size(2) == k.size(2), "q ", q.sizes(),
                    ", k ", k.sizes(), ", v ", v.sizes(), " disagree");
  TORCH_CHECK_VALUE(q.size(0) == idx.n_q && k.size(0) == idx.n_kv, "q rows ", q.size(0), " / kv rows ", k.size(0),
                    " do not match the index (", idx.n_q, ", ", idx.n_kv, ")");
}

const float* edge_tensor(const std::optional<at::Tensor>& t, const char* name, const bf_attn_index& idx, int64_t H,
                         const at::Device& dev) {
  const float* p = opt_ptr<const float>(t, name, at::kFloat, dev);
  if (p) TORCH_CHECK_VALUE(t->dim() == 2 && t->size(0) == idx.nnz && t->size(1) == H, name, " must be [", idx.nnz,
                           ", ", H, "] (got ", t->sizes(), ")");
  return p;
}

bf_attn_dropout make_dropout(double rate, int64_t seed, int64_t offset) {
  TORCH_CHECK_VALUE(rate >= 0.0 && rate <= 1.0, "dropout rate ", rate, " outside [0, 1]");
  return bf_attn_dropout{float(rate), uint64_t(seed), uint64_t(offset), nullptr};
}

// Entries the index's kv array holds room for (its capacity; nnz when sized exactly): the keep mask's
// rows, known without reading the entry count back.
int64_t kv_capacity(const c10::List<std::optional<at::Tensor>>& index) {
  const std::optional<at::Tensor> kv = index.get(1);
  return kv.has_value() ? kv->numel() : 0;
}

// Forward (bf_attn_fwd): (out [n_q, H, hn] in q's dtype, Z [n_q, H] float32, keep). With keep_mask and a
// dropout, keep is the mask of the bits drawn, uint8 [kv capacity, ceil(H / 8)], for the backward; else
// empty.
std::tuple<at::Tensor, at::Tensor, at::Tensor> sparse_attn_fwd(
    const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const c10::List<std::optional<at::Tensor>>& index,
    at::IntArrayRef sizes, const std::optional<at::Tensor>& bias, const std::optional<at::Tensor>& factor,
    double dropout_rate, int64_t dropout_seed, int64_t dropout_offset, double score_clamp, bool keep_mask) {
  TORCH_CHECK_VALUE(q.is_cuda(), "q must be a device tensor (got ", q.device(), ")");
  const c10::DeviceGuard guard(q.device());
  const at::Device dev = q.device();
  const bf_attn_index idx = make_index(index, sizes, dev);
  check_qkv(q, k, v, idx);
  const int64_t H = q.size(1), hn = q.size(2);
  const float* b = edge_tensor(bias, "bias", idx, H, dev);
  const float* f = edge_tensor(factor, "factor", idx, H, dev);
  bf_attn_dropout drop = make_dropout(dropout_rate, dropout_seed, dropout_offset);
  // the kernels read the mask by aligned dwords: its storage is rounded up to a multiple of 4 bytes
  const int64_t kb = (H + 7) / 8, rows = keep_mask && dropout_rate > 0.0 ? kv_capacity(index) : 0;
  at::Tensor keep =
      at::empty({(rows * kb + 3) / 4 * 4}, q.options().dtype(at::kByte)).narrow(0, 0, rows * kb).view({rows, kb});
  if (keep.numel()) drop.keep = keep.data_ptr<uint8_t>();
  at::Tensor out = at::empty_like(q);
  at::Tensor Z = at::empty({idx.n_q, H}, q.options().dtype(at::kFloat));
  const int64_t parts = bf_attn_partials_floats(&idx, int32_t(H), int32_t(hn));
  at::Tensor partials = at::empty({std::max<int64_t>(parts, 1)}, q.options().dtype(at::kFloat));
  check_rc(bf_attn_fwd(&idx, dtype_code(q), int32_t(H), int32_t(hn), float(score_clamp), q.data_ptr(), k.data_ptr(),
                       v.data_ptr(), b, f,
                       dropout_rate > 0.0 ? &drop : nullptr, out.data_ptr(), Z.data_ptr<float>(),
                       partials.data_ptr<float>(), stream_of(q)),
           "bf::sparse_attn_fwd");
  return {out, Z, keep};
}

// Backward (bf_attn_bwd): (dq, dk, dv, dbias); dbias is [nnz, H] float32 with need_dbias, else empty.
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> sparse_attn_bwd(
    const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const c10::List<std::optional<at::Tensor>>& index,
    at::IntArrayRef sizes, const at::Tensor& Z, const at::Tensor& dout, const std::optional<at::Tensor>& bias,
    const std::optional<at::Tensor>& factor, bool need_dbias, double dropout_rate, int64_t dropout_seed,
    int64_t dropout_offset, double score_clamp, const std::optional<at::Tensor>& keep) {
  TORCH_CHECK_VALUE(q.is_cuda(), "q must be a device tensor (got ", q.device(), ")");
  const c10::DeviceGuard guard(q.device());
  const at::Device dev = q.device();
  const bf_attn_index idx = make_index(index, sizes, dev);
  check_qkv(q, k, v, idx);
  const int64_t H = q.size(1), hn = q.size(2);
  require(dout, "dout", q.scalar_type(), dev);
  require(Z, "Z", at::kFloat, dev);
  TORCH_CHECK_VALUE(dout.sizes() == q.sizes() && Z.dim() == 2 && Z.size(0) == q.size(0) && Z.size(1) == H, "dout ",
                    dout.sizes(), " / Z ", Z.sizes(), " do not match q ", q.sizes());
  const float* b = edge_tensor(bias, "bias", idx, H, dev);
  const float* f = edge_tensor(factor, "factor", idx, H, dev);
  bf_attn_dropout drop = make_dropout(dropout_rate, dropout_seed, dropout_offset);
  if (keep.has_value() && keep->numel() && dropout_rate > 0.0) {
    // the forward's mask of this index, dropout and head count (a [kv capacity, ceil(H / 8)] byte tensor)
    drop.keep = opt_ptr<uint8_t>(keep, "keep", at::kByte, dev);
    TORCH_CHECK_VALUE(keep->dim() == 2 && keep->size(0) >= kv_capacity(index) && keep->size(1) == (H + 7) / 8 &&
                          keep->storage_offset() % 4 == 0 &&
                          int64_t(keep->storage().nbytes()) >= keep->storage_offset() + (keep->numel() + 3) / 4 * 4,
                      "keep must be the forward's [", kv_capacity(index), ", ", (H + 7) / 8, "] mask (got ",
                      keep->sizes(), ")");
  }
  at::Tensor dq = at::empty_like(q), dk = at::empty_like(k), dv = at::empty_like(v);
  at::Tensor dbias = need_dbias ? at::empty({idx.nnz, H}, q.options().dtype(at::kFloat))
                                : at::empty({0}, q.options().dtype(at::kFloat));
  at::Tensor rowstat = at::empty({idx.n_q, H, 2}, q.options().dtype(at::kFloat));
  const int64_t parts = bf_attn_partials_floats(&idx, int32_t(H), int32_t(hn));
  at::Tensor partials = at::empty({std::max<int64_t>(parts, 1)}, q.options().dtype(at::kFloat));
  check_rc(bf_attn_bwd(&idx, dtype_code(q), int32_t(H), int32_t(hn), float(score_clamp), q.data_ptr(), k.data_ptr(),
                       v.data_ptr(), b, f,
                       dropout_rate > 0.0 ? &drop : nullptr, Z.data_ptr<float>(), dout.data_ptr(), dq.data_ptr(),
                       dk.data_ptr(), dv.data_ptr(), need_dbias ? dbias.data_ptr<float>() : nullptr,
                       rowstat.data_ptr<float>(), partials.data_ptr<float>(), stream_of(q)),
           "bf::sparse_attn_bwd");
  return {dq, dk, dv, dbias};
}

// Typed-edge (Exphormer) attention: type_mod = E, float32 [2, H, hn]; the index's ids carry the types.
const float* type_mod_ptr(const at::Tensor& mod, int64_t H, int64_t hn, const at::Device& dev) {
  require(mod, "type_mod", at::kFloat, dev);
  TORCH_CHECK_VALUE(mod.numel() == 2 * H * hn && mod.size(0) == 2, "type_mod must be [2, ", H, ", ", hn, "] (got ",
                    mod.sizes(), ")");
  return mod.data_ptr<float>();
}

// Forward (bf_attn_fwd_typed): (out [n_q, H, hn] in q's dtype, Z [n_q, H] float32).
std::tuple<at::Tensor, at::Tensor> sparse_attn_fwd_typed(const at::Tensor& q, const at::Tensor& k,
                                                         const at::Tensor& v,
                                                         const c10::List<std::optional<at::Tensor>>& index,
                                                         at::IntArrayRef sizes, const at::Tensor& type_mod) {
  TORCH_CHECK_VALUE(q.is_cuda(), "q must be a device tensor (got ", q.device(), ")");
  const c10::DeviceGuard guard(q.device());
  const at::Device dev = q.device();
  const bf_attn_index idx = make_index(index, sizes, dev);
  check_qkv(q, k, v, idx);
  const int64_t H = q.size(1), hn = q.size(2);
  const float* mod = type_mod_ptr(type_mod, H, hn, dev);
  at::Tensor out = at::empty_like(q);
  at::Tensor Z = at::empty({idx.n_q, H}, q.options().dtype(at::kFloat));
  check_rc(bf_attn_fwd_typed(&idx, dtype_code(q), int32_t(H), int32_t(hn), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                             mod, out.data_ptr(), Z.data_ptr<float>(), stream_of(q)),
           "bf::sparse_attn_fwd_typed");
  return {out, Z};
}

// Backward (bf_attn_bwd_typed): (dq, dk, dv, dtype_mod [2, H, hn] float32).
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> sparse_attn_bwd_typed(
    const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const c10::List<std::optional<at::Tensor>>& index,
    at::IntArrayRef sizes, const at::Tensor& type_mod, const at::Tensor& Z, const at::Tensor& dout) {
  TORCH_CHECK_VALUE(q.is_cuda(), "q must be a device tensor (got ", q.device(), ")");
  const c10::DeviceGuard guard(q.device());
  const at::Device dev = q.device();
  const bf_attn_index idx = make_index(index, sizes, dev);
  check_qkv(q, k, v, idx);
  const int64_t H = q.size(1), hn = q.size(2);
  const float* mod = type_mod_ptr(type_mod, H, hn, dev);
  require(dout, "dout", q.scalar_type(), dev);
  require(Z, "Z", at::kFloat, dev);
  TORCH_CHECK_VALUE(dout.sizes() == q.sizes() && Z.dim() == 2 && Z.size(0) == q.size(0) && Z.size(1) == H, "dout ",
                    dout.sizes(), " / Z ", Z.sizes(), " do not match q ", q.sizes());
  at::Tensor dq = at::empty_like(q), dk = at::empty_like(k), dv = at::empty_like(v);
  at::Tensor dmod = at::empty({2, H, hn}, q.options().dtype(at::kFloat));
  at::Tensor rowstat = at::empty({idx.n_q, H, 2}, q.options().dtype(at::kFloat));
  const int64_t parts = bf_attn_typed_partials_floats(&idx, dtype_code(q), int32_t(H), int32_t(hn));
  at::Tensor partials = at::empty({std::max<int64_t>(parts, 1)}, q.options().dtype(at::kFloat));
  check_rc(bf_attn_bwd_typed(&idx, dtype_code(q), int32_t(H), int32_t(hn), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                             mod, Z.data_ptr<float>(), dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                             dmod.data_ptr<float>(), rowstat.data_ptr<float>(), partials.data_ptr<float>(),
                             stream_of(q)),
           "bf::sparse_attn_bwd_typed");
  return {dq, dk, dv, dmod};
}

// ---------------------------------------------------------------- edge construction
// Walks (bf_random_walk): int64 [n_q * P, L + 1], walk q*P + p starting at query q_lo + q.
at::Tensor rw_walk(const at::Tensor& rowptr, const at::Tensor& col, int64_t q_lo, int64_t n_q, int64_t walks_per_node,
                   int64_t walk_length, int64_t philox_seed, int64_t philox_offset, const std::optional<at::Tensor>& u) {
  const c10::DeviceGuard guard(rowptr.device());
  const at::Device dev = rowptr.device();
  require(rowptr, "rowptr", at::kLong, dev);
  require(col, "col", at::kInt, dev);
  const float* up = opt_ptr<const float>(u, "u", at::kFloat, dev);
  if (up) TORCH_CHECK_VALUE(u->numel() == n_q * walks_per_node * walk_length, "u must be [", n_q * walks_per_node,
                            ", ", walk_length, "]");
  TORCH_CHECK_VALUE(n_q >= 0 && walks_per_node >= 1 && walk_length >= 0, "rw_walk: bad sizes");
  at::Tensor walks = at::empty({n_q * walks_per_node, walk_length + 1}, rowptr.options());
  check_rc(bf_random_walk(rowptr.data_ptr<int64_t>(), col.data_ptr<int32_t>(), rowptr.numel() - 1, q_lo, n_q,
                          int32_t(walks_per_node), int32_t(walk_length), up, uint64_t(philox_seed),
                          uint64_t(philox_offset), walks.data_ptr<int64_t>(), stream_of(rowptr)),
           "bf::rw_walk");
  return walks;
}

// Budgeted table (bf_build_edge_table): (table int32 [n_q, k_real + k_rw], row_len int32 [n_q]).
std::tuple<at::Tensor, at::Tensor> build_edge_table(
    const at::Tensor& rowptr, const at::Tensor& col, const std::optional<at::Tensor>& walk_rec,
    const at::Tensor& in_ptr, const at::Tensor& in_src, int64_t q_lo, int64_t n_q, int64_t walks_per_node,
    int64_t walk_length, int64_t k_real, int64_t k_rw, int64_t edge_seed, const std::optional<at::Tensor>& u,
    int64_t philox_seed, int64_t philox_offset, const std::optional<at::Tensor>& hubs, int64_t hub_threshold,
    const std::optional<at::Tensor>& heavy, int64_t light_max) {
  const c10::DeviceGuard guard(rowptr.device());
  const at::Device dev = rowptr.device();
  require(rowptr, "rowptr", at::kLong, dev);
  require(col, "col", at::kInt, dev);
  require(in_ptr, "in_ptr", at::kLong, dev);
  require(in_src, "in_src", at::kInt, dev);
  const void* rec = opt_ptr<const void>(walk_rec, "walk_rec", at::kInt, dev);
  if (rec) TORCH_CHECK_VALUE(walk_rec->numel() == 4 * col.numel(), "walk_rec must be [", col.numel(), ", 4]");
  const float* up = opt_ptr<const float>(u, "u", at::kFloat, dev);
  if (up) TORCH_CHECK_VALUE(u->numel() == n_q * walks_per_node * walk_length, "u must be [", n_q * walks_per_node,
                            ", ", walk_length, "]");
  const int32_t* hp = opt_ptr<const int32_t>(hubs, "hubs", at::kInt, dev);
  const int32_t* vp = opt_ptr<const int32_t>(heavy, "heavy", at::kInt, dev);
  const int64_t n_hubs = hp ? hubs->numel() : 0, n_heavy = vp ? heavy->numel() : 0;
  // with light_max >= 0 the light kernel leaves rows above it to the heavy list: it must be given (it may be empty)
  TORCH_CHECK_VALUE(light_max < 0 || (heavy.has_value() && heavy->defined()), "light_max >= 0 needs the heavy-query list");
  const int64_t width = std::max<int64_t>(k_real, 0) + std::max<int64_t>(k_rw, 0);
  at::Tensor table = at::empty({n_q, width}, in_src.options());
  at::Tensor row_len = at::empty({n_q}, in_src.options());
  size_t ws_bytes = 0;
  check_rc(bf_build_edge_table_workspace_size(n_q, int32_t(std::max<int64_t>(k_rw, 0)), n_hubs,
                                              int32_t(std::max<int64_t>(k_real, 0)), &ws_bytes),
           "bf::build_edge_table");
  at::Tensor ws = scratch_bytes(ws_bytes, dev);
  check_rc(bf_build_edge_table(rowptr.data_ptr<int64_t>(), col.data_ptr<int32_t>(), rec, in_ptr.data_ptr<int64_t>(),
                               in_src.data_ptr<int32_t>(), rowptr.numel() - 1, col.numel(), q_lo, n_q,
                               int32_t(walks_per_node), int32_t(walk_length), int32_t(k_real), int32_t(k_rw),
                               edge_seed, up, uint64_t(philox_seed), uint64_t(philox_offset), hp, n_hubs,
                               hub_threshold, vp, n_heavy, light_max, table.data_ptr<int32_t>(),
                               row_len.data_ptr<int32_t>(), ws.data_ptr(), size_t(ws.numel()), stream_of(rowptr)),
           "bf::build_edge_table");
  return {table, row_len};
}

// Query-major table -> attention CSR (bf_table_csr_ptr + bf_table_to_csr): (qptr int64 [n_q + 1], kv int32 [nnz]).
// token_row as in the C ABI (< 0: no token row); reads nnz to the host once. With id_limit >= 0 the table is
// validated on the device first (bf_check_table: row lengths in [0, width], ids in [0, id_limit)).
std::tuple<at::Tensor, at::Tensor> table_to_csr(const at::Tensor& table, const at::Tensor& row_len, bool global_token,
                                                int64_t token_row, int64_t id_limit) {
  const c10::DeviceGuard guard(table.device());
  const at::Device dev = table.device();
  require(table, "table", at::kInt, dev);
  require(row_len, "row_len", at::kInt, dev);
  TORCH_CHECK_VALUE(table.dim() == 2 && row_len.dim() == 1 && row_len.size(0) == table.size(0),
                    "table must be [n, width] and row_len [n]");
  const int64_t n_rows = table.size(0);
  if (id_limit >= 0) {
    at::Tensor bad = at::empty({2}, table.options().dtype(at::kLong));
    check_rc(bf_check_table(table.data_ptr<int32_t>(), row_len.data_ptr<int32_t>(), n_rows, int32_t(table.size(1)),
                            id_limit, nullptr, bad.data_ptr(), 16, stream_of(table)),
             "bf::table_to_csr");
  }
  const int64_t lead = (global_token && token_row >= 0) ? 1 : 0;
  const int64_t n_q = n_rows + lead;
  size_t ws_bytes = 0;
  check_rc(bf_scan_workspace_size(n_q, &ws_bytes), "bf::table_to_csr");
  at::Tensor ws = scratch_bytes(ws_bytes, dev);
  at::Tensor qptr = at::empty({n_q + 1}, table.options().dtype(at::kLong));
  int64_t nnz = 0;
  void* st = stream_of(table);
  check_rc(bf_table_csr_ptr(row_len.data_ptr<int32_t>(), n_rows, global_token ? 1 : 0, token_row,
                            qptr.data_ptr<int64_t>(), &nnz, ws.data_ptr(), size_t(ws.numel()), st),
           "bf::table_to_csr");
  at::Tensor kv = at::empty({nnz}, table.options());
  check_rc(bf_table_to_csr(table.data_ptr<int32_t>(), row_len.data_ptr<int32_t>(), n_rows, int32_t(table.size(1)),
                           global_token ? 1 : 0, token_row, qptr.data_ptr<int64_t>(), kv.data_ptr<int32_t>(), nullptr,
                           0, 0, st),
           "bf::table_to_csr");
  return {qptr, kv};
}

// Key-major view of an attention CSR (bf_reverse_index): (kptr int64 [n_kv + 1], kq int32 [nnz], ks int32 [nnz]:
// each entry's query and its slot in the query's row), entries of a key in CSR order.
std::tuple<at::Tensor, at::Tensor, at::Tensor> transpose_table(const at::Tensor& qptr, const at::Tensor& kv,
                                                               int64_t n_kv) {
  const c10::DeviceGuard guard(qptr.device());
  const at::Device dev = qptr.device();
  require(qptr, "qptr", at::kLong, dev);
  require(kv, "kv", at::kInt, dev);
  const int64_t nnz = kv.numel();
  size_t ws_bytes = 0;
  check_rc(bf_reverse_index_workspace_size(nnz, n_kv, &ws_bytes), "bf::transpose_table");
  at::Tensor ws = scratch_bytes(ws_bytes, dev);
  at::Tensor kptr = at::empty({n_kv + 1}, qptr.options());
  at::Tensor kq = at::empty({nnz}, kv.options()), ks = at::empty({nnz}, kv.options());
  check_rc(bf_reverse_index(qptr.data_ptr<int64_t>(), kv.data_ptr<int32_t>(), qptr.numel() - 1, n_kv, nnz,
                            kptr.data_ptr<int64_t>(), kq.data_ptr<int32_t>(), ks.data_ptr<int32_t>(), ws.data_ptr(),
                            size_t(ws.numel()), stream_of(qptr)),
           "bf::transpose_table");
  return {kptr, kq, ks};
}

}  // namespace

TORCH_LIBRARY(bf, m) {
  m.def("sparse_attn_fwd(Tensor q, Tensor k, Tensor v, Tensor?[] index, int[] sizes, Tensor? bias=None, "
        "Tensor? factor=None, float dropout_rate=0.0, int dropout_seed=0, int dropout_offset=0, "
        "float score_clamp=5.0, bool keep_mask=False) -> (Tensor, Tensor, Tensor)");
  m.def("sparse_attn_bwd(Tensor q, Tensor k, Tensor v, Tensor?[] index, int[] sizes, Tensor Z, Tensor dout, "
        "Tensor? bias=None, Tensor? factor=None, bool need_dbias=False, float dropout_rate=0.0, int dropout_seed=0, "
        "int dropout_offset=0, float score_clamp=5.0, Tensor? keep=None) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("sparse_attn_fwd_typed(Tensor q, Tensor k, Tensor v, Tensor?[] index, int[] sizes, Tensor type_mod) "
        "-> (Tensor, Tensor)");
  m.def("sparse_attn_bwd_typed(Tensor q, Tensor k, Tensor v, Tensor?[] index, int[] sizes, Tensor type_mod, "
        "Tensor Z, Tensor dout) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("rw_walk(Tensor rowptr, Tensor col, int q_lo, int n_q, int walks_per_node, int walk_length, "
        "int philox_seed=0, int philox_offset=0, Tensor? u=None) -> Tensor");
  m.def("build_edge_table(Tensor rowptr, Tensor col, Tensor? walk_rec, Tensor in_ptr, Tensor in_src, int q_lo, "
        "int n_q, int walks_per_node, int walk_length, int k_real, int k_rw, int edge_seed, Tensor? u=None, "
        "int philox_seed=0, int philox_offset=0, Tensor? hubs=None, int hub_threshold=1024, Tensor? heavy=None, "
        "int light_max=-1) -> (Tensor, Tensor)");
  m.def("table_to_csr(Tensor table, Tensor row_len, bool global_token=False, int token_row=-1, int id_limit=-1) "
        "-> (Tensor, Tensor)");
  m.def("transpose_table(Tensor qptr, Tensor kv, int n_kv) -> (Tensor, Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(bf, CUDA, m) {
  m.impl("sparse_attn_fwd", &sparse_attn_fwd);
  m.impl("sparse_attn_bwd", &sparse_attn_bwd);
  m.impl("sparse_attn_fwd_typed", &sparse_attn_fwd_typed);
  m.impl("sparse_attn_bwd_typed", &sparse_attn_bwd_typed);
  m.impl("rw_walk", &rw_walk);
  m.impl("build_edge_table", &build_edge_table);
  m.impl("table_to_csr", &table_to_csr);
  m.impl("transpose_table", &transpose_table);
}
