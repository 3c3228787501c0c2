/*
 * budgetformer_hip.h — C ABI of the MI355X (gfx950) BudgetFormer hot path.
 *
 * Plain pointers and sizes only. Every pointer argument named like a tensor is
 * device memory (HBM) unless stated otherwise; `stream` is a hipStream_t (NULL
 * = the legacy default stream). All work is enqueued asynchronously on that
 * stream. Every entry point returns BF_OK (0) or an error code; bf_last_error()
 * returns the message of the last failure on the calling thread.
 *
 * Scratch memory is never allocated inside the library: entry points that need
 * it take a workspace pointer and have a *_workspace_size query, so callers
 * can draw it from their own allocator (e.g. PyTorch's caching allocator, which
 * turns a failed allocation into torch.cuda.OutOfMemoryError as the reference's
 * fallback handlers expect, gt_sp/utils.py:1200-1230).
 *
 * Reference interfaces each entry point replaces are cited as file:line
 * relative to the cz-up/BudgetFormer source tree.
 */
#ifndef BUDGETFORMER_HIP_H
#define BUDGETFORMER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  BF_OK = 0,
  BF_ERR_INVALID = 1,      /* bad argument (shape, range, alignment)      */
  BF_ERR_UNSUPPORTED = 2,  /* valid but not implemented (e.g. head dim)    */
  BF_ERR_HIP = 3           /* a HIP runtime call or kernel launch failed   */
};

/* Activation dtypes of the attention entry points: float32, bfloat16 and IEEE
 * float16 (the reference's bf16 / fp16 autocast, utils/parser_node_level.py:
 * 266-272; utils/fullgraph_sp_support.py:350-360, 440). Every dtype
 * accumulates in float32.                                                    */
enum { BF_DTYPE_F32 = 0, BF_DTYPE_BF16 = 1, BF_DTYPE_F16 = 2 };

/* ABI version (major*10000 + minor*100 + patch), returned by bf_version(). A
 * binding checks it for equality: any change to an entry point's arguments,
 * to a struct's fields or to their meaning bumps it. History:
 *   100  first ABI;
 *   200  bf_attn_fwd / bf_attn_bwd take score_clamp and a dropout; bf_attn_bwd
 *        no longer takes `out`; bf_reverse_slots replaces bf_reverse_entries;
 *        bf_attn_index's fifth pointer (ks) holds each reverse entry's slot in
 *        its query's row instead of its CSR position;
 *   300  BF_DTYPE_F16 (float16 activations); the in-kernel dropout is keyed by
 *        (query row, slot) instead of the CSR position (a new mask for the same
 *        seed and offset); typed-edge attention (bf_attn_fwd_typed,
 *        bf_attn_bwd_typed, bf_attn_typed_partials_floats);
 *   301  bf_gather_probe (calibration); bf_rw_select, bf_rw_select_rows,
 *        bf_real_select_merge, bf_real_select_rows and bf_assemble_rows take
 *        any budget and walk shape (they used to reject rows above 768 ids
 *        and more than 8191 walk candidates per query);
 *   302  bf_row_stream_probe (calibration);
 *   303  bf_attn_dropout gains `keep` (the forward stores its keep bits, the
 *        backward's query-major pass reads them back).                      */
#define BF_ABI_VERSION 303
int bf_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char* bf_last_error(void);

/* Optional per-kernel timing (no reference counterpart; replaces the CUDA-event
 * stage timers of gt_sp/comm_profiler.py:29-53 at kernel granularity). While
 * enabled, every kernel the library launches is bracketed by a HIP event pair
 * on its stream; bf_prof_collect waits for them and accumulates elapsed ms per
 * kernel name, read back with bf_prof_count / bf_prof_get.                  */
int bf_prof_enable(int32_t on);
int bf_prof_reset(void);
int bf_prof_collect(void);
int32_t bf_prof_count(void);
int bf_prof_get(int32_t i, const char** name, double* total_ms, int64_t* launches);

/* ======================================================================
 * Edge construction
 * ====================================================================== */

/* Uniform first-order random walks, one lane per walk.
 * Replaces _run_random_walk (gt_sp/utils.py:1387-1473), i.e. the
 * torch_cluster.random_walk / dgl.sampling.random_walk call, for the starts
 * arange(N).repeat_interleave(P) of gt_sp/utils.py:1198-1199 restricted to the
 * query range [q_lo, q_lo+n_q).
 *   rowptr [num_nodes+1] int64, col [E] int32: coalesced CSR (source rows).
 *   u: NULL, or float32 [n_q*P, L] injected uniforms (row (q-q_lo)*P+p);
 *      when NULL, u comes from Philox4x32-10 keyed by philox_seed with
 *      counter (global walk id q*P+p, philox_offset + l/4).
 *   walks: int64 [n_q*P, L+1]; walks[:,0] = start; a dead end stays.
 * Step rule: idx = (int64)(u * (float)deg) in fp32, clamped to deg-1.      */
int bf_random_walk(const int64_t* rowptr, const int32_t* col, int64_t num_nodes,
                   int64_t q_lo, int64_t n_q, int32_t walks_per_node, int32_t walk_length,
                   const float* u, uint64_t philox_seed, uint64_t philox_offset,
                   int64_t* walks, void* stream);

/* Walks from arbitrary start nodes: the general form of the _run_random_walk
 * seam (gt_sp/utils.py:1387, argument `starts`). Walk i starts at starts[i]
 * (int64 [n_walks]) and, without u, draws Philox walk id walk_id_base + i, so
 * starts = arange(N).repeat_interleave(P) with base 0 reproduces bf_random_walk. */
int bf_random_walk_starts(const int64_t* rowptr, const int32_t* col, int64_t num_nodes,
                          const int64_t* starts, int64_t n_walks, int32_t walk_length,
                          const float* u, uint64_t philox_seed, uint64_t philox_offset,
                          uint64_t walk_id_base, int64_t* walks, void* stream);

/* The RW hop pool of a walk tensor, in the reference's order.
 * Replaces the hop loop of compute_hop_buckets_random_walk (gt_sp/utils.py:
 * 1232-1248) for one bucket: for d = min_hop..L (d-major), then walk order,
 * emit (kv = walks[w,d], q = walks[w,0]) iff kv >= 0 and (d == 1 or
 * kv != walks[w,d-1]). pool_kv / pool_q int64 need capacity n_walks*(L-min_hop+1);
 * the pool size is returned in *count_host (the call synchronises the stream).
 * Workspace: bf_hop_pool_workspace_size.                                       */
int bf_hop_pool_workspace_size(int64_t n_walks, int32_t walk_length, int32_t min_hop, size_t* bytes);
int bf_hop_pool(const int64_t* walks, int64_t n_walks, int32_t walk_length, int32_t min_hop,
                int64_t* pool_kv, int64_t* pool_q, int64_t* count_host,
                void* workspace, size_t workspace_bytes, void* stream);

/* The fanout k-hop pool, the "dgl_neighbor" alternative to the walk pool
 * (compute_khop_pool_dgl_neighbor, gt_sp/utils.py:1281-1384), run hop by hop by
 * the host. The frontier starts as (origin u, node u) for every node; hop d
 * replaces each entry (o, c) by (o, s) for each s in node c's hop-d sample and,
 * from min_hop on, emits the pool pair (kv = s, q = o) when s != o.
 *
 * bf_fanout_sample: node u's hop sample of out-neighbours into sel[u*fanout ..]
 * (count in cnt[u]): all of them, in CSR order, when out-degree <= fanout; else
 * `fanout` distinct ones by Floyd's algorithm over Philox words (counter = (u,
 * offset + hop * 2^32 + i / 4), key = seed, word i % 4, t = hi32(word * (j+1))
 * for j = deg - fanout + i), in ascending index order. DGL's sampler RNG is not
 * reproduced (sample_neighbors, gt_sp/utils.py:1330-1333); a fanout of -1 (all
 * neighbours) needs no sample: pass the CSR to the frontier calls instead. */
#define BF_MAX_FANOUT 64
int bf_fanout_sample(const int64_t* rowptr, const int32_t* col, int64_t num_nodes, int32_t fanout, int32_t hop,
                     uint64_t seed, uint64_t offset, int32_t* cnt, int32_t* sel, void* stream);
/* offsets [n+1] int64 of the next frontier: the exclusive scan of each entry's
 * sample size, from a sample's cnt (ptr NULL) or a CSR's ptr (cnt NULL); the
 * next frontier's size is offsets[n]. Workspace: bf_frontier_offsets_workspace_size. */
int bf_frontier_offsets_workspace_size(int64_t n, size_t* bytes);
int bf_frontier_offsets(const int32_t* cur, int64_t n, const int64_t* ptr, const int32_t* cnt, int64_t* offsets,
                        void* workspace, size_t workspace_bytes, void* stream);
/* The next frontier: entry i writes (origin[i], s) at offsets[i] for each s of
 * its node c's sample, read from ids[c*stride ..] (a sample table, stride =
 * fanout) or ids[ptr[c] ..] (a CSR, stride 0). */
int bf_frontier_expand(const int32_t* origin, const int32_t* cur, int64_t n, const int64_t* offsets,
                       const int64_t* ptr, const int32_t* ids, int32_t stride, int32_t* new_origin, int32_t* new_cur,
                       void* stream);
/* The frontier's pool pairs in order: kv[k] = cur[i], q[k] = origin[i] for
 * every i with cur[i] != origin[i] (capacity n each); count: device int64[1].
 * Workspace: bf_frontier_emit_workspace_size. */
int bf_frontier_emit_workspace_size(int64_t n, size_t* bytes);
int bf_frontier_emit(const int32_t* origin, const int32_t* cur, int64_t n, int64_t* kv, int64_t* q, int64_t* count,
                     void* workspace, size_t workspace_bytes, void* stream);

/* The Philox uniforms bf_random_walk draws when u == NULL, written as the
 * float32 [n_q*P, L] tensor that reproduces them through the u argument. */
int bf_walk_uniforms(int64_t q_lo, int64_t n_q, int32_t walks_per_node, int32_t walk_length,
                     uint64_t philox_seed, uint64_t philox_offset, float* u, void* stream);

/* Walk records of a CSR (no reference counterpart: a layout of the CSR the
 * reference caches, gt_sp/utils.py:29-33, 1387-1473): records int32
 * [num_edges, 4], 16-byte aligned; record e = {col[e], deg(col[e]),
 * rowptr[col[e]] low word, high word}. A walk holding its node's (row start,
 * degree) reaches the next node's with one 16-byte read. Depends on the
 * topology only: built once per graph. num_edges < 2^31.                    */
int bf_walk_records(const int64_t* rowptr, const int32_t* col, int64_t num_nodes, int64_t num_edges,
                    void* records, void* stream);

/* Per-query top-k of the random-walk pool, fused with the walk.
 * Replaces build_head_hop_edges (gt_sp/utils.py:1251-1278) +
 * compute_hop_buckets_random_walk's hop loop (gt_sp/utils.py:1232-1248) +
 * _sample_edges_per_query_random(pool, k_rw, edge_seed+37)
 * (utils/fullgraph_sp_support.py:1494-1517, 1195-1228): for query q the pool
 * holds (walks[w,d], q) for its own walks w, d=1..L, kept iff d==1 or the walk
 * moved at step d; the k_rw smallest keys key(kv, q, seed) are kept counting
 * multiplicity. Output sel_kv int32 [n_q, k_rw] (key order, -1 padded),
 * sel_cnt int32 [n_q]. Any P*L below 2^32: up to 8191 candidates per query
 * are sorted in LDS, more are selected by a streaming top-k (a workgroup per
 * query re-runs its walks per batch of winners; nothing is staged), with the
 * same result. walk_rec: NULL, or bf_walk_records' records of this
 * rowptr/col (16-byte aligned): each step then reads one record instead of
 * the rowptr pair and col; the walks are the same.                           */
int bf_rw_select(const int64_t* rowptr, const int32_t* col, const void* walk_rec, int64_t num_nodes,
                 int64_t q_lo, int64_t n_q, int32_t walks_per_node, int32_t walk_length,
                 int32_t k_rw, int64_t key_seed, const float* u, uint64_t philox_seed,
                 uint64_t philox_offset, int32_t* sel_kv, int32_t* sel_cnt, void* stream);

/* bf_rw_select for an explicit query list (the Adaptive-Budget probe's
 * dst-filtered build): row i serves query qids[i] (int32 [n_q], ids outside
 * [0, num_nodes) give empty rows), its walks keep their global ids q*P+p, so
 * each row equals the full build's row for that query. With sub_ptr/sub_src
 * (an in-neighbour CSR, rows ascending) a candidate kv that is a graph edge
 * kv -> q is removed before ranking: the probe pools' RW-minus-real
 * subtraction. Replaces _build_probe_edge_pools' RW half
 * (utils/fullgraph_sp_support.py:1743-1821: filter by dst :1520-1533,
 * _subtract_edge_index :1536-1551) followed by the RW sampling of
 * _assemble_edges_from_pools (:1824-1879, via :1262-1309). u, when given, is
 * float32 [n_q*P, L] in row order. walk_rec as in bf_rw_select.            */
int bf_rw_select_rows(const int64_t* rowptr, const int32_t* col, const void* walk_rec, int64_t num_nodes,
                      const int32_t* qids, int64_t n_q, int32_t walks_per_node,
                      int32_t walk_length, int32_t k_rw, int64_t key_seed, const float* u,
                      uint64_t philox_seed, uint64_t philox_offset, const int64_t* sub_ptr,
                      const int32_t* sub_src, int32_t* sel_kv, int32_t* sel_cnt, void* stream);

/* Per-query top-k of the real (graph) edges merged with an RW selection into
 * the query-major table. Replaces _sample_edges_per_query_random(edge_index,
 * k_real, edge_seed+17) (utils/fullgraph_sp_support.py:1312-1491, 1195-1228)
 * followed by _merge_edge_index_list (gt_sp/utils.py:877-887) as used by
 * _build_merged_edges (utils/fullgraph_sp_support.py:2943-3026).
 *   in_ptr [num_nodes+1] int64, in_src int32: in-neighbour CSR (row q lists the
 *     sources of edges into q; equals the CSR for a symmetric graph).
 *   k_real <= 0 drops the real part; rw_kv/rw_cnt NULL (or k_rw 0) drops the
 *   RW part. dedup != 0 merges as a set (the reference coalesces when both
 *   parts are globally non-empty); dedup == 0 keeps duplicates.
 *   hubs int32 [n_hubs] (ascending query ids whose in-degree exceeds
 *     hub_threshold, or n_hubs = 0): their top-k is computed by one workgroup
 *     each into hub_sel int32 [n_hubs, k_real] / hub_cnt int32 [n_hubs]
 *     (caller-provided scratch) instead of by a 16-lane group.
 *   light_max >= 0 (with k_real <= 16, k_rw <= 16) splits the work: queries of
 *     in-degree <= light_max are served one per thread; heavy int32 [n_heavy]
 *     must list every query of [q_lo, q_lo+n_q) with in-degree > light_max,
 *     ascending (hubs included), and those take the 16-lane group path.
 *     light_max < 0: no split (heavy ignored). The table is the same either way.
 *   table int32 [n_q, width] rows ascending, -1 padded; row_len int32 [n_q].
 *   Any budgets, width >= k_real + k_rw: a merged row of up to 768 ids is
 *   ranked in LDS, a wider one by a workgroup in its own table slots (the
 *   hub arrays are then not used).                                          */
int bf_real_select_merge(const int64_t* in_ptr, const int32_t* in_src, int64_t num_nodes,
                         int64_t q_lo, int64_t n_q, int32_t k_real, int64_t key_seed,
                         const int32_t* rw_kv, const int32_t* rw_cnt, int32_t k_rw,
                         int32_t dedup, int32_t* table, int32_t width, int32_t* row_len,
                         const int32_t* hubs, int64_t n_hubs, int64_t hub_threshold,
                         int32_t* hub_sel, int32_t* hub_cnt, const int32_t* heavy,
                         int64_t n_heavy, int64_t light_max, void* stream);

/* Real-edge top-k_real for an explicit query list, in key order (so every
 * smaller budget is a prefix: the probe's nested candidates). Replaces the
 * probe's real pool (_filter_edge_index_by_dst / _filter_by_dst_csr,
 * utils/fullgraph_sp_support.py:1520-1533, 1766-1777) sampled by
 * _sample_edges_per_query_random(real_pool, k_real, edge_seed+17) in
 * _assemble_edges_from_pools (:1824-1879, via :1262-1309).
 *   qids int32 [n_q]; sel_kv int32 [n_q, k_real] (-1 padded), sel_cnt [n_q].
 *   hubs: ascending query ids (a subset of qids) whose in-degree exceeds
 *   hub_threshold, with hub_sel [n_hubs, k_real] / hub_cnt [n_hubs] scratch. */
int bf_real_select_rows(const int64_t* in_ptr, const int32_t* in_src, int64_t num_nodes,
                        const int32_t* qids, int64_t n_q, int32_t k_real, int64_t key_seed,
                        const int32_t* hubs, int64_t n_hubs, int64_t hub_threshold,
                        int32_t* hub_sel, int32_t* hub_cnt, int32_t* sel_kv, int32_t* sel_cnt,
                        void* stream);

/* One budget candidate from key-ordered selections: per row the first b_real
 * entries of real_kv and the first b_rw of rw_kv, merged as
 * _assemble_edges_from_pools merges them (utils/fullgraph_sp_support.py:
 * 1824-1879 -> gt_sp/utils.py:877-887): dedup != 0 gives the set union
 * ascending (both parts globally non-empty), else the multiset ascending.
 * NULL real_kv / rw_kv (or a zero budget) drops that part. Any budgets; a
 * row of more than 768 ids is finished by a workgroup in its table slots.
 *   table int32 [n_rows, width] (-1 padded), row_len int32 [n_rows], not
 *   overlapping the selections.                                            */
int bf_assemble_rows(const int32_t* real_kv, const int32_t* real_cnt, int32_t real_stride,
                     int32_t b_real, const int32_t* rw_kv, const int32_t* rw_cnt,
                     int32_t rw_stride, int32_t b_rw, int32_t dedup, int64_t n_rows,
                     int32_t* table, int32_t width, int32_t* row_len, void* stream);

/* One layer of the probe's reception-cone expansion
 * (_expand_probe_idx_for_reception, utils/fullgraph_sp_support.py:2261-2309):
 * reached[s] = 1 for every edge s -> v of the in-neighbour CSR with
 * frontier[v] != 0. frontier, reached: uint8 [num_nodes]; reached is not
 * cleared first.                                                           */
int bf_mark_in_neighbors(const int64_t* in_ptr, const int32_t* in_src, int64_t num_nodes,
                         const uint8_t* frontier, uint8_t* reached, void* stream);

/* Whole budgeted build: bf_rw_select then bf_real_select_merge with
 * key seeds edge_seed+37 / edge_seed+17 (utils/fullgraph_sp_support.py:970-972,
 * 1413, 1514) and the reference's global merge rule (dedup iff both parts are
 * non-empty). Replaces _build_merged_edges (utils/fullgraph_sp_support.py:
 * 2943-3026) without the Graphormer token. width = k_real + k_rw. hubs /
 * n_hubs / hub_threshold and heavy / n_heavy / light_max as in
 * bf_real_select_merge (n_hubs may be 0; light_max < 0 disables the split).
 * walk_rec: NULL or bf_walk_records' records, as in bf_rw_select.
 * Workspace: bf_build_edge_table_workspace_size.                            */
int bf_build_edge_table_workspace_size(int64_t n_q, int32_t k_rw, int64_t n_hubs, int32_t k_real,
                                       size_t* bytes);
int bf_build_edge_table(const int64_t* rowptr, const int32_t* col, const void* walk_rec,
                        const int64_t* in_ptr, const int32_t* in_src, int64_t num_nodes,
                        int64_t num_edges, int64_t q_lo, int64_t n_q,
                        int32_t walks_per_node, int32_t walk_length,
                        int32_t k_real, int32_t k_rw, int64_t edge_seed,
                        const float* u, uint64_t philox_seed, uint64_t philox_offset,
                        const int32_t* hubs, int64_t n_hubs, int64_t hub_threshold,
                        const int32_t* heavy, int64_t n_heavy, int64_t light_max,
                        int32_t* table, int32_t* row_len,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Synthetic symmetric power-law (Chung-Lu) graph generated on the device (no
 * reference counterpart: the reference loads datasets from disk; the benchmark
 * shapes here are synthetic). Expected degree of node i is proportional to
 * (i + i0)^(-1/(exponent-1)), scaled to sum 2*pairs and capped at max_degree
 * (<= 0: no cap); `pairs` distinct unordered pairs are drawn (Philox keyed by
 * seed), then symmetrised. rowptr int64 [num_nodes+1], col int32 [2*pairs];
 * *num_edges_host = 2*pairs. Synchronises the stream. Workspace:
 * bf_chung_lu_workspace_size.                                                */
int bf_chung_lu_workspace_size(int64_t num_nodes, int64_t pairs, size_t* bytes);
int bf_chung_lu(int64_t num_nodes, int64_t pairs, double exponent, double i0, double max_degree,
                uint64_t seed, int64_t* rowptr, int32_t* col, int64_t* num_edges_host,
                void* workspace, size_t workspace_bytes, void* stream);

/* ======================================================================
 * Edge index formats
 * ====================================================================== */

/* Query-major table -> attention CSR (qptr int64 [n_q+1], kv int32 [nnz]).
 * global_token != 0 applies the Graphormer virtual node (fix_edge_index,
 * gt_sp/utils.py:113-130): ids shift by one and every table row also attends
 * to kv 0, first in its row. token_row says where the token's own row is:
 *   token_row >= 0: attention row 0 is the token row, attending to kv
 *     1..token_row (the graph's N nodes), and table row r is query r+1, so
 *     n_q = n_rows + 1 (the full query set: token_row = n_rows; a query shard
 *     that starts at node 0: token_row = N);
 *   token_row < 0: no token row — a query shard [q_lo, q_lo + n_rows) with
 *     q_lo > 0, whose table row r is attention row r; n_q = n_rows.
 * With global_token == 0 token_row is ignored and n_q = n_rows.
 * bf_table_csr_ptr writes qptr (a prefix sum of the row lengths) and returns
 * nnz = qptr[n_q] on the host (it synchronises the stream, so the caller can
 * size kv; with nnz_host NULL it only enqueues the scan and the caller reads
 * qptr[n_q] when it needs it, or sizes kv and rkey for every row full, of
 * which only the first nnz / key count are written); bf_table_to_csr then fills kv, and, when rkey is not NULL,
 * rkey uint64 = (id << (q_bits + slot_bits) | query << slot_bits | slot) for
 * each of the table's own entries in CSR order (slot = position in the query's
 * row), the sort keys bf_reverse_index_packed takes: [nnz] without the token,
 * [sum of row_len] with it (the token's entries, kv 0 of every row and the
 * token row, have a fixed place in the reverse index and get no key). Needs
 * q_bits >= bits of n_q, slot_bits >= bits of width and q_bits + slot_bits
 * <= 33 (BF_ERR_INVALID otherwise). Workspace: bf_scan_workspace_size(n_q). */
int bf_scan_workspace_size(int64_t n, size_t* bytes);

/* Device-side validation of an externally supplied table before its index
 * is built (the edge builder's own tables are valid by construction): counts
 * the rows whose row_len lies outside [0, width] and the ids of each row's
 * first row_len slots outside [0, id_limit) (id_limit = n_kv, or n_kv - 1
 * with global_token, whose ids shift by one), writes the two counts to
 * bad_host (may be NULL) and returns BF_ERR_INVALID when either is nonzero.
 * Synchronises the stream. Workspace: 16 bytes of device memory. The
 * reference builds its edge lists itself; the nearest check is
 * fix_edge_index's id arithmetic (gt_sp/utils.py:113-130).                 */
int bf_check_table(const int32_t* table, const int32_t* row_len, int64_t n_rows, int32_t width,
                   int64_t id_limit, int64_t* bad_host, void* workspace, size_t workspace_bytes, void* stream);
int bf_table_csr_ptr(const int32_t* row_len, int64_t n_rows, int32_t global_token, int64_t token_row,
                     int64_t* qptr, int64_t* nnz_host, void* workspace, size_t workspace_bytes, void* stream);
int bf_table_to_csr(const int32_t* table, const int32_t* row_len, int64_t n_rows, int32_t width,
                    int32_t global_token, int64_t token_row, const int64_t* qptr, int32_t* kv, uint64_t* rkey,
                    int32_t q_bits, int32_t slot_bits, void* stream);

/* Reference COO edge_index [2, nnz] (row 0 = key/value node, row 1 = query
 * node; models/graphormer_dist_node_level.py:231-232) -> attention CSR with
 * rows ascending in kv. Workspace: bf_coo_to_csr_workspace_size.            */
int bf_coo_to_csr_workspace_size(int64_t nnz, int64_t n_q, size_t* bytes);
int bf_coo_to_csr(const int64_t* src, const int64_t* dst, int64_t nnz, int64_t n_q, int64_t n_kv,
                  int64_t* qptr, int32_t* kv, void* workspace, size_t workspace_bytes, void* stream);

/* Coalesce of a COO edge list: torch_geometric.utils.coalesce as used by
 * _merge_edge_index_list (gt_sp/utils.py:877-887): sorted by (src, dst) with
 * duplicates removed. out_src / out_dst int64 need capacity nnz; the number of
 * unique edges is returned in *count_host (the call synchronises the stream).
 * Workspace: bf_coalesce_workspace_size.                                       */
int bf_coalesce_workspace_size(int64_t nnz, size_t* bytes);
int bf_coalesce(const int64_t* src, const int64_t* dst, int64_t nnz, int64_t num_nodes,
                int64_t* out_src, int64_t* out_dst, int64_t* count_host,
                void* workspace, size_t workspace_bytes, void* stream);

/* Reverse (key-major) index of an attention CSR: kptr int64 [n_kv+1], and for
 * each reverse entry its query kq int32 [nnz] and its slot ks int32 [nnz] (its
 * position in the query's row: CSR position = qptr[kq] + ks), sorted by (kv,
 * position) — i.e. by (src, dst), the order PyG's coalesce gives
 * (gt_sp/utils.py:887). Drives the deterministic dK/dV pass and the COO
 * adaptor. Workspace: bf_reverse_index_workspace_size.                      */
int bf_reverse_index_workspace_size(int64_t nnz, int64_t n_kv, size_t* bytes);
int bf_reverse_index(const int64_t* qptr, const int32_t* kv, int64_t n_q, int64_t n_kv, int64_t nnz,
                     int64_t* kptr, int32_t* kq, int32_t* ks,
                     void* workspace, size_t workspace_bytes, void* stream);

/* bf_reverse_index from bf_table_to_csr's sort keys: one radix sort of the
 * 8-byte keys over their id bits only (stable, so each id's entries stay in
 * CSR order) into sorted uint64 [keys], then one pass that writes kptr and
 * decodes kq. (global_token, token_row) as given to bf_table_to_csr: the
 * token's entries, which have no key, take their fixed places (kv 0's segment
 * first, row by row; each token-row entry first in its kv's segment), the
 * sorted keys the rest. nnz counts every entry, or is any capacity above that
 * count (the keys, sorted, kq and ks then sized for it): the kernels take the
 * count itself from qptr[n_q] on the device. ks (may be NULL) is decoded in
 * the same pass, from the key's slot field; the dk/dv pass needs it only with
 * a bias, factor or dropout, so a caller may also keep `sorted` and call
 * bf_reverse_slots later. Same kptr / kq / ks as bf_reverse_index.
 * Workspace: bf_reverse_index_packed_workspace_size(nnz).                   */
int bf_reverse_index_packed_workspace_size(int64_t nnz, size_t* bytes);
int bf_reverse_index_packed(const uint64_t* rkey, const int64_t* qptr, int64_t nnz, int64_t n_q, int64_t n_kv,
                            int32_t q_bits, int32_t slot_bits, int32_t global_token, int64_t token_row,
                            uint64_t* sorted, int64_t* kptr, int32_t* kq, int32_t* ks, void* workspace,
                            size_t workspace_bytes, void* stream);
/* The stable radix sort bf_reverse_index_packed uses, on its own: in[0, n)
 * uint64 sorted by bits [begin_bit, end_bit) into out (n < 2^31; in and out
 * must not overlap). 8- or 9-bit digits, whichever needs fewer passes; each
 * pass counts digits per tile, scans the counts per digit and scatters. No
 * counterpart in the reference (torch.sort / coalesce sort inside PyTorch).
 * Workspace: bf_radix_sort_workspace_size(n, begin_bit, end_bit).          */
int bf_radix_sort_workspace_size(int64_t n, int32_t begin_bit, int32_t end_bit, size_t* bytes);
int bf_radix_sort_keys(const uint64_t* in, uint64_t* out, int64_t n, int32_t begin_bit, int32_t end_bit,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ks [nnz] from bf_reverse_index_packed's sorted keys (the same nnz, n_q,
 * key fields and token arguments): no counterpart in the reference.        */
int bf_reverse_slots(const uint64_t* sorted, const int64_t* qptr, int64_t nnz, int64_t n_q, int32_t q_bits,
                     int32_t slot_bits, int32_t global_token, int64_t token_row, int32_t* ks, void* stream);

/* Row id of every entry of a CSR (rows[i] = r for ptr[r] <= i < ptr[r+1]). */
int bf_expand_rows(const int64_t* ptr, int64_t n_rows, int64_t nnz, int64_t* rows, void* stream);

/* Split plan for rows longer than `threshold`: such a row is processed as
 * n = bf_split_row_items(len, item_size) items of ceil(len/n) entries (the
 * last one shorter), one workgroup each, whose partial sums are reduced in
 * item order by one workgroup per split row, so results are deterministic.
 * n = min(ceil(len/item_size), BF_MAX_ITEMS_PER_ROW): the cap keeps the reduce
 * of a long row (the Graphormer token row and column) short; a row of more
 * than BF_MAX_ITEMS_PER_ROW * BF_LONG_ROW_FACTOR * item_size entries (the
 * token row of a 100M-node graph) takes ceil(len / (item_size *
 * BF_LONG_ROW_FACTOR)) items instead, enough to spread it over the chip.
 *   nitems int32 [n_rows] (0 for short rows), item_off int32 [n_rows],
 *   item_row int32 [item_cap], heavy_rows int32 [heavy_cap] (the split rows,
 *   ascending), counts int32 [2] on the device = (#items, #split rows).
 *   Capacities: bf_split_item_capacity / bf_split_row_capacity.              */
#define BF_MAX_ITEMS_PER_ROW 160
#define BF_LONG_ROW_FACTOR 64
int64_t bf_split_row_items(int64_t len, int32_t item_size);
int64_t bf_split_item_capacity(int64_t nnz, int32_t threshold, int32_t item_size);
int64_t bf_split_row_capacity(int64_t nnz, int32_t threshold);
int bf_split_plan_workspace_size(int64_t n_rows, size_t* bytes);
int bf_split_plan(const int64_t* ptr, int64_t n_rows, int32_t threshold, int32_t item_size,
                  int32_t* nitems, int32_t* item_off, int32_t* item_row, int64_t item_cap,
                  int32_t* heavy_rows, int64_t heavy_cap, int32_t* counts,
                  void* workspace, size_t workspace_bytes, void* stream);

/* The split plan of a CSR whose only row longer than the threshold is row 0
 * (the Graphormer token row of a table's CSR, every other row holding at most
 * the table width + 1 entries), cut into n_items items (0: no split row):
 * the same arrays and counts bf_split_plan writes, in one pass and without a
 * scan. The caller vouches for the premise; n_items = bf_split_row_items of
 * row 0's length. */
int bf_split_plan_first_row(int64_t n_rows, int32_t n_items, int32_t* nitems, int32_t* item_off,
                            int32_t* item_row, int64_t item_cap, int32_t* heavy_rows, int64_t heavy_cap,
                            int32_t* counts, void* stream);

/* Rows of a CSR ordered longest-first (lengths capped at 255; rows of equal
 * capped length in an unspecified order that may change from call to call).
 * The key-major attention pass walks its rows in this order so the groups
 * sharing a wavefront carry similar work; a row's arithmetic does not depend
 * on its place. spans (may be NULL; needs ptr[n_rows] < 2^32) receives, per
 * slot, the slot's row as (ptr[row] << 32 | row length), so a reader walking
 * the order finds each row's entries without a random read of ptr.
 * Workspace: bf_row_order_workspace_size.                                    */
int bf_row_order_workspace_size(int64_t n_rows, size_t* bytes);
int bf_row_order(const int64_t* ptr, int64_t n_rows, int32_t* order, uint64_t* spans, void* workspace,
                 size_t workspace_bytes, void* stream);

/* bf_row_order, then the split plan of the rows it puts first (what
 * bf_split_plan writes for the rows that split). With 1 <= threshold <= 254
 * the rows longer than the threshold have the highest capped lengths, so they
 * are the order's first slots, and there are at most heavy_cap of them
 * (bf_split_row_capacity): the plan is scanned over min(heavy_cap, n_rows)
 * slots instead of all rows, from item counts the order pass writes as it
 * places each row. The split rows (heavy_rows) and their items are numbered in
 * slot order, longest first, instead of ascending row id, and only the split
 * rows' nitems / item_off entries are written. No counterpart in the
 * reference: it replaces bf_row_order + bf_split_plan over the reverse index. */
int bf_row_order_and_plan_workspace_size(int64_t n_rows, int64_t heavy_cap, size_t* bytes);
int bf_row_order_and_plan(const int64_t* ptr, int64_t n_rows, int32_t threshold, int32_t item_size,
                          int32_t* order, uint64_t* spans, int32_t* nitems, int32_t* item_off,
                          int32_t* item_row, int64_t item_cap, int32_t* heavy_rows, int64_t heavy_cap,
                          int32_t* counts, void* workspace, size_t workspace_bytes, void* stream);

/* ======================================================================
 * Sparse edge attention
 * ====================================================================== */

/* Everything the attention kernels need to walk one edge set. */
typedef struct bf_attn_index {
  int64_t n_q;                  /* queries (rows of qptr)                          */
  int64_t n_kv;                 /* key/value rows                                   */
  int64_t nnz;                  /* edges                                            */
  const int64_t* qptr;          /* [n_q+1]                                          */
  const int32_t* kv;            /* [nnz]   kv id per edge, query-major              */
  const int64_t* kptr;          /* [n_kv+1] reverse offsets (backward only)         */
  const int32_t* kq;            /* [nnz]   query per reverse entry (backward only)  */
  const int32_t* ks;            /* [nnz]   slot of each reverse entry in its query's
                                   row (backward with a bias, factor, dropout or
                                   dbias only; else may be NULL)                   */
  int32_t chunk;                /* rows longer than this use the split plan         */
  int32_t item;                 /* entries per split item                           */
  int32_t q_items, q_heavy;     /* query-side plan (bf_split_plan on qptr): counts  */
  const int32_t* q_nitems;
  const int32_t* q_item_off;
  const int32_t* q_item_row;
  const int32_t* q_heavy_rows;
  int32_t k_items, k_heavy;     /* key-side plan (bf_split_plan on kptr)            */
  const int32_t* k_nitems;
  const int32_t* k_item_off;
  const int32_t* k_item_row;
  const int32_t* k_heavy_rows;
  const int32_t* k_order;       /* [n_kv] key rows longest-first (bf_row_order), or NULL */
  int32_t token_column;         /* 1: key 0 is the Graphormer token column — attended by
                                   queries 1..n_q-1 exactly once each, at the first
                                   position of their rows, and by no other entry
                                   (bf_table_to_csr with global_token and a token row
                                   gives this); 2: the same for every query 0..n_q-1
                                   (a query shard without the token row, token_row < 0).
                                   The dq pass then also sums key 0's dK/dV terms,
                                   which the dk/dv pass would otherwise re-gather.
                                   0: no such promise. */
  const uint64_t* k_spans;      /* [n_kv] or NULL: bf_row_order's spans of k_order (needs
                                   k_order); the dk/dv pass then reads each row's entry
                                   range from its slot instead of from kptr            */
  const int32_t* plan_counts;   /* NULL: q_items, q_heavy, k_items, k_heavy above are the
                                   plans' counts. Else a device int32 [4] holding them
                                   (bf_split_plan's counts, query side then key side),
                                   and the four fields above are upper bounds — the
                                   capacities the plans were built with — which size the
                                   grids and the scratch; workgroups past the true counts
                                   exit. No host read is then needed between building
                                   an index and running attention on it.            */
} bf_attn_index;

/* GraphGPS attention dropout drawn inside the kernels
 * (models/graphgps_dist_node_level.py:166-176; rate = attention_dropout_rate,
 * utils/parser_node_level.py:58). The entry at slot s of query row r (its
 * place in the row's ascending kv order) and head h are kept iff u < 1 - rate,
 * where u = word h % 4 of Philox4x32-10 with counter (s, r, (offset + h/4)_lo,
 * (offset + h/4)_hi) and key (seed_lo, seed_hi), mapped to (x >> 8) * 2^-24
 * (the key-major pass knows an entry by its query kq and slot ks, so the mask
 * needs no CSR position there); a kept entry's V message
 * (after the softmax normalisation) is scaled by 1/(1 - rate). Forward and
 * backward given the same struct draw the same mask. Pass NULL (or rate 0)
 * for none.
 *   keep: NULL, or a byte mask of ceil(H/8) bytes per CSR position (byte b of
 *   entry e, at e * ceil(H/8) + b, holds heads 8b .. 8b + 7, bit h % 8 set
 *   when head h is kept), 4-byte aligned, of at least nnz * ceil(H/8) bytes
 *   rounded up to a multiple of 4 (the kernels read it by aligned dwords).
 *   bf_attn_fwd stores every entry's bits there; bf_attn_bwd, given the same
 *   struct after that forward, reads them back in its query-major pass when
 *   the call has no bias, factor or dbias and H <= 8 (the pass then skips the
 *   Philox rounds) and draws them elsewhere: the same bits either way, so the
 *   results are the same bit for bit with or without it.                    */
typedef struct bf_attn_dropout {
  float rate;          /* drop probability in [0, 1] */
  uint64_t seed;       /* Philox key */
  uint64_t offset;     /* Philox counter offset */
  uint8_t* keep;       /* NULL or the keep mask (above) */
} bf_attn_dropout;

/* float32 scratch the attention calls need for split rows (and, with
 * token_column, one record of 2*D floats per dq-pass workgroup). */
int64_t bf_attn_partials_floats(const bf_attn_index* idx, int32_t num_heads, int32_t head_dim);

/* Forward. Replaces CoreAttention.sparse_attention_bias
 * (models/graphormer_dist_node_level.py:155-265; GT models/gt_dist_node_level.py:
 * 179-262; GraphGPS models/graphgps_dist_node_level.py:151-177) on one edge set:
 *   a = clamp(sum_j k[s,h,j]*q[t,h,j]/sqrt(hn), -c, c) [+ bias[e,h]],
 *   p = exp(a), Z[t,h] = sum_e p, out[t,h,:] = sum_e p*f[e,h]*v[s,h,:] / (Z+1e-6)
 * with f = factor (GPS dropout keep*scale) or 1.
 *   score_clamp c in (0, 5]: 5 on the reference's tensor paths; GT's per-head
 *   edge lists (models/gt_dist_node_level.py:195-218) take exp(clamp(q.k, -5,
 *   5) / sqrt(hn)), which is c = 5 / sqrt(hn);
 *   q [n_q, H*hn], k, v [n_kv, H*hn] in `dtype`, rows 16-byte aligned;
 *   bias, factor: NULL or float32 [nnz, H] (per CSR position);
 *   dropout: NULL or the in-kernel GraphGPS dropout (its factor multiplies f);
 *   out [n_q, H*hn] in `dtype`; Z float32 [n_q, H];
 *   partials: float32 [bf_attn_partials_floats].                           */
int bf_attn_fwd(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim, float score_clamp,
                const void* q, const void* k, const void* v, const float* bias, const float* factor,
                const bf_attn_dropout* dropout, void* out, float* Z, float* partials, void* stream);

/* Backward of bf_attn_fwd (the autograd of the reference graph of ops,
 * models/graphormer_dist_node_level.py:231-263). Deterministic: dq by a
 * query-major pass, dk/dv by a key-major pass over the reverse index; no atomics.
 * Per query and head, Delta = sum_j dO*out is summed from the query's entries
 * (sum_e p f (dO . v_s) / D', D' = Z + 1e-6) in float32, so the forward's
 * output tensor is not read: a bfloat16 out would carry its rounding into the
 * gradients (the reference, under autocast, keeps out in float32).
 *   dbias: NULL or float32 [nnz, H] (per CSR position; needs idx->ks, as do
 *   a bias, a factor and a dropout: the key-major pass knows each entry by its
 *   query and slot, which key the dropout, and finds the CSR position a bias,
 *   factor or dbias is indexed by as qptr[kq] + ks);
 *   rowstat: float32 [n_q, H, 2] scratch (per query and head
 *   {1/D', Delta/D'}, written by the query-major pass and read by the
 *   key-major pass).                                                         */
int bf_attn_bwd(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim, float score_clamp,
                const void* q, const void* k, const void* v, const float* bias, const float* factor,
                const bf_attn_dropout* dropout, const float* Z, const void* dout, void* dq, void* dk, void* dv,
                float* dbias, float* rowstat, float* partials, void* stream);

/* Typed edges (Exphormer). Replace ExphormerCoreAttention.forward's typed
 * path (models/exphormer_dist_node_level.py:77-121: an edge_index with a type
 * row, score = clamp(sum_j k*q*E[type] / sqrt(hn), -5, 5), E =
 * edge_proj(edge_type_emb(type)), no bias, factor or dropout) and its autograd.
 * The index is typed: bit 31 of each kv id (query-major CSR) and of each kq id
 * (reverse index) is the entry's type (0 or 1), the other bits the id (ids and
 * sizes below 2^31); it has no token column and splits no query row
 * (q_items = 0; key rows may be split). type_mod: E, float32 [2, H * hn].
 * Forward: out [n_q, H * hn] in `dtype`, Z float32 [n_q, H].
 * Backward: dq, dk, dv, and dtype_mod = dE, float32 [2, H * hn] (summed over
 * the entries of each type in a fixed order); rowstat float32 [n_q, H, 2];
 * partials float32 [bf_attn_typed_partials_floats].                        */
int64_t bf_attn_typed_partials_floats(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim);
int bf_attn_fwd_typed(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim, const void* q,
                      const void* k, const void* v, const float* type_mod, void* out, float* Z, void* stream);
int bf_attn_bwd_typed(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim, const void* q,
                      const void* k, const void* v, const float* type_mod, const float* Z, const void* dout, void* dq,
                      void* dk, void* dv, float* dtype_mod, float* rowstat, float* partials, void* stream);

/* bf_attn_bwd for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference: its backward is autograd over torch_scatter. The caller passes
 * the inputs and outputs; the row stats and split partials live in a
 * file-scope device array of BF_ATTN_NOALLOC_SCRATCH_BYTES per GPU (held until
 * the process ends), so the call allocates nothing: no hipMalloc, no library
 * allocation, the per-kernel timer paused. An index whose scratch
 * (n_q*H*8 bytes, 256-aligned, + 4 * bf_attn_partials_floats) exceeds the
 * array is rejected with BF_ERR_INVALID before any launch. Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (any streams) race.
 * Results equal bf_attn_bwd's bit for bit.                                   */
#define BF_ATTN_NOALLOC_SCRATCH_BYTES (64u << 20)
int bf_attn_bwd_noalloc(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim,
                        float score_clamp, const void* q, const void* k, const void* v, const float* bias,
                        const float* factor, const bf_attn_dropout* dropout, const float* Z, const void* dout,
                        void* dq, void* dk, void* dv, float* dbias, void* stream);

/* How bf_attn_bwd runs its key-major (dk/dv) pass on this index, for callers
 * and tests that need to know which kernel instance a shape takes (host-only,
 * launches nothing): rows_per_group = short kv rows per lane group (1, or 4
 * past 16M kv rows in float32 / 1M in the 2-byte dtypes); stream_rows = 1 when
 * the q and dO tables exceed the 256 MB Infinity Cache and are gathered
 * non-temporally; prefetch_slots = 1 when a group's row slots are loaded in
 * one round before its loop (a 2-byte dtype with several rows per group). No
 * reference counterpart: the reference's scatter backward has no such choice. */
int bf_attn_bwd_kv_variant(const bf_attn_index* idx, int32_t dtype, int32_t num_heads, int32_t head_dim,
                           int32_t* rows_per_group, int32_t* stream_rows, int32_t* prefetch_slots);

/* ======================================================================
 * Measurement
 * ====================================================================== */

/* Gather-rate calibration (no reference counterpart: it serves the benchmark,
 * as a plain copy kernel serves a bandwidth figure). For e in [0, n_ids) reads
 * row ids[e] & id_mask of each non-NULL table t0..t2 (row_bytes of 16 to 512,
 * a multiple of 16; rows at a stride of their size; 16-byte aligned) with
 * 16-byte loads, non-temporal when `nontemporal` != 0, and writes nothing
 * (sink, a device uint32, is written only in the practically impossible case
 * that the folded words equal a fixed constant). The ids must lie in the
 * tables. Timing it on an attention pass's own ids and tables (the key-major
 * pass: kq over q, dO and the row stats; the query-major passes: kv over k
 * and v) gives the time those gathers alone take.                          */
int bf_gather_probe(const void* t0, int32_t row_bytes0, const void* t1, int32_t row_bytes1, const void* t2,
                    int32_t row_bytes2, const int32_t* ids, int64_t n_ids, uint32_t id_mask,
                    int32_t nontemporal, uint32_t* sink, void* stream);

/* Row-stream calibration, the other half of a pass's memory floor (no
 * reference counterpart). For e in [0, n_rows), row ids[e] (row e when ids is
 * NULL) is read from each non-NULL r0, r1 (non-temporal loads when
 * `nontemporal` != 0) and overwritten with zeros in each non-NULL w0, w1
 * (non-temporal stores), row_bytes (16 to 1024, a multiple of 16) per row,
 * tables 16-byte aligned at a stride of their row size; sink as for
 * bf_gather_probe. The ids must lie in the tables (negative ids are skipped).
 * On a pass's own rows in its own order (the key-major pass: its kv rows in
 * k_order, k and v read, dK and dV written; the forward: q read, out written;
 * the dq pass: q and dO read, dq written) it gives the time those rows alone
 * take; with the gathers' time it bounds the pass from below.               */
int bf_row_stream_probe(const void* r0, const void* r1, void* w0, void* w1, int32_t row_bytes,
                        const int32_t* ids, int64_t n_rows, int32_t nontemporal, uint32_t* sink,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BUDGETFORMER_HIP_H */
