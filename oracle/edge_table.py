"""CPU restatement (numpy) of BudgetFormer's budgeted query-centric edge build.

TEST INFRASTRUCTURE ONLY: imported by tests/, smoke() and bench.py's CPU
baseline leg; never by the product package.

Reference call chain restated here (all paths relative to the reference root):
  _build_merged_edges            utils/fullgraph_sp_support.py:2943-3026
    _resolve_real_edges_for_state  utils/fullgraph_sp_support.py:1312-1491
    _build_or_retrieve_full_rw_pool utils/fullgraph_sp_support.py:1656-1740
      build_head_hop_edges           gt_sp/utils.py:1251-1278
      compute_khop_pool_dgl_neighbor gt_sp/utils.py:1281-1384 (rw_edge_mode
                                     "dgl_neighbor"; sampler RNG defined here)
      compute_hop_buckets_random_walk gt_sp/utils.py:1074-1248
      _get_random_walk_graph         gt_sp/utils.py:890-936
      _run_random_walk               gt_sp/utils.py:1387-1473 (torch_cluster 1.6.3 /
                                     dgl 2.4.0 walk; RNG injected, see below)
    _resolve_rw_edges_for_state    utils/fullgraph_sp_support.py:1494-1517
    _sample_edges_per_query_random utils/fullgraph_sp_support.py:1195-1228
      (_sort :975-1004, _minhash_mask :1007-1065; both restated)
    _merge_edge_index_list         gt_sp/utils.py:877-887 (PyG 2.6.1 coalesce)
    fix_edge_index                 gt_sp/utils.py:113-130
    adjust_edge_index_nomerge      gt_sp/utils.py:540-545 (identity at SP=1)

Walk RNG contract. torch_cluster / DGL draw their own uniforms; neither package
is vendored or importable here, so the exact RNG->neighbour mapping of the
reference is *parity unpinned* at that boundary. The build defines the walk by
an injected uniform tensor ``u[N*P, L]`` (float32): at a node with ``deg``
out-neighbours, step index ``idx = int(float32(u) * float32(deg))`` (fp32
multiply, round-to-nearest, truncate), clamped to ``deg-1``; a node with
``deg == 0`` repeats itself (torch_cluster semantics; the DGL branch rewrites
its -1 to the previous node, gt_sp/utils.py:1431-1439).

Pinning (tests/test_oracle_edges.py):
  edge_key          literal known-answer values, a uint32-wrap formulation,
                    and the per-dst bijection (no ties for distinct src)
  random_walk       RNG-free chain/cycle graphs, dead-end stays, first/last
                    neighbour at u=0 / u=1-2^-24, an fp32-vs-fp64 rounding case
  hop_edges         hand-built walks with known pools (d=1 self-edge kept,
                    later stays dropped)
  khop_fanout_pool  all-neighbour hops against path counts (powers of the
                    adjacency matrix); samples shared per node and hop
  fanout_sample     subsets of the right size of distinct out-neighbours,
                    every neighbour equally likely (chi-square over seeds)
  sample_*          brute-force Python loops on small inputs; the sort branch
                    and the minhash branch agree as multisets
  merge/fix         Python set union; closed-form virtual edges
  build_merged_edges  pure-Python loop pipeline on small graphs
"""
from __future__ import annotations

import numpy as np

KEY_A = 1103515245
KEY_B = 214013
KEY_C_MUL = 2654435761
KEY_C_ADD = 12345
KEY_SCALE = 1 << 31
REAL_SEED_OFFSET = 17   # utils/fullgraph_sp_support.py:1413
RW_SEED_OFFSET = 37     # utils/fullgraph_sp_support.py:1514


def edge_block_seed(base_seed: int, offset: int) -> int:
    """``_edge_block_seed`` (utils/fullgraph_sp_support.py:970-972)."""
    return int(base_seed) + int(offset)


def edge_key(src, dst, seed: int) -> np.ndarray:
    """Hash key of (src, dst) under ``seed``.

    utils/fullgraph_sp_support.py:984-989 (sort branch), :1018-1023 (minhash
    branch), :1154-1161 (CSR-CPU branch): ``(src*1103515245 + dst*214013 +
    seed*2654435761 + 12345) mod 2^31`` in int64, non-negative.
    """
    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int64)
    const = int(seed) * KEY_C_MUL + KEY_C_ADD
    key = src * KEY_A + dst * KEY_B + np.int64(const)
    return np.mod(key, KEY_SCALE)


def csr_from_coo(edge_index: np.ndarray, num_nodes: int):
    """Coalesced CSR of ``edge_index`` rows (sources).

    ``SparseTensor(row=ei[0], col=ei[1]).coalesce().csr()`` (gt_sp/utils.py:926-931):
    sorted by (row, col), duplicates removed. Returns (rowptr int64[N+1], col int64[E]).
    """
    ei = np.asarray(edge_index, dtype=np.int64)
    if ei.size == 0:
        return np.zeros(num_nodes + 1, dtype=np.int64), np.zeros(0, dtype=np.int64)
    lin = np.unique(ei[0] * num_nodes + ei[1])
    row = lin // num_nodes
    col = lin % num_nodes
    rowptr = np.zeros(num_nodes + 1, dtype=np.int64)
    np.add.at(rowptr, row + 1, 1)
    return np.cumsum(rowptr), col


def random_walk(rowptr, col, starts, walk_length: int, u: np.ndarray) -> np.ndarray:
    """Uniform first-order walk under the injected-uniform contract.

    Restates ``_run_random_walk`` (gt_sp/utils.py:1387-1473): output
    ``[len(starts), L+1]`` int64 with ``walks[:,0] = starts``; a dead end
    repeats the current node. ``u`` is float32 ``[len(starts), L]``.
    """
    rowptr = np.asarray(rowptr, dtype=np.int64)
    col = np.asarray(col, dtype=np.int64)
    cur = np.asarray(starts, dtype=np.int64).copy()
    u = np.asarray(u, dtype=np.float32)
    n = cur.shape[0]
    walks = np.empty((n, walk_length + 1), dtype=np.int64)
    walks[:, 0] = cur
    for step in range(walk_length):
        beg = rowptr[cur]
        deg = rowptr[cur + 1] - beg
        prod = u[:, step] * deg.astype(np.float32)        # fp32 multiply, RNE
        idx = np.minimum(prod.astype(np.int64), np.maximum(deg - 1, 0))
        moving = deg > 0
        nxt = cur.copy()
        nxt[moving] = col[beg[moving] + idx[moving]]
        cur = nxt
        walks[:, step + 1] = cur
    return walks


def hop_edges_from_walks(walks: np.ndarray, min_hop: int = 1) -> np.ndarray:
    """RW pool from walks: the hop loop of compute_hop_buckets_random_walk.

    gt_sp/utils.py:1232-1248 with num_buckets=1: for d = min_hop..L, keep
    (kv=walks[:,d], q=walks[:,0]) iff kv >= 0 and (d == 1 or kv != walks[:,d-1]).
    Order: d-major, then walk id. Duplicates kept.
    """
    walk_length = walks.shape[1] - 1
    q = walks[:, 0]
    parts = []
    for d in range(max(1, min_hop), walk_length + 1):
        kv = walks[:, d]
        valid = kv >= 0
        if d > 1:
            valid &= kv != walks[:, d - 1]
        if valid.any():
            parts.append(np.stack([kv[valid], q[valid]]))
    if not parts:
        return np.zeros((2, 0), dtype=np.int64)
    return np.concatenate(parts, axis=1)


def fanout_sample(rowptr, col, num_nodes: int, fanout: int, hop: int, seed: int, offset: int = 0):
    """One hop's neighbour sample of every node (the sampler behind compute_khop_pool_dgl_neighbor,
    gt_sp/utils.py:1330-1333, ``dgl.sampling.sample_neighbors(g, nodes, fanout, edge_dir="out")``), as a
    CSR (ptr [N+1], ids). DGL's sampler RNG is not reproducible outside DGL (parity unpinned, as the walk's);
    the build defines the sample: a node with deg <= fanout (or fanout -1) keeps all its out-neighbours in
    CSR order; otherwise Floyd's algorithm draws `fanout` distinct indices of [0, deg): for i = 0..f-1 and
    j = deg - f + i, t = hi32(r_i * (j + 1)) with r_i word i % 4 of Philox(counter = (u_lo, u_hi, b_lo,
    b_hi), key = seed), b = offset + hop * 2^32 + i // 4; t joins the sample unless it is already in it,
    then j does. The sample is kept in ascending index order."""
    from .philox import philox4x32_10
    rowptr = np.asarray(rowptr, dtype=np.int64)
    col = np.asarray(col, dtype=np.int64)
    deg = np.diff(rowptr)
    f = int(fanout)
    take = deg if f < 0 else np.minimum(deg, f)
    ptr = np.concatenate([[0], np.cumsum(take)]).astype(np.int64)
    ids = np.empty(int(ptr[-1]), dtype=np.int64)
    big = np.nonzero(deg > f)[0] if f >= 0 else np.zeros(0, dtype=np.int64)
    small = np.ones(num_nodes, dtype=bool)
    small[big] = False
    for u in np.nonzero(small)[0]:
        ids[ptr[u]:ptr[u + 1]] = col[rowptr[u]:rowptr[u + 1]]
    if big.size and f > 0:
        seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        key = (seed & 0xFFFFFFFF, seed >> 32)
        uu = big.astype(np.uint64)
        words = np.empty((big.size, f), dtype=np.uint64)
        for blk in range((f + 3) // 4):
            b = (int(offset) + (int(hop) << 32) + blk) & 0xFFFFFFFFFFFFFFFF
            ctr = np.stack([uu & np.uint64(0xFFFFFFFF), uu >> np.uint64(32), np.full_like(uu, b & 0xFFFFFFFF),
                            np.full_like(uu, b >> 32)], axis=-1)
            r = philox4x32_10(ctr, key).astype(np.uint64)
            for w in range(4):
                i = blk * 4 + w
                if i < f:
                    words[:, i] = r[:, w]
        for row, u in enumerate(big):
            d = int(deg[u])
            chosen = []
            for i in range(f):
                j = d - f + i
                t = int((int(words[row, i]) * (j + 1)) >> 32)
                chosen.append(j if t in chosen else t)
            chosen.sort()
            ids[ptr[u]:ptr[u + 1]] = col[rowptr[u] + np.asarray(chosen, dtype=np.int64)]
    return ptr, ids


def khop_fanout_pool(rowptr, col, num_nodes: int, fanout, seed: int = 0, offset: int = 0, min_hop: int = 1,
                     samples=None) -> np.ndarray:
    """compute_khop_pool_dgl_neighbor (gt_sp/utils.py:1281-1384) -> pool [2, M] (row 0 kv, row 1 query).

    The frontier starts as (origin u, node u) for every node. Hop d (1-based) replaces every entry
    (o, c) by (o, s) for each s in c's hop-d sample, in order -- one sample per node and hop, shared by
    every entry at that node (the reference samples the frontier's unique nodes once) -- and, from
    min_hop on, emits (s -> o) for s != o; self pairs stay in the frontier. Hop-major, then frontier
    order. ``samples`` (a list of per-hop (ptr, ids) CSRs) replaces the sampler, to test the expansion
    on given samples."""
    fanout = list(fanout)
    rowptr = np.asarray(rowptr, dtype=np.int64)
    origin = np.arange(num_nodes, dtype=np.int64)
    cur = origin.copy()
    parts = []
    for d in range(1, len(fanout) + 1):
        if cur.size == 0:
            break
        ptr, ids = samples[d - 1] if samples is not None else fanout_sample(rowptr, col, num_nodes, fanout[d - 1],
                                                                              d, seed, offset)
        cnt = ptr[cur + 1] - ptr[cur]
        new_origin = np.repeat(origin, cnt)
        first = np.repeat(ptr[cur], cnt)
        within = np.arange(int(cnt.sum()), dtype=np.int64) - np.repeat(np.cumsum(cnt) - cnt, cnt)
        new_cur = ids[first + within] if within.size else np.zeros(0, dtype=np.int64)
        if d >= min_hop:
            keep = new_cur != new_origin
            parts.append(np.stack([new_cur[keep], new_origin[keep]]))
        origin, cur = new_origin, new_cur
    if not parts:
        return np.zeros((2, 0), dtype=np.int64)
    return np.concatenate(parts, axis=1).astype(np.int64)


def walk_starts(num_nodes: int, walks_per_node: int, q_lo: int = 0, q_hi: int | None = None) -> np.ndarray:
    """``arange(N).repeat_interleave(P)`` (gt_sp/utils.py:1198-1199); walk id w = n*P + p."""
    q_hi = num_nodes if q_hi is None else q_hi
    return np.repeat(np.arange(q_lo, q_hi, dtype=np.int64), walks_per_node)


def build_head_hop_edges(rowptr, col, num_nodes: int, walk_length: int, walks_per_node: int,
                         u: np.ndarray) -> np.ndarray:
    """build_head_hop_edges (gt_sp/utils.py:1251-1278) -> shared RW pool [2, M]."""
    starts = walk_starts(num_nodes, walks_per_node)
    walks = random_walk(rowptr, col, starts, walk_length, u)
    return hop_edges_from_walks(walks, min_hop=1)


def sample_edges_per_query_random(edge_index: np.ndarray, k: int, seed: int) -> np.ndarray:
    """Per-dst top-K by key, sort branch (utils/fullgraph_sp_support.py:975-1004).

    For each dst keep the K entries with the smallest key; ties (only duplicate
    (src,dst) pairs, since the key is a bijection of src for a fixed dst) are
    broken by original position (stable order). Returned in (dst, key) order.
    """
    ei = np.asarray(edge_index, dtype=np.int64)
    if ei.shape[1] == 0 or k <= 0:
        return ei
    if ei.shape[1] <= k:                       # :980-981
        return ei
    src, dst = ei[0], ei[1]
    key = edge_key(src, dst, seed)
    perm = np.lexsort((np.arange(src.size), key, dst))
    dst_sorted = dst[perm]
    is_new = np.ones(dst_sorted.size, dtype=bool)
    is_new[1:] = dst_sorted[1:] != dst_sorted[:-1]
    arange = np.arange(dst_sorted.size)
    group_start = np.maximum.accumulate(np.where(is_new, arange, 0))
    keep = (arange - group_start) < k
    return ei[:, perm[keep]]


def sample_edges_per_query_random_minhash(edge_index: np.ndarray, k: int, seed: int) -> np.ndarray:
    """Minhash branch (utils/fullgraph_sp_support.py:1007-1065), as an independent
    formulation: K rounds, each taking per-dst the (min key, min position) among
    the still-active entries. Returns the kept entries in original order.
    """
    ei = np.asarray(edge_index, dtype=np.int64)
    if ei.shape[1] == 0 or k <= 0 or ei.shape[1] <= k:
        return ei
    src, dst = ei[0], ei[1]
    key = edge_key(src, dst, seed)
    n = src.size
    groups = int(dst.max()) + 1
    active = np.ones(n, dtype=bool)
    keep = np.zeros(n, dtype=bool)
    pos = np.arange(n)
    for _ in range(k):
        if not active.any():
            break
        min_key = np.full(groups, KEY_SCALE, dtype=np.int64)
        np.minimum.at(min_key, dst, np.where(active, key, KEY_SCALE))
        chosen = active & (key == min_key[dst])
        min_pos = np.full(groups, n, dtype=np.int64)
        np.minimum.at(min_pos, dst, np.where(chosen, pos, n))
        chosen &= pos == min_pos[dst]
        keep |= chosen
        active &= ~chosen
    return ei[:, keep]


def coalesce(edge_index: np.ndarray, num_nodes: int) -> np.ndarray:
    """PyG ``coalesce`` (torch_geometric 2.6.1): sort by row*N+col and drop duplicates."""
    ei = np.asarray(edge_index, dtype=np.int64)
    lin = np.unique(ei[0] * num_nodes + ei[1])
    return np.stack([lin // num_nodes, lin % num_nodes])


def merge_edge_index_list(parts):
    """_merge_edge_index_list (gt_sp/utils.py:877-887).

    Drops None/empty parts; >=2 parts -> concatenated and coalesced (deduplicated,
    src-major sorted, N' = max id + 1); exactly 1 part -> returned as is
    (duplicates kept); no part -> the first entry (None or empty).
    """
    tensors = [p for p in parts if p is not None and p.size > 0]
    if not tensors:
        return parts[0] if parts else None
    if len(tensors) == 1:
        return tensors[0]
    ei = np.concatenate(tensors, axis=1).astype(np.int64)
    n = int(max(ei[0].max(), ei[1].max())) + 1
    return coalesce(ei, n)


def fix_edge_index(edge_index: np.ndarray, num_node: int) -> np.ndarray:
    """Graphormer virtual global token (gt_sp/utils.py:113-130).

    ids + 1, then append (v+1 -> 0) for v < N followed by (0 -> v+1) for v < N.
    """
    ei = np.asarray(edge_index, dtype=np.int64)
    ar = np.arange(num_node, dtype=np.int64)
    to_tok = np.stack([ar + 1, np.zeros(num_node, dtype=np.int64)])
    from_tok = np.stack([np.zeros(num_node, dtype=np.int64), ar + 1])
    return np.concatenate([ei + 1, to_tok, from_tok], axis=1)


def budget_split(max_total: int, walks_per_node: int = 2):
    """Default (real, rw) split of B: (ceil(B/2), floor(B/2)) when walks are on,
    (B, 0) otherwise (utils/fullgraph_sp_support.py:863-886)."""
    if walks_per_node <= 0:
        return int(max_total), 0
    return (int(max_total) + 1) // 2, int(max_total) // 2


def build_merged_edges(edge_index_global: np.ndarray, num_nodes: int, b_real: int, b_rw: int,
                       walk_length: int, walks_per_node: int, edge_seed: int, u: np.ndarray,
                       graphormer_global_token: bool = False) -> np.ndarray:
    """_build_merged_edges with a fixed (b_real, b_rw) budget state.

    utils/fullgraph_sp_support.py:2943-3026: real part = top-b_real of the graph
    edges per dst under seed+17 (dropped when b_real <= 0); RW part = top-b_rw
    of the walk pool per dst under seed+37 (dropped when b_rw <= 0 or no walks);
    then _merge_edge_index_list and, for Graphormer, fix_edge_index.
    ``u`` is the injected uniform tensor [N*P, L] for the walk.
    """
    parts = []
    ei = np.asarray(edge_index_global, dtype=np.int64)
    if b_real > 0:
        parts.append(sample_edges_per_query_random(ei, b_real, edge_block_seed(edge_seed, REAL_SEED_OFFSET)))
    if b_rw > 0 and walks_per_node > 0:
        rowptr, col = csr_from_coo(ei, num_nodes)
        pool = build_head_hop_edges(rowptr, col, num_nodes, walk_length, walks_per_node, u)
        parts.append(sample_edges_per_query_random(pool, b_rw, edge_block_seed(edge_seed, RW_SEED_OFFSET)))
    merged = merge_edge_index_list(parts) if parts else None
    if merged is None:
        merged = np.zeros((2, 0), dtype=np.int64)
    if graphormer_global_token:
        merged = fix_edge_index(merged, num_nodes)
    return merged


def coo_to_table(edge_index: np.ndarray, num_queries: int, width: int):
    """Query-major fixed-stride table of a COO edge list (the build's own format).

    Row q lists the kv ids of all entries with dst == q in ascending order
    (duplicates kept), padded with -1 to ``width``. Returns (table int32[n, width],
    row_len int32[n]). Raises if a row exceeds ``width``.
    """
    ei = np.asarray(edge_index, dtype=np.int64)
    src, dst = ei[0], ei[1]
    order = np.lexsort((src, dst))
    src, dst = src[order], dst[order]
    row_len = np.bincount(dst, minlength=num_queries).astype(np.int64)
    if row_len.size > num_queries:
        raise ValueError("dst id beyond num_queries")
    if row_len.size and row_len.max() > width:
        raise ValueError(f"row of length {row_len.max()} exceeds table width {width}")
    starts = np.concatenate([[0], np.cumsum(row_len)[:-1]])
    slot = np.arange(src.size) - starts[dst]
    table = np.full((num_queries, width), -1, dtype=np.int32)
    table[dst, slot] = src
    return table, row_len.astype(np.int32)


def build_edge_table(rowptr, col, num_nodes: int, b_real: int, b_rw: int, walk_length: int,
                     walks_per_node: int, edge_seed: int, u: np.ndarray, q_lo: int = 0, n_q: int = None):
    """The [n_q, b_real+b_rw] table the GPU builder must reproduce bit-exactly.

    Same semantics as build_merged_edges without the global token, on a graph
    given as coalesced CSR (source rows); real candidates of query q are the
    sources of edges into q. With a query range [q_lo, q_lo+n_q) only those
    queries are built (every selection is per query, so rows equal the full
    build's); ``u`` then holds the range's walks, [n_q*P, L]. Both parts are
    judged non-empty globally, as the reference's merge does.
    """
    rowptr = np.asarray(rowptr, dtype=np.int64)
    col = np.asarray(col, dtype=np.int64)
    n_q = num_nodes - q_lo if n_q is None else n_q
    if q_lo == 0 and n_q == num_nodes:
        src = np.repeat(np.arange(num_nodes, dtype=np.int64), np.diff(rowptr))
        merged = build_merged_edges(np.stack([src, col]), num_nodes, b_real, b_rw, walk_length, walks_per_node,
                                    edge_seed, u)
        return coo_to_table(merged, num_nodes, max(1, b_real + b_rw))
    parts = []
    if b_real > 0 and col.size > 0:
        src = np.repeat(np.arange(num_nodes, dtype=np.int64), np.diff(rowptr))
        keep = (col >= q_lo) & (col < q_lo + n_q)
        ei = np.stack([src[keep], col[keep]])
        if ei.shape[1]:
            parts.append(sample_edges_per_query_random(ei, b_real, edge_block_seed(edge_seed, REAL_SEED_OFFSET)))
    both = b_real > 0 and col.size > 0 and b_rw > 0 and walks_per_node > 0
    if b_rw > 0 and walks_per_node > 0:
        walks = random_walk(rowptr, col, walk_starts(num_nodes, walks_per_node, q_lo, q_lo + n_q), walk_length, u)
        pool = hop_edges_from_walks(walks, 1)
        parts.append(sample_edges_per_query_random(pool, b_rw, edge_block_seed(edge_seed, RW_SEED_OFFSET)))
    if both:
        merged = coalesce(np.concatenate(parts, axis=1), num_nodes)
    else:
        merged = parts[0] if parts else np.zeros((2, 0), dtype=np.int64)
    merged = np.stack([merged[0], merged[1] - q_lo])
    return coo_to_table(merged, n_q, max(1, b_real + b_rw))


# ---------------------------------------------------------------- adaptive-budget probe
# The budget controller's gain probe (utils/fullgraph_sp_support.py): the dst
# filter (:2261-2309), the filtered pools (:1743-1821) and the per-candidate
# assembly (:1824-1879, sampling by :1262-1309).
def reception_cone(edge_index: np.ndarray, probe_ids, n_layers: int):
    """_expand_probe_idx_for_reception (utils/fullgraph_sp_support.py:2261-2309).

    probe ids plus every node reaching them within n_layers-1 hops along the
    edges (src -> dst); the mask is sized by edge_index.max()+1, so probe ids
    at or beyond it are dropped. Returns probe_ids unchanged for n_layers <= 1,
    an empty probe set or an edgeless graph.
    """
    probe = np.asarray(probe_ids, dtype=np.int64).reshape(-1)
    ei = np.asarray(edge_index, dtype=np.int64)
    if n_layers <= 1 or probe.size == 0 or ei.size == 0:
        return probe_ids
    n = int(ei.max()) + 1
    probe = probe[(probe >= 0) & (probe < n)]
    reached = np.zeros(n, dtype=bool)
    reached[probe] = True
    frontier = probe
    for _ in range(n_layers - 1):
        if frontier.size == 0:
            break
        edges = ei[:, np.isin(ei[1], frontier)]
        if edges.size == 0:
            break
        srcs = np.unique(edges[0])
        srcs = srcs[(srcs >= 0) & (srcs < n)]
        new = srcs[~reached[srcs]]
        if new.size == 0:
            break
        reached[new] = True
        frontier = new
    return np.nonzero(reached)[0].astype(np.int64)


def filter_edge_index_by_dst(edge_index: np.ndarray, dst_nodes) -> np.ndarray:
    """_filter_edge_index_by_dst (utils/fullgraph_sp_support.py:1520-1533): entries whose dst is listed."""
    ei = np.asarray(edge_index, dtype=np.int64)
    if ei.size == 0:
        return ei
    dst_nodes = np.asarray(dst_nodes, dtype=np.int64).reshape(-1)
    return ei[:, np.isin(ei[1], dst_nodes)]


def subtract_edge_index(a: np.ndarray, b: np.ndarray, num_nodes: int) -> np.ndarray:
    """_subtract_edge_index (utils/fullgraph_sp_support.py:1536-1551): drop entries of a whose pair is in b."""
    if a is None or a.size == 0 or b is None or b.size == 0:
        return a
    n = max(1, int(num_nodes))
    keep = ~np.isin(a[0] * n + a[1], b[0] * n + b[1])
    return a[:, keep]


def probe_edge_pools(edge_index_global: np.ndarray, num_nodes: int, dst_filter, walk_length: int,
                     walks_per_node: int, u: np.ndarray, use_real: bool = True, use_rw: bool = True) -> dict:
    """_build_probe_edge_pools (utils/fullgraph_sp_support.py:1743-1821).

    real = graph edges into the filter; rw = the full RW pool (walks from every
    node, ``u`` [N*P, L]) restricted to the filter, minus every pair of the real
    pool when both pools are non-empty.
    """
    ei = np.asarray(edge_index_global, dtype=np.int64)
    real = filter_edge_index_by_dst(ei, dst_filter) if use_real else None
    rw = None
    if use_rw and walks_per_node > 0:
        rowptr, col = csr_from_coo(ei, num_nodes)
        pool = build_head_hop_edges(rowptr, col, num_nodes, walk_length, walks_per_node, u)
        rw = filter_edge_index_by_dst(pool, dst_filter)
        if rw.size and real is not None and real.size:
            rw = subtract_edge_index(rw, real, num_nodes)
    return {"real": real, "rw": rw}


def assemble_edges_from_pools(pools: dict, num_nodes: int, b_real: int, b_rw: int, edge_seed: int,
                              graphormer_global_token: bool = False, exphormer: bool = False) -> np.ndarray:
    """_assemble_edges_from_pools (utils/fullgraph_sp_support.py:1824-1879).

    Per pool: the top-b per dst under seed+17 (real) / seed+37 (rw), a zero
    budget dropping the pool (:1262-1309); then the typed [3, E] concatenation
    for Exphormer, else _merge_edge_index_list and, for Graphormer,
    fix_edge_index.
    """
    real, rw = pools.get("real"), pools.get("rw")
    if real is not None:
        real = sample_edges_per_query_random(real, b_real, edge_block_seed(edge_seed, REAL_SEED_OFFSET)) \
            if b_real > 0 else None
    if rw is not None:
        rw = sample_edges_per_query_random(rw, b_rw, edge_block_seed(edge_seed, RW_SEED_OFFSET)) if b_rw > 0 else None
    if exphormer:
        typed = [np.concatenate([x, np.full((1, x.shape[1]), t, dtype=np.int64)])
                 for t, x in ((0, real), (1, rw)) if x is not None and x.size > 0]
        return np.concatenate(typed, axis=1) if typed else np.zeros((3, 0), dtype=np.int64)
    parts = [x for x in (real, rw) if x is not None and x.size > 0]
    merged = merge_edge_index_list(parts) if parts else None
    if merged is None:
        merged = np.zeros((2, 0), dtype=np.int64)
    if graphormer_global_token:
        merged = fix_edge_index(merged, num_nodes)
    return merged
