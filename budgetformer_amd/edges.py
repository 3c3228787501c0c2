"""Budgeted query-centric edge construction on the HIP kernels.

``build_attention_edges`` is the device-side equivalent of the reference's
per-epoch build (``_build_merged_edges``, utils/fullgraph_sp_support.py:
2943-3026, driven by ``_build_attention_edges`` :3341-3362) for a fixed budget
state (b_real, b_rw): it returns an ``EdgeTable`` — the query-major
``[n_q, b_real+b_rw]`` int32 table plus row lengths — which the attention
modules consume directly, or which ``EdgeTable.to_edge_index()`` turns into the
reference's COO ``[2, E']`` (coalesced src-major order, then the Graphormer
virtual edges in fix_edge_index order, gt_sp/utils.py:113-130).

RNG: with ``u`` (float32 [n_q*P, L]) the walk consumes injected uniforms (the
parity contract); without it the walk draws Philox4x32-10 uniforms keyed by
``philox_seed`` (default: the edge seed) and the global walk id, so any query
shard draws exactly what a full build would.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

from . import hip_ops
from .graph import CSRGraph
from .gt_sp.utils import estimate_edge_build_bytes, estimate_hot_path_bytes, plan_edge_build
from .hip_ops import AttentionIndex

REAL_SEED_OFFSET = 17   # utils/fullgraph_sp_support.py:1413
RW_SEED_OFFSET = 37     # utils/fullgraph_sp_support.py:1514


@dataclass
class EdgeTable:
    table: torch.Tensor            # int32 [n_q, width], rows ascending kv, -1 padded
    row_len: torch.Tensor          # int32 [n_q]
    num_nodes: int
    q_lo: int = 0
    global_token: bool = False     # Graphormer virtual node applied when indexing
    query_ids: Optional[torch.Tensor] = None   # int32 [n_q] ascending: row i serves query_ids[i] (filtered builds)
    _index: dict = field(default_factory=dict, repr=False)

    @property
    def n_rows(self) -> int:
        return int(self.table.shape[0])

    @property
    def width(self) -> int:
        return int(self.table.shape[1])

    @property
    def holds_token_row(self) -> bool:
        """With the global token: whether this table's queries include node 0's shard, which then also
        carries the token's own row (query 0, attending every node)."""
        return self.global_token and self.query_ids is None and self.q_lo == 0

    def attention_index(self, chunk: int = hip_ops.DEFAULT_CHUNK, item: int = hip_ops.DEFAULT_ITEM) -> AttentionIndex:
        """CSR view for the attention kernels (cached per split setting).

        Query rows: the table's rows, preceded by the token row when ``holds_token_row`` (so a full
        build has N + 1 rows, ids shifted by one). A query shard [q_lo, q_lo + n) with q_lo > 0 has n
        rows, row r serving node q_lo + r (attention id q_lo + r + 1), each opening with kv 0; kv rows
        are always all N (+ 1) nodes."""
        idx = self._index.get((chunk, item))
        if idx is None and self.query_ids is not None:
            n_kv = self.num_nodes + (1 if self.global_token else 0)
            idx = AttentionIndex.from_coo(self.to_edge_index(), n_kv, n_kv, chunk=chunk, item=item)
            self._index[(chunk, item)] = idx
        if idx is None:
            n_kv = self.num_nodes + (1 if self.global_token else 0)
            token_row = (self.num_nodes if self.holds_token_row else -1) if self.global_token else None
            idx = AttentionIndex.from_table(self.table, self.row_len, self.global_token, n_kv=n_kv, chunk=chunk,
                                            item=item, check=False, token_row=token_row)
            self._index[(chunk, item)] = idx
        return idx

    def to_edge_index(self) -> torch.Tensor:
        """Reference-format COO [2, E'] int64 (row 0 kv/src, row 1 query/dst, global ids).

        Merged part in coalesce order (sorted by (src, dst)); with the global
        token, ids shifted by one and the virtual edges appended as
        fix_edge_index does (gt_sp/utils.py:113-130): [(v+1) -> 0 for every node
        v] when this table holds the token row, then [0 -> (q+1)] for each of
        its queries q (all N for a full build).
        """
        base = AttentionIndex.from_table(self.table, self.row_len, False, n_kv=self.num_nodes)
        coo = base.to_coo()
        if self.query_ids is not None:
            coo = torch.stack([coo[0], self.query_ids.to(torch.int64)[coo[1]]])
        elif self.q_lo:
            coo = torch.stack([coo[0], coo[1] + self.q_lo])
        if not self.global_token:
            return coo
        n = self.num_nodes
        ar = torch.arange(1, n + 1, dtype=torch.int64, device=coo.device)
        if self.query_ids is not None:
            # a filtered (probe) build keeps every virtual edge, as the reference applies fix_edge_index
            # to the whole probe edge set
            return torch.cat([coo + 1, torch.stack([ar, torch.zeros_like(ar)]),
                              torch.stack([torch.zeros_like(ar), ar])], dim=1)
        qs = torch.arange(self.q_lo + 1, self.q_lo + self.n_rows + 1, dtype=torch.int64, device=coo.device)
        parts = [coo + 1]
        if self.holds_token_row:
            parts.append(torch.stack([ar, torch.zeros_like(ar)]))
        parts.append(torch.stack([torch.zeros_like(qs), qs]))
        return torch.cat(parts, dim=1)


def build_attention_edges(graph: CSRGraph, *, real_edges_per_query: int, rw_edges_per_query: int,
                          walk_length: int = 4, walks_per_node: int = 2, edge_seed: int = 42,
                          q_lo: int = 0, n_q: Optional[int] = None, u: Optional[torch.Tensor] = None,
                          philox_seed: Optional[int] = None, philox_offset: int = 0,
                          global_token: bool = False, usable_bytes: Optional[int] = None) -> EdgeTable:
    """Budgeted edge table for queries [q_lo, q_lo+n_q) of ``graph``.

    b_real <= 0 drops the real part, b_rw <= 0 (or walks_per_node <= 0) drops
    the RW part (utils/fullgraph_sp_support.py:1395-1400, 1506-1508); both parts
    present -> set union per query, one part -> its multiset.

    The build is planned by ``gt_sp.utils.plan_edge_build``: when its transient
    does not fit next to the table (``usable_bytes``, default: the device's free
    HBM), the query range is built in shards on the device — bit-identical,
    since every walk's RNG counter is its global walk id.
    """
    n_q = graph.num_nodes - q_lo if n_q is None else n_q
    b_r = max(int(real_edges_per_query), 0)
    b_w = max(int(rw_edges_per_query), 0) if walks_per_node > 0 else 0
    if b_r + b_w <= 0:
        raise ValueError("empty edge budget: real_edges_per_query + rw_edges_per_query must be > 0")
    walk_length = max(1, int(walk_length))
    P = max(int(walks_per_node), 1)
    seed = int(edge_seed if philox_seed is None else philox_seed)
    all_hubs = graph.hubs() if b_r > 0 else None
    # queries above LIGHT_MAX in-neighbours take the group path; the rest one thread each (k <= 16)
    light = b_r > 0 and b_r <= 16 and b_w <= 16
    all_heavy = graph.heavy() if light else None
    # the table's attention index follows the build: its bytes beyond the table are reserved while
    # planning the build, and the graph's walk records are kept only where both still fit beside them
    est = estimate_hot_path_bytes(graph.num_nodes, graph.num_edges, n_q, b_r, b_w, global_token=global_token,
                                  holds_token_row=q_lo == 0, n_hubs=0 if all_hubs is None else all_hubs.numel())
    table_bytes = estimate_edge_build_bytes(n_q, b_r, b_w)["output"]
    walk_rec = graph.walk_records(reserve_bytes=est["peak"]) if b_w > 0 else None
    plan = plan_edge_build(graph.device, n_q, b_r, b_w, q_lo=q_lo, usable_bytes=usable_bytes,
                           reserve_bytes=est["peak"] - table_bytes)

    def in_range(lst, lo, cnt):
        if lst is None or lst.numel() == 0:
            return None
        if lo == 0 and cnt == graph.num_nodes:
            return lst
        bounds = torch.tensor([lo, lo + cnt], dtype=torch.int32, device=lst.device)
        a, b = torch.searchsorted(lst, bounds).tolist()
        return lst[a:b] if b > a else None

    def split_args(lo, cnt):
        if not light:
            return {"hubs": in_range(all_hubs, lo, cnt)}
        heavy = in_range(all_heavy, lo, cnt)
        return {"hubs": in_range(all_hubs, lo, cnt), "light_max": hip_ops.LIGHT_MAX,
                "heavy": heavy if heavy is not None else torch.empty(0, dtype=torch.int32, device=graph.device)}

    if len(plan.shards) == 1:
        table, row_len = hip_ops.build_edge_table(
            graph.rowptr, graph.col, graph.in_ptr, graph.in_src, graph.num_edges, q_lo, n_q, P, walk_length,
            b_r, b_w, int(edge_seed), u=u, philox_seed=seed, philox_offset=philox_offset, walk_rec=walk_rec,
            **split_args(q_lo, n_q))
    else:
        table = torch.empty(n_q, b_r + b_w, dtype=torch.int32, device=graph.device)
        row_len = torch.empty(n_q, dtype=torch.int32, device=graph.device)
        for lo, cnt in plan.shards:
            a = lo - q_lo
            u_s = None if u is None else u[a * P:(a + cnt) * P]
            hip_ops.build_edge_table(graph.rowptr, graph.col, graph.in_ptr, graph.in_src, graph.num_edges, lo, cnt,
                                     P, walk_length, b_r, b_w, int(edge_seed), u=u_s, philox_seed=seed,
                                     philox_offset=philox_offset, out=(table[a:a + cnt], row_len[a:a + cnt]),
                                     walk_rec=walk_rec, **split_args(lo, cnt))
    return EdgeTable(table, row_len, graph.num_nodes, q_lo=q_lo, global_token=global_token)
