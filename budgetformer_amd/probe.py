"""Adaptive-Budget probe build on the HIP kernels.

Reference (utils/fullgraph_sp_support.py), the budget controller's gain probe:

- ``_expand_probe_idx_for_reception`` (:2261-2309): the dst filter is the probe
  set plus its (n_layers-1)-hop in-neighbours;
- ``_build_probe_edge_pools`` (:1743-1821): the real pool is every graph edge
  into the filter, the RW pool is the epoch's full walk pool restricted to the
  filter minus every (src, dst) pair already in the real pool;
- ``_assemble_edges_from_pools`` (:1824-1879): each candidate budget samples
  both pools per dst with the training seeds (edge_seed+17 / +37) and merges
  them like the training build (or keeps them typed for Exphormer).

Device design. Every pool entry of dst q comes from q's in-neighbour row or
q's own walks, so neither pool is materialised: ``bf_real_select_rows`` and
``bf_rw_select_rows`` rank each filtered query's candidates once, at the
largest budgets asked for, and keep the winners in key order. Since the top-K
by a fixed key is nested in K, every candidate (base, real+block, rw+block) is
a prefix of that one ranking, and ``bf_assemble_rows`` merges the prefixes of
one candidate into a table row. Walk ids stay global (q*P + p), so a probe row
draws exactly the walks of the training build's row for q.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import hip_ops
from .edges import REAL_SEED_OFFSET, RW_SEED_OFFSET, EdgeTable
from .graph import CSRGraph


def _edge_id_bound(graph: CSRGraph) -> int:
    """max node id appearing in an edge + 1 (0 without edges): the reference
    sizes its reception mask by ``edge_index.max() + 1`` (:2284-2286)."""
    if graph.num_edges == 0:
        return 0
    deg = graph.rowptr[1:] - graph.rowptr[:-1]
    has_out = torch.nonzero(deg > 0).view(-1)
    top_src = int(has_out[-1]) if has_out.numel() else -1
    return max(int(graph.col.max()), top_src) + 1


def reception_cone(graph: CSRGraph, probe_ids: torch.Tensor, n_layers: int) -> torch.Tensor:
    """``_expand_probe_idx_for_reception`` (:2261-2309) as a device BFS over the in-neighbour CSR.

    Returns ``probe_ids`` unchanged for n_layers <= 1, an empty probe set or an
    edgeless graph; otherwise the ascending int64 ids of the probe nodes (those
    inside the edge id range) and every node reaching them within n_layers-1
    hops.
    """
    if n_layers <= 1 or probe_ids is None or probe_ids.numel() == 0 or graph.num_edges == 0:
        return probe_ids
    n = graph.num_nodes
    bound = _edge_id_bound(graph)
    ids = probe_ids.to(graph.device, torch.int64).view(-1)
    ids = ids[(ids >= 0) & (ids < bound)]
    mask = torch.zeros(n, dtype=torch.uint8, device=graph.device)
    mask[ids] = 1
    frontier = mask.clone()
    for _ in range(n_layers - 1):
        reached = torch.zeros_like(mask)
        hip_ops.mark_in_neighbors(graph.in_ptr, graph.in_src, frontier, reached)
        new = reached & (1 - mask)
        if not bool(new.any()):
            break
        mask |= new
        frontier = new
    return torch.nonzero(mask).view(-1)


@dataclass
class ProbeBuild:
    """Key-ordered selections of one probe at the largest budgets; ``table(b_r, b_w)`` assembles a candidate."""

    graph: CSRGraph
    query_ids: torch.Tensor                    # int32 ascending, the dst filter
    real: Optional[tuple]                      # (sel [n, max_real] key order, cnt [n]) or None
    rw: Optional[tuple]
    real_nonempty: bool                        # the filtered real pool holds an edge
    rw_nonempty: bool                          # the filtered RW pool (after subtraction) holds an entry
    global_token: bool = False

    def _parts(self, b_real: int, b_rw: int):
        real = self.real if (self.real is not None and b_real > 0) else None
        rw = self.rw if (self.rw is not None and b_rw > 0) else None
        if real is not None and b_real > real[0].shape[1]:
            raise ValueError(f"b_real {b_real} exceeds the probe's ranked budget {real[0].shape[1]}")
        if rw is not None and b_rw > rw[0].shape[1]:
            raise ValueError(f"b_rw {b_rw} exceeds the probe's ranked budget {rw[0].shape[1]}")
        return real, rw

    def table(self, b_real: int, b_rw: int) -> EdgeTable:
        """One candidate as an EdgeTable over ``query_ids`` (set union per dst when both parts are
        non-empty over the filter, the sampled multiset otherwise)."""
        real, rw = self._parts(b_real, b_rw)
        n = self.query_ids.numel()
        dev = self.graph.device
        if real is None and rw is None:
            t = torch.empty(n, 1, dtype=torch.int32, device=dev).fill_(-1)
            return EdgeTable(t, torch.zeros(n, dtype=torch.int32, device=dev), self.graph.num_nodes,
                             global_token=self.global_token, query_ids=self.query_ids)
        dedup = real is not None and rw is not None and self.real_nonempty and self.rw_nonempty
        t, rl = hip_ops.assemble_rows(real, rw, b_real, b_rw, dedup=dedup)
        return EdgeTable(t, rl, self.graph.num_nodes, global_token=self.global_token, query_ids=self.query_ids)

    def typed_edge_index(self, b_real: int, b_rw: int) -> torch.Tensor:
        """Exphormer form ``[3, E]``: the sampled real part (type 0) then the sampled RW part (type 1),
        not merged (:1842-1861)."""
        real, rw = self._parts(b_real, b_rw)
        qids = self.query_ids.to(torch.int64)
        out = []
        for t, part, b in ((0, real, b_real), (1, rw, b_rw)):
            if part is None:
                continue
            tab, rl = hip_ops.assemble_rows(part, None, b, 0, dedup=False) if t == 0 else \
                hip_ops.assemble_rows(None, part, 0, b, dedup=False)
            coo = EdgeTable(tab, rl, self.graph.num_nodes, query_ids=self.query_ids).to_edge_index()
            if coo.numel():
                out.append(torch.cat([coo, torch.full((1, coo.shape[1]), t, dtype=torch.int64, device=coo.device)]))
        if not out:
            return torch.zeros((3, 0), dtype=torch.int64, device=qids.device)
        return torch.cat(out, dim=1)


def build_probe(graph: CSRGraph, dst_filter: torch.Tensor, *, max_real: int, max_rw: int, walk_length: int = 4,
                walks_per_node: int = 2, edge_seed: int = 42, use_real: bool = True, use_rw: bool = True,
                u: Optional[torch.Tensor] = None, philox_seed: Optional[int] = None, philox_offset: int = 0,
                global_token: bool = False, hub_threshold: int = hip_ops.HUB_THRESHOLD) -> ProbeBuild:
    """Rank the probe pools of ``dst_filter`` once (``_build_probe_edge_pools`` + the sampling of
    ``_assemble_edges_from_pools``) for budgets up to (max_real, max_rw).

    ``use_real`` / ``use_rw`` say whether the reference builds each pool
    (``_use_real_edges`` / ``_use_rw_edges``). The RW pool is cut by the real
    pool only when both pools are non-empty (:1797-1812). ``u`` (float32
    [n*P, L], rows in ascending filter order) injects the walk uniforms.
    """
    dev = graph.device
    qids = torch.unique(dst_filter.to(dev).view(-1)).to(torch.int32)
    n = qids.numel()
    P = max(int(walks_per_node), 1)
    L = max(int(walk_length), 1)
    seed = int(edge_seed if philox_seed is None else philox_seed)
    real_nonempty = False
    real = rw = None
    if use_real and n:
        deg = graph.in_ptr[qids.long() + 1] - graph.in_ptr[qids.long()]
        real_nonempty = bool((deg > 0).any())
        if max_real > 0:
            hubs = graph.hubs(hub_threshold)
            hubs = hubs[torch.isin(hubs, qids)] if hubs.numel() else hubs
            real = hip_ops.real_select_rows(graph.in_ptr, graph.in_src, qids, int(max_real),
                                            int(edge_seed) + REAL_SEED_OFFSET, hubs=hubs if hubs.numel() else None,
                                            hub_threshold=hub_threshold)
    rw_nonempty = False
    if use_rw and walks_per_node > 0 and n:
        subtract = (graph.in_ptr, graph.in_src) if real_nonempty else None
        k = max(int(max_rw), 1)
        sel, cnt = hip_ops.rw_select_rows(graph.rowptr, graph.col, qids, P, L, k, int(edge_seed) + RW_SEED_OFFSET,
                                          u=u, philox_seed=seed, philox_offset=philox_offset, subtract=subtract,
                                          walk_rec=graph.walk_records())
        rw_nonempty = bool((cnt > 0).any())
        if max_rw > 0:
            rw = (sel, cnt)
    return ProbeBuild(graph, qids, real, rw, real_nonempty, rw_nonempty, global_token=global_token)
