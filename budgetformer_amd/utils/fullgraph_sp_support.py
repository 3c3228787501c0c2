"""The per-epoch edge pipeline of utils/fullgraph_sp_support.py on the HIP kernels.

Same function names and argument meaning as the reference; the work runs in
the fused device builder (``budgetformer_amd.edges``) or, for the per-seam
functions, in the matching HIP entry points.
"""
from __future__ import annotations

import torch

from .. import hip_ops
from ..edges import build_attention_edges
from ..graph import CSRGraph
from ..gt_sp.utils import _merge_edge_index_list, fix_edge_index  # noqa: F401  (re-exported seams)

_GRAPHORMER_VIRTUAL_NODE_MODELS = frozenset({"graphormer"})   # utils/fullgraph_sp_support.py:60-63
_EXPHORMER_MODELS = frozenset({"exphormer"})
_GRAPH_CACHE: dict = {}


def _edge_block_seed(args, edge_seed, offset: int) -> int:
    """utils/fullgraph_sp_support.py:970-972."""
    base = getattr(args, "seed", 0) if edge_seed is None else int(edge_seed)
    return int(base) + int(offset)


def _fixed_edge_budget_state_from_args(args):
    """utils/fullgraph_sp_support.py:842-855."""
    fixed_real = getattr(args, "fixed_real_edges_per_query", None)
    fixed_rw = getattr(args, "fixed_rw_edges_per_query", None)
    if fixed_real is None or fixed_rw is None:
        return None
    state = {"real_edges_per_query": int(fixed_real), "rw_edges_per_query": int(fixed_rw)}
    if getattr(args, "fixed_walk_length", None) is not None:
        state["walk_length"] = int(args.fixed_walk_length)
    return state


def _get_real_edge_budget(args, edge_budget_state=None, adaptive_edge_budget_cfg=None) -> int:
    """utils/fullgraph_sp_support.py:863-873: (B+1)//2 by default, B without walks."""
    state = edge_budget_state if edge_budget_state is not None else _fixed_edge_budget_state_from_args(args)
    if state is not None and "real_edges_per_query" in state:
        return int(state["real_edges_per_query"])
    max_tot = int(adaptive_edge_budget_cfg.max_total_edges_per_query) if adaptive_edge_budget_cfg is not None \
        else int(getattr(args, "max_total_edges_per_query", 0))
    if int(getattr(args, "walks_per_node", 0)) <= 0:
        return max_tot
    return (max_tot + 1) // 2


def _get_rw_edge_budget(args, edge_budget_state=None, adaptive_edge_budget_cfg=None) -> int:
    """utils/fullgraph_sp_support.py:876-886: B//2 by default, 0 without walks."""
    state = edge_budget_state if edge_budget_state is not None else _fixed_edge_budget_state_from_args(args)
    if state is not None and "rw_edges_per_query" in state:
        return int(state["rw_edges_per_query"])
    if int(getattr(args, "walks_per_node", 0)) <= 0:
        return 0
    max_tot = int(adaptive_edge_budget_cfg.max_total_edges_per_query) if adaptive_edge_budget_cfg is not None \
        else int(getattr(args, "max_total_edges_per_query", 0))
    return max_tot // 2


def _resolve_walk_length(args, edge_budget_state=None, walk_length_override=None) -> int:
    """utils/fullgraph_sp_support.py:3029-3037."""
    if walk_length_override is not None:
        return max(1, int(walk_length_override))
    if edge_budget_state is not None and "walk_length" in edge_budget_state:
        return max(1, int(edge_budget_state["walk_length"]))
    if getattr(args, "fixed_walk_length", None) is not None:
        return max(1, int(args.fixed_walk_length))
    return max(1, int(getattr(args, "walk_length", 4)))


def _sample_edges_per_query_random(edge_index, max_edges_per_query: int, seed: int, *, dst_stats=None):
    """Per-dst top-K by key(src, dst, seed) (utils/fullgraph_sp_support.py:1195-1228), on the device.

    Same multiset as every reference branch; returned dst-major with ascending
    src within a dst (the reference's order differs by branch).
    """
    _ = dst_stats
    if edge_index is None or edge_index.numel() == 0 or int(max_edges_per_query) <= 0:
        return edge_index
    k = int(max_edges_per_query)
    if edge_index.size(1) <= k:
        return edge_index
    if k > 32:
        raise NotImplementedError("per-query budgets above 32 are outside the kernel's register lists")
    n = int(edge_index[:2].max().item()) + 1
    in_ptr, in_src = hip_ops.coo_to_csr(edge_index[:2], n, n)
    table, row_len = hip_ops.real_select_merge(in_ptr, in_src, 0, n, k, int(seed), dedup=False, width=k)
    idx = hip_ops.AttentionIndex.from_table(table, row_len)
    rows = idx.entry_rows()
    return torch.stack([idx.kv.to(torch.int64), rows]).to(edge_index.dtype)


def _graph_for(edge_index_global, num_nodes, device) -> CSRGraph:
    dev = torch.device(device)
    key = (int(edge_index_global.data_ptr()), int(edge_index_global.size(1)), int(num_nodes), str(dev))
    g = _GRAPH_CACHE.get(key)
    if g is None:
        ei = hip_ops.coalesce(edge_index_global.to(dev), int(num_nodes))
        g = CSRGraph.from_edge_index(ei, int(num_nodes), symmetric=False, device=dev)
        _GRAPH_CACHE.clear()
        _GRAPH_CACHE[key] = g
    return g


def _build_merged_edges(args, edge_index_global, num_nodes, final_device, rw_device, nodes_per_rank,
                        edge_seed=None, edge_budget_state=None, adaptive_edge_budget_cfg=None,
                        walk_length_override=None):
    """utils/fullgraph_sp_support.py:2943-3026 on the fused device builder.

    Returns the reference's COO ``[2, E']`` (``[2, E'+2N]`` with the Graphormer
    token). Exphormer's typed ``[3, E]`` form is not on this path.
    """
    _ = (rw_device, nodes_per_rank)
    if getattr(args, "model", None) in _EXPHORMER_MODELS:
        raise NotImplementedError("Exphormer typed edges are not on this path")
    b_r = _get_real_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg)
    b_w = _get_rw_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg)
    P = int(getattr(args, "walks_per_node", 0))
    L = _resolve_walk_length(args, edge_budget_state, walk_length_override)
    base = getattr(args, "seed", 0) if edge_seed is None else int(edge_seed)
    graph = _graph_for(edge_index_global, num_nodes, final_device)
    token = getattr(args, "model", None) in _GRAPHORMER_VIRTUAL_NODE_MODELS and int(getattr(args, "num_global_node", 0)) > 0
    if b_r <= 0 and (b_w <= 0 or P <= 0):
        empty = torch.zeros((2, 0), dtype=torch.long, device=graph.device)
        return fix_edge_index(empty, int(num_nodes)) if token else empty
    table = build_attention_edges(graph, real_edges_per_query=b_r, rw_edges_per_query=b_w if P > 0 else 0,
                                  walk_length=L, walks_per_node=max(P, 1), edge_seed=int(base), global_token=token)
    return table.to_edge_index()
