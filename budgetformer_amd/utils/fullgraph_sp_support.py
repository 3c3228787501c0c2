"""The per-epoch edge pipeline of utils/fullgraph_sp_support.py on the HIP kernels.

Same function names and argument meaning as the reference; the work runs in
the fused device builder (``budgetformer_amd.edges``, ``budgetformer_amd.probe``)
or, for the per-seam functions, in the matching HIP entry points.

Device placement: every build runs on the HIP device. A ``rw_device`` or
``device`` of "cpu" only decides where the returned tensor lives (it is copied
there); nothing is computed on the host.
"""
from __future__ import annotations

import torch

from .. import hip_ops
from ..edges import build_attention_edges
from ..graph import CSRGraph
from ..gt_sp.utils import (_draw_walk_seed, _merge_edge_index_list, build_head_hop_edges,  # noqa: F401
                           compute_khop_pool_dgl_neighbor, fix_edge_index)
from ..probe import reception_cone

_GRAPHORMER_VIRTUAL_NODE_MODELS = frozenset({"graphormer"})   # utils/fullgraph_sp_support.py:60-63
_EXPHORMER_MODELS = frozenset({"exphormer"})
_GRAPH_CACHE: dict = {}

# edge-placement policies (utils/fullgraph_sp_support.py:218-230)
EDGE_POLICY_GPU_PERSIST = "gpu_persist"
EDGE_POLICY_GPU_EPHEMERAL = "gpu_ephemeral"
EDGE_POLICY_CPU_BROADCAST = "cpu_broadcast"
EDGE_POLICY_CPU_RANK_LOCAL_PREFETCH = "cpu_rank_local_prefetch"
EDGE_POLICY_CPU_BROADCAST_PREFETCH = "cpu_broadcast_prefetch"
_EDGE_POLICY_CHOICES = frozenset({EDGE_POLICY_GPU_PERSIST, EDGE_POLICY_GPU_EPHEMERAL, EDGE_POLICY_CPU_BROADCAST,
                                  EDGE_POLICY_CPU_RANK_LOCAL_PREFETCH, EDGE_POLICY_CPU_BROADCAST_PREFETCH})

_MERGED_EDGE_CACHE: dict = {}


def _hip_device(device) -> torch.device:
    """The HIP device a build runs on: ``device`` itself, or the current one for a host request."""
    dev = torch.device(device)
    if dev.type == "cuda":
        return dev
    if not torch.cuda.is_available():
        raise RuntimeError("the edge builder needs a HIP device; there is no host build")
    return torch.device("cuda", torch.cuda.current_device())


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


def _fixed_edge_budget_enabled(args, adaptive_edge_budget_cfg=None) -> bool:
    """utils/fullgraph_sp_support.py:857-860."""
    if adaptive_edge_budget_cfg is not None and adaptive_edge_budget_cfg.enabled:
        return False
    return _fixed_edge_budget_state_from_args(args) is not None


def _random_block_sampling_enabled(args, adaptive_edge_budget_cfg=None) -> bool:
    """utils/fullgraph_sp_support.py:830-835: per-query budgets apply (adaptive, fixed or random blocks)."""
    if adaptive_edge_budget_cfg is not None and adaptive_edge_budget_cfg.enabled:
        return True
    if _fixed_edge_budget_enabled(args, adaptive_edge_budget_cfg):
        return True
    return bool(getattr(args, "random_edge_blocks", False))


def _use_real_edges(args, adaptive_edge_budget_cfg=None) -> bool:
    """utils/fullgraph_sp_support.py:889-894."""
    if _fixed_edge_budget_enabled(args, adaptive_edge_budget_cfg) or \
            _random_block_sampling_enabled(args, adaptive_edge_budget_cfg):
        return _get_real_edge_budget(args, adaptive_edge_budget_cfg=adaptive_edge_budget_cfg) > 0
    return bool(getattr(args, "include_real_edges", 0))


def _use_real_edges_for_state(args, edge_budget_state=None, adaptive_edge_budget_cfg=None) -> bool:
    """utils/fullgraph_sp_support.py:897-902."""
    if _fixed_edge_budget_enabled(args, adaptive_edge_budget_cfg) or \
            _random_block_sampling_enabled(args, adaptive_edge_budget_cfg):
        return _get_real_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg) > 0
    return bool(getattr(args, "include_real_edges", 0))


def _use_rw_edges(args, edge_budget_state=None, adaptive_edge_budget_cfg=None) -> bool:
    """utils/fullgraph_sp_support.py:905-916 (the fanout mode needs no walks_per_node)."""
    if _rw_edge_mode(args) != "dgl_neighbor" and int(getattr(args, "walks_per_node", 0)) <= 0:
        return False
    if _fixed_edge_budget_enabled(args, adaptive_edge_budget_cfg) or \
            _random_block_sampling_enabled(args, adaptive_edge_budget_cfg):
        return _get_rw_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg) > 0
    return True


def _rw_edge_mode(args) -> str:
    mode = str(getattr(args, "rw_edge_mode", "random_walk"))
    if mode not in ("random_walk", "dgl_neighbor"):
        raise ValueError(f"unknown rw_edge_mode {mode!r} (random_walk or dgl_neighbor)")
    return mode


def _parse_fanout(fanout) -> list:
    """utils/fullgraph_sp_support.py:1642-1653: "10,5", [10, 5] or (10, 5) -> [10, 5]; -1 is every
    neighbour at that hop; None or empty -> [10, 5]."""
    if fanout is None:
        return [10, 5]
    items = list(fanout) if isinstance(fanout, (list, tuple)) else \
        [p for p in str(fanout).replace(" ", "").split(",") if p != ""]
    parsed = [int(x) for x in items]
    return parsed if parsed else [10, 5]


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
    n = int(edge_index[:2].max().item()) + 1
    in_ptr, in_src = hip_ops.coo_to_csr(edge_index[:2], n, n)
    table, row_len = hip_ops.real_select_merge(in_ptr, in_src, 0, n, k, int(seed), dedup=False, width=k)
    idx = hip_ops.AttentionIndex.from_table(table, row_len)
    rows = idx.entry_rows()
    return torch.stack([idx.kv.to(torch.int64), rows]).to(edge_index.dtype)


def _graph_for(edge_index_global, num_nodes, device) -> CSRGraph:
    dev = torch.device(device)
    key = (int(edge_index_global.data_ptr()), int(edge_index_global.size(1)), int(num_nodes), str(dev))
    hit = _GRAPH_CACHE.get(key)
    # the entry pins its source tensor, so a hit is the same tensor (same version), not a reused address
    if hit is not None and hit[0] is edge_index_global and hit[1] == edge_index_global._version:
        return hit[2]
    ei = hip_ops.coalesce(edge_index_global.to(dev), int(num_nodes))
    g = CSRGraph.from_edge_index(ei, int(num_nodes), symmetric=False, device=dev)
    _GRAPH_CACHE.clear()
    _GRAPH_CACHE[key] = (edge_index_global, edge_index_global._version, g)
    return g


def _build_or_retrieve_full_rw_pool(args, edge_index_global, num_nodes, rw_device, walk_length, walks_per_node,
                                    num_heads, edge_seed):
    """utils/fullgraph_sp_support.py:1656-1740: the full RW pool [2, M] (kv, q) of walks from every
    node, kept in a single-slot cache on ``args`` keyed by everything that shapes it.

    The walk is the device kernel (Philox keyed by ``edge_seed`` and the global
    walk id, so it draws what the fused builder draws); rw_edge_mode
    "dgl_neighbor" takes the fanout k-hop pool (``compute_khop_pool_dgl_neighbor``,
    fanout from ``args.fanout``) instead. The pool lives on ``rw_device`` (copied
    there when that is the host).
    """
    mode = _rw_edge_mode(args)
    fanout = _parse_fanout(getattr(args, "fanout", "10,5"))
    key = (id(edge_index_global), int(num_nodes), int(walk_length), int(walks_per_node), int(num_heads),
           int(edge_seed) if edge_seed is not None else None, str(rw_device), mode, tuple(fanout))
    cached = getattr(args, "_cached_full_rw_pool", None)
    if cached is not None and cached.get("key") == key:
        return cached["pool"]
    dev = _hip_device(rw_device)
    seed = _draw_walk_seed() if edge_seed is None else int(edge_seed)
    if mode == "dgl_neighbor":
        pool = compute_khop_pool_dgl_neighbor(edge_index_global.to(dev), int(num_nodes), fanout, device=dev,
                                              min_hop=1, seed=seed)
    else:
        pool = build_head_hop_edges(edge_index_global.to(dev), int(num_nodes), int(num_heads), 1, device=dev,
                                    walk_length=int(walk_length), walks_per_node=int(walks_per_node), seed=seed)
    pool = pool.to(torch.device(rw_device))
    args._cached_full_rw_pool = {"key": key, "pool": pool}
    return pool


def _resolve_real_edges_for_state(args, edge_index_global, device, edge_seed=None, edge_budget_state=None,
                                  adaptive_edge_budget_cfg=None):
    """utils/fullgraph_sp_support.py:1312-1491: the (sampled) real part, or None when unused."""
    if not _use_real_edges_for_state(args, edge_budget_state, adaptive_edge_budget_cfg):
        return None
    real = edge_index_global
    if not _random_block_sampling_enabled(args, adaptive_edge_budget_cfg):
        return real.to(torch.device(device))
    b_r = _get_real_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg)
    if b_r <= 0:
        return None
    sampled = _sample_edges_per_query_random(real.to(_hip_device(device)), b_r, _edge_block_seed(args, edge_seed, 17))
    return sampled.to(torch.device(device))


def _resolve_rw_edges_for_state(args, rw_edges, edge_seed=None, edge_budget_state=None,
                                adaptive_edge_budget_cfg=None):
    """utils/fullgraph_sp_support.py:1494-1517: the (sampled) RW part, or None."""
    if rw_edges is None:
        return None
    if not _random_block_sampling_enabled(args, adaptive_edge_budget_cfg):
        return rw_edges
    b_w = _get_rw_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg)
    if b_w <= 0:
        return None
    out_dev = rw_edges.device
    sampled = _sample_edges_per_query_random(rw_edges.to(_hip_device(out_dev)), b_w,
                                             _edge_block_seed(args, edge_seed, 37))
    return sampled.to(out_dev)


def _typed_edges(real: torch.Tensor, rw: torch.Tensor, device) -> torch.Tensor:
    """Exphormer RW mode (utils/fullgraph_sp_support.py:2999-3012): [3, E] with real = type 0, rw = type 1."""
    parts = [(x, t) for x, t in ((real, 0), (rw, 1)) if x is not None and x.numel() > 0]
    if not parts:
        return torch.zeros((3, 0), dtype=torch.long, device=device)
    return torch.cat([torch.cat([x.to(device, torch.long), torch.full((1, x.shape[1]), t, dtype=torch.long,
                                                                      device=device)]) for x, t in parts], dim=1)


def _build_merged_edges(args, edge_index_global, num_nodes, final_device, rw_device, nodes_per_rank,
                        edge_seed=None, edge_budget_state=None, adaptive_edge_budget_cfg=None,
                        walk_length_override=None):
    """utils/fullgraph_sp_support.py:2943-3026.

    Budgeted states (the adaptive / fixed / random-block modes) run the fused
    device builder and return the reference's COO ``[2, E']`` (``[2, E'+2N]``
    with the Graphormer token); Exphormer's RW mode returns the typed
    ``[3, E]`` (real part type 0, RW part type 1, not merged). Unbudgeted
    states merge the whole graph with the whole RW pool, as the reference does.
    """
    _ = nodes_per_rank
    model = getattr(args, "model", None)
    out_dev = torch.device(final_device)
    dev = _hip_device(final_device)
    token = model in _GRAPHORMER_VIRTUAL_NODE_MODELS and int(getattr(args, "num_global_node", 0)) > 0
    exphormer_rw = model in _EXPHORMER_MODELS and int(getattr(args, "expander_degree", 0)) <= 0
    if model in _EXPHORMER_MODELS and not exphormer_rw:
        raise NotImplementedError("Exphormer expander graphs (expander_degree > 0) are not on the HIP path")
    use_real = _use_real_edges_for_state(args, edge_budget_state, adaptive_edge_budget_cfg)
    use_rw = _use_rw_edges(args, edge_budget_state, adaptive_edge_budget_cfg)
    L = _resolve_walk_length(args, edge_budget_state, walk_length_override)
    P = int(getattr(args, "walks_per_node", 0))

    if not _random_block_sampling_enabled(args, adaptive_edge_budget_cfg):
        real = edge_index_global.to(dev) if use_real else None
        rw = None
        if use_rw:
            rw = _build_or_retrieve_full_rw_pool(args, edge_index_global, num_nodes, rw_device, L, P,
                                                 int(getattr(args, "num_heads", 1)), edge_seed).to(dev)
        if exphormer_rw:
            return _typed_edges(real, rw, dev).to(out_dev)
        merged = _merge_edge_index_list([x for x in (real, rw) if x is not None])
        if merged is None:
            merged = torch.zeros((2, 0), dtype=torch.long, device=dev)
        return (fix_edge_index(merged.to(torch.long), int(num_nodes)) if token else merged).to(out_dev)

    if use_rw and _rw_edge_mode(args) == "dgl_neighbor":
        # the fused builder walks; a fanout pool is ranked per query as the reference's pipeline does:
        # real part and RW part each by the edge key, then merged (utils/fullgraph_sp_support.py:2943-3026)
        real = _resolve_real_edges_for_state(args, edge_index_global, dev, edge_seed, edge_budget_state,
                                             adaptive_edge_budget_cfg)
        pool = _build_or_retrieve_full_rw_pool(args, edge_index_global, num_nodes, rw_device, L, P,
                                               int(getattr(args, "num_heads", 1)), edge_seed)
        rw = _resolve_rw_edges_for_state(args, pool.to(dev), edge_seed, edge_budget_state, adaptive_edge_budget_cfg)
        if exphormer_rw:
            return _typed_edges(real, rw, dev).to(out_dev)
        merged = _merge_edge_index_list([x for x in (real, rw) if x is not None])
        if merged is None:
            merged = torch.zeros((2, 0), dtype=torch.long, device=dev)
        return (fix_edge_index(merged.to(torch.long), int(num_nodes)) if token else merged).to(out_dev)

    b_r = _get_real_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg) if use_real else 0
    b_w = _get_rw_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg) if use_rw else 0
    base = getattr(args, "seed", 0) if edge_seed is None else int(edge_seed)
    graph = _graph_for(edge_index_global, num_nodes, dev)
    if exphormer_rw:
        parts = []
        for br, bw in ((b_r, 0), (0, b_w)):
            if br + bw > 0:
                parts.append(build_attention_edges(graph, real_edges_per_query=br, rw_edges_per_query=bw,
                                                   walk_length=L, walks_per_node=max(P, 1),
                                                   edge_seed=int(base)).to_edge_index())
            else:
                parts.append(None)
        return _typed_edges(parts[0], parts[1], dev).to(out_dev)
    if b_r <= 0 and b_w <= 0:
        empty = torch.zeros((2, 0), dtype=torch.long, device=dev)
        return (fix_edge_index(empty, int(num_nodes)) if token else empty).to(out_dev)
    table = build_attention_edges(graph, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                  walks_per_node=max(P, 1), edge_seed=int(base), global_token=token)
    return table.to_edge_index().to(out_dev)


# ------------------------------------------------------------------ topology ingest
def _to_bidirected_edge_index(edge_index: torch.Tensor, num_nodes: int) -> torch.Tensor:
    """utils/fullgraph_sp_support.py:570-572 on the device (``budgetformer_amd.graph.to_bidirected``)."""
    from ..graph import to_bidirected
    out_dev = edge_index.device
    return to_bidirected(edge_index.to(_hip_device(out_dev)), int(num_nodes)).to(out_dev)


def _torch_load_cpu(path: str):
    """utils/fullgraph_sp_support.py:690-715, restricted to the loads that execute nothing from the
    file (``weights_only=True``, with and without mmap)."""
    try:
        return torch.load(path, map_location="cpu", weights_only=True, mmap=True)
    except RuntimeError:
        return torch.load(path, map_location="cpu", weights_only=True)


# ------------------------------------------------------------------ per-epoch entry, merged-edge cache
def _resolve_edge_policy(args, edge_index_global=None, edge_policy=None) -> str:
    """utils/fullgraph_sp_support.py:379-391."""
    policy = edge_policy
    if policy is None:
        policy = getattr(args, "_runtime_edge_policy", None)
    if policy is None:
        policy = EDGE_POLICY_GPU_PERSIST if (edge_index_global is not None and edge_index_global.device.type == "cuda") \
            else EDGE_POLICY_GPU_EPHEMERAL
    policy = str(policy)
    if policy not in _EDGE_POLICY_CHOICES:
        raise ValueError(f"Unsupported edge policy: {policy!r}")
    return policy


def _edge_policy_build_devices(edge_policy: str, device, rw_device):
    """utils/fullgraph_sp_support.py:394-402: (final device, walk device) of a policy."""
    if edge_policy not in _EDGE_POLICY_CHOICES:
        raise ValueError(f"Unsupported edge policy: {edge_policy!r}")
    if edge_policy in (EDGE_POLICY_CPU_BROADCAST, EDGE_POLICY_CPU_BROADCAST_PREFETCH):
        return torch.device("cpu"), torch.device("cpu")
    if edge_policy == EDGE_POLICY_CPU_RANK_LOCAL_PREFETCH:
        return torch.device(device), torch.device("cpu")
    return torch.device(device), torch.device(rw_device)


def _make_merged_edge_cache_key(args, edge_index_global, num_nodes, rw_build_device, resolved_policy,
                                nodes_per_rank, edge_seed, edge_budget_state, adaptive_edge_budget_cfg,
                                walk_length_override) -> tuple:
    """utils/fullgraph_sp_support.py:3066-3096."""
    return (int(edge_seed), int(_get_real_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg)),
            int(_get_rw_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg)),
            int(_resolve_walk_length(args, edge_budget_state, walk_length_override)),
            int(getattr(args, "walks_per_node", 2)), str(rw_build_device), str(resolved_policy), int(nodes_per_rank),
            int(num_nodes), id(edge_index_global), int(getattr(args, "num_heads", 1)), str(getattr(args, "model", "")),
            int(getattr(args, "num_global_node", 0)))


def _store_merged_edge_cache(key: tuple, merged: torch.Tensor) -> None:
    """utils/fullgraph_sp_support.py:3099-3114: two-slot FIFO. The entry stays in HBM (288 GB per
    GPU holds a few merged edge lists easily) instead of the reference's host copy."""
    if len(_MERGED_EDGE_CACHE) >= 2:
        _MERGED_EDGE_CACHE.pop(next(iter(_MERGED_EDGE_CACHE)))
    _MERGED_EDGE_CACHE[key] = merged


def clear_merged_edge_cache() -> None:
    """utils/fullgraph_sp_support.py:3117-3119."""
    _MERGED_EDGE_CACHE.clear()


def _single_rank(sp_group) -> bool:
    import torch.distributed as dist
    if not (dist.is_available() and dist.is_initialized()):
        return True
    return dist.get_world_size(sp_group) == 1


def _build_and_broadcast_edges(args, edge_index_global, num_nodes, device, rw_device, sp_group, sp_src_rank,
                               sp_rank, nodes_per_rank, edge_seed=None, edge_budget_state=None,
                               adaptive_edge_budget_cfg=None, walk_length_override=None, edge_policy=None,
                               force_broadcast=None):
    """utils/fullgraph_sp_support.py:3171-3338 for one rank: build (or reuse the cached build of)
    the merged edges. With a fixed ``edge_seed`` the result is cached under the reference's key."""
    _ = (sp_src_rank, sp_rank, force_broadcast)
    if not _single_rank(sp_group):
        raise NotImplementedError("sequence-parallel edge broadcast (more than one rank) is not built")
    policy = _resolve_edge_policy(args, edge_index_global, edge_policy)
    final_dev, rw_dev = _edge_policy_build_devices(policy, device, rw_device)
    key = None
    if edge_seed is not None:
        key = _make_merged_edge_cache_key(args, edge_index_global, num_nodes, rw_dev, policy, nodes_per_rank,
                                          edge_seed, edge_budget_state, adaptive_edge_budget_cfg,
                                          walk_length_override)
        hit = _MERGED_EDGE_CACHE.get(key)
        if hit is not None:
            return hit.to(torch.device(device))
    merged = _build_merged_edges(args, edge_index_global, num_nodes, final_dev, rw_dev, nodes_per_rank,
                                 edge_seed=edge_seed, edge_budget_state=edge_budget_state,
                                 adaptive_edge_budget_cfg=adaptive_edge_budget_cfg,
                                 walk_length_override=walk_length_override)
    if key is not None:
        _store_merged_edge_cache(key, merged)
    return merged.to(torch.device(device))


def _build_attention_edges(args, edge_index_global, num_nodes, device, rw_device, sp_group, sp_src_rank, sp_rank,
                           nodes_per_rank, edge_seed=None, edge_budget_state=None, adaptive_edge_budget_cfg=None,
                           walk_length_override=None, edge_policy=None, force_broadcast=None):
    """utils/fullgraph_sp_support.py:3341-3362: the per-epoch edge entry point."""
    return _build_and_broadcast_edges(args, edge_index_global, num_nodes, device, rw_device, sp_group, sp_src_rank,
                                      sp_rank, nodes_per_rank, edge_seed=edge_seed,
                                      edge_budget_state=edge_budget_state,
                                      adaptive_edge_budget_cfg=adaptive_edge_budget_cfg,
                                      walk_length_override=walk_length_override, edge_policy=edge_policy,
                                      force_broadcast=force_broadcast)


# ------------------------------------------------------------------ Adaptive-Budget probe
def _expand_probe_idx_for_reception(probe_idx_global, edge_index_global, n_layers, edge_index_csr=None):
    """utils/fullgraph_sp_support.py:2261-2309 as a device BFS (``budgetformer_amd.probe.reception_cone``);
    returns host int64 ids like the reference."""
    _ = edge_index_csr
    if n_layers <= 1 or probe_idx_global is None or probe_idx_global.numel() == 0 or edge_index_global.numel() == 0:
        return probe_idx_global
    dev = _hip_device(edge_index_global.device)
    n = int(edge_index_global.max().item()) + 1
    graph = _graph_for(edge_index_global, n, dev)
    return reception_cone(graph, probe_idx_global.to(dev), int(n_layers)).cpu()


def _filter_edge_index_by_dst(edge_index, dst_nodes):
    """utils/fullgraph_sp_support.py:1520-1533."""
    if edge_index is None or dst_nodes is None or edge_index.numel() == 0:
        return edge_index
    dst_nodes = dst_nodes.to(device=edge_index.device, dtype=torch.long).view(-1)
    if dst_nodes.numel() == 0:
        return edge_index.new_zeros((edge_index.size(0), 0))
    mask = torch.isin(edge_index[1].to(torch.long), dst_nodes)
    return edge_index[:, mask]


def _subtract_edge_index(a, b, num_nodes):
    """utils/fullgraph_sp_support.py:1536-1551: drop entries of a whose (src, dst) pair is in b."""
    if a is None or a.numel() == 0 or b is None or b.numel() == 0:
        return a
    n = max(1, int(num_nodes))
    b = b.to(a.device)
    keep = ~torch.isin(a[0].to(torch.long) * n + a[1].to(torch.long), b[0].to(torch.long) * n + b[1].to(torch.long))
    return a if bool(keep.all()) else a[:, keep].contiguous()


def _compute_sorted_edge_keys(edges, num_nodes):
    """utils/fullgraph_sp_support.py:1555-1567."""
    if edges is None or edges.numel() == 0:
        return None
    n = max(1, int(num_nodes))
    return (edges[0].to(torch.long) * n + edges[1].to(torch.long)).sort()[0]


def _subtract_edge_index_sorted(a, b_keys_sorted, num_nodes):
    """utils/fullgraph_sp_support.py:1570-1591."""
    if a is None or a.numel() == 0 or b_keys_sorted is None or b_keys_sorted.numel() == 0:
        return a
    n = max(1, int(num_nodes))
    b_keys_sorted = b_keys_sorted.to(a.device)
    a_keys = a[0].to(torch.long) * n + a[1].to(torch.long)
    pos = torch.searchsorted(b_keys_sorted, a_keys).clamp(max=b_keys_sorted.numel() - 1)
    keep = b_keys_sorted[pos] != a_keys
    return a if bool(keep.all()) else a[:, keep].contiguous()


def _build_probe_edge_pools(args, edge_index_global, num_nodes, rw_device, probe_idx_global, edge_seed=None,
                            adaptive_edge_budget_cfg=None, walk_length_override=None, edge_index_csr=None,
                            edge_dst_filter=None, precomputed_real_pool=None,
                            precomputed_real_pool_sorted_keys=None):
    """utils/fullgraph_sp_support.py:1743-1821: the probe's materialised pools {"real", "rw"} (on the
    HIP device). The fused path that never materialises them is ``budgetformer_amd.probe.build_probe``."""
    _ = edge_index_csr
    dev = _hip_device(rw_device)
    dst = (edge_dst_filter if edge_dst_filter is not None else probe_idx_global).to(dev, torch.long).view(-1)
    real = None
    if _use_real_edges(args, adaptive_edge_budget_cfg):
        real = precomputed_real_pool.to(dev) if precomputed_real_pool is not None else \
            _filter_edge_index_by_dst(edge_index_global.to(dev), dst)
    rw = None
    if _use_rw_edges(args, adaptive_edge_budget_cfg=adaptive_edge_budget_cfg):
        wl = _resolve_walk_length(args, walk_length_override=walk_length_override)
        pool = _build_or_retrieve_full_rw_pool(args, edge_index_global, num_nodes, rw_device, wl,
                                               getattr(args, "walks_per_node", 2), getattr(args, "num_heads", 1),
                                               edge_seed)
        rw = _filter_edge_index_by_dst(pool.to(dev), dst)
        if rw is not None and rw.numel() > 0 and real is not None and real.numel() > 0:
            rw = _subtract_edge_index_sorted(rw, precomputed_real_pool_sorted_keys, num_nodes) \
                if precomputed_real_pool_sorted_keys is not None else _subtract_edge_index(rw, real, num_nodes)
    return {"real": real, "rw": rw}


def _sample_random_edge_blocks_with_state(args, real_edges, rw_edges, edge_seed=None, edge_budget_state=None,
                                          adaptive_edge_budget_cfg=None):
    """utils/fullgraph_sp_support.py:1268-1309: a zero budget drops that pool."""
    if not _random_block_sampling_enabled(args, adaptive_edge_budget_cfg):
        return real_edges, rw_edges
    b_r = _get_real_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg)
    b_w = _get_rw_edge_budget(args, edge_budget_state, adaptive_edge_budget_cfg)
    if real_edges is not None:
        real_edges = _sample_edges_per_query_random(real_edges, b_r, _edge_block_seed(args, edge_seed, 17)) \
            if b_r > 0 else None
    if rw_edges is not None:
        rw_edges = _sample_edges_per_query_random(rw_edges, b_w, _edge_block_seed(args, edge_seed, 37)) \
            if b_w > 0 else None
    return real_edges, rw_edges


def _assemble_edges_from_pools(args, edge_pools, num_nodes, nodes_per_rank, edge_seed=None, edge_budget_state=None,
                               adaptive_edge_budget_cfg=None):
    """utils/fullgraph_sp_support.py:1824-1879: one candidate from the shared pools."""
    _ = nodes_per_rank
    real, rw = _sample_random_edge_blocks_with_state(args, edge_pools.get("real"), edge_pools.get("rw"),
                                                     edge_seed=edge_seed, edge_budget_state=edge_budget_state,
                                                     adaptive_edge_budget_cfg=adaptive_edge_budget_cfg)
    template = edge_pools.get("real") if edge_pools.get("real") is not None else edge_pools.get("rw")
    dev = template.device if template is not None else torch.device("cpu")
    if getattr(args, "model", None) in _EXPHORMER_MODELS and int(getattr(args, "expander_degree", 0)) <= 0:
        return _typed_edges(real, rw, dev).contiguous()
    merged = _merge_edge_index_list([x for x in (real, rw) if x is not None and x.numel() > 0])
    if merged is None:
        merged = torch.zeros((2, 0), dtype=torch.long, device=dev)
    if getattr(args, "model", None) in _GRAPHORMER_VIRTUAL_NODE_MODELS and int(getattr(args, "num_global_node", 0)) > 0:
        merged = fix_edge_index(merged.to(torch.long), int(num_nodes))
    return merged.contiguous()


def _build_probe_attention_edges(args, edge_index_global, num_nodes, device, rw_device, sp_group, sp_src_rank,
                                 sp_rank, nodes_per_rank, probe_idx_global, edge_seed=None, edge_budget_state=None,
                                 adaptive_edge_budget_cfg=None, edge_pools=None, walk_length_override=None,
                                 edge_dst_filter=None):
    """utils/fullgraph_sp_support.py:1885-1934 for one rank."""
    _ = (sp_src_rank, sp_rank)
    if not _single_rank(sp_group):
        raise NotImplementedError("sequence-parallel probe broadcast (more than one rank) is not built")
    pools = edge_pools
    if pools is None:
        pools = _build_probe_edge_pools(args, edge_index_global, num_nodes, rw_device, probe_idx_global,
                                        edge_seed=edge_seed, adaptive_edge_budget_cfg=adaptive_edge_budget_cfg,
                                        walk_length_override=_resolve_walk_length(args, edge_budget_state,
                                                                                  walk_length_override),
                                        edge_dst_filter=edge_dst_filter)
    merged = _assemble_edges_from_pools(args, pools, num_nodes, nodes_per_rank, edge_seed=edge_seed,
                                        edge_budget_state=edge_budget_state,
                                        adaptive_edge_budget_cfg=adaptive_edge_budget_cfg)
    return merged.to(torch.device(device))
