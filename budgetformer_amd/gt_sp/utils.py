"""Edge-build device planning for MI355X (gt_sp/utils.py:160-487, gt_sp/multi_tier.py:851-875).

The reference estimates the transient working set of a torch_cluster walk plus
its Python hop loop (``_estimate_rw_working_set_bytes``, gt_sp/utils.py:160-236:
a 6·E·8-byte COO sort, an [N·P, L+1] int64 walk tensor and a [2, N·P·L] pool)
and moves the whole build to the CPU when it does not fit (``_safe_rw_device``,
:453-487; sticky OOM fallback :1200-1230).

The fused HIP builder never materialises walks or a pool: per query it keeps
the RW selection (4·b_rw bytes + a count) and writes its table row. Its
transient is therefore ``n_q · 4 · (b_rw + 1)`` bytes on top of the resident
topology and the output table, and the same names below answer the same
questions for it. Where the reference would fall back to the CPU, this
planner instead cuts the query range into shards whose transient fits: every
shard draws exactly the walks a single build draws (the Philox counter is the
global walk id), so the table is bit-identical. There is no CPU path.
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass
from typing import List, Tuple

import torch

_GPU_PROCESS_MEMORY_CAP_BYTES: int = 0
_FORCE_RW_ON_GPU: bool = False
_RW_DEVICE_DECISION_CACHE: dict = {}

# The library aligns each workspace slab to 256 bytes and adds one guard slab.
_WS_ALIGN = 256


def _align(x: int) -> int:
    return (int(x) + _WS_ALIGN - 1) // _WS_ALIGN * _WS_ALIGN


def set_rw_gpu_memory_cap(cap_bytes: int) -> None:
    """Register a per-process HBM cap (gt_sp/utils.py:262-270); 0 disables it."""
    global _GPU_PROCESS_MEMORY_CAP_BYTES
    _GPU_PROCESS_MEMORY_CAP_BYTES = max(0, int(cap_bytes))


def set_force_rw_on_gpu(value: bool) -> None:
    """Planner override (gt_sp/utils.py:282-290): treat the build as fitting."""
    global _FORCE_RW_ON_GPU
    _FORCE_RW_ON_GPU = bool(value)


def _clear_rw_device_cache() -> None:
    _RW_DEVICE_DECISION_CACHE.clear()


def estimate_edge_build_bytes(n_queries: int, real_edges_per_query: int, rw_edges_per_query: int) -> dict:
    """Exact device bytes of one fused build over ``n_queries`` queries.

    transient: the RW selection [n_q, b_rw] int32 + counts [n_q] int32 (the
    build's workspace, bf_build_edge_table_workspace_size); output: the table
    [n_q, b_real+b_rw] int32 + row_len [n_q] int32.
    """
    n = max(0, int(n_queries))
    b_r, b_w = max(0, int(real_edges_per_query)), max(0, int(rw_edges_per_query))
    transient = _align(n * b_w * 4) + _align(n * 4) + _WS_ALIGN
    output = n * (b_r + b_w) * 4 + n * 4
    return {"transient": int(transient), "output": int(output), "per_query_transient": 4 * (b_w + 1)}


def estimate_attention_index_bytes(n_q: int, n_kv: int, nnz: int, chunk: int = 64, item: int = 512) -> int:
    """Device bytes of an attention index: CSR, reverse index and both split plans
    (plus the reverse-index sort workspace, the largest transient)."""
    csr = 8 * (n_q + 1) + 4 * nnz
    reverse = 8 * (n_kv + 1) + 8 * nnz
    sort_ws = 3 * _align(4 * nnz) + 2 * 4 * nnz + _WS_ALIGN     # keys/values/rows slabs + radix temp
    plans = 4 * 2 * (n_q + n_kv) + 4 * 2 * (nnz // item + nnz // chunk + 1)
    return int(csr + reverse + sort_ws + plans)


def _estimate_rw_working_set_bytes(num_nodes: int, num_edges: int, walks_per_node: int, walk_length: int,
                                   num_heads: int = 1) -> int:
    """Transient bytes of an all-node fused build (gt_sp/utils.py:160-236 counterpart).

    The RW budget is at most the pool size per query (P·L, the cap used by
    _resolve_adaptive_edge_budget_config, utils/fullgraph_sp_support.py:949-952),
    so this bounds any budget state. ``num_edges`` and ``num_heads`` do not enter:
    the topology is read in place and heads share one edge set.
    """
    _ = (num_edges, num_heads)
    b_w_max = max(1, int(walks_per_node)) * max(1, int(walk_length))
    return estimate_edge_build_bytes(max(1, int(num_nodes)), 0, b_w_max)["transient"]


def _gpu_concurrent_overhead_bytes(device) -> int:
    """Per-process runtime overhead kept free (gt_sp/utils.py:367-399): HIP runtime,
    rocBLAS/hipBLASLt handles and workspaces, kernel code objects. 512 MiB."""
    try:
        dev = torch.device(device)
    except (TypeError, RuntimeError):
        return 0
    if dev.type != "cuda" or not torch.cuda.is_available():
        return 0
    return 512 * 1024 * 1024


def _expandable_segments_enabled() -> bool:
    conf = os.environ.get("PYTORCH_CUDA_ALLOC_CONF", "") + os.environ.get("PYTORCH_HIP_ALLOC_CONF", "")
    return "expandable_segments:True" in conf or "expandable_segments:true" in conf


def _rw_gpu_usable_bytes(device) -> int:
    """Bytes usable for the build on ``device`` (gt_sp/utils.py:402-447): driver free
    (+ the caching allocator's reserved slack when segments are expandable and
    the driver still has >= 256 MiB), clamped to a registered cap's headroom,
    minus the runtime overhead. -1 when no HIP device applies."""
    try:
        dev = torch.device(device)
    except (TypeError, RuntimeError):
        return -1
    if dev.type != "cuda" or not torch.cuda.is_available():
        return -1
    try:
        free, _ = torch.cuda.mem_get_info(dev)
    except (RuntimeError, AttributeError):
        return -1
    if _expandable_segments_enabled() and int(free) >= 256 * 1024 * 1024:
        free += max(0, torch.cuda.memory_reserved(dev) - torch.cuda.memory_allocated(dev))
    if _GPU_PROCESS_MEMORY_CAP_BYTES > 0:
        free = min(int(free), max(0, _GPU_PROCESS_MEMORY_CAP_BYTES - torch.cuda.memory_reserved(dev)))
    return max(0, int(free) - _gpu_concurrent_overhead_bytes(dev))


def _gpu_can_fit_rw(device, need_bytes: int) -> bool:
    """True iff ``need_bytes`` fits the usable budget (gt_sp/utils.py:430-448)."""
    if _FORCE_RW_ON_GPU:
        try:
            if torch.device(device).type == "cuda" and torch.cuda.is_available():
                return True
        except (TypeError, RuntimeError):
            pass
    usable = _rw_gpu_usable_bytes(device)
    if usable < 0:
        return True
    return int(need_bytes) <= usable


@dataclass
class EdgeBuildPlan:
    """How one edge build runs: always on the HIP device, in ``len(shards)`` query shards."""
    device: torch.device
    shards: List[Tuple[int, int]]          # (q_lo, n_q) per shard, covering [q_lo0, q_lo0 + n_q_total)
    transient_bytes: int                   # per-shard transient of the largest shard
    output_bytes: int                      # the whole table
    usable_bytes: int                      # budget the plan was made against (-1: unknown)


_SMALL_BUILD_BYTES = 64 * 1024 * 1024


def plan_edge_build(device, n_queries: int, real_edges_per_query: int, rw_edges_per_query: int, q_lo: int = 0,
                    usable_bytes: int = None) -> EdgeBuildPlan:
    """Shard the query range so each shard's transient fits next to the output table.

    Raises torch.cuda.OutOfMemoryError when not even the output table plus a
    one-query shard fits: there is no CPU build to fall back to.
    """
    dev = torch.device(device)
    full = estimate_edge_build_bytes(n_queries, real_edges_per_query, rw_edges_per_query)
    if usable_bytes is None and _GPU_PROCESS_MEMORY_CAP_BYTES <= 0 and \
            full["transient"] + full["output"] <= _SMALL_BUILD_BYTES:
        # too small to be worth sharding: one build, without querying the driver's free memory
        # (a shortfall this small surfaces as the allocator's own OutOfMemoryError)
        return EdgeBuildPlan(dev, [(q_lo, n_queries)], full["transient"], full["output"], -1)
    usable = _rw_gpu_usable_bytes(dev) if usable_bytes is None else int(usable_bytes)
    if usable < 0 or _FORCE_RW_ON_GPU or full["transient"] + full["output"] <= usable:
        return EdgeBuildPlan(dev, [(q_lo, n_queries)], full["transient"], full["output"], usable)
    room = usable - full["output"] - 2 * _WS_ALIGN
    per_q = full["per_query_transient"]
    if room < per_q:
        raise torch.cuda.OutOfMemoryError(
            f"edge build: the output table needs {full['output'] / 2**20:.0f} MiB and the usable HBM is "
            f"{usable / 2**20:.0f} MiB; no query shard fits")
    shard = max(1, room // per_q)
    n_shards = math.ceil(n_queries / shard)
    shard = math.ceil(n_queries / n_shards)
    shards = [(q_lo + i * shard, min(shard, n_queries - i * shard)) for i in range(n_shards)]
    key = ("plan_edge_build", str(dev), int(n_queries), len(shards))
    if key not in _RW_DEVICE_DECISION_CACHE and _rank0():
        print(f"[rw-device] edge build transient {full['transient'] / 2**20:.0f} MiB + table "
              f"{full['output'] / 2**20:.0f} MiB exceeds the usable {usable / 2**20:.0f} MiB; building on "
              f"{dev} in {len(shards)} query shards of <= {shard:,} (bit-identical to one build).")
    _RW_DEVICE_DECISION_CACHE[key] = (full["transient"], usable)
    return EdgeBuildPlan(dev, shards, estimate_edge_build_bytes(shard, real_edges_per_query,
                                                                rw_edges_per_query)["transient"],
                         full["output"], usable)


def _safe_rw_device(rw_dev, args, num_nodes: int, num_edges: int):
    """Device for the walk build (gt_sp/utils.py:453-487): the HIP device whenever one is
    requested — a build that does not fit whole is sharded by ``plan_edge_build``
    instead of being moved to the CPU."""
    requested = torch.device(rw_dev)
    if requested.type != "cuda":
        raise ValueError("the MI355X edge builder runs on a HIP device; there is no CPU build")
    return requested


def _rank0() -> bool:
    try:
        import torch.distributed as dist
        return not dist.is_available() or not dist.is_initialized() or dist.get_rank() == 0
    except Exception:
        return True


# ---------------------------------------------------------------------------
# The walk / pool / merge seams of gt_sp/utils.py on the HIP kernels.
# ---------------------------------------------------------------------------
_RANDOM_WALK_GRAPH_CACHE: dict = {}


def _draw_walk_seed() -> int:
    """A walk seed drawn from torch's CPU generator, as the DGL branch does
    (gt_sp/utils.py:1409-1410), so ``fixed_random_seed(edge_seed)`` makes it
    reproducible while consecutive calls still differ."""
    return int(torch.randint(0, 2 ** 63 - 1, (1,), dtype=torch.int64).item())


def _get_random_walk_graph(edge_index: torch.Tensor, num_nodes: int, device):
    """(placeholder, rowptr int64, col int32) coalesced CSR of ``edge_index`` rows on ``device``
    (gt_sp/utils.py:890-936); cached per (tensor, E, N, device)."""
    from .. import hip_ops
    dev = torch.device(device)
    key = (int(edge_index.data_ptr()), int(edge_index.size(1)), int(num_nodes), dev.type, dev.index)
    hit = _RANDOM_WALK_GRAPH_CACHE.get(key)
    # the entry pins its source tensor, so a hit is the same tensor (same version), not a reused address
    if hit is not None and hit[0] is edge_index and hit[1] == edge_index._version:
        return hit[2]
    ei = hip_ops.coalesce(edge_index.to(dev), num_nodes)
    rowptr, col = hip_ops.coo_to_csr(torch.stack([ei[1], ei[0]]), num_nodes, num_nodes)
    placeholder = torch.empty((2, 0), dtype=edge_index.dtype, device=dev)
    _RANDOM_WALK_GRAPH_CACHE.clear()
    _RANDOM_WALK_GRAPH_CACHE[key] = (edge_index, edge_index._version, (placeholder, rowptr, col))
    return _RANDOM_WALK_GRAPH_CACHE[key][2]


def _run_random_walk(edge_index, rowptr: torch.Tensor, col: torch.Tensor, starts: torch.Tensor, walk_length: int,
                     *, u: torch.Tensor = None, seed: int = None) -> torch.Tensor:
    """Uniform walks [len(starts), L+1] int64 from ``starts`` (gt_sp/utils.py:1387-1473).

    A dead end repeats the current node (the torch_cluster semantics the
    reference normalises DGL to, :1431-1439). ``u`` injects the uniforms;
    otherwise Philox draws them with ``seed`` (default: drawn from torch's CPU
    generator) and walk id = position in ``starts``.
    """
    from .. import hip_ops
    _ = edge_index
    col32 = col if col.dtype == torch.int32 else col.to(torch.int32)
    seed = _draw_walk_seed() if (seed is None and u is None) else (seed or 0)
    return hip_ops.random_walk_starts(rowptr.to(torch.int64).contiguous(), col32.contiguous(),
                                      starts.to(rowptr.device, torch.int64).contiguous(), int(walk_length), u=u,
                                      philox_seed=seed)


def compute_hop_buckets_random_walk(edge_index: torch.Tensor, num_nodes: int, num_buckets: int, device="cuda",
                                    walk_length: int = 4, walks_per_node: int = 2, min_hop: int = 1, *,
                                    u: torch.Tensor = None, seed: int = None):
    """Hop buckets of uniform walks from every node (gt_sp/utils.py:1074-1248), on the device.

    Only ``num_buckets == 1`` (the path's setting, :1251-1278) is supported.
    """
    num_buckets = max(1, int(num_buckets))
    if num_buckets != 1:
        raise NotImplementedError("only a single hop bucket is on the edge-construction path")
    walk_length, walks_per_node, min_hop = max(1, int(walk_length)), max(1, int(walks_per_node)), max(1, int(min_hop))
    if edge_index.numel() == 0:
        return [edge_index.new_zeros((2, 0))]
    num_nodes = max(int(num_nodes), int(edge_index.max().item()) + 1)
    dev = _safe_rw_device(device, None, num_nodes, int(edge_index.size(1)))
    placeholder, rowptr, col = _get_random_walk_graph(edge_index, num_nodes, dev)
    starts = torch.arange(num_nodes, device=dev, dtype=torch.int64).repeat_interleave(walks_per_node)
    walks = _run_random_walk(placeholder, rowptr, col, starts, walk_length, u=u, seed=seed)
    from .. import hip_ops
    return [hip_ops.hop_pool(walks, min_hop)]


def build_head_hop_edges(edge_index: torch.Tensor, num_nodes: int, num_heads: int, num_groups: int, device="cuda",
                         walk_length: int = 4, walks_per_node: int = 2, min_hop: int = 1, *, u=None, seed=None):
    """One shared RW pool [2, M] (gt_sp/utils.py:1251-1278)."""
    _ = (num_heads, num_groups)
    return compute_hop_buckets_random_walk(edge_index, num_nodes, 1, device, walk_length, walks_per_node, min_hop,
                                           u=u, seed=seed)[0]


def compute_khop_pool_dgl_neighbor(edge_index: torch.Tensor, num_nodes: int, fanout: List[int], device="cpu",
                                   min_hop: int = 1, seed: int = None) -> torch.Tensor:
    """Fanout k-hop pool (gt_sp/utils.py:1281-1384) on the HIP device: hop d samples up to fanout[d-1]
    out-neighbours of each frontier node (-1: all of them), one sample per node and hop shared by every
    frontier entry at that node, and from ``min_hop`` on emits (neighbour -> origin query) pairs, self pairs
    dropped. Returns [2, E] int64 on ``device`` (row 0 key/value node, row 1 query), hop-major.

    Parallel edges stay separate edges, as in ``dgl.graph``. DGL's sampler RNG is not reproduced: Philox
    keyed by ``seed`` (default: drawn from torch's generator, as the walk seed is) defines the samples."""
    from .. import hip_ops
    out_dev = torch.device(device)
    k = len(fanout)
    if edge_index.numel() == 0 or k == 0:
        return torch.zeros((2, 0), dtype=torch.long, device=out_dev)
    dev = out_dev if out_dev.type == "cuda" else torch.device("cuda", torch.cuda.current_device())
    n = max(int(num_nodes), int(edge_index.max().item()) + 1)
    ei = edge_index.to(dev)
    rowptr, col = hip_ops.coo_to_csr(torch.stack([ei[1], ei[0]]), n, n)     # out-neighbour CSR
    seed = _draw_walk_seed() if seed is None else int(seed)
    return hip_ops.khop_fanout_pool(rowptr, col, [int(f) for f in fanout], seed=seed,
                                    min_hop=int(min_hop)).to(out_dev)


def _merge_edge_index_list(edge_list):
    """Merge edge lists (gt_sp/utils.py:877-887): >= 2 non-empty parts are concatenated and
    coalesced on the device; a single part passes through; none returns the first entry."""
    from .. import hip_ops
    tensors = [e for e in edge_list if e is not None and e.numel() > 0]
    if not tensors:
        return edge_list[0] if edge_list else None
    if len(tensors) == 1:
        return tensors[0]
    device = tensors[0].device
    ei = torch.cat([t.to(device) for t in tensors], dim=1).to(torch.long)
    n = int(ei.max().item()) + 1
    return hip_ops.coalesce(ei, n)


def fix_edge_index(x: torch.Tensor, num_node: int) -> torch.Tensor:
    """Graphormer virtual node 0 (gt_sp/utils.py:113-130): ids + 1, then (v+1 -> 0) and (0 -> v+1)."""
    ar = torch.arange(1, num_node + 1, device=x.device, dtype=x.dtype)
    zeros = torch.zeros(num_node, device=x.device, dtype=x.dtype)
    return torch.cat([x + 1, torch.stack([ar, zeros]), torch.stack([zeros, ar])], dim=1)
