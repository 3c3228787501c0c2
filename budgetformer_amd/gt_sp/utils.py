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

import functools
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


_ALLOC_ROUND = 512     # the caching allocator rounds every block up to a multiple of 512 bytes


def _block(nbytes: int) -> int:
    """Bytes the caching allocator books for a tensor of ``nbytes`` (torch.empty(max(n, 1)) included)."""
    return max(1, -(-max(int(nbytes), 1) // _ALLOC_ROUND)) * _ALLOC_ROUND


def _ws_size(fn_name: str, *args) -> int:
    import ctypes as C
    from .. import _native as N
    out = C.c_size_t(0)
    N.call(fn_name, *args, C.byref(out))
    return int(out.value)


class _LiveSet:
    """Replays a sequence of device allocations and frees; ``peak`` is the largest live total."""

    def __init__(self):
        self.live, self.total, self.peak = {}, 0, 0

    def alloc(self, name: str, nbytes: int) -> None:
        b = _block(nbytes)
        self.live[name] = b
        self.total += b
        self.peak = max(self.peak, self.total)

    def free(self, *names: str) -> None:
        for n in names:
            self.total -= self.live.pop(n)


@functools.lru_cache(maxsize=64)
def estimate_hot_path_bytes(num_nodes: int, num_edges: int, n_q: int, real_edges_per_query: int,
                            rw_edges_per_query: int, *, global_token: bool = False, holds_token_row: bool = True,
                            nnz: int = None, entries: bool = False, n_hubs: int = 0, walk_records: bool = True,
                            chunk: int = 128, item: int = 768) -> dict:
    """Device bytes of one budgeted edge build and its attention index, by replaying the allocations
    ``build_attention_edges`` and ``EdgeTable.attention_index().ensure_backward(entries)`` make, with each
    workspace taken from the library's own size query (gt_sp/utils.py:160-236 and :1121-1165 estimate the
    reference's walk pipeline the same way: every transient it allocates).

    - ``walk_records``: the graph's walk records (16 bytes per edge), built once per graph and kept with
      it (``CSRGraph.walk_records``); reported apart, since a graph holds them across builds;
    - the build: the table [n_q, b_r + b_w] and row lengths, plus its workspace (the RW selection);
    - the index: row pointers, kv ids, the reverse-index sort keys (8 bytes per table entry) and their
      sorted copy, the sort's workspace, kptr / kq (/ ks with ``entries``), the query and key split plans,
      the key rows' order and spans. ``nnz``: the index's entry count when known (a table's index of more
      than 8M entries at capacity is sized exactly); None sizes it for every table row full, an upper
      bound.

    Returns the phases' peaks and ``peak`` (the largest live total over the build and the index, on top
    of what is resident before: graph, activations) and ``resident`` (what stays allocated after:
    table, row lengths and the index). Cached per argument set (a build asks once per call); the
    returned dict is shared, not to be modified."""
    from .. import _native as N
    from ..hip_ops import NO_READBACK_MAX_ENTRIES
    lib = N.load()
    n_q, N_ = int(n_q), int(num_nodes)
    b_r, b_w = max(0, int(real_edges_per_query)), max(0, int(rw_edges_per_query))
    width = max(1, b_r + b_w)
    tr = (N_ if holds_token_row else -1) if global_token else -1
    n_q_tab = n_q + (1 if tr >= 0 else 0)
    n_kv = N_ + (1 if global_token else 0)
    n_token = (n_q + max(tr, 0)) if global_token else 0
    bound = n_q * width + n_token
    exact = bound > NO_READBACK_MAX_ENTRIES
    entries_n = bound if (nnz is None or not exact) else int(nnz)
    n_keys = max(entries_n - n_token, 0)
    L = _LiveSet()
    # the build (one shard)
    L.alloc("table", 4 * n_q * width)
    L.alloc("row_len", 4 * n_q)
    L.alloc("build_ws", _ws_size("bf_build_edge_table_workspace_size", n_q, b_w, int(n_hubs), b_r))
    build_peak = L.peak
    L.free("build_ws")
    # AttentionIndex.from_table: row pointers (scan workspace), the query plan when the sizes fix it, kv, keys
    L.alloc("scan_ws", _ws_size("bf_scan_workspace_size", n_q_tab))
    L.alloc("qptr", 8 * (n_q_tab + 1))
    L.free("scan_ws")
    L.alloc("plan_counts", 16)
    known = width + (1 if global_token else 0) <= chunk
    q_item_cap = int(lib.bf_split_item_capacity(bound, chunk, item))
    q_heavy_cap = int(lib.bf_split_row_capacity(bound, chunk))
    q_plan = 4 * (2 * max(n_q_tab, 1) + max(q_item_cap, 1) + max(q_heavy_cap, 1))
    if known:
        L.alloc("q_plan", q_plan)
    L.alloc("kv", 4 * entries_n)
    L.alloc("keys", 8 * n_keys)
    if not known:                                  # split_plan over the capacity, with its workspace
        L.alloc("q_plan", q_plan)
        L.alloc("q_plan_ws", _ws_size("bf_split_plan_workspace_size", n_q_tab))
        L.free("q_plan_ws")
    # ensure_backward: the reverse index from the keys (one sort), then the key rows' order and plan
    L.alloc("rev_ws", _ws_size("bf_reverse_index_packed_workspace_size", entries_n))
    L.alloc("sorted_keys", 8 * n_keys)
    L.alloc("kptr", 8 * (n_kv + 1))
    L.alloc("kq", 4 * entries_n)
    if entries:
        L.alloc("ks", 4 * entries_n)
    L.free("rev_ws", "keys")
    k_item_cap = int(lib.bf_split_item_capacity(entries_n, chunk, item))
    k_heavy_cap = int(lib.bf_split_row_capacity(entries_n, chunk))
    L.alloc("k_order", 4 * max(n_kv, 1))
    L.alloc("k_spans", 8 * max(n_kv, 1))
    L.alloc("k_plan", 4 * (2 * max(n_kv, 1) + max(k_item_cap, 1) + max(k_heavy_cap, 1)))
    L.alloc("k_plan_ws", _ws_size("bf_row_order_and_plan_workspace_size", n_kv, k_heavy_cap))
    L.free("k_plan_ws")
    if entries:
        L.free("sorted_keys")     # the slots came with the unpack: the sorted keys go with the call
    return {"walk_records": 16 * int(num_edges) if walk_records else 0,
            "build_peak": build_peak, "peak": L.peak, "resident": L.total,
            "entries": entries_n, "exact": exact, "live_after": dict(L.live)}


def _estimate_rw_working_set_bytes(num_nodes: int, num_edges: int, walks_per_node: int, walk_length: int,
                                   num_heads: int = 1, real_edges_per_query: int = None,
                                   global_token: bool = False, walk_records_built: bool = False) -> int:
    """Working set of an all-node build and its attention index (gt_sp/utils.py:160-236 counterpart): the
    walk records when the graph has none yet, plus the peak of ``estimate_hot_path_bytes`` with every
    table row full. The RW budget is at most the pool size per query (P·L, the cap
    _resolve_adaptive_edge_budget_config uses, utils/fullgraph_sp_support.py:949-952), and so is the real
    budget unless given, which bounds any budget state. Heads share one edge set."""
    _ = num_heads
    b_w = max(1, int(walks_per_node)) * max(1, int(walk_length))
    b_r = b_w if real_edges_per_query is None else int(real_edges_per_query)
    est = estimate_hot_path_bytes(num_nodes, num_edges, num_nodes, b_r, b_w, global_token=global_token)
    return int(est["peak"] + (0 if walk_records_built else est["walk_records"]))


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
                    usable_bytes: int = None, reserve_bytes: int = 0) -> EdgeBuildPlan:
    """Shard the query range so each shard's transient fits next to the output table and ``reserve_bytes``
    (what the table's attention index will need beyond the table: ``estimate_hot_path_bytes``' peak less
    the table).

    Raises torch.cuda.OutOfMemoryError when not even the output table, the reserve and a one-query shard
    fit: there is no CPU build to fall back to.
    """
    dev = torch.device(device)
    full = estimate_edge_build_bytes(n_queries, real_edges_per_query, rw_edges_per_query)
    reserve = max(0, int(reserve_bytes))
    if usable_bytes is None and _GPU_PROCESS_MEMORY_CAP_BYTES <= 0 and \
            full["transient"] + full["output"] + reserve <= _SMALL_BUILD_BYTES:
        # too small to be worth sharding: one build, without querying the driver's free memory
        # (a shortfall this small surfaces as the allocator's own OutOfMemoryError)
        return EdgeBuildPlan(dev, [(q_lo, n_queries)], full["transient"], full["output"], -1)
    usable = _rw_gpu_usable_bytes(dev) if usable_bytes is None else int(usable_bytes)
    if usable < 0 or _FORCE_RW_ON_GPU or full["transient"] + full["output"] + reserve <= usable:
        return EdgeBuildPlan(dev, [(q_lo, n_queries)], full["transient"], full["output"], usable)
    room = usable - full["output"] - reserve - 2 * _WS_ALIGN
    per_q = full["per_query_transient"]
    if room < per_q:
        raise torch.cuda.OutOfMemoryError(
            f"edge build: the output table needs {full['output'] / 2**20:.0f} MiB and its attention index "
            f"{reserve / 2**20:.0f} MiB more, the usable HBM is {usable / 2**20:.0f} MiB; no query shard fits")
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
