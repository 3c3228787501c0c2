"""Tensor-level wrappers around the C ABI.

Each function takes device tensors, checks shapes/dtypes on the host, draws
scratch memory from PyTorch's caching allocator (so a failed allocation is a
``torch.cuda.OutOfMemoryError``) and enqueues the HIP kernels on the current
stream. PyTorch is used only for device memory and streams.
"""
from __future__ import annotations

import ctypes as C
import weakref
from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _native as N

DEFAULT_CHUNK = 128     # rows longer than this go through the split plan
DEFAULT_ITEM = 768      # entries per split item (one workgroup), before balancing
HUB_THRESHOLD = 1024    # in-degree above which a query's real-edge top-k uses a whole workgroup
LIGHT_MAX = 32          # in-degree up to which a query's real-edge top-k runs in one thread (k <= 16)


def _p(t: Optional[torch.Tensor]):
    return None if t is None else C.c_void_p(t.data_ptr())


def _u64(x: int) -> int:
    """A seed or offset as the uint64 the library takes (two's complement for negatives)."""
    return int(x) & (2 ** 64 - 1)


def _stream(device: torch.device):
    """The current HIP stream of ``device`` as a raw handle (what torch.cuda.current_stream(device).cuda_stream
    gives, without building a Stream object on every call). Every library call takes its stream from the
    device of its tensors, so a host tensor is refused here, before any pointer reaches a kernel."""
    if device.type != "cuda":
        raise ValueError(f"the HIP path takes device tensors (got tensors on {device}); it has no CPU fallback")
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return C.c_void_p(torch._C._cuda_getCurrentRawStream(idx))


def _require(t: torch.Tensor, name: str, dtype: torch.dtype, device: torch.device = None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a HIP device tensor (got {t.device}); the HIP path has no CPU fallback")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _size_query(fn_name: str, *args) -> int:
    out = C.c_size_t(0)
    N.call(fn_name, *args, C.byref(out))
    return int(out.value)


# ------------------------------------------------------------------ edge construction
def random_walk(rowptr, col, q_lo: int, n_q: int, walks_per_node: int, walk_length: int,
                u: Optional[torch.Tensor] = None, philox_seed: int = 0, philox_offset: int = 0) -> torch.Tensor:
    """Walks [n_q*P, L+1] int64 from queries [q_lo, q_lo+n_q) (bf_random_walk)."""
    dev = rowptr.device
    _require(rowptr, "rowptr", torch.int64)
    _require(col, "col", torch.int32, dev)
    if u is not None:
        _require(u, "u", torch.float32, dev)
        if tuple(u.shape) != (n_q * walks_per_node, walk_length):
            raise ValueError(f"u must be [{n_q * walks_per_node}, {walk_length}], got {tuple(u.shape)}")
    return N.load_ops().rw_walk(rowptr, col, q_lo, n_q, walks_per_node, walk_length, _i64(philox_seed),
                                _i64(philox_offset), u)


def random_walk_starts(rowptr, col, starts: torch.Tensor, walk_length: int, u: Optional[torch.Tensor] = None,
                       philox_seed: int = 0, philox_offset: int = 0, walk_id_base: int = 0) -> torch.Tensor:
    """Walks [len(starts), L+1] int64 from arbitrary start nodes (bf_random_walk_starts)."""
    dev = rowptr.device
    _require(rowptr, "rowptr", torch.int64)
    _require(col, "col", torch.int32, dev)
    _require(starts, "starts", torch.int64, dev)
    n = starts.numel()
    if n:
        lo, hi = int(starts.min().item()), int(starts.max().item())
        if lo < 0 or hi >= rowptr.numel() - 1:
            raise ValueError(f"starts outside [0, {rowptr.numel() - 1})")
    if u is not None:
        _require(u, "u", torch.float32, dev)
        if tuple(u.shape) != (n, walk_length):
            raise ValueError(f"u must be [{n}, {walk_length}], got {tuple(u.shape)}")
    walks = torch.empty(n, walk_length + 1, dtype=torch.int64, device=dev)
    N.call("bf_random_walk_starts", _p(rowptr), _p(col), rowptr.numel() - 1, _p(starts), n, walk_length, _p(u),
           philox_seed & (2 ** 64 - 1), philox_offset & (2 ** 64 - 1), walk_id_base & (2 ** 64 - 1), _p(walks),
           _stream(dev))
    return walks


def hop_pool(walks: torch.Tensor, min_hop: int = 1) -> torch.Tensor:
    """RW pool [2, M] int64 (kv, query) of a walk tensor, in the reference's d-major order."""
    dev = walks.device
    _require(walks, "walks", torch.int64)
    n, L = walks.shape[0], walks.shape[1] - 1
    cap = n * max(L - min_hop + 1, 0)
    out = torch.empty(2, max(cap, 1), dtype=torch.int64, device=dev)
    ws = _workspace(_size_query("bf_hop_pool_workspace_size", n, L, min_hop), dev)
    cnt = C.c_int64(0)
    N.call("bf_hop_pool", _p(walks), n, L, min_hop, C.c_void_p(out[0].data_ptr()), C.c_void_p(out[1].data_ptr()),
           C.byref(cnt), _p(ws), ws.numel(), _stream(dev))
    return out[:, : cnt.value]


MAX_FANOUT = 64          # largest sampled fanout (BF_MAX_FANOUT); -1 takes every neighbour at any degree


def fanout_sample(rowptr: torch.Tensor, col: torch.Tensor, fanout: int, hop: int, seed: int = 0, offset: int = 0):
    """Every node's hop-``hop`` sample of at most ``fanout`` out-neighbours (bf_fanout_sample):
    (cnt int32 [N], sel int32 [N, fanout])."""
    dev = rowptr.device
    _require(rowptr, "rowptr", torch.int64)
    _require(col, "col", torch.int32, dev)
    if not 1 <= int(fanout) <= MAX_FANOUT:
        raise ValueError(f"fanout {fanout} outside [1, {MAX_FANOUT}] (-1 takes every neighbour without a sample)")
    n = rowptr.numel() - 1
    cnt = torch.empty(max(n, 1), dtype=torch.int32, device=dev)[:n]
    sel = torch.empty(max(n * int(fanout), 1), dtype=torch.int32, device=dev)
    N.call("bf_fanout_sample", _p(rowptr), _p(col), n, int(fanout), int(hop), _u64(seed), _u64(offset), _p(cnt),
           _p(sel), _stream(dev))
    return cnt, sel[: n * int(fanout)].view(n, int(fanout))


def khop_fanout_pool(rowptr: torch.Tensor, col: torch.Tensor, fanout, seed: int = 0, offset: int = 0,
                     min_hop: int = 1) -> torch.Tensor:
    """Fanout k-hop pool [2, M] int64 (kv, query) over the out-CSR (rowptr, col): hop-major, then frontier
    order (compute_khop_pool_dgl_neighbor, gt_sp/utils.py:1281-1384). ``fanout``: one entry per hop, -1 for
    every neighbour; one host read per hop (the next frontier's size) and one per emitted hop."""
    dev = rowptr.device
    _require(rowptr, "rowptr", torch.int64)
    _require(col, "col", torch.int32, dev)
    n = rowptr.numel() - 1
    origin = torch.arange(n, dtype=torch.int32, device=dev)
    cur = origin.clone()
    parts = []
    for d, f in enumerate([int(x) for x in fanout], start=1):
        m = cur.numel()
        if m == 0 or f == 0:
            break
        if f < 0:
            ptr, cnt, ids, stride = rowptr, None, col, 0
        else:
            cnt, sel = fanout_sample(rowptr, col, f, d, seed, offset)
            ptr, ids, stride = None, sel.reshape(-1), f
        offs = torch.empty(m + 1, dtype=torch.int64, device=dev)
        ws = _workspace(_size_query("bf_frontier_offsets_workspace_size", m), dev)
        N.call("bf_frontier_offsets", _p(cur), m, _p(ptr), _p(cnt), _p(offs), _p(ws), ws.numel(), _stream(dev))
        total = int(offs[m].item())
        if total == 0:             # no frontier node has a successor: later hops are empty too
            break
        new_origin = torch.empty(total, dtype=torch.int32, device=dev)
        new_cur = torch.empty(total, dtype=torch.int32, device=dev)
        N.call("bf_frontier_expand", _p(origin), _p(cur), m, _p(offs), _p(ptr), _p(ids), stride, _p(new_origin),
               _p(new_cur), _stream(dev))
        origin, cur = new_origin, new_cur
        if d >= min_hop:
            out = torch.empty(2, total, dtype=torch.int64, device=dev)
            count = torch.zeros(1, dtype=torch.int64, device=dev)
            ws = _workspace(_size_query("bf_frontier_emit_workspace_size", total), dev)
            N.call("bf_frontier_emit", _p(origin), _p(cur), total, C.c_void_p(out[0].data_ptr()),
                   C.c_void_p(out[1].data_ptr()), _p(count), _p(ws), ws.numel(), _stream(dev))
            parts.append(out[:, : int(count.item())])
    if not parts:
        return torch.zeros((2, 0), dtype=torch.int64, device=dev)
    return torch.cat(parts, dim=1)


def coalesce(edge_index: torch.Tensor, num_nodes: int) -> torch.Tensor:
    """Sort by (src, dst) and drop duplicates (torch_geometric.utils.coalesce), on the device."""
    dev = edge_index.device
    src = edge_index[0].to(torch.int64).contiguous()
    dst = edge_index[1].to(torch.int64).contiguous()
    nnz = src.numel()
    out = torch.empty(2, max(nnz, 1), dtype=torch.int64, device=dev)
    ws = _workspace(_size_query("bf_coalesce_workspace_size", nnz), dev)
    cnt = C.c_int64(0)
    N.call("bf_coalesce", _p(src), _p(dst), nnz, num_nodes, C.c_void_p(out[0].data_ptr()),
           C.c_void_p(out[1].data_ptr()), C.byref(cnt), _p(ws), ws.numel(), _stream(dev))
    return out[:, : cnt.value]


def walk_uniforms(q_lo: int, n_q: int, walks_per_node: int, walk_length: int, philox_seed: int,
                  philox_offset: int = 0, device="cuda") -> torch.Tensor:
    """The Philox uniforms of the production walk as a [n_q*P, L] float32 tensor."""
    u = torch.empty(n_q * walks_per_node, walk_length, dtype=torch.float32, device=device)
    N.call("bf_walk_uniforms", q_lo, n_q, walks_per_node, walk_length, philox_seed & (2 ** 64 - 1),
           philox_offset & (2 ** 64 - 1), _p(u), _stream(u.device))
    return u


def walk_records(rowptr, col) -> torch.Tensor:
    """Per-edge walk records (bf_walk_records): int32 [E, 4] = (target, target degree, target row start
    low word, high word). With them a walk step reads one 16-byte record instead of the rowptr pair and
    col; the walks are the same. Topology only: build once per graph."""
    dev = rowptr.device
    _require(rowptr, "rowptr", torch.int64)
    _require(col, "col", torch.int32, dev)
    rec = torch.empty(col.numel(), 4, dtype=torch.int32, device=dev)
    N.call("bf_walk_records", _p(rowptr), _p(col), rowptr.numel() - 1, col.numel(), _p(rec), _stream(dev))
    return rec


def _walk_rec_arg(walk_rec, col, dev):
    if walk_rec is None:
        return None
    _require(walk_rec, "walk_rec", torch.int32, dev)
    if tuple(walk_rec.shape) != (col.numel(), 4):
        raise ValueError(f"walk_rec must be [{col.numel()}, 4] (got {tuple(walk_rec.shape)})")
    return _p(walk_rec)


def rw_select(rowptr, col, q_lo: int, n_q: int, walks_per_node: int, walk_length: int, k_rw: int,
              key_seed: int, u=None, philox_seed: int = 0, philox_offset: int = 0, walk_rec=None):
    """Per-query top-k_rw of the query's own walk pool: (sel_kv [n_q,k_rw], sel_cnt [n_q]).
    ``walk_rec``: ``walk_records(rowptr, col)``, or None to step through rowptr and col."""
    dev = rowptr.device
    _require(rowptr, "rowptr", torch.int64)
    _require(col, "col", torch.int32, dev)
    if u is not None:
        _require(u, "u", torch.float32, dev)
    sel = torch.empty(n_q, k_rw, dtype=torch.int32, device=dev)
    cnt = torch.empty(n_q, dtype=torch.int32, device=dev)
    N.call("bf_rw_select", _p(rowptr), _p(col), _walk_rec_arg(walk_rec, col, dev), rowptr.numel() - 1, q_lo, n_q,
           walks_per_node, walk_length, k_rw, key_seed, _p(u), philox_seed & (2 ** 64 - 1),
           philox_offset & (2 ** 64 - 1), _p(sel), _p(cnt), _stream(dev))
    return sel, cnt


def real_select_merge(in_ptr, in_src, q_lo: int, n_q: int, k_real: int, key_seed: int,
                      rw_kv=None, rw_cnt=None, k_rw: int = 0, dedup: bool = True, width: Optional[int] = None,
                      hubs: Optional[torch.Tensor] = None, hub_threshold: int = HUB_THRESHOLD,
                      heavy: Optional[torch.Tensor] = None, light_max: int = -1):
    """Real-edge top-k_real merged with an RW selection: (table [n_q,width], row_len [n_q]).

    ``light_max >= 0`` with ``heavy`` (every query of the range whose in-degree
    exceeds it, ascending) serves the light queries one per thread."""
    dev = in_ptr.device
    _require(in_ptr, "in_ptr", torch.int64)
    _require(in_src, "in_src", torch.int32, dev)
    width = width if width is not None else max(1, max(k_real, 0) + (k_rw if rw_kv is not None else 0))
    table = torch.empty(n_q, width, dtype=torch.int32, device=dev)
    row_len = torch.empty(n_q, dtype=torch.int32, device=dev)
    n_hubs = 0 if hubs is None or k_real <= 0 else hubs.numel()
    hub_sel = torch.empty(max(n_hubs * max(k_real, 0), 1), dtype=torch.int32, device=dev)
    hub_cnt = torch.empty(max(n_hubs, 1), dtype=torch.int32, device=dev)
    n_heavy = 0 if heavy is None else heavy.numel()
    if n_heavy:
        _require(heavy, "heavy", torch.int32, dev)
    if light_max >= 0 and heavy is None:
        raise ValueError("light_max >= 0 needs the heavy-query list")
    N.call("bf_real_select_merge", _p(in_ptr), _p(in_src), in_ptr.numel() - 1, q_lo, n_q, k_real, key_seed,
           _p(rw_kv), _p(rw_cnt), k_rw, int(bool(dedup)), _p(table), width, _p(row_len),
           _p(hubs) if n_hubs else None, n_hubs, hub_threshold, _p(hub_sel), _p(hub_cnt),
           _p(heavy) if n_heavy else None, n_heavy, int(light_max), _stream(dev))
    return table, row_len


def _check_qids(qids: torch.Tensor, num_nodes: int, dev) -> None:
    _require(qids, "query_ids", torch.int32, dev)
    if qids.dim() != 1:
        raise ValueError("query_ids must be 1-D")
    if qids.numel():
        lo, hi = torch.aminmax(qids)
        if int(lo) < 0 or int(hi) >= num_nodes:
            raise ValueError(f"query_ids must lie in [0, {num_nodes}) (got [{int(lo)}, {int(hi)}])")


def rw_select_rows(rowptr, col, qids: torch.Tensor, walks_per_node: int, walk_length: int, k_rw: int,
                   key_seed: int, u=None, philox_seed: int = 0, philox_offset: int = 0, subtract=None,
                   walk_rec=None):
    """bf_rw_select for an explicit query list; ``subtract=(in_ptr, in_src)`` drops candidates that are
    already graph edges into the query. Returns (sel_kv [n,k_rw] key order, sel_cnt [n])."""
    dev = rowptr.device
    _require(rowptr, "rowptr", torch.int64)
    _require(col, "col", torch.int32, dev)
    n_nodes = rowptr.numel() - 1
    _check_qids(qids, n_nodes, dev)
    n = qids.numel()
    if u is not None:
        _require(u, "u", torch.float32, dev)
        if tuple(u.shape) != (n * walks_per_node, walk_length):
            raise ValueError(f"u must be [{n * walks_per_node}, {walk_length}], got {tuple(u.shape)}")
    sub_ptr = sub_src = None
    if subtract is not None:
        sub_ptr, sub_src = subtract
        _require(sub_ptr, "subtract in_ptr", torch.int64, dev)
        _require(sub_src, "subtract in_src", torch.int32, dev)
        if sub_ptr.numel() != n_nodes + 1:
            raise ValueError("subtract in_ptr must have num_nodes + 1 entries")
    sel = torch.empty(n, k_rw, dtype=torch.int32, device=dev)
    cnt = torch.empty(n, dtype=torch.int32, device=dev)
    N.call("bf_rw_select_rows", _p(rowptr), _p(col), _walk_rec_arg(walk_rec, col, dev), n_nodes, _p(qids), n,
           walks_per_node, walk_length, k_rw, key_seed, _p(u), philox_seed & (2 ** 64 - 1),
           philox_offset & (2 ** 64 - 1), _p(sub_ptr), _p(sub_src), _p(sel), _p(cnt), _stream(dev))
    return sel, cnt


def real_select_rows(in_ptr, in_src, qids: torch.Tensor, k_real: int, key_seed: int,
                     hubs: Optional[torch.Tensor] = None, hub_threshold: int = HUB_THRESHOLD):
    """Real-edge top-k_real in key order for an explicit query list: (sel_kv [n,k_real], sel_cnt [n])."""
    dev = in_ptr.device
    _require(in_ptr, "in_ptr", torch.int64)
    _require(in_src, "in_src", torch.int32, dev)
    _check_qids(qids, in_ptr.numel() - 1, dev)
    n = qids.numel()
    sel = torch.empty(n, k_real, dtype=torch.int32, device=dev)
    cnt = torch.empty(n, dtype=torch.int32, device=dev)
    n_hubs = 0 if hubs is None else hubs.numel()
    if n_hubs:
        _require(hubs, "hubs", torch.int32, dev)
    hub_sel = torch.empty(max(n_hubs * k_real, 1), dtype=torch.int32, device=dev)
    hub_cnt = torch.empty(max(n_hubs, 1), dtype=torch.int32, device=dev)
    N.call("bf_real_select_rows", _p(in_ptr), _p(in_src), in_ptr.numel() - 1, _p(qids), n, k_real, key_seed,
           _p(hubs) if n_hubs else None, n_hubs, hub_threshold, _p(hub_sel), _p(hub_cnt), _p(sel), _p(cnt),
           _stream(dev))
    return sel, cnt


def assemble_rows(real=None, rw=None, b_real: int = 0, b_rw: int = 0, dedup: bool = True):
    """One budget candidate from key-ordered selections ``real=(sel, cnt)`` / ``rw=(sel, cnt)``:
    (table [n, b_real+b_rw], row_len [n])."""
    parts = [x for x in (real, rw) if x is not None]
    if not parts:
        raise ValueError("assemble_rows needs at least one selection")
    dev = parts[0][0].device
    n = parts[0][0].shape[0]
    for sel, cnt in parts:
        _require(sel, "selection", torch.int32, dev)
        _require(cnt, "selection counts", torch.int32, dev)
        if sel.shape[0] != n or cnt.shape != (n,):
            raise ValueError("selections must have the same row count")
    b_real = b_real if real is not None else 0
    b_rw = b_rw if rw is not None else 0
    width = max(1, b_real + b_rw)
    table = torch.empty(n, width, dtype=torch.int32, device=dev)
    row_len = torch.empty(n, dtype=torch.int32, device=dev)
    N.call("bf_assemble_rows", _p(real[0]) if real is not None else None, _p(real[1]) if real is not None else None,
           real[0].shape[1] if real is not None else 0, b_real, _p(rw[0]) if rw is not None else None,
           _p(rw[1]) if rw is not None else None, rw[0].shape[1] if rw is not None else 0, b_rw, int(bool(dedup)), n,
           _p(table), width, _p(row_len), _stream(dev))
    return table, row_len


def mark_in_neighbors(in_ptr, in_src, frontier: torch.Tensor, reached: torch.Tensor) -> None:
    """reached[s] = 1 for every edge s -> v with frontier[v] (uint8 masks over the nodes)."""
    dev = in_ptr.device
    _require(in_ptr, "in_ptr", torch.int64)
    _require(in_src, "in_src", torch.int32, dev)
    n = in_ptr.numel() - 1
    for t, name in ((frontier, "frontier"), (reached, "reached")):
        _require(t, name, torch.uint8, dev)
        if t.numel() != n:
            raise ValueError(f"{name} must have num_nodes = {n} entries")
    N.call("bf_mark_in_neighbors", _p(in_ptr), _p(in_src), n, _p(frontier), _p(reached), _stream(dev))


def build_edge_table(rowptr, col, in_ptr, in_src, num_edges: int, q_lo: int, n_q: int, walks_per_node: int,
                     walk_length: int, k_real: int, k_rw: int, edge_seed: int, u=None, philox_seed: int = 0,
                     philox_offset: int = 0, out=None, hubs: Optional[torch.Tensor] = None,
                     hub_threshold: int = HUB_THRESHOLD, heavy: Optional[torch.Tensor] = None,
                     light_max: int = -1, walk_rec=None):
    """Fused budgeted build (bf_build_edge_table): (table [n_q, k_real+k_rw], row_len [n_q]).

    ``out=(table, row_len)`` writes into caller-provided (contiguous) tensors.
    ``heavy`` / ``light_max`` as in ``real_select_merge``; ``walk_rec`` as in ``rw_select``.
    """
    dev = rowptr.device
    _require(rowptr, "rowptr", torch.int64)
    _require(col, "col", torch.int32, dev)
    _require(in_ptr, "in_ptr", torch.int64, dev)
    _require(in_src, "in_src", torch.int32, dev)
    if u is not None:
        _require(u, "u", torch.float32, dev)
        if tuple(u.shape) != (n_q * walks_per_node, walk_length):
            raise ValueError(f"u must be [{n_q * walks_per_node}, {walk_length}], got {tuple(u.shape)}")
    width = max(k_real, 0) + max(k_rw, 0)
    n_hubs = 0 if hubs is None else hubs.numel()
    if n_hubs:
        _require(hubs, "hubs", torch.int32, dev)
    n_heavy = 0 if heavy is None else heavy.numel()
    if n_heavy:
        _require(heavy, "heavy", torch.int32, dev)
    if light_max >= 0 and heavy is None:
        raise ValueError("light_max >= 0 needs the heavy-query list")
    _walk_rec_arg(walk_rec, col, dev)
    if out is None:
        return N.load_ops().build_edge_table(
            rowptr, col, walk_rec, in_ptr, in_src, q_lo, n_q, walks_per_node, walk_length, k_real, k_rw,
            int(edge_seed), u, _i64(philox_seed), _i64(philox_offset), hubs if n_hubs else None, int(hub_threshold),
            heavy, int(light_max))
    # into caller-provided tensors (a shard of a larger table): the C ABI directly
    table, row_len = out
    _require(table, "table", torch.int32, dev)
    _require(row_len, "row_len", torch.int32, dev)
    if tuple(table.shape) != (n_q, width) or tuple(row_len.shape) != (n_q,):
        raise ValueError(f"out tensors must be [{n_q}, {width}] and [{n_q}]")
    ws_bytes = _size_query("bf_build_edge_table_workspace_size", n_q, max(k_rw, 0), n_hubs, max(k_real, 0))
    ws = _workspace(ws_bytes, dev)
    N.call("bf_build_edge_table", _p(rowptr), _p(col), _walk_rec_arg(walk_rec, col, dev), _p(in_ptr), _p(in_src),
           rowptr.numel() - 1, num_edges, q_lo, n_q, walks_per_node, walk_length, k_real, k_rw, edge_seed, _p(u),
           philox_seed & (2 ** 64 - 1), philox_offset & (2 ** 64 - 1), _p(hubs) if n_hubs else None, n_hubs, hub_threshold,
           _p(heavy) if n_heavy else None, n_heavy, int(light_max), _p(table), _p(row_len), _p(ws), ws.numel(),
           _stream(dev))
    return table, row_len


# ------------------------------------------------------------------ index formats
def _bits_for(maxval: int) -> int:
    """Bits that hold every value in [0, maxval] (at least 1)."""
    return max(1, int(maxval).bit_length())


@dataclass
class ReverseKeys:
    """table_to_csr's reverse-index sort keys, id << (q_bits + slot_bits) | query << slot_bits | slot, one per
    table entry (with the Graphormer token its own entries get none: their reverse places are fixed)."""
    keys: torch.Tensor          # uint64 as int64 [table entries]
    q_bits: int
    slot_bits: int
    global_token: bool
    token_row: int              # as in table_to_csr: the token row's length, or -1 for none


def _token_row(n_rows: int, global_token: bool, token_row: Optional[int]) -> int:
    """The token row's length (>= 0) or -1 for none: by default a table with the token covers the full
    query set, so its token row lists all n_rows nodes."""
    if not global_token:
        return -1
    return n_rows if token_row is None else int(token_row)


def check_table(table: torch.Tensor, row_len: torch.Tensor, id_limit: int) -> None:
    """Device-side validation of an externally supplied table (bf_check_table): raises ValueError when a
    row length lies outside [0, width] or an id of a row's first row_len slots outside [0, id_limit).
    One kernel and one 16-byte read back."""
    dev = table.device
    _require(table, "table", torch.int32)
    _require(row_len, "row_len", torch.int32, dev)
    if table.dim() != 2 or row_len.shape != (table.shape[0],):
        raise ValueError("table must be [n, width] and row_len [n]")
    ws = torch.empty(2, dtype=torch.int64, device=dev)
    N.call("bf_check_table", _p(table), _p(row_len), table.shape[0], table.shape[1], int(id_limit), None, _p(ws), 16,
           _stream(dev))


def table_qptr(table: torch.Tensor, row_len: torch.Tensor, global_token: bool = False,
               token_row: Optional[int] = None) -> torch.Tensor:
    """qptr [n_q+1] int64 of a query-major table (bf_table_csr_ptr without the host read of nnz).
    ``token_row``: see ``table_to_csr``."""
    dev = table.device
    _require(table, "table", torch.int32)
    _require(row_len, "row_len", torch.int32, dev)
    n_rows = table.shape[0]
    tr = _token_row(n_rows, global_token, token_row)
    n_q = n_rows + (1 if tr >= 0 else 0)
    ws = _workspace(_size_query("bf_scan_workspace_size", n_q), dev)
    qptr = torch.empty(n_q + 1, dtype=torch.int64, device=dev)
    N.call("bf_table_csr_ptr", _p(row_len), n_rows, int(global_token), tr, _p(qptr), None, _p(ws), ws.numel(),
           _stream(dev))
    return qptr


def table_to_csr(table: torch.Tensor, row_len: torch.Tensor, global_token: bool = False, with_keys: bool = False,
                 qptr: Optional[torch.Tensor] = None, token_row: Optional[int] = None, exact: bool = True):
    """Query-major table -> (qptr [n_q+1] int64, kv [nnz] int32), plus the reverse-index sort keys
    (``ReverseKeys``, or None when the query and slot fields need more than 33 bits) with ``with_keys``.
    ``qptr`` from ``table_qptr`` saves the scan; nnz is read from it (one host read). Without ``exact``
    nothing is read back: kv and the keys are sized for every row full (entries past qptr[n_q] hold
    nothing), so the whole index can be built while the host runs ahead.

    With ``global_token`` every table row also attends to kv 0 and ids shift by one; ``token_row`` is the
    length of the token's own row, placed as attention row 0 (default n_rows: the full query set; N for
    a query shard that starts at node 0), or -1 for a shard without it (every row then starts with kv 0)."""
    dev = table.device
    n_rows, width = table.shape
    tr = _token_row(n_rows, global_token, token_row)
    if qptr is None:
        qptr = table_qptr(table, row_len, global_token, tr)
    n_q = n_rows + (1 if tr >= 0 else 0)
    n_token = (n_rows + max(tr, 0)) if global_token else 0    # kv 0 of every table row, the token row
    nnz = int(qptr[n_q].item()) if exact else n_rows * width + n_token
    kv = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)[:nnz]
    rk = None
    q_bits, slot_bits = _bits_for(n_q), _bits_for(width)
    if with_keys and q_bits + slot_bits <= 33:
        # the token's entries get no key
        n_keys = nnz - n_token
        rk = ReverseKeys(torch.empty(max(n_keys, 1), dtype=torch.int64, device=dev)[:n_keys], q_bits,
                         slot_bits, bool(global_token), tr)
    N.call("bf_table_to_csr", _p(table), _p(row_len), n_rows, width, int(global_token), tr, _p(qptr), _p(kv),
           _p(rk.keys) if rk is not None else None, q_bits, slot_bits, _stream(dev))
    return (qptr, kv, rk) if with_keys else (qptr, kv)


def split_row_items(length: int, item_size: int = DEFAULT_ITEM) -> int:
    """Items a split row of ``length`` entries is cut into (bf_split_row_items)."""
    return int(N.load().bf_split_row_items(int(length), int(item_size)))


def coo_to_csr(edge_index: torch.Tensor, n_q: int, n_kv: int):
    """Reference COO [2, nnz] (row 0 = kv, row 1 = query) -> (qptr, kv), rows ascending in kv."""
    dev = edge_index.device
    if edge_index.dim() != 2 or edge_index.size(0) < 2:
        raise ValueError(f"edge_index must be [2, E] (got {tuple(edge_index.shape)})")
    src = edge_index[0].to(torch.int64).contiguous()
    dst = edge_index[1].to(torch.int64).contiguous()
    nnz = src.numel()
    if nnz:
        lo = torch.stack([src.min(), dst.min()]).min().item()
        if lo < 0 or src.max().item() >= n_kv or dst.max().item() >= n_q:
            raise ValueError(f"edge_index ids outside [0,{n_kv}) x [0,{n_q})")
    ws = _workspace(_size_query("bf_coo_to_csr_workspace_size", nnz, n_q), dev)
    qptr = torch.empty(n_q + 1, dtype=torch.int64, device=dev)
    kv = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)[:nnz]
    N.call("bf_coo_to_csr", _p(src), _p(dst), nnz, n_q, n_kv, _p(qptr), _p(kv), _p(ws), ws.numel(), _stream(dev))
    return qptr, kv


def reverse_index(qptr: torch.Tensor, kv: torch.Tensor, n_kv: int):
    """Key-major view: (kptr [n_kv+1], kq [nnz], ks [nnz]) sorted by (kv, CSR position): each reverse
    entry's query and its slot in the query's row."""
    dev = qptr.device
    _require(qptr, "qptr", torch.int64)
    _require(kv, "kv", torch.int32, dev)
    nnz = kv.numel()
    ws = _workspace(_size_query("bf_reverse_index_workspace_size", nnz, n_kv), dev)
    kptr = torch.empty(n_kv + 1, dtype=torch.int64, device=dev)
    kq = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)[:nnz]
    ks = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)[:nnz]
    N.call("bf_reverse_index", _p(qptr), _p(kv), qptr.numel() - 1, n_kv, nnz, _p(kptr), _p(kq), _p(ks), _p(ws),
           ws.numel(), _stream(dev))
    return kptr, kq, ks


def reverse_index_packed(rk: ReverseKeys, qptr: torch.Tensor, n_kv: int, entries: bool = True):
    """reverse_index from table_to_csr's sort keys (one sort of the id bits, no row recovery):
    (kptr, kq, ks, sorted). ``entries=False`` skips ks (the slots, which only a bias, factor or dropout
    needs; ``reverse_slots(sorted, qptr)`` gives them later) and returns ks = None."""
    dev = qptr.device
    _require(qptr, "qptr", torch.int64)
    _require(rk.keys, "keys", torch.int64, dev)
    n_keys = rk.keys.numel()
    nnz = _entries_of(rk, qptr)
    ws = _workspace(_size_query("bf_reverse_index_packed_workspace_size", nnz), dev)
    srt = ReverseKeys(torch.empty(max(n_keys, 1), dtype=torch.int64, device=dev)[:n_keys], rk.q_bits, rk.slot_bits,
                      rk.global_token, rk.token_row)
    kptr = torch.empty(n_kv + 1, dtype=torch.int64, device=dev)
    kq = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)[:nnz]
    ks = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)[:nnz] if entries else None
    N.call("bf_reverse_index_packed", _p(rk.keys), _p(qptr), nnz, qptr.numel() - 1, n_kv, rk.q_bits, rk.slot_bits,
           int(rk.global_token), int(rk.token_row), _p(srt.keys), _p(kptr), _p(kq), _p(ks) if entries else None,
           _p(ws), ws.numel(), _stream(dev))
    return kptr, kq, ks, srt


def _entries_of(rk: ReverseKeys, qptr: torch.Tensor) -> int:
    """Entries of the index whose reverse-index keys are ``rk``: the keys plus the token's own entries."""
    if not rk.global_token:
        return rk.keys.numel()
    return rk.keys.numel() + qptr.numel() - 1 - (1 if rk.token_row >= 0 else 0) + max(rk.token_row, 0)


def reverse_slots(srt: ReverseKeys, qptr: torch.Tensor) -> torch.Tensor:
    """ks (each reverse entry's slot in its query's row, int32) from reverse_index_packed's sorted keys."""
    dev = qptr.device
    _require(qptr, "qptr", torch.int64)
    _require(srt.keys, "keys", torch.int64, dev)
    nnz = _entries_of(srt, qptr)
    ks = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)[:nnz]
    N.call("bf_reverse_slots", _p(srt.keys), _p(qptr), nnz, qptr.numel() - 1, srt.q_bits, srt.slot_bits,
           int(srt.global_token), int(srt.token_row), _p(ks), _stream(dev))
    return ks


def radix_sort_keys(keys: torch.Tensor, begin_bit: int, end_bit: int) -> torch.Tensor:
    """``keys`` (int64 holding uint64 bit patterns) stably sorted by bits [begin_bit, end_bit), through the
    reverse index's radix sort (bf_radix_sort_keys)."""
    dev = keys.device
    _require(keys, "keys", torch.int64)
    n = keys.numel()
    ws = _workspace(_size_query("bf_radix_sort_workspace_size", n, begin_bit, end_bit), dev)
    out = torch.empty_like(keys)
    N.call("bf_radix_sort_keys", _p(keys), _p(out), n, begin_bit, end_bit, _p(ws), ws.numel(), _stream(dev))
    return out


def expand_rows(ptr: torch.Tensor, nnz: int) -> torch.Tensor:
    """Row id (int64) of every CSR entry."""
    _require(ptr, "ptr", torch.int64)
    rows = torch.empty(max(nnz, 1), dtype=torch.int64, device=ptr.device)[:nnz]
    N.call("bf_expand_rows", _p(ptr), ptr.numel() - 1, nnz, _p(rows), _stream(ptr.device))
    return rows


def row_order(ptr: torch.Tensor, spans: bool = False):
    """Rows of a CSR longest-first (bf_row_order), int32 [n_rows]; with ``spans`` also each slot's row as
    (begin << 32 | length), int64 [n_rows] (needs ptr[-1] < 2**32)."""
    n_rows = ptr.numel() - 1
    order = torch.empty(max(n_rows, 1), dtype=torch.int32, device=ptr.device)
    sp = torch.empty(max(n_rows, 1), dtype=torch.int64, device=ptr.device) if spans else None
    ws = _workspace(_size_query("bf_row_order_workspace_size", n_rows), ptr.device)
    N.call("bf_row_order", _p(ptr), n_rows, _p(order), _p(sp), _p(ws), ws.numel(), _stream(ptr.device))
    return (order, sp) if spans else order


def row_order_and_plan(ptr: torch.Tensor, nnz: int, threshold: int, item_size: int,
                       counts: Optional[torch.Tensor] = None, host_copy: bool = True):
    """(order, spans, plan): ``row_order(ptr, spans=True)`` and the split plan of the rows it puts first
    (bf_row_order_and_plan; threshold in [1, 254]), split rows and their items numbered longest first.
    The plan's counts are handled as in ``split_plan(..., resolve=False)``."""
    dev = ptr.device
    lib = N.load()
    n_rows = ptr.numel() - 1
    r = max(n_rows, 1)
    item_cap = int(lib.bf_split_item_capacity(nnz, threshold, item_size))
    heavy_cap = int(lib.bf_split_row_capacity(nnz, threshold))
    order = torch.empty(r, dtype=torch.int32, device=dev)
    spans = torch.empty(r, dtype=torch.int64, device=dev)
    buf = torch.empty(2 * r + max(item_cap, 1) + max(heavy_cap, 1), dtype=torch.int32, device=dev)
    nitems, item_off, item_row, heavy_rows = torch.split(buf, [r, r, max(item_cap, 1), max(heavy_cap, 1)])
    if counts is None:
        counts = torch.empty(2, dtype=torch.int32, device=dev)
    ws = _workspace(_size_query("bf_row_order_and_plan_workspace_size", n_rows, heavy_cap), dev)
    N.call("bf_row_order_and_plan", _p(ptr), n_rows, threshold, item_size, _p(order), _p(spans), _p(nitems),
           _p(item_off), _p(item_row), item_cap, _p(heavy_rows), heavy_cap, _p(counts), _p(ws), ws.numel(),
           _stream(dev))
    plan = SplitPlan(-1, -1, nitems, item_off, item_row, heavy_rows, counts, item_cap, heavy_cap)
    if host_copy:
        _copy_counts_to_host(plan, dev)
    return order, spans, plan


@dataclass
class SplitPlan:
    """Rows longer than `threshold` cut into `item_size`-entry items.

    ``items`` / ``heavy`` are host ints once resolved (-1 while ``counts``, the
    device copy, is still pending: several plans resolve with one read)."""
    items: int
    heavy: int
    nitems: torch.Tensor
    item_off: torch.Tensor
    item_row: torch.Tensor
    heavy_rows: torch.Tensor
    counts: Optional[torch.Tensor] = None
    item_cap: int = 0           # capacities the arrays were sized for (upper bounds of the counts)
    heavy_cap: int = 0
    host_counts: Optional[torch.Tensor] = None   # pinned copy of `counts`, complete once `ready` is
    ready: Optional[object] = None               # (a torch.cuda.Event recorded after the copy)
    _slot: Optional[object] = field(default=None, repr=False)   # returns the pinned slot to its pool

    @property
    def pending(self) -> bool:
        return self.items < 0


class _PinnedCountSlots:
    """Pinned host slots (two int32 each) for the plans' count copies, from one buffer allocated once.

    A fresh pinned tensor per plan made the host stall: torch's pinned cache cannot hand back a block
    whose copy it still tracks as in flight, and a new pinned allocation (hipHostMalloc) blocks the
    host for milliseconds (measured at c2: 2.1 ms of idle GPU per build in a build + forward loop).
    A slot returns to the pool when its plan has been read, or when an unread plan is collected (after
    its copy has landed, so a late copy never lands in a slot handed out again)."""

    def __init__(self, slots: int = 4096):
        self.slots = slots
        self.buf = None
        self.free = list(range(slots - 1, -1, -1))

    def take(self):
        if not self.free:
            return None
        if self.buf is None:
            self.buf = torch.empty(2 * self.slots, dtype=torch.int32, pin_memory=True)
        i = self.free.pop()
        return i, self.buf[2 * i:2 * i + 2]

    def give(self, i: int) -> None:
        self.free.append(i)


_PINNED = _PinnedCountSlots()


def _release_slot(slot: int, ready) -> None:
    ready.synchronize()
    _PINNED.give(slot)


def _copy_counts_to_host(plan: "SplitPlan", dev) -> None:
    """Copy a plan's device counts into a pinned slot behind its kernels (left on the device when every
    slot is held by an unread plan: the plan then resolves with a device read)."""
    got = _PINNED.take()
    if got is None:
        return
    slot, host = got
    host.copy_(plan.counts, non_blocking=True)
    plan.host_counts = host
    plan.ready = torch.cuda.Event()
    plan.ready.record(torch.cuda.current_stream(dev))
    plan._slot = weakref.finalize(plan, _release_slot, slot, plan.ready)


def resolve_plans(*plans) -> None:
    """Read the counts of every pending plan: from its pinned copy once that has landed, else with a
    single device-to-host copy for all of them."""
    pending = [p for p in plans if p is not None and p.items < 0]
    for p in [p for p in pending if p.ready is not None]:
        p.ready.synchronize()
        p.items, p.heavy = (int(x) for x in p.host_counts.tolist())
        p.counts = p.host_counts = p.ready = None
        p._slot()              # the slot goes back to the pool (the finalizer runs once)
    pending = [p for p in pending if p.items < 0]
    if not pending:
        return
    # plans made with one shared counts buffer (split_plan(..., counts=...)) come back in one copy
    base = pending[0].counts
    shared = all(p.counts.untyped_storage().data_ptr() == base.untyped_storage().data_ptr() for p in pending)
    if len(pending) == 1:
        vals = base.cpu().tolist()
    elif shared:
        # copy only the span of the storage that holds the pending counts
        offs = [p.counts.storage_offset() for p in pending]
        lo, hi = min(offs), max(offs) + 2
        span = torch.empty(0, dtype=torch.int32, device=base.device).set_(base.untyped_storage(), lo, (hi - lo,))
        allv = span.cpu().tolist()
        vals = sum((allv[o - lo:o - lo + 2] for o in offs), [])
    else:
        vals = torch.cat([p.counts for p in pending]).cpu().tolist()
    for i, p in enumerate(pending):
        p.items, p.heavy, p.counts = int(vals[2 * i]), int(vals[2 * i + 1]), None


def split_plan_first_row(n_rows: int, n_items: int, nnz: int, threshold: int, item_size: int,
                         counts: torch.Tensor) -> SplitPlan:
    """Split plan of a CSR whose only row longer than ``threshold`` is row 0, cut into ``n_items`` items
    (bf_split_plan_first_row): the arrays and counts ``split_plan`` would give, in one pass."""
    dev = counts.device
    lib = N.load()
    item_cap = int(lib.bf_split_item_capacity(nnz, threshold, item_size))
    heavy_cap = int(lib.bf_split_row_capacity(nnz, threshold))
    r = max(n_rows, 1)
    buf = torch.empty(2 * r + max(item_cap, 1) + max(heavy_cap, 1), dtype=torch.int32, device=dev)
    nitems, item_off, item_row, heavy_rows = torch.split(buf, [r, r, max(item_cap, 1), max(heavy_cap, 1)])
    N.call("bf_split_plan_first_row", n_rows, n_items, _p(nitems), _p(item_off), _p(item_row), item_cap,
           _p(heavy_rows), heavy_cap, _p(counts), _stream(dev))
    return SplitPlan(n_items, 1 if n_items else 0, nitems, item_off, item_row, heavy_rows, counts, item_cap,
                     heavy_cap)


def split_plan(ptr: torch.Tensor, nnz: int, threshold: int = DEFAULT_CHUNK, item_size: int = DEFAULT_ITEM,
               resolve: bool = True, counts: Optional[torch.Tensor] = None,
               known: Optional[tuple] = None, host_copy: bool = True) -> SplitPlan:
    """Split plan of a CSR. ``counts`` (int32 [2], optional) receives the two plan counts on the device;
    plans that share one buffer resolve with a single copy. ``known`` = (items, split rows) when the
    caller knows them from the row lengths' bounds: the plan then needs no read of the counts. Without
    ``resolve`` the counts are copied to pinned host memory behind the plan's kernels (``host_copy``)
    or left on the device only."""
    dev = ptr.device
    lib = N.load()
    n_rows = ptr.numel() - 1
    item_cap = int(lib.bf_split_item_capacity(nnz, threshold, item_size))
    heavy_cap = int(lib.bf_split_row_capacity(nnz, threshold))
    r = max(n_rows, 1)
    buf = torch.empty(2 * r + max(item_cap, 1) + max(heavy_cap, 1), dtype=torch.int32, device=dev)
    nitems, item_off, item_row, heavy_rows = torch.split(buf, [r, r, max(item_cap, 1), max(heavy_cap, 1)])
    if counts is None:
        counts = torch.empty(2, dtype=torch.int32, device=dev)
    ws = _workspace(_size_query("bf_split_plan_workspace_size", n_rows), dev)
    N.call("bf_split_plan", _p(ptr), n_rows, threshold, item_size, _p(nitems), _p(item_off), _p(item_row), item_cap,
           _p(heavy_rows), heavy_cap, _p(counts), _p(ws), ws.numel(), _stream(dev))
    plan = SplitPlan(-1, -1, nitems, item_off, item_row, heavy_rows, counts, item_cap, heavy_cap)
    if known is not None:
        plan.items, plan.heavy = int(known[0]), int(known[1])
    elif resolve:
        resolve_plans(plan)
    elif host_copy:
        # the counts travel to pinned host memory behind the plan's kernels; reading them later waits
        # only for this copy, typically long done while the stream runs on
        _copy_counts_to_host(plan, dev)
    return plan


# ------------------------------------------------------------------ attention index
NO_READBACK_MAX_ENTRIES = 1 << 23   # tables of up to this many entries (at capacity) build without a host read


def _to_cap(t: torch.Tensor, cap: int) -> torch.Tensor:
    """An exact per-entry array in a buffer of the index's capacity (entries past its length hold nothing)."""
    if t.numel() == cap:
        return t
    out = torch.empty(max(cap, 1), dtype=t.dtype, device=t.device)[:cap]
    out[:t.numel()] = t
    return out


@dataclass
class AttentionIndex:
    """One edge set in the layout the attention kernels walk.

    Query-major CSR (qptr, kv) for the forward and the dq pass; the key-major
    reverse index (kptr, kq, ks) for the dk/dv pass is built on first use and
    then reused by every layer and step that shares the edge set.

    The per-entry arrays are held at a capacity (``kv_all``, ``kq_all``,
    ``ks_all``; ``cap`` >= nnz): a table's index is sized for every row full,
    so that building it reads nothing back to the host. The entry count is
    qptr[n_q]; ``nnz`` and the exact views ``kv``, ``kq``, ``ks`` read it on
    first use.
    """
    n_q: int
    n_kv: int
    qptr: torch.Tensor
    kv_all: Optional[torch.Tensor]
    chunk: int = DEFAULT_CHUNK
    item: int = DEFAULT_ITEM
    qplan: Optional[SplitPlan] = None
    kptr: Optional[torch.Tensor] = None
    kq_all: Optional[torch.Tensor] = None
    ks_all: Optional[torch.Tensor] = None    # each reverse entry's slot in its query's row
    kplan: Optional[SplitPlan] = None
    korder: Optional[torch.Tensor] = None
    kspans: Optional[torch.Tensor] = None      # per korder slot: (kptr[row] << 32 | row length)
    # key 0 is the Graphormer token column, attended once by each query row from 1 on (1) or from 0 on (2: a
    # query shard without the token row), first in the row, and by nothing else (0: no such promise): the
    # dq pass then sums its dK/dV terms instead of the dk/dv pass re-gathering them
    token_column: int = 0
    _rows: Optional[torch.Tensor] = field(default=None, repr=False)
    _rkeys: Optional[ReverseKeys] = field(default=None, repr=False)   # from_table: sort keys, until used
    _sorted: Optional[ReverseKeys] = field(default=None, repr=False)  # sorted keys, until ks is needed
    _counts: Optional[torch.Tensor] = field(default=None, repr=False)  # both plans' device counts
    # True: the plans leave their counts on the device and the attention calls size their grids for the
    # capacities (no host read at all between building the index and using it, e.g. for a caller that
    # cannot synchronise). False: a plan copies its counts to pinned host memory behind its kernels and
    # a call reads them when it is launched, by which time the copy has landed
    device_counts: bool = False
    # typed edges (Exphormer): bit 31 of each kv id and kq id is the entry's type; no query row is split
    typed: bool = False
    # (items, split rows) of the query-side plan when the row lengths fix them (from_table)
    _q_known: Optional[tuple] = field(default=None, repr=False)
    _structs: dict = field(default_factory=dict, repr=False)          # C view per (backward, with ks)
    _nnz: Optional[int] = field(default=None, repr=False)             # qptr[n_q], once read

    @property
    def cap(self) -> int:
        """The entries the per-entry arrays are sized for (>= nnz)."""
        return self.kv_all.numel()

    @property
    def nnz(self) -> int:
        """The entry count (qptr[n_q]; read from the device on first use unless the arrays are exact)."""
        if self._nnz is None:
            self._nnz = int(self.qptr[self.n_q].item()) if self.cap else 0
        return self._nnz

    @property
    def nnz_known(self) -> bool:
        return self._nnz is not None

    @property
    def kv(self) -> torch.Tensor:
        return self.kv_all[:self.nnz]

    @property
    def kq(self) -> Optional[torch.Tensor]:
        return None if self.kq_all is None else self.kq_all[:self.nnz]

    @property
    def ks(self) -> Optional[torch.Tensor]:
        return None if self.ks_all is None else self.ks_all[:self.nnz]

    @property
    def device(self):
        return self.qptr.device

    def resolve(self):
        """Read the plans' counts into host ints (one device-to-host copy)."""
        resolve_plans(self.qplan, self.kplan)
        return self

    def _host_copy(self) -> bool:
        """Whether a new plan sends its counts to pinned host memory (else they stay on the device)."""
        return not self.device_counts

    def ensure_forward(self):
        if self.qplan is None:
            self.qplan = split_plan(self.qptr, self.cap, self.chunk, self.item, resolve=False,
                                    counts=self._plan_counts(0), known=self._q_known,
                                    host_copy=self._host_copy())
        return self

    def _plan_counts(self, side: int) -> torch.Tensor:
        """Device slot for one side's plan counts; both sides share one buffer, read back together."""
        if self._counts is None:
            self._counts = torch.empty(4, dtype=torch.int32, device=self.device)
        return self._counts[2 * side:2 * side + 2]

    def ensure_backward(self, entries: bool = False):
        """The backward's parts of the index: the query-side plan, the reverse index and the key-side
        order and plan. ``entries``: also each reverse entry's slot (ks), decoded by the reverse index's
        own unpack pass rather than by a later one (``ensure_entries``)."""
        if self.qplan is None:
            self.qplan = split_plan(self.qptr, self.cap, self.chunk, self.item, resolve=False,
                                    counts=self._plan_counts(0), known=self._q_known,
                                    host_copy=self._host_copy())
        if self.kptr is None:
            if self._rkeys is not None and self._rkeys.q_bits + self._rkeys.slot_bits + _bits_for(self.n_kv) <= 64:
                self.kptr, self.kq_all, ks, srt = reverse_index_packed(self._rkeys, self.qptr, self.n_kv,
                                                                       entries=entries)
                if entries:
                    self.ks_all = ks
                else:
                    self._sorted = srt
                self._rkeys = None
            else:
                self.kptr, kq, ks = reverse_index(self.qptr, self.kv, self.n_kv)
                self.kq_all, self.ks_all = _to_cap(kq, self.cap), _to_cap(ks, self.cap)
        if self.kplan is None and self.korder is None and 1 <= self.chunk <= 254:
            # the rows to split are the longest-first order's first slots: one pass writes both
            self.korder, self.kspans, self.kplan = row_order_and_plan(
                self.kptr, self.cap, self.chunk, self.item, counts=self._plan_counts(1),
                host_copy=self._host_copy())
        if self.kplan is None:
            self.kplan = split_plan(self.kptr, self.cap, self.chunk, self.item, resolve=False,
                                    counts=self._plan_counts(1), host_copy=self._host_copy())
        if self.korder is None:
            self.korder, self.kspans = row_order(self.kptr, spans=True)
        return self

    def ensure_entries(self):
        """Each reverse entry's slot in its query's row (ks), which the dk/dv pass reads only with a bias,
        factor or dropout: (kq, ks) keys the dropout, and qptr[kq] + ks is the CSR position a bias or
        factor is indexed by."""
        self.ensure_backward()
        if self.ks_all is None and self.cap:
            self.ks_all = reverse_slots(self._sorted, self.qptr)
            self._sorted = None
        return self

    def entry_rows(self) -> torch.Tensor:
        """Query id of every CSR entry (int64), for per-edge bias gathers."""
        if self._rows is None:
            self._rows = expand_rows(self.qptr, self.nnz)
        return self._rows

    def to_coo(self) -> torch.Tensor:
        """[2, nnz] int64 in (src, dst) order — the order PyG coalesce produces."""
        self.ensure_backward()
        src = expand_rows(self.kptr, self.nnz)
        return torch.stack([src, self.kq.to(torch.int64)])

    def struct(self, backward: bool, entries: bool = False) -> N.AttnIndex:
        self.ensure_backward(entries) if backward else self.ensure_forward()
        if backward and entries:
            self.ensure_entries()
        # the index does not change once built: every layer and step reuses the same struct
        key = (backward, backward and self.ks_all is not None, self.nnz_known)
        cached = self._structs.get(key)
        if cached is not None:
            return cached
        s = self._make_struct(backward)
        self._structs[key] = s
        return s

    # bf_attn_index's pointer fields, in the order the torch operators take them (csrc/torch_ops.cpp)
    _TENSOR_FIELDS = ("qptr", "kv", "kptr", "kq", "ks", "q_nitems", "q_item_off", "q_item_row", "q_heavy_rows",
                      "k_nitems", "k_item_off", "k_item_row", "k_heavy_rows", "k_order", "k_spans", "plan_counts")
    _INT_FIELDS = ("n_q", "n_kv", "nnz", "chunk", "item", "q_items", "q_heavy", "k_items", "k_heavy", "token_column")

    def _fields(self, backward: bool):
        """bf_attn_index's fields: ({pointer field: tensor or None}, {integer field: int})."""
        t = dict.fromkeys(self._TENSOR_FIELDS)
        n = dict.fromkeys(self._INT_FIELDS, 0)
        # the kernels take the entries from the row pointers; nnz sizes only the per-edge tensors (bias,
        # factor, dbias), whose calls read it first, and otherwise passes the capacity
        n["n_q"], n["n_kv"], n["nnz"] = self.n_q, self.n_kv, self.nnz if self.nnz_known else self.cap
        t["qptr"], t["kv"] = self.qptr, self.kv_all if self.cap else None
        n["chunk"], n["item"] = self.chunk, self.item
        qp = self.qplan
        # plans with a pinned copy of their counts take them from it; the others stay pending, their
        # capacities size the grids and the kernels read the counts from the device
        resolve_plans(*[p for p in (qp, self.kplan if backward else None) if p is not None and p.ready is not None])
        # (a plan whose counts are known passes them: the device copy then holds the same values)
        on_device = qp.pending or (backward and self.kplan.pending)
        n["q_items"], n["q_heavy"] = (qp.item_cap, qp.heavy_cap) if qp.pending else (qp.items, qp.heavy)
        t["plan_counts"] = self._counts if on_device else None
        t["q_nitems"], t["q_item_off"], t["q_item_row"], t["q_heavy_rows"] = (
            qp.nitems, qp.item_off, qp.item_row, qp.heavy_rows)
        if backward:
            kp = self.kplan
            t["kptr"] = self.kptr
            t["kq"] = self.kq_all if self.cap else None
            t["ks"] = self.ks_all if (self.cap and self.ks_all is not None) else None
            n["k_items"], n["k_heavy"] = (kp.item_cap, kp.heavy_cap) if kp.pending else (kp.items, kp.heavy)
            t["k_nitems"], t["k_item_off"], t["k_item_row"], t["k_heavy_rows"] = (
                kp.nitems, kp.item_off, kp.item_row, kp.heavy_rows)
            t["k_order"] = self.korder if self.n_kv > 0 else None
            t["k_spans"] = self.kspans if (self.n_kv > 0 and self.kspans is not None) else None
        n["token_column"] = int(self.token_column)
        return t, n

    def _make_struct(self, backward: bool) -> N.AttnIndex:
        t, n = self._fields(backward)
        s = N.AttnIndex()
        for name, tensor in t.items():
            setattr(s, name, tensor.data_ptr() if tensor is not None else None)
        for name, value in n.items():
            setattr(s, name, value)
        return s

    def op_args(self, backward: bool, entries: bool = False):
        """The index as the torch operators take it: ([16 tensors or None], [10 ints]), in the order of
        bf_attn_index's fields (``_TENSOR_FIELDS``, ``_INT_FIELDS``); cached like ``struct``."""
        self.ensure_backward(entries) if backward else self.ensure_forward()
        if backward and entries:
            self.ensure_entries()
        key = ("op", backward, backward and self.ks_all is not None, self.nnz_known)
        cached = self._structs.get(key)
        if cached is None:
            t, n = self._fields(backward)
            cached = ([t[f] for f in self._TENSOR_FIELDS], [int(n[f]) for f in self._INT_FIELDS])
            self._structs[key] = cached
        return cached

    @classmethod
    def from_table(cls, table, row_len, global_token: bool = False, n_kv: Optional[int] = None,
                   chunk: int = DEFAULT_CHUNK, item: int = DEFAULT_ITEM, check: bool = True,
                   token_row: Optional[int] = None):
        """Index of a query-major table. ``check`` validates the table on the device first (row lengths
        within the width, the ids of every row's first row_len slots within [0, n_kv)) with one host
        read; the edge builder's own tables skip it (valid by construction).

        ``token_row`` (with ``global_token``): the length of the Graphormer token's own row, attention
        row 0 — by default the table's row count (the full query set); the node count N for a query
        shard that starts at node 0; -1 for a shard without it, whose attention rows are its table rows."""
        n_rows, width = table.shape
        tr = _token_row(n_rows, global_token, token_row)
        n_q_tab = n_rows + (1 if tr >= 0 else 0)
        n_kv = n_kv if n_kv is not None else n_q_tab
        if global_token and tr > n_kv - 1:
            raise ValueError(f"the token row lists kv 1..{tr}, beyond the {n_kv} kv rows")
        if check and table.numel():
            check_table(table, row_len, n_kv - (1 if global_token else 0))
        # A table row holds at most `width` entries (+ key 0 with the token), so when that is within
        # `chunk` only the token row (every node, tr entries) can be split: the query plan's counts
        # follow from the sizes, with no read of the device.
        known = None
        if width + (1 if global_token else 0) <= chunk:
            split = tr > chunk
            known = (split_row_items(tr, item) if split else 0, 1 if split else 0)
        qptr = table_qptr(table, row_len, global_token, tr)
        # the token fill puts key 0 first in every table row and shifts the table's own ids past it:
        # key 0 is then attended by every query row from 1 on (with the token row) or from 0 on (without)
        token_column = 0 if not global_token else (1 if tr >= 0 else 2)
        idx = cls(n_q=n_q_tab, n_kv=n_kv, qptr=qptr, kv_all=None, chunk=chunk, item=item,
                  token_column=token_column, _q_known=known)
        bound = n_rows * width + (n_rows if global_token else 0) + max(tr, 0)
        if known is not None:
            # only the token row can be split: its plan is written in one pass, before any read of nnz
            idx.qplan = split_plan_first_row(n_q_tab, known[0], bound, chunk, item, idx._plan_counts(0))
        # A small index is launch-bound: it is built at the capacity (every row full) with nothing read
        # back, so the host runs ahead of the kernels. A large one reads nnz once and sizes its arrays and
        # grids exactly (a B=32 table fills well under half of its capacity).
        qptr, idx.kv_all, idx._rkeys = table_to_csr(table, row_len, global_token, with_keys=True, qptr=qptr,
                                                    token_row=tr, exact=bound > NO_READBACK_MAX_ENTRIES)
        if bound > NO_READBACK_MAX_ENTRIES:
            idx._nnz = idx.kv_all.numel()
        return idx

    @classmethod
    def from_typed_coo(cls, edge_index, n_q: int, n_kv: Optional[int] = None, chunk: int = DEFAULT_CHUNK,
                       item: int = DEFAULT_ITEM):
        """Typed index of the reference's Exphormer edge set [3, E] (row 0 key/value node, row 1 query, row 2
        the edge type, 0 or 1; models/exphormer_dist_node_level.py:77-121): bit 31 of every kv id (CSR,
        rows ordered by (type, kv)) and kq id (reverse index, by (kv, CSR position)) is the entry's type,
        so the typed kernels need no type array and no typed copy of K or V. No query row is split (a
        query's row is its budget and expander edges); key rows are, as for any index."""
        n_kv = n_q if n_kv is None else n_kv
        if edge_index.dim() != 2 or edge_index.size(0) != 3:
            raise ValueError(f"a typed edge set is [3, E] (got {tuple(edge_index.shape)})")
        if 2 * n_kv >= 2 ** 31 or n_q >= 2 ** 31:
            raise ValueError("typed indexes need n_q and 2 * n_kv below 2^31")
        types = edge_index[2].to(torch.int64)
        if types.numel() and (types.min().item() < 0 or types.max().item() > 1):
            raise ValueError("edge types must be 0 or 1")
        src = edge_index[0].to(torch.int64)
        # rows ordered by (type, kv): the CSR of the type-shifted ids, then the type moved to bit 31
        qptr, kvp = coo_to_csr(torch.stack([src + types * n_kv, edge_index[1].to(torch.int64)]), n_q, 2 * n_kv)
        nnz = kvp.numel()
        kvp = kvp.to(torch.int64)
        one = kvp >= n_kv
        kv_enc = torch.where(one, kvp - n_kv - 2 ** 31, kvp).to(torch.int32)
        kptr, kq, ks = reverse_index(qptr, torch.where(one, kvp - n_kv, kvp).to(torch.int32), n_kv)
        pos = qptr[kq.to(torch.int64)] + ks.to(torch.int64)
        kq_enc = torch.where(kv_enc[pos] < 0, kq.to(torch.int64) - 2 ** 31, kq.to(torch.int64)).to(torch.int32)
        idx = cls(n_q=n_q, n_kv=n_kv, qptr=qptr, kv_all=kv_enc, chunk=chunk, item=item, _nnz=nnz, typed=True)
        # no split query rows: the query plan's threshold is above every row's length
        idx.qplan = split_plan(qptr, nnz, min(nnz + 1, 2 ** 31 - 1), item, resolve=False,
                               counts=idx._plan_counts(0), known=(0, 0), host_copy=False)
        idx.kptr, idx.kq_all, idx.ks_all = kptr, kq_enc, ks
        idx.ensure_backward()
        return idx

    @classmethod
    def from_coo(cls, edge_index, n_q: int, n_kv: Optional[int] = None, chunk: int = DEFAULT_CHUNK,
                 item: int = DEFAULT_ITEM):
        n_kv = n_q if n_kv is None else n_kv
        qptr, kv = coo_to_csr(edge_index, n_q, n_kv)
        return cls(n_q=n_q, n_kv=n_kv, qptr=qptr, kv_all=kv, chunk=chunk, item=item, _nnz=kv.numel())


# ------------------------------------------------------------------ attention
_DT = {torch.float32: N.BF_DTYPE_F32, torch.bfloat16: N.BF_DTYPE_BF16, torch.float16: N.BF_DTYPE_F16}


@dataclass(frozen=True)
class Dropout:
    """The in-kernel GraphGPS attention dropout (bf_attn_dropout): head h of the entry at slot s of query
    row r is kept iff Philox word h % 4 of counter (s, r, offset + h // 4), key seed, maps below 1 - rate;
    kept V messages scaled by 1 / (1 - rate)."""
    rate: float
    seed: int
    offset: int = 0

    def struct(self, keep=None):
        """The C struct; ``keep``: the forward's keep mask (a uint8 device tensor, bf_attn_dropout.keep)."""
        return N.AttnDropout(float(self.rate), int(self.seed) & (2 ** 64 - 1), int(self.offset) & (2 ** 64 - 1),
                             None if keep is None else keep.data_ptr())


def _dropout_arg(dropout: Optional[Dropout]):
    if dropout is None or dropout.rate <= 0.0:
        return None
    if not 0.0 <= dropout.rate <= 1.0:
        raise ValueError(f"dropout rate {dropout.rate} outside [0, 1]")
    return C.byref(dropout.struct())


def _i64(x: int) -> int:
    """A 64-bit pattern as the signed value a torch operator's int argument carries."""
    x = int(x) & (2 ** 64 - 1)
    return x - 2 ** 64 if x >= 2 ** 63 else x


def _dropout_op_args(dropout: Optional[Dropout]):
    """(rate, seed, offset) for the torch operators; rate 0 is no dropout."""
    if dropout is None or dropout.rate <= 0.0:
        return 0.0, 0, 0
    return float(dropout.rate), _i64(dropout.seed), _i64(dropout.offset)


SCORE_CLAMP = 5.0   # the reference's clamp bound on q.k / sqrt(hn)


def attn_forward(idx: AttentionIndex, q, k, v, bias=None, factor=None, dropout: Optional[Dropout] = None,
                 score_clamp: float = SCORE_CLAMP, keep_mask: bool = False):
    """out [n_q,H,hn] (activation dtype), Z [n_q,H] float32, through bf::sparse_attn_fwd (which checks
    the shapes, dtypes and devices against the index). ``score_clamp``: the bound of the clamp on
    q.k / sqrt(hn), in (0, 5]. With ``keep_mask`` also returns the dropout's keep mask (uint8
    [kv capacity, ceil(H/8)], empty without a dropout) for ``attn_backward(keep=...)``, whose dq pass then
    reads the bits instead of drawing them again (the same bits: results equal bit for bit)."""
    if bias is not None or factor is not None:
        idx.nnz      # per-edge tensors are [nnz, H]: the index passes the count itself
    t, n = idx.op_args(backward=False)
    out, Z, keep = N.load_ops().sparse_attn_fwd(q, k, v, t, n, bias, factor, *_dropout_op_args(dropout),
                                                float(score_clamp), bool(keep_mask))
    return (out, Z, keep) if keep_mask else (out, Z)


def attn_forward_typed(idx: AttentionIndex, q, k, v, type_mod):
    """Typed-edge (Exphormer) forward on a typed index (``AttentionIndex.from_typed_coo``): out [n_q,H,hn],
    Z [n_q,H] float32; type_mod = E, float32 [2, H, hn] (bf::sparse_attn_fwd_typed)."""
    if not idx.typed:
        raise ValueError("attn_forward_typed needs a typed index (AttentionIndex.from_typed_coo)")
    t, n = idx.op_args(backward=False)
    return N.load_ops().sparse_attn_fwd_typed(q, k, v, t, n, type_mod)


def attn_backward_typed(idx: AttentionIndex, q, k, v, type_mod, Z, dout):
    """(dq, dk, dv, dE) of attn_forward_typed; dE float32 [2, H, hn] (bf::sparse_attn_bwd_typed)."""
    if not idx.typed:
        raise ValueError("attn_backward_typed needs a typed index (AttentionIndex.from_typed_coo)")
    t, n = idx.op_args(backward=True)
    return N.load_ops().sparse_attn_bwd_typed(q, k, v, t, n, type_mod, Z, dout)


def kv_pass_variant(n_q: int, n_kv: int, dtype: torch.dtype, heads: int, head_dim: int) -> dict:
    """How the dk/dv pass runs for these sizes (bf_attn_bwd_kv_variant): rows per lane group, whether q
    and dO are gathered non-temporally, whether a group's row slots are prefetched."""
    s = N.AttnIndex()
    s.n_q, s.n_kv = int(n_q), int(n_kv)
    rpg, nt, pre = C.c_int32(), C.c_int32(), C.c_int32()
    N.call("bf_attn_bwd_kv_variant", C.byref(s), _DT[dtype], int(heads), int(head_dim), C.byref(rpg), C.byref(nt),
           C.byref(pre))
    return {"rows_per_group": rpg.value, "stream_rows": bool(nt.value), "prefetch_slots": bool(pre.value)}


def attn_backward(idx: AttentionIndex, q, k, v, out, Z, dout, bias=None, factor=None, need_dbias: bool = False,
                  dropout: Optional[Dropout] = None, score_clamp: float = SCORE_CLAMP, keep=None):
    """(dq, dk, dv, dbias-or-None) for attn_forward's outputs. ``out`` is accepted for the autograd
    surface but not read: the backward sums Delta = dO . out from the entries in float32. Through
    bf::sparse_attn_bwd, which checks the shapes, dtypes and devices. ``keep``: the keep mask
    ``attn_forward(keep_mask=True)`` returned for the same index and dropout, or None."""
    rate, seed, off = _dropout_op_args(dropout)
    if not 0.0 <= rate <= 1.0:
        raise ValueError(f"dropout rate {rate} outside [0, 1]")
    if bias is not None or factor is not None or need_dbias:
        idx.nnz      # per-edge tensors are [nnz, H]: the index passes the count itself
    t, n = idx.op_args(backward=True, entries=bias is not None or factor is not None or need_dbias or rate > 0.0)
    dq, dk, dv, dbias = N.load_ops().sparse_attn_bwd(q, k, v, t, n, Z, dout, bias, factor, bool(need_dbias), rate,
                                                     seed, off, float(score_clamp), keep)
    return dq, dk, dv, (dbias if need_dbias else None)
