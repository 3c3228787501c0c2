"""Graph topology in HBM and synthetic graphs of the benchmark shapes.

``CSRGraph`` holds the coalesced CSR the walk reads (source rows, ascending
neighbours; ``_get_random_walk_graph``, gt_sp/utils.py:890-936) and the
in-neighbour CSR the real-edge top-k reads (for a symmetric graph the same
arrays). Ids are int32, offsets int64, so a 1.6B-edge graph's col is 6.4 GB.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import hip_ops


@dataclass
class CSRGraph:
    rowptr: torch.Tensor          # int64 [N+1], rows = sources
    col: torch.Tensor             # int32 [E], ascending within a row
    in_ptr: torch.Tensor          # int64 [N+1], rows = destinations
    in_src: torch.Tensor          # int32 [E]
    num_nodes: int

    @property
    def num_edges(self) -> int:
        return int(self.col.numel())

    @property
    def device(self):
        return self.rowptr.device

    @property
    def symmetric(self) -> bool:
        return self.in_ptr is self.rowptr and self.in_src is self.col

    def heavy(self, light_max: int = hip_ops.LIGHT_MAX) -> torch.Tensor:
        """Ascending ids of queries whose in-degree exceeds ``light_max`` (int32), cached: the
        real-edge top-k of the others runs one query per thread."""
        return self.hubs(light_max)

    def hubs(self, threshold: int = hip_ops.HUB_THRESHOLD) -> torch.Tensor:
        """Ascending ids of queries whose in-degree exceeds ``threshold`` (int32), cached per threshold.

        The real-edge top-k of these rows runs one workgroup per row.
        """
        cache = self.__dict__.setdefault("_hubs", {})
        if threshold not in cache:
            plan = hip_ops.split_plan(self.in_ptr, self.num_edges, threshold, max(threshold, 1))
            cache[threshold] = plan.heavy_rows[: plan.heavy].clone()
        return cache[threshold]

    def walk_records(self, reserve_bytes: Optional[int] = None) -> Optional[torch.Tensor]:
        """The walk records of (rowptr, col), int32 [E, 4] (16 bytes per edge), cached: a walk step
        then reads one record instead of the rowptr pair and col. None when the graph has 2^31 edges or
        more (the records hold 32-bit degrees), or when the records and ``reserve_bytes`` (what the
        caller's build and index need next; by default an all-node build at B = 32 with its index,
        ``estimate_hot_path_bytes``) do not both fit the usable HBM; the walks then step through rowptr
        and col (the same walks). Decided once per graph."""
        if "_walk_rec" not in self.__dict__:
            from .gt_sp.utils import _rw_gpu_usable_bytes, estimate_hot_path_bytes
            rec = None
            e = self.num_edges
            if 0 < e < 2 ** 31 and self.device.type == "cuda":
                if reserve_bytes is None:
                    reserve_bytes = estimate_hot_path_bytes(self.num_nodes, e, self.num_nodes, 16, 16)["peak"]
                usable = _rw_gpu_usable_bytes(self.device)
                if usable < 0 or 16 * e + int(reserve_bytes) <= usable:
                    rec = hip_ops.walk_records(self.rowptr, self.col)
            self.__dict__["_walk_rec"] = rec
        return self.__dict__["_walk_rec"]

    @classmethod
    def from_csr(cls, rowptr, col, num_nodes: int, in_ptr=None, in_src=None, device="cuda"):
        rowptr = torch.as_tensor(rowptr, dtype=torch.int64).to(device).contiguous()
        col = torch.as_tensor(col).to(torch.int32).to(device).contiguous()
        if in_ptr is None:
            in_ptr, in_src = rowptr, col
        else:
            in_ptr = torch.as_tensor(in_ptr, dtype=torch.int64).to(device).contiguous()
            in_src = torch.as_tensor(in_src).to(torch.int32).to(device).contiguous()
        return cls(rowptr, col, in_ptr, in_src, int(num_nodes))

    @classmethod
    def from_edge_index(cls, edge_index: torch.Tensor, num_nodes: int, symmetric: bool = False, device="cuda"):
        """From the reference's coalesced ``edge_index_global`` [2, E] (row 0 source, row 1 target).

        Both CSRs are built on the device (radix sort); duplicates are kept, so
        pass a coalesced edge list as the reference does.
        """
        ei = edge_index.to(device)
        rowptr, col = hip_ops.coo_to_csr(torch.stack([ei[1], ei[0]]), num_nodes, num_nodes)
        if symmetric:
            return cls(rowptr, col, rowptr, col, int(num_nodes))
        in_ptr, in_src = hip_ops.coo_to_csr(ei, num_nodes, num_nodes)
        return cls(rowptr, col, in_ptr, in_src, int(num_nodes))


# ------------------------------------------------------------------ topology ingest
_SORT_LIMIT = (1 << 31) - 1      # entries one device radix sort takes (int32 counts)


def load_edge_index(path: str) -> torch.Tensor:
    """``edge_index.pt`` as utils/preprocess_data.py:425-427 writes it (``torch.save`` of a [2, E]
    integer tensor), loaded on the host as utils/fullgraph_sp_support.py:690-715 first tries:
    ``weights_only=True`` with ``mmap=True`` (without mmap for files that do not support it).
    The reference's ``weights_only=False`` fallbacks are not taken: they would unpickle
    arbitrary objects from the file."""
    try:
        t = torch.load(path, map_location="cpu", weights_only=True, mmap=True)
    except RuntimeError:
        t = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(t, torch.Tensor) or t.dim() != 2 or t.size(0) != 2 or t.dtype.is_floating_point:
        raise ValueError(f"{path}: expected a [2, E] integer tensor, got {type(t).__name__}"
                         f"{tuple(t.shape) if isinstance(t, torch.Tensor) else ''}")
    return t


def coalesce_edges(edge_index: torch.Tensor, num_nodes: int, max_chunk: int = _SORT_LIMIT) -> torch.Tensor:
    """torch_geometric ``coalesce`` (sort by (src, dst), drop duplicates) on the device, for any E.

    Up to ``max_chunk`` entries it is one ``bf_coalesce``; beyond that the
    entries are cut into ascending source ranges of at most ``max_chunk``
    entries each (a histogram of the sources picks the cuts), each range is
    coalesced alone and the results are concatenated, which is the same order.
    """
    n = int(num_nodes)
    E = int(edge_index.size(1))
    if E <= max_chunk:
        return hip_ops.coalesce(edge_index, n)
    src = edge_index[0]
    counts = torch.bincount(src.to(torch.int64), minlength=n)
    if int(counts.max()) > max_chunk:
        raise ValueError(f"one source holds more than {max_chunk} entries; cannot cut it into sort ranges")
    cum = torch.cumsum(counts, 0).cpu()
    parts, lo, taken = [], 0, 0
    while lo < n:
        # largest hi with cum[hi-1] - taken <= max_chunk
        hi = int(torch.searchsorted(cum, torch.tensor([taken + max_chunk]), right=True)[0])
        hi = max(hi, lo + 1)
        sel = edge_index[:, (src >= lo) & (src < hi)]
        if sel.numel():
            parts.append(hip_ops.coalesce(sel, n))
        taken = int(cum[hi - 1])
        lo = hi
    return torch.cat(parts, dim=1) if parts else edge_index.new_zeros((2, 0), dtype=torch.int64)


def to_bidirected(edge_index: torch.Tensor, num_nodes: int, max_chunk: int = _SORT_LIMIT) -> torch.Tensor:
    """``_to_bidirected_edge_index`` (utils/fullgraph_sp_support.py:570-572): coalesce(E ∪ flip(E))."""
    return coalesce_edges(torch.cat([edge_index, edge_index.flip(0)], dim=1), num_nodes, max_chunk)


def load_graph(dataset_path: str, device="cuda", to_bidirected_edges: bool = False,
               num_nodes: Optional[int] = None):
    """Topology ingest of ``_load_data`` (utils/fullgraph_sp_support.py:637-687): ``edge_index.pt``
    from ``dataset_path`` moved to the device, optionally made bidirected, and the walk CSR built there.

    ``num_nodes`` defaults to the row count of ``x.pt`` (read through mmap, as
    the reference sizes the graph by the features), else max id + 1. Returns
    (CSRGraph, edge_index_global on the device).
    """
    import os
    ei = load_edge_index(os.path.join(dataset_path, "edge_index.pt"))
    if num_nodes is None:
        x_path = os.path.join(dataset_path, "x.pt")
        if os.path.exists(x_path):
            num_nodes = int(torch.load(x_path, map_location="cpu", weights_only=True, mmap=True).shape[0])
        else:
            num_nodes = int(ei.max()) + 1 if ei.numel() else 0
    ei = ei.to(device=device, dtype=torch.int64, non_blocking=False)
    if to_bidirected_edges:
        ei = to_bidirected(ei, num_nodes)
        graph = CSRGraph.from_edge_index(ei, num_nodes, symmetric=True, device=device)
    else:
        graph = CSRGraph.from_edge_index(coalesce_edges(ei, num_nodes), num_nodes, device=device)
    return graph, ei


def chung_lu_device(num_nodes: int, num_edges: int, exponent: float = 2.1, seed: int = 42,
                    max_degree: Optional[float] = None, i0: float = 10.0, device="cuda") -> CSRGraph:
    """Symmetric Chung-Lu graph with ``num_edges // 2`` distinct pairs, generated in HBM (bf_chung_lu).

    Same degree law as ``chung_lu_csr`` but a different random stream; used for
    the large benchmark shapes (tens of millions to 1.6B edges).
    """
    import ctypes as C
    from . import _native as N
    from .hip_ops import _stream
    dev = torch.device(device)
    stream = _stream(dev)          # refuses a host device before anything is allocated
    pairs = int(num_edges) // 2
    ws_bytes = C.c_size_t(0)
    N.call("bf_chung_lu_workspace_size", num_nodes, pairs, C.byref(ws_bytes))
    ws = torch.empty(ws_bytes.value, dtype=torch.uint8, device=dev)
    rowptr = torch.empty(num_nodes + 1, dtype=torch.int64, device=dev)
    col = torch.empty(2 * pairs, dtype=torch.int32, device=dev)
    m = C.c_int64(0)
    N.call("bf_chung_lu", num_nodes, pairs, float(exponent), float(i0), float(max_degree or 0.0), seed & (2 ** 64 - 1),
           C.c_void_p(rowptr.data_ptr()), C.c_void_p(col.data_ptr()), C.byref(m), C.c_void_p(ws.data_ptr()),
           ws.numel(), stream)
    del ws
    return CSRGraph(rowptr, col, rowptr, col, int(num_nodes))


def chung_lu_csr(num_nodes: int, num_edges: int, exponent: float = 2.1, seed: int = 42,
                 max_degree: Optional[int] = None):
    """Symmetric power-law (Chung-Lu) graph as coalesced CSR numpy arrays.

    Expected degree of node i is proportional to (i + i0)^(-1/(exponent-1)),
    optionally capped at ``max_degree``; endpoints are drawn proportionally to
    it, self loops dropped, pairs symmetrised and deduplicated, and the
    directed edge count topped up / trimmed to ``num_edges`` (even).
    Returns (rowptr int64 [N+1], col int32 [E]).
    """
    rng = np.random.default_rng(seed)
    i0 = 10.0
    w = (np.arange(num_nodes, dtype=np.float64) + i0) ** (-1.0 / (exponent - 1.0))
    w *= num_edges / w.sum()
    if max_degree is not None:
        w = np.minimum(w, float(max_degree))
    p = w / w.sum()
    target_pairs = num_edges // 2
    keys = np.zeros(0, dtype=np.int64)
    draw = int(target_pairs * 1.15) + 16
    for _ in range(20):
        a = rng.choice(num_nodes, size=draw, p=p)
        b = rng.choice(num_nodes, size=draw, p=p)
        keep = a != b
        lo = np.minimum(a[keep], b[keep]).astype(np.int64)
        hi = np.maximum(a[keep], b[keep]).astype(np.int64)
        keys = np.unique(np.concatenate([keys, lo * num_nodes + hi]))
        if keys.size >= target_pairs:
            break
        draw = int((target_pairs - keys.size) * 1.5) + 16
    if keys.size > target_pairs:
        keys = rng.choice(keys, size=target_pairs, replace=False)
    lo, hi = keys // num_nodes, keys % num_nodes
    src = np.concatenate([lo, hi])
    dst = np.concatenate([hi, lo])
    lin = np.unique(src * num_nodes + dst)
    src, dst = lin // num_nodes, lin % num_nodes
    rowptr = np.zeros(num_nodes + 1, dtype=np.int64)
    np.add.at(rowptr, src + 1, 1)
    return np.cumsum(rowptr), dst.astype(np.int32)


def uniform_random_csr(num_nodes: int, num_edges: int, seed: int = 42):
    """Symmetric G(n, m) graph (config c1's plumbing graph) as coalesced CSR."""
    rng = np.random.default_rng(seed)
    pairs = set()
    target = num_edges // 2
    while len(pairs) < target:
        a = rng.integers(0, num_nodes, size=2 * (target - len(pairs)) + 8)
        b = rng.integers(0, num_nodes, size=a.size)
        for x, y in zip(a.tolist(), b.tolist()):
            if x != y:
                pairs.add((min(x, y), max(x, y)))
                if len(pairs) >= target:
                    break
    arr = np.array(sorted(pairs), dtype=np.int64)
    src = np.concatenate([arr[:, 0], arr[:, 1]])
    dst = np.concatenate([arr[:, 1], arr[:, 0]])
    lin = np.unique(src * num_nodes + dst)
    src, dst = lin // num_nodes, lin % num_nodes
    rowptr = np.zeros(num_nodes + 1, dtype=np.int64)
    np.add.at(rowptr, src + 1, 1)
    return np.cumsum(rowptr), dst.astype(np.int32)
