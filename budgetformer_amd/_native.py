"""ctypes binding of the HIP library's C ABI (include/budgetformer_hip.h).

This module is the only place that touches the shared library. Loading fails
loudly when the library has not been built: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import re

_PKG = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_PKG)
_HEADER = os.path.join(_ROOT, "include", "budgetformer_hip.h")
_LIB = os.path.join(_PKG, "_lib", "libbudgetformer_hip.so")

BF_OK, BF_ERR_INVALID, BF_ERR_UNSUPPORTED, BF_ERR_HIP = 0, 1, 2, 3
BF_DTYPE_F32, BF_DTYPE_BF16, BF_DTYPE_F16 = 0, 1, 2
ABI_VERSION = 303                   # the header's BF_ABI_VERSION this binding is written against
BF_MAX_ITEMS_PER_ROW = 160          # items a split row is cut into at most (the header's #define) ...
BF_LONG_ROW_FACTOR = 64             # ... unless it is longer than 160 * 64 items' worth (the header's #define)

i32, i64, u64, sz, f32 = C.c_int32, C.c_int64, C.c_uint64, C.c_size_t, C.c_float
vp = C.c_void_p
P_i32 = vp  # device pointers are passed as plain addresses
P_i64 = vp
P_f32 = vp


class AttnIndex(C.Structure):
    """Mirror of ``struct bf_attn_index``."""
    _fields_ = [
        ("n_q", i64), ("n_kv", i64), ("nnz", i64),
        ("qptr", vp), ("kv", vp), ("kptr", vp), ("kq", vp), ("ks", vp),
        ("chunk", i32), ("item", i32),
        ("q_items", i32), ("q_heavy", i32),
        ("q_nitems", vp), ("q_item_off", vp), ("q_item_row", vp), ("q_heavy_rows", vp),
        ("k_items", i32), ("k_heavy", i32),
        ("k_nitems", vp), ("k_item_off", vp), ("k_item_row", vp), ("k_heavy_rows", vp),
        ("k_order", vp), ("token_column", i32), ("k_spans", vp), ("plan_counts", vp),
    ]


class AttnDropout(C.Structure):
    """Mirror of ``struct bf_attn_dropout``."""
    _fields_ = [("rate", C.c_float), ("seed", u64), ("offset", u64), ("keep", vp)]


# name -> (restype, argtypes)
_SIGS = {
    "bf_version": (C.c_int, []),
    "bf_last_error": (C.c_char_p, []),
    "bf_prof_enable": (C.c_int, [i32]),
    "bf_prof_reset": (C.c_int, []),
    "bf_prof_collect": (C.c_int, []),
    "bf_prof_count": (i32, []),
    "bf_prof_get": (C.c_int, [i32, C.POINTER(C.c_char_p), C.POINTER(C.c_double), C.POINTER(i64)]),
    "bf_random_walk": (C.c_int, [P_i64, P_i32, i64, i64, i64, i32, i32, P_f32, u64, u64, P_i64, vp]),
    "bf_walk_uniforms": (C.c_int, [i64, i64, i32, i32, u64, u64, P_f32, vp]),
    "bf_random_walk_starts": (C.c_int, [P_i64, P_i32, i64, P_i64, i64, i32, P_f32, u64, u64, u64, P_i64, vp]),
    "bf_hop_pool_workspace_size": (C.c_int, [i64, i32, i32, C.POINTER(sz)]),
    "bf_hop_pool": (C.c_int, [P_i64, i64, i32, i32, P_i64, P_i64, C.POINTER(i64), vp, sz, vp]),
    "bf_fanout_sample": (C.c_int, [P_i64, P_i32, i64, i32, i32, u64, u64, P_i32, P_i32, vp]),
    "bf_frontier_offsets_workspace_size": (C.c_int, [i64, C.POINTER(sz)]),
    "bf_frontier_offsets": (C.c_int, [P_i32, i64, P_i64, P_i32, P_i64, vp, sz, vp]),
    "bf_frontier_expand": (C.c_int, [P_i32, P_i32, i64, P_i64, P_i64, P_i32, i32, P_i32, P_i32, vp]),
    "bf_frontier_emit_workspace_size": (C.c_int, [i64, C.POINTER(sz)]),
    "bf_frontier_emit": (C.c_int, [P_i32, P_i32, i64, P_i64, P_i64, P_i64, vp, sz, vp]),
    "bf_chung_lu_workspace_size": (C.c_int, [i64, i64, C.POINTER(sz)]),
    "bf_chung_lu": (C.c_int, [i64, i64, C.c_double, C.c_double, C.c_double, u64, P_i64, P_i32, C.POINTER(i64), vp, sz,
                              vp]),
    "bf_coalesce_workspace_size": (C.c_int, [i64, C.POINTER(sz)]),
    "bf_coalesce": (C.c_int, [P_i64, P_i64, i64, i64, P_i64, P_i64, C.POINTER(i64), vp, sz, vp]),
    "bf_walk_records": (C.c_int, [P_i64, P_i32, i64, i64, vp, vp]),
    "bf_rw_select": (C.c_int, [P_i64, P_i32, vp, i64, i64, i64, i32, i32, i32, i64, P_f32, u64, u64, P_i32, P_i32,
                               vp]),
    "bf_real_select_merge": (C.c_int, [P_i64, P_i32, i64, i64, i64, i32, i64, P_i32, P_i32, i32, i32, P_i32, i32,
                                       P_i32, P_i32, i64, i64, P_i32, P_i32, P_i32, i64, i64, vp]),
    "bf_rw_select_rows": (C.c_int, [P_i64, P_i32, vp, i64, P_i32, i64, i32, i32, i32, i64, P_f32, u64, u64, P_i64, P_i32,
                                    P_i32, P_i32, vp]),
    "bf_real_select_rows": (C.c_int, [P_i64, P_i32, i64, P_i32, i64, i32, i64, P_i32, i64, i64, P_i32, P_i32, P_i32,
                                      P_i32, vp]),
    "bf_assemble_rows": (C.c_int, [P_i32, P_i32, i32, i32, P_i32, P_i32, i32, i32, i32, i64, P_i32, i32, P_i32, vp]),
    "bf_mark_in_neighbors": (C.c_int, [P_i64, P_i32, i64, vp, vp, vp]),
    "bf_build_edge_table_workspace_size": (C.c_int, [i64, i32, i64, i32, C.POINTER(sz)]),
    "bf_build_edge_table": (C.c_int, [P_i64, P_i32, vp, P_i64, P_i32, i64, i64, i64, i64, i32, i32, i32, i32, i64,
                                      P_f32, u64, u64, P_i32, i64, i64, P_i32, i64, i64, P_i32, P_i32, vp, sz, vp]),
    "bf_table_csr_ptr": (C.c_int, [P_i32, i64, i32, i64, P_i64, C.POINTER(i64), vp, sz, vp]),
    "bf_check_table": (C.c_int, [P_i32, P_i32, i64, i32, i64, C.POINTER(i64), vp, sz, vp]),
    "bf_table_to_csr": (C.c_int, [P_i32, P_i32, i64, i32, i32, i64, P_i64, P_i32, vp, i32, i32, vp]),
    "bf_scan_workspace_size": (C.c_int, [i64, C.POINTER(sz)]),
    "bf_coo_to_csr_workspace_size": (C.c_int, [i64, i64, C.POINTER(sz)]),
    "bf_coo_to_csr": (C.c_int, [P_i64, P_i64, i64, i64, i64, P_i64, P_i32, vp, sz, vp]),
    "bf_reverse_index_workspace_size": (C.c_int, [i64, i64, C.POINTER(sz)]),
    "bf_reverse_index": (C.c_int, [P_i64, P_i32, i64, i64, i64, P_i64, P_i32, P_i32, vp, sz, vp]),
    "bf_reverse_index_packed_workspace_size": (C.c_int, [i64, C.POINTER(sz)]),
    "bf_reverse_index_packed": (C.c_int, [vp, P_i64, i64, i64, i64, i32, i32, i32, i64, vp, P_i64, P_i32, P_i32,
                                          vp, sz, vp]),
    "bf_radix_sort_workspace_size": (C.c_int, [i64, i32, i32, C.POINTER(sz)]),
    "bf_radix_sort_keys": (C.c_int, [vp, vp, i64, i32, i32, vp, sz, vp]),
    "bf_reverse_slots": (C.c_int, [vp, P_i64, i64, i64, i32, i32, i32, i64, P_i32, vp]),
    "bf_expand_rows": (C.c_int, [P_i64, i64, i64, P_i64, vp]),
    "bf_split_item_capacity": (i64, [i64, i32, i32]),
    "bf_split_row_capacity": (i64, [i64, i32]),
    "bf_split_row_items": (i64, [i64, i32]),
    "bf_split_plan_workspace_size": (C.c_int, [i64, C.POINTER(sz)]),
    "bf_split_plan": (C.c_int, [P_i64, i64, i32, i32, P_i32, P_i32, P_i32, i64, P_i32, i64, P_i32, vp, sz, vp]),
    "bf_split_plan_first_row": (C.c_int, [i64, i32, P_i32, P_i32, P_i32, i64, P_i32, i64, P_i32, vp]),
    "bf_row_order_workspace_size": (C.c_int, [i64, C.POINTER(sz)]),
    "bf_row_order": (C.c_int, [P_i64, i64, P_i32, vp, vp, sz, vp]),
    "bf_row_order_and_plan_workspace_size": (C.c_int, [i64, i64, C.POINTER(sz)]),
    "bf_row_order_and_plan": (C.c_int, [P_i64, i64, i32, i32, P_i32, vp, P_i32, P_i32, P_i32, i64, P_i32, i64,
                                        P_i32, vp, sz, vp]),
    "bf_attn_partials_floats": (i64, [C.POINTER(AttnIndex), i32, i32]),
    "bf_attn_bwd_noalloc": (C.c_int, [C.POINTER(AttnIndex), i32, i32, i32, f32, vp, vp, vp, P_f32, P_f32,
                                      C.POINTER(AttnDropout), P_f32, vp, vp, vp, vp, P_f32, vp]),
    "bf_attn_bwd_kv_variant": (C.c_int, [C.POINTER(AttnIndex), i32, i32, i32, C.POINTER(i32), C.POINTER(i32),
                                         C.POINTER(i32)]),
    "bf_attn_fwd": (C.c_int, [C.POINTER(AttnIndex), i32, i32, i32, f32, vp, vp, vp, P_f32, P_f32,
                              C.POINTER(AttnDropout), vp, P_f32, P_f32, vp]),
    "bf_attn_bwd": (C.c_int, [C.POINTER(AttnIndex), i32, i32, i32, f32, vp, vp, vp, P_f32, P_f32,
                              C.POINTER(AttnDropout), P_f32, vp, vp, vp, vp, P_f32, P_f32, P_f32, vp]),
    "bf_attn_typed_partials_floats": (i64, [C.POINTER(AttnIndex), i32, i32, i32]),
    "bf_gather_probe": (C.c_int, [vp, i32, vp, i32, vp, i32, P_i32, i64, C.c_uint32, i32, vp, vp]),
    "bf_row_stream_probe": (C.c_int, [vp, vp, vp, vp, i32, P_i32, i64, i32, vp, vp]),
    "bf_attn_fwd_typed": (C.c_int, [C.POINTER(AttnIndex), i32, i32, i32, vp, vp, vp, P_f32, vp, P_f32, vp]),
    "bf_attn_bwd_typed": (C.c_int, [C.POINTER(AttnIndex), i32, i32, i32, vp, vp, vp, P_f32, P_f32, vp, vp, vp, vp,
                                    P_f32, P_f32, P_f32, vp]),
}

_lib = None


def header_functions() -> list:
    """Names of every function the C header declares."""
    text = open(_HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bf_\w+)\s*\(", text)))


def lib_path() -> str:
    return _LIB


def load():
    """Load the HIP library (once). Raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.exists(path):
        raise RuntimeError(
            f"budgetformer_amd: HIP library not found at {path}; build it with "
            f"`python -m budgetformer_amd.build` (no CPU fallback exists)")
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.bf_version() != ABI_VERSION:
        raise RuntimeError(f"budgetformer_amd: {path} implements ABI {lib.bf_version()}, this binding expects "
                           f"{ABI_VERSION}; rebuild it with `python -m budgetformer_amd.build`")
    _lib = lib
    return lib


class HipError(RuntimeError):
    """A HIP runtime call or kernel launch inside the library failed."""


_OPS_LIB = os.path.join(_PKG, "_lib", "libbf_torch_ops.so")
_ops = None


def ops_path() -> str:
    return _OPS_LIB


def load_ops():
    """The TORCH_LIBRARY(bf, ...) operators (csrc/torch_ops.cpp), loaded once: returns torch.ops.bf.
    Raises if the extension was not built (no CPU fallback exists)."""
    global _ops
    if _ops is not None:
        return _ops
    import torch
    load()                      # the operators call into the HIP library: load it (and its checks) first
    if not os.path.exists(_OPS_LIB):
        raise RuntimeError(f"budgetformer_amd: torch operator library not found at {_OPS_LIB}; build it with "
                           f"`python -m budgetformer_amd.build`")
    torch.ops.load_library(_OPS_LIB)
    _ops = torch.ops.bf
    return _ops


def check(rc: int, what: str) -> None:
    if rc == BF_OK:
        return
    msg = (load().bf_last_error() or b"").decode(errors="replace")
    text = f"{what}: {msg}"
    if rc == BF_ERR_INVALID:
        raise ValueError(text)
    if rc == BF_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise HipError(text)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


class KernelTimer:
    """Per-kernel HIP-event timing inside the library (bf_prof_*)."""

    def __enter__(self):
        call("bf_prof_reset")
        call("bf_prof_enable", 1)
        return self

    def __exit__(self, *exc):
        call("bf_prof_enable", 0)
        return False

    @staticmethod
    def stats() -> dict:
        """{kernel name: (total_ms, launches)} of everything collected so far."""
        lib = load()
        call("bf_prof_collect")
        out = {}
        for i in range(lib.bf_prof_count()):
            name, ms, n = C.c_char_p(), C.c_double(), i64()
            call("bf_prof_get", i, C.byref(name), C.byref(ms), C.byref(n))
            out[name.value.decode()] = (ms.value, n.value)
        return out
