"""MI355X-native (gfx950) implementation of BudgetFormer's per-layer hot path.

  * budgeted query-centric edge construction (``edges.build_attention_edges``)
  * sparse edge attention forward/backward (``attention``)

Both run as hand-written HIP kernels behind the C ABI in
``include/budgetformer_hip.h`` (library ``_lib/libbudgetformer_hip.so``, built
by ``python -m budgetformer_amd.build``). There is no CPU fallback: every entry
point raises if the library is missing or a tensor is not on a HIP device.
"""
from . import _native
from .attention import (CoreAttention, ExphormerCoreAttention, GPSCoreAttention, GTCoreAttention,
                        sparse_edge_attention)
from .edges import EdgeTable, build_attention_edges
from .graph import CSRGraph
from .hip_ops import AttentionIndex

__all__ = [
    "AttentionIndex", "CSRGraph", "CoreAttention", "EdgeTable", "ExphormerCoreAttention", "GPSCoreAttention",
    "GTCoreAttention",
    "build_attention_edges", "sparse_edge_attention",
]


def library_path() -> str:
    return _native.lib_path()
