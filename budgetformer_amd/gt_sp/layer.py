"""``DistributedAttentionNoMerge`` with the reference's surface (gt_sp/layer.py:235-281).

Single GPU: the all-to-alls and the global-token copy are identities, so the
wrapper calls the local (HIP) attention directly; SP groups larger than one
rank raise.
"""
from __future__ import annotations

from typing import Any

import torch
from torch import Tensor
from torch.nn import Module

from .gt_layer import _sp_world_size


class DistributedAttentionNoMerge(torch.nn.Module):
    """Distributed attention for node-level tasks (no global-token merge)."""

    def __init__(self, local_attention: Module, sequence_process_group=None, scatter_idx: int = 2,
                 gather_idx: int = 1) -> None:
        super().__init__()
        self.local_attn = local_attention
        self.spg = sequence_process_group
        self.scatter_idx = scatter_idx
        self.gather_idx = gather_idx

    def forward(self, query: Tensor, key: Tensor, value: Tensor, attn_bias: Tensor, edge_index, attn_type,
                *args: Any) -> Tensor:
        if _sp_world_size(self.spg) != 1:
            raise NotImplementedError("sequence-parallel all-to-all (SP > 1) is outside this single-GPU build")
        return self.local_attn(query, key, value, attn_bias, edge_index, attn_type, *args)
