"""``DistributedAttentionNodeLevel`` with the reference's surface (gt_sp/gt_layer.py:212-253).

On one GPU the sequence-parallel all-to-all is the identity and the wrapper
calls the local (HIP) attention directly, exactly what the reference does when
sequence parallelism is not initialised (models/graphormer_dist_node_level.py:
631-637). Sequence-parallel groups of more than one rank are outside this
single-GPU build and raise.
"""
from __future__ import annotations

from typing import Any

import torch
from torch import Tensor
from torch.nn import Module


def _sp_world_size(group) -> int:
    if group is None or not torch.distributed.is_available() or not torch.distributed.is_initialized():
        return 1
    return torch.distributed.get_world_size(group)


class DistributedAttentionNodeLevel(torch.nn.Module):
    """Distributed attention for node-level tasks (GT model, no global tokens)."""

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
