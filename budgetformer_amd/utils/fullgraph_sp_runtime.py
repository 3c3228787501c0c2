"""Runtime helpers of the hot path (utils/fullgraph_sp_runtime.py)."""
from __future__ import annotations


def _edge_seed_for_epoch(epoch: int, *, args, use_epoch_seed: bool, adaptive_edge_budget_cfg):
    """Per-epoch edge seed (utils/fullgraph_sp_runtime.py:221-226).

    None when epoch seeding is off; ``args.seed`` during the static-seed epochs;
    ``args.seed + epoch`` afterwards.
    """
    if not use_epoch_seed:
        return None
    if epoch <= adaptive_edge_budget_cfg.static_seed_epochs:
        return args.seed
    return args.seed + epoch
