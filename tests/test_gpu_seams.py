"""GPU checks of the per-seam mirrors (walk from starts, hop pool, per-query sampling,
coalesce-merge, the whole _build_merged_edges) against the CPU oracle."""
import types

import numpy as np
import pytest
import torch

from oracle import edge_table as et
from oracle import philox

pytestmark = pytest.mark.gpu


def _graph(n, e, seed):
    from budgetformer_amd.graph import chung_lu_csr
    rowptr, col = chung_lu_csr(n, e, seed=seed)
    src = np.repeat(np.arange(n), np.diff(rowptr))
    return rowptr, col, np.stack([src, col.astype(np.int64)])


def test_run_random_walk_and_hop_pool_bit_exact(hip_device):
    from budgetformer_amd.gt_sp import utils as gu
    n, P, L = 1200, 2, 5
    rowptr, col, ei = _graph(n, 9000, seed=1)
    ei_t = torch.from_numpy(ei).to(hip_device)
    _, rp, cl = gu._get_random_walk_graph(ei_t, n, hip_device)
    assert np.array_equal(rp.cpu().numpy(), rowptr) and np.array_equal(cl.cpu().numpy(), col)
    starts = torch.arange(n, device=hip_device).repeat_interleave(P)
    u = np.random.default_rng(2).random((n * P, L), dtype=np.float32)
    walks = gu._run_random_walk(None, rp, cl, starts, L, u=torch.from_numpy(u).to(hip_device))
    ref_walks = et.random_walk(rowptr, col, et.walk_starts(n, P), L, u)
    assert np.array_equal(walks.cpu().numpy(), ref_walks)
    for min_hop in (1, 2):
        from budgetformer_amd import hip_ops
        assert np.array_equal(hip_ops.hop_pool(walks, min_hop).cpu().numpy(),
                              et.hop_edges_from_walks(ref_walks, min_hop))
    # Philox default stream == the fused builder's stream for the same seed
    w2 = gu._run_random_walk(None, rp, cl, starts, L, seed=77)
    assert np.array_equal(w2.cpu().numpy(),
                          et.random_walk(rowptr, col, et.walk_starts(n, P), L, philox.walk_uniforms(0, n, P, L, 77)))
    pool = gu.build_head_hop_edges(ei_t, n, 8, 1, hip_device, L, P, u=torch.from_numpy(u).to(hip_device))
    assert np.array_equal(pool.cpu().numpy(), et.hop_edges_from_walks(ref_walks))


def test_sample_edges_per_query_matches_oracle_multiset(hip_device):
    from budgetformer_amd.utils.fullgraph_sp_support import _sample_edges_per_query_random
    rng = np.random.default_rng(3)
    n = 800
    ei = np.stack([rng.integers(0, n, 9000), rng.integers(0, n, 9000)])   # duplicates included
    for k, seed in ((1, 59), (4, 79), (9, 5)):
        got = _sample_edges_per_query_random(torch.from_numpy(ei).to(hip_device), k, seed)
        ref = et.sample_edges_per_query_random(ei, k, seed)
        assert sorted(map(tuple, got.cpu().numpy().T.tolist())) == sorted(map(tuple, ref.T.tolist()))


def test_merge_edge_index_list_is_coalesce(hip_device):
    from budgetformer_amd.gt_sp.utils import _merge_edge_index_list
    rng = np.random.default_rng(4)
    a = rng.integers(0, 300, (2, 2000))
    b = rng.integers(0, 300, (2, 700))
    got = _merge_edge_index_list([torch.from_numpy(a).to(hip_device), torch.from_numpy(b).to(hip_device)])
    assert np.array_equal(got.cpu().numpy(), et.merge_edge_index_list([a, b]))
    one = torch.from_numpy(a).to(hip_device)
    assert _merge_edge_index_list([one, None]) is one


@pytest.mark.parametrize("model,b", [("graphormer", 8), ("gt", 8), ("graphormer", 5)])
def test_build_merged_edges_reference_surface(hip_device, model, b):
    from budgetformer_amd.utils.fullgraph_sp_support import _build_merged_edges
    n, P, L = 1500, 2, 4
    rowptr, col, ei = _graph(n, 12000, seed=5)
    args = types.SimpleNamespace(model=model, num_global_node=1, seed=42, walks_per_node=P, walk_length=L,
                                 max_total_edges_per_query=b, num_heads=8)
    got = _build_merged_edges(args, torch.from_numpy(ei).to(hip_device), n, hip_device, hip_device, n, edge_seed=44)
    u = philox.walk_uniforms(0, n, P, L, 44)
    ref = et.build_merged_edges(ei, n, (b + 1) // 2, b // 2, L, P, 44, u,
                                graphormer_global_token=(model == "graphormer"))
    assert np.array_equal(got.cpu().numpy(), ref)
