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


@pytest.mark.parametrize("k", [33, 40, 100])
def test_sample_edges_per_query_beyond_one_batch_keeps_multiplicity(hip_device, k):
    """K above the 32-entry register lists: the selection runs in batches, ordered by (key, position in the
    row), so a pair repeated in the pool keeps its multiplicity across a batch boundary. A few queries
    take 400-1600 candidates (a hub, several copies of the same pair each), the rest few."""
    from budgetformer_amd.utils.fullgraph_sp_support import _sample_edges_per_query_random
    rng = np.random.default_rng(k)
    n = 600
    base = np.stack([rng.integers(0, n, 20000), rng.integers(0, n, 20000)])
    hub = np.stack([rng.integers(0, 30, 1600), np.full(1600, 7)])       # 1600 candidates over 30 sources
    ei = np.concatenate([base, hub, hub[:, :400] * np.array([[1], [0]]) + np.array([[0], [9]])], axis=1)
    got = _sample_edges_per_query_random(torch.from_numpy(ei).to(hip_device), k, 11)
    ref = et.sample_edges_per_query_random(ei, k, 11)
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
                                 max_total_edges_per_query=b, num_heads=8, random_edge_blocks=True)
    got = _build_merged_edges(args, torch.from_numpy(ei).to(hip_device), n, hip_device, hip_device, n, edge_seed=44)
    u = philox.walk_uniforms(0, n, P, L, 44)
    ref = et.build_merged_edges(ei, n, (b + 1) // 2, b // 2, L, P, 44, u,
                                graphormer_global_token=(model == "graphormer"))
    assert np.array_equal(got.cpu().numpy(), ref)


def _pairs(ei):
    return sorted(zip(ei[0].tolist(), ei[1].tolist()))


def test_build_merged_edges_exphormer_typed_and_unbudgeted(hip_device):
    from budgetformer_amd.utils import fullgraph_sp_support as fs
    n, P, L, seed = 1200, 2, 4, 31
    rowptr, col, ei = _graph(n, 9000, seed=6)
    ei_t = torch.from_numpy(ei).to(hip_device)
    u = philox.walk_uniforms(0, n, P, L, seed)
    # Exphormer RW mode, fixed budgets (3, 5): real part type 0, RW part type 1, not merged
    args = types.SimpleNamespace(model="exphormer", expander_degree=0, seed=1, walks_per_node=P, walk_length=L,
                                 fixed_real_edges_per_query=3, fixed_rw_edges_per_query=5, num_heads=8)
    typed = fs._build_merged_edges(args, ei_t, n, hip_device, hip_device, n, edge_seed=seed).cpu().numpy()
    assert typed.shape[0] == 3
    real = et.build_merged_edges(ei, n, 3, 0, L, P, seed, u)
    rw = et.build_merged_edges(ei, n, 0, 5, L, P, seed, u)
    assert _pairs(typed[:2, typed[2] == 0]) == _pairs(real) and _pairs(typed[:2, typed[2] == 1]) == _pairs(rw)
    # unbudgeted (no fixed / adaptive / random-block budgets): whole graph merged with the whole pool
    args = types.SimpleNamespace(model="graphormer", num_global_node=1, seed=1, walks_per_node=P, walk_length=L,
                                 include_real_edges=1, num_heads=8)
    got = fs._build_merged_edges(args, ei_t, n, hip_device, hip_device, n, edge_seed=seed).cpu().numpy()
    pool = et.build_head_hop_edges(rowptr, col, n, L, P, u)
    assert np.array_equal(got, et.fix_edge_index(et.merge_edge_index_list([ei, pool]), n))


def test_full_rw_pool_cache_and_attention_edges_cache(hip_device):
    from budgetformer_amd.utils import fullgraph_sp_support as fs
    n, P, L, seed = 1000, 2, 4, 12
    rowptr, col, ei = _graph(n, 7000, seed=8)
    ei_t = torch.from_numpy(ei).to(hip_device)
    args = types.SimpleNamespace(model="gt", seed=3, walks_per_node=P, walk_length=L, max_total_edges_per_query=8,
                                 num_heads=8, random_edge_blocks=True)
    pool = fs._build_or_retrieve_full_rw_pool(args, ei_t, n, hip_device, L, P, 8, seed)
    assert np.array_equal(pool.cpu().numpy(),
                          et.build_head_hop_edges(rowptr, col, n, L, P, philox.walk_uniforms(0, n, P, L, seed)))
    assert fs._build_or_retrieve_full_rw_pool(args, ei_t, n, hip_device, L, P, 8, seed) is pool   # single-slot hit
    fs.clear_merged_edge_cache()
    a = fs._build_attention_edges(args, ei_t, n, hip_device, hip_device, None, 0, 0, n, edge_seed=seed)
    b = fs._build_attention_edges(args, ei_t, n, hip_device, hip_device, None, 0, 0, n, edge_seed=seed)
    assert b is a and len(fs._MERGED_EDGE_CACHE) == 1                                   # cached under the key
    ref = et.build_merged_edges(ei, n, 4, 4, L, P, seed, philox.walk_uniforms(0, n, P, L, seed))
    assert np.array_equal(a.cpu().numpy(), ref)
    c = fs._build_attention_edges(args, ei_t, n, hip_device, hip_device, None, 0, 0, n, edge_seed=seed + 1)
    assert len(fs._MERGED_EDGE_CACHE) == 2 and not torch.equal(c, a)


def test_probe_seams_match_oracle(hip_device):
    from budgetformer_amd.utils import fullgraph_sp_support as fs
    n, P, L, seed = 1500, 2, 4, 5
    rowptr, col, ei = _graph(n, 10000, seed=9)
    ei_t = torch.from_numpy(ei).to(hip_device)
    probe = torch.tensor([3, 90, 700, 1499])
    F = fs._expand_probe_idx_for_reception(probe, ei_t, 2)
    assert np.array_equal(F.numpy(), et.reception_cone(ei, probe.numpy(), 2))
    u = philox.walk_uniforms(0, n, P, L, seed)
    ref_pools = et.probe_edge_pools(ei, n, F.numpy(), L, P, u)
    for model, state in (("graphormer", {"real_edges_per_query": 4, "rw_edges_per_query": 4}),
                         ("gt", {"real_edges_per_query": 6, "rw_edges_per_query": 2}),
                         ("gt", {"real_edges_per_query": 0, "rw_edges_per_query": 3})):
        args = types.SimpleNamespace(model=model, num_global_node=1, seed=1, walks_per_node=P, walk_length=L,
                                     max_total_edges_per_query=8, num_heads=8, random_edge_blocks=True)
        got = fs._build_probe_attention_edges(args, ei_t, n, hip_device, hip_device, None, 0, 0, n, probe,
                                              edge_seed=seed, edge_budget_state=state, edge_dst_filter=F)
        ref = et.assemble_edges_from_pools(ref_pools, n, state["real_edges_per_query"], state["rw_edges_per_query"],
                                           seed, graphormer_global_token=(model == "graphormer"))
        if state["real_edges_per_query"] and state["rw_edges_per_query"]:
            assert np.array_equal(got.cpu().numpy(), ref)
        else:
            assert _pairs(got.cpu().numpy()) == _pairs(ref)


def test_graph_caches_do_not_confuse_tensors_at_a_reused_address(hip_device):
    """Two edge lists of the same shape, the first freed before the second is made: the cached CSR
    must follow the tensor, not its (reusable) device address."""
    from budgetformer_amd.utils import fullgraph_sp_support as fs
    n, P, L, seed = 900, 2, 4, 3
    args = types.SimpleNamespace(model="gt", seed=1, walks_per_node=P, walk_length=L, max_total_edges_per_query=6,
                                 num_heads=8, random_edge_blocks=True)
    for graph_seed in (21, 22):
        rowptr, col, ei = _graph(n, 6000, seed=graph_seed)
        ei_t = torch.from_numpy(ei).to(hip_device)
        got = fs._build_merged_edges(args, ei_t, n, hip_device, hip_device, n, edge_seed=seed)
        ref = et.build_merged_edges(ei, n, 3, 3, L, P, seed, philox.walk_uniforms(0, n, P, L, seed))
        assert np.array_equal(got.cpu().numpy(), ref)
        del ei_t, got
