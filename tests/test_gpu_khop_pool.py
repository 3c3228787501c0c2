"""GPU parity of the fanout k-hop pool (rw_edge_mode "dgl_neighbor", compute_khop_pool_dgl_neighbor,
gt_sp/utils.py:1281-1384) against the CPU oracle: the per-node samples, the pool (order and content) for
sampled and all-neighbour hops, and the budgeted edge pipeline built on it. Integer outputs: bit-exact."""
import types

import numpy as np
import pytest
import torch

from oracle import edge_table as et

pytestmark = pytest.mark.gpu


def _graph(n, e, seed):
    from budgetformer_amd.graph import chung_lu_csr
    rowptr, col = chung_lu_csr(n, e, seed=seed)
    src = np.repeat(np.arange(n), np.diff(rowptr))
    return rowptr, col, np.stack([src, col.astype(np.int64)])


@pytest.mark.parametrize("fanout", [1, 3, 10, 64])
def test_fanout_sample_equals_oracle(hip_device, fanout):
    from budgetformer_amd import hip_ops
    n = 3000
    rowptr, col, _ = _graph(n, 40000, seed=fanout)           # power law: hubs far above every fanout
    assert np.diff(rowptr).max() > 64
    rp = torch.from_numpy(rowptr).to(hip_device)
    cl = torch.from_numpy(col.astype(np.int32)).to(hip_device)
    for hop, seed in ((1, 5), (2, 5), (1, 2 ** 40 + 3)):
        cnt, sel = hip_ops.fanout_sample(rp, cl, fanout, hop, seed)
        ptr, ids = et.fanout_sample(rowptr, col, n, fanout, hop, seed)
        cnt, sel = cnt.cpu().numpy(), sel.cpu().numpy()
        assert np.array_equal(cnt, np.diff(ptr))
        for u in range(n):
            assert np.array_equal(sel[u, :cnt[u]], ids[ptr[u]:ptr[u + 1]]), (hop, seed, u)


@pytest.mark.parametrize("fanout,min_hop", [([10, 5], 1), ([10, 5], 2), ([-1, 3], 1), ([4, 4, 4], 1), ([2], 1),
                                            ([3, 0, 2], 1)])
def test_khop_pool_equals_oracle(hip_device, fanout, min_hop):
    from budgetformer_amd import hip_ops
    n = 2000
    rowptr, col, _ = _graph(n, 16000, seed=9)
    rp = torch.from_numpy(rowptr).to(hip_device)
    cl = torch.from_numpy(col.astype(np.int32)).to(hip_device)
    got = hip_ops.khop_fanout_pool(rp, cl, fanout, seed=77, min_hop=min_hop).cpu().numpy()
    ref = et.khop_fanout_pool(rowptr, col, n, fanout, seed=77, min_hop=min_hop)
    assert got.shape == ref.shape and np.array_equal(got, ref)


def test_khop_pool_all_neighbours_and_reference_surface(hip_device):
    """fanout -1 at both hops (no sampler: exact 2-step paths) through the reference-named entry point, on
    an edge list with a self loop, a repeated edge (both kept, as dgl.graph keeps them) and three isolated
    tail nodes."""
    from budgetformer_amd.gt_sp.utils import compute_khop_pool_dgl_neighbor
    n = 400
    _, _, ei = _graph(n, 3000, seed=2)
    ei = np.concatenate([ei, [[5], [5]], ei[:, :1]], axis=1)
    ei = ei[:, np.lexsort((ei[1], ei[0]))]
    got = compute_khop_pool_dgl_neighbor(torch.from_numpy(ei).to(hip_device), n + 3, [-1, -1], device=hip_device)
    ptr = np.concatenate([[0], np.cumsum(np.bincount(ei[0], minlength=n + 3))])
    ref = et.khop_fanout_pool(ptr, ei[1], n + 3, [-1, -1])
    assert np.array_equal(got.cpu().numpy(), ref)
    empty = torch.zeros((2, 0), dtype=torch.long, device=hip_device)
    assert compute_khop_pool_dgl_neighbor(empty, 10, [10, 5], device=hip_device).shape == (2, 0)


@pytest.mark.parametrize("model,b", [("graphormer", 8), ("gt", 6)])
def test_budgeted_pipeline_on_the_fanout_pool(hip_device, model, b):
    """_build_merged_edges with rw_edge_mode "dgl_neighbor" and random edge blocks: the real part and the
    RW part (top keys per query over the fanout pool) merged, as the reference's pipeline composes them."""
    from budgetformer_amd.utils import fullgraph_sp_support as fs
    n, seed = 1500, 44
    rowptr, col, ei = _graph(n, 12000, seed=5)
    args = types.SimpleNamespace(model=model, num_global_node=1, seed=42, walks_per_node=2, walk_length=4,
                                 max_total_edges_per_query=b, num_heads=8, random_edge_blocks=True,
                                 rw_edge_mode="dgl_neighbor", fanout="10,5")
    got = fs._build_merged_edges(args, torch.from_numpy(ei).to(hip_device), n, hip_device, hip_device, n,
                                 edge_seed=seed).cpu().numpy()
    b_r, b_w = (b + 1) // 2, b // 2
    real = et.sample_edges_per_query_random(ei, b_r, seed + 17)
    pool = et.khop_fanout_pool(rowptr, col, n, [10, 5], seed=seed)
    rw = et.sample_edges_per_query_random(pool, b_w, seed + 37)
    ref = et.merge_edge_index_list([real, rw])
    if model == "graphormer":
        ref = et.fix_edge_index(ref, n)
    assert np.array_equal(got, ref)
    # the pool is cached on args under its mode and fanout
    cached = args._cached_full_rw_pool
    assert cached["key"][-2:] == ("dgl_neighbor", (10, 5))
    assert np.array_equal(cached["pool"].cpu().numpy(), pool)
