"""Edge-build planning (a4): working-set estimates and the sharded on-GPU build."""
import pytest
import torch

from budgetformer_amd.gt_sp import utils as gu


def test_estimate_matches_library_workspace_query():
    import ctypes as C
    from budgetformer_amd import _native as N
    for n_q, b_w in ((1, 1), (1000, 4), (169_343, 4), (27_800_000, 4), (5, 16)):
        out = C.c_size_t(0)
        N.call("bf_build_edge_table_workspace_size", n_q, b_w, 0, 4, C.byref(out))
        assert gu.estimate_edge_build_bytes(n_q, 4, b_w)["transient"] == out.value


def test_fused_estimate_is_far_below_reference_pipeline_at_c5():
    # c5: 111M nodes, 1.6B edges, P=2, L=4. The reference's torch_cluster pipeline
    # (gt_sp/utils.py:160-236) needs ~6*E*8 B of sort transients plus walks and pool.
    N, E, P, L = 111_059_956, 1_600_000_000, 2, 4
    ref_like = 6 * E * 8 + N * P * (L + 1) * 8 + N * P * 33 + 2 * N * P * L * 8
    ours = gu._estimate_rw_working_set_bytes(N, E, P, L)
    assert ours == gu.estimate_edge_build_bytes(N, 0, P * L)["transient"]
    assert ours < ref_like / 10
    assert ours < 288 * 2 ** 30      # fits one MI355X


def test_plan_shards_cover_range_and_fit():
    n_q, b_r, b_w = 1_000_003, 4, 4
    out = gu.estimate_edge_build_bytes(n_q, b_r, b_w)["output"]
    usable = out + 3 * 2 ** 20
    plan = gu.plan_edge_build("cpu", n_q, b_r, b_w, q_lo=17, usable_bytes=usable)
    assert len(plan.shards) > 1
    lo = 17
    for a, cnt in plan.shards:
        assert a == lo and cnt > 0
        lo += cnt
    assert lo == 17 + n_q
    assert plan.transient_bytes + out <= usable


def test_plan_single_shard_when_it_fits():
    plan = gu.plan_edge_build("cpu", 1000, 4, 4, usable_bytes=10 ** 9)
    assert plan.shards == [(0, 1000)]


def test_plan_raises_oom_when_table_cannot_fit():
    with pytest.raises(torch.cuda.OutOfMemoryError):
        gu.plan_edge_build("cpu", 10 ** 6, 4, 4, usable_bytes=10 ** 6)


def test_no_cpu_build_device():
    with pytest.raises(ValueError):
        gu._safe_rw_device("cpu", None, 10, 10)


@pytest.mark.gpu
def test_sharded_build_is_bit_identical(hip_device):
    from budgetformer_amd.edges import build_attention_edges
    from budgetformer_amd.graph import CSRGraph, chung_lu_csr
    n = 20_000
    rowptr, col = chung_lu_csr(n, 150_000, seed=3)
    g = CSRGraph.from_csr(rowptr, col, n, device=hip_device)
    full = build_attention_edges(g, real_edges_per_query=4, rw_edges_per_query=4, edge_seed=5)
    out_bytes = gu.estimate_edge_build_bytes(n, 4, 4)["output"]
    shard = build_attention_edges(g, real_edges_per_query=4, rw_edges_per_query=4, edge_seed=5,
                                  usable_bytes=out_bytes + 60_000)
    assert torch.equal(full.table, shard.table) and torch.equal(full.row_len, shard.row_len)
    u = torch.rand(n * 2, 4, generator=torch.Generator().manual_seed(1)).to(hip_device)
    a = build_attention_edges(g, real_edges_per_query=3, rw_edges_per_query=5, edge_seed=5, u=u)
    b = build_attention_edges(g, real_edges_per_query=3, rw_edges_per_query=5, edge_seed=5, u=u,
                              usable_bytes=gu.estimate_edge_build_bytes(n, 3, 5)["output"] + 40_000)
    assert torch.equal(a.table, b.table)
