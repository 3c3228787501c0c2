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


def test_working_set_is_the_hot_path_estimate_and_fits_one_gpu_at_c5():
    """The planner's working set (gt_sp/utils.py:160-236 counterpart) is the walk records plus the peak of
    the build and its index; at c5's shard (27.8M queries, B = 8 with the token) it is a small part of one
    MI355X, and even an all-node build of the 111M-node graph at the pool's budget fits."""
    N, E, P, L = 111_059_956, 1_600_000_000, 2, 4
    est = gu.estimate_hot_path_bytes(N, E, N, P * L, P * L)
    assert gu._estimate_rw_working_set_bytes(N, E, P, L) == est["peak"] + 16 * E
    assert gu._estimate_rw_working_set_bytes(N, E, P, L, walk_records_built=True) == est["peak"]
    shard = gu.estimate_hot_path_bytes(N, E, 27_800_000, 4, 4, global_token=True, nnz=349_331_165)
    assert shard["exact"] and shard["entries"] == 349_331_165
    assert 8e9 < shard["peak"] < 16e9 and shard["walk_records"] == 16 * E
    assert gu._estimate_rw_working_set_bytes(N, E, P, L) < 288 * 2 ** 30


def test_hot_path_estimate_parts():
    """The estimate replays the allocations: the peak holds at least what stays resident, which holds the
    table, row lengths and the index arrays; an exactly sized index (more than 8M entries at capacity)
    follows the entry count it is given, a capacity-sized one (up to 8M) does not; the slots (entries)
    add 4 bytes per entry to what stays."""
    big = gu.estimate_hot_path_bytes(2_000_000, 20_000_000, 2_000_000, 8, 8)
    assert big["exact"] and big["entries"] == 32_000_000
    part = gu.estimate_hot_path_bytes(2_000_000, 20_000_000, 2_000_000, 8, 8, nnz=20_000_000)
    assert part["peak"] < big["peak"] and part["entries"] == 20_000_000
    # bytes per entry that stay: kv + kq = 8, the sorted keys 8 (kept for a later slot decode)
    per_entry = (big["resident"] - part["resident"]) / 12_000_000
    assert 15.9 < per_entry < 16.1
    small = gu.estimate_hot_path_bytes(500_000, 5_000_000, 500_000, 4, 4)
    assert not small["exact"] and gu.estimate_hot_path_bytes(500_000, 5_000_000, 500_000, 4, 4,
                                                             nnz=1000)["peak"] == small["peak"]
    ent = gu.estimate_hot_path_bytes(2_000_000, 20_000_000, 2_000_000, 8, 8, nnz=20_000_000, entries=True)
    # with the slots the sorted keys (8 B) go and ks (4 B) stays
    assert abs((part["resident"] - ent["resident"]) / 20_000_000 - 4.0) < 0.01
    for e in (big, part, small, ent):
        table = gu.estimate_edge_build_bytes(e["live_after"]["row_len"] // 4, 8, 8)["output"]
        assert e["peak"] >= e["resident"] >= e["live_after"]["table"]
        assert e["build_peak"] <= e["peak"]
        assert table > 0


def test_plan_reserves_the_index():
    """A build whose table fits but whose table plus index reserve does not is sharded so that the shard's
    transient, the table and the reserve fit; with no room left for even a one-query shard it raises."""
    n_q, b_r, b_w = 1_000_003, 4, 4
    out = gu.estimate_edge_build_bytes(n_q, b_r, b_w)["output"]
    full = gu.estimate_edge_build_bytes(n_q, b_r, b_w)["transient"]
    reserve = 50 * 2 ** 20
    usable = out + reserve + full // 3
    plan = gu.plan_edge_build("cpu", n_q, b_r, b_w, usable_bytes=usable, reserve_bytes=reserve)
    assert len(plan.shards) > 1 and plan.transient_bytes + out + reserve <= usable
    assert gu.plan_edge_build("cpu", n_q, b_r, b_w, usable_bytes=usable).shards == [(0, n_q)]
    with pytest.raises(torch.cuda.OutOfMemoryError):
        gu.plan_edge_build("cpu", n_q, b_r, b_w, usable_bytes=out + reserve, reserve_bytes=reserve)


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

    def room(b_r, b_w, extra):
        # the table, the reserve for its attention index, and `extra` bytes for the build's transient
        est = gu.estimate_hot_path_bytes(n, g.num_edges, n, b_r, b_w, n_hubs=int(g.hubs().numel()))
        return est["peak"] + extra

    shard = build_attention_edges(g, real_edges_per_query=4, rw_edges_per_query=4, edge_seed=5,
                                  usable_bytes=room(4, 4, 60_000))
    assert torch.equal(full.table, shard.table) and torch.equal(full.row_len, shard.row_len)
    u = torch.rand(n * 2, 4, generator=torch.Generator().manual_seed(1)).to(hip_device)
    a = build_attention_edges(g, real_edges_per_query=3, rw_edges_per_query=5, edge_seed=5, u=u)
    b = build_attention_edges(g, real_edges_per_query=3, rw_edges_per_query=5, edge_seed=5, u=u,
                              usable_bytes=room(3, 5, 40_000))
    assert torch.equal(a.table, b.table)


@pytest.mark.gpu
@pytest.mark.parametrize("n,e,b_r,b_w,token,entries", [(2_449_029, 30_000_000, 8, 8, False, False),
                                                        (2_000_000, 20_000_000, 4, 4, True, True),
                                                        (2_000_000, 16_000_000, 1, 1, False, False)])
def test_measured_peak_of_build_and_index_matches_the_estimate(hip_device, n, e, b_r, b_w, token, entries):
    """One edge build and its attention index (reverse index, plans, row order; the slots with
    ``entries``) on a device graph of 2M+ nodes: the caching allocator's peak above what was allocated
    before (torch.cuda.max_memory_allocated) is within 10% of estimate_hot_path_bytes' peak, and what
    stays allocated within 10% of its resident bytes. The graph's walk records, hub and heavy lists are
    built first (the graph holds them across builds). Cases: B = 16 without the token (an exactly sized
    index), B = 8 with the token row and the slots, B = 2 (an index sized at capacity, nothing read back)."""
    from budgetformer_amd.edges import build_attention_edges
    from budgetformer_amd.graph import chung_lu_device
    g = chung_lu_device(n, e, exponent=2.1, seed=7, device=hip_device)
    g.walk_records(), g.hubs(), g.heavy()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(hip_device)
    torch.cuda.reset_peak_memory_stats(hip_device)
    tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=4,
                                walks_per_node=2, edge_seed=42, global_token=token)
    idx = tab.attention_index()
    idx.ensure_backward(entries=entries)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(hip_device) - base
    resident = torch.cuda.memory_allocated(hip_device) - base
    est = gu.estimate_hot_path_bytes(n, g.num_edges, n, b_r, b_w, global_token=token, nnz=idx.nnz,
                                     entries=entries, n_hubs=int(g.hubs().numel()))
    assert est["exact"] == (b_r + b_w > 2)
    assert abs(peak - est["peak"]) <= 0.10 * est["peak"], (peak, est["peak"])
    assert abs(resident - est["resident"]) <= 0.10 * est["resident"], (resident, est["resident"])
    print(f"[memory] n={n:,} B={b_r + b_w} token={token}: peak {peak / 2**20:.1f} MiB (estimate "
          f"{est['peak'] / 2**20:.1f}), resident {resident / 2**20:.1f} MiB (estimate {est['resident'] / 2**20:.1f})")
