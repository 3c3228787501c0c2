"""GPU parity of the HIP edge builder against the CPU oracle: bit-exact integer output."""
import math

import numpy as np
import pytest
import torch

from oracle import edge_table as et
from oracle import philox
from oracle import sparse_attention as sa

pytestmark = pytest.mark.gpu


def _graph(n, e, seed, exponent=2.1):
    from budgetformer_amd.graph import chung_lu_csr
    return chung_lu_csr(n, e, exponent=exponent, seed=seed)


def _dev_graph(rowptr, col, n, dev):
    from budgetformer_amd.graph import CSRGraph
    return CSRGraph.from_csr(rowptr, col, n, device=dev)


@pytest.mark.parametrize("P,L", [(2, 4), (4, 8), (1, 1), (3, 5)])
def test_random_walk_injected_u_bit_exact(hip_device, P, L):
    from budgetformer_amd import hip_ops
    n = 3000
    rowptr, col = _graph(n, 20000, seed=P * 10 + L)
    g = _dev_graph(rowptr, col, n, hip_device)
    u = np.random.default_rng(L).random((n * P, L), dtype=np.float32)
    u[0] = np.float32(1) - np.float32(2 ** -24)      # last-neighbour edge case
    walks = hip_ops.random_walk(g.rowptr, g.col, 0, n, P, L, u=torch.from_numpy(u).to(hip_device))
    ref = et.random_walk(rowptr, col, et.walk_starts(n, P), L, u)
    assert np.array_equal(walks.cpu().numpy(), ref)
    # shard: queries [100, 700)
    us = u[100 * P:700 * P]
    ws = hip_ops.random_walk(g.rowptr, g.col, 100, 600, P, L, u=torch.from_numpy(us).to(hip_device))
    assert np.array_equal(ws.cpu().numpy(), ref[100 * P:700 * P])


def test_philox_uniforms_and_walk_bit_exact(hip_device):
    from budgetformer_amd import hip_ops
    n, P, L = 2000, 2, 6
    rowptr, col = _graph(n, 12000, seed=5)
    g = _dev_graph(rowptr, col, n, hip_device)
    for seed, off in ((42, 0), (2 ** 40 + 7, 3)):
        u_gpu = hip_ops.walk_uniforms(0, n, P, L, seed, off, device=hip_device).cpu().numpy()
        u_ref = philox.walk_uniforms(0, n, P, L, seed, off)
        assert np.array_equal(u_gpu, u_ref)
        walks = hip_ops.random_walk(g.rowptr, g.col, 0, n, P, L, philox_seed=seed, philox_offset=off)
        assert np.array_equal(walks.cpu().numpy(), et.random_walk(rowptr, col, et.walk_starts(n, P), L, u_ref))


def test_device_philox_known_answers(hip_device):
    """The device Philox against the Random123 zero vector directly: walk 0, seed 0, offset 0,
    steps 0..3 are the four published output words (0x6627E8D5, 0xE169C58D, 0xBC57AC4C,
    0x9B00DBD8) mapped to (x >> 8) * 2^-24."""
    from budgetformer_amd import hip_ops
    u = hip_ops.walk_uniforms(0, 1, 1, 4, 0, 0, device=hip_device).cpu().numpy()[0]
    words = (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)
    assert [float(x) for x in u] == [float(np.float32((w >> 8) / 16777216.0)) for w in words]


def test_philox_uniforms_are_uniform(hip_device):
    from budgetformer_amd import hip_ops
    u = hip_ops.walk_uniforms(0, 200_000, 2, 4, 1234, device=hip_device).cpu().numpy().ravel()
    assert u.min() >= 0.0 and u.max() < 1.0
    counts = np.histogram(u, bins=64, range=(0.0, 1.0))[0]
    expected = u.size / 64
    chi2 = ((counts - expected) ** 2 / expected).sum()
    assert chi2 < 120          # 63 dof: p ~ 4e-5 at 120


def _rows(table, row_len):
    return [table[i, :row_len[i]].tolist() for i in range(table.shape[0])]


@pytest.mark.parametrize("b_r,b_w,P,L", [(4, 4, 2, 4), (3, 0, 2, 4), (0, 3, 2, 4), (8, 8, 4, 4), (16, 16, 4, 8),
                                         (2, 5, 1, 3), (1, 1, 2, 4), (20, 12, 4, 8)])
def test_edge_table_bit_exact(hip_device, b_r, b_w, P, L):
    from budgetformer_amd.edges import build_attention_edges
    n = 2500
    rowptr, col = _graph(n, 30000, seed=b_r * 100 + b_w)
    g = _dev_graph(rowptr, col, n, hip_device)
    u = np.random.default_rng(b_r + 7 * b_w).random((n * P, L), dtype=np.float32)
    tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                walks_per_node=P, edge_seed=42, u=torch.from_numpy(u).to(hip_device))
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, 42, u)
    assert np.array_equal(tab.row_len.cpu().numpy(), ref_len)
    assert np.array_equal(tab.table.cpu().numpy(), ref_t)


@pytest.mark.parametrize("b_r,b_w,P,L", [(48, 48, 4, 20), (40, 0, 2, 4), (0, 40, 8, 10), (33, 64, 16, 6)])
def test_edge_table_past_the_former_caps(hip_device, b_r, b_w, P, L):
    """Budgets above 32 per part and walk shapes above 64 candidates per query (B = 96 with P*L = 80,
    P*L = 96 with 16 walks): the real top-k in batches (including rows past the hub threshold), the RW
    selection sorted in LDS, merged rows of up to 97 ids; bit-exact against the oracle."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.edges import build_attention_edges
    n = 3000
    rowptr, col = _graph(n, 240000, seed=b_r + b_w + P)
    deg = np.diff(rowptr)
    assert (deg > hip_ops.HUB_THRESHOLD).any() and (deg > 64).sum() > 20    # hub and batched rows occur
    g = _dev_graph(rowptr, col, n, hip_device)
    u = np.random.default_rng(P * L).random((n * P, L), dtype=np.float32)
    tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                walks_per_node=P, edge_seed=42, u=torch.from_numpy(u).to(hip_device))
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, 42, u)
    assert tab.width == b_r + b_w
    assert np.array_equal(tab.row_len.cpu().numpy(), ref_len)
    assert np.array_equal(tab.table.cpu().numpy(), ref_t)
    assert ref_len.max() > 32


@pytest.mark.parametrize("b_r,b_w,P,L", [(512, 512, 8, 100), (8, 64, 10, 1000), (0, 600, 100, 100),
                                         (512, 512, 100, 100)])
def test_edge_table_wide_rows_and_long_walks(hip_device, b_r, b_w, P, L):
    """Past the LDS staging. B = 1024 as (512, 512): every merged row is ranked by a workgroup in its own
    table slots (17 rows of (512, 512, 8, 100) hold more than 768 ids). P*L = 10,000 walk candidates per
    query: the streaming top-k re-runs the walks per batch of winners. (8, 64, 10, 1000) draws each pair
    about six times, so the multiset selection (64) and the merge's set union (12 to 24) both count
    repeats. Walk records, injected uniforms; bit-exact against the oracle."""
    from budgetformer_amd.edges import build_attention_edges
    n = 1500
    rowptr, col = _graph(n, 300_000, seed=b_r + b_w + P)
    g = _dev_graph(rowptr, col, n, hip_device)
    u = np.random.default_rng(P * L + b_w).random((n * P, L), dtype=np.float32)
    tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                walks_per_node=P, edge_seed=42, u=torch.from_numpy(u).to(hip_device))
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, 42, u)
    assert tab.width == b_r + b_w
    assert np.array_equal(tab.row_len.cpu().numpy(), ref_len)
    assert np.array_equal(tab.table.cpu().numpy(), ref_t)
    if (b_r, P) == (512, 8):
        assert (ref_len > 768).sum() > 10


@pytest.mark.parametrize("b_r,b_w,P,L", [(700, 300, 3, 3000), (0, 900, 4, 2500), (800, 0, 2, 4), (5, 40, 100, 90)])
def test_wide_and_streamed_paths_on_isolated_and_dense_nodes(hip_device, b_r, b_w, P, L):
    """Edge cases of the paths past LDS on a 60-node graph: ten isolated nodes (no real part; their walks
    stay, so each walk offers only its step-1 self pair, kept with multiplicity), a dense core whose rows
    fill neither budget, a chain; merged rows wider than 768 (a workgroup per row) with dedup, an RW-only
    and a real-only table (no dedup), and walk shapes of 9,000 and 10,000 candidates (streaming top-k).
    Bit-exact against the oracle."""
    from budgetformer_amd.edges import build_attention_edges
    n = 60
    rng = np.random.default_rng(b_r + b_w + P)
    pairs = {(int(a), int(b)) for a, b in rng.integers(20, n, (600, 2)) if a != b}
    pairs |= {(i, i + 1) for i in range(10, 19)}                     # a chain 10 - 19
    und = {(min(a, b), max(a, b)) for a, b in pairs}
    src = np.array([a for a, b in und] + [b for a, b in und])
    dst = np.array([b for a, b in und] + [a for a, b in und])
    order = np.lexsort((dst, src))
    src, dst = src[order], dst[order]
    rowptr = np.concatenate([[0], np.cumsum(np.bincount(src, minlength=n))]).astype(np.int64)
    col = dst.astype(np.int32)
    assert (np.diff(rowptr)[:10] == 0).all()
    g = _dev_graph(rowptr, col, n, hip_device)
    u = rng.random((n * P, L), dtype=np.float32)
    tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                walks_per_node=P, edge_seed=42, u=torch.from_numpy(u).to(hip_device))
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, 42, u)
    assert np.array_equal(tab.row_len.cpu().numpy(), ref_len)
    assert np.array_equal(tab.table.cpu().numpy(), ref_t)
    if b_w and not b_r:
        assert (ref_len[:10] == P).all()                             # the isolated nodes' self pairs


def _random_symmetric_csr(rng, n, m):
    src, dst = rng.integers(0, n, m), rng.integers(0, n, m)
    und = {(min(a, b), max(a, b)) for a, b in zip(src.tolist(), dst.tolist()) if a != b}
    s = np.array([a for a, b in und] + [b for a, b in und], dtype=np.int64)
    d = np.array([b for a, b in und] + [a for a, b in und], dtype=np.int64)
    order = np.lexsort((d, s))
    s, d = s[order], d[order]
    rowptr = np.concatenate([[0], np.cumsum(np.bincount(s, minlength=n))]).astype(np.int64)
    return rowptr, d.astype(np.int32)


def test_edge_table_randomized_small_cases(hip_device):
    """60 random small configurations (1 to 200 nodes, 0 to 4 edges per node, budgets 0 to 40 per part,
    1 to 8 walks of 1 to 12 steps, random seeds, injected or Philox uniforms) plus the degenerate ones (a
    single node, graphs without edges, one edge): bit-exact against the oracle, case by case."""
    from budgetformer_amd.edges import build_attention_edges
    rng = np.random.default_rng(2024)
    cases = [(1, 0, 2, 2, 2, 4), (5, 0, 3, 0, 2, 3), (5, 0, 0, 3, 2, 3), (2, 1, 1, 1, 1, 1), (2, 1, 0, 4, 3, 5)]
    for _ in range(60):
        b_r, b_w = int(rng.integers(0, 41)), int(rng.integers(0, 41))
        n = int(rng.integers(1, 201))
        cases.append((n, int(rng.integers(0, 4 * n + 1)), b_r, b_w if b_r + b_w else 1, int(rng.integers(1, 9)),
                      int(rng.integers(1, 13))))
    for i, (n, m, b_r, b_w, P, L) in enumerate(cases):
        rowptr, col = _random_symmetric_csr(rng, n, m)
        seed = int(rng.integers(0, 10_000))
        g = _dev_graph(rowptr, col, n, hip_device)
        philox_u = i % 3 == 2
        u = philox.walk_uniforms(0, n, P, L, seed) if philox_u else rng.random((n * P, L), dtype=np.float32)
        tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                    walks_per_node=P, edge_seed=seed,
                                    u=None if philox_u else torch.from_numpy(u).to(hip_device))
        ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, seed, u)
        case = f"case {i}: n={n} E={col.size} b=({b_r},{b_w}) P={P} L={L} seed={seed} philox={philox_u}"
        assert np.array_equal(tab.row_len.cpu().numpy(), ref_len), case
        assert np.array_equal(tab.table.cpu().numpy(), ref_t), case


def test_streamed_walk_selection_under_philox(hip_device):
    """The streaming RW selection (P*L = 10,000) with the in-kernel Philox uniforms, over the walk
    records and over rowptr/col, for the full range and a shard: equal to the oracle's table on the
    same counter stream."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.edges import build_attention_edges
    n, P, L, b_r, b_w, seed = 1000, 50, 200, 4, 40, 43
    rowptr, col = _graph(n, 60_000, seed=17)
    g = _dev_graph(rowptr, col, n, hip_device)
    tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                walks_per_node=P, edge_seed=seed)
    u = philox.walk_uniforms(0, n, P, L, seed)
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, seed, u)
    assert np.array_equal(tab.row_len.cpu().numpy(), ref_len)
    assert np.array_equal(tab.table.cpu().numpy(), ref_t)
    a = hip_ops.rw_select(g.rowptr, g.col, 200, 500, P, L, b_w, 79, philox_seed=seed)
    b = hip_ops.rw_select(g.rowptr, g.col, 200, 500, P, L, b_w, 79, philox_seed=seed,
                          walk_rec=hip_ops.walk_records(g.rowptr, g.col))
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and int(a[1].min()) == b_w


def test_edge_table_shard_matches_full(hip_device):
    from budgetformer_amd.edges import build_attention_edges
    n, P, L = 3000, 2, 4
    rowptr, col = _graph(n, 25000, seed=9)
    g = _dev_graph(rowptr, col, n, hip_device)
    full = build_attention_edges(g, real_edges_per_query=4, rw_edges_per_query=4, walk_length=L,
                                 walks_per_node=P, edge_seed=7)
    part = build_attention_edges(g, real_edges_per_query=4, rw_edges_per_query=4, walk_length=L,
                                 walks_per_node=P, edge_seed=7, q_lo=1000, n_q=900)
    assert torch.equal(part.table, full.table[1000:1900])
    assert torch.equal(part.row_len, full.row_len[1000:1900])


def test_philox_table_equals_injected_u_table(hip_device):
    from budgetformer_amd.edges import build_attention_edges
    n, P, L = 2000, 2, 4
    rowptr, col = _graph(n, 16000, seed=10)
    g = _dev_graph(rowptr, col, n, hip_device)
    tab = build_attention_edges(g, real_edges_per_query=4, rw_edges_per_query=4, walk_length=L,
                                walks_per_node=P, edge_seed=43)
    u = philox.walk_uniforms(0, n, P, L, 43)
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, 4, 4, L, P, 43, u)
    assert np.array_equal(tab.table.cpu().numpy(), ref_t)


def test_walk_records_layout(hip_device):
    """Record e = (col[e], deg(col[e]), rowptr[col[e]] low word, high word), against numpy; a row
    pointer shifted past 2^32 (read, never walked) checks the high word."""
    from budgetformer_amd import hip_ops
    n = 3000
    rowptr, col = _graph(n, 25000, seed=21)
    g = _dev_graph(rowptr, col, n, hip_device)
    c = col.astype(np.int64)
    for shift in (0, 5 << 32):
        ptr = g.rowptr if shift == 0 else g.rowptr + shift
        rec = hip_ops.walk_records(ptr, g.col).cpu().numpy().astype(np.int64)
        beg = rowptr[c] + shift
        assert np.array_equal(rec[:, 0], c)
        assert np.array_equal(rec[:, 1], rowptr[c + 1] - rowptr[c])
        assert np.array_equal((rec[:, 3] << 32) | (rec[:, 2] & 0xFFFFFFFF), beg)
    assert hip_ops.walk_records(g.rowptr, g.col[:0]).shape == (0, 4)


@pytest.mark.parametrize("P,L,k", [(2, 4, 4), (4, 8, 16), (16, 6, 40), (3, 5, 8), (2, 20, 24)])
def test_walk_records_select_equals_plain_steps(hip_device, P, L, k):
    """rw_select stepping through walk records equals stepping through rowptr and col (which the
    oracle pins), on a directed graph where every 7th node has no out-edges (a walk there stays),
    with Philox and injected uniforms, and for a query list with the probe's subtraction. P a power
    of two with L <= 16 takes the register sort, (3, 5) and (2, 20) the LDS sort."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.graph import CSRGraph
    n = 4000
    rowptr, col = _graph(n, 40000, seed=P + L)
    src = np.repeat(np.arange(n), np.diff(rowptr))
    keep = src % 7 != 0
    out_ptr = np.concatenate([[0], np.cumsum(np.bincount(src[keep], minlength=n))]).astype(np.int64)
    g = CSRGraph.from_csr(out_ptr, col[keep], n, in_ptr=rowptr, in_src=col, device=hip_device)
    rec = hip_ops.walk_records(g.rowptr, g.col)
    gen = torch.Generator(device=hip_device).manual_seed(P * L)
    u = torch.rand((n * P, L), generator=gen, device=hip_device)
    for uu in (None, u):
        a = hip_ops.rw_select(g.rowptr, g.col, 0, n, P, L, k, 79, u=uu, philox_seed=7, philox_offset=3)
        b = hip_ops.rw_select(g.rowptr, g.col, 0, n, P, L, k, 79, u=uu, philox_seed=7, philox_offset=3,
                              walk_rec=rec)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
        assert int(a[1].sum()) > 0
    qids = torch.arange(1, n, 3, dtype=torch.int32, device=hip_device)
    a = hip_ops.rw_select_rows(g.rowptr, g.col, qids, P, L, k, 79, philox_seed=9, subtract=(g.in_ptr, g.in_src))
    b = hip_ops.rw_select_rows(g.rowptr, g.col, qids, P, L, k, 79, philox_seed=9, subtract=(g.in_ptr, g.in_src),
                               walk_rec=rec)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_graphormer_coo_matches_reference_order(hip_device):
    """EdgeTable.to_edge_index reproduces _build_merged_edges + fix_edge_index exactly (order included)."""
    from budgetformer_amd.edges import build_attention_edges
    n, P, L = 1500, 2, 4
    rowptr, col = _graph(n, 12000, seed=11)
    g = _dev_graph(rowptr, col, n, hip_device)
    u = np.random.default_rng(3).random((n * P, L), dtype=np.float32)
    tab = build_attention_edges(g, real_edges_per_query=4, rw_edges_per_query=4, walk_length=L,
                                walks_per_node=P, edge_seed=42, u=torch.from_numpy(u).to(hip_device),
                                global_token=True)
    src = np.repeat(np.arange(n), np.diff(rowptr))
    ref = et.build_merged_edges(np.stack([src, col.astype(np.int64)]), n, 4, 4, L, P, 42, u,
                                graphormer_global_token=True)
    assert np.array_equal(tab.to_edge_index().cpu().numpy(), ref)
    # and the attention index built from the table holds the same edge multiset
    idx = tab.attention_index()
    assert idx.n_q == n + 1 and idx.nnz == ref.shape[1]
    got = sorted(zip(idx.kv.cpu().tolist(), idx.entry_rows().cpu().tolist()))
    assert got == sorted(zip(ref[0].tolist(), ref[1].tolist()))


def test_c2_scale_properties(hip_device):
    """Size-independent invariants at the benchmark's c2 size (169,343 nodes, 1.17M edges)."""
    from budgetformer_amd.edges import build_attention_edges
    n = 169_343
    rowptr, col = _graph(n, 1_166_243, seed=42)
    g = _dev_graph(rowptr, col, n, hip_device)
    tab = build_attention_edges(g, real_edges_per_query=4, rw_edges_per_query=4, walk_length=4,
                                walks_per_node=2, edge_seed=42)
    t = tab.table.cpu().numpy()
    rl = tab.row_len.cpu().numpy()
    assert (rl >= 1).all() and (rl <= 8).all()            # d=1 RW entry always exists
    valid = np.arange(8)[None, :] < rl[:, None]
    assert ((t >= 0) == valid).all()
    rows_sorted = np.where(valid[:, 1:], np.diff(t, axis=1) > 0, True).all()
    assert rows_sorted                                   # two parts: strictly ascending (set)
    # and the full table is bit-exact against the oracle with the same Philox uniforms
    u = philox.walk_uniforms(0, n, 2, 4, 42)
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, 4, 4, 4, 2, 42, u)
    assert np.array_equal(t, ref_t) and np.array_equal(rl, ref_len)


def test_device_chung_lu_graph_properties(hip_device):
    """The on-device generator yields a coalesced symmetric simple graph with a power-law degree profile."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.graph import chung_lu_device
    n, e = 200_000, 2_000_000
    g = chung_lu_device(n, e, exponent=2.1, seed=7, max_degree=3000, device=hip_device)
    rowptr = g.rowptr.cpu().numpy()
    col = g.col.cpu().numpy().astype(np.int64)
    assert rowptr[0] == 0 and rowptr[-1] == e and col.size == e
    deg = np.diff(rowptr)
    src = np.repeat(np.arange(n), deg)
    assert (src != col).all()                                        # no self loops
    lin = src * n + col
    assert (np.diff(lin) > 0).all()                                  # sorted, unique
    assert np.array_equal(np.sort(col * n + src), lin)               # symmetric
    assert deg.max() <= 3000 * 1.5 and deg[:100].mean() > 20 * np.median(deg[deg > 0])
    # the device transpose (in-neighbour CSR) of a symmetric graph is the graph itself
    in_ptr, in_src = hip_ops.coo_to_csr(torch.stack([torch.from_numpy(src), torch.from_numpy(col)]).to(hip_device), n, n)
    assert torch.equal(in_ptr, g.rowptr) and torch.equal(in_src, g.col)
    g2 = chung_lu_device(n, e, exponent=2.1, seed=7, max_degree=3000, device=hip_device)
    assert torch.equal(g2.col, g.col)                                # deterministic


def test_device_chung_lu_is_deterministic_at_scale(hip_device):
    """A seed gives the same graph every time at the benchmark scales too: the weights' sum and prefix sums
    are integer (fixed point), which no parallel summation order can change (a floating-point look-back
    scan rounded differently from run to run, and 1.6B-edge graphs then differed by a few edges)."""
    from budgetformer_amd.graph import chung_lu_device
    n, e = 30_000_000, 200_000_000
    g1 = chung_lu_device(n, e, exponent=2.1, seed=42, max_degree=20_000, device=hip_device)
    c1 = g1.col.clone()
    r1 = g1.rowptr.clone()
    del g1
    g2 = chung_lu_device(n, e, exponent=2.1, seed=42, max_degree=20_000, device=hip_device)
    assert int(r1[-1].item()) == e
    assert torch.equal(r1, g2.rowptr) and torch.equal(c1, g2.col)


@pytest.mark.parametrize("b_r,b_w,thr", [(4, 4, 16), (8, 8, 64), (3, 0, 8), (16, 16, 32)])
def test_hub_path_bit_exact(hip_device, b_r, b_w, thr):
    """Rows above the hub threshold take the workgroup top-k; the table must not change."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.edges import build_attention_edges
    n, P, L = 3000, 4, 4
    rowptr, col = _graph(n, 40000, seed=thr)
    g = _dev_graph(rowptr, col, n, hip_device)
    u = np.random.default_rng(thr).random((n * P, L), dtype=np.float32)
    ut = torch.from_numpy(u).to(hip_device)
    hubs = g.hubs(thr)
    assert hubs.numel() > 10 and (np.diff(rowptr)[hubs.cpu().numpy()] > thr).all()
    a = hip_ops.build_edge_table(g.rowptr, g.col, g.in_ptr, g.in_src, g.num_edges, 0, n, P, L, b_r, b_w, 42, u=ut,
                                 hubs=hubs, hub_threshold=thr)
    b = hip_ops.build_edge_table(g.rowptr, g.col, g.in_ptr, g.in_src, g.num_edges, 0, n, P, L, b_r, b_w, 42, u=ut)
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, 42, u)
    assert np.array_equal(a[0].cpu().numpy(), ref_t) and np.array_equal(b[0].cpu().numpy(), ref_t)
    # a shard whose hub list is restricted to the shard
    tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                walks_per_node=P, edge_seed=42, u=ut[200 * P:1700 * P], q_lo=200, n_q=1500)
    assert np.array_equal(tab.table.cpu().numpy(), ref_t[200:1700])


@pytest.mark.parametrize("b_r,b_w", [(4, 4), (8, 8), (3, 0), (8, 2), (16, 16), (12, 5), (5, 13), (16, 0)])
def test_light_heavy_split_bit_exact(hip_device, b_r, b_w):
    """Thread-per-query rows (in-degree <= light_max) and group rows give the same table at any cut,
    for every register-list size of the fused kernel (4, 8, 16 real x 4, 8, 16 RW)."""
    from budgetformer_amd import hip_ops
    n, L = 3000, 4
    P = 4 if b_w > 8 else 2
    rowptr, col = _graph(n, 40000, seed=b_r * 3 + b_w)
    g = _dev_graph(rowptr, col, n, hip_device)
    u = np.random.default_rng(b_r).random((n * P, L), dtype=np.float32)
    ut = torch.from_numpy(u).to(hip_device)
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, 42, u)
    for light_max in (1, 5, 32, 10 ** 9):
        heavy = g.heavy(light_max)
        t, rl = hip_ops.build_edge_table(g.rowptr, g.col, g.in_ptr, g.in_src, g.num_edges, 0, n, P, L, b_r, b_w, 42,
                                         u=ut, hubs=g.hubs(16), hub_threshold=16, heavy=heavy, light_max=light_max)
        assert np.array_equal(t.cpu().numpy(), ref_t) and np.array_equal(rl.cpu().numpy(), ref_len), light_max
    # a shard with its heavy list cut to the range
    from budgetformer_amd.edges import build_attention_edges
    tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                walks_per_node=P, edge_seed=42, u=ut[300 * P:2300 * P], q_lo=300, n_q=2000)
    assert np.array_equal(tab.table.cpu().numpy(), ref_t[300:2300])


def test_light_rows_with_unaligned_in_neighbour_array(hip_device):
    """in_src not 16-byte aligned: the light rows fall back from 16-byte chunk loads to 4-byte loads."""
    from budgetformer_amd import hip_ops
    n, P, L, b_r, b_w = 2500, 2, 4, 4, 4
    rowptr, col = _graph(n, 30000, seed=5)
    g = _dev_graph(rowptr, col, n, hip_device)
    u = torch.from_numpy(np.random.default_rng(5).random((n * P, L), dtype=np.float32)).to(hip_device)
    buf = torch.empty(g.in_src.numel() + 1, dtype=torch.int32, device=hip_device)
    buf[1:] = g.in_src
    shifted = buf[1:]
    assert shifted.data_ptr() % 16 != 0
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, 42, u.cpu().numpy())
    for src in (g.in_src, shifted):
        t, rl = hip_ops.build_edge_table(g.rowptr, g.col, g.in_ptr, src, g.num_edges, 0, n, P, L, b_r, b_w, 42, u=u,
                                         hubs=g.hubs(64), hub_threshold=64, heavy=g.heavy(8), light_max=8)
        assert np.array_equal(t.cpu().numpy(), ref_t) and np.array_equal(rl.cpu().numpy(), ref_len)


@pytest.mark.parametrize("token", [False, True])
def test_from_table_rejects_invalid_tables(hip_device, token):
    """An external table is validated on the device (bf_check_table) before any index kernel reads it:
    ids within [0, n_kv) (n_kv - 1 with the token's shift), row lengths within [0, width]; padding past
    a row's length is not read. The same check behind the table_to_csr operator's id_limit."""
    from budgetformer_amd import _native
    from budgetformer_amd.hip_ops import AttentionIndex
    n, width = 50, 4
    table = torch.full((n, width), -1, dtype=torch.int32, device=hip_device)
    row_len = torch.zeros(n, dtype=torch.int32, device=hip_device)
    table[:, 0] = torch.arange(n, dtype=torch.int32, device=hip_device)
    row_len[:] = 1
    AttentionIndex.from_table(table, row_len, token)                       # valid
    bad = table.clone()
    bad[7, 0] = n + 3                                                       # id beyond the kv rows
    bad[8, 0] = n                                                           # the first id past the limit
    with pytest.raises(ValueError, match="2 table ids outside"):
        AttentionIndex.from_table(bad, row_len, token)
    bad = table.clone()
    bad[9, 0] = -1                                                          # padding inside row_len
    with pytest.raises(ValueError, match="1 table ids outside"):
        AttentionIndex.from_table(bad, row_len, token)
    long = row_len.clone()
    long[3] = width + 1
    long[4] = -2
    with pytest.raises(ValueError, match="2 row lengths outside"):
        AttentionIndex.from_table(table, long, token)
    ops = _native.load_ops()
    tr = n if token else -1
    ops.table_to_csr(table, row_len, token, tr, n)      # n kv rows (n + 1 with the token, ids shifted by one)
    with pytest.raises(ValueError, match="ids outside"):
        ops.table_to_csr(bad, row_len, token, tr, n)


@pytest.mark.parametrize("token,token_row", [(False, None), (True, None), (True, -1), (True, 5400), (True, 3)])
def test_index_formats_against_numpy(hip_device, token, token_row):
    """table -> CSR (with the fused token fill), both reverse-index routes, the split plan and the row order.
    With the token: the full query set (token row of n entries), a query shard without the token row (-1),
    and token rows longer and shorter than the table (a shard starting at node 0 of a larger graph, and
    one whose kv ids stop short of the table's)."""
    from budgetformer_amd import hip_ops
    rng = np.random.default_rng(11 + token + (token_row or 0))
    n, width = 5000, 6
    row_len = rng.integers(0, width + 1, n).astype(np.int32)
    table = np.full((n, width), -1, dtype=np.int32)
    for r in range(n):
        table[r, :row_len[r]] = np.sort(rng.choice(n // 3 if r % 7 else 40, row_len[r], replace=False))
    t, rl = torch.from_numpy(table).to(hip_device), torch.from_numpy(row_len).to(hip_device)
    qptr, kv, rk = hip_ops.table_to_csr(t, rl, token, with_keys=True, token_row=token_row)
    tr = (n if token_row is None else token_row) if token else -1
    # numpy CSR of the same table
    rows, vals = [], []
    if tr >= 0:
        rows += [0] * tr
        vals += list(range(1, tr + 1))
    lead = 1 if tr >= 0 else 0
    for r in range(n):
        ids = ([0] if token else []) + [int(x) + (1 if token else 0) for x in table[r, :row_len[r]]]
        rows += [r + lead] * len(ids)
        vals += ids
    n_q = n + lead
    n_kv = max(n_q, tr + 1)
    assert np.array_equal(kv.cpu().numpy(), np.array(vals, dtype=np.int32))
    assert np.array_equal(np.diff(qptr.cpu().numpy()), np.bincount(np.array(rows), minlength=n_q))
    pos = np.arange(len(vals))
    # sort keys: id << (q_bits + slot_bits) | query << slot_bits | slot, in CSR order, for the table's own
    # entries only (with the token, kv 0 of every row and the token row have fixed reverse places)
    rows_a = np.array(rows, dtype=np.int64)
    slot = pos - qptr.cpu().numpy()[rows_a]
    expect = (np.array(vals, dtype=np.int64) << (rk.q_bits + rk.slot_bits)) | (rows_a << rk.slot_bits) | slot
    if token:
        expect = expect[(rows_a >= lead) & (np.array(vals) != 0)]
    assert (rk.q_bits, rk.slot_bits) == (int(n_q).bit_length(), int(width).bit_length())
    assert np.array_equal(rk.keys.cpu().numpy(), expect)
    a = hip_ops.reverse_index(qptr, kv, n_kv)
    b = hip_ops.reverse_index_packed(rk, qptr, n_kv)
    for x, y in zip(a, b[:3]):
        assert torch.equal(x, y)
    lazy = hip_ops.reverse_index_packed(rk, qptr, n_kv, entries=False)
    assert lazy[2] is None and torch.equal(lazy[0], a[0]) and torch.equal(lazy[1], a[1])
    assert torch.equal(hip_ops.reverse_slots(lazy[3], qptr), a[2])
    # the same route with nothing read back: buffers sized for every row full, the kernels taking the
    # entry count from qptr[n_q]; the first nnz entries equal the exact route's
    nnz = kv.numel()
    qc, kvc, rkc = hip_ops.table_to_csr(t, rl, token, with_keys=True, token_row=token_row, exact=False)
    assert kvc.numel() == n * width + ((n + max(tr, 0)) if token else 0) > nnz
    assert torch.equal(qc, qptr) and torch.equal(kvc[:nnz], kv)
    assert torch.equal(rkc.keys[:rk.keys.numel()], rk.keys)
    cap = hip_ops.reverse_index_packed(rkc, qc, n_kv)
    assert torch.equal(cap[0], a[0]) and torch.equal(cap[1][:nnz], a[1]) and torch.equal(cap[2][:nnz], a[2])
    lazy_c = hip_ops.reverse_index_packed(rkc, qc, n_kv, entries=False)
    assert torch.equal(hip_ops.reverse_slots(lazy_c[3], qc)[:nnz], a[2])
    order = np.lexsort((pos, np.array(vals)))                    # (kv, position) order
    assert np.array_equal(b[1].cpu().numpy(), np.array(rows)[order])
    assert np.array_equal(b[2].cpu().numpy(), slot[order])       # each entry's slot in its query's row
    # the attention index's two routes to ks: the unpack pass, or later from the sorted keys it keeps
    ia = hip_ops.AttentionIndex.from_table(t, rl, global_token=token, n_kv=n_kv, token_row=token_row, check=False)
    ib = hip_ops.AttentionIndex.from_table(t, rl, global_token=token, n_kv=n_kv, token_row=token_row, check=False)
    ia.ensure_backward(entries=True)
    ib.ensure_backward()
    assert ib.ks_all is None
    ib.ensure_entries()
    assert torch.equal(ia.ks, a[2]) and torch.equal(ib.ks, a[2]) and torch.equal(ia.kq, a[1])
    # row order: a permutation, capped lengths non-increasing
    ro, sp = hip_ops.row_order(b[0], spans=True)
    ro, sp = ro.cpu().numpy(), sp.cpu().numpy().astype(np.uint64)
    kp = b[0].cpu().numpy()
    lens = np.minimum(np.diff(kp), 255)
    assert np.array_equal(np.sort(ro), np.arange(n_kv)) and (np.diff(lens[ro]) <= 0).all()
    # spans: each slot's row as (begin << 32 | length)
    assert np.array_equal(sp >> np.uint64(32), kp[ro].astype(np.uint64))
    assert np.array_equal(sp & np.uint64(0xFFFFFFFF), (kp[ro + 1] - kp[ro]).astype(np.uint64))
    # split plan (threshold 4, items of 5) against a direct count
    plan = hip_ops.split_plan(b[0], kv.numel(), 4, 5)
    L = np.diff(b[0].cpu().numpy())
    heavy = np.nonzero(L > 4)[0]
    assert plan.heavy == heavy.size and np.array_equal(plan.heavy_rows[:plan.heavy].cpu().numpy(), heavy)
    nit = np.where(L > 4, np.minimum(-(-L // 5), 160), 0)              # BF_MAX_ITEMS_PER_ROW = 160
    assert plan.items == nit.sum() and np.array_equal(plan.nitems[:n_kv].cpu().numpy(), nit)
    assert np.array_equal(plan.item_off[:n_kv].cpu().numpy(), np.concatenate([[0], np.cumsum(nit)[:-1]]))
    assert np.array_equal(plan.item_row[:plan.items].cpu().numpy(), np.repeat(np.arange(n_kv), nit))


@pytest.mark.parametrize("n_rows,chunk,item", [(3000, 128, 768), (1000, 16, 7), (50, 128, 768)])
def test_first_row_plan_equals_the_generic_plan(hip_device, n_rows, chunk, item):
    """A table's CSR with the token: only row 0 (the token row) can be longer than `chunk`, and the
    one-pass plan of that row equals the generic count/scan/rows plan array for array."""
    from budgetformer_amd import hip_ops
    rng = np.random.default_rng(n_rows)
    width = 6
    row_len = rng.integers(0, width + 1, n_rows).astype(np.int32)
    table = np.full((n_rows, width), -1, dtype=np.int32)
    for r in range(n_rows):
        table[r, :row_len[r]] = np.sort(rng.choice(n_rows, row_len[r], replace=False))
    t = torch.from_numpy(table).to(hip_device)
    qptr = hip_ops.table_qptr(t, torch.from_numpy(row_len).to(hip_device), global_token=True)
    nnz = int(qptr[-1].item())
    gen = hip_ops.split_plan(qptr, nnz, chunk, item)
    n_items = min(-(-n_rows // item), 160) if n_rows > chunk else 0
    one = hip_ops.split_plan_first_row(n_rows + 1, n_items, nnz, chunk, item,
                                       torch.empty(2, dtype=torch.int32, device=hip_device))
    assert (one.items, one.heavy) == (gen.items, gen.heavy) == (n_items, 1 if n_items else 0)
    assert one.counts.tolist() == [gen.items, gen.heavy]
    n_q = n_rows + 1
    assert torch.equal(one.nitems[:n_q], gen.nitems[:n_q]) and torch.equal(one.item_off[:n_q], gen.item_off[:n_q])
    assert torch.equal(one.item_row[:gen.items], gen.item_row[:gen.items])
    assert torch.equal(one.heavy_rows[:gen.heavy], gen.heavy_rows[:gen.heavy])


@pytest.mark.parametrize("chunk,item,n,e", [(128, 768, 3000, 30000), (4, 5, 3000, 30000), (16, 3, 3000, 30000),
                                            (4, 5, 40000, 400000)])
def test_plan_from_the_row_order_equals_the_generic_plan(hip_device, chunk, item, n, e):
    """The split rows are the longest-first order's first slots: the plan written from them holds the
    same split rows, item counts and counts as the generic plan, only numbered in slot order. Plans of at
    most 32768 slots form their item offsets inside split_rows_kernel, larger ones through a device scan
    (the 40000-row graph): the generic plan is also checked against numpy."""
    from budgetformer_amd import hip_ops
    rowptr, col = _graph(n, e, seed=chunk * 10 + item)
    ptr = torch.from_numpy(rowptr).to(hip_device)
    nnz = int(rowptr[-1])
    gen = hip_ops.split_plan(ptr, nnz, chunk, item)
    L = np.diff(rowptr)
    nit_ref = np.where(L > chunk, np.minimum(-(-L // item), 160), 0)
    assert gen.items == nit_ref.sum() and gen.heavy == int((L > chunk).sum())
    assert np.array_equal(gen.nitems[:n].cpu().numpy(), nit_ref)
    assert np.array_equal(gen.item_off[:n].cpu().numpy(), np.concatenate([[0], np.cumsum(nit_ref)[:-1]]))
    assert np.array_equal(gen.item_row[:gen.items].cpu().numpy(), np.repeat(np.arange(n), nit_ref))
    order, spans, plan = hip_ops.row_order_and_plan(ptr, nnz, chunk, item)
    hip_ops.resolve_plans(plan)
    assert (plan.items, plan.heavy) == (gen.items, gen.heavy) and gen.heavy > 0
    ro = order.cpu().numpy()
    assert np.array_equal(np.sort(ro), np.arange(n)) and (np.diff(np.minimum(L, 255)[ro]) <= 0).all()
    heavy = plan.heavy_rows[:plan.heavy].cpu().numpy()
    assert np.array_equal(np.sort(heavy), gen.heavy_rows[:gen.heavy].cpu().numpy())
    assert np.array_equal(heavy, order[:plan.heavy].cpu().numpy())           # slot order
    nit, off = plan.nitems.cpu().numpy(), plan.item_off.cpu().numpy()
    assert np.array_equal(nit[heavy], gen.nitems.cpu().numpy()[heavy])
    # items numbered in slot order, each row's items contiguous
    assert np.array_equal(off[heavy], np.concatenate([[0], np.cumsum(nit[heavy])[:-1]]))
    assert np.array_equal(plan.item_row[:plan.items].cpu().numpy(), np.repeat(heavy, nit[heavy]))


@pytest.mark.parametrize("n,token_row", [(5000, None), (5000, -1), (5000, 7000), (0, None), (0, 3), (0, -1)])
def test_token_index_of_tables_without_own_entries(hip_device, n, token_row):
    """Tables whose rows are all empty (every key of the reverse-index sort is gone: only the token's
    entries remain, placed without a sort) and tables with no rows at all: both reverse-index routes,
    the slots, and an attention layer over the index against the oracle."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.attention import sparse_edge_attention
    from budgetformer_amd.hip_ops import AttentionIndex
    width = 4
    table = torch.full((n, width), -1, dtype=torch.int32, device=hip_device)
    row_len = torch.zeros(n, dtype=torch.int32, device=hip_device)
    tr = n if token_row is None else token_row
    qptr, kv, rk = hip_ops.table_to_csr(table, row_len, True, with_keys=True, token_row=tr)
    n_q = n + (1 if tr >= 0 else 0)
    n_kv = max(n, tr) + 1
    assert rk is not None and rk.keys.numel() == 0 and kv.numel() == n + max(tr, 0)
    a = hip_ops.reverse_index(qptr, kv, n_kv)
    b = hip_ops.reverse_index_packed(rk, qptr, n_kv)
    for x, y in zip(a, b[:3]):
        assert torch.equal(x, y)
    lazy = hip_ops.reverse_index_packed(rk, qptr, n_kv, entries=False)
    assert torch.equal(hip_ops.reverse_slots(lazy[3], qptr), a[2])
    if n_q == 0 or kv.numel() == 0:
        return
    idx = AttentionIndex.from_table(table, row_len, True, n_kv=n_kv, token_row=tr)
    H, hn = 2, 8
    gen = torch.Generator().manual_seed(n + tr)
    q = torch.randn(n_q, H, hn, generator=gen)
    k, v = (torch.randn(n_kv, H, hn, generator=gen) for _ in range(2))
    dout = torch.randn(n_q, H, hn, generator=gen)
    qd, kd, vd = (t.to(hip_device).requires_grad_(True) for t in (q, k, v))
    out = sparse_edge_attention(qd, kd, vd, idx)
    out.backward(dout.to(hip_device))
    ei = torch.stack([idx.kv.cpu().long(), idx.entry_rows().cpu()])
    ro, rZ = sa.attention_forward_stats(k.double(), q.double(), v.double(), ei)
    rdq, rdk, rdv, _ = sa.attention_backward_closed_form(k.double(), q.double(), v.double(), ei, ro, rZ,
                                                         dout.double())
    def rel(got, ref):
        return ((got.detach().double().cpu() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()

    assert rel(out, ro) < 1e-5 and rel(vd.grad, rdv) < 1e-5
    # every table row attends kv 0 alone, so its dq and its term of kv 0's dK are softmax gradients over one
    # key: differences of two equal terms, left over only through the 1e-6 in Z. kv 0's dK is held to an
    # absolute bound of 1e-6 of those terms per entry (sqrt(n) for n independent roundings); the token row's
    # kv rows 1.. keep the relative bar
    dk = kd.grad.double().cpu()
    if tr > 0:
        assert rel(dk[1:], rdk[1:]) < 1e-5
    terms = (dout.norm(dim=-1).max() * v.norm(dim=-1).max() * q.abs().max() / math.sqrt(hn)).item()
    assert (dk[0] - rdk[0]).abs().max().item() < 1e-6 * terms * math.sqrt(max(n, 1))


def test_row_pointers_across_long_runs_of_empty_rows(hip_device):
    """Row pointers from sorted ids when long ranges of rows have no entries: COO queries and kv ids
    clustered at both ends of 3M rows (gaps of ~1.5M rows inside and at the tail), and a table whose
    ids stop far below the Graphormer token row's 2M kv rows. A wave writes each long gap together;
    every pointer must equal numpy's counts."""
    from budgetformer_amd import hip_ops
    rng = np.random.default_rng(77)
    n = 3_000_000
    ids = np.concatenate([rng.integers(0, 50, 4000), rng.integers(1_500_000, 1_500_040, 3000),
                          rng.integers(n - 30, n, 2000)])
    src, dst = rng.permutation(ids), rng.permutation(ids)
    ei = torch.from_numpy(np.stack([src, dst])).to(hip_device)
    qptr, kv = hip_ops.coo_to_csr(ei, n + 5, n + 7)            # 5 and 7 empty rows past the last id
    want_q = np.concatenate([[0], np.cumsum(np.bincount(dst, minlength=n + 5))])
    assert np.array_equal(qptr.cpu().numpy(), want_q)
    kptr, kq, ks = hip_ops.reverse_index(qptr, kv, n + 7)
    want_k = np.concatenate([[0], np.cumsum(np.bincount(src, minlength=n + 7))])
    assert np.array_equal(kptr.cpu().numpy(), want_k)
    # a table of 3000 rows with ids below 3000 and a token row of 2M entries
    m, width, tr = 3000, 4, 2_000_000
    table = np.sort(rng.integers(0, m, (m, width)).astype(np.int32), axis=1)
    row_len = np.full(m, width, dtype=np.int32)
    t, rl = torch.from_numpy(table).to(hip_device), torch.from_numpy(row_len).to(hip_device)
    qptr, kv, rk = hip_ops.table_to_csr(t, rl, True, with_keys=True, token_row=tr)
    a = hip_ops.reverse_index(qptr, kv, tr + 1)
    b = hip_ops.reverse_index_packed(rk, qptr, tr + 1)
    for x, y in zip(a, b[:3]):
        assert torch.equal(x, y)
    lazy = hip_ops.reverse_index_packed(rk, qptr, tr + 1, entries=False)
    assert torch.equal(hip_ops.reverse_slots(lazy[3], qptr), a[2])
    kvn = kv.cpu().numpy()
    assert np.array_equal(a[0].cpu().numpy(), np.concatenate([[0], np.cumsum(np.bincount(kvn, minlength=tr + 1))]))


@pytest.mark.parametrize("n_rows", [2_000_000, 4_300_000])
def test_table_row_pointers_both_scan_routes(hip_device, n_rows):
    """A table's row pointers (with the token row): up to 1024 blocks of 4096 rows in two launches that
    sum the blocks before their own, past that through a device scan (4.3M rows). Both equal numpy's
    running sum."""
    from budgetformer_amd import hip_ops
    rng = np.random.default_rng(n_rows)
    row_len = rng.integers(0, 9, n_rows).astype(np.int32)
    table = torch.zeros((n_rows, 8), dtype=torch.int32, device=hip_device)
    qptr = hip_ops.table_qptr(table, torch.from_numpy(row_len).to(hip_device), global_token=True)
    lens = np.concatenate([[n_rows], row_len.astype(np.int64) + 1])        # the token row, then kv 0 + row
    assert np.array_equal(qptr.cpu().numpy(), np.concatenate([[0], np.cumsum(lens)]))


@pytest.mark.parametrize("n,width,lo", [(120_000, 12, 8), (600_000, 4, 2), (40_000, 8, 2)])
def test_packed_reverse_index_onesweep_sizes(hip_device, n, width, lo):
    """Reverse indexes of 0.1M to 2M keys: the packed route sorts only the 16 to 20 kv-id bits with the
    library's radix sort (two 9-bit passes for 18 bits, three 8-bit ones otherwise). The result must
    equal the pair-sort route and numpy's stable order."""
    from budgetformer_amd import hip_ops
    rng = np.random.default_rng(n)
    row_len = rng.integers(lo, width + 1, n).astype(np.int32)
    base = rng.integers(0, n, n)
    table = ((base[:, None] + np.arange(width)[None, :] * 104729) % n).astype(np.int32)   # distinct per row
    table[np.arange(width)[None, :] >= row_len[:, None]] = -1
    assert row_len.sum() > 65_536
    t, rl = torch.from_numpy(table).to(hip_device), torch.from_numpy(row_len).to(hip_device)
    qptr, kv, rk = hip_ops.table_to_csr(t, rl, False, with_keys=True)
    a = hip_ops.reverse_index(qptr, kv, n)
    b = hip_ops.reverse_index_packed(rk, qptr, n)
    for x, y in zip(a, b[:3]):
        assert torch.equal(x, y)
    vals = kv.cpu().numpy()
    order = np.argsort(vals, kind="stable")
    qp = qptr.cpu().numpy()
    rows = np.repeat(np.arange(n), np.diff(qp))
    assert np.array_equal(b[1].cpu().numpy(), rows[order])
    assert np.array_equal(b[2].cpu().numpy(), (np.arange(vals.size) - qp[rows])[order])   # slots
    assert np.array_equal(np.diff(b[0].cpu().numpy()), np.bincount(vals, minlength=n))
