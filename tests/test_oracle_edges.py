"""Pins for the CPU edge-construction oracle (oracle/edge_table.py).

Every check here compares the oracle with something independent of the
oracle's own formula: literal known answers, brute-force Python loops,
deterministic graphs, or an alternative branch of the reference algorithm.
"""
import itertools
import random

import numpy as np
import pytest

from oracle import edge_table as et


# --------------------------------------------------------------------- key
def test_edge_key_known_answers():
    # values worked by hand from utils/fullgraph_sp_support.py:984-989
    assert int(et.edge_key(0, 0, 0)) == 12345
    assert int(et.edge_key(1, 0, 0)) == 1103527590
    assert int(et.edge_key(3, 5, 42)) == 981296763
    assert int(et.edge_key(123456, 654321, 59)) == 1655120241
    assert int(et.edge_key(2 ** 30, 7, 79)) == 322279875
    assert int(et.edge_key(5, 3, -1)) == 716311200   # negative constant: non-negative remainder


def test_edge_key_uint32_wrap_equivalence():
    rng = np.random.default_rng(0)
    src = rng.integers(0, 2 ** 31 - 1, 4096)
    dst = rng.integers(0, 2 ** 31 - 1, 4096)
    for seed in (0, 42 + 17, 42 + 37, 10 ** 6, -3):
        c = (seed * et.KEY_C_MUL + et.KEY_C_ADD) % (1 << 32)
        w = (src.astype(np.uint64) * np.uint64(et.KEY_A) + dst.astype(np.uint64) * np.uint64(et.KEY_B)
             + np.uint64(c)) & np.uint64(0xFFFFFFFF)
        assert np.array_equal(w.astype(np.int64) & 0x7FFFFFFF, et.edge_key(src, dst, seed))


def test_edge_key_bijective_per_dst():
    src = np.arange(200_000)
    for dst in (0, 17, 99_999):
        k = et.edge_key(src, np.full_like(src, dst), 59)
        assert np.unique(k).size == src.size


# --------------------------------------------------------------------- walk
def _csr(n, edges):
    ei = np.array(edges, dtype=np.int64).T if edges else np.zeros((2, 0), np.int64)
    return et.csr_from_coo(ei, n)


def test_csr_from_coo_sorted_unique():
    rowptr, col = _csr(4, [(2, 1), (0, 3), (2, 0), (0, 3), (0, 1)])
    assert rowptr.tolist() == [0, 2, 2, 4, 4]
    assert col.tolist() == [1, 3, 0, 1]


def test_walk_chain_is_rng_free():
    # 0->1->2->3->4 (deg 1 everywhere except the sink 4)
    rowptr, col = _csr(5, [(i, i + 1) for i in range(4)])
    u = np.random.default_rng(1).random((5, 6), dtype=np.float32)
    w = et.random_walk(rowptr, col, np.arange(5), 6, u)
    for s in range(5):
        assert w[s].tolist() == [min(s + j, 4) for j in range(7)]   # sink stays


def test_walk_cycle_and_dead_end():
    rowptr, col = _csr(3, [(0, 1), (1, 2), (2, 0)])
    w = et.random_walk(rowptr, col, [0, 1], 4, np.full((2, 4), 0.99, np.float32))
    assert w.tolist() == [[0, 1, 2, 0, 1], [1, 2, 0, 1, 2]]
    rowptr, col = _csr(2, [])
    w = et.random_walk(rowptr, col, [1], 3, np.zeros((1, 3), np.float32))
    assert w.tolist() == [[1, 1, 1, 1]]


def test_walk_first_and_last_neighbour():
    star = [(0, j) for j in range(1, 8)] + [(j, 0) for j in range(1, 8)]
    rowptr, col = _csr(8, star)
    u_last = np.float32(1.0) - np.float32(2.0 ** -24)
    w = et.random_walk(rowptr, col, [0, 0], 1, np.array([[0.0], [u_last]], np.float32))
    assert w[:, 1].tolist() == [1, 7]


def test_walk_uses_fp32_product_rounding():
    # u = largest float32 below 5/6: exact u*6 = 4.99999988..., the fp32 product
    # rounds to 5.0, so the fp32 contract picks neighbour index 5 (fp64 would pick 4).
    u = np.float32(0.8333333134651184)
    assert float(u) * 6 < 5.0 and float(np.float32(u) * np.float32(6)) == 5.0
    rowptr, col = _csr(7, [(0, j) for j in range(1, 7)])
    w = et.random_walk(rowptr, col, [0], 1, np.array([[u]], np.float32))
    assert w[0, 1] == 6          # col[rowptr[0] + 5]


def test_walk_steps_are_edges():
    rng = np.random.default_rng(2)
    n = 60
    edges = {(int(a), int(b)) for a, b in rng.integers(0, n, (200, 2)) if a != b}
    rowptr, col = _csr(n, sorted(edges))
    starts = et.walk_starts(n, 3)
    u = rng.random((starts.size, 5), dtype=np.float32)
    w = et.random_walk(rowptr, col, starts, 5, u)
    for row in w:
        for a, b in zip(row[:-1], row[1:]):
            deg = rowptr[a + 1] - rowptr[a]
            assert (a, b) in edges if deg > 0 else a == b


# --------------------------------------------------------------------- hop pool
def test_hop_edges_hand_built():
    walks = np.array([[0, 0, 0, 0],      # dead end at start: d=1 self-edge kept, later stays dropped
                      [1, 2, 2, 3],      # stay at d=2 dropped
                      [4, 5, 4, 5]])     # revisits kept
    pool = et.hop_edges_from_walks(walks)
    expect = [(0, 0), (2, 1), (5, 4),    # d=1 for each walk (kv, q)
              (4, 4),                    # d=2
              (3, 1), (5, 4)]            # d=3
    assert list(map(tuple, pool.T.tolist())) == expect


# --------------------------------------------------------------------- selection
def _brute_select(ei, k, seed):
    """Per dst, sort (key, position) with Python ints and keep the first k."""
    out = []
    by_dst = {}
    for pos, (s, d) in enumerate(zip(ei[0].tolist(), ei[1].tolist())):
        key = (s * 1103515245 + d * 214013 + seed * 2654435761 + 12345) % (1 << 31)
        by_dst.setdefault(d, []).append((key, pos, s))
    for d, lst in by_dst.items():
        for key, pos, s in sorted(lst)[:k]:
            out.append((s, d))
    return sorted(out)


@pytest.mark.parametrize("trial", range(6))
def test_selection_matches_brute_force_and_minhash(trial):
    rng = random.Random(trial)
    n = rng.randint(2, 30)
    m = rng.randint(0, 150)
    ei = np.array([[rng.randrange(n) for _ in range(m)], [rng.randrange(n) for _ in range(m)]],
                  dtype=np.int64).reshape(2, m)
    for k in (1, 2, 3, 5, 9):
        seed = rng.randint(0, 1000)
        a = sorted(map(tuple, et.sample_edges_per_query_random(ei, k, seed).T.tolist()))
        b = sorted(map(tuple, et.sample_edges_per_query_random_minhash(ei, k, seed).T.tolist()))
        assert a == b == _brute_select(ei, k, seed) if m > k else a == b


def test_selection_duplicates_consume_budget():
    # dst 0 has the pair (3,0) three times and (1,0) once; with k=2 the result
    # depends only on keys: duplicates of the smallest-key pair consume budget.
    ei = np.array([[3, 3, 1, 3], [0, 0, 0, 0]])
    seed = 5
    got = sorted(map(tuple, et.sample_edges_per_query_random(ei, 2, seed).T.tolist()))
    k3, k1 = int(et.edge_key(3, 0, seed)), int(et.edge_key(1, 0, seed))
    assert got == ([(3, 0), (3, 0)] if k3 < k1 else [(1, 0), (3, 0)])


# --------------------------------------------------------------------- merge / global token
def test_merge_two_parts_dedups_one_part_passes_through():
    a = np.array([[1, 2, 2], [0, 0, 0]])
    b = np.array([[2, 5], [0, 1]])
    m = et.merge_edge_index_list([a, b])
    assert m.T.tolist() == [[1, 0], [2, 0], [5, 1]]          # src-major, unique
    assert et.merge_edge_index_list([a, None]) is a           # passthrough keeps duplicates
    assert et.merge_edge_index_list([np.zeros((2, 0)), b]) is b
    assert et.merge_edge_index_list([None, None]) is None


def test_fix_edge_index_closed_form():
    ei = np.array([[0, 2], [1, 0]])
    out = et.fix_edge_index(ei, 3)
    assert out.T.tolist() == [[1, 2], [3, 1], [1, 0], [2, 0], [3, 0], [0, 1], [0, 2], [0, 3]]


# --------------------------------------------------------------------- full pipeline
def _loop_pipeline(n, edges, b_r, b_w, L, P, seed, u):
    """Pure-Python restatement of the whole chain for small graphs."""
    adj = {i: sorted({b for a, b in edges if a == i}) for i in range(n)}
    parts = []
    if b_r > 0 and edges:
        uniq = sorted(set(edges))
        ei = np.array(uniq, dtype=np.int64).T
        parts.append(_brute_select(ei, b_r, seed + 17) if len(uniq) > b_r else sorted(uniq))
    if b_w > 0 and P > 0:
        pool = []
        for d in range(1, L + 1):
            for w in range(n * P):
                cur = w // P
                trail = [cur]
                for step in range(L):
                    nb = adj[cur]
                    if nb:
                        idx = min(int(np.float32(u[w, step]) * np.float32(len(nb))), len(nb) - 1)
                        cur = nb[idx]
                    trail.append(cur)
                if d == 1 or trail[d] != trail[d - 1]:
                    pool.append((trail[d], trail[0]))
        ei = np.array(pool, dtype=np.int64).T
        parts.append(_brute_select(ei, b_w, seed + 37) if len(pool) > b_w else sorted(pool))
    parts = [p for p in parts if p]
    if len(parts) >= 2:
        return sorted(set(itertools.chain(*parts)))
    return sorted(parts[0]) if parts else []


@pytest.mark.parametrize("trial", range(4))
def test_build_merged_edges_matches_loop_pipeline(trial):
    rng = np.random.default_rng(100 + trial)
    n = int(rng.integers(5, 25))
    raw = rng.integers(0, n, (int(rng.integers(0, 60)), 2))
    edges = sorted({(int(a), int(b)) for a, b in raw if a != b} | {(int(b), int(a)) for a, b in raw if a != b})
    L, P = int(rng.integers(1, 5)), int(rng.integers(1, 3))
    u = rng.random((n * P, L), dtype=np.float32)
    ei = np.array(edges, dtype=np.int64).T if edges else np.zeros((2, 0), np.int64)
    for b_r, b_w in [(2, 2), (3, 0), (0, 3), (1, 4)]:
        got = et.build_merged_edges(ei, n, b_r, b_w, L, P, 42, u)
        assert sorted(map(tuple, got.T.tolist())) == _loop_pipeline(n, edges, b_r, b_w, L, P, 42, u)


def test_build_edge_table_rows_sorted_and_bounded():
    rng = np.random.default_rng(7)
    n = 40
    raw = rng.integers(0, n, (150, 2))
    edges = sorted({(int(a), int(b)) for a, b in raw if a != b} | {(int(b), int(a)) for a, b in raw if a != b})
    rowptr, col = et.csr_from_coo(np.array(edges).T, n)
    u = rng.random((n * 2, 4), dtype=np.float32)
    table, row_len = et.build_edge_table(rowptr, col, n, 4, 4, 4, 2, 42, u)
    assert table.shape == (n, 8) and (row_len <= 8).all()
    for q in range(n):
        row = table[q, :row_len[q]]
        assert (np.diff(row) > 0).all()          # two parts -> deduplicated, ascending
        assert (table[q, row_len[q]:] == -1).all()


def test_query_range_build_equals_rows_of_full_build():
    from oracle import philox
    rng = np.random.default_rng(11)
    n = 400
    raw = rng.integers(0, n, (1500, 2))
    edges = sorted({(int(a), int(b)) for a, b in raw if a != b} | {(int(b), int(a)) for a, b in raw if a != b})
    rowptr, col = et.csr_from_coo(np.array(edges).T, n)
    u = philox.walk_uniforms(0, n, 2, 4, 9)
    for b_r, b_w in ((4, 4), (3, 0), (0, 3)):
        full_t, full_l = et.build_edge_table(rowptr, col, n, b_r, b_w, 4, 2, 9, u)
        for lo, cnt in ((0, n), (100, 70), (350, 50)):
            t, l = et.build_edge_table(rowptr, col, n, b_r, b_w, 4, 2, 9, u[lo * 2:(lo + cnt) * 2], q_lo=lo, n_q=cnt)
            assert np.array_equal(t, full_t[lo:lo + cnt]) and np.array_equal(l, full_l[lo:lo + cnt])


def _digraph(n, m, seed):
    rng = np.random.default_rng(seed)
    src, dst = rng.integers(0, n, m), rng.integers(0, n, m)
    keep = src != dst
    return et.csr_from_coo(np.stack([src[keep], dst[keep]]), n)


def _hop_parts(rowptr, col, n, fanout, seed=0, samples=None):
    """The pool of each hop separately (the pool of hops 1..d minus that of hops 1..d-1)."""
    parts, prev = [], 0
    for d in range(1, len(fanout) + 1):
        pool = et.khop_fanout_pool(rowptr, col, n, fanout[:d], seed=seed,
                                   samples=None if samples is None else samples[:d])
        parts.append(pool[:, prev:])
        prev = pool.shape[1]
    return parts


def _counts(pool, n):
    c = np.zeros((n, n), dtype=np.int64)
    np.add.at(c, (pool[1], pool[0]), 1)         # c[query, kv]
    return c


def test_khop_all_neighbours_equals_path_counts():
    """fanout -1 at every hop: hop d emits, per origin u and node v != u, one pair per d-step out-path
    u -> ... -> v, which is (A^d)[u, v]."""
    n = 30
    rowptr, col = _digraph(n, 120, 3)
    A = np.zeros((n, n), dtype=np.int64)
    A[np.repeat(np.arange(n), np.diff(rowptr)), col] = 1
    Ad = np.eye(n, dtype=np.int64)
    for d, part in enumerate(_hop_parts(rowptr, col, n, [-1, -1, -1]), start=1):
        Ad = Ad @ A
        want = Ad.copy()
        np.fill_diagonal(want, 0)
        assert np.array_equal(_counts(part, n), want), d


def test_khop_expansion_follows_the_given_samples():
    """With injected samples the hop-d counts are the products of the sampled adjacencies A_1 ... A_d
    (one sample per node and hop, shared by every path through that node)."""
    n = 25
    rowptr, col = _digraph(n, 150, 8)
    rng = np.random.default_rng(1)
    samples, mats = [], []
    for d in range(3):
        ptr, ids = [0], []
        M = np.zeros((n, n), dtype=np.int64)
        for u in range(n):
            nb = col[rowptr[u]:rowptr[u + 1]]
            pick = sorted(rng.choice(nb, min(len(nb), 2), replace=False).tolist()) if len(nb) else []
            ids += pick
            ptr.append(len(ids))
            M[u, pick] += 1
        samples.append((np.array(ptr), np.array(ids, dtype=np.int64)))
        mats.append(M)
    P = np.eye(n, dtype=np.int64)
    for d, part in enumerate(_hop_parts(rowptr, col, n, [2, 2, 2], samples=samples), start=1):
        P = P @ mats[d - 1]
        want = P.copy()
        np.fill_diagonal(want, 0)
        assert np.array_equal(_counts(part, n), want), d


def test_fanout_sample_subsets_of_distinct_neighbours():
    rowptr, col = _digraph(200, 3000, 4)
    for f in (0, 1, 3, 8, 40):
        ptr, ids = et.fanout_sample(rowptr, col, 200, f, hop=2, seed=11)
        for u in range(200):
            nb = col[rowptr[u]:rowptr[u + 1]]
            got = ids[ptr[u]:ptr[u + 1]]
            assert len(got) == min(len(nb), f)
            assert len(set(got.tolist())) == len(got) and set(got.tolist()) <= set(nb.tolist())
            assert np.all(np.diff(got) > 0)                   # ascending index order = ascending id here
            if len(nb) <= f:
                assert np.array_equal(got, nb)
    ptr, ids = et.fanout_sample(rowptr, col, 200, -1, hop=1, seed=11)
    assert np.array_equal(ptr, rowptr) and np.array_equal(ids, col)


def test_fanout_sample_is_uniform_and_depends_on_seed_and_hop():
    """A hub with 40 out-neighbours sampled 10 at a time: over 2000 seeds every neighbour is chosen
    about 500 times (chi-square, 39 degrees of freedom); hop and seed change the draw."""
    deg, f, trials = 40, 10, 2000
    rowptr = np.array([0, deg] + [deg] * deg, dtype=np.int64)
    col = np.arange(1, deg + 1, dtype=np.int64)
    n = deg + 1
    hits = np.zeros(n, dtype=np.int64)
    for s in range(trials):
        ptr, ids = et.fanout_sample(rowptr, col, n, f, hop=1, seed=s)
        hits[ids[ptr[0]:ptr[1]]] += 1
    expect = trials * f / deg
    chi2 = (((hits[1:] - expect) ** 2) / expect).sum()
    assert chi2 < 80.0                                  # P(chi2_39 > 80) < 1e-4
    a = et.fanout_sample(rowptr, col, n, f, hop=1, seed=5)[1]
    assert not np.array_equal(a, et.fanout_sample(rowptr, col, n, f, hop=2, seed=5)[1])
    assert not np.array_equal(a, et.fanout_sample(rowptr, col, n, f, hop=1, seed=6)[1])
