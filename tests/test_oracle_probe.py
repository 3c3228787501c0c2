"""Pins for the oracle's Adaptive-Budget probe restatement (oracle/edge_table.py, probe section)."""
import numpy as np
import pytest

from oracle import edge_table as et


def _graph(n, e, seed):
    rng = np.random.default_rng(seed)
    src = rng.integers(0, n, e)
    dst = rng.integers(0, n, e)
    keep = src != dst
    ei = np.unique(np.stack([src[keep], dst[keep]]), axis=1)
    return np.concatenate([ei, ei[::-1]], axis=1)            # symmetric, coalesced below


def _coalesced(ei, n):
    return et.coalesce(ei, n)


def test_reception_cone_chain_closed_form():
    ei = np.stack([np.arange(9), np.arange(1, 10)])          # 0 -> 1 -> ... -> 9
    assert et.reception_cone(ei, [9], 3).tolist() == [7, 8, 9]
    assert et.reception_cone(ei, [9], 1) == [9]               # n_layers <= 1: unchanged
    assert et.reception_cone(ei, [0], 4).tolist() == [0]      # nothing flows into 0
    assert et.reception_cone(ei, [12, 9], 2).tolist() == [8, 9]   # ids beyond max edge id dropped


@pytest.mark.parametrize("seed,layers", [(0, 2), (1, 3), (2, 4)])
def test_reception_cone_matches_matrix_reachability(seed, layers):
    rng = np.random.default_rng(seed)
    n = 40
    src, dst = rng.integers(0, n, 70), rng.integers(0, n, 70)
    ei = np.stack([src, dst])
    probe = rng.choice(n, 5, replace=False)
    m = int(ei.max()) + 1
    adj = np.zeros((m, m), dtype=np.int64)
    adj[ei[0], ei[1]] = 1
    r = np.zeros(m, dtype=np.int64)
    r[probe[probe < m]] = 1
    for _ in range(layers - 1):                              # r <- r or A r (sources of edges into r)
        r = np.minimum(1, r + adj @ r)
    assert et.reception_cone(ei, probe, layers).tolist() == np.nonzero(r)[0].tolist()


def test_subtract_and_filter_closed_form():
    a = np.array([[1, 2, 2, 3, 4], [0, 0, 0, 5, 5]])
    b = np.array([[2, 9], [0, 9]])
    assert et.subtract_edge_index(a, b, 10).tolist() == [[1, 3, 4], [0, 5, 5]]    # every copy of (2,0) goes
    assert et.filter_edge_index_by_dst(a, [5]).tolist() == [[3, 4], [5, 5]]


def _brute_probe(ei, n, F, b_r, b_w, L, P, seed, u, use_real=True):
    """Independent per-dst formulation: candidates of q are its in-edges and its own walks' hop entries."""
    rowptr, col = et.csr_from_coo(ei, n)
    walks = et.random_walk(rowptr, col, et.walk_starts(n, P), L, u)
    real_pairs = set(zip(ei[0].tolist(), ei[1].tolist()))
    real_any = any(int(d) in set(F) for d in ei[1])
    out_r, out_w = [], []
    for q in F:
        rc = sorted([(int(et.edge_key(s, q, seed + 17)), int(s)) for s, d in zip(*ei) if d == q])
        out_r += [(s, q) for _, s in rc[:b_r]] if b_r > 0 else []
        wc = []
        for p in range(P):
            w = walks[q * P + p]
            for d in range(1, L + 1):
                if d == 1 or w[d] != w[d - 1]:
                    if not (use_real and real_any and (int(w[d]), q) in real_pairs):
                        wc.append((int(et.edge_key(w[d], q, seed + 37)), int(w[d])))
        wc.sort()
        out_w += [(s, q) for _, s in wc[:b_w]] if b_w > 0 else []
    if out_r and out_w:
        return sorted(set(out_r) | set(out_w))
    return sorted(out_r + out_w)


@pytest.mark.parametrize("b_r,b_w", [(2, 2), (3, 0), (0, 3), (4, 5), (1, 1)])
def test_probe_assembly_matches_per_dst_brute_force(b_r, b_w):
    n, P, L, seed = 60, 2, 4, 11
    ei = _coalesced(_graph(n, 200, 3), n)
    u = np.random.default_rng(5).random((n * P, L), dtype=np.float32)
    F = [3, 7, 8, 20, 41, 59]
    pools = et.probe_edge_pools(ei, n, F, L, P, u)
    got = et.assemble_edges_from_pools(pools, n, b_r, b_w, seed)
    assert sorted(zip(got[0].tolist(), got[1].tolist())) == _brute_probe(ei, n, F, b_r, b_w, L, P, seed, u)


def test_probe_candidates_are_nested():
    n, P, L, seed = 80, 4, 4, 3
    ei = _coalesced(_graph(n, 300, 8), n)
    u = np.random.default_rng(6).random((n * P, L), dtype=np.float32)
    F = np.arange(0, n, 3)
    pools = et.probe_edge_pools(ei, n, F, L, P, u)
    prev = set()
    for b in range(1, 7):
        part = et.assemble_edges_from_pools(pools, n, 0, b, seed)
        cur = set(zip(part[0].tolist(), part[1].tolist()))
        assert prev <= cur
        prev = cur


def test_probe_over_all_nodes_without_real_is_the_training_rw_build():
    n, P, L, seed = 70, 2, 4, 9
    ei = _coalesced(_graph(n, 250, 4), n)
    u = np.random.default_rng(7).random((n * P, L), dtype=np.float32)
    pools = et.probe_edge_pools(ei, n, np.arange(n), L, P, u, use_real=False)
    got = et.assemble_edges_from_pools(pools, n, 0, 4, seed)
    ref = et.build_merged_edges(ei, n, 0, 4, L, P, seed, u)
    assert sorted(zip(*got.tolist())) == sorted(zip(*ref.tolist()))


def test_probe_exphormer_typed_and_token_forms():
    n, P, L, seed = 50, 2, 3, 2
    ei = _coalesced(_graph(n, 160, 9), n)
    u = np.random.default_rng(8).random((n * P, L), dtype=np.float32)
    F = [1, 2, 3, 30]
    pools = et.probe_edge_pools(ei, n, F, L, P, u)
    typed = et.assemble_edges_from_pools(pools, n, 2, 2, seed, exphormer=True)
    real = et.assemble_edges_from_pools({"real": pools["real"], "rw": None}, n, 2, 0, seed)
    rw = et.assemble_edges_from_pools({"real": None, "rw": pools["rw"]}, n, 0, 2, seed)
    assert typed[:2, typed[2] == 0].tolist() == real.tolist() and typed[:2, typed[2] == 1].tolist() == rw.tolist()
    tok = et.assemble_edges_from_pools(pools, n, 2, 2, seed, graphormer_global_token=True)
    merged = et.assemble_edges_from_pools(pools, n, 2, 2, seed)
    assert tok.shape[1] == merged.shape[1] + 2 * n and (tok[:, :merged.shape[1]] == merged + 1).all()
