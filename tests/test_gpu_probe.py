"""GPU parity of the Adaptive-Budget probe build (budgetformer_amd.probe) against the oracle."""
import numpy as np
import pytest
import torch

from oracle import edge_table as et
from oracle import philox

pytestmark = pytest.mark.gpu


def _setup(n, e, seed, dev):
    from budgetformer_amd.graph import CSRGraph, chung_lu_csr
    rowptr, col = chung_lu_csr(n, e, exponent=2.1, seed=seed)
    g = CSRGraph.from_csr(rowptr, col, n, device=dev)
    src = np.repeat(np.arange(n), np.diff(rowptr))
    return g, np.stack([src, col.astype(np.int64)])


def _pairs(ei):
    return sorted(zip(ei[0].tolist(), ei[1].tolist()))


@pytest.mark.parametrize("layers", [1, 2, 3])
def test_reception_cone_matches_oracle(hip_device, layers):
    from budgetformer_amd.probe import reception_cone
    g, ei = _setup(3000, 12000, 21, hip_device)
    probe = torch.tensor([5, 17, 2999, 1200, 64], dtype=torch.int64)
    got = reception_cone(g, probe.to(hip_device), layers)
    ref = et.reception_cone(ei, probe.numpy(), layers)
    assert np.array_equal(got.cpu().numpy(), np.asarray(ref))


@pytest.mark.parametrize("P,L,thr", [(2, 4, 1024), (4, 4, 16), (3, 5, 8)])
def test_probe_candidates_bit_exact(hip_device, P, L, thr):
    from budgetformer_amd.probe import build_probe, reception_cone
    n, seed = 2500, 42
    g, ei = _setup(n, 20000, P * 7 + L, hip_device)
    rng = np.random.default_rng(P + L)
    u_full = rng.random((n * P, L), dtype=np.float32)
    probe = torch.from_numpy(rng.choice(n, 40, replace=False))
    F = reception_cone(g, probe.to(hip_device), 2)
    Fn = F.cpu().numpy()
    u_F = torch.from_numpy(u_full.reshape(n, P, L)[Fn].reshape(-1, L)).to(hip_device)
    pb = build_probe(g, F, max_real=6, max_rw=6, walk_length=L, walks_per_node=P, edge_seed=seed, u=u_F,
                     hub_threshold=thr)
    pools = et.probe_edge_pools(ei, n, Fn, L, P, u_full)
    for b_r, b_w in [(4, 4), (6, 4), (4, 6), (0, 5), (3, 0), (1, 1)]:
        got = pb.table(b_r, b_w).to_edge_index().cpu().numpy()
        ref = et.assemble_edges_from_pools(pools, n, b_r, b_w, seed)
        if b_r > 0 and b_w > 0:
            assert np.array_equal(got, ref)                 # merged: coalesce order
        else:
            assert _pairs(got) == _pairs(ref)               # one part: the sampled multiset
    typed = pb.typed_edge_index(3, 4).cpu().numpy()
    ref_t = et.assemble_edges_from_pools(pools, n, 3, 4, seed, exphormer=True)
    for t in (0, 1):
        assert _pairs(typed[:2, typed[2] == t]) == _pairs(ref_t[:2, ref_t[2] == t])


def test_probe_token_form_and_attention_index(hip_device):
    from budgetformer_amd.probe import build_probe
    n, P, L, seed = 1500, 2, 4, 7
    g, ei = _setup(n, 9000, 5, hip_device)
    rng = np.random.default_rng(1)
    u_full = rng.random((n * P, L), dtype=np.float32)
    Fn = np.sort(rng.choice(n, 300, replace=False))
    u_F = torch.from_numpy(u_full.reshape(n, P, L)[Fn].reshape(-1, L)).to(hip_device)
    pb = build_probe(g, torch.from_numpy(Fn).to(hip_device), max_real=4, max_rw=4, walk_length=L,
                     walks_per_node=P, edge_seed=seed, u=u_F, global_token=True)
    tab = pb.table(4, 4)
    ref = et.assemble_edges_from_pools(et.probe_edge_pools(ei, n, Fn, L, P, u_full), n, 4, 4, seed,
                                       graphormer_global_token=True)
    assert np.array_equal(tab.to_edge_index().cpu().numpy(), ref)
    idx = tab.attention_index()
    assert idx.n_q == n + 1 and idx.nnz == ref.shape[1]


def test_probe_rows_equal_training_rows_under_philox(hip_device):
    """Without the real pool (no subtraction) a probe row is the training build's row for that query."""
    from budgetformer_amd.edges import build_attention_edges
    from budgetformer_amd.probe import build_probe
    n, P, L, seed = 4000, 2, 4, 99
    g, _ = _setup(n, 30000, 12, hip_device)
    full = build_attention_edges(g, real_edges_per_query=0, rw_edges_per_query=5, walk_length=L,
                                 walks_per_node=P, edge_seed=seed)
    F = torch.arange(7, n, 13, device=hip_device)
    pb = build_probe(g, F, max_real=0, max_rw=5, walk_length=L, walks_per_node=P, edge_seed=seed, use_real=False)
    tab = pb.table(0, 5)
    assert torch.equal(tab.table, full.table[F]) and torch.equal(tab.row_len, full.row_len[F])
    # and the injected-uniform contract reproduces the Philox draw
    u_F = philox.walk_uniforms(0, n, P, L, seed).reshape(n, P, L)[F.cpu().numpy()].reshape(-1, L)
    pb2 = build_probe(g, F, max_real=0, max_rw=5, walk_length=L, walks_per_node=P, edge_seed=seed, use_real=False,
                      u=torch.from_numpy(u_F).to(hip_device))
    assert torch.equal(pb2.table(0, 5).table, tab.table)


def test_probe_wide_budgets_and_long_walks(hip_device):
    """The probe past the LDS staging: the real ranking at max_real = 800 (a workgroup per row, key
    order kept in the row's own slots), the RW ranking of P*L = 10,000 candidates with the real pool
    subtracted (streaming top-k), and candidates of up to 1,000 ids assembled in their table slots;
    bit-exact against the oracle's pools."""
    from budgetformer_amd.probe import build_probe
    n, P, L, seed = 1500, 100, 100, 11
    g, ei = _setup(n, 300_000, 29, hip_device)
    rng = np.random.default_rng(4)
    u_full = rng.random((n * P, L), dtype=np.float32)
    Fn = np.sort(rng.choice(n, 200, replace=False))
    u_F = torch.from_numpy(u_full.reshape(n, P, L)[Fn].reshape(-1, L)).to(hip_device)
    pb = build_probe(g, torch.from_numpy(Fn).to(hip_device), max_real=800, max_rw=500, walk_length=L,
                     walks_per_node=P, edge_seed=seed, u=u_F)
    pools = et.probe_edge_pools(ei, n, Fn, L, P, u_full)
    assert int(pb.real[1].max()) > 768
    for b_r, b_w in [(800, 200), (500, 500), (300, 300), (800, 0), (0, 500)]:
        got = pb.table(b_r, b_w).to_edge_index().cpu().numpy()
        ref = et.assemble_edges_from_pools(pools, n, b_r, b_w, seed)
        if b_r > 0 and b_w > 0:
            assert np.array_equal(got, ref)
        else:
            assert _pairs(got) == _pairs(ref)
