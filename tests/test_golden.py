"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces them. GPU: the HIP kernels reproduce them.
"""
import os

import numpy as np
import pytest
import torch

from oracle import edge_table as et
from oracle import philox
from oracle import sparse_attention as sa

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return dict(np.load(os.path.join(GOLDEN, name), allow_pickle=False))


def test_oracle_reproduces_edge_fixture():
    f = _load("edge_table_n300.npz")
    n, L, P, seed = int(f["num_nodes"]), int(f["walk_length"]), int(f["walks_per_node"]), int(f["edge_seed"])
    assert np.array_equal(et.random_walk(f["rowptr"], f["col"], et.walk_starts(n, P), L, f["u"]), f["walks"])
    for b_r, b_w in ((4, 4), (0, 3), (3, 0)):
        t, rl = et.build_edge_table(f["rowptr"], f["col"], n, b_r, b_w, L, P, seed, f["u"])
        assert np.array_equal(t, f[f"table_{b_r}_{b_w}"]) and np.array_equal(rl, f[f"row_len_{b_r}_{b_w}"])
    assert np.array_equal(philox.walk_uniforms(0, 16, 2, 6, 7, 3), f["philox_u_seed7"])


def test_oracle_reproduces_attention_fixture():
    f = _load("attention_s40.npz")
    t = {k: torch.from_numpy(v) for k, v in f.items()}
    out, Z = sa.attention_forward_stats(t["k"].double(), t["q"].double(), t["v"].double(), t["edge_index"],
                                        t["bias"].double())
    assert torch.allclose(out, t["out"], rtol=1e-12, atol=1e-12)
    dq, dk, dv, db = sa.attention_backward_closed_form(t["k"].double(), t["q"].double(), t["v"].double(),
                                                       t["edge_index"], out, Z, t["dout"].double(), t["bias"].double())
    for a, b in ((dq, "dq"), (dk, "dk"), (dv, "dv"), (db, "dbias")):
        assert torch.allclose(a, t[b], rtol=1e-12, atol=1e-12)


@pytest.mark.gpu
def test_gpu_reproduces_edge_fixture(hip_device):
    from budgetformer_amd import hip_ops
    from budgetformer_amd.edges import build_attention_edges
    from budgetformer_amd.graph import CSRGraph
    f = _load("edge_table_n300.npz")
    n, L, P, seed = int(f["num_nodes"]), int(f["walk_length"]), int(f["walks_per_node"]), int(f["edge_seed"])
    g = CSRGraph.from_csr(f["rowptr"], f["col"], n, device=hip_device)
    u = torch.from_numpy(f["u"]).to(hip_device)
    assert np.array_equal(hip_ops.random_walk(g.rowptr, g.col, 0, n, P, L, u=u).cpu().numpy(), f["walks"])
    for b_r, b_w in ((4, 4), (0, 3), (3, 0)):
        tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                    walks_per_node=P, edge_seed=seed, u=u)
        assert np.array_equal(tab.table.cpu().numpy(), f[f"table_{b_r}_{b_w}"])
        assert np.array_equal(tab.row_len.cpu().numpy(), f[f"row_len_{b_r}_{b_w}"])
    tab = build_attention_edges(g, real_edges_per_query=4, rw_edges_per_query=4, walk_length=L, walks_per_node=P,
                                edge_seed=seed, u=u, global_token=True)
    assert np.array_equal(tab.to_edge_index().cpu().numpy(), f["coo_graphormer_4_4"])
    assert np.array_equal(hip_ops.walk_uniforms(0, 16, 2, 6, 7, 3, device=hip_device).cpu().numpy(),
                          f["philox_u_seed7"])


@pytest.mark.gpu
def test_gpu_reproduces_attention_fixture(hip_device):
    from budgetformer_amd.attention import sparse_edge_attention
    from budgetformer_amd.hip_ops import AttentionIndex
    f = _load("attention_s40.npz")
    t = {k: torch.from_numpy(v) for k, v in f.items()}
    S = t["q"].shape[0]
    idx = AttentionIndex.from_coo(t["edge_index"].to(hip_device), S, chunk=8, item=16)
    # the fixture's edge order is the CSR order, so per-edge bias lines up entry for entry
    assert torch.equal(idx.kv.cpu().long(), t["edge_index"][0])
    q, k, v = (t[n].to(hip_device).requires_grad_(True) for n in ("q", "k", "v"))
    bias = t["bias"].to(hip_device).requires_grad_(True)
    out = sparse_edge_attention(q, k, v, idx, bias)
    out.backward(t["dout"].to(hip_device))
    for got, ref in ((out, "out"), (q.grad, "dq"), (k.grad, "dk"), (v.grad, "dv"), (bias.grad, "dbias")):
        ref = t[ref]
        err = ((got.detach().double().cpu() - ref).abs().max() / ref.abs().max()).item()
        assert err < 1e-5, (err, ref.shape)
