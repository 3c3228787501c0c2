"""BASELINE's first configuration, c1: the reference's CPU-runnable plumbing case (a synthetic uniform graph,
N = 2,708, 10,556 directed edges; Graphormer 4 layers, hidden 64, 8 heads, walk_length 4, walks_per_node 2,
B = 8 as (4, 4), seed 42), end to end through the build: the edge table bit-exact against the oracle, then
four attention layers on the one cached index (Q/K/V/O projections and residuals, as
models/graphormer_dist_node_level.py:644-671 wraps the sparse attention), forward and backward, against the
same stack in float64 on the oracle's Graphormer attention (models/graphormer_dist_node_level.py:215-263).

Bar: the north star's float32 bar, 1e-5 relative (max |diff| / max |ref| per tensor), on the output and on
every gradient, through four layers of float32 projections (rocBLAS GEMMs) and their backward (measured:
2.5e-6 at most)."""
import numpy as np
import pytest
import torch

from oracle import edge_table as et
from oracle import sparse_attention as sa

pytestmark = pytest.mark.gpu


def _stack(x, weights, attn, S, H, hn):
    for wq, wk, wv, wo in weights:
        q, k, v = ((x @ w).view(S, H, hn) for w in (wq, wk, wv))
        x = x + attn(q, k, v).reshape(S, H * hn) @ wo
    return x


def test_c1_four_layer_stack_through_the_build(hip_device):
    from budgetformer_amd.attention import sparse_edge_attention
    from budgetformer_amd.edges import build_attention_edges
    from budgetformer_amd.graph import CSRGraph, uniform_random_csr
    n, e, P, L, hidden, H, layers = 2708, 10556, 2, 4, 64, 8, 4
    hn = hidden // H
    rowptr, col = uniform_random_csr(n, e, seed=42)
    assert int(rowptr[-1]) == e
    g = CSRGraph.from_csr(rowptr, col, n, device=hip_device)
    u = np.random.default_rng(45).random((n * P, L), dtype=np.float32)
    tab = build_attention_edges(g, real_edges_per_query=4, rw_edges_per_query=4, walk_length=L, walks_per_node=P,
                                edge_seed=42, u=torch.from_numpy(u).to(hip_device), global_token=True)
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, 4, 4, L, P, 42, u)
    assert np.array_equal(tab.table.cpu().numpy(), ref_t)
    assert np.array_equal(tab.row_len.cpu().numpy(), ref_len)
    idx = tab.attention_index()
    ei = torch.stack([idx.kv.cpu().long(), idx.entry_rows().cpu()])   # the index's edges, CSR order
    S = n + 1                                                          # the Graphormer token row first

    gen = torch.Generator().manual_seed(43)
    x0 = torch.randn(S, hidden, generator=gen)
    w0 = [[torch.randn(hidden, hidden, generator=gen) / hidden ** 0.5 for _ in range(4)] for _ in range(layers)]
    probe = torch.randn(S, hidden, generator=gen)

    xg = x0.to(hip_device).requires_grad_(True)
    wg = [[w.to(hip_device).requires_grad_(True) for w in ws] for ws in w0]
    yg = _stack(xg, wg, lambda q, k, v: sparse_edge_attention(q, k, v, idx), S, H, hn)
    (yg * probe.to(hip_device)).sum().backward()
    torch.cuda.synchronize()

    xr = x0.double().requires_grad_(True)
    wr = [[w.double().requires_grad_(True) for w in ws] for ws in w0]
    yr = _stack(xr, wr, lambda q, k, v: sa.graphormer_sparse_attention(k, q, v, ei), S, H, hn)
    (yr * probe.double()).sum().backward()

    pairs = [("out", yg.detach(), yr.detach()), ("d x", xg.grad, xr.grad)]
    for li in range(layers):
        for name, a, b in zip("qkvo", wg[li], wr[li]):
            pairs.append((f"layer {li} d W{name}", a.grad, b.grad))
    worst = (0.0, "")
    for name, got, ref in pairs:
        err = ((got.double().cpu() - ref).abs().max() / ref.abs().max()).item()
        assert err < 1e-5, f"{name}: relative error {err:.3g}"
        worst = max(worst, (err, name))
    print(f"c1 stack: {idx.nnz} entries, largest relative error {worst[0]:.3g} ({worst[1]})")
