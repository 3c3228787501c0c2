"""Degenerate topologies end to end on the GPU: edge table, reference-order COO and attention.

Each graph stresses a corner of the build that random power-law graphs reach
only rarely or not at all:
- no edges at all (every walk stays put: the RW part is P copies of the
  dead-end self-edge, the real part is globally empty, so nothing is deduped);
- a single node;
- self-loops only (the real part and the d=1 walk edge are the same pair,
  deduped because both parts are non-empty);
- a star whose centre is a hub at the default hub threshold (in-degree 2999);
- a small complete graph (every in-row longer than the budget).
The table must equal the oracle bit for bit, its COO must equal the
reference pipeline (_build_merged_edges + fix_edge_index) element for element,
and one attention layer over the table must match the float64 oracle on the
reference COO within the fp32 bar (1e-5 relative).

Where every query attends to one distinct key (edgeless, single, self-loops,
each without the global token), dq and dk are the softmax gradient over a single key: the difference of two
equal terms, left over only through the 1e-6 in Z, so they are about 1e-6 of
the terms they cancel from and fp32 rounding of those terms decides their
relative error. There they are held to an absolute bound of 1e-6 times the
size of the terms (max |dO_h|·|v_h|·|k| / sqrt(hn)); out and dv keep the
relative bar.
"""
import math
import numpy as np
import pytest
import torch

from oracle import edge_table as et
from oracle import sparse_attention as sa

pytestmark = pytest.mark.gpu


_ONE_KEY = {"edgeless", "single", "self_loops"}     # without the token every query attends to one distinct key


def _star(n):
    src = np.concatenate([np.zeros(n - 1, np.int64), np.arange(1, n)])
    dst = np.concatenate([np.arange(1, n), np.zeros(n - 1, np.int64)])
    return et.csr_from_coo(np.stack([src, dst]), n)


def _complete(n):
    a, b = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    keep = a != b
    return et.csr_from_coo(np.stack([a[keep], b[keep]]).astype(np.int64), n)


def _case(name):
    if name == "edgeless":
        n = 64
        return n, np.zeros(n + 1, np.int64), np.zeros(0, np.int32)
    if name == "single":
        return 1, np.zeros(2, np.int64), np.zeros(0, np.int32)
    if name == "self_loops":
        n = 40
        return n, np.arange(n + 1, dtype=np.int64), np.arange(n, dtype=np.int32)
    if name == "star":
        n = 3000
        rowptr, col = _star(n)
        return n, rowptr, col
    n = 24
    rowptr, col = _complete(n)
    return n, rowptr, col


def _rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    scale = ref.abs().max().clamp_min(1e-30)
    return ((got - ref).abs().max() / scale).item()


@pytest.mark.parametrize("name", ["edgeless", "single", "self_loops", "star", "complete"])
@pytest.mark.parametrize("token", [False, True])
def test_degenerate_graph_table_coo_and_attention(hip_device, name, token):
    from budgetformer_amd.attention import sparse_edge_attention
    from budgetformer_amd.graph import CSRGraph
    from budgetformer_amd.edges import build_attention_edges
    n, rowptr, col = _case(name)
    col = np.asarray(col, np.int32)
    assert rowptr[-1] == col.size
    P, L, b_r, b_w = 2, 4, 4, 4
    g = CSRGraph.from_csr(rowptr, col, n, device=hip_device)
    u = np.random.default_rng(n).random((n * P, L), dtype=np.float32)
    tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                walks_per_node=P, edge_seed=42, u=torch.from_numpy(u).to(hip_device),
                                global_token=token)
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, 42, u)
    assert np.array_equal(tab.row_len.cpu().numpy(), ref_len)
    assert np.array_equal(tab.table.cpu().numpy(), ref_t)

    src = np.repeat(np.arange(n), np.diff(rowptr))
    ref_coo = et.build_merged_edges(np.stack([src, col.astype(np.int64)]), n, b_r, b_w, L, P, 42, u,
                                    graphormer_global_token=token)
    assert np.array_equal(tab.to_edge_index().cpu().numpy(), ref_coo)

    idx = tab.attention_index()
    S = n + (1 if token else 0)
    assert idx.n_q == S and idx.nnz == ref_coo.shape[1]
    H, hn = 8, 16
    gen = torch.Generator().manual_seed(n + token)
    q, k, v, dout = (torch.randn(S, H, hn, generator=gen) for _ in range(4))
    qd, kd, vd = (t.to(hip_device).requires_grad_(True) for t in (q, k, v))
    out = sparse_edge_attention(qd, kd, vd, idx)
    out.backward(dout.to(hip_device))
    torch.cuda.synchronize()
    ei = torch.from_numpy(ref_coo)
    ro, rZ = sa.attention_forward_stats(k.double(), q.double(), v.double(), ei)
    rdq, rdk, rdv, _ = sa.attention_backward_closed_form(k.double(), q.double(), v.double(), ei, ro, rZ,
                                                        dout.double())
    for got, ref in ((out, ro), (vd.grad, rdv)):
        assert _rel_err(got, ref) < 1e-5
    if name in _ONE_KEY and not token:
        for got, ref, other in ((qd.grad, rdq, k), (kd.grad, rdk, q)):
            terms = (dout.norm(dim=-1).max() * v.norm(dim=-1).max() * other.abs().max() / math.sqrt(hn)).item()
            assert (got.double().cpu() - ref).abs().max().item() < 1e-6 * terms
    else:
        for got, ref in ((qd.grad, rdq), (kd.grad, rdk)):
            assert _rel_err(got, ref) < 1e-5
