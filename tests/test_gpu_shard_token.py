"""The Graphormer global token on a query shard (gt_sp/utils.py:113-130,
models/graphormer_dist_node_level.py:1324-1359).

A shard [q_lo, q_hi) of the queries keeps every kv row (N + 1 with the token). The
shard that starts at node 0 also carries the token's own row (query 0, attending
every node); every shard row opens with kv 0. Checked here: the shard's table
equals the oracle's rows for that range, its attention index and COO equal the
matching rows of a full-set build, its forward and dq equal the full build's rows
bit for bit, the shards' dK/dV sum to the full build's, and each shard's
attention equals the float64 oracle on the shard's own edge set.
"""
import numpy as np
import pytest
import torch

from oracle import edge_table as et
from oracle import philox
from oracle import sparse_attention as sa
from parity_helpers import assert_close

pytestmark = pytest.mark.gpu

N_NODES, P, L, B_R, B_W, SEED = 2000, 2, 4, 4, 4, 42


def _graph(dev):
    from budgetformer_amd.graph import CSRGraph, chung_lu_csr
    rowptr, col = chung_lu_csr(N_NODES, 16000, seed=5)
    return rowptr, col, CSRGraph.from_csr(rowptr, col, N_NODES, device=dev)


def _build(g, lo=0, cnt=None):
    from budgetformer_amd.edges import build_attention_edges
    return build_attention_edges(g, real_edges_per_query=B_R, rw_edges_per_query=B_W, walk_length=L,
                                 walks_per_node=P, edge_seed=SEED, q_lo=lo, n_q=cnt, global_token=True)


def _rows(lo, hi):
    """Rows of the full-set index that a shard [lo, hi) holds, in the shard's row order."""
    return ([0] if lo == 0 else []) + list(range(lo + 1, hi + 1))


def _csr_rows(qptr, kv, rows):
    return [kv[qptr[r]:qptr[r + 1]].tolist() for r in rows]


CUTS = [(0, 700, 1500, 2000), (0, 1, 1999, 2000), (0, 2000)]


@pytest.mark.parametrize("cuts", CUTS)
def test_shard_tables_indexes_and_coo_equal_the_full_build(hip_device, cuts):
    rowptr, col, g = _graph(hip_device)
    full = _build(g)
    fidx = full.attention_index()
    fq, fkv = fidx.qptr.cpu(), fidx.kv.cpu()
    fcoo = full.to_edge_index().cpu()
    n_real = int(full.row_len.sum().item())
    f_real, f_tok, f_col = fcoo[:, :n_real], fcoo[:, n_real:n_real + N_NODES], fcoo[:, n_real + N_NODES:]
    for lo, hi in zip(cuts[:-1], cuts[1:]):
        sh = _build(g, lo, hi - lo)
        # table: the oracle's rows for the range, drawn from the same Philox stream
        u = philox.walk_uniforms(lo, hi - lo, P, L, SEED)
        ref_t, ref_len = et.build_edge_table(rowptr, col, N_NODES, B_R, B_W, L, P, SEED, u, q_lo=lo, n_q=hi - lo)
        assert np.array_equal(sh.table.cpu().numpy(), ref_t) and np.array_equal(sh.row_len.cpu().numpy(), ref_len)
        assert sh.holds_token_row == (lo == 0)
        idx = sh.attention_index()
        rows = _rows(lo, hi)
        assert (idx.n_q, idx.n_kv, idx.token_column) == (len(rows), N_NODES + 1, 1 if lo == 0 else 2)
        assert _csr_rows(idx.qptr.cpu(), idx.kv.cpu(), range(idx.n_q)) == _csr_rows(fq, fkv, rows)
        # COO: the full build's real edges and virtual edges whose query lies in the shard, in order
        coo = sh.to_edge_index().cpu()
        keep_r = (f_real[1] >= lo + 1) & (f_real[1] <= hi)
        keep_c = (f_col[1] >= lo + 1) & (f_col[1] <= hi)
        want = [f_real[:, keep_r]] + ([f_tok] if lo == 0 else []) + [f_col[:, keep_c]]
        assert torch.equal(coo, torch.cat(want, dim=1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cuts", CUTS[:2])
def test_shard_attention_equals_full_rows_and_oracle(hip_device, dtype, cuts):
    from budgetformer_amd.attention import sparse_edge_attention
    _, _, g = _graph(hip_device)
    H, hn = 8, 16
    S = N_NODES + 1
    gen = torch.Generator().manual_seed(7)
    q, k, v, dout = (torch.randn(S, H, hn, generator=gen).to(dtype) for _ in range(4))

    def run(idx, rows):
        qd = q[rows].to(hip_device).requires_grad_(True)
        kd, vd = (t.to(hip_device).requires_grad_(True) for t in (k, v))
        out = sparse_edge_attention(qd, kd, vd, idx)
        out.backward(dout[rows].to(hip_device))
        torch.cuda.synchronize()
        return out.detach().cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu()

    full = _build(g)
    f_out, f_dq, f_dk, f_dv = run(full.attention_index(), list(range(S)))
    dk_sum = torch.zeros(S, H, hn, dtype=torch.float64)
    dv_sum = torch.zeros(S, H, hn, dtype=torch.float64)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for lo, hi in zip(cuts[:-1], cuts[1:]):
        sh = _build(g, lo, hi - lo)
        idx = sh.attention_index()
        rows = _rows(lo, hi)
        out, dq, dk, dv = run(idx, rows)
        # the query side computes each row from the same entries in the same order: bit for bit
        assert torch.equal(out, f_out[rows]) and torch.equal(dq, f_dq[rows])
        dk_sum += dk.double()
        dv_sum += dv.double()
        # each shard against the oracle on its own edge set (global ids; shard rows are q[rows])
        coo = sh.to_edge_index().cpu()
        remap = torch.full((S,), -1, dtype=torch.int64)
        remap[torch.tensor(rows)] = torch.arange(len(rows))
        ei = torch.stack([coo[0], remap[coo[1]]])
        assert (ei[1] >= 0).all()
        qs = q[rows].double()
        ro, rZ = sa.attention_forward_stats(k.double(), qs, v.double(), ei)
        rdq, rdk, rdv, _ = sa.attention_backward_closed_form(k.double(), qs, v.double(), ei, ro, rZ,
                                                             dout[rows].double())
        for name, got, ref in (("out", out, ro), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
            assert_close(f"[{lo},{hi}) {name}", got, ref, tol)
    # the shards' key-side gradients add up to the full build's
    assert_close("sum dk", dk_sum, f_dk, tol)
    assert_close("sum dv", dv_sum, f_dv, tol)
