"""Parity of the kernel instances and table shapes the large configurations run.

c3 (2.45M nodes, bf16, B=16, P=4), c4 (2.92M nodes, bf16, B=32, L=8) and c5 (a 27.8M-query
shard, bf16) take code paths the small parity graphs never reach:
- the dk/dv pass with non-temporal q/dO gathers (q + dO above 256 MB), four kv rows per lane
  group and prefetched row slots (past 1M kv rows in bf16) — and in fp32 past 16M kv rows;
- edge tables of power-law graphs with ~17K-degree hubs at B=16 (8, 8) P=4 L=4 and
  B=32 (16, 16) P=4 L=8, drawn from the production Philox stream.
The attention problems keep a few thousand attended rows inside the large tables, so the
float64 oracle runs on the compacted problem (the attended rows only) in seconds; every other
row must come out zero.
"""
import numpy as np
import pytest
import torch

from oracle import edge_table as et
from oracle import philox
from oracle import sparse_attention as sa
from parity_helpers import assert_close

pytestmark = pytest.mark.gpu


def _compact_problem(dev, n_q, n_kv, active_q, touched_kv, E, hub_edges, dtype, seed, H=8, hn=16):
    g = torch.Generator(device=dev).manual_seed(seed)
    qa = torch.randperm(n_q, generator=g, device=dev)[:active_q].sort().values
    kt = torch.randperm(n_kv, generator=g, device=dev)[:touched_kv].sort().values
    src_c = torch.randint(0, touched_kv, (E,), generator=g, device=dev)
    src_c[:hub_edges] = 0                           # one hub key row: key-side split items
    dst_c = torch.randint(0, active_q, (E,), generator=g, device=dev)
    q = torch.empty(n_q, H, hn, device=dev, dtype=dtype).normal_(generator=g)
    dout = torch.empty(n_q, H, hn, device=dev, dtype=dtype).normal_(generator=g)
    k = torch.empty(n_kv, H, hn, device=dev, dtype=dtype).normal_(generator=g)
    v = torch.empty(n_kv, H, hn, device=dev, dtype=dtype).normal_(generator=g)
    return qa, kt, src_c, dst_c, q, dout, k, v


def _check_compact(hip_device, n_q, n_kv, dtype, expect, tol):
    from budgetformer_amd import hip_ops
    from budgetformer_amd.hip_ops import AttentionIndex
    H, hn = 8, 16
    variant = hip_ops.kv_pass_variant(n_q, n_kv, dtype, H, hn)
    assert variant == expect, variant
    qa, kt, src_c, dst_c, q, dout, k, v = _compact_problem(hip_device, n_q, n_kv, 20_000, 6_000, 200_000, 3_000,
                                                           dtype, seed=n_kv % 1000 + 11)
    idx = AttentionIndex.from_coo(torch.stack([kt[src_c], qa[dst_c]]), n_q, n_kv)
    out, Z = hip_ops.attn_forward(idx, q, k, v)
    dq, dk, dv, _ = hip_ops.attn_backward(idx, q, k, v, out, Z, dout)
    torch.cuda.synchronize()
    idx.resolve()
    assert idx.kplan.items > 0          # the hub key row ran as split items
    ei = torch.stack([src_c, dst_c]).cpu()
    qc, doc = q[qa].double().cpu(), dout[qa].double().cpu()
    kc, vc = k[kt].double().cpu(), v[kt].double().cpu()
    ro, rZ = sa.attention_forward_stats(kc, qc, vc, ei)
    rdq, rdk, rdv, _ = sa.attention_backward_closed_form(kc, qc, vc, ei, ro, rZ, doc)
    for name, got, ref in (("out", out[qa], ro), ("dq", dq[qa], rdq), ("dk", dk[kt], rdk), ("dv", dv[kt], rdv)):
        assert_close(name, got, ref, tol)
    for t, rows in ((out, qa), (dq, qa), (dk, kt), (dv, kt)):
        t[rows] = 0
        assert not t.any()


def test_bf16_kv_pass_streaming_four_rows_prefetched_slots(hip_device):
    """attn_bwd_kv_kernel<bf16, NT, PRE>, the dominant instance of c3-c5: 600K queries (q + dO = 307 MB)
    and 2M kv rows, 20K attending queries, 6K attended kv rows (one a 3K-entry hub)."""
    _check_compact(hip_device, 600_000, 2_000_000, torch.bfloat16,
                   {"rows_per_group": 4, "stream_rows": True, "prefetch_slots": True}, 2e-2)


def _csr_edges_compacted(idx, qa, kt):
    """The index's entries in CSR order as an oracle edge list [2, nnz] over the compacted rows (kv rows as
    positions in kt, queries as positions in qa): entry e of the index is column e."""
    kv = idx.kv.long()
    rows = idx.entry_rows()
    kv_c = torch.searchsorted(kt, kv)
    q_c = torch.searchsorted(qa, rows)
    assert torch.equal(kt[kv_c], kv) and torch.equal(qa[q_c], rows)
    return torch.stack([kv_c, q_c]).cpu()


@pytest.mark.parametrize("extras", ["dropout", "bias_dbias_dropout"])
def test_bf16_kv_pass_c4_instance_with_dropout(hip_device, extras):
    """The dk/dv instance c4 times: attn_bwd_kv_kernel<bf16, NT, PRE, EX=1> (dropout 0.5 drawn in the
    kernels; q + dO above 256 MB, more than 1M kv rows: non-temporal gathers, four rows per lane group,
    prefetched slots), and its general twin EX=2 (additive bias, dbias and dropout). Each entry's keep bits
    come from its query row and its slot in that row (kq and ks in the key-major pass), so the float64
    oracle takes the index's own CSR order, remapped to the compacted rows, with the mask
    oracle.philox.dropout_keep_csr draws over the index's row pointers."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.hip_ops import AttentionIndex, Dropout
    H, hn, rate = 8, 16, 0.5
    n_q, n_kv = 600_000, 2_000_000
    variant = hip_ops.kv_pass_variant(n_q, n_kv, torch.bfloat16, H, hn)
    assert variant == {"rows_per_group": 4, "stream_rows": True, "prefetch_slots": True}, variant
    qa, kt, src_c, dst_c, q, dout, k, v = _compact_problem(hip_device, n_q, n_kv, 20_000, 6_000, 200_000, 3_000,
                                                           torch.bfloat16, seed=404)
    idx = AttentionIndex.from_coo(torch.stack([kt[src_c], qa[dst_c]]), n_q, n_kv)
    nnz = idx.nnz
    seed, offset = (3 << 33) | 77, 9
    drop = Dropout(rate, seed, offset)
    bias = None
    if extras != "dropout":
        bias = (torch.randn(nnz, H, generator=torch.Generator().manual_seed(8)) * 0.7).to(hip_device)
    out, Z = hip_ops.attn_forward(idx, q, k, v, bias=bias, dropout=drop)
    dq, dk, dv, dbias = hip_ops.attn_backward(idx, q, k, v, out, Z, dout, bias=bias, need_dbias=bias is not None,
                                              dropout=drop)
    torch.cuda.synchronize()
    idx.resolve()
    assert idx.kplan.items > 0          # the hub key row ran as split items
    ei = _csr_edges_compacted(idx, qa, kt)
    keep = torch.from_numpy(philox.dropout_keep_csr(idx.qptr.cpu().numpy(), H, rate, seed, offset))
    factor = keep.double() / (1.0 - rate)
    qc, doc = q[qa].double().cpu(), dout[qa].double().cpu()
    kc, vc = k[kt].double().cpu(), v[kt].double().cpu()
    b64 = None if bias is None else bias.double().cpu()
    ro, rZ = sa.attention_forward_stats(kc, qc, vc, ei, b64, factor)
    rdq, rdk, rdv, rdb = sa.attention_backward_closed_form(kc, qc, vc, ei, ro, rZ, doc, b64, factor)
    for name, got, ref in (("out", out[qa], ro), ("dq", dq[qa], rdq), ("dk", dk[kt], rdk), ("dv", dv[kt], rdv)):
        assert_close(name, got, ref, 2e-2)
    if bias is not None:
        assert_close("dbias", dbias, rdb, 2e-2)
    # c4's timed step as the modules run it: the forward stores its keep bits and the dq pass reads them
    # (the dropout-only instances) — every output equal to the drawing form's bit for bit, the mask equal
    # to the oracle's bits
    out1, Z1, kmask = hip_ops.attn_forward(idx, q, k, v, bias=bias, dropout=drop, keep_mask=True)
    r1 = hip_ops.attn_backward(idx, q, k, v, out1, Z1, dout, bias=bias, need_dbias=bias is not None,
                               dropout=drop, keep=kmask)
    torch.cuda.synchronize()
    for name, a, b in (("out", out1, out), ("Z", Z1, Z), ("dq", r1[0], dq), ("dk", r1[1], dk), ("dv", r1[2], dv)):
        assert torch.equal(a, b), name
    if bias is not None:
        assert torch.equal(r1[3], dbias)
    bits = keep.numpy().astype(np.uint8) << np.arange(H, dtype=np.uint8)[None, :]
    assert np.array_equal(kmask[:nnz, 0].cpu().numpy(), np.bitwise_or.reduce(bits, axis=1))
    del out1, Z1, r1, kmask
    for t, rows in ((out, qa), (dq, qa), (dk, kt), (dv, kt)):
        t[rows] = 0
        assert not t.any()
    assert abs(keep.float().mean().item() - (1 - rate)) < 0.01


@pytest.mark.parametrize("extras", ["plain", "dropout", "bias_dbias_dropout"])
def test_bf16_token_row_entries_from_lds_equal_the_gathering_form(hip_device, extras):
    """With the Graphormer token row and four kv rows per lane group (c5's dk/dv instance: more than 1M kv
    rows in bf16, q + dO above 256 MB) the dk/dv pass takes every short kv row's first entry, query 0's,
    from a per-workgroup LDS copy of q[0], dO[0] and query 0's row stats. Against the same table's index
    without the token promise (every entry gathered, key 0 too): out, dq and dbias equal bit for bit, and so
    do dK and dV of every kv row but key 0 (whose terms the token form sums per dq-pass workgroup, in
    another order: within the parity bar)."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.hip_ops import AttentionIndex, Dropout
    n, width, H, hn = 1_200_000, 4, 8, 16
    g = torch.Generator(device=hip_device).manual_seed(31)
    row_len = torch.randint(0, width + 1, (n,), generator=g, device=hip_device, dtype=torch.int32)
    ids = torch.randint(0, n, (n, width), generator=g, device=hip_device, dtype=torch.int32).sort(dim=1).values
    table = torch.where(torch.arange(width, device=hip_device)[None, :] < row_len[:, None], ids,
                        torch.full_like(ids, -1))
    # a few hub kv rows longer than the split threshold (their first item keeps gathering query 0's entry)
    table[:3000, 0] = 7
    row_len[:3000] = torch.clamp(row_len[:3000], min=1)
    S = n + 1
    variant = hip_ops.kv_pass_variant(S, S, torch.bfloat16, H, hn)
    assert variant == {"rows_per_group": 4, "stream_rows": True, "prefetch_slots": True}, variant
    q, k, v, dout = (torch.empty(S, H, hn, device=hip_device, dtype=torch.bfloat16).normal_(generator=g)
                     for _ in range(4))
    runs = []
    for token in (True, False):
        idx = AttentionIndex.from_table(table, row_len, global_token=True)
        assert idx.token_column == 1
        idx.token_column = 1 if token else 0
        bias = drop = None
        if extras != "plain":
            drop = Dropout(0.5, 1234, 2)
        if extras == "bias_dbias_dropout":
            bias = torch.empty(idx.nnz, H, device=hip_device).normal_(generator=torch.Generator(
                device=hip_device).manual_seed(5))
        out, Z = hip_ops.attn_forward(idx, q, k, v, bias=bias, dropout=drop)
        dq, dk, dv, db = hip_ops.attn_backward(idx, q, k, v, out, Z, dout, bias=bias, need_dbias=bias is not None,
                                               dropout=drop)
        runs.append((out, dq, dk, dv, db))
    torch.cuda.synchronize()
    (out_t, dq_t, dk_t, dv_t, db_t), (out_g, dq_g, dk_g, dv_g, db_g) = runs
    assert torch.equal(out_t, out_g) and torch.equal(dq_t, dq_g)
    assert (db_t is None and db_g is None) or torch.equal(db_t, db_g)
    assert torch.equal(dk_t[1:], dk_g[1:]) and torch.equal(dv_t[1:], dv_g[1:])
    assert_close("dk[0]", dk_t[:1], dk_g[:1].float(), 2e-2)
    assert_close("dv[0]", dv_t[:1], dv_g[:1].float(), 2e-2)


def test_fp32_kv_pass_past_16m_rows_streaming(hip_device):
    """fp32 with four kv rows per group (17M kv rows) and non-temporal gathers (300K queries)."""
    _check_compact(hip_device, 300_000, 17_000_000, torch.float32,
                   {"rows_per_group": 4, "stream_rows": True, "prefetch_slots": False}, 1e-5)


@pytest.mark.parametrize("b_r,b_w,P,L", [(8, 8, 4, 4), (16, 16, 4, 8)])
def test_power_law_tables_with_17k_hubs(hip_device, b_r, b_w, P, L):
    """c3 (B=16 (8,8), P=4, L=4) and c4 (B=32 (16,16), P=4, L=8) table shapes on a device-generated
    120K-node power-law graph (avg degree 50, hubs near 17K): bit-exact against the oracle with the
    Philox uniforms the production walk draws; hub rows take the workgroup-per-query path."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.edges import build_attention_edges
    from budgetformer_amd.graph import chung_lu_device
    n = 120_000
    g = chung_lu_device(n, 6_000_000, exponent=2.1, seed=5, max_degree=17_000, device=hip_device)
    rowptr = g.rowptr.cpu().numpy()
    col = g.col.cpu().numpy()
    deg = np.diff(rowptr)
    assert deg.max() > 10_000 and (deg > hip_ops.HUB_THRESHOLD).sum() > 10
    tab = build_attention_edges(g, real_edges_per_query=b_r, rw_edges_per_query=b_w, walk_length=L,
                                walks_per_node=P, edge_seed=42)
    u = philox.walk_uniforms(0, n, P, L, 42)
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, 42, u)
    got_len = tab.row_len.cpu().numpy()
    assert np.array_equal(got_len, ref_len)
    assert np.array_equal(tab.table.cpu().numpy(), ref_t)
    assert (got_len == b_r + b_w).any() and (got_len < b_r + b_w).any()   # full and short rows both occur


@pytest.mark.parametrize("module", ["gt", "gps"])
def test_gt_and_gps_modules_bf16_forward_backward(hip_device, module):
    """GTCoreAttention (models/gt_dist_node_level.py:179-262) and GPSCoreAttention._sparse
    (models/graphgps_dist_node_level.py:151-177) in bf16 on an edge table, forward and backward,
    against the float64 oracle forms (GPS: eval mode, then an injected keep mask)."""
    from budgetformer_amd.attention import GPSCoreAttention, GTCoreAttention
    from budgetformer_amd.edges import build_attention_edges
    from budgetformer_amd.graph import CSRGraph, chung_lu_csr
    n, H, hn = 3000, 8, 16
    rowptr, col = chung_lu_csr(n, 30_000, seed=9)
    g = CSRGraph.from_csr(rowptr, col, n, device=hip_device)
    tab = build_attention_edges(g, real_edges_per_query=8, rw_edges_per_query=8, walk_length=4,
                                walks_per_node=4, edge_seed=42)
    idx = tab.attention_index()
    ei = tab.to_edge_index().cpu()
    gen = torch.Generator().manual_seed(21)
    q, k, v, dout = (torch.randn(n, H, hn, generator=gen).to(torch.bfloat16) for _ in range(4))
    masks = [None]
    if module == "gps":
        masks.append(torch.rand(idx.nnz, H, generator=gen) >= 0.5)
    for mask in masks:
        qd, kd, vd = (t[None].to(hip_device).requires_grad_(True) for t in (q, k, v))
        if module == "gt":
            mod = GTCoreAttention(H * hn, 0.0, H)
            out = mod(qd, kd, vd, None, tab)
        else:
            mod = GPSCoreAttention(H * hn, 0.5, H).eval()
            drop = None if mask is None else mask.to(hip_device)
            out = mod._sparse(qd, kd, vd, tab, H, hn, drop_mask=drop)
        assert out.dtype == torch.bfloat16 and out.shape == (1, n, H * hn)
        out.backward(dout.reshape(1, n, H * hn).to(hip_device))
        q64, k64, v64 = (t.double().requires_grad_(True) for t in (q, k, v))
        if module == "gt":
            ref = sa.gt_sparse_attention(q64, k64, v64, ei)
        else:
            # the mask is per CSR entry; the oracle's edge list is the index's CSR order
            ei_o = torch.stack([idx.kv.cpu().long(), idx.entry_rows().cpu()])
            ref = sa.gps_sparse_attention(q64, k64, v64, ei_o, mask, 2.0 if mask is not None else 1.0)
        ref.backward(dout.double())
        assert_close("out", out.view(n, H, hn), ref, 2e-2)
        for name, got, r in (("dq", qd.grad[0], q64.grad), ("dk", kd.grad[0], k64.grad), ("dv", vd.grad[0], v64.grad)):
            assert_close(name, got, r, 2e-2)
