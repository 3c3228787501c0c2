"""IEEE float16 activations (the reference's fp16 autocast: utils/parser_node_level.py:266-272,
utils/fullgraph_sp_support.py:350-360 and :440, models/graphormer_dist_node_level.py:231-263) through the
three attention passes, against a float64 evaluation of the oracle on the same fp16-rounded inputs.

The bar is FP16_TOL = 5e-3, per tensor and per row (each row's scale floored at 1e-3 of the tensor's): the
kernels accumulate in float32 and round each result to fp16 once (2^-11 = 4.9e-4 of the value), so the
fp16 path is held four times tighter than bf16's 2e-2.
"""
import numpy as np
import pytest
import torch

from oracle import philox
from oracle import sparse_attention as sa
from parity_helpers import assert_close

pytestmark = pytest.mark.gpu

FP16_TOL = 5e-3
F16 = torch.float16


def _inputs(S, H, hn, E, seed, n_kv=None, mult=1.0):
    g = torch.Generator().manual_seed(seed)
    n_kv = S if n_kv is None else n_kv
    q = (torch.randn(S, H, hn, generator=g) * mult).to(F16)
    k = (torch.randn(n_kv, H, hn, generator=g) * mult).to(F16)
    v = torch.randn(n_kv, H, hn, generator=g).to(F16)
    ei = torch.stack([torch.randint(0, n_kv, (E,), generator=g), torch.randint(0, S, (E,), generator=g)])
    dout = torch.randn(S, H, hn, generator=g).to(F16)
    return q, k, v, ei, dout


def _oracle(q, k, v, ei, dout, factor_e=None):
    q64, k64, v64, d64 = (t.double() for t in (q, k, v, dout))
    f64 = None if factor_e is None else factor_e.double()
    out, Z = sa.attention_forward_stats(k64, q64, v64, ei, None, f64)
    dq, dk, dv, _ = sa.attention_backward_closed_form(k64, q64, v64, ei, out, Z, d64, None, f64)
    return out, dq, dk, dv


def _run(dev, q, k, v, idx, dout, dropout=None):
    from budgetformer_amd.attention import sparse_edge_attention
    qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = sparse_edge_attention(qd, kd, vd, idx, None, None, dropout)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    assert out.dtype == F16 and qd.grad.dtype == F16 and kd.grad.dtype == F16
    return out, qd.grad, kd.grad, vd.grad


def _coo_order(idx):
    return torch.stack([idx.kv.cpu().long(), idx.entry_rows().cpu()])


def _check(got, ref):
    for name, a, b in zip(("out", "dq", "dk", "dv"), got, ref):
        assert_close(name, a, b, FP16_TOL)


@pytest.mark.parametrize("chunk,item", [(128, 768), (6, 10)])
def test_fp16_random_coo(hip_device, chunk, item):
    """The tensor path on a random edge set (duplicates included), with and without split rows; scores
    scaled x2 so that some reach the clamp."""
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 900, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 9000, seed=61 + chunk, mult=2.0)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=chunk, item=item)
    _check(_run(hip_device, q, k, v, idx, dout), _oracle(q, k, v, ei, dout))


@pytest.mark.parametrize("chunk,item", [(128, 768), (5, 7)])
def test_fp16_table_with_token_row_and_column(hip_device, chunk, item):
    """A table index with the Graphormer token: the token row split into items, key 0's terms summed by
    the dq pass from its records."""
    from budgetformer_amd.hip_ops import AttentionIndex
    rng = np.random.default_rng(17 + chunk)
    n, width, H, hn = 1500, 6, 8, 16
    row_len = rng.integers(0, width + 1, n).astype(np.int32)
    table = np.full((n, width), -1, dtype=np.int32)
    for r in range(n):
        table[r, :row_len[r]] = np.sort(rng.choice(n, row_len[r], replace=False))
    idx = AttentionIndex.from_table(torch.from_numpy(table).to(hip_device), torch.from_numpy(row_len).to(hip_device),
                                    global_token=True, chunk=chunk, item=item)
    assert idx.token_column == 1
    S = idx.n_q
    q, k, v, _, dout = _inputs(S, H, hn, 1, seed=23)
    got = _run(hip_device, q, k, v, idx, dout)
    _check(got, _oracle(q, k, v, _coo_order(idx), dout))


@pytest.mark.parametrize("H,hn", [(2, 8), (1, 8), (4, 8)])
def test_fp16_narrow_rows(hip_device, H, hn):
    """Rows of 8 to 32 elements: groups of one, two or four lanes load the entry ids per iteration."""
    from budgetformer_amd.hip_ops import AttentionIndex
    S = 700
    q, k, v, ei, dout = _inputs(S, H, hn, 7000, seed=H * 10 + hn)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=6, item=10)
    _check(_run(hip_device, q, k, v, idx, dout), _oracle(q, k, v, ei, dout))


@pytest.mark.parametrize("rate", [0.5, 0.1])
def test_fp16_dropout(hip_device, rate):
    """The in-kernel GraphGPS dropout in fp16: the same keep bits (query row, slot) in all three passes as
    the oracle's mask."""
    from budgetformer_amd.hip_ops import AttentionIndex, Dropout
    S, H, hn = 900, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 9000, seed=71)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=16, item=24)
    seed, offset = (11 << 36) | 5, 3
    got = _run(hip_device, q, k, v, idx, dout, Dropout(rate, seed, offset))
    keep = torch.from_numpy(philox.dropout_keep_csr(idx.qptr.cpu().numpy(), H, rate, seed, offset))
    _check(got, _oracle(q, k, v, _coo_order(idx), dout, keep.double() / (1.0 - rate)))


def test_fp16_kv_pass_streaming_four_rows_prefetched_slots(hip_device):
    """The large-table dk/dv instance in fp16: 600K queries (q + dO = 307 MB, non-temporal gathers) and 2M
    kv rows (four rows per group, prefetched slots); 20K attending queries, 6K attended kv rows (one a
    3K-entry hub split into items), checked on the compacted problem; every other row comes out zero."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.hip_ops import AttentionIndex
    H, hn, n_q, n_kv = 8, 16, 600_000, 2_000_000
    assert hip_ops.kv_pass_variant(n_q, n_kv, F16, H, hn) == {"rows_per_group": 4, "stream_rows": True,
                                                               "prefetch_slots": True}
    g = torch.Generator(device=hip_device).manual_seed(91)
    qa = torch.randperm(n_q, generator=g, device=hip_device)[:20_000].sort().values
    kt = torch.randperm(n_kv, generator=g, device=hip_device)[:6_000].sort().values
    src_c = torch.randint(0, 6_000, (200_000,), generator=g, device=hip_device)
    src_c[:3_000] = 0
    dst_c = torch.randint(0, 20_000, (200_000,), generator=g, device=hip_device)
    q, dout = (torch.empty(n_q, H, hn, device=hip_device, dtype=F16).normal_(generator=g) for _ in range(2))
    k, v = (torch.empty(n_kv, H, hn, device=hip_device, dtype=F16).normal_(generator=g) for _ in range(2))
    idx = AttentionIndex.from_coo(torch.stack([kt[src_c], qa[dst_c]]), n_q, n_kv)
    out, Z = hip_ops.attn_forward(idx, q, k, v)
    dq, dk, dv, _ = hip_ops.attn_backward(idx, q, k, v, out, Z, dout)
    torch.cuda.synchronize()
    ei = torch.stack([src_c, dst_c]).cpu()
    ref = _oracle(q[qa].cpu(), k[kt].cpu(), v[kt].cpu(), ei, dout[qa].cpu())
    _check((out[qa], dq[qa], dk[kt], dv[kt]), ref)
    for t, rows in ((out, qa), (dq, qa), (dk, kt), (dv, kt)):
        t[rows] = 0
        assert not t.any()


def test_core_attention_under_fp16_autocast(hip_device):
    """The Graphormer layer as the reference runs it under `--amp_dtype fp16`: the Q/K/V projections under
    torch.autocast(float16) hand fp16 activations to CoreAttention, whose sparse path runs the fp16
    kernels; output and the gradients of the projection inputs against the oracle on the same fp16
    activations (their backward through the projections is PyTorch's)."""
    from budgetformer_amd.attention import CoreAttention
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 800, 8, 16
    D = H * hn
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, S, D, generator=g).to(hip_device)
    proj = torch.nn.Linear(D, 3 * D).to(hip_device)
    ei = torch.stack([torch.randint(0, S, (8000,), generator=g), torch.randint(0, S, (8000,), generator=g)])
    ei_d = ei.to(hip_device)
    core = CoreAttention(D, 0.0, H)
    with torch.autocast(device_type="cuda", dtype=F16):
        qkv = proj(x)
        assert qkv.dtype == F16
        q, k, v = (t.reshape(1, S, H, hn) for t in qkv.split(D, dim=-1))
        q.retain_grad(), k.retain_grad(), v.retain_grad()
        out = core(q, k, v, None, ei_d, "sparse")
    assert out.dtype == F16 and out.shape == (1, S, D)
    dout = torch.randn(1, S, D, generator=g).to(F16).to(hip_device)
    out.backward(dout)
    torch.cuda.synchronize()
    idx = AttentionIndex.from_coo(ei_d, S)
    ref = _oracle(q.detach()[0].cpu(), k.detach()[0].cpu(), v.detach()[0].cpu(), ei, dout.view(S, H, hn).cpu())
    _check((out.detach().view(S, H, hn), q.grad[0], k.grad[0], v.grad[0]), ref)
    assert idx.nnz == 8000


@pytest.mark.parametrize("chunk,item", [(128, 768), (6, 10)])
def test_fp16_bias_factor_and_dbias(hip_device, chunk, item):
    """The EX = 2 instances in fp16: a float32 bias per entry (its gradient, dbias, in float32) and a V
    factor per entry, with and without split rows; out, dq, dk, dv and dbias against the float64 oracle on
    the same fp16 inputs."""
    from budgetformer_amd.attention import sparse_edge_attention
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 900, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 9000, seed=81 + chunk)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=chunk, item=item)
    g = torch.Generator().manual_seed(5 + chunk)
    bias = torch.randn(idx.nnz, H, generator=g)
    factor = (torch.rand(idx.nnz, H, generator=g) >= 0.3).float() / 0.7
    qd, kd, vd = (t.to(hip_device).requires_grad_(True) for t in (q, k, v))
    bd = bias.to(hip_device).requires_grad_(True)
    out = sparse_edge_attention(qd, kd, vd, idx, bd, factor.to(hip_device), None)
    out.backward(dout.to(hip_device))
    torch.cuda.synchronize()
    assert out.dtype == F16 and bd.grad.dtype == torch.float32
    q64, k64, v64, d64 = (t.double() for t in (q, k, v, dout))
    ei_o = _coo_order(idx)
    r_out, r_Z = sa.attention_forward_stats(k64, q64, v64, ei_o, bias.double(), factor.double())
    r_dq, r_dk, r_dv, r_db = sa.attention_backward_closed_form(k64, q64, v64, ei_o, r_out, r_Z, d64,
                                                              bias.double(), factor.double())
    _check((out.detach(), qd.grad, kd.grad, vd.grad), (r_out, r_dq, r_dk, r_dv))
    assert_close("dbias", bd.grad, r_db, FP16_TOL)
