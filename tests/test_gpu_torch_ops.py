"""The TORCH_LIBRARY(bf, ...) operators on the GPU: each against the raw C ABI (the same kernels,
bit for bit) and against the oracle at the parity bar (fp32 1e-5, bf16 2e-2, fp16 5e-3 relative, per tensor
and per row as in test_gpu_attention; integer outputs bit-exact)."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import edge_table as et
from oracle import philox
from oracle import sparse_attention as sa
from parity_helpers import rel_err, row_rel_err

pytestmark = pytest.mark.gpu


def _ops():
    from budgetformer_amd import _native
    return _native.load_ops()


def _index(dev, S, E, seed, n_kv=None):
    from budgetformer_amd.hip_ops import AttentionIndex
    g = torch.Generator().manual_seed(seed)
    n_kv = S if n_kv is None else n_kv
    ei = torch.stack([torch.randint(0, n_kv, (E,), generator=g), torch.randint(0, S, (E,), generator=g)])
    # a few long rows so the split plans are used too
    hot = torch.stack([torch.randint(0, n_kv, (900,), generator=g), torch.full((900,), 3)])
    ei = torch.cat([ei, hot], dim=1)
    return AttentionIndex.from_coo(ei.to(dev), S, n_kv)


def _acts(dev, S, n_kv, H, hn, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(S, H, hn, generator=g).to(dtype)
    k, v = (torch.randn(n_kv, H, hn, generator=g).to(dtype) for _ in range(2))
    dout = torch.randn(S, H, hn, generator=g).to(dtype)
    return [t.to(dev).contiguous() for t in (q, k, v, dout)]


def _abi_fwd_bwd(idx, q, k, v, dout, bias, factor, drop):
    """The same calls through ctypes on the raw C ABI (bf_attn_fwd / bf_attn_bwd)."""
    from budgetformer_amd import _native as N
    H, hn = q.shape[1], q.shape[2]
    p = lambda t: C.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    st = torch.cuda.current_stream(q.device).cuda_stream
    dt = {torch.float32: N.BF_DTYPE_F32, torch.bfloat16: N.BF_DTYPE_BF16, torch.float16: N.BF_DTYPE_F16}[q.dtype]
    d = C.byref(N.AttnDropout(drop[0], drop[1], drop[2])) if drop[0] > 0 else None
    sf = idx.struct(backward=False)
    out = torch.empty_like(q)
    Z = torch.empty(q.shape[0], H, dtype=torch.float32, device=q.device)
    parts = torch.empty(max(int(N.load().bf_attn_partials_floats(C.byref(sf), H, hn)), 1), device=q.device)
    N.call("bf_attn_fwd", C.byref(sf), dt, H, hn, 5.0, p(q), p(k), p(v), p(bias), p(factor), d, p(out), p(Z),
           p(parts), C.c_void_p(st))
    sb = idx.struct(backward=True, entries=True)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    db = torch.empty(idx.nnz, H, dtype=torch.float32, device=q.device)
    rs = torch.empty(q.shape[0], H, 2, dtype=torch.float32, device=q.device)
    parts = torch.empty(max(int(N.load().bf_attn_partials_floats(C.byref(sb), H, hn)), 1), device=q.device)
    N.call("bf_attn_bwd", C.byref(sb), dt, H, hn, 5.0, p(q), p(k), p(v), p(bias), p(factor), d, p(Z), p(dout),
           p(dq), p(dk), p(dv), p(db), p(rs), p(parts), C.c_void_p(st))
    return out, Z, dq, dk, dv, db


@pytest.mark.parametrize("dtype,extras", [(torch.float32, False), (torch.float32, True), (torch.bfloat16, False),
                                          (torch.bfloat16, True), (torch.float16, False), (torch.float16, True)])
def test_attention_ops_equal_the_abi_and_the_oracle(hip_device, dtype, extras):
    S, n_kv, H, hn = 700, 650, 8, 16
    idx = _index(hip_device, S, 9000, seed=5, n_kv=n_kv)
    q, k, v, dout = _acts(hip_device, S, n_kv, H, hn, dtype, seed=6)
    bias = factor = None
    drop = (0.0, 0, 0)
    if extras:
        gen = torch.Generator(device=hip_device).manual_seed(7)
        bias = torch.randn(idx.nnz, H, generator=gen, device=hip_device) * 0.5
        factor = torch.rand(idx.nnz, H, generator=gen, device=hip_device) + 0.5
        drop = (0.3, 2 ** 63 + 11, 5)           # a seed past 2^63 travels as a signed int
    ops = _ops()
    t, n = idx.op_args(backward=False)
    seed = drop[1] - 2 ** 64 if drop[1] >= 2 ** 63 else drop[1]
    out, Z, _ = ops.sparse_attn_fwd(q, k, v, t, n, bias, factor, drop[0], seed, drop[2])
    t, n = idx.op_args(backward=True, entries=True)
    dq, dk, dv, db = ops.sparse_attn_bwd(q, k, v, t, n, Z, dout, bias, factor, True, drop[0], seed, drop[2])
    torch.cuda.synchronize()
    ref = _abi_fwd_bwd(idx, q, k, v, dout, bias, factor, drop)
    for name, a, b in zip(("out", "Z", "dq", "dk", "dv", "dbias"), (out, Z, dq, dk, dv, db), ref):
        assert torch.equal(a, b), name
    # the oracle, in CSR order, with the keep mask drawn from the Philox oracle
    ei = torch.stack([idx.kv.cpu().long(), idx.entry_rows().cpu()])
    f64 = None
    if extras:
        keep = philox.dropout_keep_csr(idx.qptr.cpu().numpy(), H, drop[0], seed=drop[1], offset=drop[2])
        f64 = factor.cpu().double() * torch.from_numpy(keep).double() / (1.0 - drop[0])
    b64 = None if bias is None else bias.cpu().double()
    q64, k64, v64, d64 = (x.cpu().double() for x in (q, k, v, dout))
    ro, rZ = sa.attention_forward_stats(k64, q64, v64, ei, b64, f64)
    rdq, rdk, rdv, rdb = sa.attention_backward_closed_form(k64, q64, v64, ei, ro, rZ, d64, b64, f64)
    tol = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 5e-3}[dtype]
    for name, a, r in (("out", out, ro), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv), ("dbias", db, rdb)):
        err = max(rel_err(a, r), row_rel_err(a, r, floor=0.1))
        assert err < tol, (name, err)


def test_attention_op_errors(hip_device):
    """Argument errors raise before any launch: ValueError for shapes, dtypes and host tensors,
    NotImplementedError for a head size the kernels do not tile."""
    ops = _ops()
    idx = _index(hip_device, 50, 300, seed=8)
    q, k, v, dout = _acts(hip_device, 50, 50, 2, 8, torch.float32, seed=9)
    t, n = idx.op_args(backward=False)
    with pytest.raises(ValueError, match="do not match the index"):
        ops.sparse_attn_fwd(q[:40], k, v, t, n)
    with pytest.raises(ValueError, match="float32, bfloat16 and float16"):
        ops.sparse_attn_fwd(q.double(), k.double(), v.double(), t, n)
    with pytest.raises(ValueError, match="bias"):
        ops.sparse_attn_fwd(q, k, v, t, n, torch.zeros(3, 2, device=hip_device))
    with pytest.raises(ValueError, match="dropout rate"):
        ops.sparse_attn_fwd(q, k, v, t, n, None, None, 1.5, 1, 0)
    q6, k6, v6, _ = _acts(hip_device, 50, 50, 2, 6, torch.float32, seed=9)
    with pytest.raises(NotImplementedError):
        ops.sparse_attn_fwd(q6, k6, v6, t, n)
    # the index tensors select the device kernel, which refuses host activations
    with pytest.raises(ValueError, match="device tensor"):
        ops.sparse_attn_fwd(q.cpu(), k.cpu(), v.cpu(), t, n)


@pytest.mark.parametrize("records", [False, True])
def test_edge_ops_against_the_oracle(hip_device, records):
    from budgetformer_amd import hip_ops
    from budgetformer_amd.graph import CSRGraph, chung_lu_csr
    ops = _ops()
    n, P, L, b_r, b_w = 2500, 2, 4, 4, 4
    rowptr, col = chung_lu_csr(n, 30000, seed=12)
    g = CSRGraph.from_csr(rowptr, col, n, device=hip_device)
    u = np.random.default_rng(13).random((n * P, L), dtype=np.float32)
    ud = torch.from_numpy(u).to(hip_device)
    walks = ops.rw_walk(g.rowptr, g.col, 0, n, P, L, 0, 0, ud)
    assert np.array_equal(walks.cpu().numpy(), et.random_walk(rowptr, col, et.walk_starts(n, P), L, u))
    walks = ops.rw_walk(g.rowptr, g.col, 0, n, P, L, 42, 3)
    u42 = philox.walk_uniforms(0, n, P, L, 42, 3)
    assert np.array_equal(walks.cpu().numpy(), et.random_walk(rowptr, col, et.walk_starts(n, P), L, u42))
    rec = hip_ops.walk_records(g.rowptr, g.col) if records else None
    table, row_len = ops.build_edge_table(g.rowptr, g.col, rec, g.in_ptr, g.in_src, 0, n, P, L, b_r, b_w, 42, ud)
    ref_t, ref_len = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, 42, u)
    assert np.array_equal(table.cpu().numpy(), ref_t) and np.array_equal(row_len.cpu().numpy(), ref_len)
    # the index formats: CSR in table order, then each key's entries in CSR order
    qptr, kv = ops.table_to_csr(table, row_len, False, -1)
    lens = ref_len.astype(np.int64)
    assert np.array_equal(qptr.cpu().numpy(), np.concatenate([[0], np.cumsum(lens)]))
    flat = np.concatenate([ref_t[i, :lens[i]] for i in range(n)])
    assert np.array_equal(kv.cpu().numpy(), flat)
    kptr, kq, ks = ops.transpose_table(qptr, kv, n)
    order = np.argsort(flat, kind="stable")
    rows = np.repeat(np.arange(n), lens)
    slots = np.arange(flat.size) - np.concatenate([[0], np.cumsum(lens)])[rows]
    assert np.array_equal(ks.cpu().numpy(), slots[order])
    assert np.array_equal(kq.cpu().numpy(), rows[order])
    assert np.array_equal(kptr.cpu().numpy(), np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=n))]))
