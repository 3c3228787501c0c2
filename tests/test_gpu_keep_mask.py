"""The dropout's keep mask (bf_attn_dropout.keep, models/graphgps_dist_node_level.py:166-176): the forward
stores the keep bits it draws, one byte per 8 heads per CSR entry, and the backward's dq pass reads them
back instead of drawing them again. The stored bytes equal the Philox oracle's bits packed (heads 8b..8b+7
in byte b, bit h % 8), and every output of a forward and backward with the mask equals the same calls
without it bit for bit, so the oracle parity of the drawing form (test_gpu_dropout.py) carries over."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import philox

pytestmark = pytest.mark.gpu


def _pack(keep: np.ndarray) -> np.ndarray:
    """bool [E, H] -> uint8 [E, ceil(H / 8)], head h at bit h % 8 of byte h // 8."""
    E, H = keep.shape
    nb = (H + 7) // 8
    pad = np.zeros((E, nb * 8), dtype=bool)
    pad[:, :H] = keep
    return np.packbits(pad.reshape(E, nb, 8), axis=-1, bitorder="little").reshape(E, nb)


def _coo_index(dev, S, n_kv, E, seed, chunk=128, item=768):
    from budgetformer_amd.hip_ops import AttentionIndex
    g = torch.Generator().manual_seed(seed)
    ei = torch.stack([torch.randint(0, n_kv, (E,), generator=g), torch.randint(0, S, (E,), generator=g)])
    hot = torch.stack([torch.randint(0, n_kv, (900,), generator=g), torch.full((900,), 3)])   # a split row
    return AttentionIndex.from_coo(torch.cat([ei, hot], 1).to(dev), S, n_kv, chunk=chunk, item=item)


def _token_index(dev, n, width, seed):
    from budgetformer_amd.hip_ops import AttentionIndex
    rng = np.random.default_rng(seed)
    row_len = rng.integers(0, width + 1, n).astype(np.int32)
    table = np.full((n, width), -1, dtype=np.int32)
    for r in range(n):
        table[r, :row_len[r]] = np.sort(rng.choice(n, row_len[r], replace=False))
    idx = AttentionIndex.from_table(torch.from_numpy(table).to(dev), torch.from_numpy(row_len).to(dev),
                                    global_token=True, chunk=16, item=24)
    assert idx.token_column
    return idx


def _acts(dev, S, n_kv, H, hn, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q, dout = (torch.randn(S, H, hn, generator=g).to(dtype) for _ in range(2))
    k, v = (torch.randn(n_kv, H, hn, generator=g).to(dtype) for _ in range(2))
    return [t.to(dev).contiguous() for t in (q, k, v, dout)]


def _both(idx, q, k, v, dout, drop, bias=None, need_dbias=False):
    """(forward + backward without the mask, the same with it, the mask)."""
    from budgetformer_amd import hip_ops
    out0, Z0 = hip_ops.attn_forward(idx, q, k, v, bias=bias, dropout=drop)
    g0 = hip_ops.attn_backward(idx, q, k, v, None, Z0, dout, bias=bias, need_dbias=need_dbias, dropout=drop)
    out1, Z1, keep = hip_ops.attn_forward(idx, q, k, v, bias=bias, dropout=drop, keep_mask=True)
    g1 = hip_ops.attn_backward(idx, q, k, v, None, Z1, dout, bias=bias, need_dbias=need_dbias, dropout=drop,
                               keep=keep)
    torch.cuda.synchronize()
    return (out0, Z0) + tuple(g0), (out1, Z1) + tuple(g1), keep


def _check(idx, H, drop, plain, masked, keep):
    for name, a, b in zip(("out", "Z", "dq", "dk", "dv", "dbias"), plain, masked):
        assert (a is None and b is None) or torch.equal(a, b), name
    nnz = idx.nnz
    assert keep.dtype == torch.uint8 and keep.shape[1] == (H + 7) // 8 and keep.shape[0] >= nnz
    want = _pack(philox.dropout_keep_csr(idx.qptr.cpu().numpy(), H, drop.rate, drop.seed, drop.offset))
    assert np.array_equal(keep[:nnz].cpu().numpy(), want)


def _shapes(dtype):
    v = 4 if dtype == torch.float32 else 8      # elements per 16-byte lane load
    # H = 8: one byte per entry; H = 12: two bytes, an odd Philox block count; H = 2 with one lane per head:
    # a group narrower than an iteration's draws (its first lane stores the bytes)
    return [(8, 16), (12, 8), (2, v)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_mask_bits_and_bitwise_equal_gradients_coo(hip_device, dtype):
    from budgetformer_amd.hip_ops import Dropout
    for H, hn in _shapes(dtype):
        S, n_kv = 700, 650
        idx = _coo_index(hip_device, S, n_kv, 9000, seed=H + hn)
        q, k, v, dout = _acts(hip_device, S, n_kv, H, hn, dtype, seed=H * hn)
        drop = Dropout(0.5, (5 << 36) | H, 3)
        plain, masked, keep = _both(idx, q, k, v, dout, drop)
        _check(idx, H, drop, plain, masked, keep)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mask_with_split_rows_and_the_token(hip_device, dtype):
    """Split query rows (items of 10 entries: the forward's items store their entries' bytes) and the
    Graphormer token row and column (the dq pass's key-0 entry reads its byte; the dq reduce, which
    finishes the split token row, draws it)."""
    from budgetformer_amd.hip_ops import Dropout
    idx = _coo_index(hip_device, 600, 600, 7000, seed=21, chunk=6, item=10)
    q, k, v, dout = _acts(hip_device, 600, 600, 8, 16, dtype, seed=22)
    drop = Dropout(0.3, 77, 0)
    plain, masked, keep = _both(idx, q, k, v, dout, drop)
    _check(idx, 8, drop, plain, masked, keep)
    tidx = _token_index(hip_device, 1200, 6, seed=23)
    S = tidx.n_q
    q, k, v, dout = _acts(hip_device, S, S, 8, 16, dtype, seed=24)
    plain, masked, keep = _both(tidx, q, k, v, dout, drop)
    _check(tidx, 8, drop, plain, masked, keep)


def test_mask_with_bias_and_dbias(hip_device):
    """With a bias the forward still stores the bits (its general instance) and the backward, which takes
    its general instance for the bias and dbias, draws them: the same results as without the mask."""
    from budgetformer_amd.hip_ops import Dropout
    idx = _coo_index(hip_device, 500, 500, 6000, seed=31)
    q, k, v, dout = _acts(hip_device, 500, 500, 8, 16, torch.bfloat16, seed=32)
    bias = torch.randn(idx.nnz, 8, generator=torch.Generator().manual_seed(33)).to(hip_device) * 0.5
    drop = Dropout(0.5, 1234, 9)
    plain, masked, keep = _both(idx, q, k, v, dout, drop, bias=bias, need_dbias=True)
    _check(idx, 8, drop, plain, masked, keep)


def test_module_keeps_the_mask_between_forward_and_backward(hip_device):
    """The autograd function asks the forward for the mask under a dropout without bias and hands it to
    the backward: gradients equal the raw calls without a mask."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.attention import sparse_edge_attention
    from budgetformer_amd.hip_ops import Dropout
    idx = _coo_index(hip_device, 400, 400, 5000, seed=41)
    q, k, v, dout = _acts(hip_device, 400, 400, 8, 16, torch.bfloat16, seed=42)
    drop = Dropout(0.5, 555, 1)
    qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = sparse_edge_attention(qd, kd, vd, idx, None, None, drop)
    out.backward(dout)
    out0, Z0 = hip_ops.attn_forward(idx, q, k, v, dropout=drop)
    dq, dk, dv, _ = hip_ops.attn_backward(idx, q, k, v, None, Z0, dout, dropout=drop)
    torch.cuda.synchronize()
    for name, a, b in (("out", out, out0), ("dq", qd.grad, dq), ("dk", kd.grad, dk), ("dv", vd.grad, dv)):
        assert torch.equal(a, b), name


def test_mask_through_the_c_abi_and_the_allocation_free_backward(hip_device):
    """bf_attn_dropout.keep through ctypes: bf_attn_fwd stores the mask, bf_attn_bwd_noalloc reads it, and
    its gradients equal bf_attn_bwd's without a mask."""
    from budgetformer_amd import _native as N
    from budgetformer_amd import hip_ops
    from budgetformer_amd.hip_ops import Dropout
    idx = _coo_index(hip_device, 500, 500, 6000, seed=51)
    H, hn = 8, 16
    q, k, v, dout = _acts(hip_device, 500, 500, H, hn, torch.bfloat16, seed=52)
    drop = Dropout(0.5, 4321, 2)
    p = lambda t: C.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    st = C.c_void_p(torch.cuda.current_stream(hip_device).cuda_stream)
    keep = torch.full((idx.nnz, 1), 0xAA, dtype=torch.uint8, device=hip_device)
    sf = idx.struct(backward=False)
    out = torch.empty_like(q)
    Z = torch.empty(q.shape[0], H, dtype=torch.float32, device=hip_device)
    parts = torch.empty(max(int(N.load().bf_attn_partials_floats(C.byref(sf), H, hn)), 1), device=hip_device)
    d = drop.struct(keep)
    N.call("bf_attn_fwd", C.byref(sf), N.BF_DTYPE_BF16, H, hn, 5.0, p(q), p(k), p(v), None, None, C.byref(d),
           p(out), p(Z), p(parts), st)
    sb = idx.struct(backward=True, entries=True)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    N.call("bf_attn_bwd_noalloc", C.byref(sb), N.BF_DTYPE_BF16, H, hn, 5.0, p(q), p(k), p(v), None, None,
           C.byref(d), p(Z), p(dout), p(dq), p(dk), p(dv), None, st)
    out0, Z0 = hip_ops.attn_forward(idx, q, k, v, dropout=drop)
    r = hip_ops.attn_backward(idx, q, k, v, None, Z0, dout, dropout=drop)
    torch.cuda.synchronize()
    for name, a, b in (("out", out, out0), ("Z", Z, Z0), ("dq", dq, r[0]), ("dk", dk, r[1]), ("dv", dv, r[2])):
        assert torch.equal(a, b), name
    want = _pack(philox.dropout_keep_csr(idx.qptr.cpu().numpy(), H, drop.rate, drop.seed, drop.offset))
    assert np.array_equal(keep.cpu().numpy(), want)


def test_keep_tensor_checks(hip_device):
    """A keep tensor of the wrong shape or dtype is refused before any launch."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.hip_ops import Dropout
    idx = _coo_index(hip_device, 300, 300, 3000, seed=61)
    q, k, v, dout = _acts(hip_device, 300, 300, 8, 16, torch.float32, seed=62)
    drop = Dropout(0.5, 1, 0)
    out, Z, keep = hip_ops.attn_forward(idx, q, k, v, dropout=drop, keep_mask=True)
    for bad in (keep[:10], keep.to(torch.int32), torch.zeros(keep.shape[0], 2, dtype=torch.uint8, device=hip_device)):
        with pytest.raises(ValueError):
            hip_ops.attn_backward(idx, q, k, v, None, Z, dout, dropout=drop, keep=bad)
    # no dropout: no mask
    out, Z, keep = hip_ops.attn_forward(idx, q, k, v, keep_mask=True)
    assert keep.numel() == 0
