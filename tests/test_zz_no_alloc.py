"""bf_attn_bwd_noalloc: the backward with its scratch (row stats, split partials) in a static
device array, for callers that cannot allocate. Called through the C ABI and checked against
bf_attn_bwd on the same inputs: two calls in a row, the second on a smaller problem (the array
then holds the first call's contents), plus the size limit, which is rejected before any launch.
"""
import ctypes as C

import pytest
import torch

pytestmark = pytest.mark.gpu


def _problem(dev, S, E, H, hn, dtype, seed, chunk, item):
    """Random edges plus the Graphormer token layout (query 0 dense, key 0 first in every other row),
    so split rows on both sides and the token column are exercised."""
    from budgetformer_amd.hip_ops import AttentionIndex
    g = torch.Generator().manual_seed(seed)
    ei = torch.stack([torch.randint(1, S, (E,), generator=g), torch.randint(1, S, (E,), generator=g)])
    ar = torch.arange(1, S)
    ei = torch.cat([torch.stack([torch.zeros_like(ar), ar]), ei, torch.stack([ar, torch.zeros_like(ar)])], 1)
    idx = AttentionIndex.from_coo(ei.to(dev), S, chunk=chunk, item=item)
    idx.token_column = 1
    q, k, v, dout = (torch.randn(S, H, hn, generator=g).to(dtype).to(dev) for _ in range(4))
    return idx, q, k, v, dout


def _noalloc(idx, q, k, v, Z, dout, bias=None, need_dbias=False):
    from budgetformer_amd import _native as N
    from budgetformer_amd import hip_ops
    H, hn = q.shape[1], q.shape[2]
    st = idx.struct(backward=True, entries=bias is not None or need_dbias)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dbias = torch.empty(idx.nnz, H, dtype=torch.float32, device=q.device) if need_dbias else None
    p = hip_ops._p
    N.call("bf_attn_bwd_noalloc", C.byref(st), hip_ops._DT[q.dtype], H, hn, 5.0, p(q), p(k), p(v), p(bias), None,
           None, p(Z), p(dout), p(dq), p(dk), p(dv), p(dbias), hip_ops._stream(q.device))
    return dq, dk, dv, dbias


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_noalloc_equals_bf_attn_bwd_on_two_calls_the_second_smaller(hip_device, dtype):
    from budgetformer_amd import hip_ops
    H, hn = 8, 16
    for S, E, chunk, item in ((3000, 30000, 8, 16), (700, 4000, 6, 10)):
        idx, q, k, v, dout = _problem(hip_device, S, E, H, hn, dtype, S, chunk, item)
        out, Z = hip_ops.attn_forward(idx, q, k, v)
        ref = hip_ops.attn_backward(idx, q, k, v, out, Z, dout)
        got = _noalloc(idx, q, k, v, Z, dout)
        torch.cuda.synchronize()
        idx.resolve()
        assert idx.qplan.items > 0 and idx.kplan.items > 0     # split rows on both sides
        for a, b in zip(got[:3], ref[:3]):
            assert torch.equal(a, b)


def test_noalloc_with_bias_and_dbias(hip_device):
    from budgetformer_amd import hip_ops
    H, hn = 8, 16
    idx, q, k, v, dout = _problem(hip_device, 900, 6000, H, hn, torch.float32, 5, 6, 9)
    bias = torch.randn(idx.nnz, H, generator=torch.Generator().manual_seed(1)).to(hip_device)
    out, Z = hip_ops.attn_forward(idx, q, k, v, bias)
    ref = hip_ops.attn_backward(idx, q, k, v, out, Z, dout, bias, need_dbias=True)
    got = _noalloc(idx, q, k, v, Z, dout, bias=bias, need_dbias=True)
    torch.cuda.synchronize()
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_noalloc_rejects_an_index_beyond_the_scratch(hip_device):
    """1.1M queries x 8 heads of row stats (70 MB) exceed the 64 MiB array: a ValueError, nothing launched."""
    from budgetformer_amd.hip_ops import AttentionIndex
    n = 1_100_000
    idx = AttentionIndex.from_coo(torch.zeros(2, 0, dtype=torch.int64, device=hip_device), n)
    q = torch.zeros(n, 8, 16, device=hip_device)
    Z = torch.zeros(n, 8, device=hip_device)
    with pytest.raises(ValueError, match="scratch"):
        _noalloc(idx, q, q, q, Z, q)
