"""The GraphGPS attention dropout drawn inside the kernels (models/graphgps_dist_node_level.py:166-176)
against the float64 oracle with the mask oracle.philox.dropout_keep draws: forward and both backward
passes see the same keep bit per entry (its query row and its slot in the row) and head, and kept V
messages are scaled by 1/(1-rate)."""
import numpy as np
import pytest
import torch

from oracle import philox
from oracle import sparse_attention as sa
from parity_helpers import assert_close

pytestmark = pytest.mark.gpu


def _run(dev, q, k, v, idx, dout, dropout):
    from budgetformer_amd.attention import sparse_edge_attention
    qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = sparse_edge_attention(qd, kd, vd, idx, None, None, dropout)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    return out, qd.grad, kd.grad, vd.grad


def _oracle(q, k, v, idx, dout, rate, seed, offset):
    H = q.shape[1]
    keep = torch.from_numpy(philox.dropout_keep_csr(idx.qptr.cpu().numpy(), H, rate, seed, offset))
    factor = keep.double() / (1.0 - rate)
    ei = torch.stack([idx.kv.cpu().long(), idx.entry_rows().cpu()])      # CSR order: entry e is column e
    q64, k64, v64, d64 = (t.double() for t in (q, k, v, dout))
    out, Z = sa.attention_forward_stats(k64, q64, v64, ei, None, factor)
    dq, dk, dv, _ = sa.attention_backward_closed_form(k64, q64, v64, ei, out, Z, d64, None, factor)
    return out, dq, dk, dv, keep


@pytest.mark.parametrize("dtype,rate", [(torch.float32, 0.5), (torch.bfloat16, 0.5), (torch.float32, 0.1)])
@pytest.mark.parametrize("chunk,item", [(128, 768), (6, 10)])
def test_dropout_coo_index(hip_device, dtype, rate, chunk, item):
    from budgetformer_amd.hip_ops import AttentionIndex, Dropout
    S, H, hn = 900, 8, 16
    g = torch.Generator().manual_seed(int(rate * 100) + chunk)
    q, k, v, dout = (torch.randn(S, H, hn, generator=g).to(dtype) for _ in range(4))
    ei = torch.stack([torch.randint(0, S, (9000,), generator=g), torch.randint(0, S, (9000,), generator=g)])
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=chunk, item=item)
    seed, offset = (7 << 40) | 123, 5
    got = _run(hip_device, q, k, v, idx, dout, Dropout(rate, seed, offset))
    ref = _oracle(q, k, v, idx, dout, rate, seed, offset)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for name, a, b in zip(("out", "dq", "dk", "dv"), got, ref[:4]):
        assert_close(name, a, b, tol)
    assert abs(ref[4].float().mean().item() - (1 - rate)) < 0.02


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dropout_table_index_with_token_column(hip_device, dtype):
    """A table index with the Graphormer token: key 0's entries are finished by the dq pass and summed
    from its records; their keep bits must be the same ones the oracle draws at their (row, slot 0)."""
    from budgetformer_amd.hip_ops import AttentionIndex, Dropout
    rng = np.random.default_rng(3)
    n, width, H, hn = 1200, 6, 8, 16
    row_len = rng.integers(0, width + 1, n).astype(np.int32)
    table = np.full((n, width), -1, dtype=np.int32)
    for r in range(n):
        table[r, :row_len[r]] = np.sort(rng.choice(n, row_len[r], replace=False))
    idx = AttentionIndex.from_table(torch.from_numpy(table).to(hip_device), torch.from_numpy(row_len).to(hip_device),
                                    global_token=True, chunk=16, item=24)
    assert idx.token_column
    S = idx.n_q
    g = torch.Generator().manual_seed(11)
    q, k, v, dout = (torch.randn(S, H, hn, generator=g).to(dtype) for _ in range(4))
    got = _run(hip_device, q, k, v, idx, dout, Dropout(0.5, 99, 0))
    ref = _oracle(q, k, v, idx, dout, 0.5, 99, 0)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for name, a, b in zip(("out", "dq", "dk", "dv"), got, ref[:4]):
        assert_close(name, a, b, tol)


def test_gps_module_training_dropout_is_drawn_in_the_kernels(hip_device):
    """GPSCoreAttention in training: the Philox key comes from torch's default generator, so the same
    torch seed gives the same output; forward and backward equal gps_sparse_attention with that mask."""
    from budgetformer_amd.attention import GPSCoreAttention
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 700, 8, 16
    g = torch.Generator().manual_seed(5)
    q, k, v, dout = (torch.randn(S, H, hn, generator=g) for _ in range(4))
    ei = torch.stack([torch.randint(0, S, (6000,), generator=g), torch.randint(0, S, (6000,), generator=g)])
    idx = AttentionIndex.from_coo(ei.to(hip_device), S)
    mod = GPSCoreAttention(H * hn, 0.5, H).train()
    outs = []
    for _ in range(2):
        torch.manual_seed(1234)
        qd, kd, vd = (t[None].to(hip_device).requires_grad_(True) for t in (q, k, v))
        out = mod._sparse(qd, kd, vd, idx, H, hn)
        out.backward(dout.reshape(1, S, H * hn).to(hip_device))
        outs.append((out.detach(), qd.grad, kd.grad, vd.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    torch.manual_seed(1234)
    seed = int(torch.randint(0, 2 ** 62, (1,), dtype=torch.int64).item())
    keep = torch.from_numpy(philox.dropout_keep_csr(idx.qptr.cpu().numpy(), H, 0.5, seed, 0))
    ei_o = torch.stack([idx.kv.cpu().long(), idx.entry_rows().cpu()])
    q64, k64, v64 = (t.double().requires_grad_(True) for t in (q, k, v))
    ref = sa.gps_sparse_attention(q64, k64, v64, ei_o, keep, 2.0)
    ref.backward(dout.double())
    out, dq, dk, dv = outs[0]
    assert_close("out", out.view(S, H, hn), ref, 1e-5)
    for name, a, b in (("dq", dq[0], q64.grad), ("dk", dk[0], k64.grad), ("dv", dv[0], v64.grad)):
        assert_close(name, a, b, 1e-5)
