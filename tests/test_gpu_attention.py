"""GPU parity of the HIP sparse attention (forward and backward) against the CPU oracle.

Tolerances (the parity bar of this path): fp32 within 1e-5 relative, bf16 within 2e-2
relative, against a float64 evaluation of the oracle on the same (rounded) inputs, as
the larger of max|got - ref| / max|ref| per tensor and the same per row with each row's
scale floored at 0.1 x the tensor's (parity_helpers; the newer tests floor bf16 rows at
1e-3).
"""
import pytest
import torch

from oracle import sparse_attention as sa
from parity_helpers import rel_err, row_rel_err

pytestmark = pytest.mark.gpu


def _rel_err(got, ref):
    return max(rel_err(got, ref), row_rel_err(got, ref, floor=0.1))


def _inputs(S, H, hn, E, seed, dtype=torch.float32, mult=1.0, n_kv=None):
    g = torch.Generator().manual_seed(seed)
    n_kv = S if n_kv is None else n_kv
    q = (torch.randn(S, H, hn, generator=g) * mult).to(dtype)
    k = (torch.randn(n_kv, H, hn, generator=g) * mult).to(dtype)
    v = torch.randn(n_kv, H, hn, generator=g).to(dtype)
    ei = torch.stack([torch.randint(0, n_kv, (E,), generator=g), torch.randint(0, S, (E,), generator=g)])
    dout = torch.randn(S, H, hn, generator=g).to(dtype)
    return q, k, v, ei, dout


def _oracle(q, k, v, ei, dout, bias_e=None, factor_e=None):
    q64, k64, v64, d64 = (t.double() for t in (q, k, v, dout))
    b64 = None if bias_e is None else bias_e.double()
    f64 = None if factor_e is None else factor_e.double()
    out, Z = sa.attention_forward_stats(k64, q64, v64, ei, b64, f64)
    dq, dk, dv, db = sa.attention_backward_closed_form(k64, q64, v64, ei, out, Z, d64, b64, f64)
    return out, Z, dq, dk, dv, db


def _run(dev, q, k, v, idx, dout, bias_e=None, factor_e=None, dropout=None):
    from budgetformer_amd.attention import sparse_edge_attention
    qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    bd = None if bias_e is None else bias_e.to(dev).float().requires_grad_(True)
    fd = None if factor_e is None else factor_e.to(dev).float()
    out = sparse_edge_attention(qd, kd, vd, idx, bd, fd, dropout)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    return out, qd.grad, kd.grad, vd.grad, (bd.grad if bd is not None else None)


def _coo_order(idx):
    """Oracle edge list in the index's CSR order (so per-entry tensors line up)."""
    rows = idx.entry_rows().cpu()
    return torch.stack([idx.kv.cpu().long(), rows])


@pytest.mark.parametrize("S,H,hn,E", [(300, 8, 16, 3000), (2708, 8, 8, 10556 + 2708), (64, 4, 32, 50)])
def test_fp32_random_coo(hip_device, S, H, hn, E):
    from budgetformer_amd.hip_ops import AttentionIndex
    q, k, v, ei, dout = _inputs(S, H, hn, E, seed=S)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S)
    out, dq, dk, dv, _ = _run(hip_device, q, k, v, idx, dout)
    ro, rZ, rdq, rdk, rdv, _ = _oracle(q, k, v, ei, dout)
    for got, ref in ((out, ro), (dq, rdq), (dk, rdk), (dv, rdv)):
        assert _rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("token_column", [False, True])
@pytest.mark.parametrize("chunk,item", [(4, 4), (4, 37), (64, 512), (4, 2), (300, 64)])
def test_fp32_global_token_split_rows(hip_device, chunk, item, token_column):
    """Graphormer token: query 0 is dense over all kv and kv 0 feeds every query. With items of 2
    the token row and column exceed the per-row item cap and run as 160 balanced items. The COO
    has the token-column layout, so key 0's terms can also come from the dq pass (token_column).
    A chunk above 254 takes the key plan from the generic count/scan/rows pass instead of the
    row order's first slots."""
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 500, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 2500, seed=7, mult=1.3)
    ei = ei[:, (ei[0] > 0) & (ei[1] > 0)]
    ar = torch.arange(1, S)
    ei = torch.cat([ei, torch.stack([ar, torch.zeros_like(ar)]), torch.stack([torch.zeros_like(ar), ar])], 1)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=chunk, item=item)
    idx.token_column = token_column
    out, dq, dk, dv, _ = _run(hip_device, q, k, v, idx, dout)
    ro, rZ, rdq, rdk, rdv, _ = _oracle(q, k, v, ei, dout)
    idx.resolve()
    assert idx.qplan.items > 0 and idx.kplan.items > 0 and idx.qplan.heavy > 0   # split paths exercised
    for got, ref in ((out, ro), (dq, rdq), (dk, rdk), (dv, rdv)):
        assert _rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("token_column", [False, True])
@pytest.mark.parametrize("chunk,item", [(4, 37), (8, 16)])
def test_bf16_split_rows_single_and_multi_item(hip_device, chunk, item, token_column):
    """Split rows with one item (finished by that item) and with several (summed by the reduce), bf16."""
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 600, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 6000, seed=17, dtype=torch.bfloat16)
    ei = ei[:, (ei[0] > 0) & (ei[1] > 0)]
    ar = torch.arange(1, S)
    ei = torch.cat([ei, torch.stack([ar, torch.zeros_like(ar)]), torch.stack([torch.zeros_like(ar), ar])], 1)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=chunk, item=item)
    idx.token_column = token_column
    idx.ensure_backward().resolve()
    for plan in (idx.qplan, idx.kplan):
        n = plan.nitems.cpu()
        heavy = plan.heavy_rows[: plan.heavy].cpu().long()
        assert (n[heavy] == 1).any() and (n[heavy] > 1).any()
    out, dq, dk, dv, _ = _run(hip_device, q, k, v, idx, dout)
    ro, rZ, rdq, rdk, rdv, _ = _oracle(q, k, v, ei, dout)
    for got, ref in ((out, ro), (dq, rdq), (dk, rdk), (dv, rdv)):
        assert _rel_err(got, ref) < 2e-2


def test_fp32_bias_and_dbias(hip_device):
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 200, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 1500, seed=11, mult=1.5)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=6, item=10)
    ei_o = _coo_order(idx)
    bias_e = torch.randn(idx.nnz, H, generator=torch.Generator().manual_seed(3))
    out, dq, dk, dv, db = _run(hip_device, q, k, v, idx, dout, bias_e=bias_e)
    ro, rZ, rdq, rdk, rdv, rdb = _oracle(q, k, v, ei_o, dout, bias_e=bias_e)
    for got, ref in ((out, ro), (dq, rdq), (dk, rdk), (dv, rdv), (db, rdb)):
        assert _rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("token", [False, True])
def test_table_index_plain_then_bias_backward(hip_device, token):
    """An index built from a table keeps its reverse entries' CSR positions lazy: a plain backward
    runs without them, a later backward with a bias and a factor derives them from the sorted keys."""
    import numpy as np
    from budgetformer_amd.hip_ops import AttentionIndex
    rng = np.random.default_rng(21 + token)
    n, width, H, hn = 400, 6, 8, 16
    row_len = rng.integers(0, width + 1, n).astype(np.int32)
    table = np.full((n, width), -1, dtype=np.int32)
    for r in range(n):
        table[r, :row_len[r]] = np.sort(rng.choice(n, row_len[r], replace=False))
    idx = AttentionIndex.from_table(torch.from_numpy(table).to(hip_device), torch.from_numpy(row_len).to(hip_device),
                                    global_token=token, chunk=5, item=7)
    S = idx.n_q
    q, k, v, _, dout = _inputs(S, H, hn, 1, seed=31, mult=1.4)
    ei_o = _coo_order(idx)
    out, dq, dk, dv, _ = _run(hip_device, q, k, v, idx, dout)
    assert idx.ks is None                       # not derived for a plain backward
    ro, rZ, rdq, rdk, rdv, _ = _oracle(q, k, v, ei_o, dout)
    for got, ref in ((out, ro), (dq, rdq), (dk, rdk), (dv, rdv)):
        assert _rel_err(got, ref) < 1e-5
    g = torch.Generator().manual_seed(5)
    bias_e = torch.randn(idx.nnz, H, generator=g)
    factor = (torch.rand(idx.nnz, H, generator=g) >= 0.3).float() / 0.7
    out, dq, dk, dv, db = _run(hip_device, q, k, v, idx, dout, bias_e=bias_e, factor_e=factor)
    assert idx.ks is not None
    ro, rZ, rdq, rdk, rdv, rdb = _oracle(q, k, v, ei_o, dout, bias_e=bias_e, factor_e=factor)
    for got, ref in ((out, ro), (dq, rdq), (dk, rdk), (dv, rdv), (db, rdb)):
        assert _rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("dtype,chunk,item,n,rate", [(torch.float32, 128, 768, 3000, 0.0),
                                                      (torch.float32, 5, 7, 400, 0.0),
                                                      (torch.bfloat16, 16, 24, 1500, 0.0),
                                                      (torch.float32, 128, 768, 60, 0.0),
                                                      (torch.bfloat16, 16, 24, 1500, 0.5),
                                                      (torch.float32, 5, 7, 400, 0.3)])
def test_token_column_terms_summed_by_the_dq_pass(hip_device, dtype, chunk, item, n, rate):
    """With a token column (key 0 first in every row t >= 1, as the table fill lays it out) the dq pass
    sums key 0's dK/dV terms per workgroup and the dk/dv pass reduces those records instead of gathering
    each query's q, dO and row stats again; and the token row (query 0, attending kv 1..n in order) opens
    every other key row's reverse entries, whose dk/dv terms then take query 0's q, dO and row stats from
    the workgroup's LDS copy instead of gathering them per key row. Against the gathering pass on the
    same index (no token promise): out, dq, dbias and every other key row equal bit for bit (the same
    arithmetic), key 0 within the parity bar (another summation order); both against the oracle.
    (chunk, item) = (5, 7) also splits the query rows, so key 0 opens item 0 of a split row; n = 60
    leaves the token column shorter than `chunk`, one group then sums every record. A third run leaves
    the split plans' counts on the device. rate > 0: the in-kernel dropout (keyed by query row and slot)."""
    import numpy as np
    from budgetformer_amd.hip_ops import AttentionIndex, Dropout
    from oracle import philox
    rng = np.random.default_rng(n + chunk)
    width, H, hn = 6, 8, 16
    row_len = rng.integers(0, width + 1, n).astype(np.int32)
    table = np.full((n, width), -1, dtype=np.int32)
    for r in range(n):
        table[r, :row_len[r]] = np.sort(rng.choice(n, row_len[r], replace=False))
    tab_d, len_d = torch.from_numpy(table).to(hip_device), torch.from_numpy(row_len).to(hip_device)
    runs = []
    for token_column, on_device in ((True, False), (False, False), (True, True)):
        idx = AttentionIndex.from_table(tab_d, len_d, global_token=True, chunk=chunk, item=item)
        assert idx.token_column
        idx.token_column, idx.device_counts = token_column, on_device
        S = idx.n_q
        q, k, v, _, dout = _inputs(S, H, hn, 1, seed=n, dtype=dtype, mult=1.3)
        g = torch.Generator().manual_seed(9)
        bias_e = torch.randn(idx.nnz, H, generator=g) if dtype == torch.float32 else None
        factor = ((torch.rand(idx.nnz, H, generator=g) >= 0.25).float() / 0.75) if dtype == torch.float32 else None
        drop = Dropout(rate, 4242, 3) if rate else None
        runs.append(_run(hip_device, q, k, v, idx, dout, bias_e=bias_e, factor_e=factor, dropout=drop))
    (out_f, dq_f, dk_f, dv_f, db_f), (out_g, dq_g, dk_g, dv_g, db_g), on_dev = runs
    # the key plan's counts left on the device (the query plan's known from the sizes): the same result
    for a, b in zip(runs[0], on_dev):
        assert (a is None and b is None) or torch.equal(a, b)
    if width + 1 <= chunk:        # the query plan's counts came from the sizes: they equal the device's
        assert idx._q_known is not None
        assert (idx.qplan.items, idx.qplan.heavy) == tuple(idx._counts[:2].tolist())
    assert torch.equal(out_f, out_g) and torch.equal(dq_f, dq_g)
    assert (db_f is None and db_g is None) or torch.equal(db_f, db_g)
    assert torch.equal(dk_f[1:], dk_g[1:]) and torch.equal(dv_f[1:], dv_g[1:])
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert _rel_err(dk_f[0], dk_g[0]) < tol and _rel_err(dv_f[0], dv_g[0]) < tol
    ei_o = _coo_order(idx)
    f_all = factor
    if rate:
        keep = torch.from_numpy(philox.dropout_keep_csr(idx.qptr.cpu().numpy(), H, rate, 4242, 3)).float()
        f_all = (keep if factor is None else factor * keep) / (1.0 - rate)
    ro, rZ, rdq, rdk, rdv, rdb = _oracle(q, k, v, ei_o, dout, bias_e=bias_e, factor_e=f_all)
    for got, ref in ((out_f, ro), (dq_f, rdq), (dk_f, rdk), (dv_f, rdv)):
        assert _rel_err(got, ref) < tol
    if db_f is not None:
        assert _rel_err(db_f, rdb) < tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_device_plan_counts_equal_host_plan_counts(hip_device, dtype):
    """With the plans' counts left on the device the grids are sized for the capacities and the kernels
    read the counts themselves; the result is the same bit for bit as with host counts (split rows on
    both sides, the token column, a bias and a factor)."""
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 700, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 5000, seed=23, dtype=dtype, mult=1.2)
    ei = ei[:, (ei[0] > 0) & (ei[1] > 0)]
    ar = torch.arange(1, S)
    ei = torch.cat([ei, torch.stack([ar, torch.zeros_like(ar)]), torch.stack([torch.zeros_like(ar), ar])], 1)
    runs = []
    for on_device in (True, False):
        idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=6, item=9)
        idx.token_column, idx.device_counts = True, on_device
        g = torch.Generator().manual_seed(2)
        bias_e = torch.randn(idx.nnz, H, generator=g) if dtype == torch.float32 else None
        factor = (torch.rand(idx.nnz, H, generator=g) >= 0.3).float() / 0.7 if dtype == torch.float32 else None
        runs.append(_run(hip_device, q, k, v, idx, dout, bias_e=bias_e, factor_e=factor))
        assert idx.qplan.pending == on_device and idx.kplan.pending == on_device
        idx.resolve()
        assert idx.qplan.items > 0 and idx.kplan.items > 0 and idx.qplan.heavy > 0 and idx.kplan.heavy > 0
    for a, b in zip(*runs):
        assert (a is None and b is None) or torch.equal(a, b)


def test_fp32_gps_dropout_factor(hip_device):
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 200, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 1500, seed=12)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S)
    ei_o = _coo_order(idx)
    keep = torch.rand(idx.nnz, H, generator=torch.Generator().manual_seed(4)) >= 0.5
    factor = keep.float() * 2.0
    out, dq, dk, dv, _ = _run(hip_device, q, k, v, idx, dout, factor_e=factor)
    ro, rZ, rdq, rdk, rdv, _ = _oracle(q, k, v, ei_o, dout, factor_e=factor)
    for got, ref in ((out, ro), (dq, rdq), (dk, rdk), (dv, rdv)):
        assert _rel_err(got, ref) < 1e-5
    # GPS module form == mask form of the oracle restatement
    ref = sa.gps_sparse_attention(q.double(), k.double(), v.double(), ei_o, keep, 2.0)
    assert _rel_err(out, ref) < 1e-5


def test_bf16_within_2e2(hip_device):
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 400, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 4000, seed=13, dtype=torch.bfloat16)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S)
    out, dq, dk, dv, _ = _run(hip_device, q, k, v, idx, dout)
    assert out.dtype == torch.bfloat16 and dk.dtype == torch.bfloat16
    ro, rZ, rdq, rdk, rdv, _ = _oracle(q, k, v, ei, dout)
    for got, ref in ((out, ro), (dq, rdq), (dk, rdk), (dv, rdv)):
        assert _rel_err(got, ref) < 2e-2


@pytest.mark.parametrize("dtype,H,hn", [(torch.bfloat16, 2, 8), (torch.bfloat16, 1, 8), (torch.bfloat16, 1, 16),
                                        (torch.bfloat16, 4, 8), (torch.float32, 1, 4), (torch.float32, 2, 4)])
@pytest.mark.parametrize("chunk,item", [(128, 768), (6, 10)])
def test_narrow_rows(hip_device, dtype, H, hn, chunk, item):
    """Rows of 8 to 32 elements: lane groups of 1, 2 or 4 lanes, narrower than the edges an iteration
    takes, so the entry ids are loaded per iteration instead of shuffled out of a chunk. Forward and
    both backward passes against the oracle, with and without split rows."""
    from budgetformer_amd.hip_ops import AttentionIndex
    from parity_helpers import assert_close
    S = 700
    q, k, v, ei, dout = _inputs(S, H, hn, 7000, seed=H * 100 + hn + chunk, dtype=dtype)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=chunk, item=item)
    out, dq, dk, dv, _ = _run(hip_device, q, k, v, idx, dout)
    ro, rZ, rdq, rdk, rdv, _ = _oracle(q, k, v, ei, dout)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for name, got, ref in (("out", out, ro), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        assert_close(name, got, ref, tol)


@pytest.mark.parametrize("dtype,H,hn", [(torch.float32, 8, 32), (torch.float32, 2, 128), (torch.float32, 16, 16),
                                        (torch.bfloat16, 8, 64), (torch.bfloat16, 4, 128), (torch.bfloat16, 32, 16),
                                        (torch.float16, 8, 64)])
@pytest.mark.parametrize("extra", ["plain", "token", "dropout"])
def test_widest_rows(hip_device, dtype, H, hn, extra):
    """Rows of 256 (float32) or 512 (bfloat16, float16) elements, the widest the kernels take: a lane
    group is a whole wavefront (64 lanes of 16 bytes), one group per wave, four per workgroup, and a
    head spans 4 to 32 lanes. Forward and both backward passes against the oracle, with split query and
    key rows (chunk 6, item 10). "token": the Graphormer token row and column (query 0 attends every key,
    every query attends key 0; the dq pass's key-0 records), with a bias and its gradient in float32.
    "dropout": the in-kernel dropout at rate 0.3 against the oracle's mask."""
    from budgetformer_amd.hip_ops import AttentionIndex, Dropout
    from oracle import philox
    from parity_helpers import assert_close
    S = 600
    q, k, v, ei, dout = _inputs(S, H, hn, 5000, seed=H * 1000 + hn, dtype=dtype, mult=1.1)
    if extra == "token":
        ei = ei[:, (ei[0] > 0) & (ei[1] > 0)]
        ar = torch.arange(1, S)
        ei = torch.cat([ei, torch.stack([ar, torch.zeros_like(ar)]), torch.stack([torch.zeros_like(ar), ar])], 1)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=6, item=10)
    idx.token_column = extra == "token"
    g = torch.Generator().manual_seed(5)
    bias_e = torch.randn(idx.nnz, H, generator=g) if (extra == "token" and dtype == torch.float32) else None
    rate, seed, off = 0.3, 91, 4
    drop = Dropout(rate, seed, off) if extra == "dropout" else None
    out, dq, dk, dv, db = _run(hip_device, q, k, v, idx, dout, bias_e=bias_e, dropout=drop)
    factor = None
    if drop is not None:
        factor = torch.from_numpy(philox.dropout_keep_csr(idx.qptr.cpu().numpy(), H, rate, seed, off)).float()
        factor = factor / (1.0 - rate)
    ro, rZ, rdq, rdk, rdv, rdb = _oracle(q, k, v, _coo_order(idx), dout, bias_e=bias_e, factor_e=factor)
    tol = 1e-5 if dtype == torch.float32 else (2e-2 if dtype == torch.bfloat16 else 5e-3)
    for name, got, ref in (("out", out, ro), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        assert_close(name, got, ref, tol)
    if bias_e is not None:
        assert_close("dbias", db, rdb, tol)
    assert idx.qplan.items > 0 and idx.kplan.items > 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_row_past_the_long_row_threshold(hip_device, dtype):
    """A token row and column longer than BF_MAX_ITEMS_PER_ROW * BF_LONG_ROW_FACTOR items' worth of
    entries (60K entries at item = 2: 469 items each, past the 160-item cap, several rounds of every
    reduce) through the forward reduce, the dq reduce and the key-side reduce; the item counts follow
    bf_split_row_items."""
    from budgetformer_amd import _native as N
    from budgetformer_amd.hip_ops import AttentionIndex, split_row_items
    from parity_helpers import assert_close
    S, H, hn, item = 60_000, 8, 16, 2
    q, k, v, ei, dout = _inputs(S, H, hn, 40_000, seed=41, dtype=dtype)
    ei = ei[:, (ei[0] > 0) & (ei[1] > 0)]
    ar = torch.arange(1, S)
    ei = torch.cat([ei, torch.stack([ar, torch.zeros_like(ar)]), torch.stack([torch.zeros_like(ar), ar])], 1)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=8, item=item)
    idx.ensure_backward().resolve()
    n0 = split_row_items(S - 1, item)
    assert n0 == -(-(S - 1) // (item * N.BF_LONG_ROW_FACTOR)) and n0 > N.BF_MAX_ITEMS_PER_ROW
    assert int(idx.qplan.nitems[0].item()) == n0 and int(idx.kplan.nitems[0].item()) == n0
    out, dq, dk, dv, _ = _run(hip_device, q, k, v, idx, dout)
    ro, rZ, rdq, rdk, rdv, _ = _oracle(q, k, v, ei, dout)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for name, got, ref in (("out", out, ro), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        assert_close(name, got, ref, tol)


def test_empty_rows_and_empty_edge_set(hip_device):
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 50, 8, 16
    q, k, v, _, dout = _inputs(S, H, hn, 1, seed=14)
    ei = torch.tensor([[3, 4, 4], [1, 1, 7]])             # duplicate edge (4 -> 1) counts twice
    idx = AttentionIndex.from_coo(ei.to(hip_device), S)
    out, dq, dk, dv, _ = _run(hip_device, q, k, v, idx, dout)
    ro, rZ, rdq, rdk, rdv, _ = _oracle(q, k, v, ei, dout)
    for got, ref in ((out, ro), (dq, rdq), (dk, rdk), (dv, rdv)):
        assert _rel_err(got, ref) < 1e-5
    assert out[0].abs().max().item() == 0 and dk[0].abs().max().item() == 0
    idx0 = AttentionIndex.from_coo(torch.zeros(2, 0, dtype=torch.long, device=hip_device), S)
    out0, dq0, dk0, dv0, _ = _run(hip_device, q, k, v, idx0, dout)
    assert out0.abs().max().item() == 0 and dq0.abs().max().item() == 0 and dv0.abs().max().item() == 0


def test_deterministic(hip_device):
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 300, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 6000, seed=15)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S, chunk=8, item=24)
    a = _run(hip_device, q, k, v, idx, dout)
    b = _run(hip_device, q, k, v, idx, dout)
    for x, y in zip(a[:4], b[:4]):
        assert torch.equal(x, y)


def test_core_attention_modules_match_reference_forms(hip_device):
    from budgetformer_amd.attention import CoreAttention, GTCoreAttention
    S, H, hn = 120, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 900, seed=16)
    bias = torch.randn(1, S, S, H, generator=torch.Generator().manual_seed(5))
    core = CoreAttention(H * hn, 0.0, H, 1)
    got = core(q[None].to(hip_device), k[None].to(hip_device), v[None].to(hip_device), bias.to(hip_device),
               ei.to(hip_device), attn_type="sparse")
    ref = sa.graphormer_sparse_attention(k.double(), q.double(), v.double(), ei, bias[0].double())
    assert got.shape == (1, S, H * hn)
    assert _rel_err(got.view(S, H, hn), ref) < 1e-5
    gt = GTCoreAttention(H * hn, 0.0, H)
    got = gt(q[None].to(hip_device), k[None].to(hip_device), v[None].to(hip_device), None, ei.to(hip_device))
    ref = sa.gt_sparse_attention(q.double(), k.double(), v.double(), ei)
    assert _rel_err(got.view(S, H, hn), ref) < 1e-5
    with pytest.raises(ValueError):
        gt(q[None].to(hip_device), k[None].to(hip_device), v[None].to(hip_device), None, ei.to(hip_device), "full")


def test_unsupported_head_dim_raises(hip_device):
    from budgetformer_amd.hip_ops import AttentionIndex
    q, k, v, ei, dout = _inputs(10, 2, 6, 20, seed=17)
    idx = AttentionIndex.from_coo(ei.to(hip_device), 10)
    with pytest.raises(NotImplementedError):
        _run(hip_device, q, k, v, idx, dout)


def test_exphormer_typed_edges_match_oracle(hip_device):
    from budgetformer_amd.attention import ExphormerCoreAttention
    S, H, hn = 150, 8, 16
    q, k, v, ei, dout = _inputs(S, H, hn, 1200, seed=31)
    types = torch.randint(0, 2, (ei.size(1),), generator=torch.Generator().manual_seed(3))
    ei3 = torch.cat([ei, types[None]])
    mod = ExphormerCoreAttention(H * hn, 0.0, H).to(hip_device)
    qd, kd, vd = (t[None].to(hip_device).requires_grad_(True) for t in (q, k, v))
    out = mod(qd, kd, vd, None, ei3.to(hip_device))
    out.backward(dout[None].to(hip_device).reshape(1, S, H * hn))
    # oracle in float64 with the module's own edge encoder
    E = mod.edge_modulation(hip_device).detach().double().cpu()
    q64, k64, v64 = (t.double().requires_grad_(True) for t in (q, k, v))
    ref = sa.exphormer_sparse_attention(q64, k64, v64, ei3, E)
    ref.backward(dout.double())
    assert _rel_err(out.view(S, H, hn), ref) < 1e-5
    for got, r in ((qd.grad[0], q64.grad), (kd.grad[0], k64.grad), (vd.grad[0], v64.grad)):
        assert _rel_err(got, r) < 1e-5
    assert mod.edge_proj.weight.grad is not None and mod.edge_type_emb.weight.grad is not None


@pytest.mark.parametrize("dtype,H,tol", [(torch.float32, 8, 1e-5), (torch.bfloat16, 16, 2e-2)])
def test_streaming_kv_pass_on_a_table_larger_than_the_cache(hip_device, dtype, H, tol):
    """q and dO tables above 256 MB take the non-temporal gathers of the dk/dv pass; same results."""
    from budgetformer_amd.hip_ops import AttentionIndex
    hn, S = 16, 300_000                                           # 2 * S * H*hn * s = 307 MB > 256 MB
    q, k, v, ei, dout = _inputs(S, H, hn, S, seed=23, dtype=dtype)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S)
    out, dq, dk, dv, _ = _run(hip_device, q, k, v, idx, dout)
    ro, rZ, rdq, rdk, rdv, _ = _oracle(q, k, v, ei, dout)
    for got, ref in ((out, ro), (dq, rdq), (dk, rdk), (dv, rdv)):
        assert _rel_err(got, ref) < tol


@pytest.mark.parametrize("n_big", [2_000_000, 17_000_000])
def test_kv_pass_with_four_rows_per_group_equals_the_compact_problem(hip_device, n_big):
    """Past 1M kv rows in bf16 (16M in fp32) the dk/dv pass gives each lane group four short rows. Every
    row is still computed alone, so the gradients of a 2M- or 17M-row problem with 30K attended rows
    must equal, bit for bit, those of the same edges over the 30K rows alone (one row per group), and
    every other row must be zero."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.hip_ops import AttentionIndex
    g = torch.Generator(device=hip_device).manual_seed(3)
    n_q, n_touch, E, H, hn = 20000, 30000, 200000, 8, 16
    touched = torch.randperm(n_big, generator=g, device=hip_device)[:n_touch].sort().values
    src_c = torch.randint(0, n_touch, (E,), generator=g, device=hip_device)
    dst = torch.randint(0, n_q, (E,), generator=g, device=hip_device)
    big = AttentionIndex.from_coo(torch.stack([touched[src_c], dst]), n_q, n_big)
    small = AttentionIndex.from_coo(torch.stack([src_c, dst]), n_q, n_touch)
    q = torch.randn(n_q, H, hn, generator=g, device=hip_device).to(torch.bfloat16)
    dout = torch.randn(n_q, H, hn, generator=g, device=hip_device).to(torch.bfloat16)
    k = torch.empty(n_big, H, hn, device=hip_device, dtype=torch.bfloat16).normal_(generator=g)
    v = torch.empty(n_big, H, hn, device=hip_device, dtype=torch.bfloat16).normal_(generator=g)
    kc, vc = k[touched].contiguous(), v[touched].contiguous()
    out_b, z_b = hip_ops.attn_forward(big, q, k, v)
    out_s, z_s = hip_ops.attn_forward(small, q, kc, vc)
    assert torch.equal(out_b, out_s) and torch.equal(z_b, z_s)
    dq_b, dk_b, dv_b, _ = hip_ops.attn_backward(big, q, k, v, out_b, z_b, dout)
    dq_s, dk_s, dv_s, _ = hip_ops.attn_backward(small, q, kc, vc, out_s, z_s, dout)
    assert torch.equal(dq_b, dq_s)
    assert torch.equal(dk_b[touched], dk_s) and torch.equal(dv_b[touched], dv_s)
    dk_b[touched] = 0
    dv_b[touched] = 0
    assert not dk_b.any() and not dv_b.any()


def test_query_passes_past_16m_rows_equal_the_compact_problem(hip_device):
    """A 17M-query problem with 30K attending queries equals its compaction bit for bit (forward and
    both backward passes), and the other queries get zero outputs and gradients."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.hip_ops import AttentionIndex
    g = torch.Generator(device=hip_device).manual_seed(4)
    n_big, n_touch, n_kv, E, H, hn = 17_000_000, 30000, 20000, 200000, 8, 16
    touched = torch.randperm(n_big, generator=g, device=hip_device)[:n_touch].sort().values
    dst_c = torch.randint(0, n_touch, (E,), generator=g, device=hip_device)
    src = torch.randint(0, n_kv, (E,), generator=g, device=hip_device)
    big = AttentionIndex.from_coo(torch.stack([src, touched[dst_c]]), n_big, n_kv)
    small = AttentionIndex.from_coo(torch.stack([src, dst_c]), n_touch, n_kv)
    q = torch.empty(n_big, H, hn, device=hip_device, dtype=torch.bfloat16).normal_(generator=g)
    dout = torch.empty(n_big, H, hn, device=hip_device, dtype=torch.bfloat16).normal_(generator=g)
    k = torch.randn(n_kv, H, hn, generator=g, device=hip_device).to(torch.bfloat16)
    v = torch.randn(n_kv, H, hn, generator=g, device=hip_device).to(torch.bfloat16)
    qc, doc = q[touched].contiguous(), dout[touched].contiguous()
    out_b, z_b = hip_ops.attn_forward(big, q, k, v)
    out_s, z_s = hip_ops.attn_forward(small, qc, k, v)
    assert torch.equal(out_b[touched], out_s) and torch.equal(z_b[touched], z_s)
    dq_b, dk_b, dv_b, _ = hip_ops.attn_backward(big, q, k, v, out_b, z_b, dout)
    dq_s, dk_s, dv_s, _ = hip_ops.attn_backward(small, qc, k, v, out_s, z_s, doc)
    assert torch.equal(dq_b[touched], dq_s) and torch.equal(dk_b, dk_s) and torch.equal(dv_b, dv_s)
    for t in (out_b, z_b, dq_b):
        t[touched] = 0
        assert not t.any()
