"""The calibration kernels: the gather probe (bf_gather_probe) reads the rows it is given and writes nothing; the
row-stream probe (bf_row_stream_probe) reads its rows and zeroes exactly the rows it is given in its outputs."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nt", [0, 1])
def test_gather_probe_reads_rows_and_writes_nothing(hip_device, nt):
    """Three tables of 256-, 256- and 64-byte rows gathered by 100K ids, some carrying the type bit (masked
    off), with normal and non-temporal loads: the call succeeds, the sink stays zero (the tables hold
    zeros and ones, whose fold never matches the sink's constant) and the tables are unchanged."""
    from budgetformer_amd import _native as N
    from budgetformer_amd import hip_ops
    n_rows = 5000
    a = torch.ones(n_rows, 64, dtype=torch.float32, device=hip_device)
    b = torch.zeros(n_rows, 64, dtype=torch.float32, device=hip_device)
    c = torch.ones(n_rows, 16, dtype=torch.float32, device=hip_device)
    g = torch.Generator(device=hip_device).manual_seed(3)
    ids = torch.randint(0, n_rows, (100_000,), generator=g, device=hip_device, dtype=torch.int32)
    ids[::7] |= torch.tensor(-2 ** 31, dtype=torch.int32, device=hip_device)
    sink = torch.zeros(1, dtype=torch.int32, device=hip_device)
    st = hip_ops._stream(hip_device)
    N.call("bf_gather_probe", hip_ops._p(a), 256, hip_ops._p(b), 256, hip_ops._p(c), 64, hip_ops._p(ids),
           ids.numel(), 0x7FFFFFFF, nt, hip_ops._p(sink), st)
    N.call("bf_gather_probe", hip_ops._p(c), 64, None, 0, None, 0, hip_ops._p(ids), ids.numel(), 0x7FFFFFFF, nt,
           hip_ops._p(sink), st)
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    assert bool((a == 1).all()) and not b.any() and bool((c == 1).all())


@pytest.mark.parametrize("row_bytes,with_ids", [(64, True), (256, True), (1024, True), (512, False)])
def test_row_stream_probe_zeroes_exactly_its_rows(hip_device, row_bytes, with_ids):
    """Rows of 64 to 1024 bytes (lane groups of 4 to 64 lanes): with ids (a random subset in random order,
    some negative, which are skipped) every listed row of both outputs is zero and every other row keeps
    its value; without ids the first n_rows rows are zeroed. The read tables are unchanged and the sink
    stays zero."""
    from budgetformer_amd import _native as N
    from budgetformer_amd import hip_ops
    n_tab, cols = 3000, row_bytes // 4
    g = torch.Generator(device=hip_device).manual_seed(row_bytes)
    r0 = torch.ones(n_tab, cols, dtype=torch.float32, device=hip_device)
    r1 = torch.full((n_tab, cols), 2.0, device=hip_device)
    w0 = torch.full((n_tab, cols), 3.0, device=hip_device)
    w1 = torch.full((n_tab, cols), 4.0, device=hip_device)
    sink = torch.zeros(1, dtype=torch.int32, device=hip_device)
    zeroed = torch.zeros(n_tab, dtype=torch.bool, device=hip_device)
    if with_ids:
        ids = torch.randperm(n_tab, generator=g, device=hip_device)[:1700].to(torch.int32)
        ids[::9] = -5
        n_rows = ids.numel()
        zeroed[ids[ids >= 0].long()] = True
    else:
        ids, n_rows = None, 2100
        zeroed[:n_rows] = True
    N.call("bf_row_stream_probe", hip_ops._p(r0), hip_ops._p(r1), hip_ops._p(w0), hip_ops._p(w1), row_bytes,
           hip_ops._p(ids) if ids is not None else None, n_rows, int(with_ids), hip_ops._p(sink),
           hip_ops._stream(hip_device))
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    assert bool((r0 == 1).all()) and bool((r1 == 2).all())
    assert bool((w0[zeroed] == 0).all()) and bool((w1[zeroed] == 0).all())
    assert bool((w0[~zeroed] == 3).all()) and bool((w1[~zeroed] == 4).all())
