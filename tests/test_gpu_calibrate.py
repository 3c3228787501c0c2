"""The gather-rate calibration kernel (bf_gather_probe): it reads the rows it is given and writes nothing."""
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
