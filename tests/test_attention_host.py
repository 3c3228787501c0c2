"""Host-side logic of the attention modules (CPU): how per-head edge lists are cut into calls, how a dense
bias of a batch is read per edge, and which attn_type each module accepts. No kernel runs here."""
import types

import pytest
import torch

from budgetformer_amd import attention as A
from oracle import sparse_attention as sa


def test_head_runs_group_consecutive_heads_of_one_set():
    a, b = torch.zeros(2, 3), torch.zeros(2, 3)
    assert A._head_runs([a, a, b, b, b, None, None, a]) == [(0, 2, a), (2, 5, b), (5, 7, None), (7, 8, a)]
    assert A._head_runs([a]) == [(0, 1, a)]
    assert A._head_runs([]) == []
    # equal contents in different tensors are different sets (identity, as the reference's list holds them)
    c = a.clone()
    assert [r[:2] for r in A._head_runs([a, c])] == [(0, 1), (1, 2)]


def test_empty_edge_sets():
    assert A._empty_edges(None)
    assert A._empty_edges(torch.zeros(2, 0, dtype=torch.long))
    assert not A._empty_edges(torch.zeros(2, 1, dtype=torch.long))


def _stub_index(src, dst):
    """What _dense_bias_to_edges reads of an AttentionIndex: kv ids and each entry's query row."""
    return types.SimpleNamespace(kv=torch.as_tensor(src, dtype=torch.int32), entry_rows=lambda: torch.as_tensor(dst))


@pytest.mark.parametrize("batch,n", [(1, 7), (3, 5)])
def test_dense_bias_per_edge_equals_the_reference_expansion(batch, n):
    H = 2
    g = torch.Generator().manual_seed(batch)
    bias = torch.randn(batch, n, n, H, generator=g)
    S = batch * n
    src = torch.randint(0, S, (40,), generator=g)
    dst = torch.randint(0, S, (40,), generator=g)
    got = A._dense_bias_to_edges(bias, _stub_index(src, dst), batch, n, H)
    full = sa.batched_dense_bias(bias, batch, n)          # the reference's unsqueeze/repeat/view
    assert torch.equal(got, full[src, dst, :])


def test_gps_takes_the_sparse_path_for_every_type_but_full_and_performer():
    mod = A.GPSCoreAttention(32, 0.0, 4)
    q = torch.zeros(1, 3, 4, 8)
    for t in ("full", "performer", "FULL"):
        with pytest.raises(NotImplementedError):
            mod(q, q, q, None, torch.zeros(2, 0, dtype=torch.long), t)
    # any other type reaches the sparse path, which refuses host tensors (no CPU fallback)
    with pytest.raises((RuntimeError, ValueError, NotImplementedError, TypeError)) as err:
        mod(q, q, q, None, torch.zeros(2, 0, dtype=torch.long), "flash")
    assert "attn_type" not in str(err.value)


def test_gt_rejects_an_empty_list_and_non_sparse_types():
    mod = A.GTCoreAttention(32, 0.0, 4)
    q = torch.zeros(1, 3, 4, 8)
    with pytest.raises(ValueError, match="empty list"):
        mod(q, q, q, None, [])
    with pytest.raises(ValueError, match="restricted"):
        mod(q, q, q, None, torch.zeros(2, 0, dtype=torch.long), "full")


def test_host_tensors_are_refused_before_any_library_call():
    """Every library call takes its stream from its tensors' device: host tensors raise there, before a
    host pointer could reach a kernel (and without touching the HIP runtime)."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.graph import chung_lu_device
    ei = torch.tensor([[0, 1], [1, 0]])
    with pytest.raises(ValueError, match="no CPU fallback"):
        hip_ops.coo_to_csr(ei, 2, 2)
    with pytest.raises(ValueError, match="no CPU fallback"):
        hip_ops.expand_rows(torch.tensor([0, 1, 2]), 2)
    with pytest.raises(ValueError, match="no CPU fallback"):
        chung_lu_device(100, 400, device="cpu")
