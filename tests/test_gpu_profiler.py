"""The library's per-kernel timer (bf_prof_*, budgetformer_amd._native.KernelTimer), which the bench's
per-kernel table reads: while enabled every launch is timed on its stream by a HIP event pair and counted
under its kernel's name; disabled, nothing is recorded."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _layer(dev):
    from budgetformer_amd.attention import sparse_edge_attention
    from budgetformer_amd.hip_ops import AttentionIndex
    g = torch.Generator().manual_seed(4)
    S, H, hn, E = 500, 8, 16, 4000
    ei = torch.stack([torch.randint(0, S, (E,), generator=g), torch.randint(0, S, (E,), generator=g)])
    idx = AttentionIndex.from_coo(ei.to(dev), S)
    q, k, v = (torch.randn(S, H, hn, generator=g).to(dev).requires_grad_(True) for _ in range(3))
    out = sparse_edge_attention(q, k, v, idx)
    out.backward(torch.randn(S, H, hn, generator=g).to(dev))
    torch.cuda.synchronize()


def test_kernel_timer_counts_each_launch_by_name(hip_device):
    from budgetformer_amd._native import KernelTimer
    _layer(hip_device)                      # index, plans and caches built outside the timed calls
    with KernelTimer():
        for _ in range(3):
            _layer(hip_device)
    stats = KernelTimer.stats()
    for name in ("attn_fwd_kernel", "attn_bwd_q_kernel", "attn_bwd_kv_kernel"):
        ms, launches = stats[name]
        assert launches == 3 and 0.0 < ms < 1e3, (name, ms, launches)
    assert all(n >= 1 and ms >= 0.0 for ms, n in stats.values())
    # disabled: a further call adds nothing, and a reset clears what was collected
    _layer(hip_device)
    assert KernelTimer.stats() == stats
    from budgetformer_amd import _native as N
    N.call("bf_prof_reset")
    assert KernelTimer.stats() == {}
