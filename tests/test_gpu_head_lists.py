"""GPU parity of the attention forms beyond one edge set at batch 1, against the CPU oracle:

- the score clamp bound of the kernels (bf_attn_fwd / bf_attn_bwd ``score_clamp``);
- Graphormer's per-head-group edge lists (models/graphormer_dist_node_level.py:175-213);
- Graphormer's dense bias of a batch (b > 1, :171-173);
- GT's per-head edge lists, which clamp q.k before the scaling (models/gt_dist_node_level.py:195-218),
  and its per-head score-mass statistics (:75-90, :218-220).

Forward and the gradients of q, k, v (and of the dense bias) are compared with a float64 evaluation of
the oracle (autograd of its list forms, which reduce to the pinned tensor path) at the path's bar:
1e-5 relative in fp32 and 2e-2 in bf16, per tensor and per row.
"""
import math

import pytest
import torch

from oracle import sparse_attention as sa
from parity_helpers import assert_close

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _acts(S, H, hn, seed, dtype, mult=1.0):
    g = torch.Generator().manual_seed(seed)
    q, k, v = ((torch.randn(S, H, hn, generator=g) * m).to(dtype) for m in (mult, mult, 1.0))
    dout = torch.randn(S, H, hn, generator=g).to(dtype)
    return q, k, v, dout


def _edges(S, E, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.stack([torch.randint(0, S, (E,), generator=g), torch.randint(0, S, (E,), generator=g)])


def _oracle_grads(fn, tensors, dout):
    """Forward and autograd gradients of the float64 oracle `fn(*tensors)`."""
    leaves = [t.detach().double().requires_grad_(True) for t in tensors]
    out = fn(*leaves)
    out.backward(dout.double())
    return out.detach(), [t.grad for t in leaves]


def _device_grads(fn, tensors, dout, dev):
    leaves = [t.to(dev).requires_grad_(True) for t in tensors]
    out = fn(*leaves)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    return out.detach(), [t.grad for t in leaves]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("clamp", [5.0, 1.25, 0.3])
def test_score_clamp_bound_against_the_closed_form(hip_device, dtype, clamp):
    from budgetformer_amd.attention import sparse_edge_attention
    from budgetformer_amd.hip_ops import AttentionIndex
    S, H, hn = 500, 8, 16
    q, k, v, dout = _acts(S, H, hn, 3, dtype)
    ei = _edges(S, 6000, 4)
    idx = AttentionIndex.from_coo(ei.to(hip_device), S)
    qd, kd, vd = (t.to(hip_device).requires_grad_(True) for t in (q, k, v))
    out = sparse_edge_attention(qd, kd, vd, idx, score_clamp=clamp)
    out.backward(dout.to(hip_device))
    ro, rZ = sa.attention_forward_stats(k.double(), q.double(), v.double(), ei, clamp=clamp)
    a_pre = (k.double()[ei[0]] * q.double()[ei[1]]).sum(-1) / math.sqrt(hn)
    assert (a_pre.abs() > clamp).float().mean() > 0.05 or clamp == 5.0     # the bound is reached
    rdq, rdk, rdv, _ = sa.attention_backward_closed_form(k.double(), q.double(), v.double(), ei, ro, rZ,
                                                         dout.double(), clamp=clamp)
    for name, got, ref in (("out", out, ro), ("dq", qd.grad, rdq), ("dk", kd.grad, rdk), ("dv", vd.grad, rdv)):
        assert_close(f"clamp {clamp} {name}", got, ref, TOL[dtype])


def test_score_clamp_outside_the_range_raises(hip_device):
    from budgetformer_amd.attention import sparse_edge_attention
    from budgetformer_amd.hip_ops import AttentionIndex
    q, k, v, _ = _acts(20, 2, 8, 5, torch.float32)
    idx = AttentionIndex.from_coo(_edges(20, 50, 6).to(hip_device), 20)
    for bad in (0.0, 6.0):
        with pytest.raises(ValueError, match="score_clamp"):
            sparse_edge_attention(q.to(hip_device), k.to(hip_device), v.to(hip_device), idx, score_clamp=bad)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_graphormer_head_group_lists(hip_device, dtype):
    from budgetformer_amd.attention import CoreAttention
    S, H, hn = 400, 8, 16
    q, k, v, dout = _acts(S, H, hn, 11, dtype)
    bias = torch.randn(1, S, S, H, generator=torch.Generator().manual_seed(12))
    a, b, c = _edges(S, 3000, 13), _edges(S, 1500, 14), _edges(S, 5000, 15)
    core = CoreAttention(H * hn, 0.0, H, 1)
    lists = [
        [a],                                  # one group: every head over a
        [a, b, c, a],                         # four groups of two heads
        [a, None, c],                         # three groups of three heads (the last has two); one None
        [b, b, a.new_zeros(2, 0), c, c, a, b, c],   # one set per head, runs of the same object, one empty
        [a, b, c, a, b, c, a],                # seven groups of two: the last group's head range is empty
    ]
    for li, edge_list in enumerate(lists):
        for with_bias in (False, True):
            bd = bias if with_bias else None

            def dev_fn(qq, kk, vv):
                return core(qq[None], kk[None], vv[None], None if bd is None else bd.to(hip_device),
                            [None if e is None else e.to(hip_device) for e in edge_list], "sparse").view(S, H, hn)

            def ref_fn(qq, kk, vv):
                return sa.graphormer_head_group_attention(kk, qq, vv, edge_list,
                                                          None if bd is None else bd[0].double())

            out, grads = _device_grads(dev_fn, (q, k, v), dout, hip_device)
            ro, rgrads = _oracle_grads(ref_fn, (q, k, v), dout)
            tag = f"list {li} bias {with_bias}"
            assert_close(f"{tag} out", out, ro, TOL[dtype])
            for name, got, ref in zip(("dq", "dk", "dv"), grads, rgrads):
                assert_close(f"{tag} {name}", got, ref, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_graphormer_dense_bias_of_a_batch(hip_device, dtype):
    from budgetformer_amd.attention import CoreAttention
    B, n, H, hn = 3, 150, 4, 16
    S = B * n
    q, k, v, dout = _acts(S, H, hn, 21, dtype)
    bias = torch.randn(B, n, n, H, generator=torch.Generator().manual_seed(22))
    ei = _edges(S, 4000, 23)
    core = CoreAttention(H * hn, 0.0, H, 1)

    def dev_fn(qq, kk, vv, bb):
        return core(qq.view(B, n, H, hn), kk.view(B, n, H, hn), vv.view(B, n, H, hn), bb, ei.to(hip_device),
                    "sparse").reshape(S, H, hn)

    def ref_fn(qq, kk, vv, bb):
        return sa.graphormer_sparse_attention(kk, qq, vv, ei, sa.batched_dense_bias(bb, B, n))

    out, grads = _device_grads(dev_fn, (q, k, v, bias), dout, hip_device)
    ro, rgrads = _oracle_grads(ref_fn, (q, k, v, bias), dout)
    assert_close("out", out, ro, TOL[dtype])
    for name, got, ref in zip(("dq", "dk", "dv", "dbias"), grads, rgrads):
        assert_close(name, got, ref, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gt_per_head_lists_clamp_before_scaling(hip_device, dtype):
    from budgetformer_amd.attention import GTCoreAttention
    S, H, hn = 400, 8, 16
    q, k, v, dout = _acts(S, H, hn, 31, dtype)        # q.k ~ N(0, 16): most scores pass +-5 before scaling
    sets = [_edges(S, 800 + 400 * h, 40 + h) for h in range(H)]
    gt = GTCoreAttention(H * hn, 0.0, H)
    x = (k.double()[sets[0][0], 0] * q.double()[sets[0][1], 0]).sum(-1)
    assert (x.abs() > 5).float().mean() > 0.1 and (x.abs() / 4 < 5).all()   # the two orders differ here
    for edge_list in (sets, sets[:3], [sets[0], None, sets[2], sets[2].new_zeros(2, 0)]):
        gt.reset_head_mass_stats()

        def dev_fn(qq, kk, vv):
            return gt(qq[None], kk[None], vv[None], None,
                      [None if e is None else e.to(hip_device) for e in edge_list]).view(S, H, hn)

        def ref_fn(qq, kk, vv):
            return sa.gt_head_list_attention(qq, kk, vv, edge_list)

        out, grads = _device_grads(dev_fn, (q, k, v), dout, hip_device)
        ro, rgrads = _oracle_grads(ref_fn, (q, k, v), dout)
        tag = f"{len(edge_list)} sets"
        assert_close(f"{tag} out", out, ro, TOL[dtype])
        for name, got, ref in zip(("dq", "dk", "dv"), grads, rgrads):
            assert_close(f"{tag} {name}", got, ref, TOL[dtype])
        # per-head mean exp score: the sum over each head's edges of exp(clamp(q.k, -5, 5) / sqrt(hn))
        q64, k64 = q.double(), k.double()
        want = torch.zeros(H, dtype=torch.float64)
        for h in range(H):
            e = edge_list[h % len(edge_list)]
            if e is None or e.numel() == 0:
                continue
            s = (k64[e[0], h] * q64[e[1], h]).sum(-1).clamp(-5, 5)
            want[h] = torch.exp(s / math.sqrt(hn)).mean()
        got = gt.get_head_mass_stats().double()
        assert torch.allclose(got, want, rtol=TOL[dtype] * 5, atol=0), (got, want)
