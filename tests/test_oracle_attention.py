"""Pins for the CPU attention oracle (oracle/sparse_attention.py)."""
import math

import pytest
import torch

from oracle import sparse_attention as sa


def _rand(S, H, hn, seed, dtype=torch.float64, mult=1.0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(S, H, hn, generator=g, dtype=dtype) * mult for _ in range(3)]


def test_dense_special_case_matches_dense_softmax():
    S, H, hn = 7, 3, 4
    q, k, v = _rand(S, H, hn, 0, mult=0.5)
    src, dst = torch.meshgrid(torch.arange(S), torch.arange(S), indexing="ij")
    ei = torch.stack([src.reshape(-1), dst.reshape(-1)])
    out = sa.graphormer_sparse_attention(k, q, v, ei)
    # dense: scores[h, t, s] = q_t . k_s / sqrt(hn); no clamp is hit at this scale
    scores = torch.einsum("thd,shd->hts", q, k) / math.sqrt(hn)
    assert scores.abs().max() < 5
    p = torch.exp(scores)
    dense = torch.einsum("hts,shd->thd", p, v) / (p.sum(-1).transpose(0, 1).unsqueeze(-1) + 1e-6)
    torch.testing.assert_close(out, dense, rtol=1e-12, atol=1e-12)


def test_single_edge_closed_form():
    q, k, v = _rand(3, 2, 4, 1)
    ei = torch.tensor([[2], [0]])
    out = sa.graphormer_sparse_attention(k, q, v, ei)
    s = ((k[2] * q[0]).sum(-1) / 2.0).clamp(-5, 5)
    expect = v[2] * (torch.exp(s) / (torch.exp(s) + 1e-6)).unsqueeze(-1)
    torch.testing.assert_close(out[0], expect)
    assert out[1].abs().max() == 0 and out[2].abs().max() == 0   # queries without edges


def test_equal_scores_give_mean_of_v():
    q, k, v = _rand(6, 2, 4, 2)
    q.zero_()
    ei = torch.tensor([[1, 2, 3, 5], [0, 0, 0, 0]])
    out = sa.graphormer_sparse_attention(k, q, v, ei)
    torch.testing.assert_close(out[0], v[[1, 2, 3, 5]].sum(0) / (4 + 1e-6))


def test_clamp_bounds_scores():
    q, k, v = _rand(4, 1, 4, 3)
    q[0] = 1.0
    k[1] = 4.0       # a = 16*4/2 = +32 -> clamps to +5
    k[2] = -3.0      # a = -6 -> clamps to -5
    ei = torch.tensor([[1, 2], [0, 0]])
    out = sa.graphormer_sparse_attention(k, q, v, ei)
    p1, p2 = math.exp(5.0), math.exp(-5.0)
    expect = (p1 * v[1] + p2 * v[2]) / (p1 + p2 + 1e-6)
    torch.testing.assert_close(out[0], expect)


def test_permutation_invariance():
    q, k, v = _rand(20, 4, 8, 4)
    g = torch.Generator().manual_seed(5)
    ei = torch.randint(0, 20, (2, 90), generator=g)
    perm = torch.randperm(90, generator=g)
    a = sa.graphormer_sparse_attention(k, q, v, ei)
    b = sa.graphormer_sparse_attention(k, q, v, ei[:, perm])
    torch.testing.assert_close(a, b)


def test_gradcheck_float64():
    q, k, v = _rand(6, 2, 4, 6)
    ei = torch.tensor([[0, 1, 2, 3, 4, 5, 1, 2], [1, 1, 1, 2, 2, 3, 5, 5]])
    bias = torch.randn(6, 6, 2, dtype=torch.float64)
    for t in (q, k, v, bias):
        t.requires_grad_(True)
    assert torch.autograd.gradcheck(lambda k_, q_, v_, b_: sa.graphormer_sparse_attention(k_, q_, v_, ei, b_),
                                    (k, q, v, bias))


@pytest.mark.parametrize("with_bias,with_mask", [(False, False), (True, False), (False, True)])
def test_closed_form_backward_matches_autograd(with_bias, with_mask):
    S, H, hn, E = 30, 4, 8, 200
    q, k, v = _rand(S, H, hn, 7, mult=1.5)        # some scores hit the clamp
    g = torch.Generator().manual_seed(8)
    ei = torch.randint(0, S, (2, E), generator=g)
    bias = torch.randn(E, H, generator=g, dtype=torch.float64) if with_bias else None
    factor = ((torch.rand(E, H, generator=g) > 0.5).double() * 2.0) if with_mask else None
    dout = torch.randn(S, H, hn, generator=g, dtype=torch.float64)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    bb = bias.clone().requires_grad_(True) if bias is not None else None
    out, Z = sa.attention_forward_stats(kk, qq, vv, ei, bb, factor)
    out.backward(dout)
    dq, dk, dv, dbias = sa.attention_backward_closed_form(k, q, v, ei, out.detach(), Z.detach(), dout, bias, factor)
    torch.testing.assert_close(dq, qq.grad)
    torch.testing.assert_close(dk, kk.grad)
    torch.testing.assert_close(dv, vv.grad)
    if with_bias:
        torch.testing.assert_close(dbias, bb.grad)


def test_stats_forward_equals_reference_forward():
    q, k, v = _rand(25, 4, 8, 9)
    g = torch.Generator().manual_seed(10)
    ei = torch.randint(0, 25, (2, 120), generator=g)
    out, _ = sa.attention_forward_stats(k, q, v, ei)
    torch.testing.assert_close(out, sa.graphormer_sparse_attention(k, q, v, ei))


def test_gps_mask_equals_factor_form():
    q, k, v = _rand(25, 4, 8, 11)
    g = torch.Generator().manual_seed(12)
    ei = torch.randint(0, 25, (2, 120), generator=g)
    keep = torch.rand(120, 4, generator=g) > 0.5
    a = sa.gps_sparse_attention(q, k, v, ei, keep, 2.0)
    b, _ = sa.attention_forward_stats(k, q, v, ei, None, keep.double() * 2.0)
    torch.testing.assert_close(a, b)
    torch.testing.assert_close(sa.gps_sparse_attention(q, k, v, ei), sa.graphormer_sparse_attention(k, q, v, ei))


def test_exphormer_oracle_reduces_to_plain_and_to_typed_keys():
    q, k, v = _rand(30, 4, 8, 21)
    g = torch.Generator().manual_seed(22)
    ei = torch.randint(0, 30, (2, 200), generator=g)
    types = torch.randint(0, 2, (200,), generator=g)
    ones = torch.ones(2, 4, 8, dtype=torch.float64)
    # E = 1 for both types: plain sparse attention
    torch.testing.assert_close(sa.exphormer_sparse_attention(q, k, v, torch.cat([ei, types[None]]), ones),
                               sa.graphormer_sparse_attention(k, q, v, ei))
    # typed keys: route type t to row src + t*N of cat(k*E0, k*E1), values cat(v, v)
    E = torch.randn(2, 4, 8, generator=g, dtype=torch.float64)
    ref = sa.exphormer_sparse_attention(q, k, v, torch.cat([ei, types[None]]), E)
    k2 = torch.cat([k * E[0], k * E[1]])
    v2 = torch.cat([v, v])
    q2 = torch.cat([q, torch.zeros_like(q)])
    shifted = torch.stack([ei[0] + types * 30, ei[1]])
    got = sa.graphormer_sparse_attention(k2, q2, v2, shifted)[:30]
    torch.testing.assert_close(got, ref)


def _edges(S, E, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.stack([torch.randint(0, S, (E,), generator=g), torch.randint(0, S, (E,), generator=g)])


def test_head_group_lists_reduce_to_the_tensor_path():
    S, H, hn = 40, 6, 4
    q, k, v = _rand(S, H, hn, 21)
    ei = _edges(S, 300, 22)
    g = torch.Generator().manual_seed(23)
    bias = torch.randn(S, S, H, generator=g, dtype=torch.float64)
    full = sa.graphormer_sparse_attention(k, q, v, ei, bias)
    # one group, and every group the same set (G = 2, 3, 4, 6, 7: the last has an empty head range)
    for G in (1, 2, 3, 4, 6, 7):
        torch.testing.assert_close(sa.graphormer_head_group_attention(k, q, v, [ei] * G, bias), full)
    # G = H distinct sets: head h is the tensor path on head h alone
    sets = [_edges(S, 50 + 30 * h, 30 + h) for h in range(H)]
    out = sa.graphormer_head_group_attention(k, q, v, sets, bias)
    for h in range(H):
        one = sa.graphormer_sparse_attention(k[:, h:h + 1], q[:, h:h + 1], v[:, h:h + 1], sets[h],
                                             bias[:, :, h:h + 1])
        torch.testing.assert_close(out[:, h:h + 1], one)
    # a None or empty set leaves its heads at zero (G = 3: heads 2, 3 belong to group 1)
    out = sa.graphormer_head_group_attention(k, q, v, [ei, None, ei])
    assert out[:, 2:4].abs().max() == 0 and out[:, :2].abs().max() > 0
    out = sa.graphormer_head_group_attention(k, q, v, [ei, ei.new_zeros(2, 0), ei])
    assert out[:, 2:4].abs().max() == 0


def test_gt_head_list_clamps_before_scaling():
    S, H, hn = 30, 4, 16
    ei = _edges(S, 200, 41)
    # small scores (|q.k| < 5): the clamp is inactive in both forms, so each head is the tensor path
    q, k, v = _rand(S, H, hn, 42, mult=0.3)
    assert (k[ei[0]] * q[ei[1]]).sum(-1).abs().max() < 5
    torch.testing.assert_close(sa.gt_head_list_attention(q, k, v, [ei] * H), sa.gt_sparse_attention(q, k, v, ei))
    # q.k in (5, 5 sqrt(hn)) for every edge: the tensor path does not clamp (q.k/4 < 5) but the list form
    # saturates every score at exp(5/4), so each query's output is the plain mean of its sources' V rows
    q = torch.ones(S, H, hn, dtype=torch.float64) * 0.4
    k = torch.ones(S, H, hn, dtype=torch.float64) * (1.0 + torch.rand(S, 1, 1, dtype=torch.float64,
                                                                      generator=torch.Generator().manual_seed(3)))
    x = (k[ei[0]] * q[ei[1]]).sum(-1)
    assert (x > 5).all() and (x / 4 < 5).all()
    out = sa.gt_head_list_attention(q, k, v, [ei])          # a list of one set, cycled over the heads
    p = math.exp(5 / 4)
    cnt = torch.zeros(S, dtype=torch.float64).index_add(0, ei[1], torch.ones(ei.size(1), dtype=torch.float64))
    mean = torch.zeros(S, H, hn, dtype=torch.float64).index_add(0, ei[1], v[ei[0]])
    expect = mean * p / (cnt * p + 1e-6).view(S, 1, 1)
    torch.testing.assert_close(out, expect)
    assert not torch.allclose(out, sa.gt_sparse_attention(q, k, v, ei))
    # and it is the stats form with the clamp bound 5 / sqrt(hn) after the scaling
    q, k, v = _rand(S, H, hn, 43, mult=1.2)
    got, _ = sa.attention_forward_stats(k, q, v, ei, clamp=5 / math.sqrt(hn))
    torch.testing.assert_close(got, sa.gt_head_list_attention(q, k, v, [ei] * H))


def test_batched_dense_bias_indexing():
    b, n, H = 3, 5, 2
    g = torch.Generator().manual_seed(9)
    bias = torch.randn(b, n, n, H, generator=g, dtype=torch.float64)
    full = sa.batched_dense_bias(bias, b, n)
    assert full.shape == (b * n, b * n, H)
    for i in range(b * n):
        for j in range(b * n):
            assert torch.equal(full[i, j], bias[i // n, i % n, j % n])
    assert torch.equal(sa.batched_dense_bias(bias[:1], 1, n), bias[0])


def test_closed_form_backward_with_a_clamp_bound_matches_autograd():
    S, H, hn = 25, 2, 4
    q, k, v = _rand(S, H, hn, 51, mult=1.5)
    ei = _edges(S, 150, 52)
    c = 5 / math.sqrt(hn)
    q, k, v = (t.requires_grad_(True) for t in (q, k, v))
    out, Z = sa.attention_forward_stats(k, q, v, ei, clamp=c)
    dout = torch.randn(S, H, hn, dtype=torch.float64, generator=torch.Generator().manual_seed(53))
    out.backward(dout)
    a_pre = (k[ei[0]] * q[ei[1]] / math.sqrt(hn)).sum(-1)
    assert (a_pre.abs() > c).any() and (a_pre.abs() < c).any()     # both sides of the bound occur
    dq, dk, dv, _ = sa.attention_backward_closed_form(k.detach(), q.detach(), v.detach(), ei, out.detach(),
                                                      Z.detach(), dout, clamp=c)
    for got, ref in ((dq, q.grad), (dk, k.grad), (dv, v.grad)):
        torch.testing.assert_close(got, ref)
