"""CPU restatement (torch, CPU tensors) of BudgetFormer's sparse edge attention.

TEST INFRASTRUCTURE ONLY: imported by tests/, smoke() and bench.py's CPU
baseline leg; never by the product package.

Restated reference code (paths relative to the reference root):
  Graphormer CoreAttention.sparse_attention_bias  models/graphormer_dist_node_level.py:155-265
      (tensor path :215-263; argument order (k, q, v, edge_index, attn_bias);
       dense bias indexed attn_bias[src, dst, h] (:242-244))
  GT CoreAttention.sparse_attention_bias          models/gt_dist_node_level.py:179-262
      (argument order (q, k, v, ...); bias [b, np, s, s] permuted to [s, s, np])
  GraphGPS GPSCoreAttention._sparse               models/graphgps_dist_node_level.py:151-177
      (normalise per edge, then dropout, then aggregate)
  Exphormer ExphormerCoreAttention.forward        models/exphormer_dist_node_level.py:77-121
      (score = sum(k*q/sqrt(d) * E[type]); E = Linear(Embedding(type)))
  Graphormer per-head-group edge lists            models/graphormer_dist_node_level.py:175-213
  Graphormer dense bias of a batch (b > 1)        models/graphormer_dist_node_level.py:171-173
  GT per-head edge lists                          models/gt_dist_node_level.py:195-218
      (exp(clamp(q.k, -5, 5) / sqrt(hn)): the clamp before the scaling)
``torch_scatter.scatter(..., reduce='add')`` into a zero tensor is restated as
``index_add_`` (same sum, deterministic order on the CPU). Backward is torch
autograd of the same graph of ops, which is what the reference trains with.

``attention_backward_closed_form`` restates the autograd result in closed form
(per query: g_W = dO/D', g_Z = -sum(dO*out)/D'; per edge:
g_b = (f*(g_W.v_s) + g_Z) * p, g_a = g_b * [-5 <= a <= 5]); it is used to pin
autograd and as the oracle for the HIP backward. The bias is added after the
clamp, so its gradient g_b carries no clamp mask.

Pinning (tests/test_oracle_attention.py): the dense special case against a
dense masked-softmax computation, the single-edge closed form, the equal-score
mean-of-V case, edge-order permutation invariance, float64 gradcheck, and the
closed-form backward against autograd. The list forms: one group, or every
group the same set, equals the tensor path; each head of a G = H list equals
the tensor path on that head alone; the GT list equals the tensor path where
no score reaches the clamp and the mean of V where every score saturates, and
equals attention_forward_stats with clamp 5/sqrt(hn); the batched bias equals
attn_bias[i // n, i % n, j % n] entry by entry.
"""
from __future__ import annotations

import math

import torch

EPS = 1e-6
CLAMP = 5.0


def _scores(k, q, edge_index, scale):
    src = k[edge_index[0].to(torch.long)]
    dest = q[edge_index[1].to(torch.long)]
    score = torch.mul(src, dest)
    score = score / scale
    return score.sum(-1, keepdim=True).clamp(-CLAMP, CLAMP)


def graphormer_sparse_attention(k, q, v, edge_index, attn_bias=None):
    """models/graphormer_dist_node_level.py:215-263 (single edge_index tensor path).

    k, q, v: [S, H, hn] (the reference views [b, S, H, hn] as [b*S, H, hn]);
    edge_index: [2, E] (row 0 = key/value node, row 1 = query node);
    attn_bias: optional dense [S, S, H] indexed [src, dst, h].
    Returns x = wV / (Z + 1e-6), shape [S, H, hn].
    """
    num_heads, hn = q.size(1), q.size(2)
    scale = math.sqrt(hn)
    score = _scores(k, q, edge_index, scale)
    if attn_bias is not None:
        score = score + attn_bias[edge_index[0].to(torch.long), edge_index[1].to(torch.long), :].unsqueeze(-1)
    score = torch.exp(score)
    msg = v[edge_index[0].to(torch.long)] * score
    wV = msg.new_zeros(v.size(0), num_heads, hn)
    wV = wV.index_add(0, edge_index[1].to(torch.long), msg)
    Z = score.new_zeros(v.size(0), num_heads, 1)
    Z = Z.index_add(0, edge_index[1].to(torch.long), score)
    return wV / (Z + EPS)


def gt_sparse_attention(q, k, v, edge_index, attn_bias=None):
    """models/gt_dist_node_level.py:215-262: same arithmetic, (q, k, v) order.

    attn_bias, if given, is [S, S, H] already permuted to key-major order
    (the reference permutes [b, np, s, s] -> [s, s, np] at :236-242).
    """
    return graphormer_sparse_attention(k, q, v, edge_index, attn_bias)


def gps_sparse_attention(q, k, v, edge_index, drop_mask=None, drop_scale=1.0):
    """models/graphgps_dist_node_level.py:151-177.

    norm = p / (Z[dst] + 1e-6); norm = dropout(norm) (here: an injected keep
    mask [E, H] and the 1/(1-rate) scale); out = scatter_add(norm * v[src]).
    """
    num_heads, hn = q.size(1), q.size(2)
    scale = math.sqrt(hn)
    score = torch.exp(_scores(k, q, edge_index, scale))
    dst = edge_index[1].to(torch.long)
    Z = score.new_zeros(v.size(0), num_heads, 1).index_add(0, dst, score)
    norm = score / (Z[dst] + EPS)
    if drop_mask is not None:
        norm = norm * drop_mask.to(norm.dtype).unsqueeze(-1) * drop_scale
    msg = v[edge_index[0].to(torch.long)] * norm
    return torch.zeros_like(v).index_add(0, dst, msg)


def exphormer_sparse_attention(q, k, v, edge_index, edge_mod=None):
    """models/exphormer_dist_node_level.py:92-119.

    edge_index: [2, E] or [3, E] (row 2 = integer edge type); edge_mod: [n_types, H, hn]
    modulation E (the module computes it as edge_proj(edge_type_emb(type))).
    """
    num_heads, hn = q.size(1), q.size(2)
    scale = math.sqrt(hn)
    edge_type = edge_index[2].long() if edge_index.size(0) == 3 else None
    ei = edge_index[:2]
    src = k[ei[0].long()]
    dest = q[ei[1].long()]
    score = torch.mul(src, dest) / scale
    if edge_type is not None:
        score = torch.mul(score, edge_mod[edge_type])
    score = torch.exp(score.sum(-1, keepdim=True).clamp(-CLAMP, CLAMP))
    msg = v[ei[0].long()] * score
    wV = torch.zeros_like(v).index_add(0, ei[1].long(), msg)
    Z = score.new_zeros(v.size(0), num_heads, 1).index_add(0, ei[1].long(), score)
    return wV / (Z + EPS)


def batched_dense_bias(attn_bias, batch_size, node_num):
    """models/graphormer_dist_node_level.py:171-173: the dense bias [b, n, n, H] of a batch, as the
    reference indexes it over the flattened [b*n] rows: unsqueeze(2).repeat(1, 1, b, 1, 1) then
    view(b*n, b*n, H), so entry (i, j) is attn_bias[i // n, i % n, j % n] for every batch of j."""
    num_heads = attn_bias.size(-1)
    rep = attn_bias.unsqueeze(2).repeat(1, 1, batch_size, 1, 1)
    return rep.view(batch_size * node_num, batch_size * node_num, num_heads)


def graphormer_head_group_attention(k, q, v, edge_list, attn_bias=None):
    """models/graphormer_dist_node_level.py:175-213: a list of G edge sets, group g serving heads
    [g*ceil(H/G), min((g+1)*ceil(H/G), H)); a None or empty set leaves its heads zero, and so does a
    group whose head range is empty. Each group's heads follow the single-set arithmetic
    (clamp of q.k/sqrt(hn), bias of those heads after the clamp). attn_bias: dense [S, S, H] or None.

    Deliberate divergence with a bias: the reference adds attn_bias[src, dst, h0:h1], shape [E, h], to a
    score of shape [E, h, 1] (:200-205), which broadcasts to [E, E, h] or raises; this restatement adds
    each entry's bias to its own heads (the `.unsqueeze(-1)` below), the evident intent. Tests of the
    list form with a bias pin that intent, not the reference's result."""
    num_heads, hn = q.size(1), q.size(2)
    scale = math.sqrt(hn)
    groups = max(1, len(edge_list))
    per = (num_heads + groups - 1) // groups
    wV = v.new_zeros(v.size(0), num_heads, hn)
    Z = v.new_zeros(v.size(0), num_heads, 1)
    for g, ei in enumerate(edge_list):
        if ei is None or ei.numel() == 0:
            continue
        h0, h1 = g * per, min((g + 1) * per, num_heads)
        if h0 >= h1:
            continue
        s_idx, t_idx = ei[0].to(torch.long), ei[1].to(torch.long)
        score = (k[s_idx, h0:h1, :] * q[t_idx, h0:h1, :] / scale).sum(-1, keepdim=True).clamp(-CLAMP, CLAMP)
        if attn_bias is not None:
            score = score + attn_bias[s_idx, t_idx, h0:h1].unsqueeze(-1)
        score = torch.exp(score)
        wV[:, h0:h1, :] = wV[:, h0:h1, :].index_add(0, t_idx, v[s_idx, h0:h1, :] * score)
        Z[:, h0:h1, :] = Z[:, h0:h1, :].index_add(0, t_idx, score)
    return wV / (Z + EPS)


def gt_head_list_attention(q, k, v, edge_list):
    """models/gt_dist_node_level.py:195-218: one edge set per head (a list of another length is
    cycled, list[h % len]); head h scores exp(clamp(q.k, -5, 5) / sqrt(hn)) (the clamp before the
    scaling, unlike the tensor path) and takes no bias; a None or empty set leaves the head zero."""
    num_heads, hn = q.size(1), q.size(2)
    scale = math.sqrt(hn)
    if len(edge_list) != num_heads:
        edge_list = [edge_list[i % len(edge_list)] for i in range(num_heads)]
    wV = torch.zeros_like(v)
    Z = v.new_zeros(v.size(0), num_heads, 1)
    for h in range(num_heads):
        e = edge_list[h]
        if e is None or e.numel() == 0:
            continue
        s_idx, t_idx = e[0].to(torch.long), e[1].to(torch.long)
        score = (k[:, h, :][s_idx] * q[:, h, :][t_idx]).sum(-1, keepdim=True).clamp(-CLAMP, CLAMP)
        score = torch.exp(score / scale)
        wV[:, h, :] = wV[:, h, :].index_add(0, t_idx, v[:, h, :][s_idx] * score)
        Z[:, h, :] = Z[:, h, :].index_add(0, t_idx, score)
    return wV / (Z + EPS)


def attention_forward_stats(k, q, v, edge_index, bias_e=None, factor_e=None, clamp=CLAMP):
    """Forward with per-edge bias [E, H] and per-edge V factor [E, H].

    Returns (out [S,H,hn], Z [S,H]). factor_e = keep_mask * drop_scale expresses
    the GPS dropout; it multiplies the V message only (Z sums unmasked p).
    ``clamp``: the bound on q.k/sqrt(hn) (5 on the tensor paths; 5/sqrt(hn)
    expresses GT's per-head lists, which clamp q.k to [-5, 5] before scaling).
    """
    num_heads, hn = q.size(1), q.size(2)
    scale = math.sqrt(hn)
    src = k[edge_index[0].to(torch.long)]
    dest = q[edge_index[1].to(torch.long)]
    a = (src * dest / scale).sum(-1).clamp(-clamp, clamp)
    if bias_e is not None:
        a = a + bias_e
    p = torch.exp(a)
    dst = edge_index[1].to(torch.long)
    w = p if factor_e is None else p * factor_e
    # one output row per query row (the reference's zeros_like(v) has the same S rows as q)
    W = v.new_zeros(q.size(0), num_heads, hn).index_add(0, dst, v[edge_index[0].to(torch.long)] * w.unsqueeze(-1))
    Z = p.new_zeros(q.size(0), num_heads).index_add(0, dst, p)
    return W / (Z + EPS).unsqueeze(-1), Z


def attention_backward_closed_form(k, q, v, edge_index, out, Z, dout, bias_e=None, factor_e=None, clamp=CLAMP):
    """Closed-form gradient of attention_forward_stats (float64-friendly).

    Returns (dq, dk, dv, dbias_e). With D' = Z + 1e-6, Delta = sum_j dO*out:
      g_p   = (f * sum_j (dO/D') * v_s  - Delta/D')
      g_b   = g_p * p                      (bias gradient: bias is added after the clamp)
      g_a   = g_b * [-c <= a_pre <= c]     (c = clamp, 5 by default)
      dv_s += p * f * dO/D';  dk_s += g_a * q_t / sqrt(hn);  dq_t += g_a * k_s / sqrt(hn)
    """
    hn = q.size(2)
    scale = math.sqrt(hn)
    s_idx = edge_index[0].to(torch.long)
    t_idx = edge_index[1].to(torch.long)
    a_pre = (k[s_idx] * q[t_idx] / scale).sum(-1)
    inside = (a_pre >= -clamp) & (a_pre <= clamp)
    a = a_pre.clamp(-clamp, clamp)
    if bias_e is not None:
        a = a + bias_e
    p = torch.exp(a)
    f = torch.ones_like(p) if factor_e is None else factor_e
    dprime = (Z + EPS)                                   # [S, H]
    gW = dout / dprime.unsqueeze(-1)                     # [S, H, hn]
    delta = (dout * out).sum(-1)                         # [S, H]
    gp = f * (gW[t_idx] * v[s_idx]).sum(-1) - (delta / dprime)[t_idx]
    gb = gp * p
    ga = gb * inside.to(p.dtype)
    dv = torch.zeros_like(v).index_add(0, s_idx, (p * f).unsqueeze(-1) * gW[t_idx])
    dk = torch.zeros_like(k).index_add(0, s_idx, ga.unsqueeze(-1) * q[t_idx] / scale)
    dq = torch.zeros_like(q).index_add(0, t_idx, ga.unsqueeze(-1) * k[s_idx] / scale)
    return dq, dk, dv, gb


def attention_fwd_bwd_autograd(k, q, v, edge_index, dout, attn_bias=None):
    """Forward + autograd backward of the Graphormer path; the timed CPU baseline.

    Returns (out, dq, dk, dv).
    """
    k = k.detach().requires_grad_(True)
    q = q.detach().requires_grad_(True)
    v = v.detach().requires_grad_(True)
    out = graphormer_sparse_attention(k, q, v, edge_index, attn_bias)
    out.backward(dout)
    return out.detach(), q.grad, k.grad, v.grad
