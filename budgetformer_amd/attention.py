"""Sparse edge attention on the HIP kernels, behind the reference's module surface.

``CoreAttention`` (Graphormer), ``GTCoreAttention`` and ``GPSCoreAttention``
keep the constructor and ``forward(q, k, v, attn_bias=None, edge_index=None,
attn_type=None)`` signatures of
  models/graphormer_dist_node_level.py:61-613   (sparse path :155-265, dispatch :591-613)
  models/gt_dist_node_level.py:51-522           (sparse path :179-262, dispatch :505-522)
  models/graphgps_dist_node_level.py:135-209    (sparse path :151-177)
  models/exphormer_dist_node_level.py:45-121    (typed-edge modulation)
and compute the sparse path with the HIP forward/backward kernels. Only
``attn_type="sparse"`` is on this path; the dense "full"/"flash"/"performer"
variants are not part of it and raise.

``edge_index`` may be the reference's COO LongTensor [2, E] (or [3, E] with a
type row, which the sparse path ignores, as the reference does), an
``AttentionIndex``, or an ``EdgeTable`` from the edge builder. COO inputs are
converted once per distinct tensor and cached, since every layer of a step
sees the same edge set (models/graphormer_dist_node_level.py:1374).
"""
from __future__ import annotations

import math
from collections import OrderedDict
from typing import Optional

import torch
import torch.nn as nn

from . import hip_ops
from .hip_ops import AttentionIndex


class _SparseEdgeAttention(torch.autograd.Function):
    """out = sum_e exp(clamp(q.k/sqrt(hn)) + bias) * f * v / (Z + 1e-6), HIP fwd/bwd."""

    @staticmethod
    def forward(ctx, q, k, v, bias_e, factor_e, index, dropout):
        out, Z = hip_ops.attn_forward(index, q, k, v, bias_e, factor_e, dropout)
        # the backward needs Z, not out (it sums Delta = dO . out from the entries in float32)
        ctx.save_for_backward(q, k, v, Z, bias_e, factor_e)
        ctx.index = index
        ctx.dropout = dropout          # the same Philox key draws the same mask in the backward
        ctx.need_dbias = bias_e is not None and ctx.needs_input_grad[3]
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, Z, bias_e, factor_e = ctx.saved_tensors
        dq, dk, dv, dbias = hip_ops.attn_backward(ctx.index, q, k, v, None, Z, dout.contiguous(), bias_e, factor_e,
                                                  need_dbias=ctx.need_dbias, dropout=ctx.dropout)
        return dq, dk, dv, dbias, None, None, None


def sparse_edge_attention(q, k, v, index: AttentionIndex, bias_e: Optional[torch.Tensor] = None,
                          factor_e: Optional[torch.Tensor] = None,
                          dropout: Optional[hip_ops.Dropout] = None) -> torch.Tensor:
    """Functional form. q [n_q,H,hn], k/v [n_kv,H,hn]; bias_e/factor_e float32 [nnz,H]; dropout: the
    in-kernel GraphGPS attention dropout (Philox keep mask per entry and head)."""
    dt = q.dtype
    q, k, v = q.contiguous(), k.to(dt).contiguous(), v.to(dt).contiguous()
    if bias_e is not None:
        bias_e = bias_e.float().contiguous()
    if factor_e is not None:
        factor_e = factor_e.float().contiguous()
    return _SparseEdgeAttention.apply(q, k, v, bias_e, factor_e, index, dropout)


class _IndexCache:
    """Small LRU of COO -> AttentionIndex conversions keyed by tensor identity."""

    def __init__(self, size: int = 4):
        self.size = size
        self._d: "OrderedDict" = OrderedDict()

    def get(self, edge_index: torch.Tensor, n_q: int, n_kv: int, chunk: int) -> AttentionIndex:
        key = (edge_index.data_ptr(), tuple(edge_index.shape), edge_index._version, str(edge_index.device),
               n_q, n_kv, chunk)
        hit = self._d.get(key)
        if hit is not None:
            self._d.move_to_end(key)
            return hit[1]
        idx = AttentionIndex.from_coo(edge_index[:2], n_q, n_kv, chunk=chunk)
        self._d[key] = (edge_index, idx)   # keep the tensor alive so its address is not reused
        while len(self._d) > self.size:
            self._d.popitem(last=False)
        return idx


_COO_CACHE = _IndexCache()


def resolve_index(edge_index, n_q: int, n_kv: int, device, chunk: int = hip_ops.DEFAULT_CHUNK) -> AttentionIndex:
    """Turn any accepted edge-set form into an AttentionIndex on `device`."""
    if isinstance(edge_index, AttentionIndex):
        idx = edge_index
    elif hasattr(edge_index, "attention_index"):
        idx = edge_index.attention_index(chunk=chunk)
    elif isinstance(edge_index, torch.Tensor):
        if edge_index.dim() != 2 or edge_index.size(0) not in (2, 3):
            raise ValueError(f"edge_index must be [2, E] or [3, E] (got {tuple(edge_index.shape)})")
        if edge_index.device != device:
            edge_index = edge_index.to(device)
        idx = _COO_CACHE.get(edge_index, n_q, n_kv, chunk)
    elif isinstance(edge_index, (list, tuple)):
        raise NotImplementedError("per-head-group edge lists are not on the single-edge-set sparse path")
    else:
        raise TypeError(f"unsupported edge_index type {type(edge_index)}")
    if idx.n_q != n_q or idx.n_kv != n_kv:
        raise ValueError(f"edge set covers ({idx.n_q} queries, {idx.n_kv} kv rows), activations have ({n_q}, {n_kv})")
    return idx


def _dense_bias_to_edges(attn_bias: torch.Tensor, idx: AttentionIndex, S: int, H: int) -> torch.Tensor:
    """bias_e[e, h] = attn_bias[src(e), dst(e), h] for a dense key-major [S, S, H] bias."""
    b = attn_bias.reshape(S, S, H)
    rows = idx.entry_rows()
    return b[idx.kv.to(torch.int64), rows, :].float()


class CoreAttention(nn.Module):
    """Graphormer core attention (models/graphormer_dist_node_level.py:61-613), sparse path on HIP."""

    def __init__(self, hidden_size, attention_dropout_rate, num_heads, attn_bias_dim=None):
        super().__init__()
        self.hidden_size_per_attention_head = hidden_size // num_heads
        self.num_attention_heads_per_partition = num_heads
        self.scale = math.sqrt(self.hidden_size_per_attention_head)
        self.num_heads = num_heads
        self.att_dropout = nn.Dropout(attention_dropout_rate)
        self.attention_dropout_rate = attention_dropout_rate

    def sparse_attention_bias(self, k, q, v, edge_index, attn_bias):
        """Argument order (k, q, v, edge_index, attn_bias) as at :155; returns [b*S, H, hn]."""
        batch_size, node_num = k.size(0), k.size(1)
        num_heads = q.size(2)
        hn = self.hidden_size_per_attention_head
        q = q.reshape(-1, num_heads, hn)
        k = k.reshape(-1, num_heads, hn)
        v = v.reshape(-1, num_heads, hn)
        S = q.size(0)
        idx = resolve_index(edge_index, S, k.size(0), q.device)
        bias_e = None
        if attn_bias is not None:
            if batch_size != 1:
                raise NotImplementedError("dense attn_bias is supported for batch size 1 (the full-graph path)")
            bias_e = _dense_bias_to_edges(attn_bias, idx, S, num_heads)
        return sparse_edge_attention(q, k, v, idx, bias_e)

    def forward(self, q, k, v, attn_bias=None, edge_index=None, attn_type=None):
        batch_size, s_len = q.size(0), q.size(1)
        if attn_type != "sparse":
            raise NotImplementedError(f"attn_type={attn_type!r} is not on the sparse edge-attention path")
        x = self.sparse_attention_bias(k, q, v, edge_index, attn_bias)
        return x.view(batch_size, s_len, -1)


class GTCoreAttention(nn.Module):
    """GT core attention (models/gt_dist_node_level.py:51-522), always sparse."""

    def __init__(self, hidden_size, attention_dropout_rate, num_heads):
        super().__init__()
        self.hidden_size_per_attention_head = hidden_size // num_heads
        self.num_attention_heads_per_partition = num_heads
        self.scale = math.sqrt(self.hidden_size_per_attention_head)
        self.num_heads = num_heads
        self.att_dropout = nn.Dropout(attention_dropout_rate)

    def sparse_attention_bias(self, q, k, v, edge_index, attn_bias):
        """Argument order (q, k, v, ...) as at :179. attn_bias [b, np, s, s] is read key-major."""
        batch_size = k.size(0)
        num_heads = q.size(2)
        hn = self.hidden_size_per_attention_head
        if isinstance(edge_index, torch.Tensor) and edge_index.dim() == 2 and edge_index.size(0) == 3:
            edge_index = edge_index[:2]
        q = q.reshape(-1, num_heads, hn)
        k = k.reshape(-1, num_heads, hn)
        v = v.reshape(-1, num_heads, hn)
        S = q.size(0)
        idx = resolve_index(edge_index, S, k.size(0), q.device)
        bias_e = None
        if attn_bias is not None:
            if batch_size != 1:
                raise NotImplementedError("dense attn_bias is supported for batch size 1 (the full-graph path)")
            bias_e = _dense_bias_to_edges(attn_bias.permute(0, 2, 3, 1), idx, S, num_heads)
        return sparse_edge_attention(q, k, v, idx, bias_e)

    def forward(self, q, k, v, attn_bias=None, edge_index=None, attn_type=None):
        batch_size, s_len = q.size(0), q.size(1)
        attn_type = "sparse" if attn_type is None else str(attn_type).lower()
        if attn_type != "sparse":
            raise ValueError(
                "GT is restricted to graph-neighborhood sparse attention to match the original implementation; "
                f"got attn_type={attn_type!r}.")
        x = self.sparse_attention_bias(q, k, v, edge_index, attn_bias)
        return x.view(batch_size, s_len, -1)


class GPSCoreAttention(nn.Module):
    """GraphGPS core attention (models/graphgps_dist_node_level.py:135-209), sparse path on HIP.

    Normalise per edge, then dropout, then aggregate (:166-176). In training the
    dropout is drawn inside the kernels (``hip_ops.Dropout``: a Philox keep bit
    per CSR entry and head, the same bit in the forward and both backward
    passes) and scales the kept V messages by 1/(1-rate), which is the
    reference's arithmetic; no [nnz, H] mask is materialised. The Philox key is
    drawn from torch's default generator, so ``torch.manual_seed`` fixes it. An
    explicit ``drop_mask`` still enters as a per-edge factor.
    """

    def __init__(self, hidden_size, attention_dropout_rate, num_heads):
        super().__init__()
        self.hidden_size_per_attention_head = hidden_size // num_heads
        self.num_attention_heads_per_partition = num_heads
        self.num_heads = num_heads
        self.scale = math.sqrt(self.hidden_size_per_attention_head)
        self.att_dropout = nn.Dropout(attention_dropout_rate)

    def _sparse(self, q, k, v, edge_index, num_heads, head_dim, drop_mask: Optional[torch.Tensor] = None):
        batch_size, s_len = q.size(0), q.size(1)
        if isinstance(edge_index, torch.Tensor) and edge_index.size(0) == 3:
            edge_index = edge_index[:2]
        qf = q.reshape(-1, num_heads, head_dim)
        kf = k.reshape(-1, num_heads, head_dim)
        vf = v.reshape(-1, num_heads, head_dim)
        idx = resolve_index(edge_index, qf.size(0), kf.size(0), q.device)
        rate = float(self.att_dropout.p)
        factor = dropout = None
        if drop_mask is not None:
            factor = drop_mask.float() / (1.0 - rate) if rate < 1.0 else torch.zeros_like(drop_mask, dtype=torch.float32)
        elif self.training and rate > 0.0:
            seed = int(torch.randint(0, 2 ** 62, (1,), dtype=torch.int64).item())
            dropout = hip_ops.Dropout(rate, seed)
        out = sparse_edge_attention(qf, kf, vf, idx, None, factor, dropout)
        return out.view(batch_size, s_len, -1)

    def forward(self, q, k, v, attn_bias=None, edge_index=None, attn_type=None):
        attn_type = "sparse" if attn_type is None else str(attn_type).lower()
        if attn_type != "sparse":
            raise NotImplementedError(f"attn_type={attn_type!r} is not on the sparse edge-attention path")
        return self._sparse(q, k, v, edge_index, q.size(2), self.hidden_size_per_attention_head)


class ExphormerCoreAttention(nn.Module):
    """Exphormer core attention (models/exphormer_dist_node_level.py:45-121) on the HIP kernels.

    score = sum_j (k_j * q_j / sqrt(d)) * E[type]_j with E = edge_proj(edge_type_emb(type)).
    Since E depends only on the edge type (2 types), edge e of type t is routed
    to key/value row ``src + t * N_kv`` of the stacked keys ``cat(k*E_0, k*E_1)``
    and values ``cat(v, v)``: the HIP kernels compute exactly the reference
    score, and autograd of the two elementwise products returns dk, dv and the
    gradients of the edge encoder.
    """

    N_EDGE_TYPES = 2

    def __init__(self, hidden_size, attention_dropout_rate, num_heads):
        super().__init__()
        self.hidden_size_per_attention_head = hidden_size // num_heads
        self.num_attention_heads_per_partition = num_heads
        self.num_heads = num_heads
        self.scale = math.sqrt(self.hidden_size_per_attention_head)
        self.att_dropout = nn.Dropout(attention_dropout_rate)
        hidden_size = num_heads * self.hidden_size_per_attention_head
        self.edge_type_emb = nn.Embedding(self.N_EDGE_TYPES, hidden_size)
        self.edge_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self._typed_key = None
        self._typed_idx = None

    def edge_modulation(self, device):
        types = torch.arange(self.N_EDGE_TYPES, device=device)
        return self.edge_proj(self.edge_type_emb(types)).view(self.N_EDGE_TYPES, self.num_heads,
                                                              self.hidden_size_per_attention_head)

    def forward(self, q, k, v, attn_bias=None, edge_index=None, attn_type=None):
        batch_size, s_len = q.size(0), q.size(1)
        num_heads, hn = q.size(2), self.hidden_size_per_attention_head
        qf = q.reshape(-1, num_heads, hn)
        kf = k.reshape(-1, num_heads, hn)
        vf = v.reshape(-1, num_heads, hn)
        n_kv = kf.size(0)
        if isinstance(edge_index, torch.Tensor) and edge_index.dim() == 2 and edge_index.size(0) == 3:
            # the key holds the edge tensor itself, so a match is that tensor, not a reused address
            key = (edge_index, edge_index._version, str(q.device), qf.size(0), n_kv)
            if self._typed_key is None or self._typed_key[0] is not edge_index or self._typed_key[1:] != key[1:]:
                ei = edge_index.to(q.device)
                shifted = torch.stack([ei[0].long() + ei[2].long() * n_kv, ei[1].long()])
                self._typed_idx = AttentionIndex.from_coo(shifted, qf.size(0), self.N_EDGE_TYPES * n_kv)
                self._typed_key = key
            idx = self._typed_idx
            E = self.edge_modulation(q.device).to(kf.dtype)
            k_typed = torch.cat([kf * E[t] for t in range(self.N_EDGE_TYPES)], dim=0)
            v_typed = torch.cat([vf] * self.N_EDGE_TYPES, dim=0)
            out = sparse_edge_attention(qf, k_typed, v_typed, idx)
        else:
            idx = resolve_index(edge_index, qf.size(0), n_kv, q.device)
            out = sparse_edge_attention(qf, kf, vf, idx)
        return out.view(batch_size, s_len, -1)
