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
sees the same edge set (models/graphormer_dist_node_level.py:1374). Graphormer
and GT also take a list of such edge sets, one per head group
(models/graphormer_dist_node_level.py:175-213) or per head
(models/gt_dist_node_level.py:195-218): heads that share a set run as one
call on their slice of q, k and v.
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
    """out = sum_e exp(clamp(q.k/sqrt(hn)) + bias) * f * v / (Z + 1e-6), HIP fwd/bwd; also returns Z
    (not differentiable)."""

    @staticmethod
    def forward(ctx, q, k, v, bias_e, factor_e, index, dropout, score_clamp):
        # a dropout without bias or factor keeps the forward's keep bits for the dq pass, which then reads
        # them instead of drawing them (with a bias or factor every pass draws: the same bits either way)
        keep_mask = dropout is not None and dropout.rate > 0.0 and bias_e is None and factor_e is None
        res = hip_ops.attn_forward(index, q, k, v, bias_e, factor_e, dropout, score_clamp, keep_mask=keep_mask)
        out, Z = res[0], res[1]
        ctx.keep = res[2] if keep_mask else None
        # the backward needs Z, not out (it sums Delta = dO . out from the entries in float32)
        ctx.save_for_backward(q, k, v, Z, bias_e, factor_e)
        ctx.index = index
        ctx.dropout = dropout          # the same Philox key draws the same mask in the backward
        ctx.score_clamp = score_clamp
        ctx.need_dbias = bias_e is not None and ctx.needs_input_grad[3]
        ctx.mark_non_differentiable(Z)
        return out, Z

    @staticmethod
    def backward(ctx, dout, _dZ):
        q, k, v, Z, bias_e, factor_e = ctx.saved_tensors
        dq, dk, dv, dbias = hip_ops.attn_backward(ctx.index, q, k, v, None, Z, dout.contiguous(), bias_e, factor_e,
                                                  need_dbias=ctx.need_dbias, dropout=ctx.dropout,
                                                  score_clamp=ctx.score_clamp, keep=ctx.keep)
        ctx.keep = None
        return dq, dk, dv, dbias, None, None, None, None


def sparse_edge_attention(q, k, v, index: AttentionIndex, bias_e: Optional[torch.Tensor] = None,
                          factor_e: Optional[torch.Tensor] = None, dropout: Optional[hip_ops.Dropout] = None,
                          score_clamp: float = hip_ops.SCORE_CLAMP, with_z: bool = False):
    """Functional form. q [n_q,H,hn], k/v [n_kv,H,hn]; bias_e/factor_e float32 [nnz,H]; dropout: the
    in-kernel GraphGPS attention dropout (Philox keep mask per entry and head); score_clamp: the bound
    of the clamp on q.k/sqrt(hn). Returns out, or (out, Z) with ``with_z`` (Z [n_q, H] float32, the
    per-query sum of exp scores, not differentiable)."""
    dt = q.dtype
    q, k, v = q.contiguous(), k.to(dt).contiguous(), v.to(dt).contiguous()
    if bias_e is not None:
        bias_e = bias_e.float().contiguous()
    if factor_e is not None:
        factor_e = factor_e.float().contiguous()
    out, Z = _SparseEdgeAttention.apply(q, k, v, bias_e, factor_e, index, dropout, float(score_clamp))
    return (out, Z) if with_z else out


class _TypedEdgeAttention(torch.autograd.Function):
    """Exphormer's typed-edge attention on a typed index: score = clamp(sum_j k q E[type] / sqrt(hn)),
    HIP fwd/bwd (bf::sparse_attn_fwd_typed / _bwd_typed); returns out and takes the gradient of E too."""

    @staticmethod
    def forward(ctx, q, k, v, type_mod, index):
        out, Z = hip_ops.attn_forward_typed(index, q, k, v, type_mod)
        ctx.save_for_backward(q, k, v, type_mod, Z)
        ctx.index = index
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, type_mod, Z = ctx.saved_tensors
        dq, dk, dv, dmod = hip_ops.attn_backward_typed(ctx.index, q, k, v, type_mod, Z, dout.contiguous())
        return dq, dk, dv, dmod, None


def typed_edge_attention(q, k, v, type_mod, index: AttentionIndex):
    """Functional form of the typed path: q [n_q,H,hn], k/v [n_kv,H,hn] (one dtype), type_mod = E
    [2, H, hn] (any float dtype: the kernels take it in float32, and its gradient flows back through the
    cast), index from ``AttentionIndex.from_typed_coo``."""
    dt = q.dtype
    q, k, v = q.contiguous(), k.to(dt).contiguous(), v.to(dt).contiguous()
    return _TypedEdgeAttention.apply(q, k, v, type_mod.float().contiguous(), index)


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
        raise TypeError("a list of edge sets is taken by the modules' per-head paths, not as one edge set")
    else:
        raise TypeError(f"unsupported edge_index type {type(edge_index)}")
    if idx.n_q != n_q or idx.n_kv != n_kv:
        raise ValueError(f"edge set covers ({idx.n_q} queries, {idx.n_kv} kv rows), activations have ({n_q}, {n_kv})")
    return idx


def _dense_bias_to_edges(attn_bias: torch.Tensor, idx: AttentionIndex, batch: int, n: int, H: int) -> torch.Tensor:
    """bias_e[e, h] for a dense key-major bias [batch, n, n, H] over the flattened batch*n rows, as
    models/graphormer_dist_node_level.py:171-173 expands it (unsqueeze(2).repeat over the batch, then
    view(b*n, b*n, H)): entry (src, dst) reads attn_bias[src // n, src % n, dst % n]. With batch 1
    that is attn_bias[0, src, dst]."""
    b = attn_bias.reshape(batch, n, n, H)
    src = idx.kv.to(torch.int64)
    dst = idx.entry_rows()
    if batch == 1:
        return b[0, src, dst, :].float()
    return b[torch.div(src, n, rounding_mode="floor"), src % n, dst % n, :].float()


def _head_runs(assign):
    """Runs (h0, h1, edges) of consecutive heads assigned the same edge-set object (or None)."""
    runs, h, H = [], 0, len(assign)
    while h < H:
        h1 = h + 1
        while h1 < H and assign[h1] is assign[h]:
            h1 += 1
        runs.append((h, h1, assign[h]))
        h = h1
    return runs


def _empty_edges(e) -> bool:
    return e is None or (isinstance(e, torch.Tensor) and e.numel() == 0)


def _per_head_attention(q, k, v, assign, score_clamp, bias_fn=None, stats=None):
    """Attention with head h over edge set assign[h]: each run of heads sharing a set is one call on its
    head slice; heads whose set is None or empty give zeros (wV = 0, Z = 0: 0 / 1e-6). bias_fn(idx, h0,
    h1) gives a run's [nnz, h1-h0] bias; stats = (sum, count) accumulates each head's sum of exp scores
    and edge count (float32 CPU tensors [H])."""
    S, H, hn = q.shape
    pieces = []
    for h0, h1, e in _head_runs(assign):
        if _empty_edges(e):
            pieces.append(q.new_zeros(S, h1 - h0, hn))
            continue
        idx = resolve_index(e, S, k.size(0), q.device)
        bias = bias_fn(idx, h0, h1) if bias_fn is not None else None
        out, Z = sparse_edge_attention(q[:, h0:h1], k[:, h0:h1], v[:, h0:h1], idx, bias, score_clamp=score_clamp,
                                       with_z=True)
        if stats is not None:
            mass = Z.sum(0).detach().cpu()
            for h in range(h0, min(h1, stats[0].numel())):
                stats[0][h] += float(mass[h - h0])
                stats[1][h] += float(idx.nnz)
        pieces.append(out)
    return pieces[0] if len(pieces) == 1 else torch.cat(pieces, dim=1)


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
        """Argument order (k, q, v, edge_index, attn_bias) as at :155; returns [b*S, H, hn]. attn_bias
        [b, S, S, H] is read as the reference expands it over the batch (:171-173). A list of G edge
        sets serves head groups of ceil(H / G) heads (:175-213)."""
        batch_size, node_num = k.size(0), k.size(1)
        num_heads = q.size(2)
        hn = self.hidden_size_per_attention_head
        q = q.reshape(-1, num_heads, hn)
        k = k.reshape(-1, num_heads, hn)
        v = v.reshape(-1, num_heads, hn)
        S = q.size(0)
        if isinstance(edge_index, (list, tuple)):
            groups = max(1, len(edge_index))
            per = (num_heads + groups - 1) // groups
            assign = [edge_index[h // per] if h // per < len(edge_index) else None for h in range(num_heads)]
            bias_fn = None
            if attn_bias is not None:
                def bias_fn(idx, h0, h1):
                    return _dense_bias_to_edges(attn_bias, idx, batch_size, node_num, num_heads)[:, h0:h1]
            return _per_head_attention(q, k, v, assign, hip_ops.SCORE_CLAMP, bias_fn)
        idx = resolve_index(edge_index, S, k.size(0), q.device)
        bias_e = None
        if attn_bias is not None:
            bias_e = _dense_bias_to_edges(attn_bias, idx, batch_size, node_num, num_heads)
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
        self._head_mass_sum = None
        self._head_mass_count = None

    def reset_head_mass_stats(self):
        """Start accumulating, per head, the sum of exp scores and the edge count of the per-head-list
        path (models/gt_dist_node_level.py:75-84, 218-220)."""
        self._head_mass_sum = torch.zeros(self.num_attention_heads_per_partition, dtype=torch.float32)
        self._head_mass_count = torch.zeros(self.num_attention_heads_per_partition, dtype=torch.float32)

    def get_head_mass_stats(self):
        """Mean exp score per head since the reset, or None (models/gt_dist_node_level.py:86-90)."""
        if self._head_mass_sum is None:
            return None
        return self._head_mass_sum / torch.clamp(self._head_mass_count, min=1.0)

    def sparse_attention_bias(self, q, k, v, edge_index, attn_bias):
        """Argument order (q, k, v, ...) as at :179. attn_bias [b, np, s, s] is read key-major, expanded
        over the batch as the Graphormer path does (the reference's own indexing of it at :236-242 fails
        for any edge whose source is not row 0). A list holds one edge set per head, cycled to H
        entries (:195-218): head h scores exp(clamp(q.k, -5, 5) / sqrt(hn)), without the bias."""
        batch_size, node_num = k.size(0), k.size(1)
        num_heads = q.size(2)
        hn = self.hidden_size_per_attention_head
        if isinstance(edge_index, torch.Tensor) and edge_index.dim() == 2 and edge_index.size(0) == 3:
            edge_index = edge_index[:2]
        q = q.reshape(-1, num_heads, hn)
        k = k.reshape(-1, num_heads, hn)
        v = v.reshape(-1, num_heads, hn)
        S = q.size(0)
        if isinstance(edge_index, (list, tuple)):
            if len(edge_index) == 0:
                raise ValueError("an empty list of per-head edge sets")
            assign = [edge_index[h % len(edge_index)] for h in range(num_heads)]
            # clamp(q.k, -5, 5) / sqrt(hn) = clamp(q.k / sqrt(hn), -5 / sqrt(hn), 5 / sqrt(hn))
            stats = (self._head_mass_sum, self._head_mass_count) if self._head_mass_sum is not None else None
            return _per_head_attention(q, k, v, assign, hip_ops.SCORE_CLAMP / math.sqrt(hn), stats=stats)
        idx = resolve_index(edge_index, S, k.size(0), q.device)
        bias_e = None
        if attn_bias is not None:
            bias_e = _dense_bias_to_edges(attn_bias.permute(0, 2, 3, 1), idx, batch_size, node_num, num_heads)
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
    per entry, keyed by its query row and its slot in that row, and head, the
    same bit in the forward and both backward passes) and scales the kept V messages by 1/(1-rate), which is the
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
        """Every attn_type but "full" and "performer" takes the sparse path, as at :201-209."""
        attn_type = "sparse" if attn_type is None else str(attn_type).lower()
        if attn_type in ("full", "performer"):
            raise NotImplementedError(f"attn_type={attn_type!r} is not on the sparse edge-attention path")
        return self._sparse(q, k, v, edge_index, q.size(2), self.hidden_size_per_attention_head)


class ExphormerCoreAttention(nn.Module):
    """Exphormer core attention (models/exphormer_dist_node_level.py:45-121) on the HIP kernels.

    score = sum_j (k_j * q_j / sqrt(d)) * E[type]_j with E = edge_proj(edge_type_emb(type)).
    A [3, E] edge set becomes a typed index (each entry's type in bit 31 of its ids) and the typed
    kernels apply E[type] inside the three passes: no typed copy of K or V is made. Their backward
    returns dq, dk, dv and dE, through which autograd reaches the edge encoder.
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
                self._typed_idx = AttentionIndex.from_typed_coo(edge_index.to(q.device), qf.size(0), n_kv)
                self._typed_key = key
            out = typed_edge_attention(qf, kf, vf, self.edge_modulation(q.device), self._typed_idx)
        else:
            idx = resolve_index(edge_index, qf.size(0), n_kv, q.device)
            out = sparse_edge_attention(qf, kf, vf, idx)
        return out.view(batch_size, s_len, -1)
