"""Precision of alternative dK/dV-pass records, on the CPU oracle (float64 on bf16-rounded inputs).

The key-major pass gathers per entry the q and dO rows plus a per-(query, head) record {1/D', Delta/D'}.
Folding 1/D' into a gathered row g_W = dO/D' held in bf16 (so the record shrinks to Delta/D') perturbs
w = g_W . v independently of the exact Delta, and the cancellation in f*w - Delta/D' turns that
rounding into dK row errors far above the output's own bf16 rounding; held in fp32 the row is exact
but doubles the gathered bytes. These checks keep the record as it is: they fail if the bf16 form ever
stops breaking the per-row bar, or if the exact form drifts from output rounding.
"""
import math

import pytest
import torch

from oracle import sparse_attention as sa
from parity_helpers import row_rel_err


def _bf(x):
    return x.to(torch.bfloat16).double()


def _inputs(S, H, hn, E, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(S, H, hn, generator=g).to(torch.bfloat16).double() for _ in range(3))
    ei = torch.stack([torch.randint(0, S, (E,), generator=g), torch.randint(0, S, (E,), generator=g)])
    d = torch.randn(S, H, hn, generator=g).to(torch.bfloat16).double()
    return q, k, v, ei, d


def _dk_dv_with_gathered_row(q, k, v, ei, d, out, Z, row_cast):
    """dK, dV of the key-major pass when it gathers g_W = dO/D' cast by `row_cast` and the exact Delta/D'."""
    hn = q.size(2)
    s, t = ei[0], ei[1]
    a_pre = (k[s] * q[t] / math.sqrt(hn)).sum(-1)
    inside = (a_pre >= -5) & (a_pre <= 5)
    p = torch.exp(a_pre.clamp(-5, 5))
    dprime = Z + 1e-6
    g_w = row_cast(d / dprime.unsqueeze(-1))
    delta = (d * out).sum(-1) / dprime
    g_a = ((g_w[t] * v[s]).sum(-1) - delta[t]) * p * inside
    dv = torch.zeros_like(v).index_add(0, s, p.unsqueeze(-1) * g_w[t])
    dk = torch.zeros_like(k).index_add(0, s, g_a.unsqueeze(-1) * q[t] / math.sqrt(hn))
    return dk, dv


@pytest.mark.parametrize("S,H,hn,E,seed", [(700, 1, 8, 7000, 236), (700, 2, 8, 7000, 336), (3000, 8, 16, 60000, 5),
                                           (3000, 4, 32, 40000, 7)])
def test_bf16_scaled_gradient_row_breaks_the_per_row_bar(S, H, hn, E, seed):
    q, k, v, ei, d = _inputs(S, H, hn, E, seed)
    out, Z = sa.attention_forward_stats(k, q, v, ei)
    _, dk, dv, _ = sa.attention_backward_closed_form(k, q, v, ei, out, Z, d)
    rounding = row_rel_err(_bf(dk), dk, 1e-3)                     # what a bf16 output costs by itself
    assert rounding < 5e-3
    dk_f, dv_f = _dk_dv_with_gathered_row(q, k, v, ei, d, out, Z, lambda x: x.float().double())
    assert row_rel_err(_bf(dk_f), dk, 1e-3) < 1.5 * rounding     # fp32 row: exact up to output rounding
    dk_b, dv_b = _dk_dv_with_gathered_row(q, k, v, ei, d, out, Z, _bf)
    err = row_rel_err(_bf(dk_b), dk, 1e-3)
    assert err > 2.5 * rounding                                   # bf16 row: several times the output's rounding
    if H == 1:
        assert err > 2e-2                                         # ... and past the bf16 parity bar
