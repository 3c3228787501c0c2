"""Exphormer's typed edges (models/exphormer_dist_node_level.py:77-121) in the kernels: each entry's type in
bit 31 of its ids, E[type] applied to the score inside the three passes, dE summed by the dq pass. Against
the float64 oracle (oracle.sparse_attention.exphormer_sparse_attention) with autograd for the gradients of
q, k, v and E; fp32 within 1e-5, bf16 within 2e-2, fp16 within 5e-3, per tensor and per row."""
import pytest
import torch

from oracle import sparse_attention as sa
from parity_helpers import assert_close

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 5e-3}


def _problem(S, n_kv, H, hn, E, seed, dtype, mult=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(S, H, hn, generator=g) * mult).to(dtype)
    k = (torch.randn(n_kv, H, hn, generator=g) * mult).to(dtype)
    v = torch.randn(n_kv, H, hn, generator=g).to(dtype)
    dout = torch.randn(S, H, hn, generator=g).to(dtype)
    ei = torch.stack([torch.randint(0, n_kv, (E,), generator=g), torch.randint(0, S, (E,), generator=g),
                      torch.randint(0, 2, (E,), generator=g)])
    mod = torch.randn(2, H, hn, generator=g) * 0.8 + 0.5
    return q, k, v, dout, ei, mod


def _oracle(q, k, v, dout, ei, mod):
    """The oracle (like the reference) indexes queries and kv rows in one node space, its output has a row
    per kv row: both sides are padded to the larger row count with zero rows, and cut back after."""
    n_q, n_kv = q.size(0), k.size(0)
    M = max(n_q, n_kv)

    def pad(t):
        out = torch.zeros(M, *t.shape[1:], dtype=torch.float64)
        out[:t.size(0)] = t.double()
        return out

    q64, k64, v64 = (pad(t).requires_grad_(True) for t in (q, k, v))
    m64 = mod.double().requires_grad_(True)
    ref = sa.exphormer_sparse_attention(q64, k64, v64, ei, m64)
    ref.backward(pad(dout))
    return ref.detach()[:n_q], q64.grad[:n_q], k64.grad[:n_kv], v64.grad[:n_kv], m64.grad


def _run(dev, q, k, v, dout, idx, mod):
    from budgetformer_amd.attention import typed_edge_attention
    qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    md = mod.to(dev).requires_grad_(True)
    out = typed_edge_attention(qd, kd, vd, md, idx)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    return out.detach(), qd.grad, kd.grad, vd.grad, md.grad


def _check(got, ref, tol):
    for name, a, b in zip(("out", "dq", "dk", "dv", "dE"), got, ref):
        assert_close(name, a, b, tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("chunk,item", [(128, 768), (6, 10)])
def test_typed_attention_against_the_oracle(hip_device, dtype, chunk, item):
    """A random typed edge set (both types, duplicate pairs of either type) with scores scaled into the
    clamp: out, dq, dk, dv and dE. (6, 10) splits the key rows into items; query rows are never split."""
    from budgetformer_amd.hip_ops import AttentionIndex
    S, n_kv, H, hn = 700, 650, 8, 16
    q, k, v, dout, ei, mod = _problem(S, n_kv, H, hn, 9000, seed=5 + chunk, dtype=dtype, mult=1.5)
    ei[:, 1] = ei[:, 0]                                    # the same pair with each type
    ei[2, 1], ei[2, 0] = 1, 0
    idx = AttentionIndex.from_typed_coo(ei.to(hip_device), S, n_kv, chunk=chunk, item=item)
    assert idx.typed and idx.n_kv == n_kv and idx.qplan.items == 0
    if chunk == 6:
        idx.resolve()
        assert idx.kplan.items > 0
    _check(_run(hip_device, q, k, v, dout, idx, mod), _oracle(q, k, v, dout, ei, mod), TOL[dtype])


@pytest.mark.parametrize("dtype,H,hn", [(torch.float32, 8, 32), (torch.float32, 2, 128), (torch.bfloat16, 8, 64),
                                        (torch.bfloat16, 4, 128), (torch.float16, 8, 64)])
def test_typed_attention_at_the_widest_rows(hip_device, dtype, H, hn):
    """Typed edges with rows of 256 (float32) or 512 (bfloat16, float16) elements, one lane group per
    wavefront, key rows split into items: out, dq, dk, dv and dE against the oracle."""
    from budgetformer_amd.hip_ops import AttentionIndex
    S, n_kv = 500, 450
    q, k, v, dout, ei, mod = _problem(S, n_kv, H, hn, 6000, seed=H + hn, dtype=dtype, mult=1.2)
    idx = AttentionIndex.from_typed_coo(ei.to(hip_device), S, n_kv, chunk=6, item=10)
    idx.resolve()
    assert idx.typed and idx.kplan.items > 0
    _check(_run(hip_device, q, k, v, dout, idx, mod), _oracle(q, k, v, dout, ei, mod), TOL[dtype])


def test_typed_long_query_rows_and_hub_keys(hip_device):
    """Query rows of up to 600 entries (no query row is split: they run whole on the row path) and a
    2,000-entry hub key row (split into items on the key side)."""
    from budgetformer_amd.hip_ops import AttentionIndex
    S, n_kv, H, hn = 300, 5000, 8, 16
    q, k, v, dout, ei, mod = _problem(S, n_kv, H, hn, 30_000, seed=9, dtype=torch.float32)
    ei[1, :3000] = torch.arange(3000) % 5                  # queries 0..4: 600 entries each
    ei[0, 5000:7000] = 17                                  # key row 17: a hub
    idx = AttentionIndex.from_typed_coo(ei.to(hip_device), S, n_kv)
    idx.resolve()
    assert idx.kplan.items > 0 and idx.qplan.items == 0
    _check(_run(hip_device, q, k, v, dout, idx, mod), _oracle(q, k, v, dout, ei, mod), 1e-5)


def test_typed_dk_dv_instance_at_scale(hip_device):
    """The large-table typed dk/dv instance (bf16: q + dO above 256 MB, 2M kv rows: non-temporal gathers,
    four rows per group, prefetched slots) on a compact problem; every unattended row comes out zero."""
    from budgetformer_amd import hip_ops
    from budgetformer_amd.hip_ops import AttentionIndex
    H, hn, n_q, n_kv, dt = 8, 16, 600_000, 2_000_000, torch.bfloat16
    assert hip_ops.kv_pass_variant(n_q, n_kv, dt, H, hn) == {"rows_per_group": 4, "stream_rows": True,
                                                             "prefetch_slots": True}
    g = torch.Generator(device=hip_device).manual_seed(12)
    qa = torch.randperm(n_q, generator=g, device=hip_device)[:20_000].sort().values
    kt = torch.randperm(n_kv, generator=g, device=hip_device)[:6_000].sort().values
    src_c = torch.randint(0, 6_000, (200_000,), generator=g, device=hip_device)
    src_c[:3_000] = 0
    dst_c = torch.randint(0, 20_000, (200_000,), generator=g, device=hip_device)
    typ = torch.randint(0, 2, (200_000,), generator=g, device=hip_device)
    q, dout = (torch.empty(n_q, H, hn, device=hip_device, dtype=dt).normal_(generator=g) for _ in range(2))
    k, v = (torch.empty(n_kv, H, hn, device=hip_device, dtype=dt).normal_(generator=g) for _ in range(2))
    mod = torch.randn(2, H, hn, generator=torch.Generator().manual_seed(3)) * 0.8 + 0.5
    idx = AttentionIndex.from_typed_coo(torch.stack([kt[src_c], qa[dst_c], typ]), n_q, n_kv)
    md = mod.to(hip_device)
    out, Z = hip_ops.attn_forward_typed(idx, q, k, v, md)
    dq, dk, dv, dmod = hip_ops.attn_backward_typed(idx, q, k, v, md, Z, dout)
    torch.cuda.synchronize()
    ei = torch.stack([src_c, dst_c, typ]).cpu()
    ref = _oracle(q[qa].cpu(), k[kt].cpu(), v[kt].cpu(), dout[qa].cpu(), ei, mod)
    _check((out[qa], dq[qa], dk[kt], dv[kt], dmod), ref, 2e-2)
    for t, rows in ((out, qa), (dq, qa), (dk, kt), (dv, kt)):
        t[rows] = 0
        assert not t.any()


def test_typed_is_deterministic_and_handles_empty_sets(hip_device):
    """Two backward runs are bit-identical (dE included: its records are summed in a fixed order); an
    empty edge set gives zero outputs and a zero dE."""
    from budgetformer_amd.hip_ops import AttentionIndex
    S, n_kv, H, hn = 400, 400, 8, 16
    q, k, v, dout, ei, mod = _problem(S, n_kv, H, hn, 5000, seed=21, dtype=torch.float32)
    idx = AttentionIndex.from_typed_coo(ei.to(hip_device), S, n_kv)
    a = _run(hip_device, q, k, v, dout, idx, mod)
    b = _run(hip_device, q, k, v, dout, idx, mod)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    e0 = AttentionIndex.from_typed_coo(torch.zeros(3, 0, dtype=torch.long, device=hip_device), S, n_kv)
    out, dq, dk, dv, dm = _run(hip_device, q, k, v, dout, e0, mod)
    for t in (out, dq, dk, dv, dm):
        assert not t.any()


def test_exphormer_module_runs_the_typed_kernels(hip_device):
    """ExphormerCoreAttention with a [3, E] edge set: the typed index over the N kv rows (no [2N] tables),
    output and the gradients of q, k, v and of the edge encoder (edge_type_emb, edge_proj) against the
    float64 oracle with the same encoder."""
    from budgetformer_amd.attention import ExphormerCoreAttention
    S, H, hn = 300, 8, 16
    q, k, v, dout, ei, _ = _problem(S, S, H, hn, 3000, seed=33, dtype=torch.float32)
    mod = ExphormerCoreAttention(H * hn, 0.0, H).to(hip_device)
    qd, kd, vd = (t[None].to(hip_device).requires_grad_(True) for t in (q, k, v))
    out = mod(qd, kd, vd, None, ei.to(hip_device))
    out.backward(dout.reshape(1, S, H * hn).to(hip_device))
    assert mod._typed_idx.typed and mod._typed_idx.n_kv == S
    ref_mod = ExphormerCoreAttention(H * hn, 0.0, H).double()
    ref_mod.load_state_dict({n: t.detach().cpu().double() for n, t in mod.state_dict().items()})
    q64, k64, v64 = (t.double().requires_grad_(True) for t in (q, k, v))
    ref = sa.exphormer_sparse_attention(q64, k64, v64, ei, ref_mod.edge_modulation("cpu"))
    ref.backward(dout.double())
    assert_close("out", out.detach().view(S, H, hn), ref, 1e-5)
    for name, got, r in (("dq", qd.grad[0], q64.grad), ("dk", kd.grad[0], k64.grad), ("dv", vd.grad[0], v64.grad)):
        assert_close(name, got, r, 1e-5)
    for name in ("edge_type_emb.weight", "edge_proj.weight"):
        got = dict(mod.named_parameters())[name].grad
        r = dict(ref_mod.named_parameters())[name].grad
        assert_close(name, got, r, 1e-5)
