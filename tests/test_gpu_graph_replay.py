"""The attention layer captured in a HIP graph (torch.cuda.CUDAGraph) and replayed.

With an index whose split-plan counts stay on the device (``device_counts``), one forward + backward
through the operators makes no host read and no memset, so it can be captured. Every replay, with new
values in the captured input tensors and other eager work between replays, must equal the eager calls
on the same inputs bit for bit (the kernels use no atomics); the first eager result is also checked
against the float64 oracle.
"""
import numpy as np
import pytest
import torch

from oracle import sparse_attention as sa
from parity_helpers import assert_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_attention_layer_graph_replays_equal_eager(hip_device, dtype):
    from budgetformer_amd import hip_ops
    from budgetformer_amd.edges import build_attention_edges
    from budgetformer_amd.graph import CSRGraph, chung_lu_csr
    n, H, hn = 3000, 8, 16
    rowptr, col = chung_lu_csr(n, 30000, seed=9)
    g = CSRGraph.from_csr(rowptr, col, n, device=hip_device)
    tab = build_attention_edges(g, real_edges_per_query=4, rw_edges_per_query=4, walk_length=4,
                                walks_per_node=2, edge_seed=3, global_token=True)
    idx = tab.attention_index(chunk=16, item=40)        # a split token row, token column and heavy kv rows
    # the query plan of a table index is known from the sizes (no device read); the key-side plan is
    # built below with its counts left on the device
    assert idx.kplan is None
    idx.device_counts = True
    idx.ensure_backward()
    assert idx.kplan.heavy_rows is not None
    S = n + 1
    gen = torch.Generator().manual_seed(5)
    base = [torch.randn(S, H, hn, generator=gen).to(dtype) for _ in range(4)]
    q, k, v, dout = (t.to(hip_device) for t in base)

    def layer():
        out, Z = hip_ops.attn_forward(idx, q, k, v)
        dq, dk, dv, _ = hip_ops.attn_backward(idx, q, k, v, None, Z, dout)
        return out, dq, dk, dv

    first = [t.clone() for t in layer()]
    ei = torch.stack([idx.kv.cpu().long(), idx.entry_rows().cpu()])
    q64, k64, v64, d64 = (t.double() for t in base)
    ro, rZ = sa.attention_forward_stats(k64, q64, v64, ei)
    rdq, rdk, rdv, _ = sa.attention_backward_closed_form(k64, q64, v64, ei, ro, rZ, d64)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for name, got, ref in zip(("out", "dq", "dk", "dv"), first, (ro, rdq, rdk, rdv)):
        assert_close(name, got, ref, tol)

    side = torch.cuda.Stream(device=hip_device)          # warm up off the capture stream, as torch asks
    side.wait_stream(torch.cuda.current_stream(hip_device))
    with torch.cuda.stream(side):
        layer()
    torch.cuda.current_stream(hip_device).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = layer()
    torch.cuda.synchronize(hip_device)

    rng = np.random.default_rng(7)
    for rep in range(3):
        scale = float(rng.uniform(0.5, 1.5))
        q.copy_(base[0].to(hip_device) * scale)
        dout.copy_(base[3].to(hip_device) * (2.0 - scale))
        graph.replay()
        torch.cuda.synchronize(hip_device)
        replayed = [t.clone() for t in captured]
        _ = torch.randn(1 << 20, device=hip_device).sum().item()   # unrelated eager work between replays
        eager = layer()
        torch.cuda.synchronize(hip_device)
        for name, a, b in zip(("out", "dq", "dk", "dv"), replayed, eager):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager call"
