"""Regenerate the golden fixtures in this directory from the CPU oracle.

    python tests/golden/make_golden.py

The fixtures are data only (inputs and expected outputs, .npz without pickles).
The CPU suite checks that the oracle still reproduces them; the GPU suite
checks the HIP kernels against them.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import edge_table as et            # noqa: E402
from oracle import philox                      # noqa: E402
from oracle import sparse_attention as sa      # noqa: E402


def _graph(n, pairs, seed):
    rng = np.random.default_rng(seed)
    w = (np.arange(n) + 5.0) ** -1.0
    p = w / w.sum()
    a = rng.choice(n, size=pairs, p=p)
    b = rng.choice(n, size=pairs, p=p)
    keep = a != b
    src = np.concatenate([a[keep], b[keep]])
    dst = np.concatenate([b[keep], a[keep]])
    return et.csr_from_coo(np.stack([src, dst]), n)


def edge_fixture():
    n, P, L = 300, 2, 4
    rowptr, col = _graph(n, 900, seed=42)
    u = np.random.default_rng(45).random((n * P, L), dtype=np.float32)
    out = {"rowptr": rowptr, "col": col.astype(np.int32), "u": u, "num_nodes": np.int64(n),
           "walk_length": np.int64(L), "walks_per_node": np.int64(P), "edge_seed": np.int64(42)}
    out["walks"] = et.random_walk(rowptr, col, et.walk_starts(n, P), L, u)
    for b_r, b_w in ((4, 4), (0, 3), (3, 0)):
        t, rl = et.build_edge_table(rowptr, col, n, b_r, b_w, L, P, 42, u)
        out[f"table_{b_r}_{b_w}"] = t
        out[f"row_len_{b_r}_{b_w}"] = rl
    src = np.repeat(np.arange(n), np.diff(rowptr))
    out["coo_graphormer_4_4"] = et.build_merged_edges(np.stack([src, col.astype(np.int64)]), n, 4, 4, L, P, 42, u,
                                                      graphormer_global_token=True)
    out["philox_u_seed7"] = philox.walk_uniforms(0, 16, 2, 6, 7, 3)
    np.savez_compressed(os.path.join(HERE, "edge_table_n300.npz"), **out)


def attention_fixture():
    import torch
    S, H, hn, E = 40, 4, 8, 220
    g = torch.Generator().manual_seed(46)
    q, k, v, dout = (torch.randn(S, H, hn, generator=g) * 1.4 for _ in range(4))
    ei = torch.stack([torch.randint(0, S, (E,), generator=g), torch.randint(0, S, (E,), generator=g)])
    # query-major order, ascending kv (the layout the HIP index uses), duplicates kept
    order = np.lexsort((ei[0].numpy(), ei[1].numpy()))
    ei = ei[:, torch.from_numpy(order)]
    bias = torch.randn(E, H, generator=g)
    q64, k64, v64, d64, b64 = (t.double() for t in (q, k, v, dout, bias))
    out, Z = sa.attention_forward_stats(k64, q64, v64, ei, b64)
    dq, dk, dv, db = sa.attention_backward_closed_form(k64, q64, v64, ei, out, Z, d64, b64)
    np.savez_compressed(os.path.join(HERE, "attention_s40.npz"),
                        q=q.numpy(), k=k.numpy(), v=v.numpy(), dout=dout.numpy(), edge_index=ei.numpy(),
                        bias=bias.numpy(), out=out.numpy(), Z=Z.numpy(), dq=dq.numpy(), dk=dk.numpy(),
                        dv=dv.numpy(), dbias=db.numpy())


if __name__ == "__main__":
    edge_fixture()
    attention_fixture()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
