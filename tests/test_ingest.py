"""Topology ingest: the safe edge_index.pt loader (CPU) and the device coalesce / bidirect / CSR build (GPU)."""
import numpy as np
import pytest
import torch

from oracle import edge_table as et


def test_load_edge_index_round_trip_and_rejects(tmp_path):
    from budgetformer_amd.graph import load_edge_index
    ei = torch.randint(0, 50, (2, 300))
    torch.save(ei, tmp_path / "edge_index.pt")
    assert torch.equal(load_edge_index(str(tmp_path / "edge_index.pt")), ei)
    torch.save({"a": ei}, tmp_path / "bad.pt")
    with pytest.raises(ValueError):
        load_edge_index(str(tmp_path / "bad.pt"))
    torch.save(torch.rand(2, 10), tmp_path / "float.pt")
    with pytest.raises(ValueError):
        load_edge_index(str(tmp_path / "float.pt"))


class _Opaque:
    pass


def test_load_edge_index_never_unpickles_objects(tmp_path):
    from budgetformer_amd.graph import load_edge_index
    torch.save(_Opaque(), tmp_path / "obj.pt")
    with pytest.raises(Exception):            # weights_only refuses arbitrary classes
        load_edge_index(str(tmp_path / "obj.pt"))


@pytest.mark.gpu
@pytest.mark.parametrize("max_chunk", [None, 700, 64])
def test_coalesce_and_bidirect_match_oracle(hip_device, max_chunk):
    from budgetformer_amd.graph import coalesce_edges, to_bidirected
    rng = np.random.default_rng(4)
    n = 500
    ei = np.stack([rng.integers(0, n, 5000), rng.integers(0, n, 5000)])
    kw = {} if max_chunk is None else {"max_chunk": max_chunk}
    t = torch.from_numpy(ei).to(hip_device)
    assert np.array_equal(coalesce_edges(t, n, **kw).cpu().numpy(), et.coalesce(ei, n))
    ref_bi = et.coalesce(np.concatenate([ei, ei[::-1]], axis=1), n)
    assert np.array_equal(to_bidirected(t, n, **kw).cpu().numpy(), ref_bi)


@pytest.mark.gpu
def test_load_graph_builds_the_walk_csr(hip_device, tmp_path):
    from budgetformer_amd.graph import load_graph
    rng = np.random.default_rng(5)
    n = 400
    ei = np.stack([rng.integers(0, n, 3000), rng.integers(0, n, 3000)])
    torch.save(torch.from_numpy(ei), tmp_path / "edge_index.pt")
    torch.save(torch.zeros(n + 7, 3), tmp_path / "x.pt")          # the features fix N (trailing isolated nodes)
    for bidir in (False, True):
        g, ei_dev = load_graph(str(tmp_path), hip_device, to_bidirected_edges=bidir)
        assert g.num_nodes == n + 7
        ref = et.coalesce(np.concatenate([ei, ei[::-1]], axis=1), n + 7) if bidir else et.coalesce(ei, n + 7)
        rowptr, col = et.csr_from_coo(ref, n + 7)
        assert np.array_equal(g.rowptr.cpu().numpy(), rowptr) and np.array_equal(g.col.cpu().numpy(), col)
        if bidir:
            assert np.array_equal(ei_dev.cpu().numpy(), ref)
