"""CPU checks of the C ABI: the library loads, exports every declared symbol,
and its host-side argument checks reject bad calls without touching a GPU."""
import ctypes as C
import os
import re

import pytest

from budgetformer_amd import _native as N


def test_library_loads_and_exports_every_header_symbol():
    lib = N.load()
    names = N.header_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
        assert name in N._SIGS, f"{name} has no ctypes signature"
    # the exact ABI version the header declares: a binding written against another one must not load
    import re
    declared = int(re.search(r"#define BF_ABI_VERSION (\d+)", open(N._HEADER).read()).group(1))
    assert declared == 303 == N.ABI_VERSION
    assert lib.bf_version() == declared


def test_every_entry_point_cites_the_reference():
    text = open(N._HEADER).read()
    for fn in ("bf_random_walk", "bf_rw_select", "bf_real_select_merge", "bf_build_edge_table",
               "bf_table_to_csr", "bf_coo_to_csr", "bf_reverse_index", "bf_attn_fwd", "bf_attn_bwd"):
        pos = text.index(fn + "(")
        block = text[max(0, text.rfind("/*", 0, pos)):pos]
        assert re.search(r"\w+\.py:\d+", block), fn


def test_argument_errors_surface_as_exceptions():
    lib = N.load()
    rc = lib.bf_random_walk(None, None, 10, 0, 5, 2, 4, None, 0, 0, None, None)
    assert rc == N.BF_ERR_INVALID
    assert b"row pointer" in lib.bf_last_error()
    with pytest.raises(ValueError):
        N.call("bf_rw_select", None, None, None, 10, 0, 5, 2, 4, 4, 0, None, 0, 0, None, None, None)
    idx = N.AttnIndex()
    with pytest.raises(NotImplementedError):     # head_dim 6 does not split into 16-byte lanes
        N.call("bf_attn_fwd", C.byref(idx), N.BF_DTYPE_F32, 2, 6, 5.0, None, None, None, None, None, None, None,
               None, None, None)
    # a dropout rate outside [0, 1] is rejected after the index checks and before any launch (the index
    # here is an empty one: qptr is host memory the call never reads)
    qptr = (C.c_int64 * 1)(0)
    idx.chunk, idx.item, idx.qptr = 128, 768, C.cast(qptr, C.c_void_p)
    drop = N.AttnDropout(1.5, 1, 0)
    with pytest.raises(ValueError, match="dropout rate"):
        N.call("bf_attn_fwd", C.byref(idx), N.BF_DTYPE_F32, 2, 8, 5.0, None, None, None, None, None, C.byref(drop),
               None, None, None, None)
    # the score clamp must lie in (0, 5] (checked before the index)
    for bad in (0.0, -1.0, 5.5, float("nan")):
        with pytest.raises(ValueError, match="score_clamp"):
            N.call("bf_attn_fwd", C.byref(idx), N.BF_DTYPE_F32, 2, 8, bad, None, None, None, None, None, None,
                   None, None, None, None)


def test_gather_probe_arguments_checked_on_the_host():
    """bf_gather_probe refuses rows that are not 16..512 bytes in 16-byte steps, an unaligned table, a call
    with no table and ids missing for a non-empty list, before any launch; an empty id list launches
    nothing (host buffers, never read)."""
    buf = (C.c_int64 * 8)()
    p = C.cast(buf, C.c_void_p)
    for rb in (8, 20, 528):
        with pytest.raises(ValueError, match="row of"):
            N.call("bf_gather_probe", p, rb, None, 0, None, 0, p, 4, 0x7FFFFFFF, 0, p, None)
    with pytest.raises(ValueError, match="16-byte aligned"):
        N.call("bf_gather_probe", C.c_void_p(p.value + 4), 64, None, 0, None, 0, p, 4, 0x7FFFFFFF, 0, p, None)
    with pytest.raises(ValueError, match="no table"):
        N.call("bf_gather_probe", None, 0, None, 0, None, 0, p, 4, 0x7FFFFFFF, 0, p, None)
    with pytest.raises(ValueError, match="bad ids"):
        N.call("bf_gather_probe", p, 64, None, 0, None, 0, None, 4, 0x7FFFFFFF, 0, p, None)
    N.call("bf_gather_probe", p, 64, p, 256, p, 512, p, 0, 0x7FFFFFFF, 1, p, None)


def test_row_stream_probe_arguments_checked_on_the_host():
    """bf_row_stream_probe refuses rows that are not 16..1024 bytes in 16-byte steps, an unaligned table, a
    call with no table, a negative row count and a missing sink, before any launch; zero rows launch
    nothing (host buffers, never touched)."""
    buf = (C.c_int64 * 8)()
    p = C.cast(buf, C.c_void_p)
    for rb in (8, 20, 1040):
        with pytest.raises(ValueError, match="row of"):
            N.call("bf_row_stream_probe", p, None, None, None, rb, None, 4, 0, p, None)
    with pytest.raises(ValueError, match="16-byte aligned"):
        N.call("bf_row_stream_probe", None, None, C.c_void_p(p.value + 4), None, 64, None, 4, 0, p, None)
    with pytest.raises(ValueError, match="no table"):
        N.call("bf_row_stream_probe", None, None, None, None, 64, None, 4, 0, p, None)
    with pytest.raises(ValueError, match="bad row count or sink"):
        N.call("bf_row_stream_probe", p, None, None, None, 64, None, -1, 0, p, None)
    with pytest.raises(ValueError, match="bad row count or sink"):
        N.call("bf_row_stream_probe", p, None, None, None, 64, None, 4, 0, None, None)
    N.call("bf_row_stream_probe", p, p, p, p, 1024, p, 0, 1, p, None)


def test_launches_past_32_bit_work_item_counts_are_refused():
    """A dispatch counts its work-items in 32 bits; a grid of 2^32 or more would be cut short without an
    error, so every launch refuses one before reaching HIP (here bf_expand_rows with 2^32 entries, one
    thread each: host buffers, never read)."""
    buf = (C.c_int64 * 4)(0, 1, 2, 3)
    p = C.cast(buf, C.c_void_p)
    with pytest.raises(ValueError, match="work-items"):
        N.call("bf_expand_rows", p, 1, 2 ** 32, p, None)


def test_walk_record_arguments_checked_on_the_host():
    """bf_walk_records refuses 2^31 edges (32-bit degree field) and an unaligned record array, and the
    walk entry points an unaligned record array, before any launch (host buffers, never read)."""
    buf = (C.c_int64 * 4)(0, 1, 2, 3)
    p = C.cast(buf, C.c_void_p)
    with pytest.raises(ValueError, match="2\\^31"):
        N.call("bf_walk_records", p, p, 2, 2 ** 31, p, None)
    with pytest.raises(ValueError, match="16-byte aligned"):
        N.call("bf_walk_records", p, p, 2, 3, C.c_void_p(p.value + 4), None)
    with pytest.raises(ValueError, match="16-byte aligned"):
        N.call("bf_rw_select", p, p, C.c_void_p(p.value + 8), 2, 0, 1, 2, 2, 2, 0, None, 0, 0, p, p, None)


def test_torch_operators_load_and_register():
    """The TORCH_LIBRARY(bf, ...) extension loads beside the C library and registers the hot path's
    operators; they have device kernels only, so CPU tensors find none (no CPU fallback)."""
    import torch
    ops = N.load_ops()
    for name in ("sparse_attn_fwd", "sparse_attn_bwd", "rw_walk", "build_edge_table", "table_to_csr",
                 "transpose_table"):
        assert str(getattr(ops, name).default._schema).startswith(f"bf::{name}(")
    z = torch.zeros(4, 2, 8)
    with pytest.raises(NotImplementedError):
        ops.sparse_attn_fwd(z, z, z, [None] * 16, [0] * 10)
    with pytest.raises(NotImplementedError):
        ops.rw_walk(torch.zeros(3, dtype=torch.int64), torch.zeros(2, dtype=torch.int32), 0, 2, 1, 2)


def test_python_constants_match_the_header():
    text = open(N._HEADER).read()
    assert int(re.search(r"#define BF_MAX_ITEMS_PER_ROW (\d+)", text).group(1)) == N.BF_MAX_ITEMS_PER_ROW
    assert int(re.search(r"#define BF_LONG_ROW_FACTOR (\d+)", text).group(1)) == N.BF_LONG_ROW_FACTOR


def test_split_row_items_rule():
    """ceil(len / item) up to the 160-item cap; past 160 * 64 items' worth, ceil(len / (64 * item)):
    the rule is continuous at the boundary and never exceeds ceil(len / item) (the capacity bound)."""
    lib = N.load()
    cap, fac = N.BF_MAX_ITEMS_PER_ROW, N.BF_LONG_ROW_FACTOR
    for item in (1, 2, 768):
        for length in (1, item, item + 1, cap * item, cap * item + 1, cap * fac * item, cap * fac * item + 1,
                       111_059_956, 27_800_000):
            n = lib.bf_split_row_items(length, item)
            plain = -(-length // item)
            want = plain if plain <= cap else max(cap, -(-length // (fac * item)))
            assert n == want, (length, item)
            assert 1 <= n <= plain
    assert lib.bf_split_row_items(111_059_956, 768) == 2260     # the c5 token row: 49,152 entries per item
    assert lib.bf_split_row_items(0, 768) == 0


def test_kv_pass_variant_thresholds():
    """bf_attn_bwd_kv_variant reports the dk/dv pass instance a shape takes (host-only): four rows per
    group past 1M kv rows in bf16 (16M in fp32), non-temporal gathers past 256 MB of q + dO, slot
    prefetch for bf16 with several rows per group."""
    import torch
    from budgetformer_amd.hip_ops import kv_pass_variant
    c3 = kv_pass_variant(2_449_030, 2_449_030, torch.bfloat16, 8, 16)
    assert c3 == {"rows_per_group": 4, "stream_rows": True, "prefetch_slots": True}
    c2 = kv_pass_variant(169_344, 169_344, torch.float32, 8, 16)
    assert c2 == {"rows_per_group": 1, "stream_rows": False, "prefetch_slots": False}
    assert kv_pass_variant(300_000, 17_000_000, torch.float32, 8, 16) == {
        "rows_per_group": 4, "stream_rows": True, "prefetch_slots": False}
    assert kv_pass_variant(600_000, 2_000_000, torch.bfloat16, 8, 16)["stream_rows"]      # 307 MB > 256 MB
    assert not kv_pass_variant(500_000, 2_000_000, torch.bfloat16, 8, 16)["stream_rows"]  # 256 MB: not above


def test_split_capacity_bound():
    """Capacities bound every row-length distribution (brute force over small cases)."""
    import itertools
    lib = N.load()
    for lens in itertools.product([0, 1, 3, 4, 5, 9, 17], repeat=3):
        nnz = sum(lens)
        for thr, item in ((1, 1), (3, 4), (4, 2), (2, 8)):
            items = sum(-(-l // item) for l in lens if l > thr)
            rows = sum(1 for l in lens if l > thr)
            assert lib.bf_split_item_capacity(nnz, thr, item) >= items
            assert lib.bf_split_row_capacity(nnz, thr) >= rows


def test_workspace_queries_run_on_cpu():
    out = C.c_size_t(0)
    N.call("bf_reverse_index_workspace_size", 1000, 100, C.byref(out))
    assert out.value >= 3 * 1000 * 4
    N.call("bf_build_edge_table_workspace_size", 1000, 4, 0, 4, C.byref(out))
    assert out.value >= 1000 * 4 * 4


def test_key_inverse_constant_recovers_sources():
    """The fused real-edge select keeps 31-bit keys only and recovers each winner's source as
    ((key - base_q) * kKeyMulInv) mod 2^31. Pin the constant in the kernel source against the oracle's
    key: it must be the inverse of the source multiplier and return every source exactly."""
    import pathlib
    import re

    import numpy as np

    from oracle import edge_table as et

    src_text = (pathlib.Path(__file__).resolve().parents[1] / "budgetformer_amd" / "csrc" / "edge_build.hip").read_text()
    mul = int(re.search(r"kKeyMul = (0x[0-9a-fA-F]+|\d+)u;", src_text).group(1), 0)
    inv = int(re.search(r"kKeyMulInv = (0x[0-9a-fA-F]+|\d+)u;", src_text).group(1), 0)
    assert (mul * inv) % 2**32 == 1
    rng = np.random.default_rng(0)
    s = rng.integers(0, 2**31 - 1, 20000, dtype=np.int64)
    q = rng.integers(0, 2**31 - 1, 20000, dtype=np.int64)
    for seed in (0, 17, 42 + 17, 987654 + 37):
        key = et.edge_key(s, q, seed).astype(np.int64)
        # base_q = q*214013 + seed*2654435761 + 12345 (mod 2^32): the key with src = 0
        base = et.edge_key(np.zeros_like(q), q, seed).astype(np.int64)
        back = (((key - base) % 2**32) * inv) % 2**32 & 0x7FFFFFFF
        assert np.array_equal(back, s)


@pytest.mark.parametrize("struct,mirror", [("bf_attn_index", "AttnIndex"), ("bf_attn_dropout", "AttnDropout")])
def test_struct_mirrors_match_the_header(tmp_path, struct, mirror):
    """The ctypes mirrors have the header's size and field offsets: a C program built against the header
    prints them (a field added to one side only, or reordered, fails here instead of shifting pointers)."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    cls = getattr(N, mirror)
    names = [f[0] for f in cls._fields_]
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "budgetformer_hip.h"', "int main(void) {",
             f'  printf("%zu\\n", sizeof({struct}));']
    lines += [f'  printf("%zu\\n", offsetof({struct}, {f}));' for f in names]
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", os.path.dirname(N._HEADER), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert got == [C.sizeof(cls)] + [getattr(cls, f).offset for f in names]
