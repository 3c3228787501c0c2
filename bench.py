#!/usr/bin/env python
"""Benchmark of BudgetFormer's per-layer hot path on one MI355X.

A step is one pass of the hot path over one configuration:
  1. budgeted edge construction (Philox walks, real/RW top-k, merge) into the
     [N, B] table, the attention CSR (with the Graphormer global token where the
     model has it), the reverse index and the split plans;
  2. one sparse-attention layer forward + backward over those edges.
Inputs (graph, q/k/v, dO) are resident in HBM before the timed region. The
W warmup steps are followed by up to 5 more while a step still grows PyTorch's
caching allocator (fresh device memory pays for its first touch, up to 2 s at
c5); `warmup_steps_run` says how many ran. The K timed steps are exactly K.

The default run measures c2 (the configuration the north-star target is quoted
on) and, in the same JSON line under `extra_configs`, c3 (bf16, a working set
above the 256 MB Infinity Cache), c4 (GraphGPS, B=32, in-kernel dropout 0.5)
and c5 (a 27.8M-query shard of a 1.6B-edge graph with the Graphormer token),
each with its own roofline and CPU baseline.

`value` is the attention layer's memory traffic rate: the bytes its kernels
move between L2 and the memory fabric per layer (request-size counter sums of
the committed rocprofv3 profile, `profiles/attention_<config>_<dtype>_pmc.json`,
per launch) over the layer's fwd+bwd HIP-event time. Requests the Infinity
Cache serves count too, so it bounds the HBM rate from above, and it cannot
exceed what the fabric moves. Beside it: the gather-model rate (every gathered
K/V/q/dO row counted at full size per edge; a work rate that exceeds the HBM
peak at c2, where the gathered rows are cache-resident) and the compulsory
(unique-tensor) rate, a lower bound of the HBM traffic; the dominant kernel's
roofline (algorithmic bytes / its HIP-event time, with its counter traffic and
rate beside it); the edge builder's RW edges/s and table entries/s; and the CPU
oracle timed on this host's cores as `cpu_baseline`.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "sparse-attn layer fwd+bwd ms & HBM GB/s; RW-edge build edges/sec; 1 GPU"
HBM_PEAK_GBS = 8000.0

CONFIGS = {
    "c1": dict(name="c1: uniform graph N=2,708 E=10,556, Graphormer hidden 64, 8 heads, L=4 P=2 B=8 (4,4), fp32",
               n=2708, e=10556, kind="uniform", H=8, hn=8, L=4, P=2, b_r=4, b_w=4, dtype="float32", token=True),
    "c2": dict(name="c2: Chung-Lu power-law N=169,343 E=1,166,243, Graphormer hidden 128, 8 heads, L=4 P=2 "
                    "B=8 (4,4), fp32",
               n=169_343, e=1_166_243, kind="chung_lu", H=8, hn=16, L=4, P=2, b_r=4, b_w=4, dtype="float32",
               token=True),
    "c3": dict(name="c3: Chung-Lu power-law N=2,449,029 E=61,859,140 (max deg 17K), GT hidden 128, 8 heads, L=4 P=4 "
                    "B=16 (8,8), bf16",
               n=2_449_029, e=61_859_140, kind="device", max_degree=17_000, H=8, hn=16, L=4, P=4, b_r=8, b_w=8,
               dtype="bfloat16", token=False, cpu_sample=100_000),
    "c4": dict(name="c4: power-law N=2,923,922 E=13,975,788, GraphGPS hidden 128, 8 heads, L=8 P=4 B=32 (16,16), "
                    "bf16, attention dropout 0.5 (training; drawn in the kernels)",
               n=2_923_922, e=13_975_788, kind="device", H=8, hn=16, L=8, P=4, b_r=16, b_w=16, dtype="bfloat16",
               token=False, dropout=0.5, cpu_sample=100_000),
    "c5": dict(name="c5: one GPU's 27.8M-query shard of a power-law graph N=111,059,956 E=1.6B (max deg 100K), "
                    "Graphormer hidden 128, 8 heads, L=4 P=2 B=8 (4,4), bf16, global token (the shard holds node 0)",
               n=111_059_956, e=1_600_000_000, kind="device", max_degree=100_000, H=8, hn=16, L=4, P=2, b_r=4,
               b_w=4, dtype="bfloat16", token=True, n_q=27_800_000, cpu_sample=250_000),
}


def attention_bytes(s, D, H, n_q, n_kv, nnz):
    """Gather-model algorithmic bytes (forward, backward) of one layer: every gathered row at full size per
    edge, every streamed row once. Forward: Q read, O written, K and V per edge, kv ids, Z. Backward: dO and
    Q read, dQ written, K and V per edge (dq pass), Q and dO per edge (dk/dv pass), dK and dV written, the
    row statistics, kv ids, reverse ids and positions (the backward does not read the forward's output)."""
    a_fwd = s * D * (2 * n_q + 2 * nnz) + 4 * nnz + 4 * n_q * H
    a_bwd = s * D * (3 * n_q + 2 * n_kv + 4 * nnz) + 8 * n_q * H + 8 * nnz * H + 12 * nnz
    return a_fwd, a_bwd


def compulsory_bytes(s, D, H, n_q, n_kv, nnz, n_kv_touched):
    """Unique-tensor bytes of one layer, each tensor read or written once: a lower bound of its HBM
    traffic. Forward: q, the attended K and V rows, out, Z, the CSR (qptr, kv). Backward: q, dO, Z, the
    attended K and V rows, dq, dK and dV of every kv row, the row stats (written, read), the CSR and the
    reverse index (kptr, kq)."""
    row = s * D
    fwd = row * (2 * n_q + 2 * n_kv_touched) + 4 * H * n_q + 8 * n_q + 4 * nnz
    bwd = (row * (3 * n_q + 2 * n_kv_touched + 2 * n_kv) + 4 * H * n_q + 16 * H * n_q + 8 * n_q + 4 * nnz
           + 8 * n_kv + 4 * nnz)
    return fwd + bwd


def token_records(s, D, n_q, q_items):
    """Records of key 0's dK/dV terms the dq pass writes with a token column: one per workgroup of 256
    lanes, a row taking the next power of two >= D*s/16 lanes."""
    lpr = 1
    while lpr < D * s // 16:
        lpr *= 2
    return q_items + -(-n_q // (256 // lpr))


def kernel_bytes(s, D, H, lens_q, lens_k, n_token_rec=0, entry_bytes=0, token_row=0, chunk=128, kv_blocks=0,
                 keep_mask=False):
    """Algorithmic bytes of the three pass kernels (each covers every entry: short rows and split items).

    With a token column (n_token_rec records) the dq pass also writes key 0's dK/dV terms, 2*D floats per
    record, and the dk/dv pass reads those records instead of gathering key 0's entries and its K, V rows.
    With the token row (token_row = its length: query 0 attends kv 1..token_row) each of the dk/dv pass's
    kv_blocks row workgroups reads query 0's q, dO and row stats once, and its short kv rows in 1..token_row
    take their first entry (query 0's) from that copy instead of gathering it.
    entry_bytes: what the dk/dv pass reads per gathered entry beyond its query id: 4 for the entry's slot in
    its query's row (with the query, the dropout's key), 12 with a bias or factor (the slot and the query's
    row start, which give the CSR position they are indexed by).
    keep_mask: a dropout's keep mask, one byte per entry and 8 heads, written by the forward and read by the
    dq pass."""
    n_q, nnz = lens_q.size, int(lens_q.sum())
    n_kv = lens_k.size
    nk_touched = int((lens_k > 0).sum())
    gathered = nnz
    rec_bytes = n_token_rec * 2 * D * 4
    if n_token_rec:
        gathered -= int(lens_k[0])
        nk_touched -= int(lens_k[0] > 0)
    row = s * D
    tok_bytes = 0
    if token_row:
        lk = lens_k[1:token_row + 1]
        gathered -= int(((lk > 0) & (lk <= chunk)).sum())
        tok_bytes = kv_blocks * (2 * row + 8 * H)
    mask = (H + 7) // 8 * nnz if keep_mask else 0
    return {
        # Q read, O write, K and V gathered per edge, kv ids, Z write, qptr (+ the keep mask written)
        "attn_fwd_kernel": row * (2 * n_q + 2 * nnz) + 4 * nnz + 4 * H * n_q + 8 * n_q + mask,
        # Q, dO read, dQ write, K and V per edge, kv ids, Z read + row stats write, qptr (+ token records,
        # + the keep mask read)
        "attn_bwd_q_kernel": row * (3 * n_q + 2 * nnz) + 4 * nnz + 12 * H * n_q + 8 * n_q + rec_bytes + mask,
        # dK, dV written for every row; K, V read for rows with entries; Q and dO per gathered entry,
        # the {1/D', Delta/D'} row stats per gathered entry, kq ids, kptr, row order (+ token records)
        "attn_bwd_kv_kernel": row * (2 * n_kv + 2 * nk_touched + 2 * gathered) + 8 * H * gathered
        + 4 * gathered + 12 * n_kv + rec_bytes + entry_bytes * gathered + tok_bytes,
    }


def rocprof_summary(stats_csv: str, top: int = 25) -> str:
    """Markdown table of a rocprofv3 ``*_kernel_stats.csv`` (kernel, calls, avg/min/max us, share)."""
    import csv
    import re
    rows = list(csv.DictReader(open(stats_csv)))
    out = ["| kernel | calls | avg us | min us | max us | % of GPU time |", "|---|---:|---:|---:|---:|---:|"]
    for r in rows[:top]:
        name = r["Name"]
        m = re.search(r"(\w+_kernel)\b", name)
        if "rocprim" in name:
            kind = re.search(r"detail::(radix_sort_onesweep_\w+?|scan_impl|init_lookback\w*?)[<(]", name)
            short = "rocprim::" + (kind.group(1) if kind else "kernel")
        elif m:
            targs = re.match(r"\s*<([^<>()]*)>", name[m.end():])
            short = m.group(1) + (f"<{targs.group(1).replace('unsigned short', 'bf16')}>" if targs else "")
        else:
            short = name.split("(")[0][:60]
        out.append(f"| {short} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                   f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
    return "\n".join(out)


def _short_kernel(name: str) -> str:
    import re
    m = re.search(r"(\w+_kernel)\b", name)
    if "rocprim" in name:
        return "rocprim"
    return m.group(1) if m else name.split("(")[0][:60]


def _counter_means(path: str) -> dict:
    """{kernel: mean Counter_Value per dispatch} from a rocprofv3 counter_collection.csv."""
    import collections
    import csv
    acc = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        acc[_short_kernel(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in acc.items()}


def pmc_summary(fetch_csv, write_csv, copy_fetch_csv, copy_write_csv, copy_bytes, kernels_of_interest):
    """HBM-side bytes per dispatch from FETCH_SIZE / WRITE_SIZE runs, each scaled by what the
    same counter reads for a plain copy of ``copy_bytes`` bytes. Returns (markdown, dict)."""
    f, w = _counter_means(fetch_csv), _counter_means(write_csv)
    cf, cw = _counter_means(copy_fetch_csv), _counter_means(copy_write_csv)
    copy_name = max(cf, key=cf.get)
    f_scale = copy_bytes / (cf[copy_name] * 1024.0)
    w_scale = copy_bytes / (cw[copy_name] * 1024.0)
    lines = [f"Calibration ({copy_name}, {copy_bytes / 2**30:.2f} GiB read + written): FETCH_SIZE reads "
             f"{cf[copy_name]:.0f} KiB -> scale {f_scale:.3f}; WRITE_SIZE reads {cw[copy_name]:.0f} KiB -> scale "
             f"{w_scale:.3f}.", "",
             "| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM-side bytes per dispatch (scaled) |",
             "|---|---:|---:|---:|"]
    out = {"fetch_scale": f_scale, "write_scale": w_scale, "kernels": {}}
    for k in kernels_of_interest:
        if k not in f or k not in w:
            continue
        traffic = f[k] * 1024.0 * f_scale + w[k] * 1024.0 * w_scale
        out["kernels"][k] = {"fetch_kib": round(f[k], 1), "write_kib": round(w[k], 1), "traffic_bytes": int(traffic)}
        lines.append(f"| {k} | {f[k]:.0f} | {w[k]:.0f} | {traffic:,.0f} |")
    return "\n".join(lines), out


def _counter_means_by_name(path: str) -> dict:
    """{kernel: {counter: mean value per dispatch}} from a rocprofv3 counter_collection.csv holding several
    counters (one row per dispatch and counter)."""
    import collections
    import csv
    acc = collections.defaultdict(lambda: collections.defaultdict(list))
    for r in csv.DictReader(open(path)):
        acc[_short_kernel(r["Kernel_Name"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {k: {c: sum(v) / len(v) for c, v in d.items()} for k, d in acc.items()}


def _req_bytes(rd: dict, wr: dict):
    """(read bytes, write bytes) of one dispatch from the request-size counters: 32-, 64- and 128-byte reads
    (TCC_EA0_RDREQ counts every read request once), 32- and 64-byte writes."""
    n, n32, n128 = rd["TCC_EA0_RDREQ_sum"], rd["TCC_EA0_RDREQ_32B_sum"], rd["TCC_EA0_RDREQ_128B_sum"]
    read = 32 * n32 + 128 * n128 + 64 * (n - n32 - n128)
    w, w64 = wr["TCC_EA0_WRREQ_sum"], wr["TCC_EA0_WRREQ_64B_sum"]
    write = 64 * w64 + 32 * (w - w64)
    return read, write


def request_summary(read_csv, write_csv, copy_read_csv, copy_write_csv, copy_bytes, kernels_of_interest):
    """HBM-side (L2-to-fabric) bytes per dispatch summed by request size: reads = 32 x RDREQ_32B + 128 x
    RDREQ_128B + 64 x the rest, writes = 64 x WRREQ_64B + 32 x the rest. A plain copy of ``copy_bytes``
    (read and written) checks the sums; no scale factor is applied. Returns (markdown, dict)."""
    rd, wr = _counter_means_by_name(read_csv), _counter_means_by_name(write_csv)
    crd, cwr = _counter_means_by_name(copy_read_csv), _counter_means_by_name(copy_write_csv)
    copy_name = max(crd, key=lambda k: crd[k].get("TCC_EA0_RDREQ_sum", 0))
    c_read, c_write = _req_bytes(crd[copy_name], cwr[copy_name])
    lines = [f"Check ({copy_name}, {copy_bytes / 2**30:.2f} GiB read + written): the request-size sums read "
             f"{c_read / copy_bytes:.3f} x and write {c_write / copy_bytes:.3f} x the copied bytes.", "",
             "| kernel | read requests (32 B / 64 B / 128 B) | write requests (32 B / 64 B) | read bytes | "
             "write bytes | HBM-side bytes per dispatch |", "|---|---|---|---:|---:|---:|"]
    out = {"method": "request-size sums (TCC_EA0_RDREQ, _32B, _128B; TCC_EA0_WRREQ, _64B)",
           "copy_check": {"read": round(c_read / copy_bytes, 4), "write": round(c_write / copy_bytes, 4)},
           "kernels": {}}
    for k in kernels_of_interest:
        if k not in rd or k not in wr:
            continue
        r, w = rd[k], wr[k]
        rb, wb = _req_bytes(r, w)
        n32, n128 = r["TCC_EA0_RDREQ_32B_sum"], r["TCC_EA0_RDREQ_128B_sum"]
        n64 = r["TCC_EA0_RDREQ_sum"] - n32 - n128
        w64 = w["TCC_EA0_WRREQ_64B_sum"]
        out["kernels"][k] = {"read_bytes": int(rb), "write_bytes": int(wb), "traffic_bytes": int(rb + wb),
                             "rdreq_32b": int(n32), "rdreq_64b": int(n64), "rdreq_128b": int(n128),
                             "wrreq_32b": int(w["TCC_EA0_WRREQ_sum"] - w64), "wrreq_64b": int(w64)}
        lines.append(f"| {k} | {n32:,.0f} / {n64:,.0f} / {n128:,.0f} | {w['TCC_EA0_WRREQ_sum'] - w64:,.0f} / "
                     f"{w64:,.0f} | {rb:,.0f} | {wb:,.0f} | {rb + wb:,.0f} |")
    return "\n".join(lines), out


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--extra", default=None,
                    help="comma-separated configs measured after the main one and reported in the same JSON line "
                         "under extra_configs (default: c3,c4,c5 when --config is c2, else none; 'none' for none)")
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle timing")
    ap.add_argument("--chunk", type=int, default=None, help="split threshold (rows longer than this are split)")
    ap.add_argument("--item", type=int, default=None, help="entries per split item")
    ap.add_argument("--rocprof-summary", metavar="KERNEL_STATS_CSV",
                    help="print a markdown summary of a rocprofv3 kernel_stats.csv and exit")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "COPY_FETCH_CSV", "COPY_WRITE_CSV"),
                    help="summarise FETCH_SIZE/WRITE_SIZE counter runs (calibrated by a copy kernel) and exit")
    ap.add_argument("--req-summary", nargs=4, metavar=("READ_CSV", "WRITE_CSV", "COPY_READ_CSV", "COPY_WRITE_CSV"),
                    help="summarise request-size counter runs (TCC_EA0_RDREQ/_32B/_128B and TCC_EA0_WRREQ/_64B) "
                         "and exit")
    ap.add_argument("--copy-bytes", type=int, default=2 ** 30, help="bytes the calibration copy reads and writes")
    ap.add_argument("--pmc-json", help="with --pmc-summary / --req-summary: also write the per-kernel traffic here")
    args = ap.parse_args(argv)
    if args.rocprof_summary:
        print(rocprof_summary(args.rocprof_summary))
        return 0
    names = ["attn_fwd_kernel", "attn_bwd_q_kernel", "attn_bwd_kv_kernel", "attn_fwd_reduce_kernel",
             "attn_bwd_q_reduce_kernel", "attn_bwd_kv_reduce_kernel", "rw_select_reg_kernel", "rw_select_kernel",
             "real_select_fused_kernel", "row_block_sums_kernel", "row_ptr_kernel", "table_fill_kernel",
             "radix_count_kernel", "radix_scan_kernel", "radix_scatter_kernel", "unpack_rkey_kernel",
             "reverse_slots_kernel", "order_count_kernel", "order_place_kernel", "split_rows_kernel", "gather_probe_kernel",
             "rocprim"]
    if args.pmc_summary or args.req_summary:
        if args.pmc_summary:
            md, data = pmc_summary(*args.pmc_summary, args.copy_bytes, names)
        else:
            md, data = request_summary(*args.req_summary, args.copy_bytes, names)
        print(md)
        if args.pmc_json:
            with open(args.pmc_json, "w") as fh:
                json.dump(data, fh, indent=1)
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the path would shard "
              f"by query range (see the sharding design), but no multi-GPU figure is produced here.",
              file=sys.stderr)
        return 2

    import torch

    from budgetformer_amd import _native

    _native.load()
    chunk = args.chunk
    item = args.item
    result = run(args.config, args.steps, args.warmup, chunk, item, with_cpu=not args.no_cpu_baseline)
    extra = args.extra if args.extra is not None else ("c3,c4,c5" if args.config == "c2" else "none")
    extras = [c for c in extra.split(",") if c and c != "none"]
    records = []
    for name in extras:
        if name not in CONFIGS:
            raise SystemExit(f"bench.py: unknown config {name!r} in --extra")
        torch.cuda.empty_cache()
        rec = run(name, args.steps, args.warmup, chunk, item, with_cpu=not args.no_cpu_baseline)
        records.append({k: rec[k] for k in ("config", "dtype", "steps", "warmup", "warmup_steps_run", "ms_per_step",
                                            "value", "unit",
                                            "value_basis", "attn_fwd_bwd_ms", "edge_build_ms", "attention",
                                            "builder", "roofline", "gather_floor", "kernels", "cpu_baseline")
                        if k in rec})
    if records:
        result["extra_configs"] = records
    print(json.dumps(result), flush=True)
    return 0


def run(config, steps, warmup, chunk=None, item=None, with_cpu=True):
    """Measures one configuration; returns its result record."""
    import numpy as np
    import torch

    from budgetformer_amd import _native, hip_ops
    from budgetformer_amd.edges import build_attention_edges
    from budgetformer_amd.graph import CSRGraph, chung_lu_csr, chung_lu_device, uniform_random_csr

    cfg = CONFIGS[config]
    dev = torch.device("cuda:0")
    t_setup = time.time()
    n = cfg["n"]
    if cfg["kind"] == "device":
        g = chung_lu_device(n, cfg["e"], exponent=2.1, seed=42, max_degree=cfg.get("max_degree"), device=dev)
    else:
        if cfg["kind"] == "chung_lu":
            rowptr, col = chung_lu_csr(n, cfg["e"], exponent=2.1, seed=42)
        else:
            rowptr, col = uniform_random_csr(n, cfg["e"], seed=42)
        g = CSRGraph.from_csr(rowptr, col, n, device=dev)
    H, hn = cfg["H"], cfg["hn"]
    D = H * hn
    dt = getattr(torch, cfg["dtype"])
    s_bytes = torch.finfo(dt).bits // 8
    n_rows = cfg.get("n_q") or n                       # queries this GPU builds (a shard from node 0 at c5)
    S = n_rows + (1 if cfg["token"] else 0)            # attention query rows (+ the token row)
    S_kv = n + (1 if cfg["token"] else 0)              # key/value rows
    gq = torch.Generator(device=dev).manual_seed(43)
    q = torch.randn(S, H, hn, generator=gq, device=dev, dtype=torch.float32).to(dt)
    k, v = (torch.randn(S_kv, H, hn, generator=gq, device=dev, dtype=torch.float32).to(dt) for _ in range(2))
    dout = torch.randn(S, H, hn, generator=torch.Generator(device=dev).manual_seed(47), device=dev,
                       dtype=torch.float32).to(dt)
    torch.cuda.synchronize()
    # the walk records are a layout of the CSR (16 B per edge), built once per graph and cached on it like
    # the CSR itself: timed here, outside the per-step build
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    r0.record()
    from budgetformer_amd.gt_sp.utils import estimate_hot_path_bytes
    reserve = estimate_hot_path_bytes(n, g.num_edges, n_rows, cfg["b_r"], cfg["b_w"], global_token=cfg["token"])
    walk_rec = g.walk_records(reserve_bytes=reserve["peak"]) if cfg["b_w"] > 0 else None
    r1.record()
    torch.cuda.synchronize()
    rec_ms = round(r0.elapsed_time(r1), 4) if walk_rec is not None else None
    print(f"[bench] {cfg['name']}: realized E={g.num_edges:,}; setup {time.time() - t_setup:.1f}s", flush=True)

    chunk = chunk or hip_ops.DEFAULT_CHUNK
    item = item or hip_ops.DEFAULT_ITEM
    rate = cfg.get("dropout", 0.0)
    step_no = [0]

    def build():
        tab = build_attention_edges(g, real_edges_per_query=cfg["b_r"], rw_edges_per_query=cfg["b_w"],
                                    walk_length=cfg["L"], walks_per_node=cfg["P"], edge_seed=42, n_q=n_rows,
                                    global_token=cfg["token"])
        idx = tab.attention_index(chunk=chunk, item=item)
        # the dropout's keep bits are keyed by (query, slot): the reverse index then carries each entry's slot
        idx.ensure_backward(entries=bool(rate))
        return tab, idx

    def layer(idx):
        # training-mode GPS: a fresh Philox key per step, the same one for the forward and the backward
        step_no[0] += 1
        drop = hip_ops.Dropout(rate, seed=1000 + step_no[0]) if rate else None
        # as the attention modules do: the forward keeps the keep bits it draws and the dq pass reads them
        out, Z, keep = hip_ops.attn_forward(idx, q, k, v, dropout=drop, keep_mask=True)
        hip_ops.attn_backward(idx, q, k, v, None, Z, dout, dropout=drop, keep=keep)

    # W warmup steps, then more (at most 5) while the last one still grew the caching allocator: a step
    # that maps fresh device memory pays for its first touch (c5, whose steps hold about 184 GB, has taken
    # 0.7-2.2 s for the step that grows it), which is setup, not the step. The timed steps stay K.
    def device_allocs():
        return torch.cuda.memory_stats(dev).get("num_device_alloc", 0)

    warm, grew = 0, True
    while warm < warmup or (grew and warm < warmup + 5):
        n0 = device_allocs()
        tab, idx = build()
        layer(idx)
        torch.cuda.synchronize()
        grew = device_allocs() != n0
        warm += 1
    print(f"[bench] {config}: warmup {warm} steps done", flush=True)

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record()
        tab, idx = build()
        ev[i][1].record()
        layer(idx)
        ev[i][2].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # per-kernel durations from a separate pass of the same steps: the library's per-launch event
    # pairs cost host time, so they stay out of the timed loop above
    with _native.KernelTimer() as timer:
        for i in range(steps):
            tab, idx = build()
            layer(idx)
        torch.cuda.synchronize()
        kstats = timer.stats()
    build_ms = sum(a.elapsed_time(b) for a, b, _ in ev) / steps
    attn_ms = sum(b.elapsed_time(c) for _, b, c in ev) / steps
    step_ms = wall * 1e3 / steps
    print(f"[bench] {config}: timed {steps} steps: {step_ms:.3f} ms/step (build {build_ms:.3f}, attn fwd+bwd "
          f"{attn_ms:.3f})", flush=True)

    nnz = idx.nnz
    idx.resolve()                                      # plan counts for the report (after the timed loops)
    lens_q = np.diff(idx.qptr.cpu().numpy())
    lens_k = np.diff(idx.kptr.cpu().numpy())
    a_fwd, a_bwd = attention_bytes(s_bytes, D, H, S, S_kv, nnz)
    attn_gbs = (a_fwd + a_bwd) / (attn_ms * 1e-3) / 1e9
    comp = compulsory_bytes(s_bytes, D, H, S, S_kv, nnz, int((lens_k > 0).sum()))
    comp_gbs = comp / (attn_ms * 1e-3) / 1e9

    # per-kernel roofline of the three pass kernels
    n_rec = token_records(s_bytes, D, idx.n_q, idx.qplan.items) if idx.token_column else 0
    kv_var = hip_ops.kv_pass_variant(idx.n_q, idx.n_kv, dt, H, hn)
    # the dk/dv pass takes the token row's entries from a per-workgroup copy with several rows per group
    tok_row = int(lens_q[0]) if idx.token_column == 1 and kv_var["rows_per_group"] > 1 else 0
    lpr = 1
    while lpr < D * s_bytes // 16:
        lpr *= 2
    kv_blocks = -(-(-(-idx.n_kv // kv_var["rows_per_group"])) // (256 // lpr))
    kb = kernel_bytes(s_bytes, D, H, lens_q, lens_k, n_rec, entry_bytes=4 if rate else 0, token_row=tok_row,
                      chunk=chunk, kv_blocks=kv_blocks, keep_mask=bool(rate))
    kernels = {}
    for name, (ms, launches) in sorted(kstats.items(), key=lambda x: -x[1][0]):
        avg = ms / max(launches, 1)
        rec = {"avg_ms": round(avg, 5), "launches": launches}
        if name in kb:
            rec["algorithmic_bytes"] = kb[name]
            rec["achieved_gbs"] = round(kb[name] / (avg * 1e-3) / 1e9, 1)
        kernels[name] = rec
    dominant = max((n_ for n_ in kernels if n_ in kb), key=lambda n_: kernels[n_]["avg_ms"])
    dom = kernels[dominant]
    # counter traffic per dispatch (request-size sums of the committed profile of this config and dtype)
    prof, traffic_src = {}, None
    pmc_path = os.path.join(ROOT, "profiles", f"attention_{config}_{cfg['dtype']}_pmc.json")
    if os.path.exists(pmc_path) and chunk == hip_ops.DEFAULT_CHUNK and item == hip_ops.DEFAULT_ITEM:
        with open(pmc_path) as fh:
            prof = json.load(fh).get("kernels", {})
        traffic_src = os.path.relpath(pmc_path, ROOT)
    for name_, rec_ in kernels.items():
        if name_ in prof:
            rec_["traffic_bytes"] = prof[name_]["traffic_bytes"]
            rec_["traffic_gbs"] = round(prof[name_]["traffic_bytes"] / (rec_["avg_ms"] * 1e-3) / 1e9, 1)
    traffic = prof.get(dominant, {}).get("traffic_bytes")
    roofline = {"kernel": dominant, "bound": "hbm", "achieved": dom["achieved_gbs"], "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(dom["achieved_gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                "algorithmic_bytes": dom["algorithmic_bytes"], "traffic_source": traffic_src,
                "achieved_basis": "the kernel's algorithmic bytes (gather model) / its HIP-event average duration",
                "traffic_gbs": dom.get("traffic_gbs"),
                "traffic_frac": round(dom["traffic_gbs"] / HBM_PEAK_GBS, 4) if "traffic_gbs" in dom else None,
                "traffic_basis": "the kernel's L2-to-fabric bytes per dispatch (request-size counter sums) / its "
                                 "HIP-event average duration"}
    floor = gather_floor(idx, q, k, v, dout, H, s_bytes, D, kv_var, tok_row, chunk, kernels,
                         reps=max(3, min(steps, 10)))
    if dominant == "attn_bwd_kv_kernel":
        roofline["gather_floor_ms"] = floor["kv_pass"]["ms"]
        roofline["frac_of_gather_floor"] = round(floor["kv_pass"]["ms"] / dom["avg_ms"], 4)
        roofline["floor_ms"] = floor["kv_pass"]["attn_bwd_kv_kernel_floor_ms"]
        roofline["frac_of_floor"] = round(roofline["floor_ms"] / dom["avg_ms"], 4)
        roofline["floor_basis"] = "the pass's gathers alone plus its kv rows alone (k, v read, dK, dV written, " \
                                  "in its row order), each timed with a probe that only moves those bytes"
    # the layer's traffic: every attention kernel's counter bytes per dispatch times its launches per layer
    attn_kernels = [n_ for n_ in kernels if n_.startswith("attn_")]
    layer_traffic = None
    if attn_kernels and all(n_ in prof for n_ in attn_kernels):
        layer_traffic = sum(prof[n_]["traffic_bytes"] * kernels[n_]["launches"] / steps for n_ in attn_kernels)

    # edge-builder figures: RW pool edges = valid hop entries (d == 1, or the walk moved at step d)
    n_walks = n_rows * cfg["P"]
    pool_edges = 0
    for lo in range(0, n_rows, 4_000_000):             # count in slices to bound the walk tensor
        cnt = min(4_000_000, n_rows - lo)
        walks = hip_ops.random_walk(g.rowptr, g.col, lo, cnt, cfg["P"], cfg["L"], philox_seed=42)
        pool_edges += cnt * cfg["P"] + int((walks[:, 2:] != walks[:, 1:-1]).sum().item())
        del walks
    rw_ms = kernels.get("rw_select_kernel", {}).get("avg_ms")
    # real-edge top-k + merge: the fused light/heavy kernel, or the hub + group kernels
    merge_ms = sum(r["avg_ms"] for n_, r in kernels.items() if n_.startswith("real_select")) or None
    table_entries = int(tab.row_len.sum().item())

    if layer_traffic is not None:
        value = layer_traffic / (attn_ms * 1e-3) / 1e9
        basis = (f"attention layer fwd+bwd: the L2-to-memory-fabric bytes of its kernels per layer "
                 f"({layer_traffic / 1e9:.3f} GB: request-size counter sums per dispatch from {traffic_src}) / its "
                 f"HIP-event time; requests the 256 MB Infinity Cache serves count too. The gather-model work rate "
                 f"and the compulsory-byte rate are under attention.*")
    else:
        value = attn_gbs
        basis = ("attention layer fwd+bwd under the gather model (every gathered row counted at full size per "
                 "edge) / its HIP-event time: no counter profile of this configuration covers every attention "
                 "kernel; a work rate, not HBM bandwidth")
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "value_basis": basis,
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "warmup_steps_run": warm,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if dt == torch.float32 else "bf16",
        "data": "synthetic (seeded Chung-Lu graph and N(0,1) activations; no dataset)",
        "config": {"workload": cfg["name"], "num_nodes": n, "num_edges": g.num_edges, "queries": S,
                   "kv_rows": S_kv,
                   "table_entries": table_entries, "attention_edges": nnz, "heads": H, "head_dim": hn,
                   "walk_length": cfg["L"], "walks_per_node": cfg["P"], "budget": [cfg["b_r"], cfg["b_w"]],
                   "global_token": cfg["token"], "attention_dropout": rate, "split_chunk": chunk,
                   "split_item": item,
                   "split_plan": {"q_items": idx.qplan.items, "q_heavy": idx.qplan.heavy,
                                  "k_items": idx.kplan.items, "k_heavy": idx.kplan.heavy}},
        "attn_fwd_bwd_ms": round(attn_ms, 4),
        "edge_build_ms": round(build_ms, 4),
        "attention": {
            "fwd_bwd_ms": round(attn_ms, 4),
            "traffic_bytes": int(layer_traffic) if layer_traffic is not None else None,
            "traffic_gbs": round(layer_traffic / (attn_ms * 1e-3) / 1e9, 1) if layer_traffic is not None else None,
            "gather_model_bytes": a_fwd + a_bwd,
            "gather_model_gbs": round(attn_gbs, 1),
            "gather_model_frac_of_hbm_peak": round(attn_gbs / HBM_PEAK_GBS, 4),
            "compulsory_bytes": comp,
            "compulsory_gbs": round(comp_gbs, 1),
            "compulsory_frac_of_hbm_peak": round(comp_gbs / HBM_PEAK_GBS, 4),
        },
        "builder": {
            "edge_build_ms": round(build_ms, 4),
            "walk_records_once_ms": rec_ms,
            "walk_records_bytes": int(walk_rec.numel() * 4) if walk_rec is not None else 0,
            "rw_pool_edges": pool_edges,
            "rw_edges_per_s": round(pool_edges / (rw_ms * 1e-3), 1) if rw_ms else None,
            "rw_walk_steps_per_s": round(n_walks * cfg["L"] / (rw_ms * 1e-3), 1) if rw_ms else None,
            "rw_select_ms": rw_ms,
            "real_select_merge_ms": merge_ms,
            "table_entries": table_entries,
            "table_entries_per_s": round(table_entries / (build_ms * 1e-3), 1),
        },
        "roofline": roofline,
        "gather_floor": floor,
        "kernels": kernels,
    }

    if with_cpu:
        result["cpu_baseline"] = cpu_baseline(cfg, g, tab, idx, q, k, v, dout, s_bytes, D, H)
    del q, k, v, dout, tab, idx, g
    return result


def gather_floor(idx, q, k, v, dout, H, s_bytes, D, kv_var, tok_row, chunk, kernels, reps):
    """Each attention pass's memory floor: its gathers alone (bf_gather_probe) plus its own rows alone
    (bf_row_stream_probe), both timed on the pass's own ids, tables and order (HIP events on the library's
    stream, the mean over ``reps`` launches after one untimed launch):

    - key-major (dk/dv) pass: gathers, per reverse entry, of the q and dO rows of its query and the query's
      row-stats record ({1/D', Delta/D'} per head, 8·H bytes), non-temporal where the pass streams them
      (kv 0's segment left out when the dq pass sums the token column, and query 0's entries of the
      unsplit kv rows when the pass takes the token row from its per-workgroup copy); rows: every kv row
      in the pass's order (k_order), k and v read, dK and dV written;
    - query-major passes: gathers, per entry, of the k and v rows of its kv id; rows: the forward reads q
      and writes out, the dq pass reads q and dO and writes dq, in row order.

    The two parts are timed apart and added: each alone keeps HBM busy, so together they take about their
    sum. A pass also does its arithmetic and its small per-row records, so its time over its floor is at
    least about 1; near 1, the pass is as fast as its memory traffic can be served."""
    import torch

    from budgetformer_amd import _native as N
    from budgetformer_amd import hip_ops

    dev = q.device
    row = D * s_bytes
    stat = torch.zeros(idx.n_q, H, 2, dtype=torch.float32, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    kq = idx.kq
    if idx.token_column:
        kq = kq[int(idx.kptr[1].item()):]
    if tok_row:
        rows = hip_ops.expand_rows(idx.kptr, idx.nnz)
        if idx.token_column:
            rows = rows[int(idx.kptr[1].item()):]
        lens = idx.kptr[rows + 1] - idx.kptr[rows]
        kq = kq[(kq != 0) | (lens > chunk)]
        del rows, lens
    kq = kq.contiguous()
    kv = idx.kv.contiguous()
    st = hip_ops._stream(dev)

    def timed(launch):
        launch()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            launch()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    def gathers(t0, b0, t1, b1, t2, b2, ids, nt):
        return timed(lambda: N.call("bf_gather_probe", hip_ops._p(t0), b0, hip_ops._p(t1), b1, hip_ops._p(t2), b2,
                                    hip_ops._p(ids), ids.numel(), 0x7FFFFFFF, int(nt), hip_ops._p(sink), st))

    def streams(r0, r1, w0, w1, ids, n_rows, nt):
        return timed(lambda: N.call("bf_row_stream_probe", hip_ops._p(r0), hip_ops._p(r1), hip_ops._p(w0),
                                    hip_ops._p(w1), row, hip_ops._p(ids) if ids is not None else None, n_rows,
                                    int(nt), hip_ops._p(sink), st))

    kv_ms = gathers(q, row, dout, row, stat, 8 * H, kq, kv_var["stream_rows"])
    qp_ms = gathers(k, row, v, row, None, 0, kv, False)
    del stat
    # the rows each pass reads and writes once (outputs into scratch of the outputs' shapes)
    out_q = torch.empty_like(q)
    fwd_rows_ms = streams(q, None, out_q, None, None, idx.n_q, True)
    dq_rows_ms = streams(q, dout, out_q, None, None, idx.n_q, True)
    del out_q
    kv_order = idx.korder.contiguous()
    w_k, w_v = torch.empty_like(k), torch.empty_like(v)
    kv_rows_ms = streams(k, v, w_k, w_v, kv_order, idx.n_kv, False)
    del w_k, w_v
    out = {"basis": gather_floor.__doc__.split("\n\n")[0].replace("\n", " ").replace("    ", " ")}
    for key, ms, ids, per, rows_part in (
            ("kv_pass", kv_ms, kq, 2 * row + 8 * H,
             {"attn_bwd_kv_kernel": (kv_rows_ms, idx.n_kv, 4 * row)}),
            ("q_passes", qp_ms, kv, 2 * row,
             {"attn_fwd_kernel": (fwd_rows_ms, idx.n_q, 2 * row), "attn_bwd_q_kernel": (dq_rows_ms, idx.n_q, 3 * row)})):
        rec = {"ids": int(ids.numel()), "bytes_per_id": per, "ms": round(ms, 5),
               "record_gbs": round(ids.numel() * per / (ms * 1e-3) / 1e9, 1)}
        for name, (rows_ms, n_rows, row_bytes) in rows_part.items():
            floor_ms = ms + rows_ms
            rec[f"{name}_rows"] = {"rows": int(n_rows), "bytes_per_row": row_bytes, "ms": round(rows_ms, 5),
                                   "gbs": round(n_rows * row_bytes / (rows_ms * 1e-3) / 1e9, 1)}
            rec[f"{name}_floor_ms"] = round(floor_ms, 5)
            if name in kernels:
                rec[f"{name}_over_gathers"] = round(kernels[name]["avg_ms"] / ms, 3)
                rec[f"{name}_over_floor"] = round(kernels[name]["avg_ms"] / floor_ms, 3)
        out[key] = rec
    return out


def cpu_baseline(cfg, g, tab, idx, q, k, v, dout, s_bytes, D, H):
    """The CPU oracle (the reference algorithm restated in torch/numpy) on this host's cores.

    Small configs run the whole workload. Large ones (``cpu_sample`` set) run a
    contiguous range of ``cpu_sample`` queries whose mean in-degree equals the
    workload's (the power-law graphs put their hubs at the lowest ids, so a range
    from node 0 would be mostly hubs):
    - attention: the range's attention rows (their edges, the touched K/V rows
      relabelled; never the Graphormer token's own row), time scaled by the
      attention entries, all rows' over the sample's;
    - edge build: the oracle build of the range, modelled as a fixed part (a
      one-query build: the oracle's passes over the whole edge list) plus a
      per-query part scaled linearly to the workload's queries.
    GraphGPS configs with dropout time the GPS form with a drawn keep mask.
    """
    import numpy as np
    import torch

    from oracle import edge_table as et
    from oracle import philox
    from oracle import sparse_attention as sa

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    n = cfg["n"]
    n_rows = cfg.get("n_q") or n
    sample = min(cfg.get("cpu_sample") or n_rows, n_rows)
    whole = sample == n_rows
    tok = 1 if cfg["token"] else 0
    q0 = 0
    if not whole:
        # the contiguous range of `sample` queries whose mean in-degree is closest to the workload's
        deg = (g.in_ptr[1:n_rows + 1] - g.in_ptr[:n_rows]).double()
        csum = torch.cat([torch.zeros(1, dtype=torch.float64, device=deg.device), deg.cumsum(0)])
        target = float(csum[-1]) / n_rows
        starts = torch.arange(0, n_rows - sample + 1, max(1, (n_rows - sample) // 512), device=deg.device)
        means = (csum[starts + sample] - csum[starts]) / sample
        q0 = int(starts[int(torch.argmin((means - target).abs()))])
    # attention rows of those queries (query x is attention row x + tok); the whole workload adds the token row
    r_lo = 0 if whole else q0 + tok
    r_hi = n_rows + tok if whole else q0 + tok + sample
    e_lo, e_hi = int(idx.qptr[r_lo].item()), int(idx.qptr[r_hi].item())
    attn_scale = idx.nnz / max(e_hi - e_lo, 1)
    print(f"[bench] cpu baseline: attention of rows {r_lo:,}..{r_hi - 1:,} ({e_hi - e_lo:,} entries) on "
          f"{threads} threads", flush=True)
    rows = idx.entry_rows()[e_lo:e_hi].cpu() - r_lo
    kv = idx.kv[e_lo:e_hi].cpu().long()
    uniq, inv = torch.unique(kv, return_inverse=True)
    ei = torch.stack([inv, rows])
    # the oracle (like the reference) indexes queries and kv rows in one node space: pad both to M rows
    M = max(r_hi - r_lo, uniq.numel())

    def padded(t):
        out = torch.zeros(M, *t.shape[1:], dtype=torch.float32)
        out[: t.shape[0]] = t.float().cpu()
        return out

    qc, dc = padded(q[r_lo:r_hi]), padded(dout[r_lo:r_hi])
    kc, vc = padded(k[uniq.to(k.device)]), padded(v[uniq.to(v.device)])
    rate = cfg.get("dropout", 0.0)
    keep = torch.rand(ei.shape[1], H, generator=torch.Generator().manual_seed(5)) >= rate if rate else None

    def attention_step():
        if not rate:
            sa.attention_fwd_bwd_autograd(kc, qc, vc, ei, dc)
            return
        kk, qq, vv = (t.detach().requires_grad_(True) for t in (kc, qc, vc))
        sa.gps_sparse_attention(qq, kk, vv, ei, keep, 1.0 / (1.0 - rate)).backward(dc)

    times = []
    t_all = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        attention_step()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_all > 12.0 or len(times) >= 3:
            break
    attn_s = min(times) * attn_scale
    nnz = idx.nnz
    a_fwd, a_bwd = attention_bytes(s_bytes, D, H, idx.n_q, idx.n_kv, nnz)
    # edge build of the same queries
    rowptr = g.rowptr.cpu().numpy()
    col = g.col.cpu().numpy()
    P, L = cfg["P"], cfg["L"]

    def build(lo, cnt):
        u = philox.walk_uniforms(lo, cnt, P, L, 42)
        t0 = time.perf_counter()
        et.build_edge_table(rowptr, col, n, cfg["b_r"], cfg["b_w"], L, P, 42, u, q_lo=lo, n_q=cnt)
        return time.perf_counter() - t0

    print(f"[bench] cpu baseline: edge build of queries {q0:,}..{q0 + sample - 1:,}", flush=True)
    t_s = build(q0, sample)
    if whole:
        build_s = t_s
        what = "the full workload"
    else:
        print("[bench] cpu baseline: edge build of one query (the fixed part)", flush=True)
        t_1 = build(q0, 1)
        per_query = max(t_s - t_1, 0.0) / max(sample - 1, 1)
        build_s = t_1 + per_query * (n_rows - 1)
        what = (f"queries {q0:,}..{q0 + sample - 1:,} of {n_rows:,} (the range whose mean in-degree is the "
                f"workload's): attention {e_hi - e_lo:,} of {nnz:,} entries, time scaled x{attn_scale:.2f} by "
                f"entries; edge build {t_s:.2f} s for the range = a fixed {t_1:.2f} s (a one-query build) + "
                f"{per_query * 1e6:.1f} us per query, scaled to {n_rows:,} queries")
    print(f"[bench] cpu baseline: attn fwd+bwd {attn_s * 1e3:.1f} ms, edge build {build_s * 1e3:.1f} ms "
          f"({threads} threads; {what})", flush=True)
    return {
        "value": round((a_fwd + a_bwd) / attn_s / 1e9, 2),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{cfg['name'].split(':')[0]}, {what}: attention fwd+bwd (torch CPU autograd, fp32, best "
                  f"of {len(times)}{', GPS form with a keep mask' if rate else ''}) and the numpy edge build",
        "attn_fwd_bwd_ms": round(attn_s * 1e3, 2),
        "edge_build_ms": round(build_s * 1e3, 2),
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


if __name__ == "__main__":
    sys.exit(main())
