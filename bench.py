#!/usr/bin/env python3
"""Benchmark of the query-indexing hot path on one MI355X.

A step is one pass of the path over one batch of synthetic input (seeded
PCG64, resident in HBM before timing starts).  Workloads (--config):

  4 (default)  prefill indexer chunk: 4096 queries x 64 heads x 128 FP8 against a
               32768-token paged FP8 context, causal -> exact Top-2048 with page-table
               slot mapping -> 656-byte latent-row gather into a reused workspace
  1            the reference example shape: 1024 queries x 1 head; coarse score over
               centers -> route (40 of 64 pages, fine table) -> shared tail staging ->
               fine score over 2688 candidates -> fused Top-2048 with mask -> C4 x4
               expansion (the unfused fallback) -> gather
  2            page management: 4096 requests (~132 K Zipf page keys) -> stable key grouping,
               match -> allocate -> publish into a 65536-page pool of 41984-byte pages,
               128-token tail staging for owner pairs, release of half the requests
  3            K/V slot gather: 1024 x 2048 ids (5% padding) through per-query
               512-page windows of a 1M-token pool of 656-byte rows
  5            decode batch: 128 requests x 64 heads, contexts 4K..128K tokens with
               their own page tables in a 2M-token pool, through the V1 route path: center
               score -> route (page_fraction 0.5) -> fine table -> tail staging -> fine
               score -> mask -> Top-2048 -> raw/logical/physical map -> gather (the
               full-scoring chain over every context key timed beside it)
  6            index build: every 1024-token bucket of a 2M-token FP8 pool (2048 buckets)
               -> member order, reordered pages and FP8 centers, one launch
  8            attention consumer: 4096 queries x 4 heads of one KV head, 2048 gathered bf16
               K/V slots each (1M-slot pool) -> decode attention
  10           context timings, microseconds per call under HIP graph replay: _sort of one
               1024-token bucket at group sizes 1024 .. 16, and the per-lease page manager
               (fingerprint, match_pages miss / hit / collision at a 4096-page pool, publish
               all-new / mixed / reuse), set up as the reference's own micro-benchmark
  7            shared sink+tail chunk: 64K published tokens, 4096 causal queries x 32 heads,
               sink 64 / window 2048, 40 history pages per query: one union of sink+tail
               pages -> FP8 score -> canonical order -> Top-2048 -> slots (per-row staging
               of the same candidates timed beside it)

Prints one JSON line: queries/sec, per-stage times, the roofline of the
dominant kernel and the CPU baseline (the reference's torch expressions on
the host cores, on a bounded sample of the same workload).  With the default
config 4 the line also carries "configs": configs 1, 2, 3, 5, 7 and 9 measured
the same way at their own shapes (--with selects others, "" none), each with its
rate, step time, stage times, dominant-kernel roofline and a shorter CPU
sample (--with-cpu-budget seconds).
"""
import argparse
import importlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0
PEAK_FP8_TFLOPS = 5000.0
# HBM traffic per dispatch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (calibrated against a
# plain copy), kept with the kernel trace of the same workload.
TRAFFIC = {
    4: (ROOT / "profiles" / "prefill_chunk_4096x32k.md",
        {"score": ("score_prep", "score_shared", "score_exact"), "topk": ("transform_rows",), "gather": ("gather_rows16",)}),
    3: (ROOT / "profiles" / "slot_gather_1024x2048.md", {"gather": ("gather_rows16",)}),
    6: (ROOT / "profiles" / "index_build_2048x1024.md", {"build": ("build_buckets_kernel",)}),
    2: (ROOT / "profiles" / "page_management_4096req.md",
        {"insert": ("pb_init", "pb_hash", "pb_classify", "pb_slow_live", "pb_slow", "pb_allocate", "pb_table",
                    "pb_publish", "pb_commit")}),
}


def measured_traffic(config, stage):
    """HBM bytes per step of a stage's kernels from the committed counter
    summary, or None when it does not list them (the insert's two small
    prefix-sum kernels, under 1 MB, are left out)."""
    if config not in TRAFFIC:
        return None
    path, stages = TRAFFIC[config]
    if stage not in stages or not path.exists():
        return None
    per_kernel, cols = {}, None
    for line in path.read_text().splitlines():
        cells = [c.strip().strip("`") for c in line.strip().strip("|").split("|")]
        if cols is None:
            if any(c.startswith("HBM read bytes") for c in cells):
                cols = ([i for i, c in enumerate(cells) if c.startswith("HBM read bytes")][0],
                        [i for i, c in enumerate(cells) if c.startswith("HBM write bytes")][0])
            continue
        if len(cells) <= max(cols) or not cells[0] or cells[0].startswith("-"):
            if not line.strip():
                cols = None
            continue
        try:
            per_kernel[cells[0].split("<")[0]] = float(cells[cols[0]]) + float(cells[cols[1]])
        except ValueError:
            continue
    vals = [per_kernel.get(k) for k in stages[stage]]
    return None if any(v is None for v in vals) else sum(vals)


def cpu_model():
    """The host processor's model name, as the kernel reports it."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=4, choices=[1, 2, 3, 4, 5, 6, 7, 8, 9, 10])
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline work (0 = skip)")
    ap.add_argument("--with", dest="with_configs", default=None, metavar="LIST",
                    help="comma-separated further configs measured after the main one and reported under "
                         "\"configs\" (default with config 4: 1,2,3,5,7,9; \"\" for none)")
    ap.add_argument("--with-cpu-budget", type=float, default=3.0,
                    help="seconds of CPU baseline work per further config")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES bytes (HBM counter calibration) and exit")
    return ap.parse_args()


def copy_calibration(nbytes):
    """A plain copy kernel of known size: its FETCH_SIZE / WRITE_SIZE counters
    give the scale between the counters and bytes moved."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "launches": 3}), flush=True)


class Pkg:
    def __init__(self):
        for name in ("workloads", "scoring", "topk", "native_kernels", "query_fused", "kernels", "pagepool",
                     "indexbuild", "tailunion", "attention"):
            setattr(self, name, importlib.import_module(f"10_20_amd.{name}"))


def _score_flops(heads, lens):
    return 2.0 * heads * 128 * float(lens.astype("int64").sum())


# MI355X last-level (Infinity) cache
LLC_BYTES = 256 << 20


def _gather_gb(torch, slots, row_bytes, pool_rows):
    """Algorithmic HBM bytes of a row gather: every workspace row written once
    and every id read once, plus the source rows: when the source pool fits
    in the last-level cache each distinct row is fetched from HBM once (the
    other reads of it are cache hits), otherwise every valid id costs one row
    read.  Counted from the slot map after the run."""
    ids = slots.reshape(-1)
    valid = ids[(ids >= 0) & (ids < pool_rows)]
    reads = int(torch.unique(valid).numel()) if pool_rows * row_bytes <= LLC_BYTES else int(valid.numel())
    return (row_bytes * ids.numel() + 4.0 * ids.numel() + row_bytes * reads) / 1e9


def setup_prefill(P, dev, torch, np):
    """Configuration 4: prefill indexer chunk."""
    wl = P.workloads.config4()
    a, prm = wl.arrays, wl.params
    rows, heads, T, row_bytes, ctx = prm["rows"], prm["heads"], prm["topk"], prm["row_bytes"], prm["ctx"]
    q = torch.from_numpy(a["q8"]).to(dev).view(torch.float8_e4m3fn)
    w = torch.from_numpy(a["w"]).to(dev)
    native = torch.from_numpy(a["native"]).to(dev)
    table = torch.from_numpy(a["table"]).to(dev)
    shared_table = table[None].expand(rows, -1)
    dense_table = shared_table.contiguous()
    lens = torch.from_numpy(a["lens"]).to(dev)
    latent = torch.from_numpy(a["latent"]).to(dev)
    logits = torch.empty((rows, ctx), device=dev, dtype=torch.float32)
    slots = torch.empty((rows, T), device=dev, dtype=torch.int32)
    raw = torch.empty_like(slots)
    work = torch.empty((rows, T, row_bytes), device=dev, dtype=torch.uint8)
    stages = [
        ("score", lambda: P.scoring.fp8_paged_mqa_logits(q, native, w, lens, shared_table, None, ctx,
                                                          clean_logits=False, out=logits)),
        ("topk", lambda: P.topk.topk_transform_512_v2(logits, lens, dense_table, slots, 64, None, raw)),
        ("gather", lambda: P.native_kernels.gather_rows(latent, slots, work)),
    ]
    L = a["lens"].astype(np.int64)
    work_units = {
        "score": (_score_flops(heads, L) / 1e12, "TFLOP/s", PEAK_FP8_TFLOPS, "mfma"),
        "topk": ((4.0 * L.sum() + 8.0 * rows * T) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "gather": (lambda: _gather_gb(torch, slots, row_bytes, latent.shape[0]), "GB/s", PEAK_HBM_GBS, "hbm"),
    }

    def cpu(budget):
        from oracle import cpu_baseline
        qps, n, threads = cpu_baseline.prefill_queries_per_second(a["q8"], a["w"], a["native"], a["table"],
                                                                  a["lens"], a["latent"], T, budget)
        return qps, threads, f"{n} of {rows} queries (score+top2048+slot map+gather)"

    meta = {"workload": "prefill indexer chunk: 4096 queries x 64 heads x 128 FP8 vs 32768-token paged FP8 "
                        "context, causal, Top-2048, 656-byte latent row gather",
            "global_batch": rows, "seq_len": ctx, "parallelism": "single GPU"}
    return rows, stages, work_units, cpu, meta, "synthetic (PCG64 seed 4)"


def setup_example(P, dev, torch, np):
    """Configuration 1: the reference example's query chain."""
    wl = P.workloads.config1()
    a, prm = wl.arrays, wl.params
    B, PG, CAP, TAKE, WIDTH, T = prm["B"], prm["P"], prm["CAP"], prm["TAKE"], prm["WIDTH"], prm["TOPK"]
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in a.items()}
    q = d["q8"].view(torch.float8_e4m3fn)
    center_lens = torch.full((B,), 512, device=dev, dtype=torch.int32)
    ctab = d["center_table"][None].expand(B, -1)
    coarse = torch.empty((B, PG * 8), device=dev)
    sel = torch.empty((B, TAKE), device=dev, dtype=torch.int32)
    ft = torch.empty((B, prm["FT_COLS"]), device=dev, dtype=torch.int32)
    logits = torch.empty((B, WIDTH), device=dev)
    physical = torch.empty((B, T), device=dev, dtype=torch.int32)
    logical = torch.empty_like(physical)
    raw = torch.empty_like(physical)
    no_exp = torch.empty_strided((B, 0), (0, 1), device=dev, dtype=torch.int32)
    expanded = torch.empty((B, 4 * T + 64), device=dev, dtype=torch.int32)  # C4 indices (x4 per token)
    work = torch.empty((B, T, P.workloads.MLA_ROW_BYTES), device=dev, dtype=torch.uint8)
    fused = P.query_fused.module()
    stages = [
        ("coarse", lambda: P.scoring.fp8_paged_mqa_logits(q, d["centers"], d["w"], center_lens, ctab, None, PG * 8,
                                                           clean_logits=True, out=coarse)),
        ("route", lambda: fused.route(coarse, d["lens"], d["takes"], sel, PG, d["rt"], ft, d["tail_rows"], CAP, True)),
        ("stage", lambda: P.kernels.stage_tail_shared[(-(-B // 32), 68)](
            d["native"], None, d["nt"], d["lens"], d["fine"], None, d["tail_rows"], CAP, PG, 68, prm["SINK"],
            prm["WINDOW"], ROWS=B, GROUP=32)),
        ("score", lambda: P.scoring.fp8_paged_mqa_logits(q, d["fine"], d["w"], d["fine_lens"], ft, None, WIDTH,
                                                          clean_logits=True, out=logits)),
        ("topk", lambda: fused.topk(logits, d["fine_lens"], d["members"], d["rt"], d["nt"], sel, d["lens"],
                                    d["takes"], physical, logical, raw, prm["WINDOW"], True, no_exp, True, True, ft,
                                    False)),
        ("expand", lambda: P.kernels.expand_logical[(B,)](logical, expanded, T, expanded.shape[1],
                                                          1 << (expanded.shape[1] - 1).bit_length())),
        ("gather", lambda: P.native_kernels.gather_rows(d["latent"], physical, work)),
    ]
    fl = a["fine_lens"].astype(np.int64)
    rb = P.workloads.MLA_ROW_BYTES
    work_units = {
        "coarse": (_score_flops(1, np.full(B, 512)) / 1e12, "TFLOP/s", PEAK_FP8_TFLOPS, "mfma"),
        "route": ((32.0 * 64 * B + 4.0 * B * (TAKE + prm["FT_COLS"])) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "stage": (2.0 * 2 * 8448 / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "score": (_score_flops(1, fl) / 1e12, "TFLOP/s", PEAK_FP8_TFLOPS, "mfma"),
        "topk": ((4.0 * fl.sum() + 12.0 * B * T) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "expand": ((4.0 * B * T + 4.0 * expanded.numel()) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "gather": (lambda: _gather_gb(torch, physical, rb, d["latent"].shape[0]), "GB/s", PEAK_HBM_GBS, "hbm"),
    }

    def cpu(budget):
        from oracle import cpu_baseline
        qps, n, threads = cpu_baseline.example_queries_per_second(a, prm, budget)
        return qps, threads, f"{n} of {B} queries (score over the 2688 candidates + top2048 + slot map + gather)"

    meta = {"workload": "reference example query chain: 1024 queries x 1 head, route 40 of 64 pages, "
                        "2688 candidates, fused Top-2048 with mask, unfused C4 x4 expansion, 656-byte row gather",
            "global_batch": B, "seq_len": WIDTH, "parallelism": "single GPU"}
    return B, stages, work_units, cpu, meta, "synthetic (PCG64 seed 19)"


def setup_whole(P, dev, torch, np):
    """Configuration 9: the reference's published whole-query shape (coarse
    score + route + fine score + fused Top-K + x4 at 1024 queries and 64K
    context, sglang/srt/layers/attention/v1_deepseek/README.txt:117) on
    synthetic data with the runtime's default geometry; no gather."""
    wl = P.workloads.config9()
    a, prm = wl.arrays, wl.params
    B, PG, CAP, TAKE, WIDTH, T = prm["B"], prm["P"], prm["CAP"], prm["TAKE"], prm["WIDTH"], prm["TOPK"]
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in a.items() if k != "latent"}
    q = d["q8"].view(torch.float8_e4m3fn)
    center_lens = torch.full((B,), prm["CENTERS"], device=dev, dtype=torch.int32)
    ctab = d["center_table"][None].expand(B, -1)
    coarse = torch.empty((B, PG * 8), device=dev)
    sel = torch.empty((B, TAKE), device=dev, dtype=torch.int32)
    ft = torch.empty((B, prm["FT_COLS"]), device=dev, dtype=torch.int32)
    logits = torch.empty((B, WIDTH), device=dev)
    physical = torch.empty((B, T), device=dev, dtype=torch.int32)
    logical = torch.empty_like(physical)
    raw = torch.empty_like(physical)
    no_exp = torch.empty_strided((B, 0), (0, 1), device=dev, dtype=torch.int32)
    expanded = torch.empty((B, 4 * T + 64), device=dev, dtype=torch.int32)
    fused = P.query_fused.module()
    stages = [
        ("coarse", lambda: P.scoring.fp8_paged_mqa_logits(q, d["centers"], d["w"], center_lens, ctab, None, PG * 8,
                                                           clean_logits=True, out=coarse)),
        ("route", lambda: fused.route(coarse, d["lens"], d["takes"], sel, PG, d["rt"], ft, d["tail_rows"], CAP, True)),
        ("stage", lambda: P.kernels.stage_tail_shared[(-(-B // 32), 68)](
            d["native"], None, d["nt"], d["lens"], d["fine"], None, d["tail_rows"], CAP, PG, 68, prm["SINK"],
            prm["WINDOW"], ROWS=B, GROUP=32)),
        ("score", lambda: P.scoring.fp8_paged_mqa_logits(q, d["fine"], d["w"], d["fine_lens"], ft, None, WIDTH,
                                                          clean_logits=True, out=logits)),
        ("topk", lambda: fused.topk(logits, d["fine_lens"], d["members"], d["rt"], d["nt"], sel, d["lens"],
                                    d["takes"], physical, logical, raw, prm["WINDOW"], True, no_exp, True, True, ft,
                                    False)),
        ("expand", lambda: P.kernels.expand_logical[(B,)](logical, expanded, T, expanded.shape[1],
                                                          1 << (expanded.shape[1] - 1).bit_length())),
    ]
    fl = a["fine_lens"].astype(np.int64)
    H = prm["H"]
    tail_bytes = 2.0 * (prm["SINK"] + prm["WINDOW"]) / 64 * 8448
    work_units = {
        "coarse": (_score_flops(H, np.full(B, prm["CENTERS"])) / 1e12, "TFLOP/s", PEAK_FP8_TFLOPS, "mfma"),
        "route": ((32.0 * prm["BUILT"] * B + 4.0 * B * (TAKE + prm["FT_COLS"])) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "stage": (tail_bytes / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "score": (_score_flops(H, fl) / 1e12, "TFLOP/s", PEAK_FP8_TFLOPS, "mfma"),
        "topk": ((4.0 * fl.sum() + 12.0 * B * T) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "expand": ((4.0 * B * T + 4.0 * expanded.numel()) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
    }

    def cpu(budget):
        from oracle import cpu_baseline
        qps, n, threads = cpu_baseline.whole_query_queries_per_second(a, prm, budget)
        return qps, threads, f"{n} of {B} queries (64-head coarse and fine scores, route, Top-2048, x4 positions)"

    meta = {"workload": "whole V1 query at the reference's published shape: 1024 queries x 64 heads FP8, 64K-token "
                        "context in 64 built 1K buckets, coarse score over 8192 centers, route 512 of 1024 pages "
                        "(page_fraction 0.5), sink 64 + window 2048, 34880 fine candidates, fused Top-2048 with "
                        "mask, x4 expansion (no gather)",
            "global_batch": B, "seq_len": WIDTH, "parallelism": "single GPU"}
    return B, stages, work_units, cpu, meta, "synthetic (PCG64 seed 9)"


def setup_gather(P, dev, torch, np):
    """Configuration 3: K/V slot gather."""
    wl = P.workloads.config3()
    a, prm = wl.arrays, wl.params
    rows, T, rb = prm["rows"], prm["top"], prm["row_bytes"]
    pool = torch.from_numpy(a["pool"]).to(dev)
    table = torch.from_numpy(a["table"]).to(dev)
    ids = torch.from_numpy(a["ids"]).to(dev)
    work = torch.empty((rows, T, rb), device=dev, dtype=torch.uint8)
    stages = [("gather", lambda: P.native_kernels.gather_rows(pool, ids, work, table=table, page_bits=6))]
    # ids are logical token positions through per-query page tables (8 B per slot: the id and its
    # table entry); the 688 MB pool is far above the last-level cache, so every valid id is a row read
    valid = int((a["ids"] >= 0).sum())
    work_units = {"gather": ((rb * valid + rb * rows * T + 8.0 * rows * T) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm")}

    def cpu(budget):
        from oracle import cpu_baseline
        qps, n, threads = cpu_baseline.gather_queries_per_second(a["pool"], a["ids"], a["table"], budget)
        return qps, threads, f"{n} of {rows} queries (2048-slot gather)"

    meta = {"workload": "K/V slot gather: 1024 queries x 2048 slots (5% padding) from a 1M-token pool of "
                        "656-byte rows through per-query 512-page windows",
            "global_batch": rows, "seq_len": T, "parallelism": "single GPU"}
    return rows, stages, work_units, cpu, meta, "synthetic (PCG64 seed 3)"


def setup_decode(P, dev, torch, np):
    """Configuration 5: decode batch through the V1 route path
    (runtime.py:417-634): center score -> route with the fine-table fill ->
    stage_tail_shared -> fine score -> fused Top-2048 (sink/tail mask in the
    segment pass, raw -> logical -> physical map in the merge) -> gather.
    Beside it: the reference's own order for <= 512 rows (fine_table_shared,
    then mask_fine -> topk_transform_512_v2 -> output_ids as separate
    kernels; the same outputs) and the full-scoring chain over every context
    key (score -> Top-2048 -> gather)."""
    wl = P.workloads.config5_route()
    a, prm = wl.arrays, wl.params
    rows, heads, T, rb = prm["rows"], prm["heads"], prm["topk"], prm["row_bytes"]
    PG, CAP, TAKE, WIDTH, FP, SINK, WIN = prm["P"], prm["CAP"], prm["TAKE"], prm["WIDTH"], prm["FP"], prm["sink"], \
        prm["window"]
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in a.items()}
    q = d["q8"].view(torch.float8_e4m3fn)
    i32 = lambda *sh: torch.empty(sh, device=dev, dtype=torch.int32)
    fl, takes, dg_lens, center_lens, tail_rows = i32(rows), i32(rows), i32(rows), i32(rows), i32(rows)
    P.kernels.query_metadata[(rows,)](d["lens"], d["nt"], fl, takes, dg_lens, center_lens, tail_rows, PG, T,
                                      prm["num"], prm["den"], SINK, WIN)
    coarse = torch.empty((rows, PG * 8), device=dev)
    sel, ft = i32(rows, TAKE), i32(rows, FP)
    scores = torch.empty((rows, WIDTH), device=dev)
    ident = torch.arange(FP, device=dev, dtype=torch.int32)[None].expand(rows, -1)
    transformed, raw, out, logical = i32(rows, T), i32(rows, T), i32(rows, T), i32(rows, T)
    # 656-byte latent rows of the 2M-token pool: byte c of row i = (131 i + 7 c) mod 256
    row_term = ((torch.arange(prm["latent_rows"], device=dev, dtype=torch.int64) * 131) & 255).to(torch.uint8)
    latent = row_term[:, None] + ((torch.arange(rb, device=dev, dtype=torch.int64) * 7) & 255).to(torch.uint8)[None]
    work = torch.empty((rows, T, rb), device=dev, dtype=torch.uint8)
    fused = P.query_fused.module()
    K = P.kernels
    no_exp = torch.empty((rows, 0), device=dev, dtype=torch.int32)
    stages = [
        ("coarse", lambda: P.scoring.fp8_paged_mqa_logits(q, d["centers"], d["w"], center_lens, d["center_table"],
                                                           None, PG * 8, clean_logits=True, out=coarse)),
        ("route", lambda: fused.route(coarse, d["lens"], takes, sel, PG, d["rt"], ft, tail_rows, CAP, True)),
        ("stage", lambda: K.stage_tail_shared[(rows, 68)](d["native"], None, d["nt"], d["lens"], d["fine"], None,
                                                          tail_rows, CAP, PG, 68, SINK, WIN, ROWS=rows, GROUP=1)),
        ("score", lambda: P.scoring.fp8_paged_mqa_logits(q, d["fine"], d["w"], dg_lens, ft, None, WIDTH,
                                                          clean_logits=True, out=scores)),
        ("topk", lambda: P.query_fused.topk_any_batch(scores, fl, d["members"], d["rt"], d["nt"], sel, d["lens"],
                                                      takes, out, logical, raw, WIN, True, no_exp, True, False, ft,
                                                      False)),
        ("gather", lambda: P.native_kernels.gather_rows(latent, out, work)),
    ]

    def unfused_chain():
        # the reference's order for <= 512 rows (runtime.py:445-448, 478-509, 538-563, 603-634)
        stages[0][1]()
        fused.route(coarse, d["lens"], takes, sel, PG, d["rt"], ft, tail_rows, CAP, False)
        K.fine_table_shared[(rows,)](d["rt"], sel, takes, d["lens"], ft, tail_rows, CAP, PG, TAKE, FP, 68,
                                     1 << (FP - 1).bit_length())
        stages[2][1]()
        stages[3][1]()
        K.mask_fine[(rows, -(-WIDTH // 256))](scores, sel, d["rt"], d["members"], d["lens"], takes, PG, TAKE, WIDTH,
                                              WIDTH, SINK, WIN)
        P.topk.topk_transform_512_v2(scores, fl, ident, transformed, 64, None, raw)
        K.output_ids[(rows, -(-T // 256))](raw, scores, d["members"], d["rt"], d["nt"], sel, d["lens"], takes, out,
                                           logical, ft, PG, PG, TAKE, WIDTH, T, SINK, WIN, MAP_PHYSICAL=True,
                                           DIRECT_FINE=False, FP=FP)
        stages[5][1]()
    meta_h = [x.cpu().numpy().astype(np.int64) for x in (fl, takes, center_lens, tail_rows)]
    F, TK_, CL, owners = meta_h[0], meta_h[1], meta_h[2], meta_h[3]
    n = a["lens"].astype(np.int64)
    built = np.maximum(n - 1, 0) // 1024 * 16
    sink = np.minimum(n, SINK)
    tail = np.maximum(sink, np.minimum(np.maximum(n - 1, 0) // 1024 * 1024, np.maximum(sink, n - WIN)))
    staged_pages = np.where(owners == np.arange(rows), np.maximum(1, -(-(sink + n - tail) // 64)), 0)
    work_units = {
        # HBM-bound stages: algorithmic bytes from the per-row lengths
        "coarse": ((132.0 * CL.sum() + rows * heads * 132.0 + 4.0 * rows * PG * 8) / 1e9, "GB/s", PEAK_HBM_GBS,
                   "hbm"),
        # route: center maxima read, selected ranks and the fine table written
        "route": ((32.0 * built.sum() + 4.0 * rows * TAKE + 4.0 * rows * FP) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "stage": ((2.0 * 8448 * staged_pages.sum()) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "score": ((132.0 * F.sum() + rows * heads * 132.0 + 4.0 * rows * WIDTH) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        # Top-K: every candidate read once, three output arrays written (the
        # map's table and member reads ride along, 4 B each per output)
        "topk": ((4.0 * F.sum() + 12.0 * rows * T + 12.0 * rows * T) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "gather": (lambda: _gather_gb(torch, out, rb, latent.shape[0]), "GB/s", PEAK_HBM_GBS, "hbm"),
    }

    # the full-scoring chain over every context key, timed beside the route path
    max_ctx = prm["max_ctx"]
    tab5 = d["nt"][:, : -(-max_ctx // 64)].contiguous()
    full_logits = torch.empty((rows, -(-max_ctx // 4) * 4), device=dev)[:, :max_ctx]
    f_slots, f_raw = i32(rows, T), i32(rows, T)

    def full_chain():
        P.scoring.fp8_paged_mqa_logits(q, d["native"], d["w"], d["lens"], tab5, None, max_ctx, clean_logits=False,
                                       out=full_logits)
        P.topk.topk_transform_512_v2(full_logits, d["lens"], tab5, f_slots, 64, None, f_raw)
        P.native_kernels.gather_rows(latent, f_slots, work)

    def cpu(budget):
        from oracle import cpu_baseline
        qps, nq, threads = cpu_baseline.decode_route_queries_per_second(a, prm, budget)
        return qps, threads, f"{nq} of {rows} requests (V1 route path: center score, route, fine score, mask, " \
                             f"top2048, slot map; gather rows left out)"

    meta = {"workload": "decode batch: 128 requests x 64 heads FP8, contexts 4K-128K tokens with per-request page "
                        "tables in a 2M-token pool, V1 route path (page_fraction 0.5, fine widths up to 67K), "
                        "Top-2048, 656-byte row gather",
            "global_batch": rows, "seq_len": WIDTH, "parallelism": "single GPU",
            "_extra": [("unfused_route_chain", unfused_chain, (float(rows), "queries/s", None, None)),
                       ("full_scoring_chain", full_chain,
                        (lambda: (132.0 * n.sum() + 4.0 * 2 * n.sum() + rows * T * (8.0 + rb * 2)) / 1e9, "GB/s",
                         PEAK_HBM_GBS, "hbm"))]}
    return rows, stages, work_units, cpu, meta, "synthetic (PCG64 seed 5)"


def setup_pages(P, dev, torch, np):
    """Configuration 2: page management (grouping, match -> allocate -> publish,
    tail staging, release) for a batch of 4096 requests."""
    wl = P.workloads.config2()
    a, prm = wl.arrays, wl.params
    R, cap, pb = prm["requests"], prm["capacity"], prm["page_bytes"]
    n = prm["entries"]
    gen = torch.Generator(device=dev).manual_seed(wl.seed)
    uniq = torch.randint(0, 256, (prm["distinct"], pb), generator=gen, device=dev, dtype=torch.uint8)
    tmp = uniq[torch.from_numpy(a["draw"]).to(dev).long()]
    del uniq
    keys = torch.from_numpy(a["keys"]).to(dev)
    req = torch.from_numpy(a["req"]).to(dev)
    table = torch.empty(n, device=dev, dtype=torch.int32)
    # one insert to fix the table the release list and the tail tables are drawn from
    probe = P.pagepool.PagePool(cap, pb, dev)
    probe.insert(keys, tmp, req, table)
    if probe.status():
        raise RuntimeError("page-management workload does not fit the pool")
    t_host = table.cpu().numpy()
    fresh = int(cap - probe.count.item())
    del probe
    tails = P.workloads.config2_tails(wl, t_host)
    rel = torch.from_numpy(P.workloads.config2_release_list(wl, t_host)).to(dev)
    pool = P.pagepool.PagePool(cap, pb, dev, scratch_pages=R * tails["scratch"])
    nt = torch.from_numpy(tails["nt"]).to(dev)
    tl = torch.from_numpy(tails["lens"]).to(dev)
    owners = torch.from_numpy(tails["tail_rows"]).to(dev)
    stages = [
        ("reset", pool.reset),
        ("insert", lambda: pool.insert(keys, tmp, req, table)),
        ("stage", lambda: P.pagepool.stage_tail_rows(pool.pages, nt, tl, pool.pages, owners, cap,
                                                     tails["scratch"])),
        ("release", lambda: pool.release(rel)),
    ]
    owners_n = int((tails["tail_rows"] == np.arange(R)).sum())
    work_units = {
        "reset": (12.0 * cap / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        # every entry's page is read at least once (compared or copied), fresh pages written once
        "insert": (((n + fresh) * pb + 8.0 * n) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "stage": (2.0 * owners_n * 2 * pb / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "release": (16.0 * rel.numel() / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
    }

    def cpu(budget):
        from oracle import cpu_baseline
        rps, done, threads = cpu_baseline.pages_requests_per_second(a["keys"], a["draw"], a["lens"], cap, pb,
                                                                    budget)
        return rps, threads, f"{done} of {R} requests (match -> allocate -> publish from an empty pool)"

    meta = {"workload": f"page management: {R} requests of 1-64 pages ({n} Zipf(1.1) page keys, {fresh} distinct "
                        f"pages) into a {cap}-page pool of 41984-byte pages, 128-token tail staging of "
                        f"{owners_n} owner requests, release of {rel.numel()} pages",
            "global_batch": R, "seq_len": int(prm['entries']), "parallelism": "single GPU"}
    return R, stages, work_units, cpu, meta, "synthetic (PCG64 seed 2; page bytes from a seeded torch generator)"


# one bucket of the index build: 16 source pages read and 16 member pages written (8448 B each), two
# center pages, the 64x16 mapping and the 1024-entry order (int32), the 16-entry table and the start
BUILD_BUCKET_BYTES = 16 * 8448 * 2 + 2 * 8448 + 4 * 1024 * 2 + 4 * 16 + 4


def setup_build(P, dev, torch, np):
    """Configuration 6: index build of every bucket of a 2M-token pool."""
    wl = P.workloads.config6()
    a, prm = wl.arrays, wl.params
    B = prm["buckets"]
    pool = torch.from_numpy(a["native"]).to(dev)
    tables = torch.from_numpy(a["tables"]).to(dev)
    starts = torch.from_numpy(a["starts"]).to(dev)
    out = (torch.empty((B, 1024), device=dev, dtype=torch.int32),
           torch.empty((B, 16, 8448), device=dev, dtype=torch.uint8),
           torch.empty((B, 16, 64), device=dev, dtype=torch.int32),
           torch.empty((B, 2, 8448), device=dev, dtype=torch.uint8))
    stages = [("build", lambda: P.indexbuild.build_buckets(pool, tables, starts, out=out))]
    work_units = {"build": (BUILD_BUCKET_BYTES * B / 1e9, "GB/s", PEAK_HBM_GBS, "hbm")}

    def cpu(budget):
        from oracle import cpu_baseline
        tps, n, threads = cpu_baseline.build_tokens_per_second(a["native"], a["tables"], a["starts"], budget)
        return tps, threads, f"{n} of {B} buckets (initialize -> 7 bisection levels -> assemble, numpy)"

    # the reference's per-bucket chain (runtime.py:171-216: initialize, 7 x (3 _dots + 2 _anchor + _sort),
    # assemble; 44 launches) through the drop-in kernels, over the first 16 buckets, timed beside the batch
    K, FG = P.kernels, importlib.import_module("10_20_amd.fused_grouping")
    chain_buckets = 16
    unit = torch.empty((1024, 128), device=dev)
    cperm = [torch.empty(1024, device=dev, dtype=torch.int32) for _ in range(2)]
    anchor = torch.empty((64, 2), device=dev, dtype=torch.int32)
    cscores = torch.empty(1024, device=dev)
    flag = torch.zeros((), device=dev, dtype=torch.int32)
    ctmp = torch.empty((16, 8448), device=dev, dtype=torch.uint8)
    ccent = torch.empty((2, 8448), device=dev, dtype=torch.uint8)
    cmap = torch.empty((16, 64), device=dev, dtype=torch.int32)
    metas = [torch.tensor([int(a["starts"][i]), 0, 1], device=dev, dtype=torch.int32) for i in range(chain_buckets)]

    def chain():
        for i in range(chain_buckets):
            tab = tables[i]
            K.initialize[(64,)](pool, pool.view(torch.float32), tab, metas[i], unit, cperm[0], flag, num_warps=4)
            cur = 0
            for n in (1024, 512, 256, 128, 64, 32, 16):
                for mode in (0, 1, 2):
                    FG._dots[(64, 1)](unit, cperm[cur], anchor, cscores, flag, n, 0, mode, num_warps=4,
                                      enable_fp_fusion=False)
                    if mode < 2:
                        FG._anchor[(1024 // n, 1)](cperm[cur], anchor, cscores, flag, n, mode, num_warps=4)
                FG._sort[(1024 // n, 1)](cperm[cur], cperm[1 - cur], cscores, flag, n, num_warps=4)
                cur = 1 - cur
            K.assemble[(16, 8)](pool, pool.view(torch.float32), tab, metas[i], cperm[cur], ctmp,
                                ctmp.view(torch.float32), ccent, ccent.view(torch.float32), cmap, num_warps=4)

    meta = {"workload": f"index build: {B} buckets of 1024 tokens (16 pages each, every page of a "
                        f"{prm['pool_pages'] * 64 // (1 << 20)}M-token FP8 pool once) -> member order, "
                        "reordered pages, 128 FP8 centers per bucket",
            "global_batch": B, "seq_len": 1024, "parallelism": "single GPU",
            "_extra": [(f"per_kernel_chain_{chain_buckets}_buckets", chain,
                        (BUILD_BUCKET_BYTES * chain_buckets / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"))]}
    return B * 1024, stages, work_units, cpu, meta, "synthetic (PCG64 seed 6)"


def setup_union(P, dev, torch, np):
    """Configuration 7: shared sink + tail chunk with a published index end."""
    wl = P.workloads.config7()
    a, prm = wl.arrays, wl.params
    rows, heads, S, W, end = prm["rows"], prm["heads"], prm["sink"], prm["window"], prm["indexed_end"]
    cap, mt, T, npg = prm["cap"], prm["max_take"], prm["topk"], prm["pages"]
    TU = P.tailunion
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in a.items()}
    q = d["q8"].view(torch.float8_e4m3fn)
    d_end = torch.tensor([end], device=dev, dtype=torch.int32)
    last = prm["history"] + rows
    c_max = min(last, S) + last - max(min(last, S), min(min(end, last), max(min(last, S), last - W)))
    first = prm["history"] + 1
    first_tail = max(min(first, S), min(min(end, first), max(min(first, S), first - W)))
    union_cap = min(npg, -(-S // 64) + -(-last // 64) - first_tail // 64 + 2)
    scratch = -(-c_max // 64)
    width = -(-(mt * 64 + c_max + 128) // 256) * 256
    fine = torch.zeros((cap + union_cap, 8448), device=dev, dtype=torch.uint8)
    fine[:cap] = d["reordered"]
    meta_t = torch.empty((rows, 3), device=dev, dtype=torch.int32)
    desc = torch.zeros(4, device=dev, dtype=torch.int32)
    table = torch.empty((rows, width // 64), device=dev, dtype=torch.int32)
    dglens = torch.empty((rows, 1), device=dev, dtype=torch.int32)
    clens = torch.empty(rows, device=dev, dtype=torch.int32)
    raw = torch.empty((rows, width), device=dev)
    scores = torch.empty((rows, width), device=dev)
    ids = torch.empty((rows, T), device=dev, dtype=torch.int32)
    ids_pages = torch.empty_like(ids)
    identity = torch.arange(width // 64, device=dev, dtype=torch.int32)[None].expand(rows, -1).contiguous()
    logical = torch.empty_like(ids)
    slots = torch.empty_like(ids)
    plan = TU.PreparedStage(d["native"], d["nt"], d["lens"], d_end, fine[cap:], meta_t, desc, S, W)
    fine4 = fine.view(-1, 64, 1, 132)

    def prepare():
        plan()
        TU.tables[(rows,)](d["lens"], d_end, d["takes"], d["selected"], desc, table, dglens, clens, cap, mt, scratch,
                           width // 64, S, W, 256, True)

    def select():
        P.topk.topk_transform_512_v2(scores, clens, identity, ids_pages, 64, None, ids)
        TU.map_topk_scores(ids, scores, d["lens"], d_end, d["takes"], d["selected"], d["members"], d["nt"], logical,
                           slots, mt, S, W)

    stages = [
        ("prepare", prepare),
        ("score", lambda: P.scoring.fp8_paged_mqa_logits(q, fine4, d["w"], dglens, table, None, width,
                                                          clean_logits=False, out=raw)),
        ("normalize", lambda: TU.normalize[(rows, width // 256)](raw, d["lens"], d_end, d["takes"], d["selected"],
                                                                 d["members"], scores, mt, width, raw.stride(0), S, W,
                                                                 256, True)),
        ("select", select),
    ]
    # per-row staging with the same candidates (baseline_published.py), timed beside the chain
    per_row = torch.empty((cap + rows * scratch, 8448), device=dev, dtype=torch.uint8)
    per_row[:cap] = d["reordered"]
    nts = d["nt"][None].expand(rows, -1).contiguous()
    owners = torch.arange(rows, device=dev, dtype=torch.int32)
    table_r = torch.empty_like(table)

    def prepare_per_row():
        TU.stage_tail_shared[(rows, scratch)](d["native"], d["native"].view(torch.float32), nts, d["lens"], d_end,
                                              per_row, per_row.view(torch.float32), owners, cap, npg, scratch, S, W,
                                              rows, 1)
        TU.tables[(rows,)](d["lens"], d_end, d["takes"], d["selected"], desc, table_r, dglens, clens, cap, mt,
                           scratch, width // 64, S, W, 256, False)

    work_units = {
        # union pages read and written once (97 here), meta and tables
        "prepare": (lambda: (2.0 * 8448 * int(desc[3]) + 12.0 * rows + 4.0 * rows * (width // 64 + 2)) / 1e9,
                    "GB/s", PEAK_HBM_GBS, "hbm"),
        "score": (lambda: 2.0 * heads * 128 * float(dglens.sum()) / 1e12, "TFLOP/s", PEAK_FP8_TFLOPS, "mfma"),
        "normalize": ((4.0 * rows * width * 2) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "select": (lambda: (4.0 * float(clens.sum()) + 4.0 * rows * T * 6) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
    }

    def cpu(budget):
        from oracle import cpu_baseline
        qps, n, threads = cpu_baseline.union_queries_per_second(a, prm, budget)
        return qps, threads, f"{n} of {rows} queries (candidates, score, Top-2048, slot map)"

    # split scoring: every row once against the 64 history pages and once against the union, both
    # with one shared page table (the MFMA kernel that stages pages in LDS), then normalize_split
    hist_tab = torch.arange(cap, device=dev, dtype=torch.int32)[None].expand(rows, -1)
    uni_tab = (cap + torch.arange(union_cap, device=dev, dtype=torch.int32))[None].expand(rows, -1)
    hist_s = torch.empty((rows, cap * 64), device=dev)
    uni_s = torch.empty((rows, union_cap * 64), device=dev)
    spans = torch.empty(rows, device=dev, dtype=torch.int32)
    full = torch.full((rows,), cap * 64, device=dev, dtype=torch.int32)

    def chain_split():
        plan()
        TU.union_spans(d["lens"], d_end, desc, spans, S, W)
        P.scoring.fp8_paged_mqa_logits(q, fine4, d["w"], full, hist_tab, None, cap * 64, clean_logits=False,
                                       out=hist_s)
        P.scoring.fp8_paged_mqa_logits(q, fine4, d["w"], spans, uni_tab, None, union_cap * 64, clean_logits=False,
                                       out=uni_s)
        TU.normalize_split(hist_s, uni_s, d["lens"], d_end, d["takes"], d["selected"], d["members"], desc, scores,
                           mt, width, S, W)
        select()

    meta = {"workload": f"shared sink+tail chunk: {prm['history']} published tokens, {rows} causal queries x "
                        f"{heads} FP8 heads, sink {S} / window {W}, {mt} history pages per query, one union of "
                        f"sink+tail pages in the fine pool -> FP8 score -> canonical order -> Top-{T} -> slots",
            "global_batch": rows, "seq_len": width, "parallelism": "single GPU",
            "_extra": [("prepare_per_row", prepare_per_row,
                        (lambda: (8448.0 * 2 * rows * scratch) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm")),
                       ("chain_split_scoring", chain_split,
                        (lambda: 2.0 * heads * 128 * (cap * 64 * rows + float(spans.sum())) / 1e12, "TFLOP/s",
                         PEAK_FP8_TFLOPS, "mfma"))]}
    return rows, stages, work_units, cpu, meta, "synthetic (PCG64 seed 7)"


def setup_consumer(P, dev, torch, np):
    """Configuration 8: the backend's inner loop for one KV head and one
    microbatch (sglang/srt/layers/attention/v1_native/backend.py:300-315):
    Top-2048 slot ids -> GatherWorkspace.gather (bf16 K / V) ->
    flash_attn_with_kvcache(qs[:, None], kg, vg)."""
    rows, T, slots, heads_kv, group = 4096, 2048, 1 << 20, 2, 4
    g = torch.Generator(device=dev).manual_seed(8)
    kp = torch.randn((slots, heads_kv, 128), device=dev, generator=g).to(torch.bfloat16)
    vp = torch.randn((slots, heads_kv, 128), device=dev, generator=g).to(torch.bfloat16)
    req = torch.randperm(slots, device=dev, generator=g).to(torch.int32)
    ids = torch.randint(0, slots, (rows, T), device=dev, generator=g, dtype=torch.int32)
    q3 = torch.randn((rows, heads_kv * group, 128), device=dev, generator=g).to(torch.bfloat16)
    qs = q3[:, :group].contiguous()
    work = P.native_kernels.GatherWorkspace(rows, dev, torch.bfloat16)
    out = torch.empty((rows, 1, group, 128), device=dev, dtype=torch.bfloat16)
    scale = 1.0 / 128 ** 0.5
    kv = {}

    def gather():
        kv["k"], kv["v"] = work.gather(kp, vp, req, ids, 0)

    stages = [
        ("gather", gather),
        ("attention", lambda: P.attention.flash_attn_with_kvcache(qs[:, None], kv["k"], kv["v"], causal=False,
                                                                  softmax_scale=scale, out=out)),
    ]
    kv_bytes = 2.0 * rows * T * 256  # K and V rows of one head
    work_units = {
        # pool rows read (1M slots x 512 B per head pair: far above the last-level cache) and workspace written
        "gather": ((2 * kv_bytes + 4.0 * rows * T) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "attention": ((kv_bytes + 2.0 * rows * group * 128 * 2) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
    }

    def cpu(budget):
        from oracle import cpu_baseline
        qps, n, threads = cpu_baseline.consumer_queries_per_second(kp, vp, req, ids, qs, scale, budget)
        return qps, threads, f"{n} of {rows} queries (2048-slot gather + 4-head attention)"

    fused_out = torch.empty_like(out)
    meta = {"workload": f"attention consumer: {rows} queries x {group} heads of one KV head, 2048 gathered bf16 "
                        f"K/V slots each from a {slots >> 20}M-slot pool -> decode attention",
            "global_batch": rows, "seq_len": T, "parallelism": "single GPU",
            # the gather folded into the attention (same result, no workspace), timed beside the chain
            "_extra": [("gather_fused_attention",
                        lambda: P.attention.attend_slots(qs, kp, vp, req, ids, 0, softmax_scale=scale, out=fused_out),
                        ((kv_bytes + 4.0 * rows * T) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"))]}
    return rows, stages, work_units, cpu, meta, "synthetic (torch generator seed 8)"


SETUPS = {1: setup_example, 2: setup_pages, 3: setup_gather, 4: setup_prefill, 5: setup_decode, 6: setup_build,
          7: setup_union, 8: setup_consumer, 9: setup_whole}
RATE_UNITS = {2: "requests/s", 6: "tokens/s"}
METRICS = {6: "index-build tokens/sec (initialize+bisection+assemble) and % of HBM roofline",
           9: "whole V1 queries/sec (coarse+route+fine score+Top2048+x4) and % of FP8-MFMA/HBM roofline"}


def run(config, steps, warmup, cpu_budget, P, dev, torch, np):
    """Sets up one workload, times `steps` steps after `warmup`, and returns
    its JSON record (the bench line without the run-wide fields)."""
    rows, stages, work_units, cpu_fn, meta, data = SETUPS[config](P, dev, torch, np)
    extra = meta.pop("_extra", [])
    names = [n for n, _ in stages]
    ev = {n: [] for n in names}

    def step(record):
        prev = None
        if record:
            prev = torch.cuda.Event(enable_timing=True)
            prev.record()
        for name, fn in stages:
            fn()
            if record:
                e = torch.cuda.Event(enable_timing=True)
                e.record()
                ev[name].append((prev, e))
                prev = e

    for _ in range(warmup):
        step(False)
    torch.cuda.synchronize()
    # The timed steps record no events: an event between every pair of stages
    # added ~36 us to the 9-stage decode step (0.325 against 0.289 ms).  The
    # per-stage breakdown comes from as many steps again, with events.
    t0 = time.perf_counter()
    for _ in range(steps):
        step(False)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / steps
    for _ in range(steps):
        step(True)
    torch.cuda.synchronize()
    stage_ms = {n: sum(x.elapsed_time(y) for x, y in ev[n]) / steps for n in names}

    # alternatives timed beside the chain (not part of a step)
    alternatives = {}
    for name, fn, unit in extra:
        for _ in range(warmup):
            fn()
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record()
        for _ in range(steps):
            fn()
        a1.record()
        a1.synchronize()
        ms = a0.elapsed_time(a1) / steps
        amount = unit[0]() if callable(unit[0]) else unit[0]
        alternatives[name] = {"ms": round(ms, 4), "achieved": round(amount / (ms / 1e3), 1), "unit": unit[1],
                              "bound": unit[3],
                              "frac": None if unit[2] is None else round(amount / (ms / 1e3) / unit[2], 4)}

    stage_info = {}
    work_units = {n: ((u[0]() if callable(u[0]) else u[0]),) + tuple(u[1:]) for n, u in work_units.items()}
    for n in names:
        amount, unit, peak, bound = work_units[n]
        ach = amount / (stage_ms[n] / 1e3)
        stage_info[n] = {"ms": round(stage_ms[n], 4), "achieved": round(ach, 1), "unit": unit, "bound": bound,
                         "frac": round(ach / peak, 4)}
    dom = max(names, key=lambda n: stage_ms[n])
    amount, unit, peak, bound = work_units[dom]
    achieved = amount / (stage_ms[dom] / 1e3)

    rate_unit = RATE_UNITS.get(config, "queries/s")
    cpu = None
    if cpu_budget > 0:
        qps_cpu, threads, sample = cpu_fn(cpu_budget)
        cpu = {"value": round(qps_cpu, 3), "unit": rate_unit, "cores": threads, "kind": "port",
               "sample": f"{sample}, torch CPU, {os.cpu_count()} host cpus visible", "cpu": cpu_model()}

    qps = rows * steps / (t1 - t0)
    line = {
        "metric": METRICS.get(config, "indexed queries/sec (score+Top2048+gather) and % of FP8-MFMA/HBM roofline"),
        "value": round(qps, 1), "unit": rate_unit, "ms_per_step": round(ms_step, 4), "data": data,
        "config": meta,
        "stages": stage_info,
        "roofline": {"kernel": dom, "bound": bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4),
                     "traffic": measured_traffic(config, dom)},
        "cpu_baseline": cpu,
    }
    if alternatives:
        line["alternatives"] = alternatives
    return line


# The reference's per-kernel graph timings on H20-3e (experiments/v1_kernel_opt_20261022/
# RESULTS.md:75-81, 105-111), reported beside this build's as context.
REFERENCE_H20_US = {
    "sort_1024": 10.769, "sort_512": 3.638, "sort_256": 2.548, "sort_128": 2.212, "sort_64": 1.942,
    "sort_32": 1.738, "sort_16": 1.696, "fingerprint": 3.194, "match_miss": 2.384, "match_hit": 4.281,
    "match_collision": 5.987, "publish_all_new": 3.484, "publish_mixed": 3.457, "publish_reuse": 1.610,
}


def micro_timings(P, dev, torch, reps=20, replays=50):
    """Configuration 10: per-call times of the grouping sort and the per-lease
    page manager under HIP graph replay, with the setups of the reference's
    micro-benchmark (experiments/v1_kernel_opt_20261022/bench_pages.py:5-40:
    16 temp pages, a 4096-page pool, miss / hit / collision and all-new /
    mixed / reuse).  Each graph holds `reps` calls and is replayed `replays`
    times; the result is microseconds per call."""
    FG = importlib.import_module("10_20_amd.fused_grouping")
    K = P.kernels
    g = torch.Generator(device=dev).manual_seed(77)

    def graph_us(fn):
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(replays):
            graph.replay()
        e1.record()
        e1.synchronize()
        return round(e0.elapsed_time(e1) * 1e3 / (replays * reps), 3)

    out = {}
    # _sort of one bucket's 1024 scores in groups of N (fused_grouping.py:64-76)
    perm = torch.arange(1024, device=dev, dtype=torch.int32)
    dst = torch.empty_like(perm)
    scores = torch.randn(1024, device=dev, generator=g)
    flag = torch.full((1,), -1, device=dev, dtype=torch.int32)
    for n in (1024, 512, 256, 128, 64, 32, 16):
        out[f"sort_{n}"] = graph_us(lambda n=n: FG._sort[(1024 // n, 1)](perm, dst, scores, flag, n))
    # page manager at a 4096-page pool
    cap = 4096
    tmp = torch.randint(0, 256, (16, 8448), device=dev, dtype=torch.uint8, generator=g)
    mp = torch.randint(-1, 262144, (16, 64), device=dev, dtype=torch.int32, generator=g)
    meta = torch.tensor([4096, 1, 1], device=dev, dtype=torch.int32)
    h = torch.empty((16, 2), device=dev, dtype=torch.int64)
    out["fingerprint"] = graph_us(lambda: K.fingerprint[(16,)](tmp, mp, meta, h))
    fine = torch.randint(0, 256, (cap, 8448), device=dev, dtype=torch.uint8, generator=g)
    members = torch.zeros((cap, 64), device=dev, dtype=torch.int32)
    hashes = torch.zeros((cap, 2), device=dev, dtype=torch.int64)
    refs = torch.zeros(cap, device=dev, dtype=torch.int32)
    match = torch.empty(16, device=dev, dtype=torch.int32)
    for mode in ("miss", "hit", "collision"):
        refs.zero_()
        hashes.zero_()
        if mode != "miss":
            fine[1:17].copy_(tmp)
            members[1:17].copy_(mp)
            hashes[1:17].copy_(h)
            refs[1:17] = 1
        if mode == "collision":
            fine[0].copy_(tmp[0])
            fine[0, 0] ^= 1
            members[0].copy_(mp[0])
            hashes[0].copy_(h[0])
            refs[0] = 1
        out[f"match_{mode}"] = graph_us(
            lambda: K.match_pages[(16,)](tmp, mp, h, meta, fine, members, hashes, refs, match, cap))
        expect = [-1] * 16 if mode == "miss" else list(range(1, 17))
        if match.tolist() != expect:
            raise RuntimeError(f"match_pages {mode}: {match.tolist()}")
    tc = torch.randint(0, 256, (2, 8448), device=dev, dtype=torch.uint8, generator=g)
    tab = torch.zeros((2, 16), device=dev, dtype=torch.int32)
    tab[1] = torch.arange(1, 17, device=dev, dtype=torch.int32)
    new = torch.ones(16, device=dev, dtype=torch.bool)
    f = torch.full_like(fine, 19)
    c = torch.full((4, 8448), 19, device=dev, dtype=torch.uint8)
    m = torch.full_like(members, -99)
    hh = torch.full_like(hashes, -99)
    for mode in ("all_new", "mixed", "reuse"):
        new.fill_(mode != "reuse")
        if mode == "mixed":
            new[::2] = False
        out[f"publish_{mode}"] = graph_us(
            lambda: K.publish[(16,)](tmp, tc, tc.view(torch.float32), mp, h, meta, tab, new, f, c,
                                     c.view(torch.float32), m, hh))
    return out


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    import gc

    import numpy as np
    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    P = Pkg()
    if args.config == 10:
        us = micro_timings(P, dev, torch)
        print(json.dumps({"metric": "microseconds per call under HIP graph replay (context timings)", "value": None,
                          "unit": "us", "n_gpus": 1, "higher_is_better": False, "data": "synthetic (seed 77)",
                          "config": {"workload": "one bucket's _sort at group sizes 1024..16; fingerprint, "
                                                 "match_pages and publish of one 16-page lease at a 4096-page pool"},
                          "timings_us": us, "reference_h20_us": REFERENCE_H20_US}), flush=True)
        return
    rec = run(args.config, args.steps, args.warmup, args.cpu_budget, P, dev, torch, np)
    line = {"metric": rec.pop("metric"), "value": rec.pop("value"), "unit": rec.pop("unit"), "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": rec.pop("ms_per_step"),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp8-e4m3 score / fp32 accumulate / int32 indices / u8 rows", **rec}
    more = args.with_configs
    if more is None:
        more = "1,2,3,5,7,9" if args.config == 4 else ""
    configs = [int(c) for c in more.split(",") if c.strip()]
    if configs:
        # the other workloads of the metric, each at its own synthetic shape,
        # measured after the headline one (secondary records: same timing,
        # roofline of the dominant kernel, a shorter CPU sample)
        line["configs"] = {}
        for c in configs:
            gc.collect()
            torch.cuda.empty_cache()
            r = run(c, args.steps, args.warmup, args.with_cpu_budget, P, dev, torch, np)
            rl = r["roofline"]
            line["configs"][str(c)] = {
                "workload": r["config"]["workload"], "metric": r["metric"], "value": r["value"], "unit": r["unit"],
                "ms_per_step": r["ms_per_step"], "data": r["data"],
                "stages": {n: {"ms": v["ms"], "frac": v["frac"], "bound": v["bound"]} for n, v in r["stages"].items()},
                "roofline": {k: rl[k] for k in ("kernel", "bound", "achieved", "peak", "unit", "frac", "traffic")},
                "cpu_baseline": r["cpu_baseline"],
            }
            print(f"config {c}: {r['value']} {r['unit']}, {r['ms_per_step']} ms per step", file=sys.stderr,
                  flush=True)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
