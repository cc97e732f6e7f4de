#!/usr/bin/env python3
"""Benchmark of the query-indexing hot path on one MI355X.

A step is one pass of the path over one batch: FP8 paged index scoring ->
exact Top-2048 with page-table slot mapping -> 656-byte latent-row gather
into a reused [rows, 2048, 656] workspace.  Default workload: the
DeepSeek-V3.2-style prefill indexer chunk (4096 queries x 64 heads x 128,
32768-token FP8 context in 64-token pages, causal).  Inputs are synthetic
(seeded PCG64) and resident in HBM before timing starts.

Prints one JSON line (queries/sec, per-stage times, roofline of the dominant
kernel, CPU baseline of the reference's torch expressions).
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
# HBM traffic per dispatch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE on this
# workload (calibrated against a plain copy), kept with the kernel trace.
TRAFFIC_PROFILE = ROOT / "profiles" / "prefill_chunk_4096x32k.md"
STAGE_KERNELS = {"score": ("score_prep", "score_shared"), "topk": ("transform_rows",), "gather": ("gather_rows16",)}


def measured_traffic(stage):
    """HBM bytes per step of a stage's kernels from the committed counter
    summary, or None when the summary does not list them."""
    if not TRAFFIC_PROFILE.exists():
        return None
    per_kernel = {}
    for line in TRAFFIC_PROFILE.read_text().splitlines():
        cells = [c.strip().strip("`") for c in line.strip().strip("|").split("|")]
        if len(cells) == 6 and cells[0] and not cells[0].startswith("-"):
            try:
                per_kernel[cells[0].split("<")[0]] = float(cells[5])
            except ValueError:
                continue
    vals = [per_kernel.get(k) for k in STAGE_KERNELS[stage]]
    return None if any(v is None for v in vals) else sum(vals)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=4, choices=[1, 3, 4, 5])
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline work (0 = skip)")
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


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    W = importlib.import_module("10_20_amd.workloads")
    SC = importlib.import_module("10_20_amd.scoring")
    TK = importlib.import_module("10_20_amd.topk")
    NK = importlib.import_module("10_20_amd.native_kernels")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.config != 4:
        raise SystemExit("only the prefill-chunk workload (config 4) is wired into bench.py so far")
    wl = W.config4()
    a, prm = wl.arrays, wl.params
    rows, heads, T, row_bytes = prm["rows"], prm["heads"], prm["topk"], prm["row_bytes"]
    ctx = prm["ctx"]
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

    stages = ["score", "topk", "gather"]
    ev = {s: [] for s in stages}

    def step(record):
        e0 = torch.cuda.Event(enable_timing=True) if record else None
        if record:
            e0.record()
        SC.fp8_paged_mqa_logits(q, native, w, lens, shared_table, None, ctx, clean_logits=False, out=logits)
        if record:
            e1 = torch.cuda.Event(enable_timing=True)
            e1.record()
        TK.topk_transform_512_v2(logits, lens, dense_table, slots, 64, None, raw)
        if record:
            e2 = torch.cuda.Event(enable_timing=True)
            e2.record()
        NK.gather_rows(latent, slots, work)
        if record:
            e3 = torch.cuda.Event(enable_timing=True)
            e3.record()
            ev["score"].append((e0, e1))
            ev["topk"].append((e1, e2))
            ev["gather"].append((e2, e3))

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    stage_ms = {s: sum(x.elapsed_time(y) for x, y in ev[s]) / args.steps for s in stages}

    L = a["lens"].astype(np.int64)
    flops = 2.0 * heads * 128 * float(L.sum())
    valid = rows * T  # every row has more than T candidates
    work_units = {
        "score": (flops / 1e12, "TFLOP/s", PEAK_FP8_TFLOPS, "mfma"),
        "topk": ((4.0 * L.sum() + 8.0 * rows * T) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
        "gather": ((row_bytes * valid + row_bytes * rows * T + 4.0 * rows * T) / 1e9, "GB/s", PEAK_HBM_GBS, "hbm"),
    }
    stage_info = {}
    for s in stages:
        amount, unit, peak, bound = work_units[s]
        ach = amount / (stage_ms[s] / 1e3)
        stage_info[s] = {"ms": round(stage_ms[s], 4), "achieved": round(ach, 1), "unit": unit, "bound": bound,
                         "frac": round(ach / peak, 4)}
    dom = max(stages, key=lambda s: stage_ms[s])
    amount, unit, peak, bound = work_units[dom]
    achieved = amount / (stage_ms[dom] / 1e3)

    cpu = None
    if args.cpu_budget > 0:
        from oracle import cpu_baseline
        qps, n, threads = cpu_baseline.prefill_queries_per_second(a["q8"], a["w"], a["native"], a["table"],
                                                                  a["lens"], a["latent"], T, args.cpu_budget)
        cpu = {"value": round(qps, 3), "unit": "queries/s", "cores": threads, "kind": "port",
               "sample": f"{n} of {rows} queries (score+top2048+slot map+gather), torch CPU, {os.cpu_count()} "
                         f"host cpus visible"}

    qps = rows * args.steps / (t1 - t0)
    line = {
        "metric": "indexed queries/sec (score+Top2048+gather) and % of FP8-MFMA/HBM roofline",
        "value": round(qps, 1), "unit": "queries/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8-e4m3 score / fp32 accumulate / int32 indices / u8 rows", "data": "synthetic (PCG64 seed 4)",
        "config": {"workload": "prefill indexer chunk: 4096 queries x 64 heads x 128 FP8 vs 32768-token paged "
                               "FP8 context, causal, Top-2048, 656-byte latent row gather",
                   "global_batch": rows, "seq_len": ctx, "parallelism": "single GPU"},
        "stages": stage_info,
        "roofline": {"kernel": dom, "bound": bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4), "traffic": measured_traffic(dom)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
