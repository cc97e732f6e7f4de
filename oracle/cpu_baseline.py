"""CPU baseline (test / measurement infrastructure only): the reference's own
torch expressions for the query path, run with torch on the host cores.

  score  (relu(q.float() @ k.T) * w[:, None]).sum(0) * scale
         experiments/fine_pool_shared_20261021/test_and_bench.py:37
  top-k  scores.topk(2048) and page -> slot mapping nt[i // 64] * 64 + i % 64
         sglang/srt/layers/attention/v1_deepseek/example_v1_query_single_head.py:55-70
  gather fancy indexing, sglang/srt/layers/attention/v1_native/test_gather_slots_small.py:18-24
"""
import time

import numpy as np
import torch


def prefill_queries_per_second(q8, w, native, table, lens, latent, topk=2048, budget_s=10.0, min_rows=8):
    """Runs whole queries (score -> Top-2048 -> slots -> gather) of a shared
    page-table prefill chunk until budget_s elapses; returns (q/s, rows, threads)."""
    threads = torch.get_num_threads()
    k_bytes = native[:, :8192].reshape(-1, 64, 128)
    k_scale = native[:, 8192:].copy().view(np.float32).reshape(-1, 64)
    ctx = int(lens.max())
    j = np.arange(ctx)
    pages = table[j // 64]
    k = torch.from_numpy(np.ascontiguousarray(k_bytes[pages, j % 64])).view(torch.float8_e4m3fn).float()
    s = torch.from_numpy(np.ascontiguousarray(k_scale[pages, j % 64]))
    tab = torch.from_numpy(table.astype(np.int64))
    lat = torch.from_numpy(latent)
    qs = torch.from_numpy(q8).view(torch.float8_e4m3fn)
    ws = torch.from_numpy(w)
    rows = q8.shape[0]
    order = np.random.default_rng(0).permutation(rows)
    done = 0
    t0 = time.perf_counter()
    while done < rows and (done < min_rows or time.perf_counter() - t0 < budget_s):
        r = int(order[done])
        n = int(lens[r])
        q = qs[r].float()
        logits = (torch.relu(q @ k[:n].T) * ws[r][:, None]).sum(0) * s[:n]
        idx = logits.topk(min(topk, n)).indices
        slots = tab[idx // 64] * 64 + idx % 64
        out = lat[slots]
        assert out.shape[0] == min(topk, n)
        done += 1
    dt = time.perf_counter() - t0
    return done / dt, done, threads
