"""CPU baseline (test / measurement infrastructure only): the reference's own
torch expressions for the query path, run with torch on the host cores.

  score  (relu(q.float() @ k.T) * w[:, None]).sum(0) * scale
         experiments/fine_pool_shared_20261021/test_and_bench.py:37
  top-k  scores.topk(2048) and page -> slot mapping nt[i // 64] * 64 + i % 64
         sglang/srt/layers/attention/v1_deepseek/example_v1_query_single_head.py:55-70
  gather fancy indexing, sglang/srt/layers/attention/v1_native/test_gather_slots_small.py:18-24
  pages  the oracle's page manager, request after request (a host port of
         sglang/srt/layers/attention/v1_deepseek/kernels.py:72-167)
  build  the oracle's index build, bucket after bucket (a host port of
         sglang/srt/layers/attention/v1_deepseek/runtime.py:171-216)
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


def _dequant_pages(native, pages):
    """fp32 keys [len(pages) * 64, 128] and scales of native pages."""
    kb = native[pages, :8192].reshape(-1, 128)
    ks = native[pages, 8192:].copy().view(np.float32).reshape(-1)
    k = torch.from_numpy(np.ascontiguousarray(kb)).view(torch.float8_e4m3fn).float()
    return k, torch.from_numpy(np.ascontiguousarray(ks))


def whole_query_queries_per_second(a, prm, budget_s=10.0, min_rows=2):
    """The example's torch path per query at many heads
    (sglang/srt/layers/attention/v1_deepseek/example_v1_query_single_head.py:38-70
    with the score sum_h w_h relu(q_h . k) of sra/v1_deepseek/kernels.py:310-313):
    coarse scores over the centers, page max, top-`TAKE` pages, candidate keys
    (their members, sink, tail), masked fine scores, Top-2048, logical
    positions and their x4 expansion."""
    threads = torch.get_num_threads()
    B, take, n, window, sink_cap = prm["B"], prm["TAKE"], prm["N"], prm["WINDOW"], prm["SINK"]
    built = prm["BUILT"]
    centers, cs = _dequant_pages(a["centers"], np.arange(a["centers"].shape[0]))
    centers = (centers * cs[:, None])[: prm["CENTERS"]]
    nt = a["nt"][0]
    keys, ks = _dequant_pages(a["native"], nt[: -(-n // 64)])
    keys = keys * ks[:, None]
    members = torch.from_numpy(a["members"].astype(np.int64))
    rt = torch.from_numpy(a["rt"][0].astype(np.int64))
    sink = min(n, sink_cap)
    tail = max(sink, min((n - 1) // 1024 * 1024, max(sink, n - window)))
    fixed = torch.cat((torch.arange(sink), torch.arange(tail, n)))
    qs = torch.from_numpy(a["q8"]).view(torch.float8_e4m3fn)
    w = torch.from_numpy(a["w"])
    done, t0 = 0, time.perf_counter()
    while done < B and (done < min_rows or time.perf_counter() - t0 < budget_s):
        q = qs[done].float()
        coarse = (torch.relu(centers @ q.T) * w[done]).sum(1)
        pages = coarse.view(built, 8).amax(1).topk(take).indices
        chosen = members[rt[pages]].reshape(-1)
        cand = torch.cat((chosen, fixed))
        valid = torch.ones(cand.shape[0], dtype=torch.bool)
        valid[: take * 64] = (chosen >= sink) & (chosen < tail)
        valid &= torch.arange(cand.shape[0]) < int(a["fine_lens"][done])
        scores = (torch.relu(keys[cand.clamp(0, n - 1)] @ q.T) * w[done]).sum(1).masked_fill(~valid, float("-inf"))
        lg = cand[scores.topk(min(2048, scores.shape[0])).indices]
        expanded = (lg[:, None] * 4 + torch.arange(4)).reshape(-1)
        assert expanded.shape[0] == 4 * lg.shape[0]
        done += 1
    return done / (time.perf_counter() - t0), done, threads


def example_queries_per_second(a, prm, budget_s=10.0, min_rows=8):
    """The reference example's torch path per query
    (sglang/srt/layers/attention/v1_deepseek/example_v1_query_single_head.py:38-70):
    coarse scores over centers, page max, top-40 pages, candidate keys (their
    members, sink, tail), masked fine scores, Top-2048, slot map, row gather."""
    threads = torch.get_num_threads()
    B, take, n, window, sink_cap = prm["B"], prm["TAKE"], prm["N"], prm["WINDOW"], prm["SINK"]
    centers, cs = _dequant_pages(a["centers"], np.arange(a["centers"].shape[0]))
    centers = centers * cs[:, None]
    nt = a["nt"][0]
    keys, ks = _dequant_pages(a["native"], nt[: -(-n // 64)])
    keys = keys * ks[:, None]
    members = torch.from_numpy(a["members"].astype(np.int64))
    rt = torch.from_numpy(a["rt"][0].astype(np.int64))
    ntt = torch.from_numpy(nt.astype(np.int64))
    lat = torch.from_numpy(a["latent"])
    sink = min(n, sink_cap)
    tail = max(sink, min((n - 1) // 1024 * 1024, max(sink, n - window)))
    fixed = torch.cat((torch.arange(sink), torch.arange(tail, n)))
    qs = torch.from_numpy(a["q8"][:, 0]).view(torch.float8_e4m3fn).float()
    w = torch.from_numpy(a["w"][:, 0])
    done, t0 = 0, time.perf_counter()
    while done < B and (done < min_rows or time.perf_counter() - t0 < budget_s):
        q = qs[done] * w[done]
        coarse = torch.relu(centers @ q)
        pages = coarse.view(64, 8).amax(1).topk(take).indices
        chosen = members[rt[pages]].reshape(-1)
        cand = torch.cat((chosen, fixed))
        valid = torch.ones(cand.shape[0], dtype=torch.bool)
        valid[: take * 64] = (chosen >= sink) & (chosen < tail)
        valid &= torch.arange(cand.shape[0]) < int(a["fine_lens"][done])
        scores = torch.relu(keys[cand.clamp(0, n - 1)] @ q).masked_fill(~valid, float("-inf"))
        raw = scores.topk(min(2048, scores.shape[0])).indices
        lg = cand[raw]
        phys = ntt[lg // 64] * 64 + lg % 64
        out = lat[phys]
        assert out.shape[0] == raw.shape[0]
        done += 1
    return done / (time.perf_counter() - t0), done, threads


def gather_queries_per_second(pool, ids, table, budget_s=10.0, min_rows=8):
    """Fancy-index gather per query (test_gather_slots_small.py:18-24) through
    the query's page window; -1 ids give zero rows."""
    threads = torch.get_num_threads()
    pool_t = torch.from_numpy(pool)
    rows = ids.shape[0]
    done, t0 = 0, time.perf_counter()
    while done < rows and (done < min_rows or time.perf_counter() - t0 < budget_s):
        i = torch.from_numpy(ids[done].astype(np.int64))
        tab = torch.from_numpy(table[done].astype(np.int64))
        ok = i >= 0
        phys = torch.where(ok, tab[i.clamp(min=0) >> 6] * 64 + (i.clamp(min=0) & 63), 0)
        out = pool_t[phys]
        out[~ok] = 0
        done += 1
    return done / (time.perf_counter() - t0), done, threads


def decode_queries_per_second(q8, w, native, table, lens, topk=2048, budget_s=10.0, min_rows=4):
    """Per request: keys of its pages, (relu(q @ k.T) * w).sum(0) * s_k, Top-2048,
    slot map (the row gather is left out of this sample)."""
    threads = torch.get_num_threads()
    rows = q8.shape[0]
    order = np.random.default_rng(0).permutation(rows)
    done, t0 = 0, time.perf_counter()
    while done < rows and (done < min_rows or time.perf_counter() - t0 < budget_s):
        r = int(order[done])
        n = int(lens[r])
        k, s = _dequant_pages(native, table[r, : -(-n // 64)])
        q = torch.from_numpy(q8[r]).view(torch.float8_e4m3fn).float()
        logits = (torch.relu(q @ k[:n].T) * torch.from_numpy(w[r])[:, None]).sum(0) * s[:n]
        idx = logits.topk(min(topk, n)).indices
        slots = torch.from_numpy(table[r].astype(np.int64))[idx // 64] * 64 + idx % 64
        assert slots.shape[0] == min(topk, n)
        done += 1
    return done / (time.perf_counter() - t0), done, threads


def decode_route_queries_per_second(a, prm, budget_s=10.0, min_rows=4):
    """The decode batch's V1 route path per request in the reference's torch
    terms (example_v1_query_single_head.py:38-70 with 64 heads and the
    scoring expression of test_and_bench.py:37): center scores, page max of
    8, top-take pages, candidate keys (their members, sink, tail), masked fine
    scores, Top-2048, slot map (the row gather is left out of this sample)."""
    threads = torch.get_num_threads()
    rows, P, topk, sink_cap, window = prm["rows"], prm["P"], prm["topk"], prm["sink"], prm["window"]
    num, den = prm["num"], prm["den"]
    members = torch.from_numpy(a["members"].astype(np.int64))
    order = np.random.default_rng(0).permutation(rows)
    done, t0 = 0, time.perf_counter()
    while done < rows and (done < min_rows or time.perf_counter() - t0 < budget_s):
        r = int(order[done])
        n = int(a["lens"][r])
        pages = max(n - 1, 0) // 1024 * 16
        take = min(pages, max(-(-pages * num // den), -(-topk // 64)))
        q = torch.from_numpy(a["q8"][r]).view(torch.float8_e4m3fn).float()
        w = torch.from_numpy(a["w"][r])
        cen, cs = _dequant_pages(a["centers"], a["center_table"][r, : pages // 8])
        coarse = (torch.relu(q @ cen.T) * w[:, None]).sum(0) * cs
        chosen_pages = coarse.view(pages, 8).amax(1).topk(take).indices
        rt = torch.from_numpy(a["rt"][r].astype(np.int64))
        chosen = members[rt[chosen_pages]].reshape(-1)
        sink = min(n, sink_cap)
        tail = max(sink, min((n - 1) // 1024 * 1024, max(sink, n - window)))
        cand = torch.cat((chosen, torch.arange(sink), torch.arange(tail, n)))
        keys, ks = _dequant_pages(a["native"], a["nt"][r, : -(-n // 64)])
        valid = torch.ones(cand.shape[0], dtype=torch.bool)
        valid[: take * 64] = (chosen >= sink) & (chosen < tail)
        scores = ((torch.relu(q @ keys[cand].T) * w[:, None]).sum(0) * ks[cand]).masked_fill(~valid, float("-inf"))
        raw = scores.topk(min(topk, scores.shape[0])).indices
        lg = cand[raw]
        phys = torch.from_numpy(a["nt"][r].astype(np.int64))[lg // 64] * 64 + lg % 64
        assert phys.shape[0] == raw.shape[0]
        done += 1
    return done / (time.perf_counter() - t0), done, threads


class _RowsOf:
    """tmp[i] = payload[inv[i]] without materialising every entry's page."""

    def __init__(self, payload, inv):
        self.payload, self.inv = payload, inv

    def __getitem__(self, i):
        return self.payload[self.inv[i]]


def pages_requests_per_second(keys, draws, lens, capacity, page_bytes, budget_s=10.0, sample_requests=4096,
                              min_requests=4, seed=1002):
    """The page manager run request after request on the host (the oracle's
    in-place match_pages -> allocate -> publish, kernels.py:72-167, with a
    key -> live pages map), over the first `sample_requests` requests of the
    workload from an empty pool of `capacity` pages of page_bytes, until the
    time budget ends.  Distinct draws get distinct seeded bytes (made before
    timing).  One thread."""
    from . import v1 as O
    R = min(sample_requests, len(lens))
    n = int(np.asarray(lens[:R], dtype=np.int64).sum())
    uniq, inv = np.unique(draws[:n], return_inverse=True)
    payload = np.random.default_rng(seed).integers(0, 256, size=(len(uniq), page_bytes), dtype=np.uint8)
    tmp = _RowsOf(payload, inv)
    pool = np.zeros((capacity, page_bytes), dtype=np.uint8)
    pool_keys = np.zeros(capacity, dtype=np.int64)
    refs = np.zeros(capacity, dtype=np.int32)
    free = np.arange(capacity, dtype=np.int32)
    count, live = capacity, {}
    table = np.empty(n, dtype=np.int32)
    starts = np.concatenate([[0], np.cumsum(lens[:R])]).astype(np.int64)
    done, t0 = 0, time.perf_counter()
    while done < R and (done < min_requests or time.perf_counter() - t0 < budget_s):
        count = O.insert_request_inplace(pool, pool_keys, refs, free, count, live, keys, tmp, starts[done],
                                         starts[done + 1], table)
        done += 1
    return done / (time.perf_counter() - t0), done, 1


def build_tokens_per_second(native, tables, starts, budget_s=10.0, min_buckets=2):
    """The index build bucket after bucket on the host (the oracle's
    initialize -> seven bisection levels -> assemble, runtime.py:171-216),
    until the time budget ends; returns (tokens/s, buckets, threads).  numpy's
    element-wise passes run on one thread."""
    from . import v1 as O
    done, t0 = 0, time.perf_counter()
    while done < len(tables) and (done < min_buckets or time.perf_counter() - t0 < budget_s):
        O.index_build(native, tables[done], int(starts[done]))
        done += 1
    return 1024.0 * done / (time.perf_counter() - t0), done, 1


def union_queries_per_second(a, prm, budget_s=10.0, min_rows=4):
    """Whole queries of the shared sink + tail chunk on the host, row after row:
    the row's candidates (its history pages' members masked to [s, t), < n and
    < the published end; sink; tail from the published end), scored with the
    reference's torch expression (experiments/fine_pool_shared_20261021/
    test_and_bench.py:25-38), Top-2048 and the slot map (kernels.py:62-76).
    Returns (q/s, rows, threads)."""
    from . import v1 as O
    threads = torch.get_num_threads()
    nk = torch.from_numpy(a["native"][:, :8192].reshape(-1, 64, 128)).view(torch.float8_e4m3fn)
    ns = torch.from_numpy(a["native"][:, 8192:].copy().view(np.float32).reshape(-1, 64))
    nt = torch.from_numpy(a["nt"].astype(np.int64))
    members = a["members"]
    S, W, end, T = prm["sink"], prm["window"], prm["indexed_end"], prm["topk"]
    rows = len(a["lens"])
    order = np.random.default_rng(0).permutation(rows)
    done, t0 = 0, time.perf_counter()
    while done < rows and (done < min_rows or time.perf_counter() - t0 < budget_s):
        r = int(order[done])
        n, take = int(a["lens"][r]), int(a["takes"][r])
        s, t, c = O.union_bounds(n, end, S, W)
        hist = members[a["selected"][r, :take]].reshape(-1)
        keep = torch.from_numpy((hist >= s) & (hist < t) & (hist < n) & (hist < end))
        ids = torch.from_numpy(np.concatenate([hist, np.arange(s), np.arange(t, n)]).astype(np.int64))
        k = nk[nt[ids // 64], ids % 64].float()
        sc = ns[nt[ids // 64], ids % 64]
        q = torch.from_numpy(a["q8"][r]).view(torch.float8_e4m3fn).float()
        score = (torch.relu(q @ k.T) * torch.from_numpy(a["w"][r])[:, None]).sum(0) * sc
        score[:take * 64].masked_fill_(~keep, -float("inf"))
        vals, top = score.topk(min(T, score.numel()))
        logical = ids[top]
        valid = (vals != -float("inf")) & (logical < n)
        slots = torch.where(valid, nt[logical // 64] * 64 + logical % 64, -1)
        del slots
        done += 1
    return done / (time.perf_counter() - t0), done, threads


def consumer_queries_per_second(kp, vp, req, ids, qs, scale, budget_s=10.0, min_rows=4):
    """The backend's gather + attention (backend.py:300-315) for one KV head, row
    after row, with torch on the host: K / V rows of the row's 2048 slots, then
    softmax(scale q k^T) v for its query heads.  Returns (q/s, rows, threads)."""
    threads = torch.get_num_threads()
    kp, vp = kp[:, 0].float().cpu(), vp[:, 0].float().cpu()
    req, ids, qs = req.cpu().long(), ids.cpu().long(), qs.float().cpu()
    rows = ids.shape[0]
    done, t0 = 0, time.perf_counter()
    while done < rows and (done < min_rows or time.perf_counter() - t0 < budget_s):
        sel = req[ids[done]]
        k, v = kp[sel], vp[sel]
        p = torch.softmax(qs[done] @ k.T * scale, -1)
        out = p @ v
        del out
        done += 1
    return done / (time.perf_counter() - t0), done, threads
