"""The entry points are stream-ordered and allocate nothing per call, so a
chain of them captures into one HIP graph: the decode chain (FP8 scoring with
per-row tables -> Top-2048 transform -> 656-byte row gather) captured once and
replayed with new queries and lengths written in place, every replay equal bit
for bit to the same chain run eagerly."""
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SC = importlib.import_module("10_20_amd.scoring")
TK = importlib.import_module("10_20_amd.topk")
NK = importlib.import_module("10_20_amd.native_kernels")
W = importlib.import_module("10_20_amd.workloads")
DEV = "cuda:0"


def test_decode_chain_replays_in_a_hip_graph():
    g = np.random.default_rng(31)
    rows, heads, pool_pages, max_ctx = 16, 64, 512, 20000
    k8, ks = W.quantize_rows(g.standard_normal((pool_pages * 64, 128)).astype(np.float32))
    native = torch.from_numpy(W.pack_pages(k8, ks)).to(DEV)
    pages = -(-max_ctx // 64)
    table = torch.from_numpy(np.stack([g.permutation(pool_pages)[:pages] for _ in range(rows)]).astype(np.int32)).to(DEV)
    latent = torch.from_numpy(g.integers(0, 256, (pool_pages * 64, 656), dtype=np.uint8)).to(DEV)
    q = torch.empty((rows, heads, 128), device=DEV, dtype=torch.uint8)
    w = torch.empty((rows, heads), device=DEV)
    lens = torch.empty(rows, device=DEV, dtype=torch.int32)
    logits = torch.empty((rows, max_ctx), device=DEV)
    slots = torch.empty((rows, 2048), device=DEV, dtype=torch.int32)
    raw = torch.empty_like(slots)
    work = torch.empty((rows, 2048, 656), device=DEV, dtype=torch.uint8)

    def inputs(seed):
        h = np.random.default_rng(seed)
        q8, _ = W.quantize_rows(h.standard_normal((rows * heads, 128)).astype(np.float32))
        q.copy_(torch.from_numpy(q8.reshape(rows, heads, 128)))
        w.copy_(torch.from_numpy(h.random((rows, heads), dtype=np.float32)))
        lens.copy_(torch.from_numpy(h.integers(1000, max_ctx + 1, rows).astype(np.int32)))

    def chain():
        SC.fp8_paged_mqa_logits(q.view(torch.float8_e4m3fn), native, w, lens, table, None, max_ctx,
                                clean_logits=False, out=logits)
        TK.topk_transform_512_v2(logits, lens, table, slots, 64, None, raw)
        NK.gather_rows(latent, slots, work)

    inputs(0)
    chain()  # first calls size and cache the workspaces
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain()
    for seed in (1, 2, 3):
        inputs(seed)
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (slots, raw, work)]
        chain()
        torch.cuda.synchronize()
        for a, b in zip(got, (slots, raw, work)):
            assert torch.equal(a, b)
        assert int((raw >= 0).sum()) > 0


def test_index_build_and_slot_attention_replay_in_a_hip_graph():
    IB = importlib.import_module("10_20_amd.indexbuild")
    AT = importlib.import_module("10_20_amd.attention")
    g = np.random.default_rng(41)
    k8, ks = W.quantize_rows(g.standard_normal((96 * 64, 128)).astype(np.float32))
    pool = torch.from_numpy(W.pack_pages(k8, ks)).to(DEV)
    tables = torch.empty((6, 16), device=DEV, dtype=torch.int32)
    starts = torch.from_numpy((np.arange(6) * 1024).astype(np.int32)).to(DEV)
    out = (torch.empty((6, 1024), device=DEV, dtype=torch.int32), torch.empty((6, 16, 8448), device=DEV, dtype=torch.uint8),
           torch.empty((6, 16, 64), device=DEV, dtype=torch.int32), torch.empty((6, 2, 8448), device=DEV, dtype=torch.uint8))
    gen = torch.Generator(device=DEV).manual_seed(41)
    kp = torch.randn((5000, 2, 128), device=DEV, generator=gen).to(torch.bfloat16)
    vp = torch.randn((5000, 2, 128), device=DEV, generator=gen).to(torch.bfloat16)
    req = torch.randperm(5000, device=DEV, generator=gen).to(torch.int32)
    ids = torch.empty((32, 2048), device=DEV, dtype=torch.int32)
    qs = torch.randn((32, 4, 128), device=DEV, generator=gen).to(torch.bfloat16)
    att = torch.empty((32, 1, 4, 128), device=DEV, dtype=torch.bfloat16)

    def inputs(seed):
        h = np.random.default_rng(seed)
        tables.copy_(torch.from_numpy(h.permutation(96)[:96].reshape(6, 16).astype(np.int32)))
        ids.copy_(torch.from_numpy(h.integers(-3, 5003, (32, 2048)).astype(np.int32)))

    def work():
        IB.build_buckets(pool, tables, starts, out=out)
        AT.attend_slots(qs, kp, vp, req, ids, 1, softmax_scale=0.09, out=att)

    inputs(0)
    work()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        work()
    for seed in (1, 2, 3):
        inputs(seed)
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (*out, att)]
        work()
        torch.cuda.synchronize()
        for a, b in zip(got, (*out, att)):
            assert torch.equal(a, b)


def test_query_chain_replays_in_a_hip_graph():
    """Query.compute's fused chain (sglang/srt/layers/attention/v1_deepseek/
    runtime.py:417-678) captured once: coarse score -> route with the fine-table
    fill -> shared tail staging -> fine score -> fused Top-2048 with the mask and
    physical map -> slot gather.  Replayed with new queries, a new context
    length for the request (pages, sink and tail move), new per-row budgets and
    a permuted reordered table (as experiments/fine_pool_shared_20261021/
    test_route_shared.py:43-48 replays route), each replay equal bit for bit to
    the chain run eagerly."""
    QF = importlib.import_module("10_20_amd.query_fused")
    K = importlib.import_module("10_20_amd.kernels")
    wl = W.config1(rows=640)  # the fused Top-K takes batches above 512 rows (v1_query.cuh:206)
    a, prm = wl.arrays, wl.params
    B, P, CAP, TAKE, WIDTH, TOP = prm["B"], prm["P"], prm["CAP"], prm["TAKE"], prm["WIDTH"], prm["TOPK"]
    SINK, WINDOW = prm["SINK"], prm["WINDOW"]
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    q = t(a["q8"])
    w = t(a["w"])
    centers, native, members, nt = t(a["centers"]), t(a["native"]), t(a["members"]), t(a["nt"])
    rt, lens, takes, tail_rows = t(a["rt"]), t(a["lens"]), t(a["takes"]), t(a["tail_rows"])
    fine_lens, fine = t(a["fine_lens"]), t(a["fine"])
    center_table = t(a["center_table"])[None].expand(B, -1)
    center_lens = torch.full((B,), 512, device=DEV, dtype=torch.int32)
    latent = t(a["latent"])
    coarse = torch.empty((B, P * 8), device=DEV)
    sel = torch.empty((B, TAKE), device=DEV, dtype=torch.int32)
    ft = torch.empty((B, prm["FT_COLS"]), device=DEV, dtype=torch.int32)
    logits = torch.empty((B, WIDTH), device=DEV)
    physical = torch.empty((B, TOP), device=DEV, dtype=torch.int32)
    logical, raw = torch.empty_like(physical), torch.empty_like(physical)
    expanded = torch.empty((B, 4 * TOP + 64), device=DEV, dtype=torch.int32)
    work = torch.empty((B, TOP, W.MLA_ROW_BYTES), device=DEV, dtype=torch.uint8)
    outs = (coarse, sel, ft, fine, logits, physical, logical, raw, expanded, work)

    def chain():
        qv = q.view(torch.float8_e4m3fn)
        SC.fp8_paged_mqa_logits(qv, centers, w, center_lens, center_table, None, P * 8, clean_logits=True, out=coarse)
        QF.module().route(coarse, lens, takes, sel, P, rt, ft, tail_rows, CAP, True)
        K.stage_tail_shared[(-(-B // 32), 68)](native, None, nt, lens, fine, None, tail_rows, CAP, P, 68, SINK, WINDOW,
                                               ROWS=B, GROUP=32)
        SC.fp8_paged_mqa_logits(qv, fine, w, fine_lens, ft, None, WIDTH, clean_logits=True, out=logits)
        QF.module().topk(logits, fine_lens, members, rt, nt, sel, lens, takes, physical, logical, raw, WINDOW, True,
                         expanded, True, True, ft, False)
        NK.gather_rows(latent, physical, work)

    def inputs(seed, n, budget, flip):
        h = np.random.default_rng(seed)
        q8, qs = W.quantize_rows(h.standard_normal((B, 128)).astype(np.float32))
        q.copy_(torch.from_numpy(q8.reshape(B, 1, 128)))
        w.copy_(torch.from_numpy(qs[:, None].astype(np.float32)))
        lens.fill_(n)
        takes.copy_(torch.from_numpy(np.minimum(budget, h.integers(8, TAKE + 1, B)).astype(np.int32)))
        # candidates below the fine width, as query_lengths gives them
        pages = (n - 1) // 1024 * 16
        sink = min(SINK, n)
        tail = max(sink, min((n - 1) // 1024 * 1024, max(sink, n - WINDOW)))
        count = np.minimum(takes.cpu().numpy(), pages) * 64 + sink + n - tail
        fine_lens.copy_(torch.from_numpy(np.minimum(count, WIDTH).astype(np.int32)))
        if flip:
            rt[:, :64] = rt[:, :64].flip(1)

    inputs(0, 4097, TAKE, False)
    chain()  # sizes the workspaces
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain()
    for seed, n, budget, flip in ((1, 4097, TAKE, False), (2, 3073, 24, True), (3, 2100, TAKE, False),
                                  (4, 4097, 16, True)):
        inputs(seed, n, budget, flip)
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        chain()
        torch.cuda.synchronize()
        for name, x, y in zip(("coarse", "sel", "ft", "fine", "logits", "physical", "logical", "raw", "expanded",
                               "work"), got, outs):
            assert torch.equal(x.view(torch.uint8) if x.dtype == torch.float32 else x,
                               y.view(torch.uint8) if y.dtype == torch.float32 else y), (seed, name)
        assert int((raw >= 0).sum()) > 0 and int((physical >= 0).sum()) > 0
