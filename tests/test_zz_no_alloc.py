"""The allocation-free score entry point (v1_score_noalloc, static per-GPU
scratch) against v1_score with a caller workspace, through the C ABI: bit for
bit equal on two calls in a row, the second smaller than the first (the shared
scratch keeps the first call's contents), with few live heads so that the
exact-zero path's page bitmaps in the scratch are exercised; and too large a
call is rejected before anything runs."""
import ctypes
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

L = importlib.import_module("10_20_amd._lib")
W = importlib.import_module("10_20_amd.workloads")
DEV = "cuda:0"
PAGE = 8448


def _inputs(seed, rows, heads, live, ctx):
    g = np.random.default_rng(seed)
    q8l, sq = W.quantize_rows(g.standard_normal((rows * live, 128), dtype=np.float32))
    q8 = np.zeros((rows, heads, 128), np.uint8)
    q8[:, :live] = q8l.reshape(rows, live, 128)
    w = np.zeros((rows, heads), np.float32)
    w[:, :live] = (sq.reshape(rows, live) * np.float32(0.0884 / live)).astype(np.float32)
    pages = -(-ctx // 64)
    k8, ks = W.quantize_rows(g.standard_normal((pages * 64, 128), dtype=np.float32))
    native = W.pack_pages(k8, ks)
    table = g.permutation(pages).astype(np.int32)
    lens = np.minimum(ctx, ctx - rows + 1 + np.arange(rows)).astype(np.int32)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    return dict(q=t(q8), w=t(w), native=t(native), table=t(table), lens=t(lens), rows=rows, heads=heads, ctx=ctx)


def _args(d, out, ws=None):
    return L.ScoreArgs(d["q"].data_ptr(), d["native"].data_ptr(), d["native"].numel() // PAGE, d["w"].data_ptr(),
                       d["lens"].data_ptr(), d["table"].data_ptr(), 0, d["table"].numel(), out.data_ptr(),
                       out.stride(0), d["ctx"], d["rows"], d["heads"], 1, 1,
                       0 if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel())


def test_noalloc_equals_workspace_entry_on_two_calls():
    lib = L.lib()
    stream = torch.cuda.current_stream().cuda_stream
    for seed, (rows, heads, live, ctx) in enumerate([(96, 32, 4, 9000), (40, 64, 64, 3000)]):
        d = _inputs(seed, rows, heads, live, ctx)
        ref = torch.full((rows, ctx), float("nan"), device=DEV)
        ws = torch.empty(lib.v1_score_workspace(rows, ctx), device=DEV, dtype=torch.uint8)
        L.check(lib.v1_score(ctypes.byref(_args(d, ref, ws)), stream), "v1_score")
        got = torch.full((rows, ctx), float("nan"), device=DEV)
        L.check(lib.v1_score_noalloc(ctypes.byref(_args(d, got)), stream), "v1_score_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), f"call {seed} differs"
        if live < 8:  # the exact path ran: the plateau of exact zeros is there
            assert int((got == 0).sum()) > 0


def test_noalloc_rejects_more_than_its_scratch():
    lib = L.lib()
    cap = lib.v1_score_noalloc_capacity()
    rows, ctx = 16384, 131072
    assert lib.v1_score_workspace(rows, ctx) > cap
    d = dict(q=torch.empty(16, device=DEV, dtype=torch.uint8), w=torch.empty(1, device=DEV),
             native=torch.empty(PAGE, device=DEV, dtype=torch.uint8), table=torch.zeros(1, device=DEV, dtype=torch.int32),
             lens=torch.zeros(1, device=DEV, dtype=torch.int32), rows=rows, heads=64, ctx=ctx)
    out = torch.empty((1, 1), device=DEV)
    a = _args(d, out)
    a.logits_stride = ctx
    rc = lib.v1_score_noalloc(ctypes.byref(a), torch.cuda.current_stream().cuda_stream)
    assert rc == L.V1_ERR_INVALID and b"static" in lib.v1_last_error()
