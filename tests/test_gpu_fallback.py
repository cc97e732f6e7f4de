"""Scoring without DeepGEMM (the reference's Triton fallbacks,
sglang/srt/layers/attention/v1_deepseek/kernels.py:182-221, 248-320, 475-486,
called at runtime.py:450-466 and 565-590) against the oracle: reduce_centers
bit for bit, coarse and fine within the score tolerance, with the same -inf
pattern."""
import numpy as np
import pytest
import torch

from conftest import pkg
from oracle import v1 as O
from test_gpu_kernels import H, T, assert_scores_close

pytestmark = pytest.mark.gpu

K = pkg("kernels")
W = pkg("workloads")


def test_reduce_centers_vs_oracle(dev):
    g = np.random.default_rng(3)
    rows, maxp, stride = 37, 96, 96 * 8 + 5
    logits = g.standard_normal((rows, stride)).astype(np.float32)
    logits[g.random((rows, stride)) < 0.05] = -np.inf
    lens = g.integers(0, 7000, rows).astype(np.int32)
    lens[:4] = [0, 1024, 1025, 6145]
    out = torch.full((rows, maxp), 7.0, device=dev)
    K.reduce_centers[(rows, -(-maxp // 32))](T(logits, dev), T(lens, dev), out, maxp, stride)
    assert np.array_equal(H(out), O.reduce_centers(logits, lens, maxp))


def _centers(g, pages):
    c8, cs = W.quantize_rows(g.standard_normal((pages * 64, 128)).astype(np.float32))
    return W.pack_pages(c8, cs)


@pytest.mark.parametrize("heads,shared", [(1, False), (64, False), (64, True), (5, False)])
def test_coarse_vs_oracle(dev, heads, shared):
    g = np.random.default_rng(heads + 10 * shared)
    rows, maxp, cpages = 24, 128, 40
    centers = _centers(g, cpages)
    q8, _ = W.quantize_rows(g.standard_normal((rows * heads, 128)).astype(np.float32))
    q8 = q8.reshape(rows, heads, 128)
    w = g.random((rows, heads)).astype(np.float32)
    if shared:
        table = np.broadcast_to(g.permutation(cpages)[:maxp // 8].astype(np.int32), (rows, maxp // 8))
        table_d = T(np.array(table[0]), dev)[None].expand(rows, -1)
    else:
        table = np.stack([g.permutation(cpages)[:maxp // 8] for _ in range(rows)]).astype(np.int32)
        table_d = T(table, dev)
    lens = g.integers(0, 9000, rows).astype(np.int32)
    lens[:3] = [1024, 1025, 8193]
    cv = T(centers, dev)
    out = torch.empty((rows, maxp), device=dev)
    K.coarse[(rows, maxp // 8)](T(q8, dev).view(torch.float8_e4m3fn), T(w, dev), cv.view(torch.float8_e4m3fn),
                                cv.view(torch.float32), table_d, T(lens, dev), out, maxp, heads, True, num_warps=4)
    ref = O.coarse(q8, w, centers, np.ascontiguousarray(table), lens, maxp)
    pages = np.minimum((np.maximum(lens - 1, 0) // 1024) * 16, maxp)
    bound = O.paged_logits(q8, w, centers, np.ascontiguousarray(table), pages * 8, maxp * 8, magnitude=True)
    bound = np.where(np.isfinite(bound), bound, 0).reshape(rows, maxp, 8).max(axis=2)
    assert_scores_close(H(out).astype(np.float64), ref.astype(np.float64), bound)


def _fine_case(seed, rows, heads):
    wl = W.config1(rows=rows)
    a, prm = wl.arrays, wl.params
    g = np.random.default_rng(seed)
    if heads > 1:
        q8, _ = W.quantize_rows(g.standard_normal((rows * heads, 128)).astype(np.float32))
        a["q8"] = q8.reshape(rows, heads, 128)
        a["w"] = g.random((rows, heads)).astype(np.float32)
    lens = g.choice([4097, 3073, 2100, 1500, 1025, 64, 0], rows).astype(np.int32)
    lens[:2] = [4097, 2100]
    takes = g.integers(0, prm["TAKE"] + 1, rows).astype(np.int32)
    takes[:2] = [prm["TAKE"], 0]
    selected = np.stack([g.permutation(64)[:prm["TAKE"]] for _ in range(rows)]).astype(np.int32)
    return a, prm, lens, takes, selected


@pytest.mark.parametrize("heads,sel64", [(1, False), (64, False), (64, True), (20, False)])
def test_fine_vs_oracle(dev, heads, sel64):
    rows = 48
    a, prm, lens, takes, selected = _fine_case(heads + sel64, rows, heads)
    WIDTH, SINK, WINDOW, TAKE, P = prm["WIDTH"], prm["SINK"], prm["WINDOW"], prm["TAKE"], prm["P"]
    fine, native = T(a["fine"], dev), T(a["native"], dev)
    sel = T(selected.astype(np.int64) if sel64 else selected, dev)
    out = torch.full((rows, WIDTH), 3.0, device=dev)
    K.fine[(rows, WIDTH // 64)](T(a["q8"], dev).view(torch.float8_e4m3fn), T(a["w"], dev),
                                fine.view(torch.float8_e4m3fn), fine.view(torch.float32),
                                native.view(torch.float8_e4m3fn), native.view(torch.float32), T(a["members"], dev),
                                T(a["rt"], dev), T(a["nt"], dev), sel, T(lens, dev), T(takes, dev), out, P,
                                a["nt"].shape[1], TAKE, WIDTH, SINK, WINDOW, heads, True)
    args = (a["q8"], a["w"], a["fine"], a["native"], a["members"], a["rt"], a["nt"], selected, lens, takes, WIDTH,
            SINK, WINDOW)
    ref = O.fine(*args)
    bound = O.fine(*args, magnitude=True)
    got = H(out).astype(np.float64)
    assert_scores_close(got, ref, np.where(np.isfinite(bound), bound, 0))
    assert np.isfinite(ref).sum() > 1000
