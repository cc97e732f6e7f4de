"""Exact ReLU zeros of the FP8 index scorer.

The reference's logit sum_h w_h * ReLU(q_h . k) * s_k is exactly 0 for a key
whose every head dot is <= 0 (sglang/srt/layers/attention/v1_deepseek/
kernels.py:310-313), and Top-K breaks the ties of that zero plateau by lower
index.  The shapes below are the reference probe's query packing
(qwen_gqa_probe_kernels.py:14-20: 4 live heads of 32, w = s_q * SCALE / 4,
zero queries and weights past them) and a single head with w = s_q * SCALE:
non-power-of-two weights, about 1/16 (resp. 1/2) of the keys exact zeros, and
rows of ~2100 keys so that the Top-2048 boundary falls inside the plateau.
Both the shared-table kernel (one page table for the whole chunk) and the
per-row kernel are checked, and the selected indices are compared with a
Top-2048 over the fp64 reference scores themselves."""
import numpy as np
import pytest
import torch

from conftest import pkg
from oracle import v1 as O
from test_gpu_kernels import H, T, assert_scores_close

pytestmark = pytest.mark.gpu

SC = pkg("scoring")
TK = pkg("topk")
W = pkg("workloads")

SOFTMAX_SCALE = 128 ** -0.5


def _probe_case(g, rows, heads, live, ctx, pool_pages, signed):
    q8l, sq = W.quantize_rows(g.standard_normal((rows * live, 128), dtype=np.float32))
    q8 = np.zeros((rows, heads, 128), np.uint8)
    q8[:, :live] = q8l.reshape(rows, live, 128)
    w = np.zeros((rows, heads), np.float32)
    w[:, :live] = (sq.reshape(rows, live) * np.float32(SOFTMAX_SCALE / live)).astype(np.float32)
    if signed:
        w[:, :live] *= np.where(g.random((rows, live)) < 0.5, -1, 1).astype(np.float32)
    k8, ks = W.quantize_rows(g.standard_normal((pool_pages * 64, 128), dtype=np.float32))
    native = W.pack_pages(k8, ks)
    blocks = -(-ctx // 64)
    table = g.permutation(pool_pages)[:blocks].astype(np.int32)
    lens = (ctx - rows + 1 + np.arange(rows)).astype(np.int32)
    return q8, w, native, table, lens


def _top_fp64(ref, lens, topk):
    """Top-`topk` per row over fp64 scores: value descending, ties by lower
    index, returned ascending (the order the Top-K kernels emit)."""
    out = np.full((ref.shape[0], topk), -1, np.int64)
    for b in range(ref.shape[0]):
        L = int(lens[b])
        order = np.lexsort((np.arange(L), -ref[b, :L]))[:topk]
        out[b, :min(L, topk)] = np.sort(order)
    return out


@pytest.mark.parametrize("shared", [True, False])
@pytest.mark.parametrize("heads,live,signed", [(1, 1, False), (32, 4, False), (32, 4, True), (64, 8, False)])
def test_relu_zeros_exact_and_topk_on_fp64_scores(dev, shared, heads, live, signed):
    g = np.random.default_rng(100 * heads + 10 * live + int(signed) + 2 * int(shared))
    rows, ctx = 40, 2120
    q8, w, native, table, lens = _probe_case(g, rows, heads, live, ctx, 96, signed)
    full = np.broadcast_to(table, (rows, table.size))
    bt = T(table, dev)[None].expand(rows, -1) if shared else T(np.ascontiguousarray(full), dev)
    out = SC.fp8_paged_mqa_logits(T(q8, dev).view(torch.float8_e4m3fn), T(native, dev), T(w, dev), T(lens, dev), bt,
                                  None, ctx, clean_logits=True)
    got = H(out)
    ref = O.paged_logits(q8, w, native, full, lens, ctx)
    bound = O.paged_logits(q8, w, native, full, lens, ctx, magnitude=True)
    assert_scores_close(got.astype(np.float64), ref, bound)
    fin = np.isfinite(ref)
    zero = fin & (ref == 0)
    # the plateau is there (about 2^-live of the keys), its scores are +0.0 bit
    # for bit, and no key with a positive head dot lands on it
    assert zero.sum() > 0.5 * fin.sum() * 2.0 ** -live
    assert (got[zero].view(np.uint32) == 0).all(), f"{int((got[zero] != 0).sum())} reference zeros scored nonzero"
    assert (got[fin & (ref != 0)] != 0).all()
    if signed or live > 4:
        return
    # Top-2048 on the GPU logits equals Top-2048 on the fp64 reference scores
    # for rows whose boundary falls inside the zero plateau
    positive = (fin & (ref > 0)).sum(axis=1)
    plateau_rows = (positive < 2048) & (positive + zero.sum(axis=1) > 2048)
    assert plateau_rows.all()
    slots = torch.empty((rows, 2048), device=dev, dtype=torch.int32)
    raw = torch.empty_like(slots)
    ident = np.arange(-(-ctx // 64), dtype=np.int32)[None].repeat(rows, 0)
    TK.topk_transform_512_v2(out, T(lens, dev), T(ident, dev), slots, 64, None, raw)
    assert np.array_equal(H(raw), _top_fp64(ref, lens, 2048))
