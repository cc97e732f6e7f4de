"""Per-row block tables of large batches: page-major and the page-union plan.

Batches of more than 512 rows with per-row tables (the fine tables of a
prefill chunk, sglang/srt/layers/attention/v1_deepseek/runtime.py:538-548)
are scored page-major over a small pool (each work-group stages 8 pool pages
once for every row of a 64-row block that lists them), or per group of 8 rows
over the union of the rows' table pages (17 heads and more, when the rows
share enough of their pages; two queries per wave up to 48 heads, one with
64).  Every test runs in both forms (`form`).  The
result must be the formula of kernels.py:310-313 through each row's own table,
whatever the tables hold: partly overlapping page sets in each row's own
order, unequal lengths (empty rows, rows past their table), a page listed
twice by one row, entries that are -1 or past the pool (their keys read as
zeros and score 0, as the per-row kernel gives), and groups that share too
little (scored row by row).  The reference maps every invalid entry and every
slot past the table to an all-zero page appended to the pool."""
import numpy as np
import pytest
import torch

from conftest import pkg
from oracle import v1 as O
from test_gpu_kernels import H, T, assert_scores_close, assert_scores_rel

pytestmark = pytest.mark.gpu

SC = pkg("scoring")
W = pkg("workloads")


@pytest.fixture(params=["pages", "union"])
def form(request):
    """page-major allowed (it takes every batch here over a small pool) or off"""
    prev = SC.page_major(request.param == "pages")
    yield request.param
    SC.page_major(prev)


def _queries(g, rows, heads, live):
    """FP8 queries and weights >= 0; heads past `live` are zero (few live
    heads put many keys on the ReLU zero plateau)."""
    q8l, sq = W.quantize_rows(g.standard_normal((rows * live, 128), dtype=np.float32))
    q8 = np.zeros((rows, heads, 128), np.uint8)
    q8[:, :live] = q8l.reshape(rows, live, 128)
    w = np.zeros((rows, heads), np.float32)
    w[:, :live] = (sq.reshape(rows, live) * g.random((rows, live), dtype=np.float32)).astype(np.float32)
    return q8, w


def _tables(g, rows, pool_pages, shared_pages, take, private, unrelated_rows=()):
    """Each row lists `take` of the chunk's `shared_pages` pages in its own
    order, then `private` pages of its own; rows in `unrelated_rows` list
    random pool pages instead.  A few rows list a page twice, a few entries
    are -1 or past the pool."""
    chunk = g.permutation(pool_pages)[:shared_pages]
    blocks = take + private
    table = np.empty((rows, blocks), np.int32)
    for r in range(rows):
        if r in unrelated_rows:
            table[r] = g.integers(0, pool_pages, blocks)
        else:
            table[r, :take] = chunk[g.permutation(shared_pages)[:take]]
            table[r, take:] = g.integers(0, pool_pages, private)
    dup = g.random(rows) < 0.05
    for r in np.nonzero(dup)[0]:
        a, b = g.choice(blocks, 2, replace=False)
        table[r, b] = table[r, a]
    table[g.random((rows, blocks)) < 0.02] = -1
    table[g.random((rows, blocks)) < 0.01] = pool_pages + 5
    return table


def _padded(native, table, width):
    """The pool with an all-zero page appended, and the table with every
    invalid entry and every slot past it (up to width) pointing there."""
    pool_pages = native.shape[0]
    pool = np.concatenate([native, np.zeros((1, native.shape[1]), np.uint8)])
    tab = np.full((table.shape[0], max(-(-width // 64), table.shape[1])), pool_pages, np.int32)
    tab[:, :table.shape[1]] = np.where((table >= 0) & (table < pool_pages), table, pool_pages)
    return pool, tab


def _certain_zeros(q8, w, pool, tab, lens, width):
    """Keys whose every live head dot lies below 0 by more than the fp32
    accumulation allowance 2^-16 * sum_d |q_d k_d|: their ReLU score is exactly
    0 whatever the summation order (a dot at or just below 0 can come out of
    an fp32 sum of FP8 products slightly positive, and ReLU keeps it)."""
    qf = O.e4m3_decode(q8).astype(np.float64)
    kk = pool[:, :8192].reshape(-1, 64, 128)
    out = np.zeros((q8.shape[0], width), bool)
    for r in range(q8.shape[0]):
        n = min(int(lens[r]), width)
        if n <= 0:
            continue
        j = np.arange(n)
        k = O.e4m3_decode(kk[tab[r, j // 64], j % 64]).astype(np.float64)
        live = w[r] != 0
        d, a = qf[r][live] @ k.T, np.abs(qf[r][live]) @ np.abs(k).T
        out[r, :n] = (d + 2.0 ** -16 * a <= 0).all(axis=0)
    return out


def _run(dev, q8, w, native, table, lens, width, relu, clean, fill=7.0):
    rows = q8.shape[0]
    out = torch.full((rows, width), fill, device=dev)
    SC.fp8_paged_mqa_logits(T(q8, dev).view(torch.float8_e4m3fn), T(native, dev), T(w, dev), T(lens, dev),
                            T(table, dev), None, width, clean_logits=clean, relu=relu, out=out)
    return H(out).astype(np.float64)


@pytest.mark.parametrize("rows,heads,live,relu,clean,take,private", [
    (520, 32, 32, True, True, 44, 0),     # 65 groups sharing almost every page
    (1031, 32, 4, True, False, 30, 4),    # last group of 7 rows, pages a wave's rows skip, unclean, zero plateau
    (777, 48, 48, False, True, 30, 4),    # signed scores, 48 heads
    (560, 64, 64, True, True, 44, 0),     # 64 heads: one query per wave
    (1031, 64, 4, True, False, 30, 4),    # 64 heads, few live ones, unclean, partial last group
    (777, 64, 64, False, True, 30, 4),    # 64 heads, signed scores
    (545, 50, 50, True, True, 40, 2),     # 50 heads: the one-row form with a partial head block
    (530, 17, 17, True, False, 30, 4),    # 17 heads: two rows per wave, a partial head block
    (600, 16, 2, True, True, 30, 4),      # one head block: row by row
    (529, 7, 7, True, True, 30, 4),       # heads not a multiple of 16: row by row
])
def test_union_plan_vs_reference(dev, form, rows, heads, live, relu, clean, take, private):
    g = np.random.default_rng(rows * 131 + heads)
    pool_pages, fill = 160, 7.0
    q8, w = _queries(g, rows, heads, live)
    if not relu:
        w *= np.where(g.random(w.shape) < 0.5, -1, 1).astype(np.float32)
    k8, ks = W.quantize_rows(g.standard_normal((pool_pages * 64, 128), dtype=np.float32))
    native = W.pack_pages(k8, ks)
    table = _tables(g, rows, pool_pages, shared_pages=48, take=take, private=private)
    blocks = table.shape[1]
    lens = g.integers(1, blocks * 64 + 1, rows).astype(np.int32)
    lens[g.random(rows) < 0.05] = 0
    lens[g.random(rows) < 0.05] = blocks * 64 + 90  # past the table: those keys score 0
    width = blocks * 64 + 128
    got = _run(dev, q8, w, native, table, lens, width, relu, clean, fill)
    pool, tab = _padded(native, table, width)
    ref = O.paged_logits(q8, w, pool, tab, lens, width, relu=relu, clean=clean)
    bound = O.paged_logits(q8, w, pool, tab, lens, width, magnitude=True, clean=False)
    if not clean:
        past = np.arange(width)[None, :] >= lens[:, None]
        assert (got[past] == fill).all(), "a column past a row's length was written"
        ref[past] = fill
    fin = np.isfinite(ref)
    assert np.array_equal(fin, np.isfinite(got))
    if relu:
        zero = fin & (ref == 0) & _certain_zeros(q8, w, pool, tab, lens, width)
        assert zero.any()
        assert (got[zero].astype(np.float32).view(np.uint32) == 0).all(), \
            f"{int((got[zero] != 0).sum())} certain reference zeros scored other than +0.0"
    if relu and live == heads and live >= 16:
        assert_scores_rel(got, ref)
    else:
        # signed sums and lone live heads cancel: the fp32 accumulation allowance
        assert_scores_close(got, ref, bound)


def test_union_plan_low_sharing_groups_fall_back(dev, form):
    """Groups whose rows share too little go to the per-row kernel: a batch
    whose first 40 groups are a chunk's rows (the plan) and the rest
    unrelated rows (row by row) gives the reference on every row."""
    g = np.random.default_rng(77)
    rows, heads, pool_pages = 640, 32, 400
    q8, w = _queries(g, rows, heads, heads)
    k8, ks = W.quantize_rows(g.standard_normal((pool_pages * 64, 128), dtype=np.float32))
    native = W.pack_pages(k8, ks)
    table = _tables(g, rows, pool_pages, shared_pages=40, take=28, private=2, unrelated_rows=set(range(320, rows)))
    blocks = table.shape[1]
    lens = g.integers(1, blocks * 64 + 1, rows).astype(np.int32)
    width = blocks * 64
    got = _run(dev, q8, w, native, table, lens, width, True, True)
    pool, tab = _padded(native, table, width)
    assert_scores_rel(got, O.paged_logits(q8, w, pool, tab, lens, width))


@pytest.mark.parametrize("heads", [32, 64])
def test_union_plan_rows_bitwise_across_kernels(dev, form, heads):
    """A row gets the same bits whichever kernel scores it: row 8 repeats
    row 0 (query, weights, table, length) inside a group of otherwise
    unrelated rows, which the plan hands to the per-row kernel, while row 0's
    group is scored over its union."""
    g = np.random.default_rng(heads)
    rows, pool_pages = 528, 300
    q8, w = _queries(g, rows, heads, heads)
    k8, ks = W.quantize_rows(g.standard_normal((pool_pages * 64, 128), dtype=np.float32))
    native = W.pack_pages(k8, ks)
    table = _tables(g, rows, pool_pages, shared_pages=40, take=30, private=2, unrelated_rows=set(range(9, 16)))
    blocks = table.shape[1]
    lens = g.integers(blocks * 32, blocks * 64 + 1, rows).astype(np.int32)
    q8[8], w[8], table[8], lens[8] = q8[0], w[0], table[0], lens[0]
    width = blocks * 64
    got = _run(dev, q8, w, native, table, lens, width, True, True).astype(np.float32)
    assert np.array_equal(got[8].view(np.uint32), got[0].view(np.uint32))
    pool, tab = _padded(native, table, width)
    assert_scores_rel(got.astype(np.float64), O.paged_logits(q8, w, pool, tab, lens, width))


def test_union_plan_probe_overflow_falls_back(dev, form):
    """A group whose pages all land on one slot of the plan's hash set (68
    pages of a 34000-page pool with the same multiplicative hash into 512
    slots) probes past the plan's limit and is scored row by row; every row
    still gives the reference."""
    g = np.random.default_rng(5)
    rows, heads, slots, pool_pages = 520, 32, 64, 34000
    width = slots * 64  # 8 x 64 pairs per group: a 512-slot hash set
    p = np.arange(pool_pages, dtype=np.uint64)
    h = ((p * np.uint64(0x9E3779B1)) & np.uint64(0xFFFFFFFF)) >> np.uint64(23)
    vals, counts = np.unique(h, return_counts=True)
    colliding = p[h == vals[np.argmax(counts)]].astype(np.int32)
    assert len(colliding) >= 66
    others = np.setdiff1d(np.arange(1024, dtype=np.int32), colliding)[:90]
    used = np.union1d(colliding, others)
    native = np.zeros((pool_pages, 8448), np.uint8)
    k8, ks = W.quantize_rows(g.standard_normal((len(used) * 64, 128), dtype=np.float32))
    native[used] = W.pack_pages(k8, ks)
    q8, w = _queries(g, rows, heads, heads)
    table = np.empty((rows, slots), np.int32)
    for r in range(rows):
        table[r] = g.permutation(colliding)[:slots] if r < 8 else g.choice(others, slots)
    lens = g.integers(width // 2, width + 1, rows).astype(np.int32)
    lens[:8] = width  # the first group lists every colliding page
    got = _run(dev, q8, w, native, table, lens, width, True, True)
    pool, tab = _padded(native, table, width)
    assert_scores_rel(got, O.paged_logits(q8, w, pool, tab, lens, width))


@pytest.mark.parametrize("heads", [32, 64])
def test_union_plan_repeats_and_empty_groups(dev, form, heads):
    """Rows that list one page three times (each later slot in an entry of its
    own), a group whose rows list no valid page at all (every live column
    scores 0, nothing is staged), and a group of empty rows, beside ordinary
    chunk rows."""
    g = np.random.default_rng(heads + 3)
    rows, pool_pages = 528, 200
    q8, w = _queries(g, rows, heads, heads)
    k8, ks = W.quantize_rows(g.standard_normal((pool_pages * 64, 128), dtype=np.float32))
    native = W.pack_pages(k8, ks)
    table = _tables(g, rows, pool_pages, shared_pages=40, take=30, private=2)
    blocks = table.shape[1]
    table[0, 3] = table[0, 9] = table[0, 17] = table[0, 1]       # three repeats in row 0
    table[5, :6] = table[5, 10]                                   # a page six times in row 5
    table[8:16] = -1                                              # group 1: no valid page
    table[16:24, ::2] = pool_pages + 7                            # group 2: every other slot out of the pool
    lens = g.integers(blocks * 32, blocks * 64 + 1, rows).astype(np.int32)
    lens[24:32] = 0                                               # group 3: empty rows
    width = blocks * 64 + 64
    got = _run(dev, q8, w, native, table, lens, width, True, True)
    pool, tab = _padded(native, table, width)
    ref = O.paged_logits(q8, w, pool, tab, lens, width)
    assert (got[8:16][np.isfinite(ref[8:16])] == 0).all()
    assert np.isneginf(got[24:32]).all()
    assert_scores_rel(got, ref)


@pytest.mark.parametrize("heads,relu,pool_pages", [(64, True, 120), (64, True, 80), (32, True, 120),
                                                    (32, False, 80), (20, True, 120), (17, True, 80)])
def test_page_major_bitwise_equals_row_kernel(dev, heads, relu, pool_pages):
    """The page-major form gives every row the bits of the row-by-row kernel
    (the same products in the same order): 600 rows scored page-major, then
    their first 300 alone (a batch of at most 512 rows goes row by row); 20
    and 17 heads load through the partial head block's range checks (16
    heads or fewer stay row by row at any batch size).  A 120-page
    pool (more than twice a row's 42 pages) is cut into chunks of listed
    pages, an 80-page one into chunks of consecutive pool pages."""
    g = np.random.default_rng(heads * 3 + relu + pool_pages)
    rows = 600
    q8, w = _queries(g, rows, heads, heads)
    if not relu:
        w *= np.where(g.random(w.shape) < 0.5, -1, 1).astype(np.float32)
    k8, ks = W.quantize_rows(g.standard_normal((pool_pages * 64, 128), dtype=np.float32))
    native = W.pack_pages(k8, ks)
    table = _tables(g, rows, pool_pages, shared_pages=50, take=36, private=3)
    blocks = table.shape[1]
    lens = g.integers(1, blocks * 64 + 1, rows).astype(np.int32)
    width = blocks * 64 + 64
    prev = SC.page_major(True)
    try:
        both = _run(dev, q8, w, native, table, lens, width, relu, True).astype(np.float32)
    finally:
        SC.page_major(prev)
    alone = _run(dev, q8[:300], w[:300], native, table[:300], lens[:300], width, relu, True).astype(np.float32)
    assert np.array_equal(both[:300].view(np.uint32), alone.view(np.uint32))
    pool, tab = _padded(native, table, width)
    if relu:
        assert_scores_rel(both.astype(np.float64), O.paged_logits(q8, w, pool, tab, lens, width))
