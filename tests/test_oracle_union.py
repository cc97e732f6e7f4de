"""Oracle of the shared sink + tail union (stage_union, tables, normalize,
map_topk) and of the per-row staging with a published index end, pinned
against the reference's own answers (experiments/tail_union_lab_20261021/
README.md:54-63, test_published_end.py:6-34) and against the independent
candidate-set rule those tests use: a row of visible length n scores exactly
sink [0, min(n, S)) + the last W positions + every position at or past the
published index end."""
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
from oracle import v1 as O  # noqa: E402

# (history, rows, sink, window, indexed_end): test_published_end.py:17-18
REFERENCE_CASES = [(65536, 4096, 64, 2048, 65536), (65536, 4096, 64, 2048, 61440), (2051, 65, 17, 0, 1025),
                   (17, 129, 65, 128, 0), (0, 65, 0, 0, 0)]


def test_readme_example_64k_4k():
    # README.md:54-63: history 65536, 4096 rows, sink 64, window 2048, published end 65536
    lens = np.arange(65537, 65537 + 4096)
    rows = {0: (64, 63489, 2112), 2047: (64, 65536, 2112), 2048: (64, 65536, 2113), 4095: (64, 65536, 4160)}
    for r, want in rows.items():
        assert O.union_bounds(int(lens[r]), 65536, 64, 2048) == want
    assert O.union_pages(lens, 65536, 64, 2048) == (1, 992, 1088, 97)
    # the last row keeps 65537 although it is outside its 2K window; the bucket
    # formula of the production staging (kernels.py:539) would have dropped it
    s, t, c = O.union_bounds(69632, 65536, 64, 2048)
    assert t <= 65537 < 69632
    old_sink, old_tail = O._bounds(69632, 2048, 64)
    assert old_tail == 67584 and not old_tail <= 65537


@pytest.mark.parametrize("case", REFERENCE_CASES + [(300, 50, 3, 5, 123), (5000, 7, 100, 10, 6000)])
def test_candidates_are_sink_window_and_unindexed(case):
    h, rows, S, W, end = case
    for n in range(h + 1, h + rows + 1):
        s, t, c = O.union_bounds(n, end, S, W)
        ids = list(range(s)) + list(range(t, n))
        expected = set(range(min(n, S))) | set(range(max(0, n - W), n)) | set(range(min(end, n), n))
        assert len(ids) == len(set(ids)) == c and set(ids) == expected


def _pool(g, pages):
    pool = g.integers(0, 256, (pages, 8448), dtype=np.uint8)
    pool[:, 8192:] = (g.random((pages, 64), dtype=np.float32) + 0.01).view(np.uint8)
    return pool


@pytest.mark.parametrize("case", [(2051, 65, 17, 0, 1025), (17, 129, 65, 128, 0), (0, 65, 0, 0, 0),
                                  (1000, 65, 64, 128, 1000), (4096, 64, 64, 300, 3001)])
def test_union_equals_per_row_staging(case):
    # test_bench.py:53-64: the union read back per row equals per-row staging byte for byte,
    # and union pages are the source pages of [0, sp) + [tp, ep)
    h, rows, S, W, end = case
    g = np.random.default_rng(h + rows)
    npg = max(1, -(-(h + rows) // 64))
    pool = _pool(g, npg)
    nt = g.permutation(npg).astype(np.int32)
    lens = np.arange(h + 1, h + rows + 1, dtype=np.int32)
    scratch = max(1, -(-O.union_bounds(h + rows, end, S, W)[2] // 64))
    union = np.full((npg + 2, 8448), 165, np.uint8)
    meta, desc = O.stage_union(pool, nt, lens, end, union, S, W)
    sp, tp, ep, total = (int(v) for v in desc)
    ids = list(range(sp)) + list(range(tp, ep))
    assert total == len(ids) and np.array_equal(union[:total], pool[nt[ids]])
    assert (union[total:] == 165).all()
    assert meta.tolist() == [list(O.union_bounds(int(n), end, S, W)) for n in lens]
    per_row = np.full((rows * scratch, 8448), 165, np.uint8)
    O.stage_tail(pool, np.tile(nt, (rows, 1)), lens, per_row, 0, scratch, S, W, indexed_end=end)
    restored = O.union_reconstruct(union, meta, desc, scratch)
    written = [i for i in range(rows * scratch) if not (per_row[i] == 165).all()]
    assert sorted(restored) == written
    for i, page in restored.items():
        assert np.array_equal(page, per_row[i])


def _content_score(pages):
    """A score that depends only on a token's bytes: what any scoring kernel
    would give two identical copies of one key."""
    k = pages[:, :8192].reshape(-1, 64, 128).astype(np.int64)
    w = (np.arange(128) % 7 + 1)
    s = pages[:, 8192:].copy().view(np.float32).reshape(-1, 64)
    return ((k * w).sum(-1).astype(np.float32) * s).astype(np.float32)  # [pages, 64]


def _fixture(h, rows, S, W, end, max_take, seed):
    """fine_pool_shared_20261021/experiment.py:15-46 at small size."""
    g = np.random.default_rng(seed)
    npg = max(1, -(-(h + rows) // 64))
    cap = max(64, max_take)
    native = _pool(g, npg)
    nt = g.permutation(npg).astype(np.int32)
    lens = np.arange(h + 1, h + rows + 1, dtype=np.int32)
    takes = g.integers(0, max_take + 1, rows).astype(np.int32)
    selected = ((np.arange(max_take)[None] + np.arange(rows)[:, None]) % cap).astype(np.int32)
    members = np.concatenate([np.arange(64), 64 + g.permutation(h - 64)[:cap * 64 - 64]]).astype(np.int32)
    members = members.reshape(cap, 64)
    nk = native[:, :8192].reshape(-1, 64, 128)
    ns = native[:, 8192:].copy().view(np.float32).reshape(-1, 64)
    page, off = nt[members // 64], members % 64
    reordered = np.zeros((cap, 8448), np.uint8)
    reordered[:, :8192] = nk[page, off].reshape(cap, 8192)
    reordered[:, 8192:] = ns[page, off].view(np.uint8).reshape(cap, 256)
    c_max = O.union_bounds(h + rows, end, S, W)[2]
    scratch = max(1, -(-c_max // 64))
    width = -(-(max_take * 64 + c_max + 128) // 256) * 256
    return dict(native=native, nt=nt, lens=lens, takes=takes, selected=selected, members=members,
                reordered=reordered, cap=cap, scratch=scratch, width=width, max_take=max_take)


def _arm(f, end, S, W, shared):
    """prepare -> score (content function over the single fine pool) -> normalize."""
    rows = len(f["lens"])
    cap, scratch, width = f["cap"], f["scratch"], f["width"]
    extra = (f["native"].shape[0] + 2) if shared else rows * scratch
    fine = np.zeros((cap + extra, 8448), np.uint8)
    fine[:cap] = f["reordered"]
    desc = np.zeros(4, np.int32)
    if shared:
        _, desc = O.stage_union(f["native"], f["nt"], f["lens"], end, fine[cap:], S, W)
    else:
        O.stage_tail(f["native"], np.tile(f["nt"], (rows, 1)), f["lens"], fine, cap, scratch, S, W,
                     indexed_end=end)
    ft, dg, cl = O.union_tables(f["lens"], end, f["takes"], f["selected"], desc, cap, f["max_take"], scratch,
                                width // 64, S, W, shared)
    score = _content_score(fine)
    raw = np.full((rows, width), np.float32(7.0), np.float32)
    for r in range(rows):
        j = np.arange(int(dg[r]))
        raw[r, j] = score[ft[r, j // 64], j % 64]
    out = O.union_normalize(raw, f["lens"], end, f["takes"], f["selected"], f["members"], f["max_take"], width, S,
                            W, shared)
    return out, cl, ft, fine


@pytest.mark.parametrize("case", [(4096, 4, 17, 0, 4096), (4096, 24, 64, 256, 3500), (5000, 16, 64, 200, 5000)])
def test_shared_and_per_row_give_one_canonical_order(case):
    # fine_pool_shared_20261021/test_and_bench.py:8-40: both layouts restore the same canonical
    # scores; the canonical order is history members (masked to [s, t), < n, < end), then sink, then tail
    h, rows, S, W, end = case
    f = _fixture(h, rows, S, W, end, 8, h + rows)
    a, cla, fta, fa = _arm(f, end, S, W, False)
    b, clb, ftb, fb = _arm(f, end, S, W, True)
    assert np.array_equal(cla, clb) and np.array_equal(a, b)
    assert fta.min() >= 0 and fta.max() < fa.shape[0] and ftb.min() >= 0 and ftb.max() < fb.shape[0]
    native_score = _content_score(f["native"])
    reordered_score = _content_score(f["reordered"])
    for r in range(rows):
        n, take = int(f["lens"][r]), int(f["takes"][r])
        s, t, c = O.union_bounds(n, end, S, W)
        tail = list(range(s)) + list(range(t, n))
        exp = np.full(f["width"], -np.inf, np.float32)
        for j in range(take * 64):
            m = int(f["members"][f["selected"][r, j // 64], j % 64])
            if s <= m < t and m < n and m < end:
                exp[j] = reordered_score[f["selected"][r, j // 64], j % 64]
        for x, lg in enumerate(tail):
            exp[take * 64 + x] = native_score[f["nt"][lg // 64], lg % 64]
        assert np.array_equal(b[r], exp)
        assert int(clb[r]) == take * 64 + c


def test_map_topk_positions_and_slots():
    h, rows, S, W, end = 4096, 24, 64, 256, 3500
    f = _fixture(h, rows, S, W, end, 8, 5)
    scores, _, _, _ = _arm(f, end, S, W, True)
    top = 300
    ids = np.argsort(-scores, axis=1, kind="stable")[:, :top].astype(np.int64)
    values = np.take_along_axis(scores, ids, 1)
    logical, slots = O.union_map_topk(ids, values, f["lens"], end, f["takes"], f["selected"], f["members"], f["nt"],
                                      S, W)
    for r in range(rows):
        n, take = int(f["lens"][r]), int(f["takes"][r])
        s, t, c = O.union_bounds(n, end, S, W)
        cand = [int(f["members"][f["selected"][r, j // 64], j % 64]) for j in range(take * 64)]
        cand += list(range(s)) + list(range(t, n))
        for i in range(top):
            if values[r, i] == -np.inf:
                assert logical[r, i] == -1 and slots[r, i] == -1
            else:
                lg = cand[ids[r, i]]
                assert logical[r, i] == lg and slots[r, i] == f["nt"][lg // 64] * 64 + lg % 64
        good = logical[r][logical[r] >= 0]
        assert len(np.unique(good)) == len(good)


@pytest.mark.parametrize("case", [(4096, 24, 64, 256, 3500), (5000, 16, 64, 200, 5000)])
def test_split_scoring_restores_the_same_canonical_scores(case):
    # every row scored once against all history pages and once against the union in union
    # coordinates: normalize_split gives the canonical vector normalize gives from per-row tables
    h, rows, S, W, end = case
    f = _fixture(h, rows, S, W, end, 8, h + rows)
    b, _, _, fine = _arm(f, end, S, W, True)
    desc = np.array(O.union_pages(f["lens"], end, S, W), np.int32)
    total = int(desc[3])
    cap = f["cap"]
    score = _content_score(fine)
    hist = np.repeat(score[:cap].reshape(1, -1), rows, 0)
    uni = np.repeat(score[cap:cap + total].reshape(1, -1), rows, 0)
    split = O.union_normalize_split(hist, uni, f["lens"], end, f["takes"], f["selected"], f["members"], desc,
                                    f["width"], S, W)
    assert np.array_equal(split, b)
