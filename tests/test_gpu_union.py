"""Shared sink + tail union on the GPU against the oracle: stage_union (with
the reference's cases, dynamic published ends and HIP-graph replays), the
published-end per-row staging, tables / normalize / map_topk, and the whole
prepare -> FP8 score -> normalize -> Top-K -> map chain, shared against
per-row staging (experiments/tail_union_lab_20261021/test_bench.py,
test_published_end.py; experiments/fine_pool_shared_20261021/test_and_bench.py)."""
import importlib
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
from oracle import v1 as O  # noqa: E402

pytestmark = pytest.mark.gpu

TU = importlib.import_module("10_20_amd.tailunion")
SC = importlib.import_module("10_20_amd.scoring")
TK = importlib.import_module("10_20_amd.topk")
W_ = importlib.import_module("10_20_amd.workloads")
DEV = "cuda:0"


def T(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return t if dtype is None else t.to(dtype)


def H(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def cdiv(a, b):
    return -(-a // b)


class Case:
    """test_bench.py:12-37: one request, rows with lengths h+1 .. h+rows."""

    def __init__(self, h, rows, S, W, end, min_end=None, seed=0):
        g = np.random.default_rng(seed + h + rows)
        self.h, self.rows, self.S, self.W, self.end = h, rows, S, W, end
        lower = end if min_end is None else min_end
        self.np = max(1, cdiv(h + rows, 64))
        pool = g.integers(0, 256, (self.np, 8448), dtype=np.uint8)
        pool[:, 8192:] = (g.random((self.np, 64), dtype=np.float32) + 0.01).view(np.uint8)
        self.pool = pool
        self.nt = g.permutation(self.np).astype(np.int32)
        self.lens = np.arange(h + 1, h + rows + 1, dtype=np.int32)
        self.scratch = max(1, cdiv(O.union_bounds(h + rows, lower, S, W)[2], 64))
        first_tail = O.union_bounds(h + 1, lower, S, W)[1]
        self.cap = min(self.np, cdiv(S, 64) + cdiv(h + rows, 64) - first_tail // 64 + 2)
        self.d_pool, self.d_nt, self.d_lens = T(pool), T(self.nt), T(self.lens)
        self.d_end = T(np.int32([end]))
        self.u = torch.full((self.cap, 8448), 165, device=DEV, dtype=torch.uint8)
        self.meta = torch.empty((rows, 3), device=DEV, dtype=torch.int32)
        self.desc = torch.empty(4, device=DEV, dtype=torch.int32)
        self.plan = TU.PreparedStage(self.d_pool, self.d_nt, self.d_lens, self.d_end, self.u, self.meta, self.desc,
                                     S, W)

    def expect(self, end, nt):
        u = np.full((self.cap, 8448), 165, np.uint8)
        meta, desc = O.stage_union(self.pool, nt, self.lens, end, u, self.S, self.W)
        return u, meta, desc

    def check(self, end, nt):
        u, meta, desc = self.expect(end, nt)
        assert np.array_equal(H(self.desc), desc)
        assert np.array_equal(H(self.meta), meta)
        total = int(desc[3])
        assert np.array_equal(H(self.u[:total]), u[:total])


@pytest.mark.parametrize("case", [(65536, 4096, 64, 2048, 65536), (65536, 4096, 64, 2048, 61440),
                                  (2051, 65, 17, 0, 1025), (17, 129, 65, 128, 0), (0, 65, 0, 0, 0),
                                  (65549, 1024, 17, 2049, 65549), (262144, 4096, 64, 2048, 262144)])
def test_stage_union_vs_oracle(case):
    c = Case(*case)
    print("stage_union", case, flush=True)
    c.plan()
    c.check(c.end, c.nt)
    if case[0] == 65536 and case[4] == 65536:
        assert H(c.meta)[-1].tolist() == [64, 65536, 4160] and H(c.desc).tolist() == [1, 992, 1088, 97]


def test_dynamic_indexed_end_and_graph_replay():
    # test_published_end.py:27-36: one captured graph, same lengths, the published end and the page
    # table changed in place between replays
    c = Case(65536, 4096, 64, 2048, 65536, min_end=61001)
    c.plan()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        c.plan()
    nt = c.nt.copy()
    for end in (65536, 61440, 61001, 65536):
        c.d_end.fill_(end)
        nt = nt[::-1].copy()
        c.d_nt.copy_(T(nt))
        c.u.fill_(165)
        g.replay()
        torch.cuda.synchronize()
        c.check(end, nt)
    # lengths shrink by 37 between replays (test_bench.py:72-80)
    c.d_lens.sub_(37)
    c.lens = c.lens - 37
    c.d_end.fill_(65536)
    g.replay()
    torch.cuda.synchronize()
    c.check(65536, nt)


@pytest.mark.parametrize("case", [(2051, 65, 17, 0, 1025), (17, 129, 65, 128, 0), (1000, 65, 64, 128, 1000),
                                  (4096, 64, 64, 300, 3001)])
def test_published_staging_vs_oracle_and_union(case):
    c = Case(*case)
    rows, scratch = c.rows, c.scratch
    per_row = torch.full((rows * scratch, 8448), 165, device=DEV, dtype=torch.uint8)
    owners = torch.arange(rows, device=DEV, dtype=torch.int32)
    nts = T(np.tile(c.nt, (rows, 1)))
    TU.stage_tail_shared[(rows, scratch)](c.d_pool, c.d_pool.view(torch.float32), nts, c.d_lens, c.d_end, per_row,
                                          per_row.view(torch.float32), owners, 0, c.np, scratch, c.S, c.W, rows, 1)
    exp = np.full((rows * scratch, 8448), 165, np.uint8)
    O.stage_tail(c.pool, np.tile(c.nt, (rows, 1)), c.lens, exp, 0, scratch, c.S, c.W, indexed_end=c.end)
    got = H(per_row)
    assert np.array_equal(got, exp)
    c.plan()
    restored = O.union_reconstruct(H(c.u), H(c.meta), H(c.desc), scratch)
    for i, page in restored.items():
        assert np.array_equal(page, got[i])


def _tables_inputs(h, rows, S, W, end, max_take, seed):
    g = np.random.default_rng(seed)
    cap = max(64, max_take)
    lens = np.arange(h + 1, h + rows + 1, dtype=np.int32)
    takes = g.integers(0, max_take + 1, rows).astype(np.int32)
    selected = ((np.arange(max_take)[None] + np.arange(rows)[:, None]) % cap).astype(np.int32)
    members = np.concatenate([np.arange(64), 64 + g.permutation(h - 64)[:cap * 64 - 64]]).astype(np.int32)
    c_max = O.union_bounds(h + rows, end, S, W)[2]
    width = cdiv(max_take * 64 + c_max + 128, 256) * 256
    return dict(lens=lens, takes=takes, selected=selected, members=members.reshape(cap, 64), cap=cap,
                scratch=max(1, cdiv(c_max, 64)), width=width, max_take=max_take)


@pytest.mark.parametrize("case", [(4096, 4, 17, 0, 4096), (65536, 512, 64, 2048, 65536), (65536, 300, 64, 2048, 61001),
                                  (5000, 64, 64, 200, 5000)])
@pytest.mark.parametrize("shared", [False, True])
def test_tables_normalize_map_vs_oracle(case, shared):
    h, rows, S, W, end = case
    f = _tables_inputs(h, rows, S, W, end, 40, h + rows)
    lens = f["lens"]
    desc = np.array(O.union_pages(lens, end, S, W), np.int32)
    fp = f["width"] // 64
    d_end = T(np.int32([end]))
    ft = torch.full((rows, fp), -7, device=DEV, dtype=torch.int32)
    dg = torch.empty((rows, 1), device=DEV, dtype=torch.int32)
    cl = torch.empty(rows, device=DEV, dtype=torch.int32)
    d_lens, d_takes, d_sel, d_mem = T(lens), T(f["takes"]), T(f["selected"]), T(f["members"])
    TU.tables[(rows,)](d_lens, d_end, d_takes, d_sel, T(desc), ft, dg, cl, f["cap"], f["max_take"], f["scratch"], fp,
                       S, W, 1 << (fp - 1).bit_length(), shared)
    e_ft, e_dg, e_cl = O.union_tables(lens, end, f["takes"], f["selected"], desc, f["cap"], f["max_take"],
                                      f["scratch"], fp, S, W, shared)
    assert np.array_equal(H(ft), e_ft) and np.array_equal(H(dg).reshape(-1), e_dg) and np.array_equal(H(cl), e_cl)
    g = np.random.default_rng(rows)
    raw = g.standard_normal((rows, f["width"] + 4)).astype(np.float32)
    out = torch.full((rows, f["width"]), 3.0, device=DEV)
    d_raw = T(raw)[:, :f["width"]]
    TU.normalize[(rows, cdiv(f["width"], 256))](d_raw, d_lens, d_end, d_takes, d_sel, d_mem, out, f["max_take"],
                                                f["width"], d_raw.stride(0), S, W, 256, shared)
    e_out = O.union_normalize(raw[:, :f["width"]], lens, end, f["takes"], f["selected"], f["members"],
                              f["max_take"], f["width"], S, W, shared)
    assert np.array_equal(H(out), e_out)
    top = 2048 if f["width"] >= 2048 else 256
    vals, ids = torch.topk(out, top, dim=1)
    nt = g.permutation(cdiv(h + rows, 64)).astype(np.int32)
    lg = torch.empty((rows, top), device=DEV, dtype=torch.int32)
    sl = torch.empty_like(lg)
    TU.map_topk[(rows,)](ids, vals, d_lens, d_end, d_takes, d_sel, d_mem, T(nt), lg, sl, f["max_take"], top, S, W,
                         1 << (top - 1).bit_length())
    e_lg, e_sl = O.union_map_topk(H(ids), H(vals), lens, end, f["takes"], f["selected"], f["members"], nt, S, W)
    assert np.array_equal(H(lg), e_lg) and np.array_equal(H(sl), e_sl)


class Chain:
    """fine_pool_shared_20261021/experiment.py:15-95 with this build's FP8 scoring
    and Top-K: prepare -> score over ONE fine pool -> normalize -> Top-2048 -> map."""

    def __init__(self, h, rows, S, W, end, max_take, shared, seed=1):
        g = np.random.default_rng(seed)
        self.h, self.rows, self.S, self.W, self.end, self.shared = h, rows, S, W, end, shared
        npg = max(1, cdiv(h + rows, 64))
        cap = max(64, max_take)
        k8, ks = W_.quantize_rows(g.standard_normal((npg * 64, 128)).astype(np.float32))
        native = W_.pack_pages(k8, ks)
        nt = g.permutation(npg).astype(np.int32)
        members = np.concatenate([np.arange(64), 64 + g.permutation(h - 64)[:cap * 64 - 64]]).astype(np.int32)
        members = members.reshape(cap, 64)
        nk = native[:, :8192].reshape(-1, 64, 128)
        ns = native[:, 8192:].copy().view(np.float32).reshape(-1, 64)
        page, off = nt[members // 64], members % 64
        reordered = np.zeros((cap, 8448), np.uint8)
        reordered[:, :8192] = nk[page, off].reshape(cap, 8192)
        reordered[:, 8192:] = ns[page, off].view(np.uint8).reshape(cap, 256)
        self.native, self.nt, self.members = native, nt, members
        c_max = O.union_bounds(h + rows, end, S, W)[2]
        self.scratch = max(1, cdiv(c_max, 64))
        self.width = cdiv(max_take * 64 + c_max + 128, 256) * 256
        first_tail = O.union_bounds(h + 1, end, S, W)[1]
        union_cap = min(npg, cdiv(S, 64) + cdiv(h + rows, 64) - first_tail // 64 + 2)
        self.cap, self.max_take, self.np = cap, max_take, npg
        extra = union_cap if shared else rows * self.scratch
        self.fine = torch.zeros((cap + extra, 8448), device=DEV, dtype=torch.uint8)
        self.fine[:cap] = T(reordered)
        self.d_native, self.d_nt, self.d_mem = T(native), T(nt), T(members)
        self.lens = np.arange(h + 1, h + rows + 1, dtype=np.int32)
        self.takes = np.full(rows, max_take, np.int32)
        self.selected = ((np.arange(max_take)[None] + np.arange(rows)[:, None]) % cap).astype(np.int32)
        self.d_lens, self.d_takes, self.d_sel = T(self.lens), T(self.takes), T(self.selected)
        self.d_end = T(np.int32([end]))
        q8, _ = W_.quantize_rows(g.standard_normal((rows * 32, 128)).astype(np.float32))
        self.q = T(q8.reshape(rows, 1, 32, 128)).view(torch.float8_e4m3fn)
        self.w = T((g.random((rows, 32), dtype=np.float32) / 32).astype(np.float32))
        self.meta = torch.empty((rows, 3), device=DEV, dtype=torch.int32)
        self.desc = torch.zeros(4, device=DEV, dtype=torch.int32)
        self.table = torch.empty((rows, self.width // 64), device=DEV, dtype=torch.int32)
        self.dglens = torch.empty((rows, 1), device=DEV, dtype=torch.int32)
        self.clens = torch.empty(rows, device=DEV, dtype=torch.int32)
        self.raw = torch.empty((rows, self.width), device=DEV)
        self.scores = torch.empty((rows, self.width), device=DEV)
        self.ids = torch.empty((rows, 2048), device=DEV, dtype=torch.int32)
        self.identity = torch.arange(cdiv(self.width, 64), device=DEV, dtype=torch.int32)[None].expand(rows, -1)
        self.identity = self.identity.contiguous()
        self.slots_raw = torch.empty_like(self.ids)
        self.logical = torch.empty_like(self.ids)
        self.slots = torch.empty_like(self.ids)
        if shared:
            self.stage = TU.PreparedStage(self.d_native, self.d_nt, self.d_lens, self.d_end, self.fine[cap:],
                                          self.meta, self.desc, S, W)
        self.owners = torch.arange(rows, device=DEV, dtype=torch.int32)
        self.nts = self.d_nt[None].expand(rows, -1).contiguous()

    def prepare(self):
        if self.shared:
            self.stage()
        else:
            TU.stage_tail_shared[(self.rows, self.scratch)](
                self.d_native, self.d_native.view(torch.float32), self.nts, self.d_lens, self.d_end, self.fine,
                self.fine.view(torch.float32), self.owners, self.cap, self.np, self.scratch, self.S, self.W,
                self.rows, 1)
        TU.tables[(self.rows,)](self.d_lens, self.d_end, self.d_takes, self.d_sel, self.desc, self.table,
                                self.dglens, self.clens, self.cap, self.max_take, self.scratch, self.width // 64,
                                self.S, self.W, 256, self.shared)

    def score(self):
        SC.fp8_paged_mqa_logits(self.q, self.fine.view(-1, 64, 1, 132), self.w, self.dglens, self.table, None,
                                self.width, clean_logits=False, out=self.raw)
        TU.normalize[(self.rows, cdiv(self.width, 256))](self.raw, self.d_lens, self.d_end, self.d_takes, self.d_sel,
                                                         self.d_mem, self.scores, self.max_take, self.width,
                                                         self.raw.stride(0), self.S, self.W, 256, self.shared)

    def select(self):
        TK.topk_transform_512_v2(self.scores, self.clens, self.identity, self.slots_raw, 64, None, self.ids)
        TU.map_topk_scores(self.ids, self.scores, self.d_lens, self.d_end, self.d_takes, self.d_sel, self.d_mem,
                           self.d_nt, self.logical, self.slots, self.max_take, self.S, self.W)

    def run(self):
        self.prepare()
        self.score()
        self.select()
        torch.cuda.synchronize()


@pytest.mark.parametrize("case", [(65536, 1024, 64, 2048, 65536), (65549, 256, 17, 2049, 61001),
                                  (4096, 4, 17, 0, 4096)])
def test_chain_shared_equals_per_row(case):
    # test_and_bench.py:8-40: the same canonical scores, Top-K and slots from both layouts; scores
    # within tolerance of the dequantised formula on the first, middle and last rows
    h, rows, S, W, end = case
    print("chain", case, flush=True)
    a = Chain(h, rows, S, W, end, 40, False)
    b = Chain(h, rows, S, W, end, 40, True)
    a.run()
    b.run()
    assert torch.equal(a.clens, b.clens)
    assert torch.equal(a.scores, b.scores)
    assert torch.equal(a.logical, b.logical) and torch.equal(a.slots, b.slots)
    # the values form of map_topk (kernels.py:62-76) agrees with values read from the scores
    values = b.scores.gather(1, b.ids.clamp_min(0).long())
    lg2, sl2 = torch.empty_like(b.logical), torch.empty_like(b.slots)
    TU.map_topk[(rows,)](b.ids, values, b.d_lens, b.d_end, b.d_takes, b.d_sel, b.d_mem, b.d_nt, lg2, sl2, b.max_take,
                         2048, S, W, 2048)
    assert torch.equal(lg2, b.logical) and torch.equal(sl2, b.slots)
    e_lg, e_sl = O.union_map_topk(H(b.ids), H(values), b.lens, end, b.takes, b.selected, b.members, b.nt, S, W)
    assert np.array_equal(H(b.logical), e_lg) and np.array_equal(H(b.slots), e_sl)
    scores, lens = H(b.scores), b.lens
    q = H(b.q.view(torch.uint8)).reshape(rows, 32, 128)
    w = H(b.w)
    nk = b.native[:, :8192].reshape(-1, 64, 128)
    ns = b.native[:, 8192:].copy().view(np.float32).reshape(-1, 64)
    for r in sorted({0, rows // 2, rows - 1}):
        n, take = int(lens[r]), int(b.takes[r])
        s, t, c = O.union_bounds(n, end, S, W)
        ids = [int(b.members[b.selected[r, j // 64], j % 64]) for j in range(take * 64)]
        ids += list(range(s)) + list(range(t, n))
        ids = np.array(ids)
        k = O.e4m3_decode(nk[b.nt[ids // 64], ids % 64]).astype(np.float64)
        sc = ns[b.nt[ids // 64], ids % 64].astype(np.float64)
        qq = O.e4m3_decode(q[r]).astype(np.float64)
        terms = np.maximum(qq @ k.T, 0) * w[r][:, None]
        ref = terms.sum(0) * sc
        keep = np.ones(len(ids), bool)
        keep[:take * 64] = [(s <= m < t and m < n and m < end) for m in ids[:take * 64]]
        got = scores[r, :len(ids)]
        assert np.isneginf(got[~keep]).all() and np.isneginf(scores[r, len(ids):]).all()
        bound = 1e-2 * np.abs(ref) + 2.0 ** -16 * (np.abs(terms).sum(0) * sc)
        assert (np.abs(got[keep] - ref[keep]) <= bound[keep]).all()
        good = H(b.logical)[r]
        good = good[good >= 0]
        assert len(np.unique(good)) == len(good)
        phys = b.nt[good // 64] * 64 + good % 64
        assert np.array_equal(H(b.slots)[r][H(b.logical)[r] >= 0], phys)


def test_unindexed_token_reaches_last_row_topk():
    # test_and_bench.py:61-67: token 65537 (past the published end, outside the last row's 2K
    # window) scores highest for the last row and is among its Top-2048
    b = Chain(65536, 4096, 64, 2048, 65536, 40, True)
    token = 65537
    page, off = int(b.nt[token // 64]), token % 64
    b.d_native[page, off * 128:(off + 1) * 128] = 0
    b.d_native[page, off * 128] = 0x7E  # e4m3 448
    b.d_native.view(torch.float32)[page, 2048 + off] = 1.0
    qq = b.q.view(torch.uint8)[-1, 0]
    qq.zero_()
    qq[:, 0] = 0x38  # e4m3 1.0 in dim 0 of every head
    b.w[-1].fill_(1 / 32)
    b.run()
    lg = H(b.logical)[-1]
    assert token in lg.tolist()


@pytest.mark.parametrize("end", [-5, 10 ** 6])
def test_stage_union_published_end_outside_lengths(end):
    # a negative published end counts as 0 (every visible token is a tail candidate); one past every
    # length leaves sink + window only (union.py:10-14)
    c = Case(3000, 70, 17, 100, end)
    c.plan()
    c.check(end, c.nt)


@pytest.mark.parametrize("case", [(65536, 300, 64, 2048, 61001), (5000, 64, 64, 200, 5000)])
def test_spans_and_normalize_split_vs_oracle(case):
    h, rows, S, W, end = case
    f = _tables_inputs(h, rows, S, W, end, 40, h + rows)
    lens = f["lens"]
    desc = np.array(O.union_pages(lens, end, S, W), np.int32)
    d_end, d_desc = T(np.int32([end])), T(desc)
    spans = torch.empty(rows, device=DEV, dtype=torch.int32)
    TU.union_spans(T(lens), d_end, d_desc, spans, S, W)
    sp, tp, total = int(desc[0]), int(desc[1]), int(desc[3])
    for r, n in enumerate(lens):
        s, t, c = O.union_bounds(int(n), end, S, W)
        # the last candidate sits at union position sp*64 + n - tp*64 - 1 (or s - 1: sink only)
        want = max(1, min(max(sp * 64 + int(n) - tp * 64 if t < n else s, s), total * 64))
        assert int(spans[r]) == want
    g = np.random.default_rng(rows)
    hist = g.standard_normal((rows, 64 * 64 + 8)).astype(np.float32)
    uni = g.standard_normal((rows, total * 64 + 4)).astype(np.float32)
    out = torch.full((rows, f["width"]), 3.0, device=DEV)
    TU.normalize_split(T(hist)[:, :4096], T(uni)[:, :total * 64], T(lens), d_end, T(f["takes"]), T(f["selected"]),
                       T(f["members"]), d_desc, out, f["max_take"], f["width"], S, W)
    e = O.union_normalize_split(hist[:, :4096], uni[:, :total * 64], lens, end, f["takes"], f["selected"],
                                f["members"], desc, f["width"], S, W)
    assert np.array_equal(H(out), e)


def test_split_scoring_chain_matches_per_row_tables():
    # every row scored once against all 64 history pages and once against the union (two shared-table
    # scorings) gives the canonical scores of the per-row-table chain, to the score tolerance
    h, rows, S, W, end = 65536, 512, 64, 2048, 65536
    b = Chain(h, rows, S, W, end, 40, True)
    b.run()
    cap = b.cap
    total = int(b.desc[3])
    ucap = b.fine.shape[0] - cap
    hist_tab = torch.arange(64, device=DEV, dtype=torch.int32)[None].expand(rows, -1)
    uni_tab = (cap + torch.arange(ucap, device=DEV, dtype=torch.int32))[None].expand(rows, -1)
    hist = torch.empty((rows, 4096), device=DEV)
    uni = torch.empty((rows, ucap * 64), device=DEV)
    spans = torch.empty(rows, device=DEV, dtype=torch.int32)
    full = torch.full((rows,), 4096, device=DEV, dtype=torch.int32)
    fine4 = b.fine.view(-1, 64, 1, 132)
    SC.fp8_paged_mqa_logits(b.q, fine4, b.w, full, hist_tab, None, 4096, clean_logits=False, out=hist)
    TU.union_spans(b.d_lens, b.d_end, b.desc, spans, S, W)
    SC.fp8_paged_mqa_logits(b.q, fine4, b.w, spans, uni_tab, None, ucap * 64, clean_logits=False, out=uni)
    out = torch.empty_like(b.scores)
    TU.normalize_split(hist, uni[:, :total * 64], b.d_lens, b.d_end, b.d_takes, b.d_sel, b.d_mem, b.desc, out,
                       b.max_take, b.width, S, W)
    got, ref = H(out), H(b.scores)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin)
    assert (np.abs(got[fin] - ref[fin]) <= 1e-2 * np.abs(ref[fin]) + 1e-3).all()
