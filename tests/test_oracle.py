"""Pins the CPU oracle against the reference's own known answers, closed forms
and brute force (CPU only)."""
import numpy as np
import pytest
import torch

from oracle import v1 as O
from conftest import pkg
import refexample as RX

W = pkg("workloads")


def test_fp8_decode_matches_torch_every_code():
    codes = np.arange(256, dtype=np.uint8)
    ours = O.e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
    assert np.array_equal(np.signbit(ours[ok]), np.signbit(ref[ok]))


def test_fp8_encode_matches_torch_cast():
    g = np.random.default_rng(0)
    x = np.concatenate([g.standard_normal(20000).astype(np.float32) * s for s in (1e-3, 0.1, 1, 30, 200)])
    x = np.clip(x, -448, 448)
    # exact ties between neighbouring codes (round-half-even) and subnormals
    vals = W.decode_table()[:127].astype(np.float64)
    mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids, np.float32([0.0, -0.0, 2 ** -10, 3 * 2 ** -10, 448.0])])
    ours = W.e4m3_encode(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)
    assert np.array_equal(W.e4m3_encode_fast(x), ours)


def test_pow2_scale_is_exact_ceiling():
    for m in [1e-6, 1e-4, 0.5, 448.0, 448.0001, 896.0, 3.7, 1000.0]:
        s = float(W.pow2_scale(np.float32(m)))
        v = float(np.float32(max(np.float32(m), np.float32(1e-4))) / np.float32(448))
        assert s >= v and s / 2 < v and s == 2.0 ** round(np.log2(s))


# ------------------------------------------------------------------ topk
def _brute(row, L, T):
    if L <= T:
        return list(range(L)) + [-1] * (T - L)
    key = [(0.0 if v == 0 else v) for v in row[:L]]  # -0.0 == +0.0
    order = sorted(range(L), key=lambda i: (-key[i], i))[:T]
    return sorted(order)


@pytest.mark.parametrize("seed", range(6))
def test_topk_select_brute_force_with_ties(seed):
    g = np.random.default_rng(seed)
    L = int(g.integers(1, 300))
    T = int(g.integers(1, 64))
    row = g.choice(np.float32([0.0, -0.0, 1.0, -1.0, 2.5, -np.inf, np.inf, 7.0]), size=L)
    row = np.where(g.random(L) < 0.3, g.standard_normal(L).astype(np.float32), row).astype(np.float32)
    assert list(O.topk_select(row, L, T)) == _brute(row, L, T)


@pytest.mark.parametrize("seed", range(4))
def test_topk_select_rows_equals_per_row(seed):
    """The batch selection (every row at once) against the per-row one and the
    brute force: ties, +-0, +-inf, NaN-free rows of every length class."""
    g = np.random.default_rng(100 + seed)
    B, cols, T = 40, 700, int(g.integers(1, 300))
    vals = np.float32([0.0, -0.0, 1.0, -1.0, 2.5, -np.inf, np.inf, 7.0])
    scores = g.choice(vals, size=(B, cols))
    scores = np.where(g.random((B, cols)) < 0.5, g.standard_normal((B, cols)), scores).astype(np.float32)
    lens = g.integers(0, cols + 50, size=B)
    lens[:3] = [0, T, T + 1]
    got = O.topk_select_rows(scores, lens, T, chunk=7)
    for b in range(B):
        L = min(int(lens[b]), cols)
        assert got[b].tolist() == O.topk_select(scores[b], L, T).tolist() == _brute(scores[b], L, T)
    table = g.integers(0, 1000, size=(B, cols // 4 + 1)).astype(np.int32)
    a = O.transform_topk_rows(scores, lens, table, T, 2)
    e = O.transform_topk(scores, lens, table, T, 2)
    assert np.array_equal(a[0], e[0]) and np.array_equal(a[1], e[1])


def test_topk_select_short_row_takes_all_even_neg_inf():
    row = np.float32([-np.inf, 3, -np.inf])
    assert list(O.topk_select(row, 3, 5)) == [0, 1, 2, -1, -1]


def test_score_key_orders_like_floats():
    v = np.float32([-np.inf, -3.5, -1e-30, -0.0, 0.0, 1e-30, 2.0, np.inf])
    k = O.score_key(v)
    assert k[3] == k[4]
    assert all(int(k[i]) < int(k[i + 1]) for i in (0, 1, 2, 4, 5, 6))


# ------------------------------------------------------------------ sort
def test_sort_kat(kats):
    kat = kats["sort_stable_signed_zero"]
    vals = np.float32([float(v) for v in kat["values"]])
    assert np.signbit(vals[4])
    out = O.sort_f32(np.int32(kat["ids"]), vals, 16, 1)
    assert out.tolist() == kat["expected"]


def test_sort_split_chain_kat(kats):
    kat = kats["sort_split_chain"]
    # dots / anchors of test_fused_grouping_small.py:101-115 on unit[:,0] = [1,-1]*8
    u = np.float32(kat["unit0"])
    perm = np.int32(kat["perm"])
    s0 = u[perm - 100] * u[perm[0] - 100]
    a0 = int(perm[int(np.argmin(s0))])
    s1 = u[perm - 100] * u[a0 - 100]
    a1 = int(perm[int(np.argmin(s1))])
    s2 = u[perm - 100] * u[a1 - 100] - s1
    assert [a0, a1] == kat["anchor"]
    assert O.sort_f32(perm, s2.astype(np.float32), 16, 1).tolist() == kat["expected"]


@pytest.mark.parametrize("n", [16, 64, 1024])
def test_sort_special_values_vs_sorted(kats, n):
    kat = kats["sort_special_pattern"]
    vals = np.float32([float(v) for v in kat["pattern"]] * kat["repeat"])
    perm = np.random.default_rng(n).permutation(4096).astype(np.int32)
    out = O.sort_f32(perm, vals, n, 4096 // n)
    for g in range(4096 // n):
        seg = vals[g * n:(g + 1) * n]
        exp = [perm[g * n + i] for i in sorted(range(n), key=lambda i: (-(0.0 if seg[i] == 0 else seg[i]), i))]
        assert out[g * n:(g + 1) * n].tolist() == exp


def test_sort_i64_matches_sorted():
    g = np.random.default_rng(3)
    keys = g.integers(-5, 5, size=256).astype(np.int64)
    keys[:3] = [np.iinfo(np.int64).min, np.iinfo(np.int64).max, 0]
    perm = np.arange(256, dtype=np.int32) + 1000
    out = O.sort_i64(perm, keys, 64)
    for s in range(4):
        k = keys[s * 64:(s + 1) * 64].tolist()
        exp = [1000 + s * 64 + i for i in sorted(range(64), key=lambda i: (-k[i], i))]
        assert out[s * 64:(s + 1) * 64].tolist() == exp


# ---------------------------------------------------------- page manager
def test_fingerprint_hand_kat(kats):
    kat = kats["fingerprint_hand"]
    tmp = np.zeros((1, 8448), np.uint8)
    tmp[0, :2] = kat["bytes_head"]
    m = np.zeros((1, 64), np.int32)
    m[0, :2] = kat["members_head"]
    assert O.fingerprint(tmp, m)[0].tolist() == kat["hash"]


def test_fingerprint_word_identity(kats):
    kat = kats["fingerprint_words"]
    b = kat["word_bytes"]
    i = 0
    assert sum(b) * (4 * i + 1) + b[1] + 2 * b[2] + 3 * b[3] == kat["weighted"]
    tmp = np.zeros((1, 8448), np.uint8)
    tmp[0, :4] = b
    assert O.fingerprint(tmp, np.zeros((1, 64), np.int32))[0, 0] == kat["weighted"]


def lifecycle_state(cap=16):
    tmp = np.repeat(np.arange(16, dtype=np.uint8)[:, None], 8448, axis=1)
    mapping = np.arange(1024, dtype=np.int32).reshape(16, 64)
    centers = np.zeros((2, 8448), np.uint8)
    centers[:, :8192] = 7
    centers[:, 8192:] = np.full((2, 64), 1.25, np.float32).view(np.uint8)
    return dict(tmp=tmp, mapping=mapping, centers=centers, fine=np.zeros_like(tmp),
                members=np.full_like(mapping, -1), live_hash=np.zeros((16, 2), np.int64),
                refs=np.zeros(cap, np.int32), free=np.arange(cap, dtype=np.int32), count=cap,
                tables=np.full(32, -1, np.int32), center_pool=np.zeros((4, 8448), np.uint8))


def test_page_lifecycle_kat(kats):
    kat = kats["page_lifecycle"]
    s = lifecycle_state(kat["capacity"])
    h = O.fingerprint(s["tmp"], s["mapping"])
    look = lambda: O.match_pages(s["tmp"], s["mapping"], h, s["fine"], s["members"], s["live_hash"], s["refs"], 16)
    assert (look() == -1).all()
    count, fresh = O.allocate(0, look(), s["free"], s["count"], s["refs"], s["tables"])
    O.publish(0, s["tmp"], s["centers"], s["mapping"], h, s["tables"], fresh, s["fine"], s["center_pool"],
              s["members"], s["live_hash"])
    s["count"] = count
    t0 = s["tables"][:16].copy()
    assert t0.tolist() == kat["first_table"] and count == kat["count_after_first"] and fresh.all()
    assert (s["fine"][t0] == s["tmp"]).all() and (s["members"][t0] == s["mapping"]).all()
    assert (s["center_pool"][:2] == s["centers"]).all() and (s["refs"] == kat["refs_after_first"]).all()
    s["tmp"][0, 0] = 99
    h2 = O.fingerprint(s["tmp"], s["mapping"])
    assert O.match_pages(s["tmp"], s["mapping"], h2, s["fine"], s["members"], s["live_hash"], s["refs"], 16)[0] == -1
    s["tmp"][0, 0] = 0
    s["mapping"][0, 0] = 9999
    h3 = O.fingerprint(s["tmp"], s["mapping"])
    assert O.match_pages(s["tmp"], s["mapping"], h3, s["fine"], s["members"], s["live_hash"], s["refs"], 16)[0] == -1
    s["mapping"][0, 0] = 0
    m = look()
    assert m.tolist() == t0.tolist()
    count, fresh = O.allocate(1, m, s["free"], s["count"], s["refs"], s["tables"])
    O.publish(1, s["tmp"], s["centers"], s["mapping"], h, s["tables"], fresh, s["fine"], s["center_pool"],
              s["members"], s["live_hash"])
    assert s["tables"][16:].tolist() == t0.tolist() and not fresh.any() and count == 0
    assert (s["refs"] == kat["refs_after_second"]).all() and (s["center_pool"][2:] == s["centers"]).all()
    count = O.release(t0, s["refs"], s["free"], count)
    assert count == 0 and (s["refs"] == kat["refs_after_release_a"]).all()
    count = O.release(s["tables"][16:], s["refs"], s["free"], count)
    assert count == kat["count_after_release_b"] and (s["refs"] == 0).all()
    assert sorted(s["free"].tolist()) == list(range(16))


@pytest.mark.parametrize("mode", ["miss", "hit", "collision"])
def test_match_modes(mode):
    g = np.random.default_rng(77)
    cap = 32
    tmp = g.integers(0, 256, (16, 8448), dtype=np.uint8)
    mp = g.integers(-1, 262144, (16, 64)).astype(np.int32)
    h = O.fingerprint(tmp, mp)
    fine = g.integers(0, 256, (cap, 8448), dtype=np.uint8)
    members = np.zeros((cap, 64), np.int32)
    hashes = np.zeros((cap, 2), np.int64)
    refs = np.zeros(cap, np.int32)
    if mode != "miss":
        fine[1:17], members[1:17], hashes[1:17], refs[1:17] = tmp, mp, h, 1
    if mode == "collision":
        fine[0], members[0], hashes[0], refs[0] = tmp[0], mp[0], h[0], 1
        fine[0, 0] ^= 1
    m = O.match_pages(tmp, mp, h, fine, members, hashes, refs, cap)
    exp = [-1] * 16 if mode == "miss" else list(range(1, 17))
    assert m.tolist() == exp


def test_release_duplicates_in_table_order():
    refs = np.int32([2, 1, 1, 0])
    free = np.full(8, -9, np.int32)
    count = O.release(np.int32([0, 1, 0, 2]), refs, free, 3)
    assert count == 6 and free[3:6].tolist() == [1, 0, 2] and refs.tolist() == [0, 0, 0, 0]


def shared_tail_inputs(kat):
    rows, np_, cap, scratch = kat["rows"], kat["np"], kat["cap"], kat["scratch"]
    native = np.zeros((np_, 8448), np.uint8)
    for page in range(np_):
        native[page, :8192] = W.e4m3_encode(np.float32([page + 1]))[0]
        native[page, 8192:] = (np.arange(64, dtype=np.float32) + 1).view(np.uint8)
    nt = np.repeat(np.arange(np_ - 1, -1, -1, dtype=np.int32)[None], rows, axis=0)
    return native, nt


def test_shared_tail_kat(kats):
    kat = kats["shared_tail"]
    native, nt = shared_tail_inputs(kat)
    rows, cap, scratch = kat["rows"], kat["cap"], kat["scratch"]
    lens, owners = np.int32(kat["lens"]), np.int32(kat["owners"])
    out = np.full((cap + rows * scratch, 8448), 255, np.uint8)
    O.stage_tail(native, nt, lens, out, cap, scratch, 64, 64, tail_rows=owners)
    for row, n in ((0, 1100), (2, 1101)):
        ids = list(range(64)) + list(range(1024, n))
        exp = np.zeros((scratch, 8448), np.uint8)
        for j, lg in enumerate(ids):
            page = nt[row, lg // 64]
            exp[j // 64, (j % 64) * 128:(j % 64) * 128 + 128] = native[page, (lg % 64) * 128:(lg % 64) * 128 + 128]
            exp[j // 64, 8192 + 4 * (j % 64):8192 + 4 * (j % 64) + 4] = native[page, 8192 + 4 * (lg % 64):8192 + 4 * (lg % 64) + 4]
        assert (out[cap + row * scratch:cap + (row + 1) * scratch] == exp).all()
    for row in (1, 3):
        assert (out[cap + row * scratch:cap + (row + 1) * scratch] == 255).all()
    assert (out[0] == 255).all()
    ft = O.fine_table(np.zeros((rows, kat["np"]), np.int32), np.zeros((rows, 1), np.int32), np.zeros(rows, np.int32),
                      scratch, cap, scratch, tail_rows=owners)
    assert ft.tolist() == kat["fine_table"]


def test_query_metadata_tail_sharing():
    nt = np.tile(np.arange(64, dtype=np.int32), (4, 1))
    nt[3, 20] = 999  # row 3 differs in a tail page
    lens = np.int32([1100, 1100, 1200, 1100])
    fl, tk, dg, cl, tr = O.query_metadata(lens, nt, 2048, 1, 2, 64, 64)
    assert tr.tolist() == [0, 0, 2, 0]  # row 3's differing page 20 is not a tail page of n=1100
    nt[3, 16] = 999  # page 16 = tail // 64 (tail = min(1024, 1100 - 64) = 1024) is
    assert O.query_metadata(lens, nt, 2048, 1, 2, 64, 64)[4].tolist() == [0, 0, 2, 3]
    pages, take, sink, tail, fine = O.geometry(1100, 2048, 1, 2, 64, 64)
    assert (pages, take, sink, tail) == (16, 16, 64, 1024) and fine == 16 * 64 + 64 + 1100 - 1024
    assert fl[0] == fine and tk[0] == take and cl[0] == 128


# ------------------------------------------------------------------ gather
def test_gather_kat(kats):
    kat = kats["gather_small"]
    x = np.arange(8 * 2 * 128, dtype=np.float32).reshape(8, 2, 128)
    k, v = x, -x - 16
    req = np.int32(kat["req"])
    ids = np.int32(kat["ids"])
    for head in (0, 1):
        kg, vg = O.gather_slots(k, v, req, ids, head)
        for r in range(2):
            for i in range(3):
                p = kat["physical"][r][i]
                assert (kg[r, i, 0] == (k[p, head] if p >= 0 else 0)).all()
                assert (vg[r, i, 0] == (v[p, head] if p >= 0 else 0)).all()


def test_gather_rows_paged_table():
    pool = np.arange(40 * 16, dtype=np.int64).astype(np.uint8).reshape(40, 16)
    table = np.int32([[3, 1], [0, 2]])
    ids = np.int32([[0, 5, -1], [7, 4, 2]])
    out = O.gather_rows(pool, ids, table, page_bits=2)
    phys = [[12, 5, -1], [11, 8, 2]]
    for r in range(2):
        for i in range(3):
            p = phys[r][i]
            assert (out[r, i] == (pool[p] if p >= 0 else 0)).all()


# ------------------------------------------------------------------- route
def test_route_reference_example(kats):
    kat = kats["route_example"]
    d = RX.route_inputs()
    B = RX.B
    sel = np.full((B, RX.TAKE), -1, np.int32)
    ft = np.full((B, RX.TAKE + 68), -1, np.int32)
    O.route(d["scores"].numpy(), d["lens"].numpy(), d["takes"].numpy(), sel, RX.P, d["rt"].numpy(), ft,
            d["tail_rows"].numpy(), RX.CAP, True)
    ref_pages = d["scores"][:, :512].view(B, 64, 8).amax(-1).topk(RX.TAKE, dim=-1).indices.numpy()
    assert (sel == ref_pages).all()
    assert sel[0, :8].tolist() == kat["first_selected"]
    assert (ft[:, :RX.TAKE] == np.take_along_axis(d["rt"].numpy(), ref_pages, 1)).all()
    assert (ft[:, RX.TAKE:] == RX.CAP + np.arange(68)).all()


def test_route_ties_to_lower_page_and_trivial_branch():
    B, P = 3, 64
    scores = np.full((B, 8 * P), -np.inf, np.float32)
    scores[:, :8 * 32] = 1.0  # all 32 active pages tie
    scores[1, 8 * 5 + 3] = 2.0
    lens = np.int32([2049, 2049, 1025])  # active 32, 32, 16
    takes = np.int32([4, 4, 20])
    sel = np.zeros((B, 6), np.int32)
    rt = np.arange(B * P, dtype=np.int32).reshape(B, P)
    ft = np.zeros((B, 10), np.int32)
    O.route(scores, lens, takes, sel, P, rt, ft, np.int32([0, 1, 2]), 500, True)
    assert sel[0].tolist() == [0, 1, 2, 3, 4, 5]
    assert sel[1].tolist() == [5, 0, 1, 2, 3, 4]
    assert sel[2].tolist() == [0, 1, 2, 3, 4, 5]  # take >= active: identity
    assert ft[1, :4].tolist() == [rt[1, 5], rt[1, 0], rt[1, 1], rt[1, 2]]
    assert ft[1, 4:].tolist() == [500 + 68 + j for j in range(6)]
    # the identity branch writes ft[i] only for i < take_stride (v1_query.cuh:17-19)
    assert ft[2, :6].tolist() == rt[2, :6].tolist() and ft[2, 6:].tolist() == [0, 0, 0, 0]


def test_route_fine_table_takes_every_rank_below_take():
    """Sorted branch with take > take_stride: selected keeps take_stride ranks,
    the fine table every rank < take (v1_query.cuh:44-48), then the tail slots."""
    P, K, W_ = 64, 6, 12
    g = np.random.default_rng(3)
    scores = np.full((1, 8 * P), -np.inf, np.float32)
    scores[0, :8 * 32] = g.permutation(8 * 32).astype(np.float32)  # distinct page maxima
    rt = (1000 + np.arange(P, dtype=np.int32))[None]
    sel = np.zeros((1, K), np.int32)
    ft = np.zeros((1, W_), np.int32)
    O.route(scores, np.int32([2049]), np.int32([9]), sel, P, rt, ft, np.int32([2]), 500, True)
    order = np.argsort(-scores[0, :256].reshape(32, 8).max(1), kind="stable")
    assert sel[0].tolist() == order[:K].tolist()
    assert ft[0, :9].tolist() == (1000 + order[:9]).tolist()
    assert ft[0, 9:].tolist() == [500 + 2 * 68 + j for j in range(3)]


# -------------------------------------------------------------- fused topk
@pytest.fixture(scope="module")
def example_after_route():
    d = RX.route_inputs()
    B = RX.B
    sel = np.full((B, RX.TAKE), -1, np.int32)
    ft = np.full((B, RX.TAKE + 68), -1, np.int32)
    O.route(d["scores"].numpy(), d["lens"].numpy(), d["takes"].numpy(), sel, RX.P, d["rt"].numpy(), ft,
            d["tail_rows"].numpy(), RX.CAP, True)
    f = RX.fine_inputs(d, torch.from_numpy(ft))
    return d, sel, ft, f


@pytest.mark.parametrize("direct", [False, True])
def test_fused_topk_reference_example(example_after_route, direct):
    d, sel, ft, f = example_after_route
    work = f["fine_scores"].numpy().copy()
    out = O.fused_topk(work, f["fine_lens"].numpy(), d["members"].numpy(), d["rt"].numpy(), d["nt"].numpy(), sel,
                       d["lens"].numpy(), d["takes"].numpy(), RX.TOP, RX.WINDOW, True, 0, True, True, ft, direct)
    ref = f["reference_scores"]
    exp_raw = ref.topk(RX.TOP, dim=-1).indices
    cand = f["candidate_ids"].numpy()
    raw = out["raw"]
    assert (np.sort(raw, 1) == exp_raw.sort(1).values.numpy()).all()
    assert (out["logical"] == np.take_along_axis(cand, raw.astype(np.int64), 1)).all()
    nt = d["nt"].numpy()
    lg = out["logical"]
    assert (out["physical"] == np.take_along_axis(nt, lg // 64, 1) * 64 + lg % 64).all()
    s = np.sort(lg, 1)
    assert (s[:, 1:] != s[:, :-1]).all()
    assert np.array_equal(work, ref.numpy())


def test_unfused_mask_and_map_equal_fused(example_after_route):
    d, sel, ft, f = example_after_route
    rows = 64
    args = lambda a: a[:rows]
    w1 = f["fine_scores"].numpy()[:rows].copy()
    w2 = w1.copy()
    fl = f["fine_lens"].numpy()[:rows]
    out = O.fused_topk(w1, fl, d["members"].numpy(), args(d["rt"].numpy()), args(d["nt"].numpy()), args(sel),
                       args(d["lens"].numpy()), args(d["takes"].numpy()), RX.TOP, RX.WINDOW, True, 0, True, False,
                       args(ft), False)
    O.mask_fine(w2, args(sel), args(d["rt"].numpy()), d["members"].numpy(), args(d["lens"].numpy()),
                args(d["takes"].numpy()), w2.shape[1], 64, RX.WINDOW)
    assert np.array_equal(w1, w2)
    raw = np.stack([O.topk_select(w2[b], int(fl[b]), RX.TOP) for b in range(rows)]).astype(np.int32)
    phys, lg = O.output_ids(raw, w2, d["members"].numpy(), args(d["rt"].numpy()), args(d["nt"].numpy()), args(sel),
                            args(d["lens"].numpy()), args(d["takes"].numpy()), w2.shape[1], RX.TOP, 64, RX.WINDOW,
                            True, False, args(ft))
    assert np.array_equal(phys, out["physical"]) and np.array_equal(lg, out["logical"])


@pytest.mark.parametrize("bucket_from_rank,direct", [(True, False), (False, True), (False, False)])
def test_fused_topk_rows_equals_per_row(example_after_route, bucket_from_rank, direct):
    """The batch mask + selection + map against fused_topk, on the reference
    example rows (masked sink/tail buckets, short and long rows)."""
    d, sel, ft, f = example_after_route
    rows = 96
    args = lambda a: a[:rows]
    w1 = f["fine_scores"].numpy()[:rows].copy()
    w1[5, 100:400] = w1[5, 99]  # a long run of ties across the selection boundary
    w2 = w1.copy()
    fl = f["fine_lens"].numpy()[:rows].copy()
    fl[7] = 1000  # a row of fewer candidates than T
    common = (d["members"].numpy(), args(d["rt"].numpy()), args(d["nt"].numpy()), args(sel),
              args(d["lens"].numpy()), args(d["takes"].numpy()), RX.TOP, RX.WINDOW, True, 4 * RX.TOP + 64, True,
              bucket_from_rank, args(ft), direct)
    a = O.fused_topk(w1, fl, *common)
    b = O.fused_topk_rows(w2, fl, *common)
    assert np.array_equal(w1, w2)
    for k in ("physical", "logical", "raw", "expanded"):
        assert np.array_equal(a[k], b[k]), k


def test_transform_closed_form():
    g = np.random.default_rng(5)
    scores = g.standard_normal((3, 300)).astype(np.float32)
    lens = np.int32([300, 10, 200])
    table = g.permutation(64).astype(np.int32)[None].repeat(3, 0)
    out, raw = O.transform_topk(scores, lens, table, 16, 6)
    for b in range(3):
        r = raw[b]
        ok = r >= 0
        assert (out[b][ok] == table[b, r[ok] >> 6] * 64 + (r[ok] & 63)).all() and (out[b][~ok] == -1).all()
    assert raw[1].tolist() == list(range(10)) + [-1] * 6


# ------------------------------------------------------------------- score
def test_score_formula_order_by_hand():
    # one query, 2 heads, one key: q0.k = 2, q1.k = -3 -> w0*relu(2) + w1*relu(-3) = 0.5*2; times s_k = 0.25
    q8 = np.zeros((1, 2, 128), np.uint8)
    q8[0, 0, 0] = W.e4m3_encode(np.float32([1.0]))[0]
    q8[0, 1, 0] = W.e4m3_encode(np.float32([-1.5]))[0]
    native = np.zeros((1, 8448), np.uint8)
    native[0, 0] = W.e4m3_encode(np.float32([2.0]))[0]
    native[0, 8192:8196] = np.float32([0.25]).view(np.uint8)
    w = np.float32([[0.5, 7.0]])
    out = O.paged_logits(q8, w, native, np.int32([[0]]), np.int32([1]), 4)
    assert out[0, 0] == pytest.approx(0.5 * 2 * 0.25)
    assert np.isneginf(out[0, 1:]).all()
    signed = O.paged_logits(q8, w, native, np.int32([[0]]), np.int32([1]), 1, relu=False)
    assert signed[0, 0] == pytest.approx((0.5 * 2 - 7.0 * 3) * 0.25)


def _onehot_pool():
    """4 native pages whose token (page p, slot s) key is the unit vector at
    dim (37 p + s) % 128 (FP8 1.0 = 0x38) with scale (1 + s/64) * 2^-p: every
    token has its own dim pattern and scale, so reading a wrong token (page and
    slot swapped, a wrong scale slot) changes the logit."""
    native = np.zeros((4, 8448), np.uint8)
    for p in range(4):
        for s in range(64):
            native[p, s * 128 + (37 * p + s) % 128] = 0x38
            native[p, 8192 + 4 * s:8196 + 4 * s] = np.float32([(1 + s / 64) * 2.0 ** -p]).view(np.uint8)
    return native


def _onehot_queries():
    """2 rows x 3 heads: q[r, h, d] = ((d + 5 h + 3 r) mod 9) - 4, exact in e4m3."""
    q = np.array([[[((d + 5 * h + 3 * r) % 9) - 4 for d in range(128)] for h in range(3)] for r in range(2)],
                 np.float32)
    return W.e4m3_encode(q.reshape(-1)).reshape(2, 3, 128)


def test_paged_logits_addressing_by_hand():
    """sglang/srt/layers/attention/v1_deepseek/kernels.py:310-313 through
    per-row permuted block tables: logit[r, j] = sum_h w[r,h] relu(q[r,h,d]) s
    with (d, s) the dim and scale of token (table[r, j // 64], j % 64)."""
    native = _onehot_pool()
    q8 = _onehot_queries()
    w = np.float32([[0.5, 1.5, 0.25], [2.0, -1.0, 0.75]])
    table = np.int32([[2, 0, 3], [1, 3, 0]])
    lens = np.int32([150, 130])
    out = O.paged_logits(q8, w, native, table, lens, 192)
    # worked by hand:
    #  [0, 0]:   page 2 slot 0 -> d 74,  q0 = (-2, 3, -1) -> 1.5*3 = 4.5, s = 0.25   -> 1.125
    #  [0, 70]:  page 0 slot 6 -> d 6,   q0 = (2, -2, 3) -> 0.5*2 + 0.25*3 = 1.75, s = 1.09375 -> 1.9140625
    #  [0, 149]: page 3 slot 21 -> d 4,  q0 = (0, -4, 1) -> 0.25, s = 1.328125/8   -> 0.0415039...
    #  [1, 129]: page 0 slot 1 -> d 1,   q1 = (0, -4, 1) -> 0.75, s = 1.015625     -> 0.76171875
    #  [1, 64]:  page 3 slot 0 -> d 111, q1 = (2, -2, 3) -> 2*2 + 0.75*3 = 6.25, s = 0.125 -> 0.78125
    #  [1, 5]:   page 1 slot 5 -> d 42,  q1 = (-4, 1, -3) -> -1*1 = -1, s = 1.078125/2 -> -0.5390625
    assert out[0, 0] == 1.125 and out[0, 70] == 1.9140625 and out[1, 129] == 0.76171875
    assert out[0, 149] == pytest.approx(0.25 * 1.328125 / 8, rel=1e-12)
    assert out[1, 64] == 0.78125 and out[1, 5] == -0.5390625
    assert np.isneginf(out[0, 150:]).all() and np.isneginf(out[1, 130:]).all()
    # every column by lookup (no matmul): the dot with a one-hot key is one element of q
    qf = O.e4m3_decode(q8).astype(np.float64)
    for r in range(2):
        for j in range(int(lens[r])):
            p, s = int(table[r, j // 64]), j % 64
            d, sc = (37 * p + s) % 128, (1 + s / 64) * 2.0 ** -p
            assert out[r, j] == pytest.approx(sum(w[r, h] * max(qf[r, h, d], 0) for h in range(3)) * sc, rel=1e-12)
    # signed rule, and one shared table (1-D) for both rows
    signed = O.paged_logits(q8, w, native, table, lens, 192, relu=False)
    assert signed[0, 0] == (0.5 * -2 + 1.5 * 3 + 0.25 * -1) * 0.25
    shared = O.paged_logits(q8, w, native, table[0], lens, 192)
    assert shared[1, 0] == pytest.approx((2.0 * max(qf[1, 0, 74], 0) - 1.0 * max(qf[1, 1, 74], 0)
                                          + 0.75 * max(qf[1, 2, 74], 0)) * 0.25)


# ------------------------------------------------- batched page manager
def _per_request_chain(pool, pool_keys, refs, free, count, keys, tmp, req):
    """The pinned per-lease oracle functions (match_pages, allocate, publish)
    called request after request, with the key as h0 and h1 = 0, members 0."""
    pool, pool_keys, refs, free = pool.copy(), pool_keys.copy(), refs.copy(), free.copy()
    cap = len(refs)
    members = np.zeros((cap, 64), np.int32)
    table = np.empty(len(keys), np.int32)
    for r in np.unique(req):
        sel = np.flatnonzero(req == r)
        t, mp = tmp[sel], np.zeros((len(sel), 64), np.int32)
        h = np.stack([keys[sel], np.zeros(len(sel), np.int64)], 1)
        hashes = np.stack([pool_keys, np.zeros(cap, np.int64)], 1)
        m = O.match_pages(t, mp, h, pool, members, hashes, refs, cap)
        tables = np.full(len(sel), -1, np.int32)
        count, fresh = O.allocate(0, m, free, count, refs, tables)
        centers_tmp = np.zeros((-(-len(sel) * 8 // 64), 8448), np.uint8)
        O.publish(0, t, centers_tmp, mp, h, tables, fresh, pool, np.zeros_like(centers_tmp), members, hashes)
        pool_keys = hashes[:, 0].copy()
        table[sel] = tables
    return table, pool, pool_keys, refs, free, count


def _small_pool_case(seed, cap=160, requests=24, max_pages=9, page_bytes=32, collide=4):
    wl = W.config2(seed=seed, requests=requests, max_pages=max_pages, capacity=cap, collide=collide)
    a = wl.arrays
    payload = W.config2_payload(wl, page_bytes)
    return wl, a["keys"], payload[a["draw"]], a["req"]


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_page_insert_batch_equals_per_request_chain(seed):
    wl, keys, tmp, req = _small_pool_case(seed)
    cap = 160
    g = np.random.default_rng(seed)
    # pre-live pages: some hold batch keys (same or other bytes), some are unrelated
    pool = g.integers(0, 256, (cap, tmp.shape[1]), dtype=np.uint8)
    pool_keys = g.integers(-2**62, 2**62, cap)
    refs = np.zeros(cap, np.int32)
    pick = g.choice(len(keys), 12, replace=False)
    live = g.choice(cap, 24, replace=False)
    pool[live[:12]] = tmp[pick]
    pool_keys[live[:12]] = keys[pick]
    pool_keys[live[12:18]] = keys[pick[:6]]          # equal key, other bytes: collision with a live page
    refs[live] = g.integers(1, 4, 24)
    free_pages = np.setdiff1d(np.arange(cap), live)
    free = np.concatenate([g.permutation(free_pages), np.full(len(live), -7)]).astype(np.int32)
    count = len(free_pages)
    got = O.page_insert_batch(pool, pool_keys, refs, free, count, keys, tmp, req)
    exp = _per_request_chain(pool, pool_keys, refs, free, count, keys, tmp, req)
    for x, y in zip(got, exp):
        assert np.array_equal(x, y)
    table, pool2, _, refs2, free2, count2 = got
    # invariants: every entry holds one reference; table pages hold the entry's bytes
    assert (refs2 - refs).sum() == len(keys) and np.array_equal(np.bincount(table, minlength=cap), refs2 - refs)
    assert np.array_equal(pool2[table], tmp)
    assert sorted(free2[:count2].tolist() + np.flatnonzero(refs2 > 0).tolist()) == list(range(cap))


def test_page_insert_batch_lifecycle_kat(kats):
    """The reference lifecycle (test_page_management_and_tail_small.py:14-57)
    as two one-request batches and two releases."""
    kat = kats["page_lifecycle"]
    cap = kat["capacity"]
    tmp = np.repeat(np.arange(16, dtype=np.uint8)[:, None], 8448, axis=1)
    keys = np.arange(16, dtype=np.int64) * 1000003
    req = np.zeros(16, np.int32)
    state = (np.zeros_like(tmp), np.zeros(cap, np.int64), np.zeros(cap, np.int32), np.arange(cap, dtype=np.int32),
             cap)
    t0, pool, pk, refs, free, count = O.page_insert_batch(*state, keys, tmp, req)
    assert t0.tolist() == kat["first_table"] and count == kat["count_after_first"]
    assert (refs == kat["refs_after_first"]).all()
    t1, pool, pk, refs, free, count = O.page_insert_batch(pool, pk, refs, free, count, keys, tmp, req)
    assert t1.tolist() == t0.tolist() and (refs == kat["refs_after_second"]).all() and count == 0
    refs, free, count = O.page_release_batch(t0, refs, free, count)
    assert count == 0 and (refs == kat["refs_after_release_a"]).all()
    refs, free, count = O.page_release_batch(t1, refs, free, count)
    assert count == kat["count_after_release_b"] and sorted(free.tolist()) == list(range(16))


def test_page_insert_batch_same_request_duplicates_take_fresh_pages():
    """Entries of one request never match each other (match_pages only sees
    live pages, kernels.py:72-113); a later request takes the lowest of them."""
    tmp = np.zeros((5, 16), np.uint8)
    keys = np.full(5, 42, np.int64)
    req = np.int32([0, 0, 0, 1, 1])
    t, pool, pk, refs, free, count = O.page_insert_batch(
        np.zeros((8, 16), np.uint8), np.zeros(8, np.int64), np.zeros(8, np.int32), np.arange(8, dtype=np.int32), 8,
        keys, tmp, req)
    assert t.tolist() == [7, 6, 5, 5, 5] and count == 5 and refs.tolist() == [0] * 5 + [3, 1, 1]


def test_page_insert_batch_exhaustion_is_all_or_nothing():
    tmp = np.arange(6, dtype=np.uint8)[:, None].repeat(16, 1)
    with pytest.raises(RuntimeError, match="exhausted"):
        O.page_insert_batch(np.zeros((4, 16), np.uint8), np.zeros(4, np.int64), np.zeros(4, np.int32),
                            np.arange(4, dtype=np.int32), 4, np.arange(6, dtype=np.int64), tmp,
                            np.int32([0, 0, 0, 1, 1, 1]))


def test_page_release_batch_underflow_and_order():
    refs = np.int32([2, 1, 1, 0])
    free = np.full(8, -9, np.int32)
    refs2, free2, count = O.page_release_batch(np.int32([0, 1, 0, 2]), refs, free, 3)
    assert count == 6 and free2[3:6].tolist() == [1, 0, 2] and refs2.tolist() == [0, 0, 0, 0]
    assert refs.tolist() == [2, 1, 1, 0]  # inputs untouched
    with pytest.raises(RuntimeError, match="underflow"):
        O.page_release_batch(np.int32([0, 0, 0]), refs, free, 3)
    with pytest.raises(RuntimeError, match="out of range"):
        O.page_release_batch(np.int32([4]), refs, free, 3)


def test_config2_shape():
    wl = W.config2()
    p = wl.params
    assert p["requests"] == 4096 and 125000 < p["entries"] < 140000 and p["distinct"] < p["capacity"]
    assert p["page_bytes"] == 41984 and wl.arrays["keys"].dtype == np.int64
    assert np.all(np.diff(wl.arrays["req"]) >= 0)


def _as_rows(pages8448):
    """Native pages re-laid as 64 rows of 132 bytes (128 key bytes + fp32 scale)."""
    k = pages8448[:, :8192].reshape(-1, 64, 128)
    s = pages8448[:, 8192:].reshape(-1, 64, 4)
    return np.concatenate([k, s], axis=2).reshape(len(pages8448), 64 * 132)


def test_stage_tail_rows_equals_native_layout(kats):
    """Row-layout staging equals the pinned native-layout staging after the
    re-layout, on the reference shared-tail KAT and on random lengths."""
    kat = kats["shared_tail"]
    native, nt = shared_tail_inputs(kat)
    rows, cap, scratch = kat["rows"], kat["cap"], kat["scratch"]
    for lens, owners in ((np.int32(kat["lens"]), np.int32(kat["owners"])),
                         (np.int32([1, 64, 65, 700]), None), (np.int32([1100, 128, 1088, 2000]), np.int32([0, 1, 1, 3]))):
        lens = np.minimum(lens, nt.shape[1] * 64)
        a = np.full((cap + rows * scratch, 8448), 255, np.uint8)
        O.stage_tail(native, nt, lens, a, cap, scratch, 64, 64, tail_rows=owners)
        b = np.full((cap + rows * scratch, 64 * 132), 255, np.uint8)
        O.stage_tail_rows(_as_rows(native), nt, lens, b, cap, scratch, 64, 64, 132, tail_rows=owners)
        touched = ~(a == 255).all(axis=1)
        assert np.array_equal(touched, ~(b == 255).all(axis=1))
        assert np.array_equal(_as_rows(a[touched]), b[touched])


def test_expand_logical_kat_and_fused_equality(example_after_route):
    # hand-computed: index 3 -> 12..15, -1 -> four -1s, 0 -> 0..3, padding -1
    out = np.full((1, 16), 7, np.int32)
    O.expand_logical(np.array([[3, -1, 0]], np.int32), out)
    assert out.tolist() == [[12, 13, 14, 15, -1, -1, -1, -1, 0, 1, 2, 3, -1, -1, -1, -1]]
    # BLOCK below STRIDE: columns past BLOCK keep their contents
    out = np.full((1, 16), 7, np.int32)
    O.expand_logical(np.array([[3, -1, 0]], np.int32), out, block=8)
    assert out.tolist() == [[12, 13, 14, 15, -1, -1, -1, -1] + [7] * 8]
    # int32 wraps like the reference's tl arithmetic
    out = np.zeros((1, 4), np.int32)
    O.expand_logical(np.array([[2 ** 29 + 1]], np.int32), out)
    assert out.tolist() == [[-2 ** 31 + 4, -2 ** 31 + 5, -2 ** 31 + 6, -2 ** 31 + 7]]
    # the unfused expansion of the fused Top-K's logical ids equals its fused expansion
    # (v1_query.cuh:143-151 vs kernels.py:594-600), on the reference example
    d, sel, ft, f = example_after_route
    rows = 32
    args = lambda a: a[:rows]
    work = f["fine_scores"].numpy()[:rows].copy()
    res = O.fused_topk(work, f["fine_lens"].numpy()[:rows], d["members"].numpy(), args(d["rt"].numpy()),
                       args(d["nt"].numpy()), args(sel), args(d["lens"].numpy()), args(d["takes"].numpy()), RX.TOP,
                       RX.WINDOW, True, 4 * RX.TOP + 64, True, True, args(ft), False)
    assert (res["logical"] >= 0).any() and (res["expanded"][:, 4 * RX.TOP:] == -1).all()
    out = np.full(res["expanded"].shape, 7, np.int32)
    O.expand_logical(res["logical"], out)
    assert np.array_equal(out, res["expanded"])


# ------------------------------------------- scoring without DeepGEMM
def test_reduce_centers_by_hand():
    """kernels.py:475-486: page p of a row = max of center logits 8p..8p+7 for
    p < max(n-1, 0) // 1024 * 16 (capped at maxp), -inf elsewhere."""
    logits = np.full((3, 160), -5.0, np.float32)
    logits[0, :128] = np.arange(128, dtype=np.float32)  # page p: max 8p + 7
    logits[1, :128] = -np.arange(128, dtype=np.float32)  # page p: max -8p
    logits[1, 9] = -np.inf
    got = O.reduce_centers(logits, np.array([2049, 1025, 1024]), 20)
    # row 0: 32 pages capped at maxp 20; logits past column 127 are -5
    exp0 = np.array([8 * p + 7 if p < 16 else -5 for p in range(20)], np.float32)
    assert np.array_equal(got[0], exp0)
    # row 1: 16 pages; page 1's center 9 is -inf, the max is still -8
    exp1 = np.array([-8.0 * p if p < 16 else -np.inf for p in range(20)], np.float32)
    assert np.array_equal(got[1], exp1)
    # row 2: n = 1024 gives no built page
    assert np.all(np.isneginf(got[2]))


def test_coarse_by_brute_force():
    """kernels.py:182-221 by explicit loops: center page table[r, b] holds the
    centers of pages 8b..8b+7, page p = max over its 8 centers g of
    sum_h w_h relu(q_h . c) s_c, -inf from pages(n) on."""
    g = np.random.default_rng(77)
    c8, cs = W.quantize_rows(g.standard_normal((3 * 64, 128)).astype(np.float32))
    centers = W.pack_pages(c8, cs)  # 3 center pages
    q8, _ = W.quantize_rows(g.standard_normal((2 * 3, 128)).astype(np.float32))
    q8 = q8.reshape(2, 3, 128)
    w = g.random((2, 3)).astype(np.float32)
    table = np.array([[2, 0], [1, 2]], np.int32)  # maxp = 16: two center pages per row
    lens = np.array([1025, 4000])  # 16 pages for both (capped at maxp)
    got = O.coarse(q8, w, centers, table, lens, 16)
    qf = O.e4m3_decode(q8).astype(np.float64)
    for r in range(2):
        for p in range(16):
            page = table[r, p // 8]
            best = -np.inf
            for c in range(8):
                slot = (p % 8) * 8 + c
                k = O.e4m3_decode(c8[page * 64 + slot]).astype(np.float64)
                v = sum(float(w[r, h]) * max(float(qf[r, h] @ k), 0.0) for h in range(3)) * float(cs[page * 64 + slot])
                best = max(best, v)
            assert np.isclose(got[r, p], best, rtol=1e-6, atol=0), (r, p)
    # a request of one bucket (n = 1025) has 16 pages; n = 1024 has none
    assert np.all(np.isneginf(O.coarse(q8, w, centers, table, np.array([1024, 1]), 16)))


def test_fine_equals_staged_table_scoring_with_mask():
    """kernels.py:248-320 against the optimised path built from pinned pieces:
    fine_table + stage_tail (scratch pages per row) + paged_logits over the
    fine table + mask_fine (kernels.py:379-441, 444-472) give the same scores,
    including rows whose take is 0, rows shorter than the built pages and
    candidates past count."""
    wl = W.config1(rows=6)
    a, prm = wl.arrays, wl.params
    B, CAP, TAKE, WIDTH, SINK, WINDOW = prm["B"], prm["CAP"], prm["TAKE"], prm["WIDTH"], prm["SINK"], prm["WINDOW"]
    g = np.random.default_rng(8)
    lens = np.array([4097, 4097, 3073, 2100, 1500, 4097], np.int32)
    takes = np.array([40, 0, 17, 24, 3, 40], np.int32)
    selected = np.stack([g.permutation(64)[:TAKE] for _ in range(B)]).astype(np.int32)
    scratch = 68
    fine = np.zeros((CAP + B * scratch, a["fine"].shape[1]), np.uint8)
    fine[:CAP] = a["fine"][:CAP]
    ft = O.fine_table(a["rt"], selected, takes, TAKE + scratch, CAP, scratch)
    O.stage_tail(a["native"], a["nt"], lens, fine, CAP, scratch, SINK, WINDOW)
    count = np.array([t * 64 + O._bounds(int(n), WINDOW, SINK)[0] + int(n) - O._bounds(int(n), WINDOW, SINK)[1]
                      for n, t in zip(lens, takes)])
    staged = O.paged_logits(a["q8"], a["w"], fine, ft, np.minimum(count, WIDTH), WIDTH)
    O.mask_fine(staged, selected, a["rt"], a["members"], lens, takes, WIDTH, SINK, WINDOW)
    got = O.fine(a["q8"], a["w"], fine, a["native"], a["members"], a["rt"], a["nt"], selected, lens, takes, WIDTH,
                 SINK, WINDOW)
    assert np.array_equal(np.isneginf(got), np.isneginf(staged))
    fin = np.isfinite(staged)
    assert fin.sum() > 5000
    assert np.allclose(got[fin], staged[fin], rtol=1e-12, atol=0)
