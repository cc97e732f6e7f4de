"""GPU parity of every kernel against the CPU oracle (bit-exact for integer,
byte and index outputs; FP8 scores within 1e-2 relative of the fp64
dequantised formula).  All calls go through the C ABI of libv1idx.so."""
import numpy as np
import pytest
import torch

from conftest import pkg
from oracle import v1 as O
import refexample as RX

pytestmark = pytest.mark.gpu

QF = pkg("query_fused")
K = pkg("kernels")
FG = pkg("fused_grouping")
NK = pkg("native_kernels")
SC = pkg("scoring")
TK = pkg("topk")
W = pkg("workloads")


def T(x, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    return t if dtype is None else t.to(dtype)


def H(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


# ------------------------------------------------------------------ gather
def test_gather_small_kat(dev, kats):
    kat = kats["gather_small"]
    x = torch.arange(8 * 2 * 128, device=dev, dtype=torch.float32).reshape(8, 2, 128)
    k, v = x.to(torch.bfloat16), (-x - 16).to(torch.bfloat16)
    req = torch.tensor(kat["req"], device=dev, dtype=torch.int32)
    backing = torch.tensor([[0, 2, -1, 99], [4, 1, 4, 99]], device=dev, dtype=torch.int32)
    ids = backing[:, :3]
    kp = torch.empty((8, 2, 256), device=dev, dtype=torch.bfloat16)[:, :, ::2]
    kp.copy_(k)
    vp = torch.empty((8, 4, 128), device=dev, dtype=torch.bfloat16)[:, ::2, :]
    vp.copy_(v)
    before_k, before_v = kp.clone(), vp.clone()
    out_k = torch.empty((2, 3, 1, 128), device=dev, dtype=torch.bfloat16)
    out_v = torch.empty_like(out_k)
    for head in (0, 1):
        NK._gather_slots[(1,)](kp, vp, req, ids, out_k, out_v, 2, 3, head, *kp.stride(), *vp.stride(),
                               ids.stride(0), 32, num_warps=4)
        ek, ev = O.gather_slots(H(kp.float()), H(vp.float()), np.int32(kat["req"]), H(ids), head)
        assert np.array_equal(H(out_k.float()), ek) and np.array_equal(H(out_v.float()), ev)
    assert torch.equal(kp, before_k) and torch.equal(vp, before_v)


def test_gather_workspace_reuse(dev):
    x = torch.arange(8 * 2 * 128, device=dev, dtype=torch.float32).reshape(8, 2, 128)
    k, v = x.to(torch.bfloat16), (-x - 16).to(torch.bfloat16)
    req = torch.tensor([5, 1, 7, 0, 6, 2], device=dev, dtype=torch.int32)
    ids = (torch.arange(4096, device=dev) % 6).to(torch.int32).reshape(2, 2048)
    work = NK.GatherWorkspace(2, dev, torch.bfloat16)
    a, b = work.gather(k, v, req, ids, 0)
    ek, ev = O.gather_slots(H(k.float()), H(v.float()), H(req), H(ids), 0)
    assert np.array_equal(H(a.float()), ek) and np.array_equal(H(b.float()), ev)
    addresses = (a.data_ptr(), b.data_ptr())
    changed = ids.flip(1).contiguous()
    a, b = work.gather(k, v, req, changed, 1)
    assert addresses == (a.data_ptr(), b.data_ptr())
    ek, ev = O.gather_slots(H(k.float()), H(v.float()), H(req), H(changed), 1)
    assert np.array_equal(H(a.float()), ek) and np.array_equal(H(b.float()), ev)
    work.clear()
    assert work.k is None and work.v is None


@pytest.mark.parametrize("row_bytes,paged", [(656, True), (656, False), (256, True), (16, False)])
def test_gather_rows_vs_oracle(dev, row_bytes, paged):
    g = np.random.default_rng(row_bytes + paged)
    rows, top, pool_rows = 37, 300, 4096
    pool = g.integers(0, 256, (pool_rows, row_bytes), dtype=np.uint8)
    if paged:
        table = np.stack([g.permutation(pool_rows // 64)[:16] for _ in range(rows)]).astype(np.int32)
        ids = g.integers(0, 16 * 64, (rows, top)).astype(np.int32)
    else:
        table = None
        ids = g.integers(0, pool_rows, (rows, top)).astype(np.int32)
    ids[g.random((rows, top)) < 0.05] = -1
    out = torch.full((rows, top, row_bytes), 7, device=dev, dtype=torch.uint8)
    NK.gather_rows(T(pool, dev), T(ids, dev), out, None if table is None else T(table, dev), 6 if paged else 0)
    assert np.array_equal(H(out), O.gather_rows(pool, ids, table, 6 if paged else 0))


@pytest.mark.parametrize("row_bytes", [16, 656, 65520])
@pytest.mark.parametrize("big", [False, True])
def test_gather_rows_tiles_and_passes(dev, row_bytes, big):
    """Both copy shapes: pools up to 64 MB (1024 threads x 11 loads per pass)
    and larger ones (512 threads x 6), with tiles of 1024 one-chunk rows, 256
    or 64 rows of 41 chunks, and 4095-chunk rows that take one slot per tile
    and two passes (larger pool) or two slots in one pass; slot counts that
    end in a partial tile, padding ids and per-row page tables."""
    g = np.random.default_rng(row_bytes * 2 + big)
    pool_bytes = (72 << 20) if big else (3 << 20)
    pool_rows = max(64, (pool_bytes // row_bytes) // 64 * 64)
    rows, top = (3, 37) if row_bytes > 4096 else (5, 1111)
    pool = g.integers(0, 256, (pool_rows, row_bytes), dtype=np.uint8)
    pages = pool_rows // 64
    table = np.stack([g.permutation(pages)[:min(pages, 16)] for _ in range(rows)]).astype(np.int32)
    ids = g.integers(0, table.shape[1] * 64, (rows, top)).astype(np.int32)
    ids[g.random((rows, top)) < 0.05] = -1
    out = torch.full((rows, top, row_bytes), 7, device=dev, dtype=torch.uint8)
    NK.gather_rows(T(pool, dev), T(ids, dev), out, T(table, dev), 6)
    assert np.array_equal(H(out), O.gather_rows(pool, ids, table, 6))


def test_gather_slots_empty_pool(dev):
    """A pool with no slots: every slot is padding and comes out as zeros."""
    kp = torch.empty((0, 2, 128), device=dev, dtype=torch.bfloat16)
    req = torch.tensor([0, 1], device=dev, dtype=torch.int32)
    ids = torch.tensor([[0, 1, -1]], device=dev, dtype=torch.int32)
    out_k = torch.full((1, 3, 1, 128), 5.0, device=dev, dtype=torch.bfloat16)
    out_v = torch.full_like(out_k, 5.0)
    NK._gather_slots[(1,)](kp, kp, req, ids, out_k, out_v, 1, 3, 0, *kp.stride(), *kp.stride(), ids.stride(0), 32,
                           num_warps=4)
    assert not H(out_k.float()).any() and not H(out_v.float()).any()


def test_gather_rows_shared_map_and_bad_ids(dev):
    pool = np.arange(64 * 32, dtype=np.int64).astype(np.uint8).reshape(64, 32)
    req = np.int32([5, 1, 70, 0])  # entry 2 points past the pool
    ids = np.int32([[0, 1, 2, 3, 4, -1]])  # id 4 is past the map
    out = torch.full((1, 6, 32), 9, device=dev, dtype=torch.uint8)
    NK.gather_rows(T(pool, dev), T(ids, dev), out, T(req, dev), 0)
    got = H(out)[0]
    assert (got[0] == pool[5]).all() and (got[1] == pool[1]).all() and (got[3] == pool[0]).all()
    assert (got[2] == 0).all() and (got[4] == 0).all() and (got[5] == 0).all()


# -------------------------------------------------------------------- sort
def test_sort_kat_and_flag(dev, kats):
    kat = kats["sort_stable_signed_zero"]
    vals = torch.tensor([float(v) for v in kat["values"]], device=dev)
    perm = torch.tensor(kat["ids"], device=dev, dtype=torch.int32)
    out = torch.full((16,), -99, device=dev, dtype=torch.int32)
    flag = torch.tensor(-1, device=dev, dtype=torch.int32)
    FG._sort[(1, 1)](perm, out, vals, flag, 16, num_warps=4)
    assert H(out).tolist() == kat["expected"]
    assert H(perm).tolist() == kat["ids"]
    flag.fill_(0)
    out.fill_(-99)
    FG._sort[(1, 1)](perm, out, vals, flag, 16, num_warps=4)
    assert (H(out) == -99).all()


@pytest.mark.parametrize("n", [4096, 1024, 512, 256, 128, 64, 32, 16])
def test_sort_random_and_special(dev, kats, n):
    g = np.random.default_rng(n)
    heads = 2
    perm = np.concatenate([g.permutation(4096) for _ in range(heads)]).astype(np.int32)
    for special in (False, True):
        if special:
            pat = [float(v) for v in kats["sort_special_pattern"]["pattern"]]
            vals = np.float32(pat * (heads * 4096 // len(pat)))
        else:
            vals = np.round(g.standard_normal(heads * 4096) * 4).astype(np.float32)  # many ties
        out = torch.empty(heads * 4096, device=dev, dtype=torch.int32)
        flag = torch.tensor(-1, device=dev, dtype=torch.int32)
        FG._sort[(4096 // n, heads)](T(perm, dev), out, T(vals, dev), flag, n)
        exp = O.sort_f32(perm, vals, n, 4096 // n, heads=heads)
        assert np.array_equal(H(out), exp)


def test_sort_i64(dev):
    g = np.random.default_rng(1)
    keys = g.integers(-20, 20, 8 * 512).astype(np.int64)
    keys[:2] = [np.iinfo(np.int64).min, np.iinfo(np.int64).max]
    perm = (np.arange(keys.size) + 7).astype(np.int32)
    out = torch.empty(keys.size, device=dev, dtype=torch.int32)
    FG.sort_groups_i64(T(perm, dev), out, T(keys, dev), 512)
    assert np.array_equal(H(out), O.sort_i64(perm, keys, 512))


# ------------------------------------------------------------------- route
def test_route_reference_example(dev, kats):
    d = RX.route_inputs()
    B = RX.B
    sel = torch.full((B, RX.TAKE), -1, device=dev, dtype=torch.int32)
    ft = torch.full((B, RX.TAKE + 68), -1, device=dev, dtype=torch.int32)
    QF.module().route(d["scores"].to(dev), d["lens"].to(dev), d["takes"].to(dev), sel, RX.P, d["rt"].to(dev), ft,
                      d["tail_rows"].to(dev), RX.CAP, True)
    ref_pages = d["scores"][:, :512].view(B, 64, 8).amax(-1).topk(RX.TAKE, dim=-1).indices
    assert torch.equal(sel.cpu().long(), ref_pages)
    assert H(sel)[0, :8].tolist() == kats["route_example"]["first_selected"]
    assert torch.equal(ft.cpu()[:, :RX.TAKE], d["rt"].gather(1, ref_pages))
    assert torch.equal(ft.cpu()[:, RX.TAKE:], (RX.CAP + torch.arange(68, dtype=torch.int32))[None].expand(B, -1))


@pytest.mark.parametrize("pages,bits", [(64, 32), (128, 64), (256, 64), (512, 32), (1024, 32), (2048, 64), (4096, 32)])
def test_route_random_vs_oracle(dev, pages, bits):
    g = np.random.default_rng(pages)
    B = 24
    scores = np.round(g.standard_normal((B, pages * 8)) * 3).astype(np.float32)  # ties
    scores[g.random(scores.shape) < 0.02] = -np.inf
    lens = g.integers(1, pages * 64 + 2, B).astype(np.int32)
    K_ = min(pages, 48)
    # takes past the selected width too: the fine table then takes every rank < take (v1_query.cuh:44-48)
    takes = g.integers(0, K_ + 41, B).astype(np.int32)
    rt = g.integers(0, 10000, (B, pages)).astype(np.int32)
    tail = g.integers(0, 5, B).astype(np.int32)
    sel0 = np.full((B, K_), -7, np.int64 if bits == 64 else np.int32)
    ft0 = np.full((B, K_ + 68), -7, np.int32)
    sel, ft = sel0.copy(), ft0.copy()
    O.route(scores, lens, takes, sel, pages, rt, ft, tail, 1000, True)
    s_d = T(sel0, dev)
    f_d = T(ft0, dev)
    QF.module().route(T(scores, dev), T(lens, dev), T(takes, dev), s_d, pages, T(rt, dev), f_d, T(tail, dev), 1000,
                      True)
    assert np.array_equal(H(s_d), sel) and np.array_equal(H(f_d), ft)


@pytest.mark.parametrize("pages", [256, 2048])
def test_route_sorts_only_active_prefix(dev, pages):
    """The route kernel sorts only the first power of two of slots that holds
    a row's active pages; a selected array as wide as the table checks the
    ranks past that prefix (pages at or past `active`, in ascending order)."""
    g = np.random.default_rng(pages + 5)
    actives = [16, 48, 80, 128, 144, pages // 2 + 16, pages]
    B = len(actives)
    scores = np.round(g.standard_normal((B, pages * 8)) * 3).astype(np.float32)
    scores[g.random(scores.shape) < 0.02] = -np.inf
    lens = (np.int32(actives) // 16 * 1024 + 1 + g.integers(0, 1024, B)).astype(np.int32)
    takes = (np.int32(actives) // 2).astype(np.int32)
    rt = g.integers(0, 10000, (B, pages)).astype(np.int32)
    tail = np.arange(B, dtype=np.int32)
    sel, ft = np.full((B, pages), -7, np.int32), np.full((B, pages + 68), -7, np.int32)
    s_d, f_d = T(sel, dev), T(ft, dev)
    O.route(scores, lens, takes, sel, pages, rt, ft, tail, 1000, True)
    QF.module().route(T(scores, dev), T(lens, dev), T(takes, dev), s_d, pages, T(rt, dev), f_d, T(tail, dev), 1000,
                      True)
    assert np.array_equal(H(s_d), sel) and np.array_equal(H(f_d), ft)


def test_route_rejects_like_reference(dev):
    m = QF.module()
    B = 4
    z = lambda *s: torch.zeros(s, device=dev, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="Invalid V1 route capacity"):
        m.route(torch.zeros((B, 8 * 32), device=dev), z(B), z(B), z(B, 8), 32, z(B, 32), z(B, 8), z(B), 10, True)
    with pytest.raises(RuntimeError, match="Invalid fine page table"):
        m.route(torch.zeros((B, 8 * 64), device=dev), z(B), z(B), z(B, 8), 64, z(B, 64), z(B, 4), z(B), 10, True)


# ------------------------------------------------------------------- topk
@pytest.fixture(scope="module")
def example_after_route():
    d = RX.route_inputs()
    B = RX.B
    sel = np.full((B, RX.TAKE), -1, np.int32)
    ft = np.full((B, RX.TAKE + 68), -1, np.int32)
    O.route(d["scores"].numpy(), d["lens"].numpy(), d["takes"].numpy(), sel, RX.P, d["rt"].numpy(), ft,
            d["tail_rows"].numpy(), RX.CAP, True)
    return d, sel, ft, RX.fine_inputs(d, torch.from_numpy(ft))


@pytest.mark.parametrize("direct", [False, True])
def test_fused_topk_reference_example(dev, example_after_route, direct):
    """The reference example's own assertions (example_v1_query_single_head.py:61-73)
    plus exact equality with the oracle (ascending order, lower-index ties)."""
    d, sel, ft, f = example_after_route
    B, TOP = RX.B, RX.TOP
    work = f["fine_scores"].to(dev).clone()
    physical = torch.empty((B, TOP), device=dev, dtype=torch.int32)
    logical = torch.empty_like(physical)
    raw = torch.empty_like(physical)
    no_expansion = torch.empty_strided((B, 0), (0, 1), device=dev, dtype=torch.int32)
    QF.module().topk(work, f["fine_lens"].to(dev), d["members"].to(dev), d["rt"].to(dev), d["nt"].to(dev),
                     T(sel, dev), d["lens"].to(dev), d["takes"].to(dev), physical, logical, raw, RX.WINDOW, True,
                     no_expansion, True, True, T(ft, dev), direct)
    torch.cuda.synchronize()
    expected_raw = f["reference_scores"].topk(TOP, dim=-1).indices
    assert torch.equal(raw.cpu().sort(1).values.long(), expected_raw.sort(1).values)
    assert torch.equal(logical.cpu(), f["candidate_ids"].gather(1, raw.cpu().long()))
    nt = d["nt"]
    lg = logical.cpu()
    assert torch.equal(physical.cpu(), nt.gather(1, (lg // 64).long()) * 64 + lg % 64)
    s = lg.sort(1).values
    assert bool((s[:, 1:] != s[:, :-1]).all())
    assert torch.equal(work.cpu(), f["reference_scores"])
    exp = O.fused_topk(f["fine_scores"].numpy().copy(), f["fine_lens"].numpy(), d["members"].numpy(),
                       d["rt"].numpy(), d["nt"].numpy(), sel, d["lens"].numpy(), d["takes"].numpy(), TOP, RX.WINDOW,
                       True, 0, True, True, ft, direct)
    assert np.array_equal(H(raw), exp["raw"]) and np.array_equal(H(logical), exp["logical"])
    assert np.array_equal(H(physical), exp["physical"])


def _v1_case(g, B, cols, take_max, ties):
    pages = 64
    members_pages = 80
    members = np.full((members_pages, 64), -1, np.int32)
    for p in range(members_pages):
        base = g.integers(0, 8) * 1024
        members[p] = base + g.permutation(1024)[:64]
    lens = g.integers(1, pages * 64 + 1, B).astype(np.int32)  # n <= 64 * pages (nt row length)
    takes = g.integers(0, take_max + 1, B).astype(np.int32)
    K_ = take_max
    sel = g.integers(0, pages, (B, K_)).astype(np.int32)
    rt = g.integers(0, members_pages, (B, pages)).astype(np.int32)
    nt = g.integers(0, 5000, (B, pages * 2)).astype(np.int32)[:, :pages]
    if ties:
        scores = np.round(g.standard_normal((B, cols)) * 2).astype(np.float32)
        scores[g.random(scores.shape) < 0.1] = -0.0
    else:
        scores = g.standard_normal((B, cols)).astype(np.float32)
    scores[g.random(scores.shape) < 0.05] = -np.inf
    fine_lens = g.integers(0, cols + 1, B).astype(np.int32)
    fine_lens[: B // 4] = cols
    ft = g.integers(0, members_pages, (B, K_ + 3)).astype(np.int32)
    return dict(scores=scores, fine_lens=fine_lens, members=members, rt=rt, nt=nt, sel=sel, lens=lens, takes=takes,
                ft=ft)


@pytest.mark.parametrize("cols,topk,ties", [(700, 256, True), (2688, 2048, True), (6000, 2048, False),
                                             (20000, 2048, True), (32768, 2048, False), (70000, 2048, True),
                                             (40000, 512, False), (200000, 2048, True)])
def test_fused_topk_random_vs_oracle(dev, cols, topk, ties):
    """Register-resident rows (<= 8192 columns), streamed rows (one pass up to
    40960 columns in a batch of 513 rows), and segmented rows whose merge
    holds the candidates in registers (<= 4 segments at T = 2048) or streams
    them (5 segments at 200000 columns)."""
    g = np.random.default_rng(cols + topk)
    B = 513
    c = _v1_case(g, B, cols, 40, ties)
    rows = np.arange(B) % 9 == 0  # oracle on a row subset (all rows run on the GPU)
    for direct, bucket_rank, expand in ((False, True, False), (True, False, True)):
        work = T(c["scores"], dev)
        phys = torch.empty((B, topk), device=dev, dtype=torch.int32)
        lg = torch.empty_like(phys)
        raw = torch.empty_like(phys)
        es = 4 * topk + 64 if expand else 0
        exp_t = torch.full((B, es), 5, device=dev, dtype=torch.int32) if expand else \
            torch.empty_strided((B, 0), (0, 1), device=dev, dtype=torch.int32)
        QF.module().topk(work, T(c["fine_lens"], dev), T(c["members"], dev), T(c["rt"], dev), T(c["nt"], dev),
                         T(c["sel"], dev), T(c["lens"], dev), T(c["takes"], dev), phys, lg, raw, 64, True, exp_t, True,
                         bucket_rank, T(c["ft"], dev), direct)
        sub = lambda a: a[rows]
        s_or = c["scores"][rows].copy()
        exp = O.fused_topk(s_or, sub(c["fine_lens"]), c["members"], sub(c["rt"]), sub(c["nt"]), sub(c["sel"]),
                           sub(c["lens"]), sub(c["takes"]), topk, 64, True, es, True, bucket_rank, sub(c["ft"]),
                           direct)
        assert np.array_equal(H(raw)[rows], exp["raw"])
        assert np.array_equal(H(lg)[rows], exp["logical"])
        assert np.array_equal(H(phys)[rows], exp["physical"])
        assert np.array_equal(H(work)[rows], s_or)
        if expand:
            assert np.array_equal(H(exp_t)[rows], exp["expanded"])


def test_fused_topk_rejects_like_reference(dev):
    m = QF.module()
    B = 16
    z = lambda *s: torch.zeros(s, device=dev, dtype=torch.int32)
    e = torch.empty_strided((B, 0), (0, 1), device=dev, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="Unsupported fused V1 TopK"):
        m.topk(torch.zeros((B, 100), device=dev), z(B), z(4, 64), z(B, 8), z(B, 8), z(B, 4), z(B), z(B), z(B, 16),
               z(B, 16), z(B, 16), 64, True, e, True, True, z(B, 4), False)


@pytest.mark.parametrize("B,cols,topk", [(16, 5000, 2048), (128, 131072, 2048), (3, 100000, 64), (600, 3000, 700),
                                         (6, 70000, 2047), (4, 200000, 2048)])
def test_topk_transform_vs_oracle(dev, B, cols, topk):
    """Single-pass rows (register-resident up to 8192 columns) and segmented
    rows; the merge holds the segments' candidates in registers while they
    fit 8192 (up to 4 segments at T = 2048) and streams them past that
    (7 segments at 200000 columns)."""
    g = np.random.default_rng(B * cols)
    scores = np.round(g.standard_normal((B, cols)) * 50).astype(np.float32)
    lens = g.integers(1, cols + 1, B).astype(np.int32)
    lens[0] = cols
    lens[1] = min(cols, topk)
    table = g.integers(0, 1 << 20, (B, (cols + 63) // 64)).astype(np.int32)
    out = torch.empty((B, topk), device=dev, dtype=torch.int32)
    raw = torch.empty_like(out)
    TK.topk_transform_512_v2(T(scores, dev), T(lens, dev), T(table, dev), out, 64, None, raw)
    rows = np.arange(B) if B <= 16 else np.arange(B)[np.arange(B) % 8 == 0]
    e_out, e_raw = O.transform_topk(scores[rows], lens[rows], table[rows], topk, 6)
    assert np.array_equal(H(raw)[rows], e_raw) and np.array_equal(H(out)[rows], e_out)


@pytest.mark.parametrize("cols,offset", [(3000, 0), (2999, 1)])
def test_mask_fine_and_output_ids_vs_oracle(dev, cols, offset):
    """mask_fine takes 4 columns per thread (one 16-byte member load when the
    member table is 16-byte aligned); a width that is not a multiple of 4 and a
    member table at a 4-byte offset take the partial and scalar paths."""
    g = np.random.default_rng(11)
    B, topk = 40, 512
    c = _v1_case(g, B, cols, 40, True)
    w_d = T(c["scores"], dev)
    mem = T(c["members"], dev)
    if offset:
        buf = torch.empty(mem.numel() + offset, device=dev, dtype=torch.int32)
        buf[offset:] = mem.reshape(-1)
        mem = buf[offset:].view(mem.shape)
    K.mask_fine[(B, -(-cols // 256))](w_d, T(c["sel"], dev), T(c["rt"], dev), mem, T(c["lens"], dev),
                                      T(c["takes"], dev), 64, 40, cols, cols, 64, 64)
    w_o = c["scores"].copy()
    O.mask_fine(w_o, c["sel"], c["rt"], c["members"], c["lens"], c["takes"], cols, 64, 64)
    assert np.array_equal(H(w_d), w_o)
    raw = np.stack([O.topk_select(w_o[b], int(c["fine_lens"][b]), topk) for b in range(B)]).astype(np.int32)
    for direct in (False, True):
        out = torch.empty((B, topk), device=dev, dtype=torch.int32)
        lg = torch.empty_like(out)
        K.output_ids[(B, 2)](T(raw, dev), w_d, T(c["members"], dev), T(c["rt"], dev), T(c["nt"], dev),
                             T(c["sel"], dev), T(c["lens"], dev), T(c["takes"], dev), out, lg, T(c["ft"], dev), 64, 64,
                             40, cols, topk, 64, 64, MAP_PHYSICAL=True, DIRECT_FINE=direct, FP=c["ft"].shape[1])
        e_out, e_lg = O.output_ids(raw, w_o, c["members"], c["rt"], c["nt"], c["sel"], c["lens"], c["takes"], cols,
                                   topk, 64, 64, True, direct, c["ft"])
        assert np.array_equal(H(out), e_out) and np.array_equal(H(lg), e_lg)


# ----------------------------------------------------------- page manager
def test_page_lifecycle_kat(dev, kats):
    kat = kats["page_lifecycle"]
    cap = kat["capacity"]
    t = lambda x, dtype=torch.int32: torch.tensor(x, device=dev, dtype=dtype)
    tmp = torch.arange(16, device=dev, dtype=torch.uint8)[:, None].expand(16, 8448).contiguous()
    mapping = torch.arange(1024, device=dev, dtype=torch.int32).reshape(16, 64)
    meta = t([0, 0, 1])
    hashes = torch.empty((16, 2), device=dev, dtype=torch.int64)
    centers = torch.zeros((2, 8448), device=dev, dtype=torch.uint8)
    centers[:, :8192] = 7
    centers.view(torch.float32)[:, 2048:] = 1.25
    fine = torch.zeros_like(tmp)
    members = torch.full_like(mapping, -1)
    live_hash = torch.zeros_like(hashes)
    refs = torch.zeros(cap, device=dev, dtype=torch.int32)
    free = torch.arange(cap, device=dev, dtype=torch.int32)
    count = t(cap)
    tables = torch.full((2, 16), -1, device=dev, dtype=torch.int32)
    new = torch.empty(16, device=dev, dtype=torch.bool)
    match = torch.empty(16, device=dev, dtype=torch.int32)
    center_pool = torch.zeros((4, 8448), device=dev, dtype=torch.uint8)

    def lookup():
        K.match_pages[(16,)](tmp, mapping, hashes, meta, fine, members, live_hash, refs, match, cap, 16)

    def alloc_publish():
        K.allocate[(1,)](meta, match, free, count, refs, tables, new, debug=True)
        K.publish[(16,)](tmp, centers, centers.view(torch.float32), mapping, hashes, meta, tables, new, fine,
                         center_pool, center_pool.view(torch.float32), members, live_hash)

    K.fingerprint[(16,)](tmp, mapping, meta, hashes)
    assert np.array_equal(H(hashes), O.fingerprint(H(tmp), H(mapping)))
    lookup()
    assert bool((match == -1).all())
    alloc_publish()
    assert H(tables[0]).tolist() == kat["first_table"]
    assert count.item() == 0 and bool(new.all())
    assert torch.equal(fine[tables[0].long()], tmp) and torch.equal(members[tables[0].long()], mapping)
    assert torch.equal(center_pool[:2], centers) and bool((refs == 1).all())
    tmp[0, 0] = 99
    lookup()
    assert match[0].item() == -1
    tmp[0, 0] = 0
    mapping[0, 0] = 9999
    lookup()
    assert match[0].item() == -1
    mapping[0, 0] = 0
    meta[1] = 1
    lookup()
    assert torch.equal(match, tables[0])
    alloc_publish()
    assert torch.equal(tables[1], tables[0]) and not bool(new.any())
    assert count.item() == 0 and bool((refs == 2).all()) and torch.equal(center_pool[2:], centers)
    K.release[(1,)](tables[0], refs, free, count)
    assert count.item() == 0 and bool((refs == 1).all()) and torch.equal(fine[tables[1].long()], tmp)
    K.release[(1,)](tables[1], refs, free, count)
    assert count.item() == 16 and bool((refs == 0).all())
    assert torch.equal(free.sort().values, torch.arange(16, device=dev, dtype=torch.int32))
    # inactive records leave every output untouched
    meta[2] = 0
    hashes.fill_(-99)
    match.fill_(-99)
    K.fingerprint[(16,)](tmp, mapping, meta, hashes)
    lookup()
    assert bool((hashes == -99).all()) and bool((match == -99).all())


@pytest.mark.parametrize("mode", ["miss", "hit", "collision"])
def test_match_modes_vs_oracle(dev, mode):
    g = np.random.default_rng(77)
    cap = 257
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
    h_d = torch.empty((16, 2), device=dev, dtype=torch.int64)
    meta = torch.tensor([4096, 1, 1], device=dev, dtype=torch.int32)
    K.fingerprint[(16,)](T(tmp, dev), T(mp, dev), meta, h_d)
    assert np.array_equal(H(h_d), h)
    m = torch.empty(16, device=dev, dtype=torch.int32)
    K.match_pages[(16,)](T(tmp, dev), T(mp, dev), h_d, meta, T(fine, dev), T(members, dev), T(hashes, dev),
                         T(refs, dev), m, cap, 512)
    exp = O.match_pages(tmp, mp, h, fine, members, hashes, refs, cap)
    assert np.array_equal(H(m), exp)
    assert H(m).tolist() == ([-1] * 16 if mode == "miss" else list(range(1, 17)))


def test_release_duplicates_in_table_order(dev):
    refs = torch.tensor([2, 1, 1, 0] + [1] * 12, device=dev, dtype=torch.int32)
    table = torch.tensor([0, 1, 0, 2] + [3] * 12, device=dev, dtype=torch.int32)
    free = torch.full((32,), -9, device=dev, dtype=torch.int32)
    count = torch.tensor(3, device=dev, dtype=torch.int32)
    K.release[(1,)](table, refs, free, count)
    r_o = np.int32([2, 1, 1, 0] + [1] * 12)
    f_o = np.full(32, -9, np.int32)
    c_o = O.release(np.int32([0, 1, 0, 2] + [3] * 12), r_o, f_o, 3)
    assert count.item() == c_o and np.array_equal(H(free), f_o) and np.array_equal(H(refs), r_o)


def test_allocate_exhaustion_sets_status(dev):
    meta = torch.tensor([0, 0, 1], device=dev, dtype=torch.int32)
    match = torch.full((16,), -1, device=dev, dtype=torch.int32)
    free = torch.arange(16, device=dev, dtype=torch.int32)
    count = torch.tensor(3, device=dev, dtype=torch.int32)
    refs = torch.zeros(16, device=dev, dtype=torch.int32)
    tables = torch.full((1, 16), -1, device=dev, dtype=torch.int32)
    new = torch.zeros(16, device=dev, dtype=torch.bool)
    st = K.allocation_status(dev)
    st.zero_()
    K.allocate[(1,)](meta, match, free, count, refs, tables, new)
    assert st.item() & 1 and count.item() == 3 and bool((refs == 0).all()) and bool((tables == -1).all())
    st.zero_()


# ------------------------------------------------- metadata, tables, tails
def test_shared_tail_kat(dev, kats):
    kat = kats["shared_tail"]
    rows, np_, cap, scratch = kat["rows"], kat["np"], kat["cap"], kat["scratch"]
    native = torch.zeros((np_, 8448), device=dev, dtype=torch.uint8)
    for page in range(np_):
        native[page, :8192].view(torch.float8_e4m3fn).fill_(page + 1)
        native.view(torch.float32)[page, 2048:] = torch.arange(64, device=dev) + 1
    nt = torch.arange(np_ - 1, -1, -1, device=dev, dtype=torch.int32)[None].expand(rows, -1).contiguous()
    lens = torch.tensor(kat["lens"], device=dev, dtype=torch.int32)
    owners = torch.tensor(kat["owners"], device=dev, dtype=torch.int32)
    out = torch.full((cap + rows * scratch, 8448), 255, device=dev, dtype=torch.uint8)
    K.stage_tail_shared[(1, scratch)](native.view(torch.float8_e4m3fn), native.view(torch.float32), nt, lens,
                                      out.view(torch.float8_e4m3fn), out.view(torch.float32), owners, cap, np_, scratch,
                                      64, 64, ROWS=rows, GROUP=4, num_warps=4)
    exp = np.full((cap + rows * scratch, 8448), 255, np.uint8)
    O.stage_tail(H(native), H(nt), H(lens), exp, cap, scratch, 64, 64, tail_rows=H(owners))
    assert np.array_equal(H(out), exp)
    rt = torch.zeros((rows, np_), device=dev, dtype=torch.int32)
    selected = torch.zeros((rows, 1), device=dev, dtype=torch.int32)
    takes = torch.zeros(rows, device=dev, dtype=torch.int32)
    ft = torch.empty((rows, scratch), device=dev, dtype=torch.int32)
    K.fine_table_shared[(rows,)](rt, selected, takes, lens, ft, owners, cap, np_, 1, scratch, scratch, 4)
    assert H(ft).tolist() == kat["fine_table"]


def test_stage_tail_and_tables_random_vs_oracle(dev):
    g = np.random.default_rng(8)
    rows, np_, cap, scratch, native_pages = 24, 40, 30, 68, 300
    native = g.integers(0, 256, (native_pages, 8448), dtype=np.uint8)
    nt = g.integers(0, native_pages, (rows, np_)).astype(np.int32)
    lens = g.integers(1, np_ * 64 + 1, rows).astype(np.int32)
    owners = np.where(np.arange(rows) % 3 == 1, np.arange(rows) - 1, np.arange(rows)).astype(np.int32)
    for shared in (True, False):
        out = np.full((cap + rows * scratch, 8448), 3, np.uint8)
        o_d = T(out, dev)
        if shared:
            K.stage_tail_shared[(-(-rows // 32), scratch)](T(native, dev), None, T(nt, dev), T(lens, dev), o_d, None,
                                                           T(owners, dev), cap, np_, scratch, 64, 200, ROWS=rows,
                                                           GROUP=32)
        else:
            K.stage_tail[(rows, scratch)](T(native, dev), None, T(nt, dev), T(lens, dev), o_d, None, cap, np_,
                                          scratch, 64, 200)
        O.stage_tail(native, nt, lens, out, cap, scratch, 64, 200, tail_rows=owners if shared else None)
        assert np.array_equal(H(o_d), out)
    sel = g.integers(0, np_, (rows, 20)).astype(np.int64)
    takes = g.integers(0, 21, rows).astype(np.int32)
    rt = g.integers(0, 999, (rows, np_)).astype(np.int32)
    for shared in (True, False):
        ft = torch.empty((rows, 30), device=dev, dtype=torch.int32)
        if shared:
            K.fine_table_shared[(rows,)](T(rt, dev), T(sel, dev), T(takes, dev), T(lens, dev), ft, T(owners, dev), cap,
                                         np_, 20, 30, scratch, 32)
        else:
            K.fine_table[(rows,)](T(rt, dev), T(sel, dev), T(takes, dev), T(lens, dev), ft, cap, np_, 20, 30, scratch,
                                  32)
        exp = O.fine_table(rt, sel, takes, 30, cap, scratch, tail_rows=owners if shared else None)
        assert np.array_equal(H(ft), exp)


@pytest.mark.parametrize("rows", [9, 520])
def test_stage_tail_page_groups_and_pool_edges(dev, rows):
    """Both work-group shapes of the staging kernel (one page per work-group
    below 512 rows, four from 512 on): scratch widths that are not a multiple
    of four pages, candidate counts that end inside a group or past the
    scratch, table entries past the native pool (their slots read as zeros)
    and a fine pool that ends inside the last row's scratch (pages past it are
    not written)."""
    g = np.random.default_rng(21 + rows)
    np_, cap, native_pages, extra = 12, 7, 50, 6
    cases = ((6, 300), (5, 200), (9, 520), (1, 100)) if rows < 512 else ((6, 300), (9, 520))
    for scratch, window in cases:
        native = g.integers(0, 256, (native_pages, 8448), dtype=np.uint8)
        nt = g.integers(0, native_pages + extra, (rows, np_)).astype(np.int32)
        lens = g.integers(1, np_ * 64 + 1, rows).astype(np.int32)
        full = cap + rows * scratch
        fine_pages = full - 3
        out = T(np.full((fine_pages, 8448), 5, np.uint8), dev)
        K.stage_tail[(rows, scratch)](T(native, dev), None, T(nt, dev), T(lens, dev), out, None, cap, np_, scratch,
                                      64, window)
        # the oracle over a pool padded with zero pages: a table entry past the
        # kernel's pool then reads zeros, as the kernel's range check gives
        padded = np.concatenate([native, np.zeros((extra, 8448), np.uint8)])
        exp = np.full((full, 8448), 5, np.uint8)
        O.stage_tail(padded, nt, lens, exp, cap, scratch, 64, window)
        assert np.array_equal(H(out), exp[:fine_pages]), (scratch, window)


def test_query_metadata_vs_oracle(dev):
    g = np.random.default_rng(9)
    rows, NP = 50, 256
    lens = g.integers(0, NP * 64, rows).astype(np.int32)
    lens[1::3] = lens[0]
    nt = np.tile(g.integers(0, 9999, NP).astype(np.int32), (rows, 1))
    nt[5, 3:] += 1
    outs = [torch.empty(rows, device=dev, dtype=torch.int32) for _ in range(5)]
    K.query_metadata[(rows,)](T(lens, dev), T(nt, dev), *outs, NP, 2048, 1, 2, 64, 2048)
    exp = O.query_metadata(lens, nt, 2048, 1, 2, 64, 2048)
    for got, e in zip(outs, exp):
        assert np.array_equal(H(got), e)
    fl = torch.empty(rows, device=dev, dtype=torch.int32)
    tk = torch.empty_like(fl)
    K.query_lengths[(rows,)](T(lens, dev), fl, tk, 512, 2048, 1, 2, 64, 2048)
    assert np.array_equal(H(fl), exp[0]) and np.array_equal(H(tk), exp[1])


# ------------------------------------------------------------------- score
def _score_case(g, rows, heads, ctx_max, shared, pool_pages):
    q8, _ = W.quantize_rows(g.standard_normal((rows * heads, 128), dtype=np.float32))
    q8 = q8.reshape(rows, heads, 128)
    w = g.random((rows, heads), dtype=np.float32)
    k8, ks = W.quantize_rows(g.standard_normal((pool_pages * 64, 128), dtype=np.float32))
    native = W.pack_pages(k8, ks)
    blocks = -(-ctx_max // 64)
    if shared:
        table = g.permutation(pool_pages)[:blocks].astype(np.int32)
        lens = np.minimum(ctx_max, ctx_max - rows + 1 + np.arange(rows)).astype(np.int32)
    else:
        table = np.stack([g.permutation(pool_pages)[:blocks] for _ in range(rows)]).astype(np.int32)
        lens = g.integers(1, ctx_max + 1, rows).astype(np.int32)
    return q8, w, native, table, lens


@pytest.mark.parametrize("rows,heads,ctx,shared", [(37, 64, 3000, True), (24, 64, 5000, False), (19, 1, 2688, False),
                                                   (20, 32, 1100, True), (9, 16, 700, False), (33, 16, 2688, True),
                                                   (25, 1, 2688, True)])
def test_score_vs_dequantised_reference(dev, rows, heads, ctx, shared):
    g = np.random.default_rng(rows * heads + ctx)
    q8, w, native, table, lens = _score_case(g, rows, heads, ctx, shared, 200)
    table2 = table if not shared else table
    bt = T(table2, dev)
    if shared:
        bt = bt[None].expand(rows, -1)
    out = SC.fp8_paged_mqa_logits(T(q8, dev).view(torch.float8_e4m3fn), T(native, dev), T(w, dev), T(lens, dev), bt,
                                  None, ctx, clean_logits=True)
    ref = O.paged_logits(q8, w, native, np.broadcast_to(table, (rows, table.shape[-1])) if shared else table, lens,
                         ctx)
    got = H(out).astype(np.float64)
    bound = O.paged_logits(q8, w, native, np.broadcast_to(table, (rows, table.shape[-1])) if shared else table,
                           lens, ctx, magnitude=True)
    assert_scores_close(got, ref, bound)


@pytest.mark.parametrize("rows,ctx", [(45, 5000), (300, 700), (8, 9000)])
def test_score_shared_uneven_lengths(dev, rows, ctx):
    """Shared table with unordered lengths, empty rows and a column limit past
    every context: the work split by equal page spans must still write every
    logit once (unwritten columns would keep the NaN fill)."""
    g = np.random.default_rng(rows + ctx)
    q8, w, native, table, _ = _score_case(g, rows, 64, ctx, True, 200)
    lens = g.integers(0, ctx + 1, rows).astype(np.int32)
    lens[g.random(rows) < 0.2] = 0
    width = ctx + 100
    out = torch.full((rows, width + 4), float("nan"), device=dev)
    bt = T(table, dev)[None].expand(rows, -1)
    SC.fp8_paged_mqa_logits(T(q8, dev).view(torch.float8_e4m3fn), T(native, dev), T(w, dev), T(lens, dev), bt, None,
                            width, clean_logits=True, out=out)
    full = np.broadcast_to(table, (rows, table.shape[-1]))
    ref = O.paged_logits(q8, w, native, full, lens, width)
    bound = O.paged_logits(q8, w, native, full, lens, width, magnitude=True)
    got = H(out).astype(np.float64)
    assert np.isnan(got[:, width:]).all()
    assert_scores_close(got[:, :width], ref, bound)


@pytest.mark.parametrize("rows,heads,relu", [(45, 64, True), (21, 48, False), (13, 7, True), (300, 64, False)])
def test_score_shared_unclean_leaves_columns(dev, rows, heads, relu):
    """Shared table, clean_logits off: columns at or past each row's length
    keep the caller's values (whole pages of a row past its length issue no
    store into the logits), with or without the ReLU."""
    g = np.random.default_rng(rows * 7 + heads)
    ctx = 4500
    q8, w, native, table, _ = _score_case(g, rows, heads, ctx, True, 200)
    lens = g.integers(0, ctx + 1, rows).astype(np.int32)
    lens[g.random(rows) < 0.2] = 0
    lens[::5] = ctx
    out = torch.full((rows, ctx), 7.0, device=dev)
    bt = T(table, dev)[None].expand(rows, -1)
    SC.fp8_paged_mqa_logits(T(q8, dev).view(torch.float8_e4m3fn), T(native, dev), T(w, dev), T(lens, dev), bt, None,
                            ctx, clean_logits=False, relu=relu, out=out)
    full = np.broadcast_to(table, (rows, table.shape[-1]))
    ref = O.paged_logits(q8, w, native, full, lens, ctx, relu=relu, clean=False)
    bound = O.paged_logits(q8, w, native, full, lens, ctx, clean=False, magnitude=True)
    got = H(out).astype(np.float64)
    past = np.arange(ctx)[None, :] >= lens[:, None]
    assert (got[past] == 7.0).all()
    ref[past] = 7.0
    assert_scores_close(got, ref, bound)


def assert_scores_close(got, ref, bound):
    """1e-2 relative, plus the fp32 accumulation allowance 2^-16 * sum|w q k s|
    that a near-zero (cancelling) dot product needs."""
    fin = np.isfinite(ref)
    assert np.array_equal(fin, np.isfinite(got))
    err = np.abs(got[fin] - ref[fin])
    tol = 1e-2 * np.abs(ref[fin]) + 2.0 ** -16 * bound[fin]
    bad = err > tol
    if bad.any():
        i = int(np.argmax(err - tol))
        raise AssertionError(f"{int(bad.sum())} scores out of tolerance; worst got={got[fin][i]!r} "
                             f"ref={ref[fin][i]!r} magnitude={bound[fin][i]!r}")


def assert_scores_rel(got, ref):
    """The score tolerance where every head weight is >= 0 (so every
    reference score is >= 0): each finite score within 1e-2 relative of the
    fp64 reference, exactly +0.0 (bit for bit) where the reference is 0, and
    the same -inf pattern."""
    fin = np.isfinite(ref)
    assert np.array_equal(fin, np.isfinite(got)) and (got[~fin] == ref[~fin]).all()
    g, r = got[fin], ref[fin]
    assert (r >= 0).all(), "negative reference score: weights below 0"
    zero = r == 0
    bad_zero = zero & ((g != 0) | np.signbit(g))
    if bad_zero.any():
        raise AssertionError(f"{int(bad_zero.sum())} scores not +0.0 where the reference is 0")
    rel = np.abs(g[~zero] - r[~zero]) / r[~zero]
    if rel.size and rel.max() > 1e-2:
        i = int(np.argmax(rel))
        raise AssertionError(f"{int((rel > 1e-2).sum())} scores beyond 1e-2 relative; worst got={g[~zero][i]!r} "
                             f"ref={r[~zero][i]!r} rel={rel[i]:.3e}")
    return float(rel.max()) if rel.size else 0.0


def _adversarial_rows(kind, g, cols):
    if kind == "plateau":  # one value everywhere but a few larger ones: candidate count >> cap
        r = np.full(cols, 3.0, np.float32)
        r[g.choice(cols, 500, replace=False)] = g.random(500).astype(np.float32) + 4
        return r
    if kind == "ascending":  # strided sample sees a uniform ramp; the top is one contiguous run
        return np.linspace(-1, 1, cols).astype(np.float32)
    if kind == "descending":
        return np.linspace(1, -1, cols).astype(np.float32)
    if kind == "neg_inf_heavy":  # fewer real keys than T
        r = np.full(cols, -np.inf, np.float32)
        r[g.choice(cols, 1500, replace=False)] = g.standard_normal(1500).astype(np.float32)
        return r
    if kind == "two_values":
        return np.where(g.random(cols) < 0.5, 1.0, 2.0).astype(np.float32)
    if kind == "tiny_spread":  # keys differ only in the lowest mantissa bits
        return (np.float32(1.0) + g.integers(0, 64, cols).astype(np.float32) * np.float32(2 ** -23)).astype(np.float32)
    if kind == "signed_zero":
        return np.where(g.random(cols) < 0.5, np.float32(0.0), np.float32(-0.0)).astype(np.float32)
    if kind == "nan_sprinkled":  # +NaN above +inf, -NaN below -inf, payload order among NaNs
        r = g.standard_normal(cols).astype(np.float32)
        bits = r.view(np.uint32)
        pos = g.random(cols) < 0.01
        neg = ~pos & (g.random(cols) < 0.01)
        bits[pos] = 0x7f800001 + g.integers(0, 1 << 22, int(pos.sum())).astype(np.uint32)
        bits[neg] = 0xff800001 + g.integers(0, 1 << 22, int(neg.sum())).astype(np.uint32)
        return r
    if kind == "sparse_nan":  # fewer keys above -inf than T, with -NaNs below -inf and +NaNs above +inf
        r = np.full(cols, -np.inf, np.float32)
        at = g.permutation(cols)
        r[at[:1200]] = g.standard_normal(min(1200, cols)).astype(np.float32)
        bits = r.view(np.uint32)
        neg, pos = at[1200:1400], at[1400:1500]
        bits[neg] = 0xff800001 + g.integers(0, 1 << 22, neg.size).astype(np.uint32)
        bits[pos] = 0x7f800001 + g.integers(0, 1 << 22, pos.size).astype(np.uint32)
        return r
    if kind == "nan_heavy":  # more +NaNs than T: the pivot falls in the NaN key range
        r = g.standard_normal(cols).astype(np.float32)
        bits = r.view(np.uint32)
        at = g.choice(cols, min(cols, 3000), replace=False)
        bits[at] = 0x7fc00000 + g.integers(0, 1 << 22, at.size).astype(np.uint32) % (1 << 22)
        return r
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["plateau", "ascending", "descending", "neg_inf_heavy", "two_values", "tiny_spread",
                                  "signed_zero", "nan_sprinkled", "nan_heavy", "sparse_nan"])
@pytest.mark.parametrize("cols", [2049, 8192, 9000, 32768, 100000])
def test_topk_adversarial_rows(dev, kind, cols):
    g = np.random.default_rng(cols)
    B = 4
    stride = -(-cols // 4) * 4  # the reference requires a row stride that is a multiple of 4
    scores = np.zeros((B, stride), np.float32)
    scores[:, :cols] = np.stack([_adversarial_rows(kind, g, cols) for _ in range(B)])
    lens = np.int32([cols, cols - 1, 2049, min(cols, 2048)])
    table = np.arange((cols + 63) // 64, dtype=np.int32)[None].repeat(B, 0)
    out = torch.empty((B, 2048), device=dev, dtype=torch.int32)
    raw = torch.empty_like(out)
    TK.topk_transform_512_v2(T(scores, dev)[:, :cols], T(lens, dev), T(table, dev), out, 64, None, raw)
    e_out, e_raw = O.transform_topk(scores[:, :cols], lens, table, 2048, 6)
    assert np.array_equal(H(raw), e_raw) and np.array_equal(H(out), e_out)


@pytest.mark.parametrize("cols", [2100, 9000, 32768, 40960])
def test_topk_large_batch_vs_oracle(dev, cols):
    """1100 rows (more than four per CU) of varying lengths with every
    adversarial row kind mixed in (their pivot misses take the re-aimed pivot
    or the exact passes), rows of at most T candidates and a padded row
    stride, up to the 40960 columns one work-group selects over (a 640-entry
    page table); every row compared with the oracle."""
    g = np.random.default_rng(cols + 7)
    B = 1100
    stride = -(-cols // 4) * 4 + 4
    scores = g.standard_normal((B, stride)).astype(np.float32)
    kinds = ["plateau", "ascending", "descending", "neg_inf_heavy", "two_values", "tiny_spread", "signed_zero",
             "nan_sprinkled", "nan_heavy"]
    for i, kind in enumerate(kinds):
        for j in range(4):
            scores[37 * i + j, :cols] = _adversarial_rows(kind, g, cols)
    lens = g.integers(2049, cols + 1, B).astype(np.int32)
    lens[[5, 600]] = [2048, 100]
    lens[[6, 601]] = cols
    table = np.arange(-(-cols // 64), dtype=np.int32)[None].repeat(B, 0)
    out = torch.empty((B, 2048), device=dev, dtype=torch.int32)
    raw = torch.empty_like(out)
    TK.topk_transform_512_v2(T(scores, dev)[:, :cols], T(lens, dev), T(table, dev), out, 64, None, raw)
    e_out, e_raw = O.transform_topk(scores[:, :cols], lens, table, 2048, 6)
    raw_h, out_h = H(raw), H(out)
    bad = np.flatnonzero((raw_h != e_raw).any(axis=1))
    assert bad.size == 0, f"rows {bad[:10].tolist()} differ"
    assert np.array_equal(out_h, e_out)


@pytest.mark.parametrize("page_size", [16, 64, 128, 1024])
@pytest.mark.parametrize("short_table", [False, True])
@pytest.mark.parametrize("cols", [32768, 6000, 40000])
def test_topk_transform_page_sizes(dev, page_size, short_table, cols):
    """Page sizes either side of 64 tokens (the register-resident rows take
    tables of at most 512 entries, smaller pages stream), a page table that
    covers only part of each row (positions past it map to -1), rows of every
    length class, more rows than CUs, and no raw output on half the calls;
    at 6000 columns every row is held in registers (the short-row kernel)."""
    g = np.random.default_rng(page_size + short_table)
    B = 700
    scores = np.round(g.standard_normal((B, cols)) * 30).astype(np.float32)
    lens = g.integers(1, cols + 1, B).astype(np.int32)
    lens[:4] = [cols, 2048, 2049, 1]
    entries = -(-cols // page_size)
    if short_table:
        entries = entries * 3 // 4
    table = g.integers(0, 1 << 18, (B, entries)).astype(np.int32)
    bits = page_size.bit_length() - 1
    full = np.zeros((B, -(-cols // page_size)), np.int32)
    full[:, :entries] = table
    e_out, e_raw = O.transform_topk(scores, lens, full, 2048, bits)
    e_out[(e_raw >> bits) >= entries] = -1  # no table entry: unmapped
    out = torch.empty((B, 2048), device=dev, dtype=torch.int32)
    raw = torch.empty_like(out)
    TK.topk_transform_512_v2(T(scores, dev), T(lens, dev), T(table, dev), out, page_size, None, raw)
    assert np.array_equal(H(raw), e_raw) and np.array_equal(H(out), e_out)
    out2 = torch.empty_like(out)
    TK.topk_transform_512_v2(T(scores, dev), T(lens, dev), T(table, dev), out2, page_size, None, None)
    assert np.array_equal(H(out2), e_out)


@pytest.mark.parametrize("topk", [1, 37, 2047, 2048])
def test_topk_transform_odd_topk_single_pass(dev, topk):
    """Rows within one work-group's span with T not a multiple of 4: the
    slot-order output then takes the element-wise stores (output rows are
    not 16-byte aligned), with ties, -inf and rows shorter than T."""
    g = np.random.default_rng(topk)
    B, cols = 300, 20000
    scores = np.round(g.standard_normal((B, cols)) * 8).astype(np.float32)
    scores[g.random((B, cols)) < 0.01] = -np.inf
    lens = g.integers(1, cols + 1, B).astype(np.int32)
    lens[:3] = [cols, topk, max(1, topk - 1)]
    table = g.integers(0, 1 << 20, (B, -(-cols // 64))).astype(np.int32)
    out = torch.empty((B, topk), device=dev, dtype=torch.int32)
    raw = torch.empty_like(out)
    TK.topk_transform_512_v2(T(scores, dev), T(lens, dev), T(table, dev), out, 64, None, raw)
    e_out, e_raw = O.transform_topk(scores, lens, table, topk, 6)
    assert np.array_equal(H(raw), e_raw) and np.array_equal(H(out), e_out)


# ------------------------------------------------- unfused C4 x4 expansion
@pytest.mark.parametrize("rows,topk,stride,block,offset", [
    (64, 2048, 4 * 2048 + 64, 16384, 0),   # runtime.py:638-641 shape (BLOCK = next power of two)
    (7, 5, 23, 32, 0),                     # odd stride: scalar stores
    (5, 6, 40, 16, 0),                     # BLOCK < STRIDE: columns past BLOCK untouched
    (9, 10, 12, 16, 0),                    # stride < 4 * topk: truncated
    (33, 300, 4 * 300 + 64, 2048, 1),      # output rows not 16-byte aligned
])
def test_expand_logical_vs_oracle(dev, rows, topk, stride, block, offset):
    g = np.random.default_rng(rows * 1000 + topk)
    logical = g.integers(0, 1 << 20, (rows, topk)).astype(np.int32)
    logical[g.random((rows, topk)) < 0.1] = -1
    logical[0, :2] = [2 ** 29 + 1, np.iinfo(np.int32).max]  # int32 wrap of 4 * index
    backing = torch.full((rows * stride + offset,), 7, device=dev, dtype=torch.int32)
    out = backing[offset:].view(rows, stride)
    K.expand_logical[(rows,)](T(logical, dev), out, topk, stride, block)
    exp = np.full((rows, stride), 7, np.int32)
    O.expand_logical(logical, exp, block)
    assert np.array_equal(H(out), exp)
    assert int(backing[:offset].ne(7).sum()) == 0 if offset else True
