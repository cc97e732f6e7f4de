"""End-to-end GPU parity on the benchmark workloads at their full sizes.

Each stage runs through the C ABI on the GPU; its output is checked against the
oracle on the same inputs (the GPU result of the previous stage), bit-exact for
ids, tables and bytes and within the score tolerance for logits.  Where the
oracle cannot cover every row in seconds, a fixed sample of rows (always the
first, the last and the longest) is compared and the rest is checked through
size-independent properties.
"""
import numpy as np
import pytest
import torch

from conftest import pkg
from oracle import v1 as O
from test_gpu_kernels import H, T, assert_scores_close, assert_scores_rel

pytestmark = pytest.mark.gpu

QF = pkg("query_fused")
K = pkg("kernels")
NK = pkg("native_kernels")
SC = pkg("scoring")
TK = pkg("topk")
W = pkg("workloads")


def _sample_rows(n, g, extra=()):
    rows = {0, n - 1, *extra}
    rows.update(int(x) for x in g.choice(n, min(n, 6), replace=False))
    return np.array(sorted(rows))


def test_config1_query_chain(dev):
    """Reference example shape (1024 queries, 1 head, P=128, 40 of 64 pages,
    2688 candidates): coarse score -> route (+ fine table) -> shared tail
    staging -> fine score -> fused Top-2048 with mask -> slot gather, the
    order of Query.compute (sglang/srt/layers/attention/v1_deepseek/runtime.py:417-678)."""
    wl = W.config1()
    a, prm = wl.arrays, wl.params
    B, P, CAP, TAKE, WIDTH, TOP = prm["B"], prm["P"], prm["CAP"], prm["TAKE"], prm["WIDTH"], prm["TOPK"]
    q = T(a["q8"], dev).view(torch.float8_e4m3fn)
    w = T(a["w"], dev)
    # coarse: 512 centers (8 per built page), columns of the 128-page route width
    center_lens = np.full(B, 512, np.int32)
    ctab = np.broadcast_to(a["center_table"], (B, a["center_table"].shape[0]))
    coarse = SC.fp8_paged_mqa_logits(q, T(a["centers"], dev), w, T(center_lens, dev),
                                     T(a["center_table"], dev)[None].expand(B, -1), None, P * 8, clean_logits=True)
    ref = O.paged_logits(a["q8"], a["w"], a["centers"], ctab, center_lens, P * 8)
    bound = O.paged_logits(a["q8"], a["w"], a["centers"], ctab, center_lens, P * 8, magnitude=True)
    coarse_h = H(coarse)
    # One head: a dot at or just below 0 can come out of the fp32 MFMA
    # accumulation slightly positive (its FP8 products span more than the 24
    # bits of an fp32 sum), and ReLU keeps it, so scores near 0 get the
    # accumulation allowance; the 64-head workloads below use the plain
    # relative bound with exact zeros.
    assert_scores_close(coarse_h.astype(np.float64), ref, bound)

    # route with the fine-table fill
    sel = torch.empty((B, TAKE), device=dev, dtype=torch.int32)
    ft = torch.empty((B, prm["FT_COLS"]), device=dev, dtype=torch.int32)
    QF.module().route(coarse, T(a["lens"], dev), T(a["takes"], dev), sel, P, T(a["rt"], dev), ft,
                      T(a["tail_rows"], dev), CAP, True)
    e_sel = np.full((B, TAKE), -1, np.int32)
    e_ft = np.full((B, prm["FT_COLS"]), -1, np.int32)
    O.route(coarse_h, a["lens"], a["takes"], e_sel, P, a["rt"], e_ft, a["tail_rows"], CAP, True)
    sel_h, ft_h = H(sel), H(ft)
    assert np.array_equal(sel_h, e_sel) and np.array_equal(ft_h, e_ft)
    # the unfused table kernel gives the same table
    ft2 = torch.empty_like(ft)
    K.fine_table_shared[(B,)](T(a["rt"], dev), sel, T(a["takes"], dev), T(a["lens"], dev), ft2, T(a["tail_rows"], dev),
                              CAP, P, TAKE, prm["FT_COLS"], 68, 32)
    assert np.array_equal(H(ft2), ft_h)

    # shared tail staging into the fine pool (one owner: every row shares row 0's tail)
    fine = a["fine"].copy()
    fine_d = T(fine, dev)
    K.stage_tail_shared[(-(-B // 32), 68)](T(a["native"], dev), None, T(a["nt"], dev), T(a["lens"], dev), fine_d, None,
                                           T(a["tail_rows"], dev), CAP, P, 68, prm["SINK"], prm["WINDOW"], ROWS=B,
                                           GROUP=32)
    O.stage_tail(a["native"], a["nt"], a["lens"], fine, CAP, 68, prm["SINK"], prm["WINDOW"], tail_rows=a["tail_rows"],
                 rows=B)
    fine_h = H(fine_d)
    assert np.array_equal(fine_h, fine)

    # fine score over each row's fine table
    fl = a["fine_lens"]
    logits = SC.fp8_paged_mqa_logits(q, fine_d, w, T(fl, dev), ft, None, WIDTH, clean_logits=True)
    ref = O.paged_logits(a["q8"], a["w"], fine_h, ft_h, fl, WIDTH)
    bound = O.paged_logits(a["q8"], a["w"], fine_h, ft_h, fl, WIDTH, magnitude=True)
    logits_h = H(logits)
    assert_scores_close(logits_h.astype(np.float64), ref, bound)

    # fused Top-2048 with the sink/tail mask, then the slot gather
    physical = torch.empty((B, TOP), device=dev, dtype=torch.int32)
    logical = torch.empty_like(physical)
    raw = torch.empty_like(physical)
    expanded = torch.empty((B, 4 * TOP + 64), device=dev, dtype=torch.int32)
    QF.module().topk(logits, T(fl, dev), T(a["members"], dev), T(a["rt"], dev), T(a["nt"], dev), sel,
                     T(a["lens"], dev), T(a["takes"], dev), physical, logical, raw, prm["WINDOW"], True, expanded,
                     True, True, ft, False)
    masked = logits_h.copy()
    exp = O.fused_topk(masked, fl, a["members"], a["rt"], a["nt"], sel_h, a["lens"], a["takes"], TOP, prm["WINDOW"],
                       True, 4 * TOP + 64, True, True, ft_h, False)
    assert np.array_equal(H(logits), masked)
    for name, got in (("raw", raw), ("logical", logical), ("physical", physical), ("expanded", expanded)):
        assert np.array_equal(H(got), exp[name]), name
    out = torch.empty((B, TOP, W.MLA_ROW_BYTES), device=dev, dtype=torch.uint8)
    NK.gather_rows(T(a["latent"], dev), physical, out)
    assert np.array_equal(H(out), O.gather_rows(a["latent"], exp["physical"]))


def test_config9_whole_query(dev):
    """The reference's published whole-query shape (1024 queries x 64 heads,
    64K context, route of 512 of 1024 pages, 34880 candidates): coarse score
    -> route (+ fine table) -> shared tail staging -> fine score -> fused
    Top-2048 with mask (rows above 32768 columns: segments and merge) -> x4
    expansion, as bench.py runs it.  Route, table, staging and expansion are
    compared on every row, the scores and the Top-K on sampled rows (the
    Top-K oracle on the GPU's logits)."""
    wl = W.config9()
    a, prm = wl.arrays, wl.params
    B, P, CAP, TAKE, WIDTH, TOP = prm["B"], prm["P"], prm["CAP"], prm["TAKE"], prm["WIDTH"], prm["TOPK"]
    rows = _sample_rows(B, np.random.default_rng(9))
    q = T(a["q8"], dev).view(torch.float8_e4m3fn)
    w = T(a["w"], dev)
    center_lens = np.full(B, prm["CENTERS"], np.int32)
    ctab = np.broadcast_to(a["center_table"], (B, a["center_table"].shape[0]))
    coarse = SC.fp8_paged_mqa_logits(q, T(a["centers"], dev), w, T(center_lens, dev),
                                     T(a["center_table"], dev)[None].expand(B, -1), None, P * 8, clean_logits=True)
    coarse_h = H(coarse)
    args = (a["q8"][rows], a["w"][rows], a["centers"], ctab[rows], center_lens[rows], P * 8)
    assert_scores_rel(coarse_h[rows].astype(np.float64), O.paged_logits(*args))

    sel = torch.empty((B, TAKE), device=dev, dtype=torch.int32)
    ft = torch.empty((B, prm["FT_COLS"]), device=dev, dtype=torch.int32)
    QF.module().route(coarse, T(a["lens"], dev), T(a["takes"], dev), sel, P, T(a["rt"], dev), ft,
                      T(a["tail_rows"], dev), CAP, True)
    e_sel = np.full((B, TAKE), -1, np.int32)
    e_ft = np.full((B, prm["FT_COLS"]), -1, np.int32)
    O.route(coarse_h, a["lens"], a["takes"], e_sel, P, a["rt"], e_ft, a["tail_rows"], CAP, True)
    sel_h, ft_h = H(sel), H(ft)
    assert np.array_equal(sel_h, e_sel) and np.array_equal(ft_h, e_ft)

    fine = a["fine"].copy()
    fine_d = T(fine, dev)
    K.stage_tail_shared[(-(-B // 32), 68)](T(a["native"], dev), None, T(a["nt"], dev), T(a["lens"], dev), fine_d, None,
                                           T(a["tail_rows"], dev), CAP, P, 68, prm["SINK"], prm["WINDOW"], ROWS=B,
                                           GROUP=32)
    O.stage_tail(a["native"], a["nt"], a["lens"], fine, CAP, 68, prm["SINK"], prm["WINDOW"], tail_rows=a["tail_rows"],
                 rows=B)
    fine_h = H(fine_d)
    assert np.array_equal(fine_h, fine)

    fl = a["fine_lens"]
    logits = SC.fp8_paged_mqa_logits(q, fine_d, w, T(fl, dev), ft, None, WIDTH, clean_logits=True)
    logits_h = H(logits)
    args = (a["q8"][rows], a["w"][rows], fine_h, ft_h[rows], fl[rows], WIDTH)
    worst = assert_scores_rel(logits_h[rows].astype(np.float64), O.paged_logits(*args))

    physical = torch.empty((B, TOP), device=dev, dtype=torch.int32)
    logical = torch.empty_like(physical)
    raw = torch.empty_like(physical)
    no_exp = torch.empty_strided((B, 0), (0, 1), device=dev, dtype=torch.int32)
    QF.module().topk(logits, T(fl, dev), T(a["members"], dev), T(a["rt"], dev), T(a["nt"], dev), sel,
                     T(a["lens"], dev), T(a["takes"], dev), physical, logical, raw, prm["WINDOW"], True, no_exp,
                     True, True, ft, False)
    expanded = torch.full((B, 4 * TOP + 64), 5, device=dev, dtype=torch.int32)
    K.expand_logical[(B,)](logical, expanded, TOP, expanded.shape[1], 1 << (expanded.shape[1] - 1).bit_length())
    # every row: the in-place mask, the Top-K and its raw -> logical ->
    # physical map against the oracle on the GPU's logits
    masked = logits_h.copy()
    exp = O.fused_topk_rows(masked, fl, a["members"], a["rt"], a["nt"], sel_h, a["lens"], a["takes"], TOP,
                            prm["WINDOW"], True, 0, True, True, ft_h, False)
    assert np.array_equal(H(logits), masked)
    for name, got in (("raw", raw), ("logical", logical), ("physical", physical)):
        assert np.array_equal(H(got), exp[name]), name
    logical_h = H(logical)
    e_exp = np.full((B, 4 * TOP + 64), 5, np.int32)
    O.expand_logical(logical_h, e_exp, 1 << (e_exp.shape[1] - 1).bit_length())
    assert np.array_equal(H(expanded), e_exp)
    print(f"config 9: {B} rows mask/Top-K/map equal; fine scores of {len(rows)} rows within {worst:.2e} relative")


def test_config3_gather_full(dev):
    """1024 x 2048 ids (5% -1) through per-row 512-page windows of a 1M-row
    pool of 656-byte rows, every output byte compared."""
    wl = W.config3()
    a, prm = wl.arrays, wl.params
    out = torch.empty((prm["rows"], prm["top"], prm["row_bytes"]), device=dev, dtype=torch.uint8)
    NK.gather_rows(T(a["pool"], dev), T(a["ids"], dev), out, table=T(a["table"], dev), page_bits=prm["page_bits"])
    exp = O.gather_rows(a["pool"], a["ids"], a["table"], prm["page_bits"])
    assert np.array_equal(H(out), exp)


def test_config4_prefill_chunk(dev):
    """4096 queries x 64 heads over a 32768-token causal context: score, Top-2048
    slot map and gather for every row on the GPU.  The Top-K indices and slots
    of every row equal the oracle's Top-K on the GPU's logits; scores of sampled
    rows are within 1e-2 relative of the fp64 reference (exact zeros bit for
    bit); gathered bytes of 64 rows are compared byte for byte."""
    wl = W.config4()
    a, prm = wl.arrays, wl.params
    rows, ctx, TOP = prm["rows"], prm["ctx"], prm["topk"]
    table = T(a["table"], dev)
    logits = SC.fp8_paged_mqa_logits(T(a["q8"], dev).view(torch.float8_e4m3fn), T(a["native"], dev), T(a["w"], dev),
                                     T(a["lens"], dev), table[None].expand(rows, -1), None, ctx, clean_logits=True)
    slots = torch.empty((rows, TOP), device=dev, dtype=torch.int32)
    raw = torch.empty_like(slots)
    TK.topk_transform_512_v2(logits, T(a["lens"], dev), table[None].expand(rows, -1).contiguous(), slots, 64, None, raw)
    out = torch.empty((rows, TOP, prm["row_bytes"]), device=dev, dtype=torch.uint8)
    NK.gather_rows(T(a["latent"], dev), slots, out)

    g = np.random.default_rng(4)
    pick = _sample_rows(rows, g)
    lg = H(logits[torch.from_numpy(pick).to(dev)]).astype(np.float64)
    full = np.broadcast_to(a["table"], (len(pick), a["table"].shape[0]))
    ref = O.paged_logits(a["q8"][pick], a["w"][pick], a["native"], full, a["lens"][pick], ctx)
    worst = assert_scores_rel(lg, ref)
    # every row's Top-K and slots against the oracle on the GPU's logits
    table_all = np.broadcast_to(a["table"], (rows, a["table"].shape[0]))
    e_slots, e_raw = O.transform_topk_rows(H(logits), a["lens"], table_all, TOP, 6)
    raw_h, slots_h = H(raw), H(slots)
    assert np.array_equal(raw_h, e_raw) and np.array_equal(slots_h, e_slots)
    # gathered bytes: 64 rows (first, last and a seeded sample)
    grows = np.unique(np.concatenate([[0, rows - 1], g.choice(rows, 62, replace=False)]))
    assert np.array_equal(H(out[torch.from_numpy(grows).to(dev)]), O.gather_rows(a["latent"], e_slots[grows]))
    print(f"config 4: {rows} rows Top-K/slots equal; scores of {len(pick)} rows within {worst:.2e} relative; "
          f"gather of {len(grows)} rows equal")


def test_config5_decode_batch(dev):
    """128 requests with their own page tables into the 2M-token (32768-page)
    pool, contexts 4K..128K tokens (rows past 32768 candidates take the
    segmented Top-K), scored over every context key; the 656-byte latent rows
    follow a closed form built on the device."""
    wl = W.config5()
    a, prm = wl.arrays, wl.params
    rows, TOP, max_ctx = prm["rows"], prm["topk"], prm["max_ctx"]
    table = T(a["table"], dev)
    # the Top-K reads rows with 16-byte loads: row stride padded to 4 columns
    logits = torch.empty((rows, -(-max_ctx // 4) * 4), device=dev)[:, :max_ctx]
    SC.fp8_paged_mqa_logits(T(a["q8"], dev).view(torch.float8_e4m3fn), T(a["native"], dev), T(a["w"], dev),
                            T(a["lens"], dev), table, None, max_ctx, clean_logits=True, out=logits)
    slots = torch.empty((rows, TOP), device=dev, dtype=torch.int32)
    raw = torch.empty_like(slots)
    TK.topk_transform_512_v2(logits, T(a["lens"], dev), table, slots, 64, None, raw)
    g = np.random.default_rng(5)
    rb = prm["row_bytes"]
    row_term = ((torch.arange(prm["latent_rows"], device=dev, dtype=torch.int64) * 131) & 255).to(torch.uint8)
    col_term = ((torch.arange(rb, device=dev, dtype=torch.int64) * 7) & 255).to(torch.uint8)
    latent = row_term[:, None] + col_term[None]  # uint8 addition wraps mod 256
    out = torch.empty((rows, TOP, rb), device=dev, dtype=torch.uint8)
    NK.gather_rows(latent, slots, out)

    pick = _sample_rows(rows, g, extra=(int(np.argmax(a["lens"])), int(np.argmin(a["lens"]))))
    lg = H(logits[torch.from_numpy(pick).to(dev)]).astype(np.float64)
    ref = O.paged_logits(a["q8"][pick], a["w"][pick], a["native"], a["table"][pick], a["lens"][pick], max_ctx)
    assert_scores_rel(lg, ref)
    e_slots, e_raw = O.transform_topk(lg.astype(np.float32), a["lens"][pick], a["table"][pick], TOP, 6)
    raw_h, slots_h = H(raw), H(slots)
    assert np.array_equal(raw_h[pick], e_raw) and np.array_equal(slots_h[pick], e_slots)
    got = H(out[torch.from_numpy(pick).to(dev)])
    assert np.array_equal(got, np.where((e_slots >= 0)[..., None], _latent_rows(np.maximum(e_slots, 0), rb), 0))
    assert (np.diff(raw_h, axis=1) > 0).all() and (raw_h < a["lens"][:, None]).all()


def _latent_rows(ids, row_bytes):
    """Closed-form 656-byte latent rows (byte c of row i = (131 i + 7 c) mod 256)."""
    ids = np.asarray(ids, np.int64)
    return ((ids[..., None] * 131 + np.arange(row_bytes) * 7) & 255).astype(np.uint8)


@pytest.fixture(scope="module")
def config5_route():
    return W.config5_route()


def test_config5_route_chain(dev, config5_route):
    """The decode batch as the reference runs it for <= 512 rows
    (sglang/srt/layers/attention/v1_deepseek/runtime.py:417-634, page_fraction
    0.5): center score -> fused route -> fine_table_shared -> stage_tail_shared
    -> fine score -> mask_fine -> topk_transform_512_v2 -> output_ids -> gather,
    128 requests of 4K..128K tokens over the 2M-token pool.  Integer hand-offs
    are compared on every row, scores, staging, mask and gather on the first,
    last, longest and shortest rows and a seeded sample; fine widths reach
    ~67 K columns (segmented Top-K)."""
    wl = config5_route
    a, prm = wl.arrays, wl.params
    rows, P, CAP, TAKE, WIDTH, FP = prm["rows"], prm["P"], prm["CAP"], prm["TAKE"], prm["WIDTH"], prm["FP"]
    TOP, SINK, WIN = prm["topk"], prm["sink"], prm["window"]
    d = {k: T(v, dev) for k, v in a.items() if k not in ("fine",)}
    fine_d = T(a["fine"], dev)
    q = d["q8"].view(torch.float8_e4m3fn)
    i32 = lambda *s: torch.empty(s, device=dev, dtype=torch.int32)

    # per-row lengths and owners (kernels.py:568-591)
    fl, takes, dg_lens, center_lens, tail_rows = i32(rows), i32(rows), i32(rows), i32(rows), i32(rows)
    K.query_metadata[(rows,)](d["lens"], d["nt"], fl, takes, dg_lens, center_lens, tail_rows, P, TOP, prm["num"],
                              prm["den"], SINK, WIN)
    meta = O.query_metadata(a["lens"], a["nt"], TOP, prm["num"], prm["den"], SINK, WIN)
    for got, exp in zip((fl, takes, dg_lens, center_lens, tail_rows), meta):
        assert np.array_equal(H(got), exp)
    fl_h, takes_h, tail_h = meta[0], meta[1], meta[4]
    assert fl_h.max() > 32768  # segmented Top-K rows are part of the batch

    g = np.random.default_rng(55)
    pick = _sample_rows(rows, g, extra=(int(np.argmax(a["lens"])), int(np.argmin(a["lens"]))))
    pick_d = torch.from_numpy(pick).to(dev)

    # center score over each row's center table (8 centers per built page)
    coarse = SC.fp8_paged_mqa_logits(q, d["centers"], d["w"], center_lens, d["center_table"], None, P * 8,
                                     clean_logits=True)
    coarse_h = H(coarse)
    ref = O.paged_logits(a["q8"][pick], a["w"][pick], a["centers"], a["center_table"][pick], meta[3][pick], P * 8)
    assert_scores_rel(coarse_h[pick].astype(np.float64), ref)

    # fused route (no table fill, runtime.py:445-448), then fine_table_shared
    sel, ft = i32(rows, TAKE), i32(rows, FP)
    QF.module().route(coarse, d["lens"], takes, sel, P, d["rt"], ft, tail_rows, CAP, False)
    e_sel = np.zeros((rows, TAKE), np.int32)
    O.route(coarse_h, a["lens"], takes_h, e_sel, P, a["rt"], np.zeros((rows, FP), np.int32), tail_h, CAP, False)
    sel_h = H(sel)
    assert np.array_equal(sel_h, e_sel)
    K.fine_table_shared[(rows,)](d["rt"], sel, takes, d["lens"], ft, tail_rows, CAP, P, TAKE, FP, 68,
                                 1 << (FP - 1).bit_length())
    ft_h = H(ft)
    assert np.array_equal(ft_h, O.fine_table(a["rt"], e_sel, takes_h, FP, CAP, 68, tail_rows=tail_h))

    # shared tail staging into each owner's 68 scratch pages
    K.stage_tail_shared[(rows, 68)](d["native"], None, d["nt"], d["lens"], fine_d, None, tail_rows, CAP, P, 68, SINK,
                                    WIN, ROWS=rows, GROUP=1)
    fine_h = H(fine_d)
    for r in pick:
        if tail_h[r] != r:
            continue
        exp = np.zeros((68, 8448), np.uint8)
        O.stage_tail(a["native"], a["nt"][r:r + 1], a["lens"][r:r + 1], exp, 0, 68, SINK, WIN)
        assert np.array_equal(fine_h[CAP + r * 68:CAP + (r + 1) * 68], exp), f"staged tail of row {r}"

    # fine score over each row's fine table, then the sink/tail mask
    scores = SC.fp8_paged_mqa_logits(q, fine_d, d["w"], dg_lens, ft, None, WIDTH, clean_logits=True)
    pre = H(scores[pick_d])
    ref = O.paged_logits(a["q8"][pick], a["w"][pick], fine_h, ft_h[pick], meta[2][pick], WIDTH)
    assert_scores_rel(pre.astype(np.float64), ref)
    K.mask_fine[(rows, -(-WIDTH // 256))](scores, sel, d["rt"], d["members"], d["lens"], takes, P, TAKE,
                                          scores.stride(0), WIDTH, SINK, WIN)
    post = H(scores)
    O.mask_fine(pre, sel_h[pick], a["rt"][pick], a["members"], a["lens"][pick], takes_h[pick], WIDTH, SINK, WIN)
    assert np.array_equal(post[pick], pre)

    # Top-2048 over each row's fine candidates, then the raw -> logical -> physical map
    ident = torch.arange(FP, device=dev, dtype=torch.int32)[None].expand(rows, -1)
    transformed, raw = i32(rows, TOP), i32(rows, TOP)
    TK.topk_transform_512_v2(scores, fl, ident, transformed, 64, None, raw)
    e_tr, e_raw = O.transform_topk(post, fl_h, np.broadcast_to(np.arange(FP, dtype=np.int32), (rows, FP)), TOP, 6)
    raw_h = H(raw)
    assert np.array_equal(raw_h, e_raw) and np.array_equal(H(transformed), e_tr)
    out, logical = i32(rows, TOP), i32(rows, TOP)
    K.output_ids[(rows, -(-TOP // 256))](raw, scores, d["members"], d["rt"], d["nt"], sel, d["lens"], takes, out,
                                         logical, ft, P, P, TAKE, scores.stride(0), TOP, SINK, WIN, MAP_PHYSICAL=True,
                                         DIRECT_FINE=False, FP=FP)
    e_out, e_lg = O.output_ids(e_raw, post, a["members"], a["rt"], a["nt"], sel_h, a["lens"], takes_h,
                               scores.stride(0), TOP, SINK, WIN, True, False, ft_h)
    out_h = H(out)
    assert np.array_equal(out_h, e_out) and np.array_equal(H(logical), e_lg)
    # the same outputs from the fused Top-K for small batches (mask applied
    # in the segment pass, map in the merge) on the unmasked fine scores
    scores2 = SC.fp8_paged_mqa_logits(q, fine_d, d["w"], dg_lens, ft, None, WIDTH, clean_logits=True)
    phys2, lg2, raw2 = i32(rows, TOP), i32(rows, TOP), i32(rows, TOP)
    QF.topk_any_batch(scores2, fl, d["members"], d["rt"], d["nt"], sel, d["lens"], takes, phys2, lg2, raw2, WIN, True,
                      torch.empty((rows, 0), device=dev, dtype=torch.int32), True, False, ft, False)
    assert np.array_equal(H(raw2), e_raw) and np.array_equal(H(lg2), e_lg) and np.array_equal(H(phys2), e_out)
    # every selected token lies in its request's context, once
    for r in range(rows):
        lg = e_lg[r][e_lg[r] >= 0]
        assert lg.max() < a["lens"][r] and np.unique(lg).size == lg.size

    # gather of 656-byte latent rows through the physical slots
    rb = prm["row_bytes"]
    row_term = ((torch.arange(prm["latent_rows"], device=dev, dtype=torch.int64) * 131) & 255).to(torch.uint8)
    col_term = ((torch.arange(rb, device=dev, dtype=torch.int64) * 7) & 255).to(torch.uint8)
    latent = row_term[:, None] + col_term[None]  # uint8 addition wraps mod 256
    work = torch.empty((rows, TOP, rb), device=dev, dtype=torch.uint8)
    NK.gather_rows(latent, out, work)
    got = H(work[pick_d])
    exp = np.where((e_out[pick] >= 0)[..., None], _latent_rows(np.maximum(e_out[pick], 0), rb), 0)
    assert np.array_equal(got, exp)


def _top_fp64(scores, lens, topk):
    """Top-`topk` of each row of fp64 scores over its first lens[r] columns:
    value descending, ties toward the lower index, returned ascending."""
    out = np.full((scores.shape[0], topk), -1, np.int64)
    for b in range(scores.shape[0]):
        L = int(lens[b])
        order = np.lexsort((np.arange(L), -scores[b, :L]))[:topk]
        out[b, :min(L, topk)] = np.sort(order)
    return out


def _disagreement(got, exp, ref, bound):
    """(count of selected indices that differ, largest fp64 score inversion
    between a differing pair in units of 2^-16 * magnitude) over all rows;
    asserts each inversion is within the two scores' tolerances (a near-tie)."""
    count, worst = 0, 0.0
    for b in range(got.shape[0]):
        g, e = set(got[b][got[b] >= 0].tolist()), set(exp[b][exp[b] >= 0].tolist())
        only_got, only_exp = sorted(g - e), sorted(e - g)
        assert len(only_got) == len(only_exp)
        count += len(only_got)
        for x in only_exp:
            for y in only_got:
                gap = ref[b, x] - ref[b, y]
                tol = 1e-2 * (abs(ref[b, x]) + abs(ref[b, y])) + 2.0 ** -16 * (bound[b, x] + bound[b, y])
                assert gap <= tol, (b, x, y, gap, tol)
                worst = max(worst, gap / (2.0 ** -16 * max(bound[b, x], bound[b, y])))
    return count, worst


def test_index_agreement_with_fp64_reference_topk(dev):
    """End to end: the Top-2048 the GPU chain selects from its FP8-MFMA logits
    against a Top-2048 over the fp64 dequantised reference scores
    (sglang/srt/layers/attention/v1_deepseek/kernels.py:310-313), as the
    reference example checks its Top-K against topk on reference scores
    (example_v1_query_single_head.py:55-70).  Indices can differ only where
    two scores are within fp32 rounding of each other across the selection
    boundary: every differing pair is checked to be such a near-tie, and the
    counts are printed."""
    report = []
    # prefill chunk (4096 x 64 heads x 32K keys): sampled rows
    wl = W.config4()
    a, prm = wl.arrays, wl.params
    rows, ctx, TOP = prm["rows"], prm["ctx"], prm["topk"]
    table = T(a["table"], dev)
    logits = SC.fp8_paged_mqa_logits(T(a["q8"], dev).view(torch.float8_e4m3fn), T(a["native"], dev), T(a["w"], dev),
                                     T(a["lens"], dev), table[None].expand(rows, -1), None, ctx, clean_logits=True)
    slots = torch.empty((rows, TOP), device=dev, dtype=torch.int32)
    raw = torch.empty_like(slots)
    TK.topk_transform_512_v2(logits, T(a["lens"], dev), table[None].expand(rows, -1).contiguous(), slots, 64, None, raw)
    pick = _sample_rows(rows, np.random.default_rng(40))
    full = np.broadcast_to(a["table"], (len(pick), a["table"].shape[0]))
    ref = O.paged_logits(a["q8"][pick], a["w"][pick], a["native"], full, a["lens"][pick], ctx)
    bound = O.paged_logits(a["q8"][pick], a["w"][pick], a["native"], full, a["lens"][pick], ctx, magnitude=True)
    diff4, gap4 = _disagreement(H(raw)[pick], _top_fp64(ref, a["lens"][pick], TOP), ref, bound)
    report.append(f"prefill 4096x32K: {diff4} of {len(pick) * TOP} selected indices differ ({len(pick)} rows), "
                  f"largest inversion {gap4:.3g}")
    # reference example chain (1024 queries x 2688 candidates, masked): every row
    wl = W.config1()
    a, prm = wl.arrays, wl.params
    B, P, CAP, TAKE, WIDTH = prm["B"], prm["P"], prm["CAP"], prm["TAKE"], prm["WIDTH"]
    q, w, fl = T(a["q8"], dev).view(torch.float8_e4m3fn), T(a["w"], dev), a["fine_lens"]
    coarse = SC.fp8_paged_mqa_logits(q, T(a["centers"], dev), w, T(np.full(B, 512, np.int32), dev),
                                     T(a["center_table"], dev)[None].expand(B, -1), None, P * 8, clean_logits=True)
    sel = torch.empty((B, TAKE), device=dev, dtype=torch.int32)
    ft = torch.empty((B, prm["FT_COLS"]), device=dev, dtype=torch.int32)
    QF.module().route(coarse, T(a["lens"], dev), T(a["takes"], dev), sel, P, T(a["rt"], dev), ft,
                      T(a["tail_rows"], dev), CAP, True)
    fine = a["fine"].copy()
    O.stage_tail(a["native"], a["nt"], a["lens"], fine, CAP, 68, prm["SINK"], prm["WINDOW"], tail_rows=a["tail_rows"],
                 rows=B)
    logits1 = SC.fp8_paged_mqa_logits(q, T(fine, dev), w, T(fl, dev), ft, None, WIDTH, clean_logits=True)
    physical = torch.empty((B, TOP), device=dev, dtype=torch.int32)
    logical, raw1 = torch.empty_like(physical), torch.empty_like(physical)
    QF.module().topk(logits1, T(fl, dev), T(a["members"], dev), T(a["rt"], dev), T(a["nt"], dev), sel,
                     T(a["lens"], dev), T(a["takes"], dev), physical, logical, raw1, prm["WINDOW"], True,
                     torch.empty((B, 0), device=dev, dtype=torch.int32), True, True, ft, False)
    ref1 = O.paged_logits(a["q8"], a["w"], fine, H(ft), fl, WIDTH)
    ref1[np.isneginf(H(logits1))] = -np.inf  # the sink/tail mask the kernel applied in place
    bound1 = O.paged_logits(a["q8"], a["w"], fine, H(ft), fl, WIDTH, magnitude=True)
    exp1 = _top_fp64(ref1, fl, TOP)
    diff1, gap1 = _disagreement(H(raw1), exp1, ref1, bound1)
    report.append(f"reference example 1024x2688: {diff1} of {int((exp1 >= 0).sum())} selected indices differ, "
                  f"largest inversion {gap1:.3g}")
    print("; ".join(report))
