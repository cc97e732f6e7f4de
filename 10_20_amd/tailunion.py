"""Shared sink + tail staging with a published index end, and the single-pool
page tables, score normalisation and Top-K mapping around it.

Mirrors experiments/tail_union_lab_20261021/union.py (stage_union, launch,
PreparedStage), experiments/fine_pool_shared_20261021/kernels.py (tables,
normalize, map_topk) and the per-row baseline with the same candidate rule
(experiments/tail_union_lab_20261021/baseline_published.py: stage_tail_shared
with INDEXED_END).  Launchers keep the reference's `kernel[grid](*args)` form
and argument order; block sizes, PAGE and num_warps only tune the reference's
Triton launch and are accepted and ignored.  One launch of stage_union copies
every union page that fits the destination (the reference's grid is sized
from the destination the same way).

Row bounds (union.py:10-14): s = min(n, S), t = max(s, min(min(max(end, 0),
n), max(s, n - W))), count = s + n - t; the candidates of a row with visible
length n are exactly sink [0, s), the last W positions and every position at
or past the published index end.
"""
import torch

from . import _lib
from .kernels import _Kernel

PAGE_BYTES = 8448


def _byte_pages(t):
    """Whole 8448-byte pages in a contiguous pool (any element view)."""
    if not t.is_contiguous():
        raise ValueError("page pools must be contiguous")
    return (t.numel() * t.element_size()) // PAGE_BYTES


def _i32(*tensors):
    for t in tensors:
        if t is not None and (t.dtype != torch.int32 or not t.is_contiguous()):
            raise ValueError("index tensors must be contiguous int32")


def _stage_union(grid, SRC, NT, LENS, INDEXED_END, DST, META, DESC, R, S, W, B=512, PAGE=False):
    """union.py:16-40: the union of every row's sink and tail pages -> DST,
    META[r] = (s, t, count), DESC = (sp, tp, ep, total)."""
    _lib.require_gpu(SRC, NT, LENS, INDEXED_END, DST, META, DESC)
    _i32(NT, LENS, INDEXED_END, META, DESC)
    R = int(R)
    if R < 1 or LENS.numel() < R or META.numel() < 3 * R or DESC.numel() < 4:
        raise ValueError("stage_union: R rows need R lengths, R x 3 meta and a 4-entry descriptor")
    _lib.call("v1_stage_union", _lib.ptr(SRC), _byte_pages(SRC), _lib.ptr(NT), NT.numel(), _lib.ptr(LENS), R,
              _lib.ptr(INDEXED_END), _lib.ptr(DST), _byte_pages(DST), _lib.ptr(META), _lib.ptr(DESC), int(S), int(W),
              _lib.stream_of(DST))


stage_union = _Kernel("stage_union", _stage_union)


def launch(src, nt, lens, indexed_end, dst, meta, desc, sink, window, block=512, page=False, warps=4):
    """union.py:44-46."""
    stage_union[(1,)](src.view(torch.int32), nt, lens, indexed_end, dst.view(torch.int32), meta, desc, lens.numel(),
                      sink, window, block, page, num_warps=warps)


class PreparedStage:
    """union.py:48-71: binds the views and launch parameters once; call it after
    updating lens / nt / indexed_end in place (graph-capturable, no host reads).
    dst must hold the union for every length and index end the caller replays."""

    def __init__(self, src, nt, lens, indexed_end, dst, meta, desc, sink, window, block=None, warps=4):
        checks = [
            (src.dtype == dst.dtype == torch.uint8, "src and dst must be uint8"),
            (src.is_contiguous() and dst.is_contiguous(), "src and dst must be contiguous"),
            (src.ndim == dst.ndim == 2 and src.shape[1] == dst.shape[1] == PAGE_BYTES, "pools must be [pages, 8448]"),
            (nt.ndim == lens.ndim == 1 and lens.numel() > 0, "nt and lens must be 1-D, lens non-empty"),
            (nt.is_contiguous() and lens.is_contiguous(), "nt and lens must be contiguous"),
            (nt.dtype == lens.dtype == meta.dtype == desc.dtype == indexed_end.dtype == torch.int32,
             "index tensors must be int32"),
            (tuple(indexed_end.shape) == (1,) and indexed_end.is_contiguous(), "indexed_end must be a [1] tensor"),
            (tuple(meta.shape) == (lens.numel(), 3) and desc.numel() == 4, "meta must be [rows, 3], desc 4 entries"),
            (meta.is_contiguous() and desc.is_contiguous(), "meta and desc must be contiguous"),
            (src.is_cuda and all(x.device == src.device for x in (nt, lens, indexed_end, dst, meta, desc)),
             "all tensors must be on one GPU"),
            (sink >= 0 and window >= 0, "sink and window must be non-negative"),
        ]
        for ok, msg in checks:
            if not ok:
                raise AssertionError(msg)
        self.args = (src, nt, lens, indexed_end, dst, meta, desc, lens.numel(), int(sink), int(window))

    def __call__(self):
        stage_union[(1,)](*self.args)


def _tables(grid, LENS, END, TAKES, SELECTED, DESC, FT, DGLENS, CLENS, CAP, MAXTAKE, SCRATCH, FP, S, W, B=None,
            SHARED=True):
    """kernels.py:13-35: program r writes FT[r, :FP], DGLENS[r], CLENS[r]."""
    _lib.require_gpu(LENS, END, TAKES, SELECTED, DESC, FT, DGLENS, CLENS)
    _i32(LENS, END, TAKES, SELECTED, DESC, FT, DGLENS, CLENS)
    rows = grid[0]
    if rows > 0 and (FT.numel() < rows * int(FP) or LENS.numel() < rows or TAKES.numel() < rows
                     or SELECTED.numel() < rows * int(MAXTAKE) or DGLENS.numel() < rows or CLENS.numel() < rows):
        raise ValueError("tables: tensors smaller than the grid addresses")
    _lib.call("v1_union_tables", _lib.ptr(LENS), _lib.ptr(END), _lib.ptr(TAKES), _lib.ptr(SELECTED), _lib.ptr(DESC),
              _lib.ptr(FT), _lib.ptr(DGLENS), _lib.ptr(CLENS), rows, int(CAP), int(MAXTAKE), int(SCRATCH), int(FP),
              int(S), int(W), int(bool(SHARED)), _lib.stream_of(FT))


def _normalize(grid, RAW, LENS, END, TAKES, SELECTED, MEMBERS, OUT, MAXTAKE, WIDTH, STRIDE, S, W, B=None,
               SHARED=True):
    """kernels.py:38-59: OUT[r, :WIDTH] = raw scores in canonical candidate order,
    -inf where masked."""
    _lib.require_gpu(RAW, LENS, END, TAKES, SELECTED, MEMBERS, OUT)
    _i32(LENS, END, TAKES, SELECTED, MEMBERS)
    if RAW.dtype != torch.float32 or OUT.dtype != torch.float32 or not OUT.is_contiguous():
        raise ValueError("normalize: RAW and OUT must be float32 (OUT contiguous)")
    rows, width = grid[0], int(WIDTH)
    if rows > 0 and OUT.numel() < rows * width:
        raise ValueError("normalize: OUT smaller than rows x WIDTH")
    raw_cols = RAW.shape[-1] if RAW.dim() >= 2 else RAW.numel()
    _lib.call("v1_union_normalize", _lib.ptr(RAW), int(STRIDE), raw_cols, _lib.ptr(LENS), _lib.ptr(END),
              _lib.ptr(TAKES), _lib.ptr(SELECTED), _lib.ptr(MEMBERS), MEMBERS.numel() // 64, _lib.ptr(OUT), rows,
              int(MAXTAKE), width, int(S), int(W), int(bool(SHARED)), _lib.stream_of(OUT))


def _map_topk(grid, IDS, VALUES, LENS, END, TAKES, SELECTED, MEMBERS, NT, LOGICAL, SLOTS, MAXTAKE, TOP, S, W,
              B=None):
    """kernels.py:62-76: Top-K candidate ids -> LOGICAL positions and SLOTS."""
    _lib.require_gpu(IDS, VALUES, LENS, END, TAKES, SELECTED, MEMBERS, NT, LOGICAL, SLOTS)
    _i32(LENS, END, TAKES, SELECTED, MEMBERS, NT, LOGICAL, SLOTS)
    if IDS.dtype not in (torch.int32, torch.int64) or not IDS.is_contiguous():
        raise ValueError("map_topk: IDS must be contiguous int32 or int64")
    if VALUES.dtype != torch.float32 or not VALUES.is_contiguous():
        raise ValueError("map_topk: VALUES must be contiguous float32")
    rows, top = grid[0], int(TOP)
    if rows > 0 and min(IDS.numel(), VALUES.numel(), LOGICAL.numel(), SLOTS.numel()) < rows * top:
        raise ValueError("map_topk: tensors smaller than rows x TOP")
    _lib.call("v1_union_map_topk", _lib.ptr(IDS), 64 if IDS.dtype == torch.int64 else 32, _lib.ptr(VALUES), 0, 0,
              0, _lib.ptr(LENS), _lib.ptr(END), _lib.ptr(TAKES), _lib.ptr(SELECTED), _lib.ptr(MEMBERS),
              MEMBERS.numel() // 64, _lib.ptr(NT), NT.numel(), _lib.ptr(LOGICAL), _lib.ptr(SLOTS), rows, int(MAXTAKE),
              top, int(S), int(W), _lib.stream_of(LOGICAL))


def map_topk_scores(ids, scores, lens, indexed_end, takes, selected, members, nt, logical, slots, max_take, sink,
                    window):
    """map_topk with each id's value read from the canonical scores it was
    selected from (scores[r, id]) instead of a separate values tensor: the
    form a Top-K that returns ids only (topk.topk_transform_512_v2's raw
    indices) hands over without a gather."""
    _lib.require_gpu(ids, scores, lens, indexed_end, takes, selected, members, nt, logical, slots)
    _i32(ids, lens, indexed_end, takes, selected, members, nt, logical, slots)
    if scores.dtype != torch.float32 or scores.dim() != 2 or scores.stride(1) != 1:
        raise ValueError("map_topk_scores: scores must be float32 [rows, cols] with unit inner stride")
    rows, top = ids.shape
    if scores.shape[0] != rows or logical.shape != ids.shape or slots.shape != ids.shape:
        raise ValueError("map_topk_scores: ids, logical, slots [rows, top] and scores [rows, *] must agree")
    _lib.call("v1_union_map_topk", _lib.ptr(ids), 32, 0, _lib.ptr(scores), scores.stride(0), scores.shape[1],
              _lib.ptr(lens), _lib.ptr(indexed_end), _lib.ptr(takes), _lib.ptr(selected), _lib.ptr(members),
              members.numel() // 64, _lib.ptr(nt), nt.numel(), _lib.ptr(logical), _lib.ptr(slots), rows,
              int(max_take), top, int(sink), int(window), _lib.stream_of(logical))


def _stage_tail_shared(grid, NATIVE, NS, NT, LENS, INDEXED_END, K, KS, TAIL_ROWS, CAP, NP, SCRATCH, SINK, WINDOW,
                       ROWS=0, GROUP=1):
    """baseline_published.py:4-61: per-row staging (owner rows of TAIL_ROWS)
    into scratch pages CAP + row * SCRATCH + p, tail from INDEXED_END."""
    _lib.require_gpu(NATIVE, NT, LENS, INDEXED_END, K, TAIL_ROWS)
    _i32(NT, LENS, INDEXED_END, TAIL_ROWS)
    rows = int(ROWS) if int(ROWS) > 0 else grid[0] * int(GROUP)
    _lib.call("v1_stage_tail_published", _lib.ptr(NATIVE), _lib.ptr(NT), _lib.ptr(LENS), _lib.ptr(INDEXED_END),
              _lib.ptr(K), _lib.ptr(TAIL_ROWS), rows, int(CAP), int(NP), int(SCRATCH), int(SINK), int(WINDOW),
              _byte_pages(NATIVE), _byte_pages(K), _lib.stream_of(NT))


tables = _Kernel("tables", _tables)
normalize = _Kernel("normalize", _normalize)
map_topk = _Kernel("map_topk", _map_topk)
stage_tail_shared = _Kernel("stage_tail_shared", _stage_tail_shared)


def union_spans(lens, indexed_end, desc, spans, sink, window):
    """Each row's span in union coordinates (the end of its last candidate):
    the context length for scoring every row against the union pages with one
    shared table (stride-0 page table, see normalize_split)."""
    _lib.require_gpu(lens, indexed_end, desc, spans)
    _i32(lens, indexed_end, desc, spans)
    _lib.call("v1_union_spans", _lib.ptr(lens), _lib.ptr(indexed_end), _lib.ptr(desc), _lib.ptr(spans), lens.numel(),
              int(sink), int(window), _lib.stream_of(spans))
    return spans


def normalize_split(hist, uni, lens, indexed_end, takes, selected, members, desc, out, max_take, width, sink,
                    window):
    """normalize's canonical candidate order from two shared-table scorings:
    hist [rows, >= 64 * history pages] (every row against every history page,
    position page * 64 + slot) and uni [rows, >= span] (every row against the
    union pages in union coordinates).  Same masks and order as normalize."""
    _lib.require_gpu(hist, uni, lens, indexed_end, takes, selected, members, desc, out)
    _i32(lens, indexed_end, takes, selected, members, desc)
    for t in (hist, uni):
        if t.dtype != torch.float32 or t.dim() != 2 or t.stride(1) != 1:
            raise ValueError("normalize_split: score arrays must be float32 [rows, cols] with unit inner stride")
    if out.dtype != torch.float32 or not out.is_contiguous() or out.numel() < lens.numel() * int(width):
        raise ValueError("normalize_split: out must be contiguous float32 [rows, width]")
    rows = lens.numel()
    _lib.call("v1_union_normalize_split", _lib.ptr(hist), hist.stride(0), hist.shape[1], _lib.ptr(uni), uni.stride(0),
              uni.shape[1], _lib.ptr(lens), _lib.ptr(indexed_end), _lib.ptr(takes), _lib.ptr(selected),
              _lib.ptr(members), members.numel() // 64, _lib.ptr(desc), _lib.ptr(out), rows, int(max_take),
              int(width), int(sink), int(window), _lib.stream_of(out))
    return out

