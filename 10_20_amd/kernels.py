"""Drop-in kernel objects for sglang/srt/layers/attention/v1_deepseek/kernels.py.

Each object keeps the reference's launch protocol `kernel[grid](*args, **kw)`
and argument order (the reference itself swaps Triton kernels for objects with
`__getitem__(grid) -> launch`, bench_v1_dynamic_budget_metadata.py:30-34).
`num_warps`, `debug` and other Triton launch options are accepted and
ignored.  Tensors passed as fp8 / fp32 views of one byte pool are used by
their data pointer, exactly like the Triton kernels address them.
"""
import ctypes

import torch

from . import _lib
from ._workspace import workspace

PAGE_BYTES = 8448
_TRITON_OPTIONS = {"num_warps", "num_stages", "debug", "enable_fp_fusion", "num_ctas"}


class _Kernel:
    def __init__(self, name, launch):
        self.__name__ = name
        self._launch = launch

    def __getitem__(self, grid):
        if callable(grid):
            raise TypeError(f"{self.__name__}: grid must be a tuple of ints")
        grid = tuple(int(g) for g in (grid if isinstance(grid, (tuple, list)) else (grid,)))

        def run(*args, **kwargs):
            extra = {k: v for k, v in kwargs.items() if k not in _TRITON_OPTIONS}
            return self._launch(grid, *args, **extra)

        return run

    def __repr__(self):
        return f"<libv1idx kernel {self.__name__}>"


def _stream(t):
    return _lib.stream_of(t)


def _sel_bits(t):
    if t.dtype == torch.int32:
        return 32
    if t.dtype == torch.int64:
        return 64
    raise ValueError("SELECTED must be int32 or int64")


def _page_bytes(tmp):
    """Bytes per page of a [pages, page_bytes] byte tensor (8448 in the reference)."""
    return tmp.stride(0) * tmp.element_size()


# -------------------------------------------------------------- page manager
def _fingerprint(grid, TMP, MAP, META, HASH):
    _lib.require_gpu(TMP, MAP, META, HASH)
    _lib.call("v1_fingerprint", _lib.ptr(TMP), _lib.ptr(MAP), _lib.ptr(META), _lib.ptr(HASH), grid[0],
              _page_bytes(TMP), _stream(TMP))


def _match_pages(grid, TMP, MAP, HASH, META, FINE, MEMBERS, HASHES, REFS, MATCH, CAP, SCAN=None):
    _lib.require_gpu(TMP, MAP, HASH, META, FINE, MEMBERS, HASHES, REFS, MATCH)
    _lib.call("v1_match_pages", _lib.ptr(TMP), _lib.ptr(MAP), _lib.ptr(HASH), _lib.ptr(META), _lib.ptr(FINE),
              _lib.ptr(MEMBERS), _lib.ptr(HASHES), _lib.ptr(REFS), _lib.ptr(MATCH), grid[0], int(CAP),
              _page_bytes(TMP), _stream(TMP))


_ALLOC_STATUS = {}


def allocation_status(device):
    """int32 device word whose bit 0 is set when an allocate found the free
    stack exhausted (the reference's device_assert, kernels.py:125)."""
    key = torch.device(device)
    if key not in _ALLOC_STATUS:
        _ALLOC_STATUS[key] = torch.zeros(1, dtype=torch.int32, device=key)
    return _ALLOC_STATUS[key]


def _allocate(grid, META, MATCH, FREE, COUNT, REFS, TABLES, NEW):
    _lib.require_gpu(META, MATCH, FREE, COUNT, REFS, TABLES, NEW)
    pages = MATCH.numel()
    _lib.call("v1_allocate", _lib.ptr(META), _lib.ptr(MATCH), _lib.ptr(FREE), _lib.ptr(COUNT), _lib.ptr(REFS),
              _lib.ptr(TABLES), _lib.ptr(NEW), pages, _lib.ptr(allocation_status(META.device)), _stream(META))


def _publish(grid, TMP, TC, TCS, MAP, HASH, META, TABLES, NEW, FINE, CENTERS, CS, MEMBERS, HASHES):
    _lib.require_gpu(TMP, TC, MAP, HASH, META, TABLES, NEW, FINE, CENTERS, MEMBERS, HASHES)
    _lib.call("v1_publish", _lib.ptr(TMP), _lib.ptr(TC), _lib.ptr(MAP), _lib.ptr(HASH), _lib.ptr(META),
              _lib.ptr(TABLES), _lib.ptr(NEW), _lib.ptr(FINE), _lib.ptr(CENTERS), _lib.ptr(MEMBERS),
              _lib.ptr(HASHES), grid[0], _page_bytes(TMP), _stream(TMP))


def _release(grid, TABLE, REFS, FREE, COUNT):
    _lib.require_gpu(TABLE, REFS, FREE, COUNT)
    _lib.call("v1_release", _lib.ptr(TABLE), _lib.ptr(REFS), _lib.ptr(FREE), _lib.ptr(COUNT), 16, _stream(TABLE))


# -------------------------------------------------------------- index build
def _initialize(grid, K, KS, TABLE, META, UNIT, PERM, FLAG):
    """kernels.py:9-30: 16 tokens per program; FLAG = -1 when META[2] else 0."""
    _lib.require_gpu(K, KS, TABLE, META, UNIT, PERM, FLAG)
    if UNIT.dtype != torch.float32 or PERM.dtype != torch.int32:
        raise ValueError("initialize: UNIT must be float32 and PERM int32")
    _lib.call("v1_build_initialize", _lib.ptr(K), _lib.ptr(KS), _lib.ptr(TABLE), _lib.ptr(META), _lib.ptr(UNIT),
              _lib.ptr(PERM), _lib.ptr(FLAG), grid[0], _stream(UNIT))


def _assemble(grid, K, KS, TABLE, META, IDS, TMP, TMPS, CENTERS, CS, MAP):
    """kernels.py:33-54: program (page, g) copies members g*8..g*8+7 of page
    and writes their FP8 center."""
    _lib.require_gpu(K, KS, TABLE, META, IDS, TMP, TMPS, CENTERS, CS, MAP)
    _lib.call("v1_build_assemble", _lib.ptr(K), _lib.ptr(KS), _lib.ptr(TABLE), _lib.ptr(META), _lib.ptr(IDS),
              _lib.ptr(TMP), _lib.ptr(TMPS), _lib.ptr(CENTERS), _lib.ptr(CS), _lib.ptr(MAP), grid[0],
              grid[1] if len(grid) > 1 else 1, _stream(TMP))


initialize = _Kernel("initialize", _initialize)
assemble = _Kernel("assemble", _assemble)
fingerprint = _Kernel("fingerprint", _fingerprint)
match_pages = _Kernel("match_pages", _match_pages)
allocate = _Kernel("allocate", _allocate)
publish = _Kernel("publish", _publish)
release = _Kernel("release", _release)


# ---------------------------------------------------- metadata and tables
def _query_metadata(grid, LENS, NT, FLENS, TAKES, DG_LENS, CENTER_LENS, TAIL_ROWS, NP, TOPK, NUM, DEN, SINK,
                    WINDOW):
    _lib.require_gpu(LENS, NT, FLENS, TAKES, DG_LENS, CENTER_LENS, TAIL_ROWS)
    _lib.call("v1_query_metadata", _lib.ptr(LENS), _lib.ptr(NT), _lib.ptr(FLENS), _lib.ptr(TAKES),
              _lib.ptr(DG_LENS), _lib.ptr(CENTER_LENS), _lib.ptr(TAIL_ROWS), grid[0], int(NP), int(TOPK), int(NUM),
              int(DEN), int(SINK), int(WINDOW), _stream(LENS))


def _query_lengths(grid, LENS, FLENS, TAKES, MAXTAKE, TOPK, NUM, DEN, SINK, WINDOW):
    _lib.require_gpu(LENS, FLENS, TAKES)
    _lib.call("v1_query_lengths", _lib.ptr(LENS), _lib.ptr(FLENS), _lib.ptr(TAKES), grid[0], int(TOPK), int(NUM),
              int(DEN), int(SINK), int(WINDOW), _stream(LENS))


def _fine_table(grid, RT, SELECTED, TAKES, LENS, FT, CAP, MAXP, TAKE, FP, SCRATCH, B):
    _lib.require_gpu(RT, SELECTED, TAKES, LENS, FT)
    _lib.call("v1_fine_table", _lib.ptr(RT), _lib.ptr(SELECTED), _sel_bits(SELECTED), _lib.ptr(TAKES),
              _lib.ptr(FT), 0, grid[0], int(CAP), int(MAXP), int(TAKE), int(FP), int(SCRATCH), _stream(RT))


def _fine_table_shared(grid, RT, SELECTED, TAKES, LENS, FT, TAIL_ROWS, CAP, MAXP, TAKE, FP, SCRATCH, B):
    _lib.require_gpu(RT, SELECTED, TAKES, LENS, FT, TAIL_ROWS)
    _lib.call("v1_fine_table", _lib.ptr(RT), _lib.ptr(SELECTED), _sel_bits(SELECTED), _lib.ptr(TAKES),
              _lib.ptr(FT), _lib.ptr(TAIL_ROWS), grid[0], int(CAP), int(MAXP), int(TAKE), int(FP), int(SCRATCH),
              _stream(RT))


def _pool_pages(t):
    return t.numel() * t.element_size() // 8448


def _stage_tail(grid, NATIVE, NS, NT, LENS, K, KS, CAP, NP, SCRATCH, SINK, WINDOW):
    _lib.require_gpu(NATIVE, NT, LENS, K)
    _lib.call("v1_stage_tail", _lib.ptr(NATIVE), _lib.ptr(NT), _lib.ptr(LENS), _lib.ptr(K), 0, grid[0], int(CAP),
              int(NP), int(SCRATCH), int(SINK), int(WINDOW), _pool_pages(NATIVE), _pool_pages(K), _stream(NT))


def _stage_tail_shared(grid, NATIVE, NS, NT, LENS, K, KS, TAIL_ROWS, CAP, NP, SCRATCH, SINK, WINDOW, ROWS=0,
                       GROUP=1):
    _lib.require_gpu(NATIVE, NT, LENS, K, TAIL_ROWS)
    rows = int(ROWS) if int(ROWS) > 0 else grid[0] * int(GROUP)
    _lib.call("v1_stage_tail", _lib.ptr(NATIVE), _lib.ptr(NT), _lib.ptr(LENS), _lib.ptr(K), _lib.ptr(TAIL_ROWS),
              rows, int(CAP), int(NP), int(SCRATCH), int(SINK), int(WINDOW), _pool_pages(NATIVE), _pool_pages(K),
              _stream(NT))


query_metadata = _Kernel("query_metadata", _query_metadata)
query_lengths = _Kernel("query_lengths", _query_lengths)
fine_table = _Kernel("fine_table", _fine_table)
fine_table_shared = _Kernel("fine_table_shared", _fine_table_shared)
stage_tail = _Kernel("stage_tail", _stage_tail)
stage_tail_shared = _Kernel("stage_tail_shared", _stage_tail_shared)


# ------------------------------------------------------- unfused mask / map
def _mask_fine(grid, SCORES, SELECTED, RT, MEMBERS, LENS, TAKES, MAXP, TAKE, STRIDE, WIDTH, SINK, WINDOW):
    _lib.require_gpu(SCORES, SELECTED, RT, MEMBERS, LENS, TAKES)
    _lib.call("v1_mask_fine", _lib.ptr(SCORES), int(STRIDE), _lib.ptr(SELECTED), _sel_bits(SELECTED), _lib.ptr(RT),
              _lib.ptr(MEMBERS), _lib.ptr(LENS), _lib.ptr(TAKES), grid[0], int(MAXP), int(TAKE), int(WIDTH),
              int(SINK), int(WINDOW), _stream(SCORES))


def _output_ids(grid, RAW, SCORES, MEMBERS, RT, NT, SELECTED, LENS, TAKES, OUT, LOGICAL, FT, MAXP, NP, TAKE, WIDTH,
                TOPK, SINK, WINDOW, MAP_PHYSICAL=True, DIRECT_FINE=False, FP=0):
    _lib.require_gpu(RAW, SCORES, MEMBERS, RT, NT, SELECTED, LENS, TAKES, OUT, LOGICAL, FT)
    _lib.call("v1_output_ids", _lib.ptr(RAW), _lib.ptr(SCORES), int(WIDTH), _lib.ptr(MEMBERS), _lib.ptr(RT),
              _lib.ptr(NT), _lib.ptr(SELECTED), _sel_bits(SELECTED), _lib.ptr(LENS), _lib.ptr(TAKES), _lib.ptr(OUT),
              _lib.ptr(LOGICAL), _lib.ptr(FT), grid[0], int(MAXP), int(NP), int(TAKE), int(WIDTH), int(TOPK),
              int(SINK), int(WINDOW), int(bool(MAP_PHYSICAL)), int(bool(DIRECT_FINE)), int(FP), _stream(SCORES))


def _expand_logical(grid, LOGICAL, OUT, TOPK, STRIDE, BLOCK):
    """kernels.py:594-600: program r writes columns j < min(STRIDE, BLOCK) of
    OUT row r (rows STRIDE ints apart) from LOGICAL row r (TOPK ints)."""
    _lib.require_gpu(LOGICAL, OUT)
    if LOGICAL.dtype != torch.int32 or OUT.dtype != torch.int32:
        raise ValueError("expand_logical: LOGICAL and OUT must be int32")
    rows, topk, stride = grid[0], int(TOPK), int(STRIDE)
    if rows > 0 and (LOGICAL.numel() < rows * topk or OUT.numel() < (rows - 1) * stride + min(stride, int(BLOCK))):
        raise ValueError("expand_logical: tensors smaller than the grid addresses")
    _lib.call("v1_expand_logical", _lib.ptr(LOGICAL), _lib.ptr(OUT), rows, topk, stride, min(stride, int(BLOCK)),
              _stream(OUT))


# --------------------------------------------- scoring without DeepGEMM
def _pool(view, scales, name):
    """Byte pointer and page count of a pool passed as its FP8 view and its
    fp32 view (the same storage, kernels.py:205-207)."""
    if view.data_ptr() != scales.data_ptr():
        raise ValueError(f"{name}: the FP8 and fp32 views must be the same pool")
    if not view.is_contiguous() or (view.numel() * view.element_size()) % PAGE_BYTES:
        raise ValueError(f"{name}: the pool must be contiguous whole 8448-byte pages")
    return _lib.ptr(view), view.numel() * view.element_size() // PAGE_BYTES


def _holds(t, dtype, count, name):
    """t is a contiguous `dtype` tensor of at least `count` elements (the
    kernels address these buffers by row strides of their own)."""
    if t.dtype != dtype or not t.is_contiguous() or t.numel() < count:
        raise ValueError(f"{name} must be a contiguous {dtype} tensor of at least {count} elements")


def _reduce_centers(grid, LOGITS, LENS, SCORES, MAXP, STRIDE):
    """kernels.py:475-486: SCORES[r, p] = max of LOGITS[r, 8p..8p+7] for pages
    below max(n-1, 0) // 1024 * 16, else -inf."""
    _lib.require_gpu(LOGITS, LENS, SCORES)
    rows, maxp = grid[0], int(MAXP)
    if LOGITS.dtype != torch.float32 or LOGITS.stride(-1) != 1 or (rows > 0 and LOGITS.numel() < (rows - 1) * int(STRIDE)
                                                                    + 8 * maxp):
        raise ValueError("reduce_centers: LOGITS must be float32 rows of STRIDE elements holding 8 * MAXP logits")
    _holds(LENS, torch.int32, rows, "reduce_centers: LENS")
    _holds(SCORES, torch.float32, rows * maxp, "reduce_centers: SCORES")
    _lib.call("v1_reduce_centers", _lib.ptr(LOGITS), int(STRIDE), _lib.ptr(LENS), _lib.ptr(SCORES), grid[0],
              int(MAXP), _stream(SCORES))


def _coarse(grid, Q, W, C, CS, TABLE, LENS, SCORES, MAXP, H, RELU):
    """kernels.py:182-221 (called at runtime.py:453-466): page scores as the
    max of their 8 center logits, through the FP8 scoring kernel."""
    _lib.require_gpu(Q, W, C, LENS, SCORES, TABLE)
    rows = grid[0]
    centers, blocks = _pool(C, CS, "coarse")
    if TABLE.dtype != torch.int32 or TABLE.dim() != 2 or TABLE.stride(1) != 1:
        raise ValueError("coarse: TABLE must be an int32 [rows, MAXP // 8] table")
    if Q.element_size() != 1 or not Q.is_contiguous() or Q.numel() != rows * int(H) * 128:
        raise ValueError("coarse: Q must be a contiguous FP8 [rows, H, 128] tensor")
    if TABLE.shape[0] < rows or TABLE.shape[1] < int(MAXP) // 8:
        raise ValueError("coarse: TABLE must hold MAXP // 8 center pages per row")
    _holds(W, torch.float32, rows * int(H), "coarse: W")
    _holds(LENS, torch.int32, rows, "coarse: LENS")
    _holds(SCORES, torch.float32, rows * int(MAXP), "coarse: SCORES")
    need = _lib.lib().v1_coarse_workspace(rows, int(MAXP), TABLE.stride(0))
    ws, ws_bytes = workspace(Q.device, need, "coarse")
    a = _lib.CoarseArgs(_lib.ptr(Q), _lib.ptr(W), centers, blocks, _lib.ptr(TABLE), TABLE.stride(0), _lib.ptr(LENS),
                        _lib.ptr(SCORES), rows, int(H), int(MAXP), int(bool(RELU)), ws, ws_bytes)
    _lib.check(_lib.lib().v1_coarse(ctypes.byref(a), _stream(SCORES)), "coarse")


def _fine(grid, Q, W, K, KS, NATIVE, NS, MEMBERS, RT, NT, SELECTED, LENS, TAKES, SCORES, MAXP, NP, TAKE, WIDTH, SINK,
          WINDOW, H, RELU):
    """kernels.py:248-320 (called at runtime.py:565-590): fine candidates
    scored straight from the fine and native pools."""
    _lib.require_gpu(Q, W, K, NATIVE, MEMBERS, RT, NT, SELECTED, LENS, TAKES, SCORES)
    rows = grid[0]
    fine, fine_blocks = _pool(K, KS, "fine")
    native, native_blocks = _pool(NATIVE, NS, "fine")
    if MEMBERS.dtype != torch.int32 or not MEMBERS.is_contiguous() or MEMBERS.numel() % 64:
        raise ValueError("fine: MEMBERS must be a contiguous int32 [pages, 64] tensor")
    fine_blocks = min(fine_blocks, MEMBERS.numel() // 64)  # pages with a member row
    if Q.element_size() != 1 or not Q.is_contiguous() or Q.numel() != rows * int(H) * 128:
        raise ValueError("fine: Q must be a contiguous FP8 [rows, H, 128] tensor")
    _holds(W, torch.float32, rows * int(H), "fine: W")
    _holds(RT, torch.int32, rows * int(MAXP), "fine: RT")
    _holds(NT, torch.int32, rows * int(NP), "fine: NT")
    _holds(SELECTED, SELECTED.dtype, rows * int(TAKE), "fine: SELECTED")
    _holds(LENS, torch.int32, rows, "fine: LENS")
    _holds(TAKES, torch.int32, rows, "fine: TAKES")
    _holds(SCORES, torch.float32, rows * int(WIDTH), "fine: SCORES")
    a = _lib.FineArgs(_lib.ptr(Q), _lib.ptr(W), fine, fine_blocks, native, native_blocks, _lib.ptr(MEMBERS),
                      _lib.ptr(RT), _lib.ptr(NT), _lib.ptr(SELECTED), _sel_bits(SELECTED), _lib.ptr(LENS),
                      _lib.ptr(TAKES), _lib.ptr(SCORES), rows, int(H), int(MAXP), int(NP), int(TAKE), int(WIDTH),
                      int(SINK), int(WINDOW), int(bool(RELU)))
    _lib.check(_lib.lib().v1_fine(ctypes.byref(a), _stream(SCORES)), "fine")


reduce_centers = _Kernel("reduce_centers", _reduce_centers)
coarse = _Kernel("coarse", _coarse)
fine = _Kernel("fine", _fine)
mask_fine = _Kernel("mask_fine", _mask_fine)
output_ids = _Kernel("output_ids", _output_ids)
expand_logical = _Kernel("expand_logical", _expand_logical)
