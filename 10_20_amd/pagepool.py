"""Batched page manager over a device page pool.

`PagePool` holds the state the reference keeps per index
(sglang/srt/layers/attention/v1_deepseek/runtime.py:771-825): page bytes,
one int64 key per page (the reference's (h0, h1) fingerprint,
kernels.py:57-69), reference counts, the free stack and its count.
`insert` runs match_pages -> allocate -> publish (kernels.py:72-167) for a
whole batch of requests with the result of calling them request after request;
`release` is kernels.py:170-179 over a list of pages.  Both are a fixed
sequence of launches on the current stream with no host synchronisation;
`status()` reads the failure bits (a failed batch changes nothing).
"""
import torch

from . import _lib
from ._workspace import workspace

STATUS_EXHAUSTED = 1
STATUS_COLLISIONS = 2
STATUS_BAD_ORDER = 4
STATUS_UNDERFLOW = 8
STATUS_BAD_STATE = 16


def _check_i32(name, t, n=None):
    if t.dtype != torch.int32 or not t.is_contiguous() or (n is not None and t.numel() != n):
        raise ValueError(f"{name} must be a contiguous int32 tensor" + (f" of {n} elements" if n else ""))


class PagePool:
    """`capacity` managed pages, followed in the same byte pool by
    `scratch_pages` pages that the manager never hands out (the tail scratch
    region that stage_tail writes from page `capacity` on)."""

    def __init__(self, capacity, page_bytes, device="cuda", scratch_pages=0):
        if capacity <= 0 or page_bytes <= 0 or page_bytes % 16 or scratch_pages < 0:
            raise ValueError("capacity must be positive and page_bytes a positive multiple of 16")
        device = torch.device(device)
        self.capacity = int(capacity)
        self.page_bytes = int(page_bytes)
        self.pages = torch.zeros(self.capacity + int(scratch_pages), self.page_bytes, dtype=torch.uint8,
                                 device=device)
        self.pool = self.pages[:self.capacity]
        self.keys = torch.zeros(self.capacity, dtype=torch.int64, device=device)
        self.refs = torch.zeros(self.capacity, dtype=torch.int32, device=device)
        self.free = torch.arange(self.capacity, dtype=torch.int32, device=device)
        self.count = torch.full((1,), self.capacity, dtype=torch.int32, device=device)
        self.status_word = torch.zeros(1, dtype=torch.int32, device=device)

    @property
    def device(self):
        return self.pool.device

    def reset(self):
        """Every page free (free stack 0..capacity-1, page 0 popped last), no
        references; page bytes and keys are left as they are."""
        self.refs.zero_()
        torch.arange(self.capacity, dtype=torch.int32, device=self.device, out=self.free)
        self.count.fill_(self.capacity)

    def status(self, clear=True):
        """Failure bits OR-ed by the calls since the last clear (reads the device)."""
        v = int(self.status_word.item())
        if clear:
            self.status_word.zero_()
        return v

    def raise_on_status(self):
        v = self.status()
        if v & STATUS_EXHAUSTED:
            raise RuntimeError("V1 DeepSeek page arena exhausted")
        if v & STATUS_UNDERFLOW:
            raise RuntimeError("page release underflow: a released page had no reference")
        if v & STATUS_BAD_STATE:
            raise RuntimeError("page pool state is inconsistent (count or free stack out of range)")
        if v & STATUS_COLLISIONS:
            raise RuntimeError("page insert: too many key collisions in one batch")
        if v & STATUS_BAD_ORDER:
            raise ValueError("page insert: request ids must be non-decreasing")

    def insert(self, keys, tmp, req, table=None):
        """keys int64 [n], tmp uint8 [n, page_bytes], req int32 [n] (request of
        each entry, non-decreasing).  Returns int32 [n] pages (table)."""
        n = keys.numel()
        _lib.require_gpu(keys, tmp, req, self.pool)
        if keys.dtype != torch.int64 or not keys.is_contiguous():
            raise ValueError("keys must be a contiguous int64 tensor")
        if tmp.dtype != torch.uint8 or tmp.shape != (n, self.page_bytes) or not tmp.is_contiguous():
            raise ValueError(f"tmp must be a contiguous uint8 [{n}, {self.page_bytes}] tensor")
        _check_i32("req", req, n)
        if table is None:
            table = torch.empty(n, dtype=torch.int32, device=self.device)
        _check_i32("table", table, n)
        nbytes = _lib.lib().v1_page_insert_workspace(self.capacity, n)
        wp, wn = workspace(self.device, nbytes, "page_insert")
        _lib.call("v1_page_insert", _lib.ptr(self.pool), _lib.ptr(self.keys), _lib.ptr(self.refs),
                  _lib.ptr(self.free), _lib.ptr(self.count), self.capacity, self.page_bytes, _lib.ptr(keys),
                  _lib.ptr(tmp), _lib.ptr(req), n, _lib.ptr(table), _lib.ptr(self.status_word), wp, wn,
                  _lib.stream_of(self.pool))
        return table

    def release(self, pages):
        """Decrements in list order; pages reaching 0 go on the free stack."""
        _lib.require_gpu(pages, self.pool)
        _check_i32("pages", pages)
        n = pages.numel()
        nbytes = _lib.lib().v1_page_release_workspace(self.capacity, n)
        wp, wn = workspace(self.device, nbytes, "page_release")
        _lib.call("v1_page_release", _lib.ptr(pages), n, _lib.ptr(self.refs), _lib.ptr(self.free),
                  _lib.ptr(self.count), self.capacity, _lib.ptr(self.status_word), wp, wn,
                  _lib.stream_of(self.pool))


def requests_of(lengths, device):
    """int32 request id of every entry, for per-request page counts."""
    lengths = torch.as_tensor(lengths, dtype=torch.int64)
    return torch.repeat_interleave(torch.arange(lengths.numel(), dtype=torch.int32), lengths).to(device)


def sort_pairs_u64(keys, vals):
    """Stable ascending sort of (uint64 bits of int64 keys, int32 values)."""
    _lib.require_gpu(keys, vals)
    n = keys.numel()
    ko = torch.empty_like(keys)
    vo = torch.empty_like(vals)
    nbytes = _lib.lib().v1_sort_pairs_u64_workspace(n)
    wp, wn = workspace(keys.device, nbytes, "sort_pairs")
    _lib.call("v1_sort_pairs_u64", _lib.ptr(keys), _lib.ptr(vals), _lib.ptr(ko), _lib.ptr(vo), n, 64, wp, wn,
              _lib.stream_of(keys))
    return ko, vo


def stage_tail_rows(native, nt, lens, fine, tail_rows, capacity, scratch, sink=64, window=64):
    """stage_tail_shared (kernels.py:518-564; tail_rows None: stage_tail
    :407-441) over uint8 pools [pages, 64 * row_bytes] of row pages: owner row r
    copies its sink and tail tokens to pages capacity + r * scratch + p."""
    _lib.require_gpu(native, nt, lens, fine, tail_rows)
    if native.dtype != torch.uint8 or fine.dtype != torch.uint8 or native.dim() != 2 or fine.dim() != 2:
        raise ValueError("native and fine must be uint8 [pages, 64 * row_bytes] tensors")
    if native.shape[1] != fine.shape[1] or native.shape[1] % (64 * 16):
        raise ValueError("pages must hold 64 rows of a multiple of 16 bytes, equal in both pools")
    if not (native.is_contiguous() and fine.is_contiguous()):
        raise ValueError("native and fine must be contiguous")
    _check_i32("nt", nt)
    _check_i32("lens", lens, nt.shape[0])
    if tail_rows is not None:
        _check_i32("tail_rows", tail_rows, nt.shape[0])
    _lib.call("v1_stage_tail_rows", _lib.ptr(native), _lib.ptr(nt), _lib.ptr(lens), _lib.ptr(fine),
              _lib.ptr(tail_rows), nt.shape[0], int(capacity), nt.shape[1], int(scratch), int(sink), int(window),
              native.shape[0], fine.shape[0], native.shape[1] // 64, _lib.stream_of(native))
