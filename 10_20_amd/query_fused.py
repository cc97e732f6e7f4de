"""Drop-in for sglang/srt/layers/attention/v1_deepseek/query_fused.py:1-10.

`module()` returns an object with `.route` and `.topk`, positional signatures
identical to V1QueryKernel::route / ::topk
(sglang/kernels/jit/csrc/deepseek_v4/v1_query.cuh:155-158, 181-184), backed by
the gfx950 kernels of libv1idx.  Argument checks mirror the reference's
TensorMatcher / RuntimeCheck rules (v1_query.cuh:160-172, 186-206) and raise
RuntimeError with the same messages before anything is launched.
"""
import ctypes
import functools

import torch

from . import _lib
from ._workspace import workspace


def _need(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _i32(t, shape, name):
    _need(t.dtype == torch.int32, f"{name} must be int32")
    _need(tuple(t.shape) == tuple(shape), f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    _need(t.is_contiguous() or t.numel() == 0, f"{name} must be contiguous")


def _selected(t, B, name="selected"):
    _need(t.dtype in (torch.int32, torch.int64), f"{name} must be int32 or int64")
    _need(t.dim() == 2 and t.shape[0] == B and t.is_contiguous(), f"{name} must be a contiguous [batch, take] tensor")
    return 32 if t.dtype == torch.int32 else 64


def _scores(t):
    _need(t.dtype == torch.float32 and t.dim() == 2, "scores must be a float32 [batch, cols] tensor")
    _need(t.stride(1) == 1, "scores rows must be contiguous")
    return t.shape[0], t.shape[1], t.stride(0)


class V1QueryModule:
    """The fused V1 query operators (route, topk) on MI355X."""

    def route(self, scores, lens, takes, selected, pages, rt, ft, tail_rows, capacity, fill_table):
        _lib.require_gpu(scores, lens, takes, selected, rt, ft, tail_rows)
        B, L, S = _scores(scores)
        _i32(lens, (B,), "lens")
        _i32(takes, (B,), "takes")
        bits = _selected(selected, B)
        K = selected.shape[1]
        _i32(rt, (B, pages), "rt")
        _need(ft.dtype == torch.int32 and ft.dim() == 2 and ft.shape[0] == B and ft.is_contiguous(),
              "ft must be a contiguous int32 [batch, *] tensor")
        _i32(tail_rows, (B,), "tail_rows")
        _need(capacity > 0 and ft.shape[1] >= K, "Invalid fine page table")
        _need(64 <= pages <= 4096 and L >= pages * 8 and K <= pages and S % 4 == 0, "Invalid V1 route capacity")
        a = _lib.RouteArgs(_lib.ptr(scores), S, B, L, _lib.ptr(lens), _lib.ptr(takes), _lib.ptr(selected), bits, K,
                           int(pages), _lib.ptr(rt), _lib.ptr(ft), ft.shape[1], _lib.ptr(tail_rows), int(capacity),
                           int(bool(fill_table)))
        _lib.check(_lib.lib().v1_route(ctypes.byref(a), _lib.stream_of(scores)), "route")

    def topk(self, scores, fine_lens, members, rt, nt, selected, lens, takes, physical, logical, raw, window, mask,
             expanded, physical_output, bucket_from_rank, fine_table, direct_fine):
        self._topk(scores, fine_lens, members, rt, nt, selected, lens, takes, physical, logical, raw, window, mask,
                   expanded, physical_output, bucket_from_rank, fine_table, direct_fine, min_batch=513)

    def _topk(self, scores, fine_lens, members, rt, nt, selected, lens, takes, physical, logical, raw, window, mask,
              expanded, physical_output, bucket_from_rank, fine_table, direct_fine, min_batch):
        _lib.require_gpu(scores, fine_lens, members, rt, nt, selected, lens, takes, physical, logical, raw,
                         expanded, fine_table)
        B, L, S = _scores(scores)
        _i32(fine_lens, (B,), "fine_lens")
        _need(members.dtype == torch.int32 and members.dim() == 2 and members.shape[1] == 64
              and members.is_contiguous(), "members must be a contiguous int32 [*, 64] tensor")
        _need(rt.dim() == 2 and rt.shape[0] == B, "rt must be [batch, pages]")
        P = rt.shape[1]
        _i32(rt, (B, P), "rt")
        _i32(nt, (B, P), "nt")
        bits = _selected(selected, B)
        K = selected.shape[1]
        _i32(lens, (B,), "lens")
        _i32(takes, (B,), "takes")
        _need(physical.dim() == 2, "physical must be [batch, topk]")
        T = physical.shape[1]
        _i32(physical, (B, T), "physical")
        _i32(logical, (B, T), "logical")
        _i32(raw, (B, T), "raw")
        _need(expanded.dtype == torch.int32 and expanded.dim() == 2 and expanded.shape[0] == B,
              "expanded must be an int32 [batch, *] tensor")
        _need(fine_table.dtype == torch.int32 and fine_table.dim() == 2 and fine_table.shape[0] == B
              and fine_table.is_contiguous(), "fine_table must be a contiguous int32 [batch, *] tensor")
        _need(not direct_fine or fine_table.shape[1] >= K, "Invalid direct fine table")
        es = expanded.shape[1]
        _need(es == 0 or es == T * 4 + 64, "Invalid expansion buffer")
        _need(es == 0 or expanded.is_contiguous(), "expanded must be contiguous")
        _need(B >= min_batch and 0 < T <= 2048 and 0 <= window <= 4096, "Unsupported fused V1 TopK")
        ws, ws_bytes = workspace(scores.device, _lib.lib().v1_topk_workspace(B, L, T), "topk")
        a = _lib.TopkArgs(
            _lib.ptr(scores), S, B, L, _lib.ptr(fine_lens), _lib.ptr(members), members.shape[0], _lib.ptr(rt),
            _lib.ptr(nt), P, _lib.ptr(selected), bits, K, _lib.ptr(lens), _lib.ptr(takes), _lib.ptr(physical),
            _lib.ptr(logical), _lib.ptr(raw), T, int(window), int(bool(mask)), _lib.ptr(expanded) if es else 0, es,
            int(bool(physical_output)), int(bool(bucket_from_rank)), _lib.ptr(fine_table), fine_table.shape[1],
            int(bool(direct_fine)), ws, ws_bytes)
        _lib.check(_lib.lib().v1_topk(ctypes.byref(a), _lib.stream_of(scores)), "topk")


def topk_any_batch(scores, fine_lens, members, rt, nt, selected, lens, takes, physical, logical, raw, window, mask,
                   expanded, physical_output, bucket_from_rank, fine_table, direct_fine):
    """module().topk for batches of any size.  The reference's fused kernel
    takes more than 512 rows (v1_query.cuh:203) and smaller batches run
    mask_fine -> topk_transform_512_v2 -> output_ids (runtime.py:549-634).
    With mask on, members-derived buckets (bucket_from_rank off), fine_lens
    equal to each row's candidate count, selected ranks inside rt and each
    fine page's members inside one 1024-token bucket (as the index build
    makes them), this call gives that chain's raw / logical / physical
    outputs, in one launch pair (segments, merge) instead of three kernels
    and a masked-score round trip."""
    module()._topk(scores, fine_lens, members, rt, nt, selected, lens, takes, physical, logical, raw, window, mask,
                   expanded, physical_output, bucket_from_rank, fine_table, direct_fine, min_batch=1)


@functools.lru_cache(maxsize=None)
def module():
    """Same role as the reference's load_jit module: loads the library once."""
    _lib.lib()
    return V1QueryModule()
