"""Top-K with page-table transform: drop-in for the external
`sglang.kernels.ops.attention.dsv4.topk.topk_transform_512_v2` / `plan_topk_v2`
called at sglang/srt/layers/attention/v1_deepseek/runtime.py:373-376, 427-431,
603-611 (kernel contract: sglang/kernels/jit/csrc/deepseek_v4/topk_v2.cuh:352-460).

    page_indices[b, t] = raw < 0 ? -1 : (page_table[b, raw >> bits] << bits) | (raw & (page_size - 1))

with raw = the t-th selected candidate (ascending candidate index; score
descending, ties toward the lower index), or -1 past min(seq_len, topk).
"""
import ctypes

import torch

from . import _lib
from ._workspace import workspace


def plan_topk_v2(seq_lens, metadata, *_):
    """The reference plans its cluster path here; this implementation sizes
    its work from the lengths, so the plan is an untouched buffer."""
    return metadata


def topk_transform_512_v2(scores, seq_lens, page_table, page_indices, page_size, metadata=None, raw_indices=None):
    _lib.require_gpu(scores, seq_lens, page_table, page_indices, raw_indices)
    if scores.dtype != torch.float32 or scores.dim() != 2 or scores.stride(1) != 1:
        raise RuntimeError("scores must be float32 [batch, cols] with unit inner stride")
    B, L = scores.shape
    if scores.stride(0) % 4:
        raise RuntimeError("score_stride must be a multiple of 4 (16-byte vectorized load)")
    if seq_lens.dtype != torch.int32 or seq_lens.numel() != B:
        raise RuntimeError("seq_lens must be int32 [batch]")
    if page_table.dtype != torch.int32 or page_table.dim() != 2 or page_table.shape[0] != B or page_table.stride(1) != 1:
        raise RuntimeError("page_table must be int32 [batch, *]")
    if page_indices.dtype != torch.int32 or page_indices.dim() != 2 or page_indices.shape[0] != B \
            or not page_indices.is_contiguous():
        raise RuntimeError("page_indices must be contiguous int32 [batch, topk]")
    T = page_indices.shape[1]
    if not 0 < T <= 2048:
        raise RuntimeError("topk must be in (0, 2048]")
    if page_size <= 0 or page_size & (page_size - 1):
        raise RuntimeError("page_size must be power of 2")
    if raw_indices is not None and (tuple(raw_indices.shape) != (B, T) or raw_indices.dtype != torch.int32
                                    or not raw_indices.is_contiguous()):
        raise RuntimeError("raw_indices must be contiguous int32 [batch, topk]")
    ws, ws_bytes = workspace(scores.device, _lib.lib().v1_topk_workspace(B, L, T), "topk")
    a = _lib.TopkTransformArgs(_lib.ptr(scores), scores.stride(0), B, L, _lib.ptr(seq_lens), _lib.ptr(page_table),
                               page_table.stride(0), page_table.shape[1], int(page_size).bit_length() - 1,
                               _lib.ptr(page_indices), _lib.ptr(raw_indices), T, ws, ws_bytes)
    _lib.check(_lib.lib().v1_topk_transform(ctypes.byref(a), _lib.stream_of(scores)), "topk_transform")
    return page_indices
