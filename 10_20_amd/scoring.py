"""FP8 paged MQA index logits (the DeepGEMM `fp8_paged_mqa_logits` contract
used at sglang/srt/layers/attention/v1_deepseek/runtime.py:422-444, 538-548 and
experiments/fine_pool_shared_20261021/experiment.py:82-83):

    logits[r, j] = sum_h w[r, h] * ReLU(q[r, h] . k[j]) * s_k[j],  j < context_lens[r]

k / s_k come from 8448-byte native pages ([64, 1, 132] byte view: 64x128 FP8
then 64 fp32 scales) through block_table[r, j // 64].  A block table with row
stride 0 (e.g. `table[None].expand(rows, -1)`) marks rows that share one
table; they are tiled together so each key page is staged once per 8 rows.
Per-row tables of more than 512 rows (a prefill chunk's fine tables) over a
pool small enough for a dense (row, pool page) table are scored page-major:
each work-group stages 8 pool pages once for every row of a 64-row block that
lists them.  Over larger pools, rows with more than 16 heads are planned per
8-row group over the union of their pages, staged the same way.
"""
import ctypes

import torch

from . import _lib
from ._workspace import workspace

PAGE_BYTES = 8448


def _as_bytes(t):
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


def fp8_paged_mqa_logits(q, kv_cache, weights, context_lens, block_table, schedule_meta=None, max_context_len=None,
                         clean_logits=True, relu=True, out=None):
    """q [rows, H, 128] (or [batch, 1, H, 128]) e4m3fn; kv_cache native pages;
    weights [rows, H] fp32; context_lens [rows] or [rows, 1] int32;
    block_table [rows, blocks] int32.  Returns logits [rows, max_context_len]."""
    _lib.require_gpu(q, kv_cache, weights, context_lens, block_table, out)
    if q.dim() == 4:
        if q.shape[1] != 1:
            raise ValueError("fp8_paged_mqa_logits: next_n must be 1")
        q = q[:, 0]
    if q.dim() != 3 or q.shape[2] != 128 or q.element_size() != 1 or not q.is_contiguous():
        raise ValueError("q must be a contiguous [rows, heads, 128] FP8 tensor")
    rows, heads = q.shape[0], q.shape[1]
    if weights.dtype != torch.float32 or tuple(weights.shape) != (rows, heads) or not weights.is_contiguous():
        raise ValueError("weights must be a contiguous float32 [rows, heads] tensor")
    lens = context_lens.reshape(-1)
    if lens.dtype != torch.int32 or lens.numel() != rows or not lens.is_contiguous():
        raise ValueError("context_lens must hold one int32 length per row")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != rows \
            or block_table.stride(1) != 1:
        raise ValueError("block_table must be an int32 [rows, blocks] tensor with unit inner stride")
    kv = _as_bytes(kv_cache)
    if not kv.is_contiguous() or kv.numel() % PAGE_BYTES:
        raise ValueError("kv_cache must be contiguous whole 8448-byte pages")
    if max_context_len is None:
        max_context_len = block_table.shape[1] * 64
    if out is None:
        out = torch.empty((rows, max_context_len), dtype=torch.float32, device=q.device)
    elif out.dtype != torch.float32 or out.shape[0] != rows or out.shape[1] < max_context_len or out.stride(1) != 1:
        raise ValueError("out must be float32 [rows, >= max_context_len]")
    # shared tables need the workspace; per-row tables of large batches use
    # it for the page-major pair table over a small pool, else for the
    # page-union plan (0 bytes: each row on its own)
    kv_blocks = kv.numel() // PAGE_BYTES
    if block_table.stride(0) == 0:
        need = _lib.lib().v1_score_workspace(rows, int(max_context_len))
    else:
        need = max(_lib.lib().v1_score_pages_workspace(rows, int(max_context_len), kv_blocks),
                   _lib.lib().v1_score_tables_workspace(rows, int(max_context_len)))
    ws, ws_bytes = workspace(q.device, need, "score")
    a = _lib.ScoreArgs(_lib.ptr(q), _lib.ptr(kv), kv_blocks, _lib.ptr(weights), _lib.ptr(lens),
                       _lib.ptr(block_table), block_table.stride(0), block_table.shape[1], _lib.ptr(out), out.stride(0),
                       int(max_context_len), rows, heads, int(bool(relu)), int(bool(clean_logits)), ws, ws_bytes)
    _lib.check(_lib.lib().v1_score(ctypes.byref(a), _lib.stream_of(q)), "fp8_paged_mqa_logits")
    return out


def page_major(enable):
    """Allow (True, the default) or forbid the page-major form for per-row
    tables of large batches over a small pool; returns the previous setting.
    A switch for tests and measurements."""
    prev = ctypes.c_int32(0)
    _lib.check(_lib.lib().v1_score_page_major(int(bool(enable)), ctypes.byref(prev)), "score_page_major")
    return bool(prev.value)


def get_paged_mqa_logits_metadata(context_lens, block_size, num_sms):
    """Schedule placeholder with DeepGEMM's [num_sms + 1, 2] int32 shape: these
    kernels size their grid from the lengths themselves."""
    if block_size != 64:
        raise ValueError("block_size must be 64")
    return torch.zeros((num_sms + 1, 2), dtype=torch.int32, device=context_lens.device)
