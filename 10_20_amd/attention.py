"""Decode attention over the gathered workspace: the consumer after the slot
gather.  sglang/srt/layers/attention/v1_native/backend.py:306-315 calls
flash_attn_with_kvcache(q[:, None], kg, vg, causal=False,
softmax_scale=layer.scaling) with q [rows, 1, 4, 128] and kg / vg
[rows, 2048, 1, 128] from GatherWorkspace.gather; flash_attn_with_kvcache here
keeps that call shape for one query position per row (bf16, head dim 128, at
most 4 query heads per KV head).  With one query position, causal masking
changes nothing, so `causal` is accepted either way.  Rows attend their first
cache_seqlens[b] keys (all keys when it is None); a row without keys gives
zeros.
"""
import math

import torch

from . import _lib


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, rotary_cos=None, rotary_sin=None,
                            cache_seqlens=None, cache_batch_idx=None, cache_leftpad=None, block_table=None,
                            softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                            rotary_interleaved=True, alibi_slopes=None, num_splits=0, return_softmax_lse=False,
                            out=None):
    """FA3's keyword interface; `num_splits` only tunes FA3's launch and is
    ignored, `rotary_interleaved` has no effect without rotary tables; the
    options that change the result and are not implemented here raise."""
    unsupported = {"k": k, "v": v, "rotary_cos": rotary_cos, "rotary_sin": rotary_sin,
                   "cache_batch_idx": cache_batch_idx, "cache_leftpad": cache_leftpad, "block_table": block_table,
                   "alibi_slopes": alibi_slopes}
    bad = sorted(name for name, val in unsupported.items() if val is not None)
    if tuple(window_size) != (-1, -1):
        bad.append("window_size")
    if softcap:
        bad.append("softcap")
    if return_softmax_lse:
        bad.append("return_softmax_lse")
    if bad:
        raise NotImplementedError(f"flash_attn_with_kvcache: unsupported options {bad}")
    _lib.require_gpu(q, k_cache, v_cache, cache_seqlens, out)
    if q.dim() != 4 or q.shape[1] != 1:
        raise ValueError("q must be [batch, 1, heads, 128] (one query position per row)")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache and v_cache must be [batch, keys, kv_heads, 128] of one shape")
    if not (q.dtype == k_cache.dtype == v_cache.dtype == torch.bfloat16):
        raise ValueError("q, k_cache and v_cache must be bfloat16")
    B, _, Hq, D = q.shape
    Bk, S, Hkv, Dk = k_cache.shape
    if D != 128 or Dk != 128 or Bk != B:
        raise ValueError("head dim must be 128 and batch sizes must agree")
    if Hq % Hkv or Hq // Hkv > 4:
        raise ValueError("query heads must be a multiple of KV heads, at most 4 per KV head")
    if q.stride(3) != 1 or k_cache.stride(3) != 1 or v_cache.stride(3) != 1:
        raise ValueError("the head dimension must be contiguous")
    if cache_seqlens is not None and (cache_seqlens.dtype != torch.int32 or cache_seqlens.numel() != B
                                      or not cache_seqlens.is_contiguous()):
        raise ValueError("cache_seqlens must be a contiguous int32 [batch] tensor")
    if out is None:
        out = torch.empty((B, 1, Hq, D), device=q.device, dtype=torch.bfloat16)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (B, 1, Hq, D) or out.stride(3) != 1:
        raise ValueError("out must be bfloat16 [batch, 1, heads, 128] with a contiguous head dimension")
    scale = float(softmax_scale) if softmax_scale is not None else 1.0 / math.sqrt(D)
    _lib.call("v1_decode_attention", _lib.ptr(q), q.stride(0), q.stride(2), _lib.ptr(k_cache), k_cache.stride(0),
              k_cache.stride(1), k_cache.stride(2), _lib.ptr(v_cache), v_cache.stride(0), v_cache.stride(1),
              v_cache.stride(2), _lib.ptr(cache_seqlens), _lib.ptr(out), out.stride(0), out.stride(2), B, Hq, Hkv, S,
              scale, _lib.stream_of(q))
    return out


def attend_slots(q, k_pool, v_pool, request_slots, ids, head, softmax_scale=None, out=None):
    """GatherWorkspace.gather(k_pool, v_pool, request_slots, ids, head) followed by
    flash_attn_with_kvcache(q[:, None], kg, vg) in one pass over the pools, no
    workspace: q [rows, heads, 128] (or [rows, 1, heads, 128]) bf16 with at most
    4 heads, pools [slots, kv_heads, 128] bf16 (head dim contiguous), ids
    [rows, keys] int32 into request_slots.  Returns [rows, 1, heads, 128],
    equal bit for bit to the two-step form."""
    _lib.require_gpu(q, k_pool, v_pool, request_slots, ids, out)
    if q.dim() == 4:
        if q.shape[1] != 1:
            raise ValueError("q must hold one query position per row")
        q = q[:, 0]
    if q.dim() != 3 or q.shape[2] != 128 or q.dtype != torch.bfloat16 or q.stride(2) != 1:
        raise ValueError("q must be bfloat16 [rows, heads, 128] with a contiguous head dimension")
    for pool in (k_pool, v_pool):
        if pool.dim() != 3 or pool.shape[2] != 128 or pool.dtype != torch.bfloat16 or pool.stride(2) != 1:
            raise ValueError("pools must be bfloat16 [slots, kv_heads, 128] with a contiguous head dimension")
    if k_pool.shape[:2] != v_pool.shape[:2] or not 0 <= int(head) < k_pool.shape[1]:
        raise ValueError("k_pool and v_pool must agree and head must be one of their KV heads")
    if request_slots.dtype != torch.int32 or request_slots.dim() != 1 or not request_slots.is_contiguous():
        raise ValueError("request_slots must be a contiguous int32 vector")
    if ids.dtype != torch.int32 or ids.dim() != 2 or ids.shape[0] != q.shape[0] or ids.stride(1) != 1:
        raise ValueError("ids must be int32 [rows, keys] with a contiguous inner dimension")
    rows, heads, _ = q.shape
    if out is None:
        out = torch.empty((rows, 1, heads, 128), device=q.device, dtype=torch.bfloat16)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (rows, 1, heads, 128) or out.stride(3) != 1:
        raise ValueError("out must be bfloat16 [rows, 1, heads, 128] with a contiguous head dimension")
    scale = float(softmax_scale) if softmax_scale is not None else 1.0 / math.sqrt(128)
    _lib.call("v1_decode_attention_slots", _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k_pool), k_pool.stride(0),
              k_pool.stride(1), _lib.ptr(v_pool), v_pool.stride(0), v_pool.stride(1), k_pool.shape[0], int(head),
              _lib.ptr(request_slots), request_slots.numel(), _lib.ptr(ids), ids.stride(0), _lib.ptr(out),
              out.stride(0), out.stride(2), rows, heads, ids.shape[1], scale, _lib.stream_of(q))
    return out

