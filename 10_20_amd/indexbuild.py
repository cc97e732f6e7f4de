"""Batched index build: the producer chain of
sglang/srt/layers/attention/v1_deepseek/runtime.py:171-216 (initialize,
seven levels of _dots / _anchor / _sort, assemble) for many 1024-token
buckets in one launch, one work-group per bucket.

build_buckets(pool, tables, starts) -> (perm, tmp, mapping, centers):
  pool     uint8 [pages, 8448] native pages (128 FP8 bytes per token, then 64
           fp32 scales)
  tables   int32 [buckets, 16]: the bucket's 16 source pages
  starts   int32 [buckets]: the bucket's first logical token (META[0])
  perm     int32 [buckets, 1024]: member order (token index in the bucket)
  tmp      uint8 [buckets, 16, 8448]: the members' keys and scales in order
  mapping  int32 [buckets, 16, 64]: starts[b] + perm
  centers  uint8 [buckets, 2, 8448]: 128 FP8 centers (means of 8 members)
           with their power-of-two scales
Results equal the chain of the per-kernel drop-ins (kernels.initialize,
fused_grouping._dots/_anchor/_sort, kernels.assemble) bit for bit.
"""
import torch

from . import _lib

PAGE_BYTES = 8448


def build_buckets(pool, tables, starts, out=None):
    _lib.require_gpu(pool, tables, starts)
    if pool.dtype != torch.uint8 or pool.dim() != 2 or pool.shape[1] != PAGE_BYTES or not pool.is_contiguous():
        raise ValueError("pool must be a contiguous uint8 [pages, 8448] tensor")
    if tables.dtype != torch.int32 or tables.dim() != 2 or tables.shape[1] != 16 or not tables.is_contiguous():
        raise ValueError("tables must be a contiguous int32 [buckets, 16] tensor")
    B = tables.shape[0]
    if starts.dtype != torch.int32 or starts.numel() != B or not starts.is_contiguous():
        raise ValueError("starts must hold one int32 per bucket")
    dev = pool.device
    if out is None:
        out = (torch.empty((B, 1024), device=dev, dtype=torch.int32),
               torch.empty((B, 16, PAGE_BYTES), device=dev, dtype=torch.uint8),
               torch.empty((B, 16, 64), device=dev, dtype=torch.int32),
               torch.empty((B, 2, PAGE_BYTES), device=dev, dtype=torch.uint8))
    perm, tmp, mapping, centers = out
    _lib.call("v1_build_buckets", _lib.ptr(pool), pool.shape[0], _lib.ptr(tables), _lib.ptr(starts), B,
              _lib.ptr(perm), _lib.ptr(tmp), _lib.ptr(mapping), _lib.ptr(centers), _lib.stream_of(pool))
    return perm, tmp, mapping, centers
