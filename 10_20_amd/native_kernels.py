"""Drop-in slot gather of sglang/srt/layers/attention/v1_native/kernels.py:62-111.

`_gather_slots[grid](K, V, REQ, IDS, KG, VG, ROWS, TOP, HEAD, KS0, KS1, KS2,
VS0, VS1, VS2, IS0, BLOCK)` and `GatherWorkspace` keep the reference
signatures; `gather_rows` is the same contract for opaque byte rows (e.g. the
656-byte MLA latent row: 512 FP8 + 64 bf16 RoPE + fp32 scales) with an
optional per-row page table.
"""
import torch

from . import _lib
from .kernels import _Kernel


def _gather_launch(grid, K, V, REQ, IDS, KG, VG, ROWS, TOP, HEAD, KS0, KS1, KS2, VS0, VS1, VS2, IS0, BLOCK=32):
    _lib.require_gpu(K, V, REQ, IDS, KG, VG)
    if K.element_size() != V.element_size() or KG.dtype != K.dtype or VG.dtype != V.dtype:
        raise ValueError("_gather_slots: K/V pools and outputs must share one dtype")
    if REQ.dtype != torch.int32 or IDS.dtype != torch.int32:
        raise ValueError("_gather_slots: REQ and IDS must be int32")
    _lib.call("v1_gather_slots", _lib.ptr(K), _lib.ptr(V), K.shape[0], K.element_size(), int(KS0), int(KS1),
              int(KS2), int(VS0), int(VS1), int(VS2), int(HEAD), _lib.ptr(REQ), REQ.numel(), _lib.ptr(IDS),
              int(IS0), int(ROWS), int(TOP), _lib.ptr(KG), _lib.ptr(VG), _lib.stream_of(K))


_gather_slots = _Kernel("_gather_slots", _gather_launch)


class GatherWorkspace:
    """The gathered K and V of up to `rows` decode queries x 2048 slots, held
    by the attention backend and reused by every call (sglang/srt/layers/
    attention/v1_native/kernels.py:80-111 is the interface): the buffers are
    made on first use, `gather` fills the first len(ids) rows and returns them,
    and a batch larger than `rows` is an error."""

    def __init__(self, rows, device, dtype):
        self.rows, self.device, self.dtype = rows, device, dtype
        self.k = self.v = None

    def release_request(self, slot):
        pass

    def clear(self):
        self.k = self.v = None

    def ensure_allocated(self):
        if self.k is None:
            k = torch.empty((self.rows, 2048, 1, 128), device=self.device, dtype=self.dtype)
            v = torch.empty_like(k)
            self.k, self.v = k, v

    def gather(self, k_pool, v_pool, request_slots, ids, head):
        rows = len(ids)
        if rows > self.rows:
            raise ValueError("Gather workspace microbatch exceeded")
        self.ensure_allocated()
        k, v = self.k[:rows], self.v[:rows]
        _gather_slots[(max(1, -(-rows * 2048 // 32)),)](
            k_pool, v_pool, request_slots, ids, k, v, rows, 2048, head, *k_pool.stride(), *v_pool.stride(),
            ids.stride(0), 32)
        return k, v


def gather_rows(pool, ids, out, table=None, page_bits=0):
    """out[r, i] = pool row of ids[r, i] (zeros for ids < 0).

    pool:  [pool_rows, row_bytes] uint8 (row stride may exceed row_bytes)
    ids:   [rows, top] int32 (row stride free)
    out:   [rows, top, row_bytes] uint8, contiguous
    table: None (ids are pool rows), a 1-D map shared by all rows, or a
           [rows, entries] per-row map; physical = (table[r, id >> page_bits]
           << page_bits) | (id & (2**page_bits - 1)).
    """
    _lib.require_gpu(pool, ids, out, table)
    if pool.dtype != torch.uint8 or pool.dim() != 2 or pool.stride(1) != 1:
        raise ValueError("gather_rows: pool must be a uint8 [rows, row_bytes] tensor with unit inner stride")
    rows, top = ids.shape
    row_bytes = pool.shape[1]
    if tuple(out.shape) != (rows, top, row_bytes) or out.dtype != torch.uint8 or not out.is_contiguous():
        raise ValueError("gather_rows: out must be a contiguous uint8 [rows, top, row_bytes] tensor")
    if ids.dtype != torch.int32 or ids.stride(1) != 1:
        raise ValueError("gather_rows: ids must be int32 with unit inner stride")
    map_ptr, map_len, map_stride = 0, 0, 0
    if table is not None:
        if table.dtype != torch.int32:
            raise ValueError("gather_rows: table must be int32")
        if table.dim() == 1:
            map_len, map_stride = table.shape[0], 0
        else:
            if table.shape[0] != rows or table.stride(1) != 1:
                raise ValueError("gather_rows: per-row table must be [rows, entries] with unit inner stride")
            map_len, map_stride = table.shape[1], table.stride(0)
        map_ptr = _lib.ptr(table)
    _lib.call("v1_gather_rows", _lib.ptr(pool), pool.shape[0], row_bytes, pool.stride(0), map_ptr, map_len,
              map_stride, int(page_bits), _lib.ptr(ids), ids.stride(0), rows, top, _lib.ptr(out), _lib.stream_of(pool))
    return out
