"""Drop-ins `_dots`, `_anchor` and `_sort` of
sglang/srt/layers/attention/v1_native/fused_grouping.py:38-76.

`_dots[(programs, heads)](U, P, A, S, FLAG, N, START, MODE)`: 16 positions per
program; the score of position i is the dot of member P[i] with its group's
first member (MODE 0) or anchor A[group, MODE-1] (MODE 1, 2), minus the
previous score for MODE 2 (four-partial fp32 sums, no fused multiply-add).
`_anchor[(groups, heads)](P, A, S, FLAG, N, SLOT)`: A[group, SLOT] = the member
at the group's leftmost minimum score.

`_sort[(groups, heads)](P, O, S, FLAG, N)`: when FLAG < 0, every group g of N
members of head h (offset h*4096, as in the reference) is reordered by
score descending, ties by ascending position: O[g*N+i] = P[g*N+pos_i].
-0.0 and +0.0 compare equal.  P is left unchanged; P and O must not alias.

`sort_groups_i64` applies the same rule to signed int64 keys (one head).
"""
import torch

from . import _lib
from .kernels import _Kernel

HEAD_STRIDE = 4096


def _sort_launch(grid, P, O, S, FLAG, N):
    _lib.require_gpu(P, O, S, FLAG)
    if P.dtype != torch.int32 or O.dtype != torch.int32 or S.dtype != torch.float32:
        raise ValueError("_sort: P/O must be int32 and S float32")
    groups = grid[0]
    heads = grid[1] if len(grid) > 1 else 1
    _lib.call("v1_sort_f32", _lib.ptr(P), _lib.ptr(O), _lib.ptr(S), _lib.ptr(FLAG), int(N), groups, heads,
              HEAD_STRIDE, _lib.stream_of(P))


_sort = _Kernel("_sort", _sort_launch)


def _dots_launch(grid, U, P, A, S, FLAG, N, START, MODE):
    _lib.require_gpu(U, P, A, S, FLAG)
    if U.dtype != torch.float32 or S.dtype != torch.float32 or P.dtype != torch.int32 or A.dtype != torch.int32:
        raise ValueError("_dots: U/S must be float32 and P/A int32")
    _lib.call("v1_group_dots", _lib.ptr(U), _lib.ptr(P), _lib.ptr(A), _lib.ptr(S), _lib.ptr(FLAG), int(N),
              int(START), int(MODE), grid[0], grid[1] if len(grid) > 1 else 1, _lib.stream_of(U))


def _anchor_launch(grid, P, A, S, FLAG, N, SLOT):
    _lib.require_gpu(P, A, S, FLAG)
    if S.dtype != torch.float32 or P.dtype != torch.int32 or A.dtype != torch.int32:
        raise ValueError("_anchor: S must be float32 and P/A int32")
    _lib.call("v1_group_anchor", _lib.ptr(P), _lib.ptr(A), _lib.ptr(S), _lib.ptr(FLAG), int(N), int(SLOT), grid[0],
              grid[1] if len(grid) > 1 else 1, _lib.stream_of(S))


_dots = _Kernel("_dots", _dots_launch)
_anchor = _Kernel("_anchor", _anchor_launch)


def sort_groups_i64(perm, out, keys, n, flag=None):
    """Stable descending sort of int64 keys inside groups of n (power of two)."""
    _lib.require_gpu(perm, out, keys, flag)
    if keys.dtype != torch.int64 or perm.dtype != torch.int32 or out.dtype != torch.int32:
        raise ValueError("sort_groups_i64: keys int64, perm/out int32")
    if keys.numel() % n:
        raise ValueError("sort_groups_i64: key count must be a multiple of n")
    _lib.call("v1_sort_i64", _lib.ptr(perm), _lib.ptr(out), _lib.ptr(keys), _lib.ptr(flag), int(n),
              keys.numel() // n, _lib.stream_of(keys))
