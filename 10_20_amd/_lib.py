"""ctypes binding of libv1idx.so (the C ABI declared in include/v1idx.h).

The library is loaded once, from lib/libv1idx.so next to this file.  There is
no fallback: if the library is missing every operator raises, so a run can
never silently compute on another path.
"""
import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libv1idx.so"

V1_OK = 0
V1_ERR_INVALID = -1

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


class RouteArgs(ctypes.Structure):
    _fields_ = [
        ("scores", _vp), ("score_stride", _c_i64), ("batch", _c_i32), ("score_cols", _c_i32),
        ("lens", _vp), ("takes", _vp), ("selected", _vp), ("selected_bits", _c_i32), ("take_stride", _c_i32),
        ("pages", _c_i32), ("rt", _vp), ("ft", _vp), ("ft_cols", _c_i32), ("tail_rows", _vp),
        ("capacity", _c_i32), ("fill_table", _c_i32),
    ]


class TopkArgs(ctypes.Structure):
    _fields_ = [
        ("scores", _vp), ("score_stride", _c_i64), ("batch", _c_i32), ("cols", _c_i32),
        ("fine_lens", _vp), ("members", _vp), ("member_pages", _c_i64), ("rt", _vp), ("nt", _vp),
        ("pages", _c_i32), ("selected", _vp), ("selected_bits", _c_i32), ("take_stride", _c_i32),
        ("lens", _vp), ("takes", _vp), ("physical", _vp), ("logical", _vp), ("raw", _vp), ("topk", _c_i32),
        ("window", _c_i32), ("mask", _c_i32), ("expanded", _vp), ("expansion_stride", _c_i32),
        ("physical_output", _c_i32), ("bucket_from_rank", _c_i32), ("fine_table", _vp),
        ("fine_table_cols", _c_i32), ("direct_fine", _c_i32), ("workspace", _vp), ("workspace_bytes", _c_i64),
    ]


class TopkTransformArgs(ctypes.Structure):
    _fields_ = [
        ("scores", _vp), ("score_stride", _c_i64), ("batch", _c_i32), ("cols", _c_i32),
        ("seq_lens", _vp), ("page_table", _vp), ("page_table_stride", _c_i64), ("page_table_cols", _c_i32),
        ("page_bits", _c_i32), ("page_indices", _vp), ("raw_indices", _vp), ("topk", _c_i32),
        ("workspace", _vp), ("workspace_bytes", _c_i64),
    ]


class ScoreArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("kv_pages", _vp), ("kv_blocks", _c_i64), ("weights", _vp), ("context_lens", _vp),
        ("block_table", _vp), ("block_table_stride", _c_i64), ("max_blocks", _c_i32), ("logits", _vp),
        ("logits_stride", _c_i64), ("max_context_len", _c_i32), ("rows", _c_i32), ("heads", _c_i32),
        ("relu", _c_i32), ("clean_logits", _c_i32), ("workspace", _vp), ("workspace_bytes", _c_i64),
    ]


class CoarseArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("weights", _vp), ("centers", _vp), ("center_blocks", _c_i64), ("table", _vp),
        ("table_stride", _c_i64), ("lens", _vp), ("scores", _vp), ("rows", _c_i32), ("heads", _c_i32),
        ("maxp", _c_i32), ("relu", _c_i32), ("workspace", _vp), ("workspace_bytes", _c_i64),
    ]


class FineArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("weights", _vp), ("fine_pages", _vp), ("fine_blocks", _c_i64), ("native_pages", _vp),
        ("native_blocks", _c_i64), ("members", _vp), ("rt", _vp), ("nt", _vp), ("selected", _vp),
        ("selected_bits", _c_i32), ("lens", _vp), ("takes", _vp), ("scores", _vp), ("rows", _c_i32),
        ("heads", _c_i32), ("maxp", _c_i32), ("np", _c_i32), ("take_stride", _c_i32), ("width", _c_i32),
        ("sink", _c_i32), ("window", _c_i32), ("relu", _c_i32),
    ]


# name -> (restype, argtypes)
_SIGNATURES = {
    "v1_last_error": (ctypes.c_char_p, []),
    "v1_abi_version": (_c_i32, []),
    "v1_route": (_c_i32, [ctypes.POINTER(RouteArgs), _vp]),
    "v1_topk": (_c_i32, [ctypes.POINTER(TopkArgs), _vp]),
    "v1_topk_workspace": (_c_i64, [_c_i32, _c_i32, _c_i32]),
    "v1_topk_transform": (_c_i32, [ctypes.POINTER(TopkTransformArgs), _vp]),
    "v1_score": (_c_i32, [ctypes.POINTER(ScoreArgs), _vp]),
    "v1_reduce_centers": (_c_i32, [_vp, _c_i64, _vp, _vp, _c_i32, _c_i32, _vp]),
    "v1_coarse_workspace": (_c_i64, [_c_i32, _c_i32, _c_i64]),
    "v1_coarse": (_c_i32, [ctypes.POINTER(CoarseArgs), _vp]),
    "v1_fine": (_c_i32, [ctypes.POINTER(FineArgs), _vp]),
    "v1_score_workspace": (_c_i64, [_c_i32, _c_i32]),
    "v1_score_tables_workspace": (_c_i64, [_c_i32, _c_i32]),
    "v1_score_pages_workspace": (_c_i64, [_c_i32, _c_i32, _c_i64]),
    "v1_score_page_major": (_c_i32, [_c_i32, ctypes.POINTER(_c_i32)]),
    "v1_score_noalloc": (_c_i32, [ctypes.POINTER(ScoreArgs), _vp]),
    "v1_score_noalloc_capacity": (_c_i64, []),
    "v1_gather_slots": (_c_i32, [_vp, _vp, _c_i64, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32,
                                 _vp, _c_i64, _vp, _c_i64, _c_i32, _c_i32, _vp, _vp, _vp]),
    "v1_gather_rows": (_c_i32, [_vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i32, _vp, _c_i64, _c_i32,
                                _c_i32, _vp, _vp]),
    "v1_sort_f32": (_c_i32, [_vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i64, _vp]),
    "v1_build_initialize": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i32, _vp]),
    "v1_group_dots": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "v1_group_anchor": (_c_i32, [_vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "v1_build_assemble": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i32, _c_i32, _vp]),
    "v1_build_buckets": (_c_i32, [_vp, _c_i64, _vp, _vp, _c_i32, _vp, _vp, _vp, _vp, _vp]),
    "v1_sort_i64": (_c_i32, [_vp, _vp, _vp, _vp, _c_i32, _c_i32, _vp]),
    "v1_fingerprint": (_c_i32, [_vp, _vp, _vp, _vp, _c_i32, _c_i64, _vp]),
    "v1_match_pages": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i64, _vp]),
    "v1_allocate": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i32, _vp, _vp]),
    "v1_publish": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i32, _c_i64, _vp]),
    "v1_release": (_c_i32, [_vp, _vp, _vp, _vp, _c_i32, _vp]),
    "v1_sort_pairs_u64_workspace": (_c_i64, [_c_i64]),
    "v1_sort_pairs_u64": (_c_i32, [_vp, _vp, _vp, _vp, _c_i64, _c_i32, _vp, _c_i64, _vp]),
    "v1_page_insert_workspace": (_c_i64, [_c_i32, _c_i32]),
    "v1_page_insert": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _c_i32, _c_i64, _vp, _vp, _vp, _c_i32, _vp, _vp, _vp,
                                _c_i64, _vp]),
    "v1_page_release_workspace": (_c_i64, [_c_i32, _c_i32]),
    "v1_page_release": (_c_i32, [_vp, _c_i32, _vp, _vp, _vp, _c_i32, _vp, _vp, _c_i64, _vp]),
    "v1_query_metadata": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                   _c_i32, _c_i32, _vp]),
    "v1_query_lengths": (_c_i32, [_vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "v1_fine_table": (_c_i32, [_vp, _vp, _c_i32, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                               _vp]),
    "v1_stage_tail": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64,
                               _c_i64, _vp]),
    "v1_stage_tail_rows": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                    _c_i64, _c_i64, _c_i32, _vp]),
    "v1_mask_fine": (_c_i32, [_vp, _c_i64, _vp, _c_i32, _vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32,
                              _c_i32, _c_i32, _vp]),
    "v1_output_ids": (_c_i32, [_vp, _vp, _c_i64, _vp, _vp, _vp, _vp, _c_i32, _vp, _vp, _vp, _vp, _vp, _c_i32,
                               _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                               _vp]),
    "v1_expand_logical": (_c_i32, [_vp, _vp, _c_i32, _c_i32, _c_i64, _c_i32, _vp]),
    "v1_decode_attention": (_c_i32, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64,
                                     _vp, _vp, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, ctypes.c_float, _vp]),
    "v1_decode_attention_slots": (_c_i32, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64,
                                           _c_i32, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_i64, _c_i32, _c_i32,
                                           _c_i32, ctypes.c_float, _vp]),
    "v1_union_spans": (_c_i32, [_vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _vp]),
    "v1_union_normalize_split": (_c_i32, [_vp, _c_i64, _c_i32, _vp, _c_i64, _c_i32, _vp, _vp, _vp, _vp, _vp, _c_i64,
                                          _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "v1_stage_tail_published": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                         _c_i32, _c_i64, _c_i64, _vp]),
    "v1_stage_union": (_c_i32, [_vp, _c_i64, _vp, _c_i32, _vp, _c_i32, _vp, _vp, _c_i32, _vp, _vp, _c_i32,
                                _c_i32, _vp]),
    "v1_union_tables": (_c_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32,
                                 _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "v1_union_normalize": (_c_i32, [_vp, _c_i64, _c_i32, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _c_i32, _c_i32,
                                    _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "v1_union_map_topk": (_c_i32, [_vp, _c_i32, _vp, _vp, _c_i64, _c_i32, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp,
                                   _c_i32, _vp, _vp,
                                   _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
}

_lock = threading.Lock()
_lib = None


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build the HIP extension first "
                        "(__graft_entry__.build() or python <package>/build.py)")
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in _SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def exported_symbols():
    return sorted(_SIGNATURES)


def check(rc, what):
    if rc == V1_OK:
        return
    msg = lib().v1_last_error().decode(errors="replace")
    if rc == V1_ERR_INVALID:
        raise ValueError(msg or what)
    raise RuntimeError(f"{what} failed ({rc}): {msg}")


def call(name, *args):
    check(getattr(lib(), name)(*args), name)


def ptr(t):
    return 0 if t is None else t.data_ptr()


def stream_of(t):
    """Raw hipStream_t of the current stream on the tensor's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("V1 index operators need device (cuda/HIP) tensors")
    dev = {t.device for t in tensors if t is not None}
    if len(dev) > 1:
        raise ValueError("all tensors must be on the same device")
