"""MI355X (gfx950) query-indexing hot path of the V1 sparse-attention indexer:
page route, FP8 index scoring, exact Top-2048 with slot mapping, grouping sort,
page manager with shared tail staging, and the K/V slot gather.

Every operator runs a hand-written HIP kernel from lib/libv1idx.so (C ABI in
include/v1idx.h); see build.py for the build recipe.
"""
from . import _lib
from .build import build

__all__ = ["build", "load"]


def load():
    """Loads libv1idx.so (raises if it was not built) and returns it."""
    return _lib.lib()
