"""C ABI checks that need no GPU: libv1idx.so loads, exports every function
include/v1idx.h declares, the ctypes binding covers each with the header's
arity, and argument validation rejects bad calls before any launch."""
import ctypes
import re
from pathlib import Path

import pytest

from conftest import pkg

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "v1idx.h"


def declared():
    """name -> number of parameters, for every function the header declares."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"#.*", "", text)
    out = {}
    for m in re.finditer(r"\b(v1_\w+)\s*\(([^;{)]*)\)\s*;", text, flags=re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    _lib = pkg("_lib")
    if not _lib.LIB_PATH.exists():
        pkg("build").build()
    return _lib


def test_header_parses():
    names = declared()
    assert len(names) >= 20
    assert names["v1_route"] == 2 and names["v1_last_error"] == 0 and names["v1_gather_slots"] == 20


def test_library_exports_every_declared_symbol(lib):
    handle = ctypes.CDLL(str(lib.LIB_PATH))
    missing = [n for n in declared() if not hasattr(handle, n)]
    assert not missing, f"libv1idx.so lacks {missing}"


def test_binding_matches_header(lib):
    names = declared()
    assert set(lib.exported_symbols()) == set(names)
    for name, arity in names.items():
        assert len(lib._SIGNATURES[name][1]) == arity, name


def test_binding_loads_and_version(lib):
    handle = lib.lib()
    assert handle.v1_abi_version() >= 1


def test_null_args_rejected_without_launch(lib):
    h = lib.lib()
    for name in ("v1_route", "v1_topk", "v1_topk_transform", "v1_score"):
        rc = getattr(h, name)(None, None)
        assert rc == lib.V1_ERR_INVALID, name
        assert b"null" in h.v1_last_error()


def test_validation_messages(lib):
    h = lib.lib()
    a = lib.TopkArgs()
    a.batch, a.cols, a.pages, a.topk, a.selected_bits, a.member_pages = 4, 64, 1, 4096, 32, 1
    assert h.v1_topk(ctypes.byref(a), None) == lib.V1_ERR_INVALID
    assert b"topk must be in (0, 2048]" in h.v1_last_error()
    with pytest.raises(ValueError, match="2048"):
        lib.check(h.v1_topk(ctypes.byref(a), None), "v1_topk")
    a.topk, a.window = 16, 5000
    assert h.v1_topk(ctypes.byref(a), None) == lib.V1_ERR_INVALID
    assert b"window" in h.v1_last_error()


def test_workspace_sizes_are_host_arithmetic(lib):
    h = lib.lib()
    assert h.v1_topk_workspace(4096, 32768, 2048) == 0       # large batch: one work-group per row
    assert h.v1_topk_workspace(4096, 65536, 2048) == 4096 * 2 * (2048 * 8 + 4)
    assert h.v1_topk_workspace(128, 131072, 2048) == 128 * 4 * (2048 * 8 + 4)
    # rows up to 40960 columns: one pass from 512 rows on, segments of at most 32768 columns below
    assert h.v1_topk_workspace(1024, 34880, 2048) == 0
    assert h.v1_topk_workspace(128, 34880, 2048) == 128 * 2 * (2048 * 8 + 4)
    assert h.v1_score_workspace(4096, 32768) >= 4096 * (8 * 128 + 8 * 4 + 16 * 4)
    # per-row tables: the page-union plan only for more than 512 rows of at most 65536 columns
    assert h.v1_score_tables_workspace(512, 34880) == 0
    assert h.v1_score_tables_workspace(1024, 65537) == 0
    need = h.v1_score_tables_workspace(1024, 34880)
    assert need >= h.v1_score_workspace(1024, 34880) + 128 * 8 * 545 * (4 + 4 + 32) and need % 256 == 0


def test_sort_rejects_bad_group_size(lib):
    h = lib.lib()
    rc = h.v1_sort_f32(None, None, None, None, 3, 1, 1, 0, None)
    assert rc == lib.V1_ERR_INVALID
