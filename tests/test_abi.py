"""The C ABI library loads and exports what include/sfa.h declares; host-only
entry points (no GPU needed) validate their arguments."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from strataflow_amd import _lib
from strataflow_amd._lib import SfaKvDesc

HEADER = Path(__file__).resolve().parent.parent / "include" / "sfa.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"SFA_API\s+[\w\s\*]+?\b(sfa_\w+)\s*\(", text))


def test_header_matches_binding_list():
    assert declared_symbols() == set(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def desc(**kw) -> SfaKvDesc:
    d = SfaKvDesc()
    d.n_head, d.n_head_kv, d.head_dim, d.page_size = 32, 8, 128, 256
    d.kv_type, d.n_pages = _lib.SFA_KV_F16, 16
    d.k_pages = d.v_pages = 0x1000  # never dereferenced by host-only calls
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def test_status_strings():
    assert _lib.status_str(0) == "ok"
    assert _lib.status_str(1) == "invalid argument"
    assert _lib.status_str(12345) == "unknown status"


def test_row_and_page_bytes():
    lib = _lib.load()
    assert lib.sfa_row_bytes(ctypes.byref(desc())) == 256
    assert lib.sfa_page_bytes(ctypes.byref(desc())) == 256 * 8 * 256
    q8 = desc(kv_type=_lib.SFA_KV_Q8_0)
    assert lib.sfa_row_bytes(ctypes.byref(q8)) == 136
    assert lib.sfa_page_bytes(ctypes.byref(q8)) == 136 * 8 * 256


@pytest.mark.parametrize("field,value,status", [
    ("n_head", 30, _lib.SFA_ERR_INVALID_ARGUMENT),     # not a multiple of n_head_kv
    ("head_dim", 96, _lib.SFA_ERR_UNSUPPORTED),
    ("page_size", 100, _lib.SFA_ERR_INVALID_ARGUMENT),  # not a multiple of 32
    ("kv_type", 2, _lib.SFA_ERR_UNSUPPORTED),
    ("n_head_kv", 2, _lib.SFA_ERR_UNSUPPORTED),         # group size 16
    ("k_pages", None, _lib.SFA_ERR_INVALID_ARGUMENT),
])
def test_desc_check_rejects(field, value, status):
    lib = _lib.load()
    assert lib.sfa_kv_desc_check(ctypes.byref(desc())) == 0
    assert lib.sfa_kv_desc_check(ctypes.byref(desc(**{field: value}))) == status


def test_page_table_check():
    import numpy as np
    lib = _lib.load()
    d = desc(n_pages=4)
    pt = np.array([[3, 1, -1], [0, -1, -1]], np.int32)
    sl = np.array([300, 256], np.int32)
    ok = lib.sfa_page_table_check(ctypes.byref(d), pt.ctypes.data, 3, sl.ctypes.data, None, 2)
    assert ok == 0
    sl2 = np.array([600, 256], np.int32)  # needs logical page 2 of seq 0 (-1)
    assert lib.sfa_page_table_check(ctypes.byref(d), pt.ctypes.data, 3, sl2.ctypes.data, None, 2) == 1
    pt2 = pt.copy()
    pt2[1, 0] = 4  # outside the pool
    assert lib.sfa_page_table_check(ctypes.byref(d), pt2.ctypes.data, 3, sl.ctypes.data, None, 2) == 1
    # a window start past the missing page makes it unnecessary
    lo = np.array([0, 0], np.int32)
    pt3 = pt.copy()
    pt3[0, 0] = -1
    lo[0] = 256
    assert lib.sfa_page_table_check(ctypes.byref(d), pt3.ctypes.data, 3, sl.ctypes.data, lo.ctypes.data, 2) == 0


def test_decode_workspace_bytes():
    lib = _lib.load()
    d = desc()
    n1 = lib.sfa_decode_workspace_bytes(ctypes.byref(d), 1, 4096)
    n8 = lib.sfa_decode_workspace_bytes(ctypes.byref(d), 8, 32768)
    assert n1 > 0 and n8 >= n1
    assert lib.sfa_decode_workspace_bytes(ctypes.byref(d), 0, 4096) == 0
    assert lib.sfa_decode_workspace_bytes(ctypes.byref(desc(head_dim=96)), 1, 4096) == 0
    # a long Q8_0 batch runs the column layout: 2048 / Hkv = 256 split records
    # per kv head, each g * (head_dim + 4) floats
    q8 = desc(kv_type=_lib.SFA_KV_Q8_0)
    assert lib.sfa_decode_workspace_bytes(ctypes.byref(q8), 8, 32768) >= 8 * 256 * 4 * (128 + 4) * 4
