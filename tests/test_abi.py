"""The C ABI library loads and exports what include/sfa.h declares; host-only
entry points (no GPU needed) validate their arguments."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from strataflow_amd import _lib
from strataflow_amd._lib import SfaKvDesc

INCLUDE = Path(__file__).resolve().parent.parent / "include"
HEADER = INCLUDE / "sfa.h"


def declared_symbols(header: Path = HEADER) -> set[str]:
    text = header.read_text()
    return set(re.findall(r"SFA_API\s+[\w\s\*]+?\b(sfa_\w+)\s*\(", text))


def test_header_matches_binding_list():
    assert declared_symbols() == set(_lib.EXPORTS)
    assert declared_symbols(INCLUDE / "sfa_layer.h") == set(_lib.LAYER_EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols() | declared_symbols(INCLUDE / "sfa_layer.h"):
        assert hasattr(lib, name), name


def test_layer_entry_points_validate_on_the_host():
    """Argument checks return before any device work (no GPU needed)."""
    lib = _lib.load()
    F16, F32 = _lib.SFA_KV_F16, _lib.SFA_KV_F32
    bad, uns = _lib.SFA_ERR_INVALID_ARGUMENT, _lib.SFA_ERR_UNSUPPORTED
    p = 0x1000  # never dereferenced
    assert lib.sfa_rms_norm(None, p, p, 1, 256, 1e-5, None) == bad
    assert lib.sfa_rms_norm(p, p, p, 1, 0, 1e-5, None) == bad
    assert lib.sfa_rms_norm(p, p, p, 0, 256, 1e-5, None) == _lib.SFA_OK  # nothing to do
    assert lib.sfa_mul_mat_vec(p, F16, p, None, p, 1, 100, 64, None) == uns      # n_in % 8
    assert lib.sfa_mul_mat_vec(p, 8, p, None, p, 1, 128, 64, None) == uns        # Q8_0 weights
    assert lib.sfa_mul_mat_vec(p, F32, None, None, p, 1, 128, 64, None) == bad
    assert lib.sfa_moe_route(p, 1, 65, 2, p, p, None) == uns                     # > 64 experts
    assert lib.sfa_moe_route(p, 1, 8, 9, p, p, None) == bad                      # n_used > n_expert
    assert lib.sfa_moe_norm_gate(p, p, 1e-5, p, F32, 1, 8200, 8, 2, p, p, p, None) == uns  # row past LDS
    assert lib.sfa_moe_norm_gate(p, p, 1e-5, p, F32, 1, 4100, 8, 2, p, p, p, None) == uns  # n_embd % 8
    assert lib.sfa_moe_norm_gate(p, p, 1e-5, p, F16, 1, 4096, 65, 2, p, p, p, None) == uns  # > 64 experts
    assert lib.sfa_moe_norm_gate(p, p, 1e-5, p, 8, 1, 4096, 8, 2, p, p, p, None) == uns    # Q8_0 weights
    assert lib.sfa_moe_norm_gate(p, p, 1e-5, p, F32, 1, 4096, 8, 9, p, p, p, None) == bad  # n_used > n_expert
    assert lib.sfa_moe_norm_gate(None, p, 1e-5, p, F32, 1, 4096, 8, 2, p, p, p, None) == bad
    assert lib.sfa_moe_norm_gate(p, p, -1.0, p, F32, 1, 4096, 8, 2, p, p, p, None) == bad  # eps < 0
    assert lib.sfa_moe_norm_gate(p, p, 1e-5, p, F32, 0, 4096, 8, 2, p, p, p, None) == _lib.SFA_OK
    d = desc()
    assert lib.sfa_qkv_rope_kv_append(ctypes.byref(desc(kv_type=_lib.SFA_KV_Q8_0)), p, F16, p, 4096, p, p, p, 1,
                                      p, 16, 1e6, None) == uns                   # Q8_0 cache
    assert lib.sfa_qkv_rope_kv_append(ctypes.byref(d), p, F16, p, 4100, p, p, p, 1, p, 16, 1e6, None) == uns
    assert lib.sfa_qkv_rope_kv_append(ctypes.byref(d), p, 8, p, 4096, p, p, p, 1, p, 16, 1e6, None) == uns
    assert lib.sfa_qkv_rope_kv_append(ctypes.byref(d), p, F16, p, 4096, p, p, p, 1, p, 16, 0.0, None) == bad
    assert lib.sfa_qkv_rope_kv_append(ctypes.byref(d), p, F16, p, 4096, None, p, p, 1, p, 16, 1e6, None) == bad
    assert lib.sfa_qkv_rope_kv_append(ctypes.byref(d), p, F16, p, 4096, p, p, p, 0, p, 16, 1e6, None) == _lib.SFA_OK
    assert lib.sfa_qkv_rope_kv_append(ctypes.byref(d), p, F16, p, 4096, p, p, p, 70000, p, 16, 1e6, None) == uns
    assert lib.sfa_moe_workspace_bytes(2, 2, 512) == 2 * 2 * 512 * 4
    assert lib.sfa_moe_workspace_bytes(0, 2, 512) == 0
    ws = lib.sfa_moe_workspace_bytes(1, 2, 512)
    assert lib.sfa_moe_ffn(p, p, p, p, p, p, p, F32, 1, 256, 512, 8, 2, p, ws - 4, p, None) == bad
    assert lib.sfa_moe_ffn(p, p, p, p, p, p, p, F32, 1, 256, 500, 8, 2, p, ws, p, None) == uns


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


def test_q8_0_head_dim_32_is_unsupported():
    """A Q8_0 cache with head_dim 32 (one block per row) is refused by the
    descriptor check, so every entry point over it returns
    SFA_ERR_UNSUPPORTED from the host, before any device work: the append and
    the fused RoPE + append as well as decode and prefill (a cache that nothing
    could attend over is never written)."""
    lib = _lib.load()
    d = desc(kv_type=_lib.SFA_KV_Q8_0, head_dim=32)
    uns = _lib.SFA_ERR_UNSUPPORTED
    assert lib.sfa_kv_desc_check(ctypes.byref(d)) == uns
    assert lib.sfa_kv_desc_check(ctypes.byref(desc(kv_type=_lib.SFA_KV_Q8_0, head_dim=64))) == _lib.SFA_OK
    p = 0x1000  # never dereferenced
    assert lib.sfa_kv_append(ctypes.byref(d), p, p, p, p, 4, p, 4, None) == uns
    assert lib.sfa_rope_kv_append(ctypes.byref(d), p, p, p, p, p, 4, p, 4, 1e4, None) == uns
    assert lib.sfa_decode_workspace_bytes(ctypes.byref(d), 1, 256) == 0
    assert lib.sfa_attn_decode(ctypes.byref(d), p, p, p, 4, p, None, 1, 256, 0.1, p, 1 << 20,
                               None) == uns
    assert lib.sfa_attn_prefill(ctypes.byref(d), p, p, p, 4, 0, 16, 0, 0.1, None) == uns


@pytest.mark.parametrize("page_size", [32, 96, 100])
def test_pager_refuses_page_sizes_the_prefill_cannot_tile(page_size):
    """A pager attends multi-token steps with the chunked prefill, whose
    64-position tiles must not straddle a page: sfa_pager_create refuses a
    page size that is not a multiple of 64 up front (host check, before any
    allocation), instead of refusing the attention after a step has begun."""
    lib = _lib.load_host()
    c = _lib.SfaPagerConfig(2, 32, 8, 128, _lib.SFA_KV_F16, page_size, 2, 2048, 300,
                            _lib.SFA_ATTEND_LOSSLESS, 0, 0, 0)
    h = ctypes.c_void_p()
    assert lib.sfa_pager_create(ctypes.byref(c), ctypes.byref(h)) == _lib.SFA_ERR_UNSUPPORTED
    assert not h.value
    # a Q8_0 cache of head_dim 32 is refused by the pager's shape check too
    c = _lib.SfaPagerConfig(2, 8, 4, 32, _lib.SFA_KV_Q8_0, 256, 2, 2048, 300,
                            _lib.SFA_ATTEND_LOSSLESS, 0, 0, 0)
    assert lib.sfa_pager_create(ctypes.byref(c), ctypes.byref(h)) == _lib.SFA_ERR_UNSUPPORTED


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
