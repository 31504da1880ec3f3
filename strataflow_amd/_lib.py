"""ctypes binding of libsfa.so (include/sfa.h).

The library is built in-tree by ``strataflow_amd.build``.  Loading fails loudly
when it is missing: there is no CPU fallback for the attention path.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsfa.so"

SFA_OK = 0
SFA_ERR_INVALID_ARGUMENT = 1
SFA_ERR_UNSUPPORTED = 3
SFA_ERR_OUT_OF_MEMORY = 4
SFA_ERR_RUNTIME = 7

SFA_KV_F32 = 0
SFA_KV_F16 = 1
SFA_KV_Q8_0 = 8

#: scratch bytes of sfa_attn_decode_noalloc (SFA_NOALLOC_SCRATCH_BYTES)
SFA_NOALLOC_SCRATCH_BYTES = 8 << 20

#: every symbol include/sfa.h declares
EXPORTS = (
    "sfa_status_str",
    "sfa_version",
    "sfa_row_bytes",
    "sfa_page_bytes",
    "sfa_kv_desc_check",
    "sfa_kv_append",
    "sfa_rope_kv_append",
    "sfa_decode_workspace_bytes",
    "sfa_workspace_init",
    "sfa_attn_decode",
    "sfa_attn_decode_append",
    "sfa_attn_decode_split",
    "sfa_attn_decode_merge",
    "sfa_attn_decode_noalloc",
    "sfa_attn_prefill",
    "sfa_page_table_check",
)

# include/sfa_layer.h (the rest of the decode layer; also in libsfa.so)
LAYER_EXPORTS = (
    "sfa_rms_norm",
    "sfa_mul_mat_vec",
    "sfa_moe_route",
    "sfa_moe_gate",
    "sfa_moe_norm_gate",
    "sfa_qkv_rope_kv_append",
    "sfa_moe_workspace_bytes",
    "sfa_moe_ffn",
)


class SfaKvDesc(ctypes.Structure):
    _fields_ = [
        ("n_head", ctypes.c_int32),
        ("n_head_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("kv_type", ctypes.c_int32),
        ("n_pages", ctypes.c_int32),
        ("k_pages", ctypes.c_void_p),
        ("v_pages", ctypes.c_void_p),
        ("n_cold_pages", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("k_cold", ctypes.c_void_p),
        ("v_cold", ctypes.c_void_p),
    ]


class SfaError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {status_str(status)} ({status})")


_lib = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Loads libsfa.so (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path or os.environ.get("SFA_LIB", LIB_PATH))
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: build the HIP library first "
            "(python -m strataflow_amd.build); there is no CPU fallback"
        )
    lib = ctypes.CDLL(str(p))
    P = ctypes.c_void_p
    i32 = ctypes.c_int32
    D = ctypes.POINTER(SfaKvDesc)
    lib.sfa_status_str.argtypes = [ctypes.c_int]
    lib.sfa_status_str.restype = ctypes.c_char_p
    lib.sfa_version.argtypes = []
    lib.sfa_version.restype = ctypes.c_char_p
    lib.sfa_row_bytes.argtypes = [D]
    lib.sfa_row_bytes.restype = ctypes.c_size_t
    lib.sfa_page_bytes.argtypes = [D]
    lib.sfa_page_bytes.restype = ctypes.c_size_t
    lib.sfa_kv_desc_check.argtypes = [D]
    lib.sfa_kv_desc_check.restype = ctypes.c_int
    lib.sfa_kv_append.argtypes = [D, P, P, P, P, i32, P, i32, P]
    lib.sfa_kv_append.restype = ctypes.c_int
    lib.sfa_rope_kv_append.argtypes = [D, P, P, P, P, P, i32, P, i32, ctypes.c_float, P]
    lib.sfa_rope_kv_append.restype = ctypes.c_int
    lib.sfa_decode_workspace_bytes.argtypes = [D, i32, i32]
    lib.sfa_decode_workspace_bytes.restype = ctypes.c_size_t
    lib.sfa_workspace_init.argtypes = [P, ctypes.c_size_t, P]
    lib.sfa_workspace_init.restype = ctypes.c_int
    lib.sfa_attn_decode.argtypes = [D, P, P, P, i32, P, P, i32, i32, ctypes.c_float, P,
                                    ctypes.c_size_t, P]
    lib.sfa_attn_decode.restype = ctypes.c_int
    lib.sfa_attn_decode_append.argtypes = [D, P, P, P, P, P, i32, P, P, i32, i32, ctypes.c_float, P,
                                           ctypes.c_size_t, P]
    lib.sfa_attn_decode_append.restype = ctypes.c_int
    for name in ("sfa_attn_decode_split", "sfa_attn_decode_merge"):
        f = getattr(lib, name)
        f.argtypes = lib.sfa_attn_decode.argtypes
        f.restype = ctypes.c_int
    lib.sfa_attn_decode_noalloc.argtypes = [D, P, P, P, i32, P, P, i32, i32, ctypes.c_float, P]
    lib.sfa_attn_decode_noalloc.restype = ctypes.c_int
    lib.sfa_attn_prefill.argtypes = [D, P, P, P, i32, i32, i32, i32, ctypes.c_float, P]
    lib.sfa_attn_prefill.restype = ctypes.c_int
    lib.sfa_page_table_check.argtypes = [D, P, i32, P, P, i32]
    lib.sfa_page_table_check.restype = ctypes.c_int
    # the rest of the decode layer (include/sfa_layer.h)
    lib.sfa_rms_norm.argtypes = [P, P, P, i32, i32, ctypes.c_float, P]
    lib.sfa_rms_norm.restype = ctypes.c_int
    lib.sfa_mul_mat_vec.argtypes = [P, i32, P, P, P, i32, i32, i32, P]
    lib.sfa_mul_mat_vec.restype = ctypes.c_int
    lib.sfa_moe_route.argtypes = [P, i32, i32, i32, P, P, P]
    lib.sfa_moe_route.restype = ctypes.c_int
    lib.sfa_moe_gate.argtypes = [P, i32, P, i32, i32, i32, i32, P, P, P]
    lib.sfa_moe_gate.restype = ctypes.c_int
    lib.sfa_moe_norm_gate.argtypes = [P, P, ctypes.c_float, P, i32, i32, i32, i32, i32, P, P, P, P]
    lib.sfa_moe_norm_gate.restype = ctypes.c_int
    lib.sfa_qkv_rope_kv_append.argtypes = [D, P, i32, P, i32, P, P, P, i32, P, i32, ctypes.c_float, P]
    lib.sfa_qkv_rope_kv_append.restype = ctypes.c_int
    lib.sfa_moe_workspace_bytes.argtypes = [i32, i32, i32]
    lib.sfa_moe_workspace_bytes.restype = ctypes.c_size_t
    lib.sfa_moe_ffn.argtypes = [P, P, P, P, P, P, P, i32, i32, i32, i32, i32, i32, P, ctypes.c_size_t, P, P]
    lib.sfa_moe_ffn.restype = ctypes.c_int
    _lib = lib
    return lib


def status_str(status: int) -> str:
    return load().sfa_status_str(int(status)).decode()


def check(status: int, what: str) -> None:
    if status != SFA_OK:
        raise SfaError(status, what)


# ---- libsfa_host.so (include/sfa_pager.h) -----------------------------------

HOST_LIB_PATH = Path(__file__).resolve().parent / "libsfa_host.so"

SFA_ATTEND_LOSSLESS = 0
SFA_ATTEND_WINDOW = 1

#: every symbol include/sfa_pager.h declares
HOST_EXPORTS = (
    "sfa_pager_create",
    "sfa_pager_destroy",
    "sfa_pager_begin",
    "sfa_pager_append",
    "sfa_pager_rope_append",
    "sfa_pager_attend",
    "sfa_pager_append_attend",
    "sfa_pager_reset",
    "sfa_pager_stats_get",
    "sfa_pager_desc",
    "sfa_pager_max_pages",
    "sfa_pager_device_tables",
    "sfa_pager_tables",
)


class SfaPagerConfig(ctypes.Structure):
    _fields_ = [
        ("n_layer", ctypes.c_int32),
        ("n_head", ctypes.c_int32),
        ("n_head_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("kv_type", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("n_seq", ctypes.c_int32),
        ("n_ctx", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("attend", ctypes.c_int32),
        ("n_pages", ctypes.c_int32),
        ("n_cold_pages", ctypes.c_int32),
        ("seed", ctypes.c_uint64),
    ]


class SfaPagerStats(ctypes.Structure):
    _fields_ = [
        ("pages_allocated", ctypes.c_int64),
        ("pages_evicted", ctypes.c_int64),
        ("pages_dropped", ctypes.c_int64),
        ("dev_pages_in_use", ctypes.c_int64),
        ("cold_pages_in_use", ctypes.c_int64),
        ("bytes_evicted", ctypes.c_int64),
        ("pages_in_flight", ctypes.c_int64),
    ]


_host = None


def load_host(path: Path | str | None = None) -> ctypes.CDLL:
    """Loads libsfa_host.so (once; it loads libsfa.so next to it)."""
    global _host
    if _host is not None:
        return _host
    load()
    p = Path(path or os.environ.get("SFA_HOST_LIB", HOST_LIB_PATH))
    if not p.exists():
        raise RuntimeError(f"{p} is missing: build it first (python -m strataflow_amd.build)")
    lib = ctypes.CDLL(str(p))
    P = ctypes.c_void_p
    i32 = ctypes.c_int32
    lib.sfa_pager_create.argtypes = [ctypes.POINTER(SfaPagerConfig), ctypes.POINTER(P)]
    lib.sfa_pager_create.restype = ctypes.c_int
    lib.sfa_pager_destroy.argtypes = [P]
    lib.sfa_pager_destroy.restype = None
    lib.sfa_pager_begin.argtypes = [P, P, P]
    lib.sfa_pager_begin.restype = ctypes.c_int
    lib.sfa_pager_append.argtypes = [P, i32, P, P, P]
    lib.sfa_pager_append.restype = ctypes.c_int
    lib.sfa_pager_rope_append.argtypes = [P, i32, P, P, P, ctypes.c_float, P]
    lib.sfa_pager_rope_append.restype = ctypes.c_int
    lib.sfa_pager_attend.argtypes = [P, i32, P, P, P]
    lib.sfa_pager_attend.restype = ctypes.c_int
    lib.sfa_pager_append_attend.argtypes = [P, i32, P, P, P, P, P]
    lib.sfa_pager_append_attend.restype = ctypes.c_int
    lib.sfa_pager_reset.argtypes = [P, i32, P]
    lib.sfa_pager_reset.restype = ctypes.c_int
    lib.sfa_pager_stats_get.argtypes = [P, ctypes.POINTER(SfaPagerStats)]
    lib.sfa_pager_stats_get.restype = ctypes.c_int
    lib.sfa_pager_desc.argtypes = [P, i32, ctypes.POINTER(SfaKvDesc)]
    lib.sfa_pager_desc.restype = ctypes.c_int
    lib.sfa_pager_max_pages.argtypes = [P]
    lib.sfa_pager_max_pages.restype = i32
    lib.sfa_pager_device_tables.argtypes = [P, ctypes.POINTER(P), ctypes.POINTER(P), ctypes.POINTER(P)]
    lib.sfa_pager_device_tables.restype = ctypes.c_int
    lib.sfa_pager_tables.argtypes = [P, P, P]
    lib.sfa_pager_tables.restype = ctypes.c_int
    _host = lib
    return lib
