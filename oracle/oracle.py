"""ctypes binding of the CPU oracle (liboracle.so, built from sfa_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and the bench's
CPU-baseline leg, to check results against.  The product path never imports it.
Pools here are host numpy arrays [n_pages, page_bytes] (uint8) holding the same
bytes as the device pools.
"""
from __future__ import annotations

import ctypes
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

KV_F32, KV_F16, KV_Q8_0 = 0, 1, 8
GGML, EXACT = 0, 1
#: forms of ggml's quantize_row_q8_0 (see orc_set_q8_variant in sfa_oracle.c)
Q8_SCALAR, Q8_AVX2, Q8_NEON = 0, 1, 2


class OrcPagedKv(ctypes.Structure):
    _fields_ = [
        ("n_head_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("kv_type", ctypes.c_int32),
        ("n_pages", ctypes.c_int32),
        ("n_cold_pages", ctypes.c_int32),
        ("k_pages", ctypes.c_void_p),
        ("v_pages", ctypes.c_void_p),
        ("k_cold", ctypes.c_void_p),
        ("v_cold", ctypes.c_void_p),
    ]


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        import subprocess
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    lib = ctypes.CDLL(str(LIB_PATH))
    P, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
    lib.orc_f32_to_f16.restype = ctypes.c_uint16
    lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.orc_f16_to_f32.restype = ctypes.c_float
    lib.orc_f32_to_f16_row.argtypes = [P, P, i64]
    lib.orc_f16_to_f32_row.argtypes = [P, P, i64]
    lib.orc_quantize_row_q8_0.argtypes = [P, P, i64]
    lib.orc_dequantize_row_q8_0.argtypes = [P, P, i64]
    lib.orc_row_bytes.argtypes = [ctypes.POINTER(OrcPagedKv)]
    lib.orc_row_bytes.restype = i64
    lib.orc_page_bytes.argtypes = [ctypes.POINTER(OrcPagedKv)]
    lib.orc_page_bytes.restype = i64
    lib.orc_kv_append.argtypes = [ctypes.POINTER(OrcPagedKv), P, P, P, P, i32, P, i32]
    lib.orc_kv_append.restype = ctypes.c_int
    lib.orc_attention.argtypes = [ctypes.POINTER(OrcPagedKv), P, P, i32, P, i32, P, P, i32, i32,
                                  ctypes.c_float, ctypes.c_int, ctypes.c_int]
    lib.orc_attention.restype = ctypes.c_int
    lib.orc_rope_normal.argtypes = [P, P, i32, i32, i32, ctypes.c_float]
    lib.orc_set_q8_variant.argtypes = [ctypes.c_int]
    lib.orc_set_q8_variant.restype = ctypes.c_int
    lib.orc_max_threads.argtypes = []
    lib.orc_max_threads.restype = ctypes.c_int
    _lib = lib
    return lib


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    load().orc_f32_to_f16_row(x.ctypes.data, y.ctypes.data, x.size)
    return y


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16)
    y = np.empty(h.shape, np.float32)
    load().orc_f16_to_f32_row(h.ctypes.data, y.ctypes.data, h.size)
    return y


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """x [..., k] f32 (k % 32 == 0) -> bytes [..., k/32*34]."""
    x = _c(x, np.float32)
    k = x.shape[-1]
    y = np.empty(x.shape[:-1] + (k // 32 * 34,), np.uint8)
    load().orc_quantize_row_q8_0(x.ctypes.data, y.ctypes.data, x.size)
    return y


def dequantize_q8_0(b: np.ndarray) -> np.ndarray:
    b = _c(b, np.uint8)
    k = b.shape[-1] // 34 * 32
    y = np.empty(b.shape[:-1] + (k,), np.float32)
    load().orc_dequantize_row_q8_0(b.ctypes.data, y.ctypes.data, y.size)
    return y


def row_bytes(kv_type: int, head_dim: int) -> int:
    return {KV_F32: head_dim * 4, KV_F16: head_dim * 2, KV_Q8_0: head_dim // 32 * 34}[kv_type]


class HostPagedKv:
    """Host-side paged pools with the device layout (page = page_size columns of
    n_head_kv rows)."""

    def __init__(self, n_head_kv: int, head_dim: int, page_size: int, kv_type: int,
                 n_pages: int, n_cold_pages: int = 0):
        self.n_head_kv, self.head_dim, self.page_size = n_head_kv, head_dim, page_size
        self.kv_type, self.n_pages, self.n_cold_pages = kv_type, n_pages, n_cold_pages
        self.page_bytes = row_bytes(kv_type, head_dim) * n_head_kv * page_size
        self.k = np.zeros((max(n_pages, 1), self.page_bytes), np.uint8)
        self.v = np.zeros((max(n_pages, 1), self.page_bytes), np.uint8)
        self.k_cold = np.zeros((max(n_cold_pages, 1), self.page_bytes), np.uint8)
        self.v_cold = np.zeros((max(n_cold_pages, 1), self.page_bytes), np.uint8)

    def desc(self) -> OrcPagedKv:
        return OrcPagedKv(self.n_head_kv, self.head_dim, self.page_size, self.kv_type,
                          self.n_pages, self.n_cold_pages, self.k.ctypes.data, self.v.ctypes.data,
                          self.k_cold.ctypes.data, self.v_cold.ctypes.data)

    def append(self, k: np.ndarray, v: np.ndarray, seq: np.ndarray, pos: np.ndarray,
               page_table: np.ndarray) -> int:
        k, v = _c(k, np.float32), _c(v, np.float32)
        seq, pos = _c(seq, np.int32), _c(pos, np.int32)
        pt = _c(page_table, np.int32)
        d = self.desc()
        return load().orc_kv_append(ctypes.byref(d), k.ctypes.data, v.ctypes.data,
                                    seq.ctypes.data, pos.ctypes.data, int(seq.size),
                                    pt.ctypes.data, int(pt.shape[-1]))

    def attention(self, q: np.ndarray, n_head: int, page_table: np.ndarray, seq_len,
                  kv_lo=None, T: int = 1, scale: float | None = None, mode: int = GGML,
                  n_threads: int = 0) -> np.ndarray:
        """q [B, T, Hq, hd] (or [B, Hq, hd] for T == 1) -> out of the same shape."""
        q = _c(q, np.float32)
        B = int(np.asarray(seq_len).size)
        out = np.empty_like(q)
        pt = _c(page_table, np.int32).reshape(B, -1)
        sl = _c(seq_len, np.int32).reshape(B)
        lo = None if kv_lo is None else _c(kv_lo, np.int32).reshape(B)
        if scale is None:
            scale = 1.0 / np.sqrt(self.head_dim)
        d = self.desc()
        rc = load().orc_attention(ctypes.byref(d), q.ctypes.data, out.ctypes.data, n_head,
                                  pt.ctypes.data, int(pt.shape[1]), sl.ctypes.data,
                                  None if lo is None else lo.ctypes.data, B, T,
                                  float(scale), mode, n_threads)
        if rc != 0:
            raise RuntimeError(f"orc_attention failed ({rc})")
        return out

    def time_attention(self, *args, reps: int = 3, **kw) -> float:
        """Median seconds of one attention call."""
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            self.attention(*args, **kw)
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))


def rope_normal(x: np.ndarray, pos: np.ndarray, freq_base: float) -> np.ndarray:
    """RoPE NORMAL of x [n_tok, n_heads, head_dim] (a rotated copy), through
    orc_rope_normal (ggml's f32 theta recurrence, engine.cpp:1892-1897)."""
    y = _c(x, np.float32).copy()
    pos = _c(pos, np.int32)
    n_tok, n_heads, hd = y.shape
    load().orc_rope_normal(y.ctypes.data, pos.ctypes.data, n_tok, n_heads, hd, float(freq_base))
    return y


class q8_variant:
    """Context manager selecting the form of ggml's quantize_row_q8_0 the
    oracle runs (Q8_SCALAR, Q8_AVX2 or Q8_NEON) for Q8_0 cache appends and the
    Q8_0 conversion of Q; restores the scalar form on exit."""

    def __init__(self, variant: int):
        self.variant = variant

    def __enter__(self):
        if load().orc_set_q8_variant(int(self.variant)) != 0:
            raise ValueError(f"unknown Q8_0 quantiser form {self.variant}")
        return self

    def __exit__(self, *exc):
        load().orc_set_q8_variant(Q8_SCALAR)
        return False


def max_threads() -> int:
    return int(load().orc_max_threads())
