"""Python handle on the C++ host page manager (include/sfa_pager.h).

``KvPager`` owns one ``sfa_pager``: the device pool of every layer's K/V
pages, the host-pinned cold pool and the page tables, with KvStore window
semantics (src/kv/kv_store.h:30-95) at page granularity.  A step is
``begin(n_tok)`` then, per layer, ``append`` and ``attend``; every call is
ordered on the current torch stream.  This wrapper only marshals arguments.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import SFA_ATTEND_LOSSLESS, SFA_ATTEND_WINDOW, SFA_KV_F16, SFA_KV_F32, SFA_KV_Q8_0

__all__ = ["KvPager", "SFA_ATTEND_LOSSLESS", "SFA_ATTEND_WINDOW", "SFA_KV_F32", "SFA_KV_F16",
           "SFA_KV_Q8_0"]


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class KvPager:
    def __init__(self, *, n_layer: int, n_head: int, n_head_kv: int, head_dim: int, kv_type: int,
                 page_size: int, n_seq: int, n_ctx: int, window: int = 0,
                 attend: int = SFA_ATTEND_LOSSLESS, n_pages: int = 0, n_cold_pages: int = 0,
                 seed: int = 0):
        self._h = None
        lib = _lib.load_host()
        c = _lib.SfaPagerConfig(n_layer, n_head, n_head_kv, head_dim, kv_type, page_size, n_seq,
                                n_ctx, window, attend, n_pages, n_cold_pages, seed)
        h = ctypes.c_void_p()
        _lib.check(lib.sfa_pager_create(ctypes.byref(c), ctypes.byref(h)), "sfa_pager_create")
        self._h = h
        self.n_layer, self.n_head, self.n_head_kv, self.head_dim = n_layer, n_head, n_head_kv, head_dim
        self.n_seq, self.n_ctx, self.page_size, self.attend_mode = n_seq, n_ctx, page_size, attend
        self.window = window if 0 < window <= n_ctx else n_ctx
        self.max_pages = int(lib.sfa_pager_max_pages(h))
        self.n_tok = np.zeros(n_seq, dtype=np.int32)

    def close(self) -> None:
        if self._h is not None:
            _lib.load_host().sfa_pager_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def begin(self, n_tok) -> int:
        """Plans the next n_tok[b] positions of every sequence; returns the
        sf_status (0 on success) so callers can test out-of-pages."""
        n = np.ascontiguousarray(n_tok, dtype=np.int32)
        assert n.shape == (self.n_seq,)
        rc = _lib.load_host().sfa_pager_begin(self._h, n.ctypes.data, _stream())
        if rc == 0:
            self.n_tok = n.copy()
        return rc

    @property
    def n_tokens(self) -> int:
        return int(self.n_tok.sum())

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        assert k.is_contiguous() and v.is_contiguous() and k.dtype == torch.float32
        assert k.shape == (self.n_tokens, self.n_head_kv, self.head_dim) and v.shape == k.shape
        _lib.check(_lib.load_host().sfa_pager_append(self._h, layer, k.data_ptr(), v.data_ptr(),
                                                     _stream()), "sfa_pager_append")

    def rope_append(self, layer: int, q: torch.Tensor | None, k: torch.Tensor, v: torch.Tensor,
                    freq_base: float) -> None:
        """Fused RoPE NORMAL + append: q (rotated in place, or None) and k pre-RoPE."""
        assert k.is_contiguous() and v.is_contiguous() and k.dtype == torch.float32
        assert k.shape == (self.n_tokens, self.n_head_kv, self.head_dim) and v.shape == k.shape
        if q is not None:
            assert q.is_contiguous() and q.shape == (self.n_tokens, self.n_head, self.head_dim)
        _lib.check(_lib.load_host().sfa_pager_rope_append(
            self._h, layer, None if q is None else q.data_ptr(), k.data_ptr(), v.data_ptr(),
            float(freq_base), _stream()), "sfa_pager_rope_append")

    def attend(self, layer: int, q: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        assert q.is_contiguous() and q.dtype == torch.float32
        assert q.shape == (self.n_tokens, self.n_head, self.head_dim)
        if out is None:
            out = torch.empty((self.n_tokens, self.n_head * self.head_dim), dtype=torch.float32,
                              device=q.device)
        _lib.check(_lib.load_host().sfa_pager_attend(self._h, layer, q.data_ptr(), out.data_ptr(),
                                                     _stream()), "sfa_pager_attend")
        return out

    def append_attend(self, layer: int, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor,
                      out: torch.Tensor | None = None) -> torch.Tensor:
        """append then attend in one call (fused for a one-token-per-sequence
        step over an F16 or F32 cache)."""
        assert k.is_contiguous() and v.is_contiguous() and k.dtype == torch.float32
        assert k.shape == (self.n_tokens, self.n_head_kv, self.head_dim) and v.shape == k.shape
        assert q.is_contiguous() and q.dtype == torch.float32
        assert q.shape == (self.n_tokens, self.n_head, self.head_dim)
        if out is None:
            out = torch.empty((self.n_tokens, self.n_head * self.head_dim), dtype=torch.float32,
                              device=q.device)
        _lib.check(_lib.load_host().sfa_pager_append_attend(self._h, layer, k.data_ptr(), v.data_ptr(),
                                                            q.data_ptr(), out.data_ptr(), _stream()),
                   "sfa_pager_append_attend")
        return out

    def reset(self, seq: int) -> None:
        _lib.check(_lib.load_host().sfa_pager_reset(self._h, seq, _stream()), "sfa_pager_reset")

    def stats(self) -> dict:
        s = _lib.SfaPagerStats()
        _lib.check(_lib.load_host().sfa_pager_stats_get(self._h, ctypes.byref(s)), "stats")
        return {name: int(getattr(s, name)) for name, _ in s._fields_}

    def desc(self, layer: int) -> _lib.SfaKvDesc:
        d = _lib.SfaKvDesc()
        _lib.check(_lib.load_host().sfa_pager_desc(self._h, layer, ctypes.byref(d)), "desc")
        return d

    def device_tables(self) -> tuple[int, int, int]:
        """Device addresses of the pager's page tables [n_seq, max_pages],
        seq_len [n_seq] and kv_lo [n_seq] (int32)."""
        pt, sl, lo = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        _lib.check(_lib.load_host().sfa_pager_device_tables(self._h, ctypes.byref(pt), ctypes.byref(sl),
                                                            ctypes.byref(lo)), "device_tables")
        return pt.value, sl.value, lo.value

    @property
    def max_span(self) -> int:
        """The max_seq_len the pager's decode passes: n_ctx, or the window."""
        return self.window if self.attend_mode == SFA_ATTEND_WINDOW else self.n_ctx

    def tables(self) -> tuple[np.ndarray, np.ndarray]:
        """Host mirror: page tables [n_seq, max_pages] and fill positions [n_seq]."""
        pt = np.empty((self.n_seq, self.max_pages), dtype=np.int32)
        used = np.empty(self.n_seq, dtype=np.int32)
        _lib.check(_lib.load_host().sfa_pager_tables(self._h, pt.ctypes.data, used.ctypes.data),
                   "tables")
        return pt, used
