"""Device-side paged KV cache and the attention entry points over the C ABI.

``PagedKV`` owns per-layer K/V page pools in HBM (torch device memory is only
the allocator here) and calls libsfa.so for the append, decode and prefill.
It mirrors the engine's KV ownership (src/model/engine/engine.cpp:1253-1286:
per-layer K and V caches owned for the engine's lifetime) with pages in place
of one tensor per layer.  Page tables, seq_len and kv_lo are device int32
tensors, so a call does no host-to-device copy.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from ._lib import SFA_KV_F16, SFA_KV_F32, SFA_KV_Q8_0, SfaKvDesc

__all__ = ["PagedKV", "row_bytes", "SFA_KV_F32", "SFA_KV_F16", "SFA_KV_Q8_0"]


def row_bytes(kv_type: int, head_dim: int) -> int:
    if kv_type == SFA_KV_F32:
        return head_dim * 4
    if kv_type == SFA_KV_F16:
        return head_dim * 2
    if kv_type == SFA_KV_Q8_0:
        return head_dim // 32 * 34
    raise ValueError(f"unsupported kv type {kv_type}")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


class PagedKV:
    """Per-layer paged K/V pools: k[layer] is [n_pages, page_bytes] uint8."""

    def __init__(self, n_layer: int, n_head: int, n_head_kv: int, head_dim: int, kv_type: int,
                 page_size: int, n_pages: int, device: str | torch.device = "cuda",
                 n_cold_pages: int = 0):
        self.n_layer, self.n_head, self.n_head_kv = n_layer, n_head, n_head_kv
        self.head_dim, self.kv_type, self.page_size = head_dim, kv_type, page_size
        self.n_pages, self.n_cold_pages = n_pages, n_cold_pages
        self.device = torch.device(device)
        self.page_bytes = row_bytes(kv_type, head_dim) * n_head_kv * page_size
        self.k = torch.zeros((n_layer, n_pages, self.page_bytes), dtype=torch.uint8, device=self.device)
        self.v = torch.zeros_like(self.k)
        if n_cold_pages:
            # host-pinned cold pool, readable by the GPU over the host link
            self.k_cold = torch.zeros((n_layer, n_cold_pages, self.page_bytes), dtype=torch.uint8,
                                      pin_memory=True)
            self.v_cold = torch.zeros_like(self.k_cold, pin_memory=True)
        else:
            self.k_cold = self.v_cold = None
        self._ws = None
        self._ws_need = {}
        self._descs = [self._make_desc(layer) for layer in range(n_layer)]
        lib = _lib.load()
        _lib.check(lib.sfa_kv_desc_check(ctypes.byref(self.desc(0))), "kv descriptor")

    def desc(self, layer: int) -> SfaKvDesc:
        """The sfa_kv_desc of one layer (built once; pool pointers are stable)."""
        return self._descs[layer]

    def _make_desc(self, layer: int) -> SfaKvDesc:
        d = SfaKvDesc()
        d.n_head, d.n_head_kv, d.head_dim = self.n_head, self.n_head_kv, self.head_dim
        d.page_size, d.kv_type, d.n_pages = self.page_size, self.kv_type, self.n_pages
        d.k_pages = self.k[layer].data_ptr()
        d.v_pages = self.v[layer].data_ptr()
        d.n_cold_pages = self.n_cold_pages
        if self.n_cold_pages:
            d.k_cold = self.k_cold[layer].data_ptr()
            d.v_cold = self.v_cold[layer].data_ptr()
        return d

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)

    # -- workspace -------------------------------------------------------------
    def workspace(self, B: int, max_seq_len: int) -> torch.Tensor:
        lib = _lib.load()
        need = self._ws_need.get((B, max_seq_len))
        if need is None:
            need = lib.sfa_decode_workspace_bytes(ctypes.byref(self.desc(0)), B, max_seq_len)
            if need == 0:
                raise ValueError("invalid decode shape")
            self._ws_need[(B, max_seq_len)] = need
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
            _lib.check(lib.sfa_workspace_init(self._ws.data_ptr(), self._ws.numel(), _stream(None)),
                       "workspace init")
        return self._ws

    # -- entry points ------------------------------------------------------------
    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor, seq: torch.Tensor,
               pos: torch.Tensor, page_table: torch.Tensor, stream=None) -> None:
        """k, v [n_tok, Hkv, hd] f32 on device; seq/pos [n_tok] int32."""
        n_tok = int(seq.numel())
        assert k.is_contiguous() and v.is_contiguous() and k.dtype == torch.float32
        assert k.shape == (n_tok, self.n_head_kv, self.head_dim) and v.shape == k.shape
        lib = _lib.load()
        d = self.desc(layer)
        _lib.check(lib.sfa_kv_append(ctypes.byref(d), k.data_ptr(), v.data_ptr(), seq.data_ptr(),
                                     pos.data_ptr(), n_tok, page_table.data_ptr(),
                                     int(page_table.shape[-1]), _stream(stream)), "sfa_kv_append")

    def rope_append(self, layer: int, q: torch.Tensor | None, k: torch.Tensor, v: torch.Tensor,
                    seq: torch.Tensor, pos: torch.Tensor, page_table: torch.Tensor, freq_base: float,
                    stream=None) -> None:
        """Fused RoPE NORMAL + append: q [n_tok, Hq, hd] (rotated in place, or
        None), k pre-RoPE and v raw [n_tok, Hkv, hd] f32 on device."""
        n_tok = int(seq.numel())
        assert k.is_contiguous() and v.is_contiguous() and k.dtype == torch.float32
        assert k.shape == (n_tok, self.n_head_kv, self.head_dim) and v.shape == k.shape
        if q is not None:
            assert q.is_contiguous() and q.dtype == torch.float32
            assert q.shape == (n_tok, self.n_head, self.head_dim)
        lib = _lib.load()
        d = self.desc(layer)
        _lib.check(lib.sfa_rope_kv_append(ctypes.byref(d), _ptr(q), k.data_ptr(), v.data_ptr(),
                                          seq.data_ptr(), pos.data_ptr(), n_tok, page_table.data_ptr(),
                                          int(page_table.shape[-1]), float(freq_base), _stream(stream)),
                   "sfa_rope_kv_append")

    def qkv_rope_append(self, layer: int, w_qkv: torch.Tensor, x: torch.Tensor, seq: torch.Tensor,
                        pos: torch.Tensor, page_table: torch.Tensor, freq_base: float,
                        q: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """The stacked Q/K/V product of x [n_tok, n_embd] (w_qkv
        [(Hq + 2 Hkv) hd, n_embd], f32 or f16), RoPE and the append in one
        launch -> q [n_tok, Hq, hd] rotated."""
        from .layer import weight_type
        n_tok = int(seq.numel())
        n_embd = int(x.shape[-1])
        assert x.is_contiguous() and x.dtype == torch.float32 and x.shape == (n_tok, n_embd)
        assert w_qkv.is_contiguous() and w_qkv.shape == ((self.n_head + 2 * self.n_head_kv) * self.head_dim, n_embd)
        if q is None:
            q = torch.empty((n_tok, self.n_head, self.head_dim), dtype=torch.float32, device=x.device)
        assert q.is_contiguous() and q.dtype == torch.float32 and q.shape == (n_tok, self.n_head, self.head_dim)
        lib = _lib.load()
        d = self.desc(layer)
        _lib.check(lib.sfa_qkv_rope_kv_append(ctypes.byref(d), w_qkv.data_ptr(), weight_type(w_qkv), x.data_ptr(),
                                              n_embd, q.data_ptr(), seq.data_ptr(), pos.data_ptr(), n_tok,
                                              page_table.data_ptr(), int(page_table.shape[-1]), float(freq_base),
                                              _stream(stream)),
                   "sfa_qkv_rope_kv_append")
        return q

    def decode(self, layer: int, q: torch.Tensor, page_table: torch.Tensor, seq_len: torch.Tensor,
               max_seq_len: int, kv_lo: torch.Tensor | None = None, out: torch.Tensor | None = None,
               scale: float | None = None, stream=None, split_end_event=None) -> torch.Tensor:
        """q [B, Hq, hd] f32 -> out [B, Hq*hd] f32.  With `split_end_event` the
        two passes are issued separately and the event is recorded between
        them (timing of the split-K pass)."""
        B = int(seq_len.numel())
        assert q.is_contiguous() and q.dtype == torch.float32
        assert q.shape == (B, self.n_head, self.head_dim)
        assert page_table.dtype == torch.int32 and page_table.shape[0] == B
        if out is None:
            out = torch.empty((B, self.n_head * self.head_dim), dtype=torch.float32, device=q.device)
        ws = self.workspace(B, max_seq_len)
        lib = _lib.load()
        d = self._descs[layer]
        args = (ctypes.byref(d), q.data_ptr(), out.data_ptr(), page_table.data_ptr(),
                int(page_table.shape[1]), seq_len.data_ptr(), _ptr(kv_lo), B, int(max_seq_len),
                float(scale if scale is not None else self.scale), ws.data_ptr(), ws.numel(),
                _stream(stream))
        if split_end_event is None:
            _lib.check(lib.sfa_attn_decode(*args), "sfa_attn_decode")
        else:
            _lib.check(lib.sfa_attn_decode_split(*args), "sfa_attn_decode_split")
            split_end_event.record()
            _lib.check(lib.sfa_attn_decode_merge(*args), "sfa_attn_decode_merge")
        return out

    def decode_append(self, layer: int, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor,
                      page_table: torch.Tensor, seq_len: torch.Tensor, max_seq_len: int,
                      kv_lo: torch.Tensor | None = None, out: torch.Tensor | None = None,
                      scale: float | None = None, stream=None) -> torch.Tensor:
        """Appends each sequence's new token (k, v [B, Hkv, hd] f32, token b at
        position seq_len[b] - 1) and attends: out [B, Hq*hd] f32.  F16 or F32 pools."""
        B = int(seq_len.numel())
        assert q.is_contiguous() and q.dtype == torch.float32 and q.shape == (B, self.n_head, self.head_dim)
        for t in (k, v):
            assert t.is_contiguous() and t.dtype == torch.float32 and t.shape == (B, self.n_head_kv, self.head_dim)
        assert page_table.dtype == torch.int32 and page_table.shape[0] == B
        if out is None:
            out = torch.empty((B, self.n_head * self.head_dim), dtype=torch.float32, device=q.device)
        ws = self.workspace(B, max_seq_len)
        lib = _lib.load()
        _lib.check(lib.sfa_attn_decode_append(ctypes.byref(self._descs[layer]), k.data_ptr(), v.data_ptr(),
                                              q.data_ptr(), out.data_ptr(), page_table.data_ptr(),
                                              int(page_table.shape[1]), seq_len.data_ptr(), _ptr(kv_lo), B,
                                              int(max_seq_len),
                                              float(scale if scale is not None else self.scale),
                                              ws.data_ptr(), ws.numel(), _stream(stream)),
                   "sfa_attn_decode_append")
        return out

    def prefill(self, layer: int, q: torch.Tensor, page_table: torch.Tensor, q_pos0: int,
                kv_lo: int = 0, out: torch.Tensor | None = None, scale: float | None = None,
                stream=None) -> torch.Tensor:
        """q [T, Hq, hd] f32 of one sequence -> out [T, Hq*hd] f32."""
        T = int(q.shape[0])
        assert q.is_contiguous() and q.dtype == torch.float32
        if out is None:
            out = torch.empty((T, self.n_head * self.head_dim), dtype=torch.float32, device=q.device)
        lib = _lib.load()
        d = self.desc(layer)
        _lib.check(lib.sfa_attn_prefill(ctypes.byref(d), q.data_ptr(), out.data_ptr(),
                                        page_table.data_ptr(), int(page_table.numel()),
                                        int(q_pos0), T, int(kv_lo),
                                        float(scale if scale is not None else self.scale),
                                        _stream(stream)), "sfa_attn_prefill")
        return out
