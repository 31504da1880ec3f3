"""Seeded synthetic inputs for the attention path.

Q, K, V are N(0, 1) float32; Q and K get RoPE NORMAL at their positions (the
reference stores K post-RoPE and V raw, src/model/engine/engine.cpp:1877-1897).
Pages of a sequence are placed by a seeded permutation of the pool, so logical
order never equals physical order.
"""
from __future__ import annotations

import ctypes
import ctypes.util

import numpy as np


def powf(x: float, y: float) -> np.float32:
    """C's powf, the f32 pow ggml uses for theta_scale; the theta recurrence
    amplifies a one-ulp difference in its factor, so numpy's float32 power is
    not used for it."""
    global _libm
    if _libm is None:
        _libm = ctypes.CDLL(ctypes.util.find_library("m"))
        _libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
        _libm.powf.restype = ctypes.c_float
    return np.float32(_libm.powf(float(x), float(y)))


_libm = None


def rope_normal(x: np.ndarray, pos: np.ndarray, freq_base: float) -> np.ndarray:
    """RoPE NORMAL (ggml_rope_ext mode 0, freq_scale 1, ext_factor 0,
    attn_factor 1; engine.cpp:1892-1897) on x [n_tok, n_heads, head_dim].

    Adjacent pairs (x[2i], x[2i+1]) rotate by theta_i = pos * base^(-2i/hd);
    theta follows ggml's float32 recurrence theta *= base^(-2/hd)."""
    x = np.asarray(x, dtype=np.float32)
    n_tok, _, hd = x.shape
    theta_scale = powf(np.float32(freq_base), np.float32(-2.0) / np.float32(hd))
    theta = np.empty((n_tok, hd // 2), dtype=np.float32)
    cur = np.asarray(pos, dtype=np.float32).copy()
    for i in range(hd // 2):
        theta[:, i] = cur
        cur = (cur * theta_scale).astype(np.float32)
    c = np.cos(theta)[:, None, :]
    s = np.sin(theta)[:, None, :]
    x0 = x[..., 0::2]
    x1 = x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x0 * s + x1 * c
    return out


def qkv(rng: np.random.Generator, n_tok: int, n_head: int, n_head_kv: int, head_dim: int,
        pos: np.ndarray, freq_base: float = 1e6, bf16: bool = False):
    """Q [n_tok, Hq, hd], K, V [n_tok, Hkv, hd]: N(0,1), RoPE on Q and K."""
    q = rng.standard_normal((n_tok, n_head, head_dim), dtype=np.float32)
    k = rng.standard_normal((n_tok, n_head_kv, head_dim), dtype=np.float32)
    v = rng.standard_normal((n_tok, n_head_kv, head_dim), dtype=np.float32)
    if bf16:
        q, k, v = (bf16_round(t) for t in (q, k, v))
    q = rope_normal(q, pos, freq_base)
    k = rope_normal(k, pos, freq_base)
    if bf16:
        q, k = bf16_round(q), bf16_round(k)
    return q, k, v


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Rounds float32 to the nearest bfloat16-representable value (RNE)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def page_tables(rng: np.random.Generator, seq_lens, page_size: int, n_pages: int,
                max_pages: int | None = None) -> np.ndarray:
    """Per-sequence page tables [B, max_pages] drawing distinct physical pages
    from a seeded permutation of the pool; unused entries are -1."""
    need = [(int(n) + page_size - 1) // page_size for n in seq_lens]
    if max_pages is None:
        max_pages = max(max(need), 1)
    if sum(need) > n_pages:
        raise ValueError(f"pool of {n_pages} pages cannot hold {sum(need)}")
    perm = rng.permutation(n_pages).astype(np.int32)
    pt = np.full((len(seq_lens), max_pages), -1, dtype=np.int32)
    off = 0
    for b, k in enumerate(need):
        pt[b, :k] = perm[off:off + k]
        off += k
    return pt


def rope_normal_torch(x, pos, freq_base: float):
    """rope_normal on a torch tensor x [n_tok, n_heads, head_dim] (device)."""
    import torch
    n_tok, _, hd = x.shape
    theta_scale = float(powf(np.float32(freq_base), np.float32(-2.0) / np.float32(hd)))
    i = torch.arange(hd // 2, device=x.device, dtype=torch.float64)
    theta = (pos.to(torch.float64)[:, None] * torch.pow(torch.tensor(theta_scale, dtype=torch.float64,
                                                                      device=x.device), i)).float()
    c, s = torch.cos(theta)[:, None, :], torch.sin(theta)[:, None, :]
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x0 * s + x1 * c
    return out
