"""Shared helpers of the test suite: golden fixtures, page layout, tolerances."""
from __future__ import annotations

from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"

# parity bar for attention outputs (f16 KV and Q8_0 KV alike)
MAX_ABS = 2e-3
REL_L2 = 1e-3


def golden(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def errors(out: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    out = np.asarray(out, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    max_abs = float(np.max(np.abs(out - ref))) if out.size else 0.0
    den = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(out - ref) / den) if den > 0 else float(np.linalg.norm(out - ref))
    return max_abs, rel


def assert_close(out, ref, max_abs=MAX_ABS, rel_l2=REL_L2, what=""):
    ma, rl = errors(out, ref)
    assert ma <= max_abs and rl <= rel_l2, f"{what}: max_abs {ma:.3e} (<= {max_abs}), rel_l2 {rl:.3e} (<= {rel_l2})"
    return ma, rl


def scatter_columns(cols: np.ndarray, page_size: int, n_pages: int, rng: np.random.Generator,
                    B: int = 1, max_pages: int | None = None):
    """Lays per-sequence column bytes [B][n_kv][Hkv*row_bytes] (or [n_kv][...])
    into a pool [n_pages, page_bytes] through seeded shuffled page tables.
    Returns (pool, page_table [B, max_pages])."""
    cols = np.asarray(cols, np.uint8)
    if cols.ndim == 2:
        cols = cols[None]
    Bc, n_kv, col_bytes = cols.shape
    need = (n_kv + page_size - 1) // page_size
    mp = max_pages or need
    perm = rng.permutation(n_pages).astype(np.int32)
    pt = np.full((Bc, mp), -1, np.int32)
    pool = np.zeros((n_pages, page_size * col_bytes), np.uint8)
    for b in range(Bc):
        for lp in range(need):
            pid = int(perm[b * need + lp])
            pt[b, lp] = pid
            chunk = cols[b, lp * page_size:(lp + 1) * page_size].reshape(-1)
            pool[pid, :chunk.size] = chunk
    return pool, pt


def f16_cols(x: np.ndarray) -> np.ndarray:
    """[n_kv, Hkv, hd] float16 values -> column bytes [n_kv, Hkv*hd*2]."""
    x = np.ascontiguousarray(x, np.float16)
    return x.view(np.uint8).reshape(x.shape[0], -1)


class Case:
    """One seeded paged-cache workload held identically on the host (oracle
    pools) and on the device (PagedKV pools): the device bytes are a copy of
    the oracle's appended bytes."""

    def __init__(self, oracle_mod, *, seq_lens, n_head=32, n_head_kv=8, head_dim=128,
                 page_size=256, kv_type=1, seed=0, extra_pages=3, kv_lo=None, freq_base=1e6,
                 n_layer=1, device="cuda", k_boost=None):
        import torch

        from strataflow_amd import synth
        from strataflow_amd.paged_kv import PagedKV

        rng = np.random.default_rng(seed)
        self.seq_lens = np.asarray(seq_lens, np.int32)
        B = self.B = int(self.seq_lens.size)
        self.n_head, self.n_head_kv, self.head_dim = n_head, n_head_kv, head_dim
        self.page_size, self.kv_type = page_size, kv_type
        need = sum((int(n) + page_size - 1) // page_size for n in self.seq_lens)
        self.n_pages = need + extra_pages
        self.max_pages = max(max((int(n) + page_size - 1) // page_size for n in self.seq_lens), 1)
        self.page_table = synth.page_tables(rng, self.seq_lens, page_size, self.n_pages, self.max_pages)
        self.host = oracle_mod.HostPagedKv(n_head_kv, head_dim, page_size, kv_type, self.n_pages)
        for b in range(B):
            n = int(self.seq_lens[b])
            if n == 0:
                continue
            pos = np.arange(n, dtype=np.int32)
            _, k, v = synth.qkv(rng, n, 1, n_head_kv, head_dim, pos, freq_base)
            if k_boost is not None:
                # (period, phase, factor): keys at positions p % period ==
                # phase scaled, so later tiles hold scores far above earlier ones
                period, phase, factor = k_boost
                k[pos % period == phase] *= factor
            assert self.host.append(k, v, np.full(n, b, np.int32), pos, self.page_table) == 0
        qpos = np.maximum(self.seq_lens - 1, 0)
        self.q = np.stack([synth.qkv(rng, 1, n_head, n_head_kv, head_dim, np.array([p]), freq_base)[0][0]
                           for p in qpos]).astype(np.float32)
        self.kv_lo = None if kv_lo is None else np.asarray(kv_lo, np.int32)
        self.dev = PagedKV(n_layer, n_head, n_head_kv, head_dim, kv_type, page_size, self.n_pages,
                           device=device)
        for layer in range(n_layer):
            self.dev.k[layer].copy_(torch.from_numpy(self.host.k[: self.n_pages]))
            self.dev.v[layer].copy_(torch.from_numpy(self.host.v[: self.n_pages]))
        self.t_pt = torch.from_numpy(self.page_table).to(device)
        self.t_sl = torch.from_numpy(self.seq_lens).to(device)
        self.t_lo = None if self.kv_lo is None else torch.from_numpy(self.kv_lo).to(device)
        self.t_q = torch.from_numpy(self.q).to(device)

    def oracle(self, mode):
        return self.host.attention(self.q, self.n_head, self.page_table, self.seq_lens, self.kv_lo,
                                   mode=mode).reshape(self.B, -1)

    def decode(self, layer=0, max_seq_len=None, **kw):
        import torch
        out = self.dev.decode(layer, self.t_q, self.t_pt, self.t_sl,
                              int(max_seq_len or max(int(self.seq_lens.max()), 1)),
                              kv_lo=self.t_lo, **kw)
        torch.cuda.synchronize()
        return out.cpu().numpy()


class OracleAttention:
    """The attention node on the CPU oracle, with the call shape of
    strataflow_amd.tiny_moe.HipAttention: per layer a host paged cache (f16 by
    default), append at pos0.., attention of the T new tokens (causal)."""

    def __init__(self, oracle_mod, cfg, n_ctx: int, mode: int, kv_type: int | None = None):
        self.o, self.cfg, self.mode = oracle_mod, cfg, mode
        n_pages = (n_ctx + cfg.page_size - 1) // cfg.page_size
        self.pt = np.arange(n_pages, dtype=np.int32)[None]
        kt = oracle_mod.KV_F16 if kv_type is None else kv_type
        self.host = [oracle_mod.HostPagedKv(cfg.n_head_kv, cfg.head_dim, cfg.page_size, kt, n_pages)
                     for _ in range(cfg.n_layer)]

    def __call__(self, layer, q, k, v, pos0):
        T = q.shape[0]
        pos = np.arange(pos0, pos0 + T, dtype=np.int32)
        h = self.host[layer]
        assert h.append(k, v, np.zeros(T, np.int32), pos, self.pt) == 0
        out = h.attention(np.ascontiguousarray(q, np.float32)[None], self.cfg.n_head, self.pt,
                          np.array([pos0 + T], np.int32), T=T, mode=self.mode)
        return out.reshape(T, -1)
