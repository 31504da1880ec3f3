"""Chunked causal prefill on the GPU (sfa_attn_prefill) against the oracle's
ggml-semantics path with the causal -INF mask."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import assert_close, f16_cols, golden, scatter_columns

pytestmark = pytest.mark.gpu


def build(oracle_mod, gpu, *, Hq, Hkv, hd, n_cached, T, page_size=256, seed=0, bf16=False, kv_type=1,
          k_boost=None):
    import torch
    from strataflow_amd import synth
    from strataflow_amd.paged_kv import PagedKV
    rng = np.random.default_rng(seed)
    n_kv = n_cached + T
    n_pages = (n_kv + page_size - 1) // page_size + 2
    pt = synth.page_tables(rng, [n_kv], page_size, n_pages)
    host = oracle_mod.HostPagedKv(Hkv, hd, page_size, kv_type, n_pages)
    pos = np.arange(n_kv, dtype=np.int32)
    q, k, v = synth.qkv(rng, n_kv, Hq, Hkv, hd, pos, 1e6, bf16=bf16)
    if k_boost is not None:
        # (period, phase, factor): keys at positions p % period == phase scaled
        period, phase, factor = k_boost
        k[pos % period == phase] *= factor
    assert host.append(k, v, np.zeros(n_kv, np.int32), pos, pt) == 0
    q = np.ascontiguousarray(q[n_cached:])
    dev = PagedKV(1, Hq, Hkv, hd, kv_type, page_size, n_pages, device=gpu)
    dev.k[0].copy_(torch.from_numpy(host.k))
    dev.v[0].copy_(torch.from_numpy(host.v))
    return host, dev, pt, q, n_kv


def run(dev, gpu, pt, q, q_pos0, kv_lo=0):
    import torch
    out = dev.prefill(0, torch.from_numpy(q).to(gpu), torch.from_numpy(pt[0]).to(gpu), q_pos0, kv_lo)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_prefill_golden(gpu, oracle_mod):
    import torch
    from strataflow_amd.paged_kv import PagedKV
    g = golden("attn_f16_mha_prefill")
    n_kv, Hkv, hd = g["k_f16"].shape
    Hq, T = int(g["n_head"]), g["q"].shape[0]
    ps, n_pages = 64, (n_kv + 63) // 64 + 2
    kp, pt = scatter_columns(f16_cols(g["k_f16"]), ps, n_pages, np.random.default_rng(2))
    vp, _ = scatter_columns(f16_cols(g["v_f16"]), ps, n_pages, np.random.default_rng(2))
    dev = PagedKV(1, Hq, Hkv, hd, 1, ps, n_pages, device=gpu)
    dev.k[0].copy_(torch.from_numpy(kp))
    dev.v[0].copy_(torch.from_numpy(vp))
    out = dev.prefill(0, torch.from_numpy(g["q"]).to(gpu), torch.from_numpy(pt[0]).to(gpu), n_kv - T,
                      int(g["kv_lo"]), scale=float(g["scale"]))
    out = out.cpu().numpy().reshape(g["exact"].shape)
    assert_close(out, g["ggml"], what="vs ggml golden")
    assert_close(out, g["exact"], what="vs exact golden")


@pytest.mark.parametrize("shape,n_cached,T,kv_lo", [
    ((32, 8, 128), 300, 256, 0),
    ((8, 4, 32), 50, 100, 0),
    ((16, 2, 128), 0, 64, 0),
    ((8, 8, 64), 70, 130, 0),
    ((32, 8, 128), 200, 150, 120),
    ((8, 1, 128), 10, 33, 0),
])
def test_prefill_vs_oracle(gpu, oracle_mod, shape, n_cached, T, kv_lo, page_size=256):
    Hq, Hkv, hd = shape
    host, dev, pt, q, n_kv = build(oracle_mod, gpu, Hq=Hq, Hkv=Hkv, hd=hd, n_cached=n_cached, T=T,
                                   page_size=page_size, seed=T + hd)
    out = run(dev, gpu, pt, q, n_cached, kv_lo)
    ref = host.attention(q[None], Hq, pt, np.array([n_kv], np.int32), np.array([kv_lo], np.int32),
                         T=T, mode=oracle_mod.GGML)[0].reshape(T, -1)
    assert_close(out, ref, what=f"{shape} T={T} vs ggml")
    ex = host.attention(q[None], Hq, pt, np.array([n_kv], np.int32), np.array([kv_lo], np.int32),
                        T=T, mode=oracle_mod.EXACT)[0].reshape(T, -1)
    assert_close(out, ex, what=f"{shape} T={T} vs exact")


def test_prefill_mixtral_chunk_2048_on_2048(gpu, oracle_mod):
    # full chunk: 2048 tokens at positions 2048..4095, bf16-representable
    # inputs; rows checked against the oracle's decode at n_kv = qpos + 1
    # (a causal row equals that decode, pinned by the oracle tests)
    Hq, Hkv, hd, n_cached, T = 32, 8, 128, 2048, 2048
    host, dev, pt, q, n_kv = build(oracle_mod, gpu, Hq=Hq, Hkv=Hkv, hd=hd, n_cached=n_cached, T=T,
                                   seed=3, bf16=True)
    out = run(dev, gpu, pt, q, n_cached)
    rows = np.unique(np.concatenate([[0, 1, 63, 64, 127, 128, T - 1],
                                     np.random.default_rng(5).integers(0, T, 9)]))
    for t in rows:
        ref = host.attention(q[t][None], Hq, pt, np.array([n_cached + t + 1], np.int32),
                             mode=oracle_mod.GGML)[0].reshape(-1)
        assert_close(out[t], ref, what=f"row {t}")
    assert np.all(np.isfinite(out))


@pytest.mark.parametrize("shape,n_cached,T,kv_lo,page_size", [
    ((16, 8, 64), 333, 97, 77, 128),     # unaligned window start, 128-position pages
    ((32, 8, 128), 1000, 300, 0, 64),    # smallest page the prefill tiles allow
    ((32, 4, 128), 129, 260, 0, 512),    # g = 8, 512-position pages
    ((4, 4, 32), 0, 1, 0, 64),           # one token, no history
])
def test_prefill_pages_and_windows(gpu, oracle_mod, shape, n_cached, T, kv_lo, page_size):
    test_prefill_vs_oracle(gpu, oracle_mod, shape, n_cached, T, kv_lo, page_size)


def test_prefill_rejects_unsupported(gpu, oracle_mod):
    import ctypes
    import torch
    from strataflow_amd import _lib
    host, dev, pt, q, n_kv = build(oracle_mod, gpu, Hq=8, Hkv=4, hd=32, n_cached=10, T=5, page_size=256)
    lib = _lib.load()
    d = dev.desc(0)
    tq = torch.from_numpy(q).to(gpu)
    out = torch.empty((5, 8 * 32), device=gpu)
    tpt = torch.from_numpy(pt[0]).to(gpu)
    s = torch.cuda.current_stream().cuda_stream
    # positions past the page table
    assert lib.sfa_attn_prefill(ctypes.byref(d), tq.data_ptr(), out.data_ptr(), tpt.data_ptr(), 1,
                                300, 5, 0, 0.17, s) == _lib.SFA_ERR_INVALID_ARGUMENT
    # a page size the 64-position tiles cannot cover
    d32 = _lib.SfaKvDesc()
    ctypes.memmove(ctypes.byref(d32), ctypes.byref(d), ctypes.sizeof(d))
    d32.page_size = 32
    assert lib.sfa_attn_prefill(ctypes.byref(d32), tq.data_ptr(), out.data_ptr(), tpt.data_ptr(),
                                int(pt.shape[1]), 10, 5, 0, 0.17, s) == _lib.SFA_ERR_UNSUPPORTED
    # a Q8_0 cache needs head_dim >= 64 (two 16-byte halves per block per lane)
    d8 = _lib.SfaKvDesc()
    ctypes.memmove(ctypes.byref(d8), ctypes.byref(d), ctypes.sizeof(d))
    d8.kv_type = 8
    assert lib.sfa_attn_prefill(ctypes.byref(d8), tq.data_ptr(), out.data_ptr(), tpt.data_ptr(),
                                int(pt.shape[1]), 10, 5, 0, 0.17, s) == _lib.SFA_ERR_UNSUPPORTED
    # T == 0 is a no-op
    assert lib.sfa_attn_prefill(ctypes.byref(d), tq.data_ptr(), out.data_ptr(), tpt.data_ptr(),
                                int(pt.shape[1]), 10, 0, 0, 0.17, s) == _lib.SFA_OK


# ---- F32 cache: f32 MFMA, no operand conversion; bars 50x tighter than parity
F32_MAX_ABS, F32_REL = 4e-5, 2e-5


@pytest.mark.parametrize("shape,n_cached,T,kv_lo,page_size", [
    ((32, 8, 128), 300, 256, 0, 256),
    ((8, 4, 32), 50, 100, 0, 64),
    ((8, 8, 64), 70, 130, 0, 128),
    ((16, 8, 64), 333, 97, 77, 128),     # unaligned window start
    ((32, 4, 128), 129, 260, 0, 512),    # g = 8
    ((4, 4, 32), 0, 1, 0, 64),           # one token, no history
])
def test_prefill_f32_vs_oracle(gpu, oracle_mod, shape, n_cached, T, kv_lo, page_size):
    Hq, Hkv, hd = shape
    host, dev, pt, q, n_kv = build(oracle_mod, gpu, Hq=Hq, Hkv=Hkv, hd=hd, n_cached=n_cached, T=T,
                                   page_size=page_size, seed=T + hd + 1, kv_type=0)
    out = run(dev, gpu, pt, q, n_cached, kv_lo)
    ref = host.attention(q[None], Hq, pt, np.array([n_kv], np.int32), np.array([kv_lo], np.int32),
                         T=T, mode=oracle_mod.GGML)[0].reshape(T, -1)
    assert_close(out, ref, max_abs=F32_MAX_ABS, rel_l2=F32_REL, what=f"f32 {shape} T={T} vs ggml")


def test_prefill_f32_rows_equal_f32_decode(gpu, oracle_mod):
    # a causal prefill row is the decode of its position (both f32 paths)
    import torch
    Hq, Hkv, hd, n_cached, T = 32, 8, 128, 512, 192
    host, dev, pt, q, n_kv = build(oracle_mod, gpu, Hq=Hq, Hkv=Hkv, hd=hd, n_cached=n_cached, T=T,
                                   seed=17, kv_type=0)
    out = run(dev, gpu, pt, q, n_cached)
    rows = [0, 1, 63, 64, 100, T - 1]
    tq = torch.from_numpy(q[rows]).to(gpu)
    tpt = torch.from_numpy(np.repeat(pt, len(rows), axis=0)).to(gpu)
    sl = torch.tensor([n_cached + t + 1 for t in rows], dtype=torch.int32, device=gpu)
    dec = dev.decode(0, tq, tpt, sl, n_kv).cpu().numpy().reshape(len(rows), -1)
    assert_close(out[rows], dec, max_abs=F32_MAX_ABS, rel_l2=F32_REL, what="f32 prefill rows vs decode")


# ---- Q8_0 cache: ggml's integer block dots (Q quantised to Q8_0), V
# dequantised to f16; gated against the ggml-semantics oracle at the parity bar
Q8_EXACT_ABS, Q8_EXACT_REL = 2e-2, 2e-2  # vs float64: the Q quantisation error


def test_prefill_q8_golden(gpu, oracle_mod):
    import torch
    from strataflow_amd.paged_kv import PagedKV
    g = golden("attn_q8_gqa2_prefill")
    n_kv, Hkv = g["k_q8"].shape[:2]
    hd = g["k_q8"].shape[2] // 34 * 32
    Hq, T = int(g["n_head"]), g["q"].shape[0]
    ps, n_pages = 64, (n_kv + 63) // 64 + 2
    kp, pt = scatter_columns(g["k_q8"].reshape(n_kv, -1), ps, n_pages, np.random.default_rng(3))
    vp, _ = scatter_columns(g["v_q8"].reshape(n_kv, -1), ps, n_pages, np.random.default_rng(3))
    dev = PagedKV(1, Hq, Hkv, hd, 8, ps, n_pages, device=gpu)
    dev.k[0].copy_(torch.from_numpy(kp))
    dev.v[0].copy_(torch.from_numpy(vp))
    q_pos0 = int(g["qpos"][0])
    out = dev.prefill(0, torch.from_numpy(g["q"]).to(gpu), torch.from_numpy(pt[0]).to(gpu), q_pos0,
                      int(g["kv_lo"]), scale=float(g["scale"]))
    out = out.cpu().numpy().reshape(g["exact"].shape)
    assert_close(out, g["ggml"], what="q8 prefill vs ggml golden")
    assert_close(out, g["exact"], max_abs=Q8_EXACT_ABS, rel_l2=Q8_EXACT_REL, what="q8 prefill vs exact golden")


@pytest.mark.parametrize("shape,n_cached,T,kv_lo,page_size", [
    ((32, 8, 128), 300, 256, 0, 256),
    ((8, 8, 64), 70, 130, 0, 128),
    ((16, 8, 64), 333, 97, 77, 128),     # unaligned window start
    ((32, 4, 128), 129, 260, 0, 512),    # g = 8
    ((16, 16, 128), 1000, 64, 0, 64),    # g = 1, smallest page the tiles allow
    ((8, 4, 64), 0, 1, 0, 64),           # one token, no history
])
def test_prefill_q8_vs_oracle(gpu, oracle_mod, shape, n_cached, T, kv_lo, page_size):
    Hq, Hkv, hd = shape
    host, dev, pt, q, n_kv = build(oracle_mod, gpu, Hq=Hq, Hkv=Hkv, hd=hd, n_cached=n_cached, T=T,
                                   page_size=page_size, seed=T + hd + 8, kv_type=8)
    out = run(dev, gpu, pt, q, n_cached, kv_lo)
    ref = host.attention(q[None], Hq, pt, np.array([n_kv], np.int32), np.array([kv_lo], np.int32),
                         T=T, mode=oracle_mod.GGML)[0].reshape(T, -1)
    assert_close(out, ref, what=f"q8 {shape} T={T} vs ggml")
    ex = host.attention(q[None], Hq, pt, np.array([n_kv], np.int32), np.array([kv_lo], np.int32),
                        T=T, mode=oracle_mod.EXACT)[0].reshape(T, -1)
    assert_close(out, ex, max_abs=Q8_EXACT_ABS, rel_l2=Q8_EXACT_REL, what=f"q8 {shape} T={T} vs exact")


def test_prefill_q8_rows_match_q8_decode(gpu, oracle_mod):
    # a causal prefill row and the Q8_0 decode at its position share the
    # integer QK arithmetic; they differ only in P*V accumulation order
    import torch
    Hq, Hkv, hd, n_cached, T = 32, 8, 128, 700, 150
    host, dev, pt, q, n_kv = build(oracle_mod, gpu, Hq=Hq, Hkv=Hkv, hd=hd, n_cached=n_cached, T=T,
                                   seed=19, kv_type=8)
    out = run(dev, gpu, pt, q, n_cached)
    rows = [0, 1, 63, 64, 149]
    tq = torch.from_numpy(q[rows]).to(gpu)
    tpt = torch.from_numpy(np.repeat(pt, len(rows), axis=0)).to(gpu)
    sl = torch.tensor([n_cached + t + 1 for t in rows], dtype=torch.int32, device=gpu)
    dec = dev.decode(0, tq, tpt, sl, n_kv).cpu().numpy().reshape(len(rows), -1)
    assert_close(out[rows], dec, max_abs=1e-3, rel_l2=5e-4, what="q8 prefill rows vs decode")


@pytest.mark.parametrize("kv_type", [0, 1, 8])
def test_prefill_late_rescale(gpu, oracle_mod, kv_type):
    # every 200th key from position 150 scaled x5: each row's first 64-position
    # tile holds ordinary scores and a later tile scores far above them, so the
    # lazy reference moves and O and l are rescaled after the first tile
    Hq, Hkv, hd, n_cached, T = 32, 8, 128, 1500, 256
    host, dev, pt, q, n_kv = build(oracle_mod, gpu, Hq=Hq, Hkv=Hkv, hd=hd, n_cached=n_cached, T=T,
                                   seed=500 + kv_type, kv_type=kv_type, k_boost=(200, 150, 5.0))
    out = run(dev, gpu, pt, q, n_cached)
    ref = host.attention(q[None], Hq, pt, np.array([n_kv], np.int32), None,
                         T=T, mode=oracle_mod.GGML)[0].reshape(T, -1)
    if kv_type == 0:
        assert_close(out, ref, max_abs=F32_MAX_ABS, rel_l2=F32_REL, what="f32 late rescale vs ggml")
    else:
        assert_close(out, ref, what=f"type {kv_type} late rescale vs ggml")


@pytest.mark.parametrize("kv_type", [0, 1, 8])
@pytest.mark.parametrize("bad", ["missing", "out_of_pool"])
def test_prefill_invalid_first_page(gpu, oracle_mod, kv_type, bad):
    # the history's first page has no valid id (-1, or an id past the pool):
    # its tiles arrive as zeros, are masked and contribute nothing, so every
    # row equals attention over the positions from the second page on (the
    # same call with kv_lo at that page's first position); nothing is read out
    # of bounds
    ps, n_cached, T = 256, 600, 100
    host, dev, pt, q, n_kv = build(oracle_mod, gpu, Hq=32, Hkv=8, hd=128, n_cached=n_cached, T=T,
                                   page_size=ps, seed=31 + kv_type, kv_type=kv_type)
    bad_pt = pt.copy()
    bad_pt[0, 0] = -1 if bad == "missing" else dev.n_pages + 100
    out = run(dev, gpu, bad_pt, q, n_cached)
    ref = host.attention(q[None], 32, pt, np.array([n_kv], np.int32), np.array([ps], np.int32),
                         T=T, mode=oracle_mod.GGML)[0].reshape(T, -1)
    assert np.all(np.isfinite(out))
    assert_close(out, ref, what=f"type {kv_type}, {bad} first page")
