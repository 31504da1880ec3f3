"""Decode attention on the GPU (sfa_attn_decode through the C ABI) against the
oracle: ggml CPU semantics (max-abs <= 2e-3, rel-L2 <= 1e-3) and float64."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import Case, assert_close, errors, f16_cols, golden, scatter_columns

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["attn_f16_gqa2_decode", "attn_f16_gqa4_window"])
def test_decode_golden(gpu, oracle_mod, name):
    import torch
    from strataflow_amd.paged_kv import PagedKV
    g = golden(name)
    n_kv, Hkv, hd = g["k_f16"].shape
    Hq = int(g["n_head"])
    ps, n_pages = 32, (n_kv + 31) // 32 + 3
    kp, pt = scatter_columns(f16_cols(g["k_f16"]), ps, n_pages, np.random.default_rng(1))
    vp, _ = scatter_columns(f16_cols(g["v_f16"]), ps, n_pages, np.random.default_rng(1))
    dev = PagedKV(1, Hq, Hkv, hd, 1, ps, n_pages, device=gpu)
    dev.k[0].copy_(torch.from_numpy(kp))
    dev.v[0].copy_(torch.from_numpy(vp))
    q = torch.from_numpy(g["q"]).to(gpu)  # [1, Hq, hd]
    lo = torch.tensor([int(g["kv_lo"])], dtype=torch.int32, device=gpu)
    out = dev.decode(0, q, torch.from_numpy(pt).to(gpu), torch.tensor([n_kv], dtype=torch.int32, device=gpu),
                     n_kv, kv_lo=lo, scale=float(g["scale"]))
    out = out.cpu().numpy().reshape(g["exact"].shape)
    assert_close(out, g["ggml"], what="vs ggml golden")
    assert_close(out, g["exact"], what="vs exact golden")


@pytest.mark.parametrize("shape", [(32, 8, 128), (8, 4, 32), (8, 8, 64), (16, 2, 128), (16, 16, 128)])
@pytest.mark.parametrize("n_kv", [1, 31, 33, 257, 1000])
def test_decode_shapes(gpu, oracle_mod, shape, n_kv):
    Hq, Hkv, hd = shape
    c = Case(oracle_mod, seq_lens=[n_kv], n_head=Hq, n_head_kv=Hkv, head_dim=hd, page_size=64,
             seed=n_kv + hd)
    out = c.decode()
    assert_close(out, c.oracle(oracle_mod.GGML), what=f"{shape} n_kv={n_kv} vs ggml")
    assert_close(out, c.oracle(oracle_mod.EXACT), what=f"{shape} n_kv={n_kv} vs exact")


def test_decode_mixtral_ctx4096(gpu, oracle_mod):
    # Mixtral attention shape at context 4096, 256-token pages shuffled
    c = Case(oracle_mod, seq_lens=[4096], seed=42)
    out = c.decode()
    ma, rl = assert_close(out, c.oracle(oracle_mod.GGML), what="ctx4096 vs ggml")
    print(f"ctx4096 f16: max_abs {ma:.3e} rel_l2 {rl:.3e}")
    assert_close(out, c.oracle(oracle_mod.EXACT), what="ctx4096 vs exact")


def test_decode_batch_varlen_window(gpu, oracle_mod):
    # B=5 sequences sharing one pool, different lengths; two use a sliding
    # window start (kv_lo), one is empty (all masked -> zeros)
    seq = [700, 1, 4096, 300, 0]
    lo = [0, 0, 3000, 290, 0]
    c = Case(oracle_mod, seq_lens=seq, kv_lo=lo, seed=7)
    out = c.decode(max_seq_len=4096)
    ref = c.oracle(oracle_mod.GGML)
    assert_close(out, ref, what="varlen vs ggml")
    assert np.all(out[4] == 0)


@pytest.mark.parametrize("kv_type,page_size", [(1, 32), (1, 512), (8, 32), (8, 512)])
def test_decode_page_sizes_varlen(gpu, oracle_mod, kv_type, page_size):
    # smallest and a large page size, a batch with an empty sequence, a
    # one-token sequence and sliding-window starts inside a page
    seq = [0, 1, 2500, 777, 64]
    lo = [0, 0, 1999, 13, 32]
    c = Case(oracle_mod, seq_lens=seq, kv_lo=lo, kv_type=kv_type, page_size=page_size,
             seed=page_size + kv_type)
    out = c.decode(max_seq_len=2500)
    assert_close(out, c.oracle(oracle_mod.GGML), what=f"type {kv_type} page {page_size}")
    assert np.all(out[0] == 0)


def test_decode_page_placement_bit_identical(gpu, oracle_mod):
    # paged == contiguous, bit for bit (the reference's test_kv_paging.cpp:243
    # invariant): same logical cache, different physical page orders
    import torch
    c = Case(oracle_mod, seq_lens=[2000], seed=9, extra_pages=6)
    base = c.decode()
    n_pages = c.n_pages
    for seed in (1, 2):
        perm = np.random.default_rng(seed).permutation(n_pages).astype(np.int32)
        # move every physical page p to perm[p]
        k2 = torch.empty_like(c.dev.k[0])
        v2 = torch.empty_like(c.dev.v[0])
        k2[torch.from_numpy(perm).long().to(gpu)] = c.dev.k[0]
        v2[torch.from_numpy(perm).long().to(gpu)] = c.dev.v[0]
        c.dev.k[0].copy_(k2)
        c.dev.v[0].copy_(v2)
        pt = c.page_table.copy()
        valid = pt >= 0
        pt[valid] = perm[pt[valid]]
        c.page_table = pt
        c.t_pt = torch.from_numpy(pt).to(gpu)
        out = c.decode()
        assert np.array_equal(out.view(np.uint32), base.view(np.uint32))


def test_decode_deterministic_and_workspace_reuse(gpu, oracle_mod):
    c = Case(oracle_mod, seq_lens=[3000, 1500], seed=11)
    a = c.decode()
    b = c.decode()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # a smaller call on the same (grown) workspace, then the big one again
    small = Case(oracle_mod, seq_lens=[100], seed=12)
    small.dev._ws = c.dev._ws
    assert_close(small.decode(), small.oracle(oracle_mod.GGML), what="small after big")
    assert np.array_equal(c.decode().view(np.uint32), a.view(np.uint32))


def test_decode_bad_page_id_skipped(gpu, oracle_mod):
    # an out-of-pool page id is caught by the kernel's own bounds check: that
    # tile contributes nothing and nothing is read out of bounds
    import torch
    c = Case(oracle_mod, seq_lens=[600], page_size=256, seed=13)
    pt = c.page_table.copy()
    pt[0, 1] = c.n_pages + 100
    c.t_pt = torch.from_numpy(pt).to(gpu)
    out = c.decode()
    assert np.all(np.isfinite(out))


def test_decode_rejects_small_workspace(gpu, oracle_mod):
    import ctypes
    import torch
    from strataflow_amd import _lib
    c = Case(oracle_mod, seq_lens=[100], seed=14)
    lib = _lib.load()
    d = c.dev.desc(0)
    out = torch.empty((1, 32 * 128), device=gpu)
    ws = torch.zeros(16, dtype=torch.uint8, device=gpu)
    rc = lib.sfa_attn_decode(ctypes.byref(d), c.t_q.data_ptr(), out.data_ptr(), c.t_pt.data_ptr(),
                             c.max_pages, c.t_sl.data_ptr(), None, 1, 100, 0.088, ws.data_ptr(), 16,
                             torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.SFA_ERR_INVALID_ARGUMENT


# ---- Q8_0 KV ------------------------------------------------------------------
# The gate is the ggml-semantics oracle (Q quantised to Q8_0, integer block
# dots, the reference's own CPU arithmetic for a Q8_0 cache); the float64
# exact-dequant reading differs from ggml's by the Q quantisation error
# (about 0.5% rel-L2 at N(0,1) inputs), so against it the bound is 2e-2.
Q8_EXACT_REL = 2e-2
Q8_EXACT_ABS = 2e-2


def test_decode_q8_golden(gpu, oracle_mod):
    import torch
    from strataflow_amd.paged_kv import PagedKV
    g = golden("attn_q8_gqa4_decode")
    n_kv, Hkv = g["k_q8"].shape[:2]
    hd = g["k_q8"].shape[2] // 34 * 32
    Hq = int(g["n_head"])
    ps, n_pages = 32, (n_kv + 31) // 32 + 3
    kp, pt = scatter_columns(g["k_q8"].reshape(n_kv, -1), ps, n_pages, np.random.default_rng(1))
    vp, _ = scatter_columns(g["v_q8"].reshape(n_kv, -1), ps, n_pages, np.random.default_rng(1))
    dev = PagedKV(1, Hq, Hkv, hd, 8, ps, n_pages, device=gpu)
    dev.k[0].copy_(torch.from_numpy(kp))
    dev.v[0].copy_(torch.from_numpy(vp))
    q = torch.from_numpy(g["q"]).to(gpu)
    out = dev.decode(0, q, torch.from_numpy(pt).to(gpu), torch.tensor([n_kv], dtype=torch.int32, device=gpu),
                     n_kv, scale=float(g["scale"]))
    out = out.cpu().numpy().reshape(g["exact"].shape)
    assert_close(out, g["ggml"], what="q8 vs ggml golden")
    assert_close(out, g["exact"], max_abs=Q8_EXACT_ABS, rel_l2=Q8_EXACT_REL, what="q8 vs exact golden")


@pytest.mark.parametrize("shape", [(32, 8, 128), (8, 4, 64), (16, 2, 128), (16, 2, 64), (8, 8, 128),
                                   (16, 16, 64)])
@pytest.mark.parametrize("n_kv", [1, 33, 257, 1000])
def test_decode_q8_shapes(gpu, oracle_mod, shape, n_kv):
    Hq, Hkv, hd = shape
    c = Case(oracle_mod, seq_lens=[n_kv], n_head=Hq, n_head_kv=Hkv, head_dim=hd, page_size=64,
             kv_type=8, seed=n_kv + hd + 1)
    out = c.decode()
    assert_close(out, c.oracle(oracle_mod.GGML), what=f"q8 {shape} n_kv={n_kv} vs ggml")
    assert_close(out, c.oracle(oracle_mod.EXACT), max_abs=Q8_EXACT_ABS, rel_l2=Q8_EXACT_REL,
                 what=f"q8 {shape} n_kv={n_kv} vs exact")


def test_decode_q8_ctx32768(gpu, oracle_mod):
    # long-context Q8_0 decode, Mixtral shape, batch 1
    c = Case(oracle_mod, seq_lens=[32768], kv_type=8, seed=44)
    out = c.decode()
    ma, rl = assert_close(out, c.oracle(oracle_mod.GGML), what="q8 32k vs ggml")
    ma2, rl2 = errors(out, c.oracle(oracle_mod.EXACT))
    print(f"q8 32k: vs ggml max_abs {ma:.2e} rel_l2 {rl:.2e}; vs exact max_abs {ma2:.2e} rel_l2 {rl2:.2e}")
    assert ma2 <= Q8_EXACT_ABS and rl2 <= Q8_EXACT_REL


def test_decode_q8_batch8_varlen(gpu, oracle_mod):
    # batch 8, lengths uniform in [8k, 32k], one shared page pool
    lens = np.random.default_rng(45).integers(8192, 32769, 8)
    c = Case(oracle_mod, seq_lens=lens, kv_type=8, seed=46)
    out = c.decode(max_seq_len=32768)
    assert_close(out, c.oracle(oracle_mod.GGML), what="q8 b8 vs ggml")


def test_decode_q8_window_and_placement(gpu, oracle_mod):
    import torch
    c = Case(oracle_mod, seq_lens=[3000, 700], kv_lo=[1000, 33], kv_type=8, seed=47, extra_pages=4)
    base = c.decode()
    assert_close(base, c.oracle(oracle_mod.GGML), what="q8 window vs ggml")
    perm = np.random.default_rng(3).permutation(c.n_pages).astype(np.int32)
    k2 = torch.empty_like(c.dev.k[0]); v2 = torch.empty_like(c.dev.v[0])
    idx = torch.from_numpy(perm).long().to(gpu)
    k2[idx] = c.dev.k[0]; v2[idx] = c.dev.v[0]
    c.dev.k[0].copy_(k2); c.dev.v[0].copy_(v2)
    pt = c.page_table.copy(); valid = pt >= 0; pt[valid] = perm[pt[valid]]
    c.t_pt = torch.from_numpy(pt).to(gpu)
    assert np.array_equal(c.decode().view(np.uint32), base.view(np.uint32))


@pytest.mark.parametrize("kv_type", [1, 8])
@pytest.mark.parametrize("B", [2, 64, 65, 100, 256, 333])
def test_decode_split_plan_batches(gpu, oracle_mod, kv_type, B):
    # the split plan deals each kv head's row of workgroups out by sequence
    # length: a lane per sequence up to 64 sequences, rounds of 64 above;
    # lengths span empty, one token, one tile and a few thousand positions,
    # some with a window start, and max_seq_len overstates the longest span
    rng = np.random.default_rng(100 + B + kv_type)
    seq = rng.integers(0, 2400, B)
    seq[0], seq[-1] = 0, 1
    if B > 2:
        seq[1] = 32
        seq[B // 2] = 2400
    lo = np.where(rng.random(B) < 0.25, rng.integers(0, 400, B), 0)
    lo = np.minimum(lo, np.maximum(seq - 1, 0))
    c = Case(oracle_mod, seq_lens=seq, kv_lo=lo, n_head=8, n_head_kv=2, head_dim=128,
             kv_type=kv_type, seed=200 + B)
    out = c.decode(max_seq_len=3000)
    assert_close(out, c.oracle(oracle_mod.GGML), what=f"B={B} type {kv_type} vs ggml")
    assert np.all(out[0] == 0)


@pytest.mark.parametrize("shape", [(8, 8, 128), (8, 4, 64), (12, 6, 64), (4, 1, 128), (64, 16, 128),
                                   (48, 12, 64), (16, 8, 64)])
def test_decode_q8_column_layout(gpu, oracle_mod, shape):
    # a batch with >= 1024 tiles in all takes the staged kernel when 4 | Hkv
    # (8 kv heads per workgroup when 8 | Hkv: Hkv 8, 16; else 4: Hkv 4, 12),
    # otherwise the column layout (one wave per kv head: Hkv 6, 1)
    Hq, Hkv, hd = shape
    B = 40
    rng = np.random.default_rng(300 + Hkv)
    seq = rng.integers(1, 900, B)
    seq[3] = 899
    seq[5] = 0
    c = Case(oracle_mod, seq_lens=seq, n_head=Hq, n_head_kv=Hkv, head_dim=hd, kv_type=8, seed=310 + Hkv)
    out = c.decode(max_seq_len=900)
    assert_close(out, c.oracle(oracle_mod.GGML), what=f"q8 column layout {shape} vs ggml")
    assert np.all(out[5] == 0)


def test_decode_span_beyond_max_seq_len(gpu, oracle_mod):
    # a span longer than max_seq_len is attended in full by longer splits
    c = Case(oracle_mod, seq_lens=[3000, 200], seed=210)
    out = c.decode(max_seq_len=500)
    assert_close(out, c.oracle(oracle_mod.GGML), what="span beyond max_seq_len")


def test_decode_one_sequence_beyond_max_seq_len(gpu, oracle_mod):
    # one sequence, a max_seq_len that plans a single split (no merge pass):
    # the longer span is still attended in full, by that one split
    c = Case(oracle_mod, seq_lens=[1500], seed=211)
    out = c.decode(max_seq_len=100)
    assert_close(out, c.oracle(oracle_mod.GGML), what="one sequence beyond max_seq_len")


# ---- F32 KV (the reference's own cache type) -----------------------------------
# ggml converts nothing for an F32 cache, so the kernel (f32 MFMA for both
# products, P kept in f32) tracks the ggml-semantics oracle to f32 accumulation
# rounding; the bars are 50x tighter than the parity bar, so an f16 rounding of
# Q, K, P or V anywhere would fail them.
F32_MAX_ABS, F32_REL = 4e-5, 2e-5


@pytest.mark.parametrize("shape", [(32, 8, 128), (8, 4, 32), (8, 8, 64), (16, 2, 128)])
@pytest.mark.parametrize("n_kv", [1, 33, 257, 1000])
def test_decode_f32_shapes(gpu, oracle_mod, shape, n_kv):
    Hq, Hkv, hd = shape
    c = Case(oracle_mod, seq_lens=[n_kv], n_head=Hq, n_head_kv=Hkv, head_dim=hd, page_size=64,
             kv_type=0, seed=n_kv + hd + 3)
    out = c.decode()
    assert_close(out, c.oracle(oracle_mod.GGML), max_abs=F32_MAX_ABS, rel_l2=F32_REL,
                 what=f"f32 {shape} n_kv={n_kv} vs ggml")


def test_decode_f32_ctx4096_and_placement(gpu, oracle_mod):
    import torch
    c = Case(oracle_mod, seq_lens=[4096], kv_type=0, seed=48, extra_pages=2)
    base = c.decode()
    ma, rl = assert_close(base, c.oracle(oracle_mod.GGML), max_abs=F32_MAX_ABS, rel_l2=F32_REL,
                          what="f32 ctx4096 vs ggml")
    print(f"f32 ctx4096: max_abs {ma:.2e} rel_l2 {rl:.2e}")
    perm = np.random.default_rng(4).permutation(c.n_pages).astype(np.int32)
    k2 = torch.empty_like(c.dev.k[0]); v2 = torch.empty_like(c.dev.v[0])
    idx = torch.from_numpy(perm).long().to(gpu)
    k2[idx] = c.dev.k[0]; v2[idx] = c.dev.v[0]
    c.dev.k[0].copy_(k2); c.dev.v[0].copy_(v2)
    pt = c.page_table.copy(); valid = pt >= 0; pt[valid] = perm[pt[valid]]
    c.t_pt = torch.from_numpy(pt).to(gpu)
    assert np.array_equal(c.decode().view(np.uint32), base.view(np.uint32))


@pytest.mark.parametrize("page_size", [32, 512])
def test_decode_f32_varlen_window(gpu, oracle_mod, page_size):
    seq = [0, 1, 2500, 777, 64, 300]
    lo = [0, 0, 1999, 13, 32, 290]
    c = Case(oracle_mod, seq_lens=seq, kv_lo=lo, kv_type=0, page_size=page_size, seed=page_size + 5)
    out = c.decode(max_seq_len=2500)
    assert_close(out, c.oracle(oracle_mod.GGML), max_abs=F32_MAX_ABS, rel_l2=F32_REL,
                 what=f"f32 varlen page {page_size}")
    assert np.all(out[0] == 0)


@pytest.mark.parametrize("B", [3, 70])
def test_decode_f32_batches(gpu, oracle_mod, B):
    rng = np.random.default_rng(300 + B)
    seq = rng.integers(0, 1500, B)
    seq[0] = 0
    c = Case(oracle_mod, seq_lens=seq, n_head=8, n_head_kv=2, head_dim=128, kv_type=0, seed=310 + B)
    out = c.decode(max_seq_len=1600)
    assert_close(out, c.oracle(oracle_mod.GGML), max_abs=F32_MAX_ABS, rel_l2=F32_REL,
                 what=f"f32 B={B}")


@pytest.mark.parametrize("kv_type", [0, 1, 8])
@pytest.mark.parametrize("shape,n_kv", [((16, 2, 128), 20000), ((8, 1, 64), 40000), ((16, 4, 128), 9000),
                                        ((4, 4, 32), 30000)])
def test_decode_one_sequence_many_splits(gpu, oracle_mod, kv_type, shape, n_kv):
    # one sequence whose kv-head rows have 65 .. 256 split records (few kv
    # heads, long context): the wide merge pass
    Hq, Hkv, hd = shape
    if kv_type == 8 and hd < 64:
        # a Q8_0 cache of head_dim 32 is refused for every entry point
        from strataflow_amd import _lib
        with pytest.raises(_lib.SfaError) as e:
            Case(oracle_mod, seq_lens=[n_kv], n_head=Hq, n_head_kv=Hkv, head_dim=hd, kv_type=kv_type,
                 seed=n_kv + Hkv)
        assert e.value.status == _lib.SFA_ERR_UNSUPPORTED
        return
    c = Case(oracle_mod, seq_lens=[n_kv], n_head=Hq, n_head_kv=Hkv, head_dim=hd, kv_type=kv_type,
             seed=n_kv + Hkv)
    out = c.decode()
    if kv_type == 8:
        assert_close(out, c.oracle(oracle_mod.GGML), what=f"q8 {shape} n_kv={n_kv} vs ggml")
    else:
        assert_close(out, c.oracle(oracle_mod.GGML), what=f"type {kv_type} {shape} n_kv={n_kv} vs ggml")


# ---- Q8_0, one sequence --------------------------------------------------------
# g = 1..8 and even / odd n_head_kv; short, ragged, windowed and long spans over
# several page sizes (one split, the 32- and 64-slot merges and the wide merge).
@pytest.mark.parametrize("shape", [(32, 8, 128), (24, 6, 128), (16, 2, 64), (64, 8, 128), (4, 4, 64),
                                   (12, 3, 64)])
@pytest.mark.parametrize("n_kv,lo,page_size", [(1, None, 32), (45, None, 32), (5000, None, 256),
                                               (3001, 1000, 64), (12345, 17, 32)])
def test_decode_q8_one_sequence(gpu, oracle_mod, shape, n_kv, lo, page_size):
    Hq, Hkv, hd = shape
    c = Case(oracle_mod, seq_lens=[n_kv], kv_lo=None if lo is None else [lo], n_head=Hq, n_head_kv=Hkv,
             head_dim=hd, page_size=page_size, kv_type=8, seed=n_kv + Hq + hd)
    out = c.decode()
    assert_close(out, c.oracle(oracle_mod.GGML), what=f"q8 {shape} n_kv={n_kv} lo={lo} vs ggml")


def test_decode_q8_one_sequence_placement_and_plans(gpu, oracle_mod):
    # bit-identical under any physical page order; one split (max_seq_len
    # small: no merge pass) and a span beyond max_seq_len still match the oracle
    import torch
    c = Case(oracle_mod, seq_lens=[5000], kv_lo=[700], kv_type=8, page_size=64, seed=212, extra_pages=5)
    base = c.decode()
    assert_close(base, c.oracle(oracle_mod.GGML), what="q8 one sequence window vs ggml")
    perm = np.random.default_rng(5).permutation(c.n_pages).astype(np.int32)
    k2 = torch.empty_like(c.dev.k[0]); v2 = torch.empty_like(c.dev.v[0])
    idx = torch.from_numpy(perm).long().to(gpu)
    k2[idx] = c.dev.k[0]; v2[idx] = c.dev.v[0]
    c.dev.k[0].copy_(k2); c.dev.v[0].copy_(v2)
    pt = c.page_table.copy(); valid = pt >= 0; pt[valid] = perm[pt[valid]]
    c.t_pt = torch.from_numpy(pt).to(gpu)
    assert np.array_equal(c.decode().view(np.uint32), base.view(np.uint32))
    for msl in (100, 1000):
        assert_close(c.decode(max_seq_len=msl), c.oracle(oracle_mod.GGML), what=f"q8 one sequence msl={msl}")


def test_decode_q8_one_sequence_bad_page_id(gpu, oracle_mod):
    # an out-of-pool page id: the tile's loads get a zero-byte range, it
    # contributes nothing and the output stays finite
    import torch
    c = Case(oracle_mod, seq_lens=[600], page_size=256, kv_type=8, seed=213)
    pt = c.page_table.copy()
    pt[0, 1] = c.n_pages + 100
    c.t_pt = torch.from_numpy(pt).to(gpu)
    assert np.all(np.isfinite(c.decode()))


# ---- Q8_0 batches on the staged kernel: windows, page sizes, placement ----------
@pytest.mark.parametrize("Hkv,page_size", [(8, 32), (8, 256), (4, 64)])
def test_decode_q8_staged_windows(gpu, oracle_mod, Hkv, page_size):
    # 4 sequences of 3000..9000 positions (>= 1024 tiles in all), window
    # starts on and off the 32-position grid, one empty sequence
    lens = [9000, 3001, 0, 7777]
    lo = [4000, 17, 0, 3]
    c = Case(oracle_mod, seq_lens=lens, kv_lo=lo, n_head=4 * Hkv, n_head_kv=Hkv, head_dim=128,
             page_size=page_size, kv_type=8, seed=320 + Hkv + page_size)
    out = c.decode(max_seq_len=9000)
    assert_close(out, c.oracle(oracle_mod.GGML), what=f"q8 staged window Hkv={Hkv} page={page_size} vs ggml")
    assert np.all(out[2] == 0)


@pytest.mark.parametrize("head_dim", [128, 64])
@pytest.mark.parametrize("n_head_kv", [8, 4])
def test_decode_q8_staged_late_rescale(gpu, oracle_mod, n_head_kv, head_dim):
    # every 61st key scaled x5: most waves of the staged kernel (eight and
    # four kv heads per workgroup) meet scores more than the lazy-rescale
    # margin above their running reference after their first tile, so O and
    # l are rescaled mid-split in both halves of the lanes
    c = Case(oracle_mod, seq_lens=[12000, 5000, 9000], n_head=4 * n_head_kv, n_head_kv=n_head_kv,
             head_dim=head_dim, kv_type=8, seed=400 + n_head_kv + head_dim, k_boost=(61, 30, 5.0))
    out = c.decode()
    assert_close(out, c.oracle(oracle_mod.GGML),
                 what=f"q8 staged Hkv={n_head_kv} hd={head_dim} late rescale vs ggml")

@pytest.mark.parametrize("kv_type", [0, 1, 8])
@pytest.mark.parametrize("lens,shape", [([20000], (32, 8, 128)), ([12000, 5000, 9000], (16, 2, 128)),
                                        ([3000, 7000], (8, 8, 64))])
def test_decode_late_rescale(gpu, oracle_mod, kv_type, lens, shape):
    # every 61st key scaled x5, so waves whose first tile misses those keys
    # rescale O and l mid-split: one sequence, a batch (the Q8_0 column layout
    # for two kv heads) and head_dim 64
    Hq, Hkv, hd = shape
    c = Case(oracle_mod, seq_lens=lens, n_head=Hq, n_head_kv=Hkv, head_dim=hd, kv_type=kv_type,
             seed=600 + kv_type + len(lens), k_boost=(61, 30, 5.0))
    out = c.decode()
    what = f"type {kv_type} {shape} B={len(lens)} late rescale vs ggml"
    if kv_type == 0:
        assert_close(out, c.oracle(oracle_mod.GGML), max_abs=F32_MAX_ABS, rel_l2=F32_REL, what=what)
    else:
        assert_close(out, c.oracle(oracle_mod.GGML), what=what)

def test_decode_q8_staged_placement_and_bad_page(gpu, oracle_mod):
    # bit-identical under any physical page order; an out-of-pool page id in
    # one sequence leaves every output finite
    import torch
    lens = [9000, 8000, 6000, 3000]  # 4 x 282 tiles: the staged kernel
    c = Case(oracle_mod, seq_lens=lens, kv_type=8, page_size=64, seed=330, extra_pages=5)
    base = c.decode()
    assert_close(base, c.oracle(oracle_mod.GGML), what="q8 staged batch vs ggml")
    perm = np.random.default_rng(7).permutation(c.n_pages).astype(np.int32)
    k2 = torch.empty_like(c.dev.k[0]); v2 = torch.empty_like(c.dev.v[0])
    idx = torch.from_numpy(perm).long().to(gpu)
    k2[idx] = c.dev.k[0]; v2[idx] = c.dev.v[0]
    c.dev.k[0].copy_(k2); c.dev.v[0].copy_(v2)
    pt = c.page_table.copy(); valid = pt >= 0; pt[valid] = perm[pt[valid]]
    c.t_pt = torch.from_numpy(pt).to(gpu)
    assert np.array_equal(c.decode().view(np.uint32), base.view(np.uint32))
    pt[1, 3] = c.n_pages + 100
    c.t_pt = torch.from_numpy(pt).to(gpu)
    assert np.all(np.isfinite(c.decode()))
