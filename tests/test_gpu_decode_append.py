"""The decode node with its append fused in (sfa_attn_decode_append,
sfa_pager_append_attend) against the two calls it replaces: sfa_kv_append of
each sequence's new token at position seq_len - 1, then sfa_attn_decode.
Outputs and pool bytes must be equal bit for bit; one case is also checked
against the oracle with the token appended on the host."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import Case, assert_close

pytestmark = pytest.mark.gpu


def _new_tokens(gpu, B, Hkv, hd, seed):
    import torch
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    return (torch.randn((B, Hkv, hd), device=gpu, generator=g),
            torch.randn((B, Hkv, hd), device=gpu, generator=g))


def _unfused_vs_fused(c, k, v, max_seq_len):
    """Layer 0: append then decode; layer 1 (the same bytes): the fused call."""
    import torch
    B = c.B
    seq = torch.arange(B, dtype=torch.int32, device=k.device)
    pos = (c.t_sl - 1).to(torch.int32)
    c.dev.append(0, k, v, seq, pos, c.t_pt)
    out0 = c.dev.decode(0, c.t_q, c.t_pt, c.t_sl, max_seq_len, kv_lo=c.t_lo)
    out1 = c.dev.decode_append(1, k, v, c.t_q, c.t_pt, c.t_sl, max_seq_len, kv_lo=c.t_lo)
    torch.cuda.synchronize()
    return out0, out1


def _assert_same(c, out0, out1, what):
    import torch
    assert torch.equal(out0.view(torch.int32), out1.view(torch.int32)), f"{what}: outputs differ"
    assert torch.equal(c.dev.k[0], c.dev.k[1]), f"{what}: K pools differ"
    assert torch.equal(c.dev.v[0], c.dev.v[1]), f"{what}: V pools differ"


@pytest.mark.parametrize("kv_type", [1, 0])
@pytest.mark.parametrize("shape", [(32, 8, 128), (8, 2, 64), (8, 4, 32), (16, 16, 128)])
@pytest.mark.parametrize("n_kv,page_size", [(1, 256), (33, 32), (256, 256), (257, 256), (4096, 256),
                                            (3001, 64)])
def test_decode_append_one_sequence(gpu, oracle_mod, kv_type, shape, n_kv, page_size):
    # the new token on the first position, a tile's first row, a page's last
    # and first rows, at ctx 4096; F16 and F32 caches
    Hq, Hkv, hd = shape
    c = Case(oracle_mod, seq_lens=[n_kv], n_head=Hq, n_head_kv=Hkv, head_dim=hd, page_size=page_size,
             seed=n_kv + hd, n_layer=2, kv_type=kv_type)
    k, v = _new_tokens(gpu, 1, Hkv, hd, n_kv + 1)
    out0, out1 = _unfused_vs_fused(c, k, v, n_kv)
    _assert_same(c, out0, out1, f"{shape} n_kv={n_kv}")


@pytest.mark.parametrize("seq,lo", [
    ([700, 1, 4096, 300, 0], [0, 0, 3000, 290, 0]),   # window starts, one token, an empty sequence
    ([100, 50, 33], [0, 60, 32]),                      # seq_len <= kv_lo: nothing attended, row written
    ([4097, 4000, 129, 2], None),                      # the window leg's shape, lossless
])
@pytest.mark.parametrize("kv_type", [1, 0])
def test_decode_append_batches(gpu, oracle_mod, seq, lo, kv_type):
    c = Case(oracle_mod, seq_lens=seq, kv_lo=lo, seed=len(seq) * 7, n_layer=2, kv_type=kv_type)
    k, v = _new_tokens(gpu, c.B, c.n_head_kv, c.head_dim, 5)
    out0, out1 = _unfused_vs_fused(c, k, v, max(seq))
    _assert_same(c, out0, out1, f"seq {seq} lo {lo}")


@pytest.mark.parametrize("kv_type", [1, 0])
def test_decode_append_batch_over_64(gpu, oracle_mod, kv_type):
    # more sequences than a wave has lanes: the kernel reads seq_len per sequence
    rng = np.random.default_rng(70)
    seq = rng.integers(1, 600, 70)
    c = Case(oracle_mod, seq_lens=seq, n_head=8, n_head_kv=2, head_dim=64, page_size=64, seed=70,
             n_layer=2, kv_type=kv_type)
    k, v = _new_tokens(gpu, c.B, c.n_head_kv, c.head_dim, 71)
    out0, out1 = _unfused_vs_fused(c, k, v, int(seq.max()))
    _assert_same(c, out0, out1, "B=70")


@pytest.mark.parametrize("kv_type", [1, 0])
def test_decode_append_missing_page(gpu, oracle_mod, kv_type):
    # the new token's page id is -1 for sequence 1: the append skips it and
    # its tile is masked, in both forms
    import torch
    c = Case(oracle_mod, seq_lens=[500, 300, 40], seed=3, n_layer=2, page_size=64, kv_type=kv_type)
    lp = (300 - 1) // 64
    c.page_table[1, lp] = -1
    c.t_pt = torch.from_numpy(c.page_table).to(gpu)
    k, v = _new_tokens(gpu, c.B, c.n_head_kv, c.head_dim, 4)
    out0, out1 = _unfused_vs_fused(c, k, v, 500)
    _assert_same(c, out0, out1, "missing page")


def test_decode_append_matches_oracle(gpu, oracle_mod):
    # Mixtral shape, the new token appended on the host too: the oracle's result
    c = Case(oracle_mod, seq_lens=[4096, 1000], kv_lo=[0, 200], seed=11, n_layer=2)
    k, v = _new_tokens(gpu, c.B, c.n_head_kv, c.head_dim, 12)
    out0, out1 = _unfused_vs_fused(c, k, v, 4096)
    _assert_same(c, out0, out1, "mixtral")
    pos = (c.seq_lens - 1).astype(np.int32)
    assert c.host.append(k.cpu().numpy(), v.cpu().numpy(), np.arange(c.B, dtype=np.int32), pos,
                         c.page_table) == 0
    assert_close(out1.cpu().numpy(), c.oracle(oracle_mod.GGML), what="fused vs ggml")


@pytest.mark.parametrize("kv_type", [1, 0])
def test_decode_append_cold_page(gpu, kv_type):
    # the new position on a cold page (id -2): written to the host-pinned pool
    import torch
    from strataflow_amd.paged_kv import PagedKV
    Hq, Hkv, hd, ps = 16, 4, 128, 32
    kv = PagedKV(2, Hq, Hkv, hd, kv_type, ps, 4, device=gpu, n_cold_pages=2)
    g = torch.Generator(device="cpu")
    g.manual_seed(9)
    # the same values (|x| < 2) in both layers' device and cold pools
    dt, es = (torch.float16, 2) if kv_type == 1 else (torch.float32, 4)
    for pool in (kv.k, kv.v, kv.k_cold, kv.v_cold):
        vals = (torch.rand(pool[0].numel() // es, generator=g) * 4 - 2).to(dt)
        pool.copy_(vals.view(torch.uint8).view(pool[0].shape).expand_as(pool))
    pt = torch.tensor([[0, -2, 1]], dtype=torch.int32, device=gpu)  # positions 32..63 cold page 0
    sl = torch.tensor([45], dtype=torch.int32, device=gpu)
    q = torch.randn((1, Hq, hd), device=gpu)
    k, v = _new_tokens(gpu, 1, Hkv, hd, 10)
    kv.append(0, k, v, torch.zeros(1, dtype=torch.int32, device=gpu), sl - 1, pt)
    out0 = kv.decode(0, q, pt, sl, 45)
    out1 = kv.decode_append(1, k, v, q, pt, sl, 45)
    torch.cuda.synchronize()
    assert torch.equal(out0.view(torch.int32), out1.view(torch.int32))
    assert torch.equal(kv.k_cold[0], kv.k_cold[1]) and torch.equal(kv.v_cold[0], kv.v_cold[1])
    assert torch.equal(kv.k[0], kv.k[1]) and torch.equal(kv.v[0], kv.v[1])


@pytest.mark.parametrize("kv_type", [8])
def test_decode_append_refuses_q8(gpu, oracle_mod, kv_type):
    from strataflow_amd import _lib
    c = Case(oracle_mod, seq_lens=[100], kv_type=kv_type, seed=1, n_layer=1)
    k, v = _new_tokens(gpu, 1, c.n_head_kv, c.head_dim, 2)
    with pytest.raises(_lib.SfaError) as e:
        c.dev.decode_append(0, k, v, c.t_q, c.t_pt, c.t_sl, 100)
    assert e.value.status == _lib.SFA_ERR_UNSUPPORTED


@pytest.mark.parametrize("kv_type", ["f16", "f32", "q8_0"])
@pytest.mark.parametrize("attend", ["window", "lossless"])
def test_pager_append_attend_equals_two_calls(gpu, attend, kv_type):
    # two pagers with the same placement: append + attend against the fused
    # call over decode steps that cross pages and evict (a wrong row written at
    # one step shows in the next steps' outputs)
    import torch
    from strataflow_amd.pager import (SFA_ATTEND_LOSSLESS, SFA_ATTEND_WINDOW, SFA_KV_F16, SFA_KV_F32,
                                      SFA_KV_Q8_0, KvPager)
    B, Hq, Hkv, hd, ps = 3, 16, 4, 128, 64
    mode = SFA_ATTEND_WINDOW if attend == "window" else SFA_ATTEND_LOSSLESS
    kvt = {"f16": SFA_KV_F16, "f32": SFA_KV_F32, "q8_0": SFA_KV_Q8_0}[kv_type]  # Q8_0: the two calls
    mk = lambda: KvPager(n_layer=1, n_head=Hq, n_head_kv=Hkv, head_dim=hd, kv_type=kvt,
                         page_size=ps, n_seq=B, n_ctx=1024, window=256, attend=mode, seed=5)
    pa, pb = mk(), mk()
    g = torch.Generator(device=gpu)
    g.manual_seed(6)
    # the prompt: appended only (a windowed pager attends one token per
    # sequence and step), in steps of at most one page per sequence
    left = np.array([300, 200, 64], np.int32)
    while left.any():
        chunk = np.minimum(left, ps).astype(np.int32)
        assert pa.begin(chunk) == 0 and pb.begin(chunk) == 0
        n = int(chunk.sum())
        k = torch.randn((n, Hkv, hd), device=gpu, generator=g)
        v = torch.randn((n, Hkv, hd), device=gpu, generator=g)
        pa.append(0, k, v)
        pb.append(0, k, v)
        left -= chunk
    for s in range(80):
        ones = np.ones(B, np.int32)
        assert pa.begin(ones) == 0 and pb.begin(ones) == 0
        k = torch.randn((B, Hkv, hd), device=gpu, generator=g)
        v = torch.randn((B, Hkv, hd), device=gpu, generator=g)
        q = torch.randn((B, Hq, hd), device=gpu, generator=g)
        pa.append(0, k, v)
        oa = pa.attend(0, q)
        ob = pb.append_attend(0, k, v, q)
        torch.cuda.synchronize()
        assert torch.equal(oa.view(torch.int32), ob.view(torch.int32)), f"step {s}"
    pa.close()
    pb.close()


@pytest.mark.parametrize("case", range(24))
def test_decode_append_sweep(gpu, oracle_mod, case):
    # seeded random shapes, page sizes, batches, window starts and cache types:
    # the fused call against append-then-decode, bit for bit
    rng = np.random.default_rng(1000 + case)
    Hq, Hkv, hd = [(32, 8, 128), (8, 2, 64), (16, 4, 128), (8, 8, 32), (16, 2, 64)][case % 5]
    ps = int(rng.choice([32, 64, 128, 256]))
    B = int(rng.integers(1, 7))
    seq = rng.integers(1, 1500, B)
    seq[rng.random(B) < 0.15] = 0
    lo = None
    if case % 3 == 1:
        lo = [int(rng.integers(0, max(int(n), 1))) for n in seq]
    kv_type = [1, 0][case % 2]
    c = Case(oracle_mod, seq_lens=seq, kv_lo=lo, n_head=Hq, n_head_kv=Hkv, head_dim=hd, page_size=ps,
             seed=case, n_layer=2, kv_type=kv_type)
    k, v = _new_tokens(gpu, c.B, Hkv, hd, 2000 + case)
    out0, out1 = _unfused_vs_fused(c, k, v, max(int(seq.max()), 1))
    _assert_same(c, out0, out1, f"case {case}: {(Hq, Hkv, hd)} ps {ps} seq {seq.tolist()} lo {lo}")
