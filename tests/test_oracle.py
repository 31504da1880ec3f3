"""Pins the CPU oracle (oracle/sfa_oracle.c) before anything is checked
against it: numpy's IEEE half conversion, hand-computed Q8_0 blocks, the
independent float64 golden vectors, and closed forms of the attention node
(src/model/engine/engine.cpp:1751-1761)."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import assert_close, errors, f16_cols, golden, scatter_columns

GOLDEN_CASES = [
    "attn_f16_gqa2_decode",
    "attn_f16_gqa4_window",
    "attn_f16_mha_prefill",
    "attn_q8_gqa4_decode",
    "attn_q8_gqa2_prefill",
]


# ---- half conversion ---------------------------------------------------------

def test_f32_to_f16_matches_numpy(oracle_mod):
    rng = np.random.default_rng(0)
    x = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2**-24, 2**-25,
                      2**-25 * 1.0000001, 6.1e-5, 3.0517578e-05, np.inf, -np.inf], np.float32)
    x = np.concatenate([x, edges])
    got = oracle_mod.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    ok = ~np.isnan(x)
    assert np.array_equal(got[ok], ref[ok])
    assert np.all(np.isnan(got[~ok].view(np.float16)))


def test_f16_to_f32_exhaustive(oracle_mod):
    h = np.arange(65536, dtype=np.uint16)
    got = oracle_mod.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))


# ---- Q8_0 --------------------------------------------------------------------

def test_q8_0_hand_computed_block(oracle_mod):
    # amax 127 -> d = 1, id = 1: codes are roundf(x), ties away from zero
    x = np.zeros(32, np.float32)
    x[:8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.4, 3.49]
    b = oracle_mod.quantize_q8_0(x)
    assert b.shape == (34,)
    assert b[:2].view(np.float16)[0] == np.float16(1.0)
    q = b[2:].view(np.int8)
    assert list(q[:8]) == [127, 3, -3, 1, -1, 2, -126, 3]
    assert np.all(q[8:] == 0)


def test_q8_0_zero_block_and_scale(oracle_mod):
    b = oracle_mod.quantize_q8_0(np.zeros(32, np.float32))
    assert np.all(b == 0)
    # all ones: d = 1/127 (stored fp16), every code 127
    b = oracle_mod.quantize_q8_0(np.full(32, -1.0, np.float32))
    assert b[:2].view(np.float16)[0] == np.float16(np.float32(1.0) / np.float32(127.0))
    assert np.all(b[2:].view(np.int8) == -127)


def test_q8_0_roundtrip_bound(oracle_mod):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 128)).astype(np.float32) * 3
    b = oracle_mod.quantize_q8_0(x)
    y = oracle_mod.dequantize_q8_0(b)
    xb = x.reshape(64, 4, 32)
    d = np.abs(xb).max(-1, keepdims=True) / 127
    d16 = b.reshape(64, 4, 34)[..., :2].copy().view(np.float16).astype(np.float64)
    # |x - d16*q| <= d/2 + 127*|d16 - d|
    bound = d / 2 + 127 * np.abs(d16 - d) + 1e-7
    assert np.all(np.abs(y.reshape(64, 4, 32) - xb) <= bound)
    # the block maximum maps to +-127
    q = b.reshape(64, 4, 34)[..., 2:].view(np.int8)
    amax_idx = np.abs(xb).argmax(-1)
    assert np.all(np.abs(np.take_along_axis(q, amax_idx[..., None], -1)) == 127)


def test_q8_0_simd_forms_round_ties_to_even(oracle_mod):
    # the same amax-127 block as above under ggml's SIMD quantisers (x86 and
    # Arm): codes are rounded to nearest even, so the ties go the other way
    x = np.zeros(32, np.float32)
    x[:8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.4, 3.49]
    for form in (oracle_mod.Q8_AVX2, oracle_mod.Q8_NEON):
        with oracle_mod.q8_variant(form):
            b = oracle_mod.quantize_q8_0(x)
        assert b[:2].view(np.float16)[0] == np.float16(1.0)
        assert list(b[2:].view(np.int8)[:8]) == [127, 2, -2, 0, 0, 2, -126, 3], form
    # and the scalar form is restored on exit
    assert list(oracle_mod.quantize_q8_0(x)[2:].view(np.int8)[:3]) == [127, 3, -3]


def test_q8_0_avx2_form_scales_by_127_over_amax(oracle_mod):
    # amax 1.4442534: in f32, 127/amax = 87.93471 while 1/(amax/127) = 87.9347,
    # so x = 0.017058112 lands at 1.5000001 (x86 form: code 2) or 1.4999999
    # (scalar and Arm forms: code 1)
    x = np.zeros(32, np.float32)
    x[0], x[1] = np.float32(1.4442534), np.float32(0.017058112)
    assert np.float32(127) / x[0] != np.float32(1) / (x[0] / np.float32(127))
    codes = {}
    for form in (oracle_mod.Q8_SCALAR, oracle_mod.Q8_AVX2, oracle_mod.Q8_NEON):
        with oracle_mod.q8_variant(form):
            codes[form] = oracle_mod.quantize_q8_0(x)[2:].view(np.int8)[:2].tolist()
    assert codes == {oracle_mod.Q8_SCALAR: [127, 1], oracle_mod.Q8_AVX2: [127, 2],
                     oracle_mod.Q8_NEON: [127, 1]}


def test_q8_0_forms_differ_rarely(oracle_mod):
    # on N(0,1) data the three forms store the same scale and differ in very
    # few codes (exact ties and one-ulp differences of id at a half-integer)
    x = np.random.default_rng(3).standard_normal((4096, 128)).astype(np.float32)
    out = {}
    for form in (oracle_mod.Q8_SCALAR, oracle_mod.Q8_AVX2, oracle_mod.Q8_NEON):
        with oracle_mod.q8_variant(form):
            out[form] = oracle_mod.quantize_q8_0(x).reshape(-1, 34)
    base = out[oracle_mod.Q8_SCALAR]
    for form in (oracle_mod.Q8_AVX2, oracle_mod.Q8_NEON):
        assert np.array_equal(out[form][:, :2], base[:, :2])
        diff = np.count_nonzero(out[form][:, 2:] != base[:, 2:])
        assert diff <= 1e-4 * x.size, (form, diff)
        dq = np.abs(out[form][:, 2:].view(np.int8).astype(int) - base[:, 2:].view(np.int8).astype(int))
        assert dq.max() <= 1


@pytest.mark.parametrize("name", ["attn_q8_gqa4_decode", "attn_q8_gqa2_prefill"])
def test_q8_0_matches_golden_bytes(oracle_mod, name):
    g = golden(name)
    assert np.array_equal(oracle_mod.quantize_q8_0(g["k_f32"]), g["k_q8"])
    assert np.array_equal(oracle_mod.quantize_q8_0(g["v_f32"]), g["v_q8"])


# ---- attention -----------------------------------------------------------------

def _host_kv(oracle_mod, g, page_size=32, seed=0, n_pages=None):
    """Pool + page table holding a golden case's cache, pages shuffled."""
    kv_type = int(g["kv_type"])
    if kv_type == oracle_mod.KV_F16:
        kc, vc = f16_cols(g["k_f16"]), f16_cols(g["v_f16"])
        n_kv, Hkv, hd = g["k_f16"].shape
    else:
        kc = g["k_q8"].reshape(g["k_q8"].shape[0], -1)
        vc = g["v_q8"].reshape(g["v_q8"].shape[0], -1)
        n_kv, Hkv = g["k_q8"].shape[:2]
        hd = g["k_q8"].shape[2] // 34 * 32
    need = (n_kv + page_size - 1) // page_size
    n_pages = n_pages or need + 3
    kvh = oracle_mod.HostPagedKv(Hkv, hd, page_size, kv_type, n_pages)
    kp, pt = scatter_columns(kc, page_size, n_pages, np.random.default_rng(seed))
    vp, pt2 = scatter_columns(vc, page_size, n_pages, np.random.default_rng(seed))
    assert np.array_equal(pt, pt2)
    kvh.k[:] = kp
    kvh.v[:] = vp
    return kvh, pt, n_kv


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_attention_matches_golden(oracle_mod, name):
    g = golden(name)
    kvh, pt, n_kv = _host_kv(oracle_mod, g)
    T = g["q"].shape[0]
    q = g["q"][None]
    lo = np.array([int(g["kv_lo"])], np.int32)
    sl = np.array([n_kv], np.int32)
    ex = kvh.attention(q, int(g["n_head"]), pt, sl, lo, T=T, scale=float(g["scale"]),
                       mode=oracle_mod.EXACT)[0]
    assert_close(ex, g["exact"], max_abs=2e-6, rel_l2=1e-6, what="exact")
    gg = kvh.attention(q, int(g["n_head"]), pt, sl, lo, T=T, scale=float(g["scale"]),
                       mode=oracle_mod.GGML)[0]
    # same roundings, different summation precision: a P value on an f16
    # rounding boundary may land one ulp apart
    assert_close(gg, g["ggml"], max_abs=5e-5, rel_l2=2e-5, what="ggml")


@pytest.mark.parametrize("kv_type", [0, 1, 8])
def test_single_position_returns_v(oracle_mod, kv_type):
    # n_kv == 1 => p == 1 exactly => O = V[0] (the reference's pos-0 case)
    rng = np.random.default_rng(3)
    Hq, Hkv, hd = 8, 2, 64
    kvh = oracle_mod.HostPagedKv(Hkv, hd, 32, kv_type, 2)
    k = rng.standard_normal((1, Hkv, hd)).astype(np.float32)
    v = rng.standard_normal((1, Hkv, hd)).astype(np.float32)
    pt = np.array([[1]], np.int32)
    assert kvh.append(k, v, np.zeros(1, np.int32), np.zeros(1, np.int32), pt) == 0
    q = rng.standard_normal((1, Hq, hd)).astype(np.float32)
    if kv_type == 0:
        vq = v
    elif kv_type == 1:
        vq = v.astype(np.float16).astype(np.float32)
    else:
        vq = oracle_mod.dequantize_q8_0(oracle_mod.quantize_q8_0(v))
    for mode in (oracle_mod.EXACT, oracle_mod.GGML):
        o = kvh.attention(q, Hq, pt, np.array([1], np.int32), mode=mode)
        for h in range(Hq):
            assert np.array_equal(o[0, h], vq[0, h // (Hq // Hkv)])


def _filled(oracle_mod, rng, Hkv, hd, n_kv, page_size=32, kv_type=1, k=None, v=None):
    n_pages = (n_kv + page_size - 1) // page_size + 2
    kvh = oracle_mod.HostPagedKv(Hkv, hd, page_size, kv_type, n_pages)
    if k is None:
        k = rng.standard_normal((n_kv, Hkv, hd)).astype(np.float32)
    if v is None:
        v = rng.standard_normal((n_kv, Hkv, hd)).astype(np.float32)
    pt = rng.permutation(n_pages).astype(np.int32)[None, : (n_kv + page_size - 1) // page_size]
    assert kvh.append(k, v, np.zeros(n_kv, np.int32), np.arange(n_kv, dtype=np.int32), pt) == 0
    return kvh, pt, k, v


def test_gqa_head_map_closed_form(oracle_mod):
    # V[j][kvh][:] = kvh + 1 => O[h] = h // g + 1 for every query head h
    rng = np.random.default_rng(4)
    Hq, Hkv, hd, n = 8, 2, 32, 77
    v = np.broadcast_to(np.arange(1, Hkv + 1, dtype=np.float32)[None, :, None], (n, Hkv, hd)).copy()
    kvh, pt, _, _ = _filled(oracle_mod, rng, Hkv, hd, n, v=v)
    q = rng.standard_normal((1, Hq, hd)).astype(np.float32)
    o = kvh.attention(q, Hq, pt, np.array([n], np.int32), mode=oracle_mod.EXACT)
    for h in range(Hq):
        np.testing.assert_allclose(o[0, h], h // (Hq // Hkv) + 1, rtol=0, atol=1e-6)


@pytest.mark.parametrize("kv_type", [0, 1])
def test_uniform_weights_give_mean(oracle_mod, kv_type):
    # identical keys, or q == 0, => softmax uniform => O = mean(V)
    rng = np.random.default_rng(5)
    Hq, Hkv, hd, n = 4, 4, 32, 90
    k = np.broadcast_to(rng.standard_normal((1, Hkv, hd)).astype(np.float32), (n, Hkv, hd)).copy()
    kvh, pt, _, v = _filled(oracle_mod, rng, Hkv, hd, n, k=k, kv_type=kv_type)
    vq = (v if kv_type == 0 else v.astype(np.float16)).astype(np.float64)
    q = rng.standard_normal((1, Hq, hd)).astype(np.float32)
    o = kvh.attention(q, Hq, pt, np.array([n], np.int32), mode=oracle_mod.EXACT)
    np.testing.assert_allclose(o[0], vq.mean(0), atol=1e-6)
    o = kvh.attention(np.zeros_like(q), Hq, pt, np.array([n], np.int32), mode=oracle_mod.EXACT)
    np.testing.assert_allclose(o[0], vq.mean(0), atol=1e-6)


def test_aligned_key_one_hot(oracle_mod):
    rng = np.random.default_rng(6)
    Hq, Hkv, hd, n = 2, 2, 32, 64
    kvh, pt, k, v = _filled(oracle_mod, rng, Hkv, hd, n)
    j = 41
    q = (k[j][None] * 50.0).astype(np.float32)  # score gap >> 1 at position j
    o = kvh.attention(q, Hq, pt, np.array([n], np.int32), mode=oracle_mod.EXACT)
    np.testing.assert_allclose(o[0], v[j].astype(np.float16).astype(np.float32), atol=1e-4)


def test_kv_lo_masks_prefix(oracle_mod):
    # positions below kv_lo are excluded exactly: same as a history that starts there
    rng = np.random.default_rng(7)
    Hq, Hkv, hd, n, lo = 4, 2, 64, 150, 61
    kvh, pt, k, v = _filled(oracle_mod, rng, Hkv, hd, n)
    kvh2, pt2, _, _ = _filled(oracle_mod, rng, Hkv, hd, n - lo, k=k[lo:], v=v[lo:])
    q = rng.standard_normal((1, Hq, hd)).astype(np.float32)
    for mode in (oracle_mod.EXACT, oracle_mod.GGML):
        a = kvh.attention(q, Hq, pt, np.array([n], np.int32), np.array([lo], np.int32), mode=mode)
        b = kvh2.attention(q, Hq, pt2, np.array([n - lo], np.int32), mode=mode)
        assert np.array_equal(a, b)


def test_page_placement_is_bit_invariant(oracle_mod):
    # the reference's paged == full-resident bit identity (test_kv_paging.cpp:243)
    rng = np.random.default_rng(8)
    Hq, Hkv, hd, n = 8, 2, 64, 200
    k = rng.standard_normal((n, Hkv, hd)).astype(np.float32)
    v = rng.standard_normal((n, Hkv, hd)).astype(np.float32)
    q = rng.standard_normal((1, Hq, hd)).astype(np.float32)
    outs = []
    for seed in range(3):
        kvh, pt, _, _ = _filled(oracle_mod, np.random.default_rng(100 + seed), Hkv, hd, n, k=k, v=v)
        outs.append(kvh.attention(q, Hq, pt, np.array([n], np.int32), mode=oracle_mod.GGML))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_causal_prefill_rows_equal_decode(oracle_mod):
    # causal mask: prefill token t == decode with n_kv = qpos_t + 1
    rng = np.random.default_rng(9)
    Hq, Hkv, hd, n, T = 4, 2, 32, 100, 12
    kvh, pt, _, _ = _filled(oracle_mod, rng, Hkv, hd, n)
    q = rng.standard_normal((1, T, Hq, hd)).astype(np.float32)
    for mode in (oracle_mod.EXACT, oracle_mod.GGML):
        pre = kvh.attention(q, Hq, pt, np.array([n], np.int32), T=T, mode=mode)
        for t in range(T):
            dec = kvh.attention(q[:, t], Hq, pt, np.array([n - T + t + 1], np.int32), mode=mode)
            if mode == oracle_mod.EXACT:
                assert np.array_equal(pre[0, t], dec[0])
            else:
                # ggml rows span the whole history (masked columns weigh 0), so
                # only the f32 summation grouping differs
                np.testing.assert_allclose(pre[0, t], dec[0], rtol=0, atol=1e-6)


def test_ggml_and_exact_modes_within_parity_bar(oracle_mod):
    rng = np.random.default_rng(10)
    Hq, Hkv, hd, n = 32, 8, 128, 1000
    kvh, pt, _, _ = _filled(oracle_mod, rng, Hkv, hd, n)
    q = rng.standard_normal((1, Hq, hd)).astype(np.float32)
    a = kvh.attention(q, Hq, pt, np.array([n], np.int32), mode=oracle_mod.GGML)
    b = kvh.attention(q, Hq, pt, np.array([n], np.int32), mode=oracle_mod.EXACT)
    ma, rl = errors(a, b)
    assert ma < 2e-3 and rl < 1e-3


def test_missing_page_is_reported(oracle_mod):
    rng = np.random.default_rng(11)
    kvh, pt, _, _ = _filled(oracle_mod, rng, 2, 32, 64)
    bad = pt.copy()
    bad[0, 1] = -1
    q = rng.standard_normal((1, 4, 32)).astype(np.float32)
    with pytest.raises(RuntimeError):
        kvh.attention(q, 4, bad, np.array([64], np.int32))


def test_f32_cache_ggml_mode_is_exact_to_f32_rounding(oracle_mod):
    # an F32 cache has no operand conversion in ggml (the vec_dot_type of F32
    # is F32): the ggml-semantics reading equals the float64 one up to f32
    # accumulation rounding, far inside the parity bar; a stray f16 rounding
    # of Q, K, P or V (2^-11 relative) would fail it
    rng = np.random.default_rng(21)
    Hq, Hkv, hd, n = 8, 2, 128, 700
    kvh, pt, _, _ = _filled(oracle_mod, rng, Hkv, hd, n, kv_type=0)
    q = rng.standard_normal((1, Hq, hd)).astype(np.float32)
    sl = np.array([n], np.int32)
    gg = kvh.attention(q, Hq, pt, sl, mode=oracle_mod.GGML)
    ex = kvh.attention(q, Hq, pt, sl, mode=oracle_mod.EXACT)
    assert_close(gg, ex, max_abs=2e-6, rel_l2=1e-6, what="f32 ggml vs exact")
