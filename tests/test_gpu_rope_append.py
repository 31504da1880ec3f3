"""Fused RoPE + KV append on the GPU (sfa_rope_kv_append through the C ABI)
against the oracle: orc_rope_normal on Q and K followed by orc_kv_append.

Bars: rotated Q within 1e-6 of each pair's magnitude (cosf/sinf may differ by
an ulp between the device and the host libm; theta itself follows the same f32
recurrence on both, from the same host powf); V bytes identical (the append's
conversion, unchanged); rotated K in an f32 cache within the Q bar, in an f16
cache within one f16 ulp of the oracle's bytes; in a Q8_0 cache the block
scales within one f16 ulp and every dequantised value within one quantisation
step."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32, F16, Q8 = 0, 1, 8


def _tokens(rng, n_seq, per_seq, page_size, max_pages):
    seq, pos = [], []
    for b in range(n_seq):
        # a run of consecutive positions plus scattered ones up to the table's end
        start = int(rng.integers(0, page_size * max_pages - per_seq))
        p = np.concatenate([start + np.arange(per_seq // 2),
                            rng.choice(page_size * max_pages, per_seq - per_seq // 2, replace=False)])
        p = np.unique(p)
        seq.append(np.full(p.size, b, np.int32))
        pos.append(p.astype(np.int32))
    return np.concatenate(seq), np.concatenate(pos)


def _rows(pool, pt, seq, pos, page_size, col_bytes):
    """Column bytes of each (seq, pos) token from a pool [n_pages, page_bytes]."""
    out = np.empty((seq.size, col_bytes), np.uint8)
    for t, (b, p) in enumerate(zip(seq, pos)):
        pid = pt[b, p // page_size]
        off = (p % page_size) * col_bytes
        out[t] = pool[pid, off:off + col_bytes]
    return out


def _f16_ulps(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    # sign-magnitude to a monotone integer line
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(a - b)


@pytest.mark.parametrize("kv_type", [F32, F16, Q8])
@pytest.mark.parametrize("shape", [(32, 8, 128), (8, 4, 32), (16, 8, 64)])
def test_rope_append_vs_oracle(gpu, oracle_mod, kv_type, shape):
    import torch
    from strataflow_amd.paged_kv import PagedKV
    Hq, Hkv, hd = shape
    rng = np.random.default_rng(hd + kv_type)
    ps, max_pages, n_seq = 64, 24, 3
    n_pages = n_seq * max_pages + 2
    seq, pos = _tokens(rng, n_seq, 120, ps, max_pages)
    pt = rng.permutation(n_pages)[:n_seq * max_pages].reshape(n_seq, max_pages).astype(np.int32)
    n = seq.size
    q = (3 * rng.standard_normal((n, Hq, hd))).astype(np.float32)
    k = (3 * rng.standard_normal((n, Hkv, hd))).astype(np.float32)
    v = (3 * rng.standard_normal((n, Hkv, hd))).astype(np.float32)
    base = 1e6 if hd == 128 else 1e4
    if kv_type == Q8 and hd < 64:
        # a Q8_0 cache of head_dim 32 is refused for every entry point
        from strataflow_amd import _lib
        with pytest.raises(_lib.SfaError) as e:
            PagedKV(1, Hq, Hkv, hd, kv_type, ps, n_pages, device=gpu)
        assert e.value.status == _lib.SFA_ERR_UNSUPPORTED
        return

    dev = PagedKV(1, Hq, Hkv, hd, kv_type, ps, n_pages, device=gpu)
    tq = torch.from_numpy(q).to(gpu)
    dev.rope_append(0, tq, torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu),
                    torch.from_numpy(seq).to(gpu), torch.from_numpy(pos).to(gpu),
                    torch.from_numpy(pt).to(gpu), base)
    torch.cuda.synchronize()

    q_ref = oracle_mod.rope_normal(q, pos, base)
    k_ref = oracle_mod.rope_normal(k, pos, base)
    host = oracle_mod.HostPagedKv(Hkv, hd, ps, kv_type, n_pages)
    assert host.append(k_ref, v, seq, pos, pt) == 0

    qg = tq.cpu().numpy()
    mag = (np.abs(q[..., 0::2]) + np.abs(q[..., 1::2])).astype(np.float64)
    err = np.maximum(np.abs(qg[..., 0::2] - q_ref[..., 0::2]), np.abs(qg[..., 1::2] - q_ref[..., 1::2]))
    assert np.all(err <= 1e-6 * mag + 1e-7), float(np.max(err / (mag + 1e-7)))

    kd = dev.k[0].cpu().numpy().reshape(n_pages, -1)
    vd = dev.v[0].cpu().numpy().reshape(n_pages, -1)
    assert np.array_equal(vd, host.v[:n_pages]), "V bytes differ from the oracle's append"
    if kv_type == F32:
        # the rotated K stored as is: the rotation bar of the Q check
        rows = _rows(kd, pt, seq, pos, ps, Hkv * hd * 4).view(np.float32).reshape(n, Hkv, hd)
        kmag = np.repeat(np.abs(k[..., 0::2]) + np.abs(k[..., 1::2]), 2, axis=-1).astype(np.float64)
        assert np.all(np.abs(rows - k_ref) <= 1e-6 * kmag + 1e-7), float(np.max(np.abs(rows - k_ref)))
    elif kv_type == F16:
        # per token: the device's f16 K row against the unrounded f32 oracle
        # rotation; f16 rounding (half an ulp, or 2^-25 below the normal
        # range) plus the rotation bar
        rows = _rows(kd, pt, seq, pos, ps, Hkv * hd * 2).view(np.uint16).reshape(n, Hkv, hd)
        got = oracle_mod.f16_bits_to_f32(rows)
        kmag = np.repeat(np.abs(k[..., 0::2]) + np.abs(k[..., 1::2]), 2, axis=-1).astype(np.float64)
        bound = 2.0 ** -11 * np.abs(k_ref) + 2.0 ** -25 + 1e-6 * kmag
        assert np.all(np.abs(got - k_ref) <= bound), float(np.max(np.abs(got - k_ref) - bound))
        ulps = _f16_ulps(kd.view(np.uint16), host.k[:n_pages].view(np.uint16))
        assert np.mean(ulps == 0) > 0.99
    else:
        rb = hd // 32 * 34
        rows_d = kd.reshape(-1, rb)
        rows_h = host.k[:n_pages].reshape(-1, rb)
        deq_d = oracle_mod.dequantize_q8_0(rows_d)
        deq_h = oracle_mod.dequantize_q8_0(rows_h)
        blk_d = rows_d.reshape(-1, 34)
        blk_h = rows_h.reshape(-1, 34)
        d_ulps = _f16_ulps(blk_d[:, :2].copy().view(np.uint16).ravel(), blk_h[:, :2].copy().view(np.uint16).ravel())
        assert d_ulps.max() <= 1, int(d_ulps.max())
        step = np.abs(oracle_mod.f16_bits_to_f32(blk_h[:, :2].copy().view(np.uint16).ravel()))
        step = np.repeat(step, 32).reshape(deq_h.shape) * (1 + 1e-3)
        assert np.all(np.abs(deq_d - deq_h) <= step + 1e-12)


def test_rope_append_skips_and_k_only(gpu, oracle_mod):
    """seq < 0 or pos < 0 skips a token (its Q row untouched, nothing written);
    q = NULL rotates only K."""
    import torch
    from strataflow_amd.paged_kv import PagedKV
    Hq, Hkv, hd, ps, n_pages = 8, 4, 64, 32, 6
    rng = np.random.default_rng(11)
    seq = np.array([0, -1, 0, 0], np.int32)
    pos = np.array([5, 6, -1, 40], np.int32)
    pt = np.array([[3, 1, 4, -1]], np.int32)
    q = rng.standard_normal((4, Hq, hd)).astype(np.float32)
    k = rng.standard_normal((4, Hkv, hd)).astype(np.float32)
    v = rng.standard_normal((4, Hkv, hd)).astype(np.float32)
    dev = PagedKV(1, Hq, Hkv, hd, F16, ps, n_pages, device=gpu)
    tq = torch.from_numpy(q).to(gpu)
    args = (torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu), torch.from_numpy(seq).to(gpu),
            torch.from_numpy(pos).to(gpu), torch.from_numpy(pt).to(gpu), 1e4)
    dev.rope_append(0, tq, *args)
    torch.cuda.synchronize()
    qg = tq.cpu().numpy()
    assert np.array_equal(qg[1], q[1]) and np.array_equal(qg[2], q[2])
    ref = oracle_mod.rope_normal(q[[0, 3]], pos[[0, 3]], 1e4)
    assert np.max(np.abs(qg[[0, 3]] - ref)) <= 1e-5
    host = oracle_mod.HostPagedKv(Hkv, hd, ps, F16, n_pages)
    keep = np.array([0, 3])
    assert host.append(oracle_mod.rope_normal(k[keep], pos[keep], 1e4), v[keep], seq[keep], pos[keep], pt) == 0
    kd = dev.k[0].cpu().numpy().reshape(n_pages, -1)
    assert _f16_ulps(kd.view(np.uint16), host.k[:n_pages].view(np.uint16)).max() <= 1
    # K only: Q untouched, the cache the same as with Q
    dev2 = PagedKV(1, Hq, Hkv, hd, F16, ps, n_pages, device=gpu)
    dev2.rope_append(0, None, *args)
    torch.cuda.synchronize()
    assert np.array_equal(dev2.k[0].cpu().numpy(), dev.k[0].cpu().numpy())


def test_rope_append_rejects_bad_arguments(gpu):
    import ctypes

    import torch
    from strataflow_amd import _lib
    from strataflow_amd.paged_kv import PagedKV
    dev = PagedKV(1, 8, 4, 64, F16, 32, 4, device=gpu)
    lib = _lib.load()
    d = dev.desc(0)
    x = torch.zeros((1, 4, 64), device=gpu)
    i = torch.zeros(1, dtype=torch.int32, device=gpu)
    pt = torch.zeros((1, 2), dtype=torch.int32, device=gpu)
    rc = lib.sfa_rope_kv_append(ctypes.byref(d), None, x.data_ptr(), x.data_ptr(), i.data_ptr(),
                                i.data_ptr(), 1, pt.data_ptr(), 2, 0.0, None)
    assert rc == _lib.SFA_ERR_INVALID_ARGUMENT
    rc = lib.sfa_rope_kv_append(ctypes.byref(d), None, None, x.data_ptr(), i.data_ptr(),
                                i.data_ptr(), 1, pt.data_ptr(), 2, 1e4, None)
    assert rc == _lib.SFA_ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("kv_type", [F32, F16])
@pytest.mark.parametrize("wdtype", ["f32", "f16"])
@pytest.mark.parametrize("shape,n_embd", [((32, 8, 128), 4096), ((8, 4, 32), 256), ((16, 8, 64), 512),
                                          ((8, 2, 64), 2056)])
def test_qkv_rope_append_equals_product_then_rope_append(gpu, kv_type, wdtype, shape, n_embd):
    """sfa_qkv_rope_kv_append gives the bits of sfa_mul_mat_vec followed by
    sfa_rope_kv_append on its Q, K and V parts: the rotated Q and every byte of
    both pools, with a skipped token (seq -1, Q as computed) and a token whose
    page id lies outside the pool (Q rotated, nothing written)."""
    import torch
    from strataflow_amd import layer
    from strataflow_amd.paged_kv import PagedKV
    Hq, Hkv, hd = shape
    rng = np.random.default_rng(11 * hd + kv_type + n_embd)
    ps, max_pages, n_seq = 64, 8, 2
    n_pages = n_seq * max_pages + 2
    seq, pos = _tokens(rng, n_seq, 6, ps, max_pages)
    pt = rng.permutation(n_pages)[:n_seq * max_pages].reshape(n_seq, max_pages).astype(np.int32)
    seq[1] = -1
    pt[seq[2], pos[2] // ps] = n_pages + 5
    n = seq.size
    n_out = (Hq + 2 * Hkv) * hd
    w = (rng.standard_normal((n_out, n_embd)) / np.sqrt(n_embd)).astype(np.float32)
    if wdtype == "f16":
        w = w.astype(np.float16)
    x = rng.standard_normal((n, n_embd)).astype(np.float32)
    base = 1e6 if hd == 128 else 1e4
    tw, tx = torch.from_numpy(w).to(gpu), torch.from_numpy(x).to(gpu)
    ts, tp, tpt = (torch.from_numpy(a).to(gpu) for a in (seq, pos, pt))
    a = PagedKV(1, Hq, Hkv, hd, kv_type, ps, n_pages, device=gpu)
    b = PagedKV(1, Hq, Hkv, hd, kv_type, ps, n_pages, device=gpu)
    qa = a.qkv_rope_append(0, tw, tx, ts, tp, tpt, base)
    qkv = layer.mul_mat_vec(tw, tx)
    qb = qkv[:, :Hq * hd].contiguous().view(n, Hq, hd)
    kb = qkv[:, Hq * hd:(Hq + Hkv) * hd].contiguous().view(n, Hkv, hd)
    vb = qkv[:, (Hq + Hkv) * hd:].contiguous().view(n, Hkv, hd)
    b.rope_append(0, qb, kb, vb, ts, tp, tpt, base)
    torch.cuda.synchronize()
    assert np.array_equal(qa.cpu().numpy().view(np.uint32), qb.cpu().numpy().view(np.uint32))
    assert np.array_equal(a.k[0].cpu().numpy(), b.k[0].cpu().numpy())
    assert np.array_equal(a.v[0].cpu().numpy(), b.v[0].cpu().numpy())
    # the skipped token's Q is the product as computed, and something was written
    assert np.array_equal(qa[1].cpu().numpy().ravel(), qkv[1, :Hq * hd].cpu().numpy())
    assert a.k[0].abs().sum().item() > 0
