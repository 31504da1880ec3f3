"""Writes the attention golden vectors (tests/golden/*.npz).

An independent float64 restatement in numpy of the reference attention node
(src/model/engine/engine.cpp:1751-1761): s = scale * q.k over the history of
the query's kv head (h // g), softmax over positions kv_lo..qpos, o = p.v.
Two expected outputs per case:
  exact - K/V as stored (f16 values, or Q8_0 dequantised d*q), Q as given;
  ggml  - with ggml's CPU operand conversions: for F16 K, Q rounded to f16;
          for Q8_0 K, Q quantised to Q8_0 (d = amax/127, q = round(x/d), half
          away from zero) with the dot taken on the integer codes; for F16 V,
          the normalised P rounded to f16 before P.V.
Inputs are seeded; the cache is given in the column layout [n_kv][Hkv][hd]
(f16 values or Q8_0 bytes) so a reader can place it in any page order.

Run: python tests/golden/make_golden.py   (numpy only)
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def q8_quant(x: np.ndarray):
    """Per 32-block Q8_0 of x [..., k]: returns (d as float16, q int8)."""
    xb = x.reshape(x.shape[:-1] + (-1, 32)).astype(np.float32)
    amax = np.abs(xb).max(axis=-1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    y = (xb * inv[..., None]).astype(np.float32)
    q = (np.sign(y) * np.floor(np.abs(y) + 0.5)).astype(np.int8)  # roundf: half away from 0
    return d.astype(np.float16), q


def q8_bytes(d16: np.ndarray, q: np.ndarray) -> np.ndarray:
    nb = q.shape[-2]
    out = np.empty(q.shape[:-2] + (nb * 34,), np.uint8)
    for b in range(nb):
        out[..., b * 34:b * 34 + 2] = d16[..., b:b + 1].view(np.uint8).reshape(d16.shape[:-1] + (2,))
        out[..., b * 34 + 2:b * 34 + 34] = q[..., b, :].view(np.uint8)
    return out


def attention(q, k, v, g, qpos, lo, scale, k_q8=None, f16_p=False, q_round=None):
    """q [T, Hq, hd]; k, v [n_kv, Hkv, hd] float64; returns [T, Hq, hd]."""
    T, Hq, hd = q.shape
    out = np.zeros((T, Hq, hd))
    for t in range(T):
        hi = qpos[t] + 1
        if hi <= lo:
            continue
        for h in range(Hq):
            kvh = h // g
            qr = q[t, h].astype(np.float64)
            if q_round == "f16":
                qr = qr.astype(np.float16).astype(np.float64)
            if q_round == "q8":
                dq, qq = q8_quant(q[t, h].astype(np.float32))
                kd, kq = k_q8
                sdot = np.einsum("jbi,bi->jb", kq[lo:hi, kvh].astype(np.int64), qq.astype(np.int64))
                s = (sdot * (kd[lo:hi, kvh].astype(np.float64) * dq.astype(np.float64))).sum(-1)
            else:
                s = k[lo:hi, kvh] @ qr
            s = s * scale
            p = np.exp(s - s.max())
            p = p / p.sum()
            if f16_p:
                p = p.astype(np.float16).astype(np.float64)
            out[t, h] = p @ v[lo:hi, kvh]
    return out


def make_case(name, seed, Hq, Hkv, hd, n_kv, T, lo, kv_type):
    rng = np.random.default_rng(seed)
    g = Hq // Hkv
    scale = 1.0 / np.sqrt(hd)
    q = rng.standard_normal((T, Hq, hd)).astype(np.float32)
    kf = rng.standard_normal((n_kv, Hkv, hd)).astype(np.float32)
    vf = rng.standard_normal((n_kv, Hkv, hd)).astype(np.float32)
    qpos = np.arange(n_kv - T, n_kv)
    case = dict(q=q, qpos=qpos.astype(np.int32), kv_lo=np.int32(lo), n_head=np.int32(Hq),
                scale=np.float32(scale), kv_type=np.int32(kv_type))
    if kv_type == 1:
        k16, v16 = kf.astype(np.float16), vf.astype(np.float16)
        case.update(k_f16=k16, v_f16=v16)
        k64, v64 = k16.astype(np.float64), v16.astype(np.float64)
        case["exact"] = attention(q, k64, v64, g, qpos, lo, scale).astype(np.float32)
        case["ggml"] = attention(q, k64, v64, g, qpos, lo, scale, f16_p=True,
                                 q_round="f16").astype(np.float32)
    else:
        kd, kq = q8_quant(kf)
        vd, vq = q8_quant(vf)
        case.update(k_f32=kf, v_f32=vf, k_q8=q8_bytes(kd, kq), v_q8=q8_bytes(vd, vq))
        k64 = (kq.astype(np.float64) * kd.astype(np.float64)[..., None]).reshape(n_kv, Hkv, hd)
        v64 = (vq.astype(np.float64) * vd.astype(np.float64)[..., None]).reshape(n_kv, Hkv, hd)
        case["exact"] = attention(q, k64, v64, g, qpos, lo, scale).astype(np.float32)
        case["ggml"] = attention(q, k64, v64, g, qpos, lo, scale, k_q8=(kd, kq),
                                 q_round="q8").astype(np.float32)
    np.savez_compressed(HERE / f"{name}.npz", **case)
    print(f"wrote {name}.npz")


def main():
    make_case("attn_f16_gqa2_decode", 11, Hq=4, Hkv=2, hd=32, n_kv=70, T=1, lo=0, kv_type=1)
    make_case("attn_f16_gqa4_window", 12, Hq=8, Hkv=2, hd=64, n_kv=120, T=1, lo=37, kv_type=1)
    make_case("attn_f16_mha_prefill", 13, Hq=2, Hkv=2, hd=32, n_kv=96, T=40, lo=0, kv_type=1)
    make_case("attn_q8_gqa4_decode", 14, Hq=8, Hkv=2, hd=128, n_kv=100, T=1, lo=0, kv_type=8)
    make_case("attn_q8_gqa2_prefill", 15, Hq=4, Hkv=2, hd=64, n_kv=64, T=16, lo=5, kv_type=8)


if __name__ == "__main__":
    main()
