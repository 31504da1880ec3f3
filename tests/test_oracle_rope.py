"""Pins the oracle's RoPE NORMAL (orc_rope_normal, the restatement of
ggml_rope_ext mode 0 that engine.cpp:1892-1897 applies to Qcur and Kcur)
against what the mathematics fixes: position 0 is the identity, a one-pair
known answer, float64 rotations by the same f32 theta sequence, the closed form
theta_i = pos * base^(-2i/n_dims) at small positions, pair-norm preservation and
the relative-position property of the rotated dot product."""
from __future__ import annotations

import ctypes
import ctypes.util

import numpy as np
import pytest


def _powf(x: float, y: float) -> np.float32:
    """C powf (the f32 pow ggml calls); the theta recurrence amplifies a one-ulp
    difference in its factor, so numpy's own float32 power is not a substitute."""
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    libm.powf.restype = ctypes.c_float
    return np.float32(libm.powf(x, y))


def _thetas_f32(pos, hd, base):
    """ggml's recurrence: theta_0 = pos, theta_{i+1} = theta_i * powf(base, -2/hd) in f32."""
    scale = _powf(np.float32(base), np.float32(-2.0) / np.float32(hd))
    th = np.empty((len(pos), hd // 2), np.float32)
    cur = np.asarray(pos, np.float32).copy()
    for i in range(hd // 2):
        th[:, i] = cur
        cur = (cur * scale).astype(np.float32)
    return th


def _rotate_f64(x, th):
    x = np.asarray(x, np.float64)
    c, s = np.cos(th.astype(np.float64))[:, None, :], np.sin(th.astype(np.float64))[:, None, :]
    out = np.empty_like(x)
    out[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
    out[..., 1::2] = x[..., 0::2] * s + x[..., 1::2] * c
    return out


def test_position_zero_is_identity(oracle_mod):
    x = np.random.default_rng(0).standard_normal((3, 4, 64)).astype(np.float32)
    y = oracle_mod.rope_normal(x, np.zeros(3, np.int32), 1e6)
    assert np.array_equal(y, x)


def test_one_pair_known_answer(oracle_mod):
    # head_dim 2: one pair rotated by theta = pos
    x = np.array([[[0.75, -1.5]]], np.float32)
    y = oracle_mod.rope_normal(x, np.array([1], np.int32), 10000.0)
    c, s = np.cos(1.0), np.sin(1.0)
    want = np.array([0.75 * c + 1.5 * s, 0.75 * s - 1.5 * c])
    np.testing.assert_allclose(y[0, 0], want, rtol=0, atol=4e-7)


@pytest.mark.parametrize("hd,base", [(128, 1e6), (32, 1e4), (64, 5e5)])
def test_matches_float64_rotation_of_ggml_thetas(oracle_mod, hd, base):
    rng = np.random.default_rng(hd)
    pos = np.concatenate([np.arange(0, 40), rng.integers(0, 70000, 60)]).astype(np.int32)
    x = rng.standard_normal((pos.size, 3, hd)).astype(np.float32)
    y = oracle_mod.rope_normal(x, pos, base)
    want = _rotate_f64(x, _thetas_f32(pos, hd, base))
    mag = np.abs(x[..., 0::2]).astype(np.float64) + np.abs(x[..., 1::2])
    err = np.maximum(np.abs(y[..., 0::2] - want[..., 0::2]), np.abs(y[..., 1::2] - want[..., 1::2]))
    assert np.all(err <= 1e-6 * mag + 1e-7), float(np.max(err / (mag + 1e-7)))


def test_closed_form_at_small_positions(oracle_mod):
    hd, base = 128, 1e6
    pos = np.arange(0, 48, dtype=np.int32)
    x = np.random.default_rng(3).standard_normal((pos.size, 2, hd)).astype(np.float32)
    y = oracle_mod.rope_normal(x, pos, base)
    i = np.arange(hd // 2)
    th = pos[:, None].astype(np.float64) * np.power(base, -2.0 * i / hd)[None, :]
    want = _rotate_f64(x, th)
    assert np.max(np.abs(y - want)) <= 5e-5


def test_pair_norms_preserved(oracle_mod):
    rng = np.random.default_rng(5)
    pos = rng.integers(0, 1 << 16, 50).astype(np.int32)
    x = rng.standard_normal((50, 4, 128)).astype(np.float32)
    y = oracle_mod.rope_normal(x, pos, 1e6)
    n_in = np.hypot(x[..., 0::2], x[..., 1::2]).astype(np.float64)
    n_out = np.hypot(y[..., 0::2].astype(np.float64), y[..., 1::2])
    np.testing.assert_allclose(n_out, n_in, rtol=2e-6, atol=1e-7)


def test_dot_depends_on_relative_position(oracle_mod):
    rng = np.random.default_rng(7)
    hd = 128
    q = rng.standard_normal((1, 1, hd)).astype(np.float32)
    k = rng.standard_normal((1, 1, hd)).astype(np.float32)
    dots = []
    for shift in (0, 17, 150):
        rq = oracle_mod.rope_normal(q, np.array([40 + shift], np.int32), 1e4)
        rk = oracle_mod.rope_normal(k, np.array([12 + shift], np.int32), 1e4)
        dots.append(float(np.dot(rq.ravel().astype(np.float64), rk.ravel())))
    scale = float(np.linalg.norm(q) * np.linalg.norm(k))
    assert max(dots) - min(dots) <= 1e-4 * scale, dots


def test_numpy_restatement_agrees(oracle_mod):
    from strataflow_amd import synth
    rng = np.random.default_rng(9)
    pos = rng.integers(0, 40000, 30).astype(np.int32)
    x = rng.standard_normal((30, 2, 64)).astype(np.float32)
    a = oracle_mod.rope_normal(x, pos, 1e6)
    b = synth.rope_normal(x, pos, 1e6)
    np.testing.assert_allclose(a, b, rtol=0, atol=2e-6 * float(np.abs(x).max()))
