"""Seeded random chunked-prefill cases through sfa_attn_prefill against the
ggml-semantics oracle with the causal mask (max-abs <= 2e-3, rel-L2 <= 1e-3):
KV type (F32, F16, Q8_0 at head_dim >= 64), head shape (g = 1..8), history
length, chunk length (1..300), page size (a multiple of the 64-position tile)
and window start."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import assert_close
from tests.test_gpu_prefill import build, run

pytestmark = pytest.mark.gpu

SHAPES = [(32, 8, 128), (8, 2, 128), (8, 4, 64), (8, 8, 128), (12, 6, 64), (4, 1, 128), (32, 4, 128),
          (16, 16, 64), (8, 4, 32)]


def _cases(n=24, seed=5):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        Hq, Hkv, hd = SHAPES[rng.integers(len(SHAPES))]
        kv_type = int(rng.choice([0, 1, 8])) if hd >= 64 else int(rng.choice([0, 1]))
        n_cached = int(rng.integers(0, 601))
        T = int(rng.integers(1, 301))
        page = int(rng.choice([64, 128, 256]))
        kv_lo = int(rng.integers(0, n_cached + 1)) if rng.random() < 0.3 else 0
        out.append((i, (Hq, Hkv, hd), kv_type, n_cached, T, page, kv_lo))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"case{c[0]}")
def test_prefill_random_case(gpu, oracle_mod, case):
    i, (Hq, Hkv, hd), kv_type, n_cached, T, page, kv_lo = case
    host, dev, pt, q, n_kv = build(oracle_mod, gpu, Hq=Hq, Hkv=Hkv, hd=hd, n_cached=n_cached, T=T,
                                   page_size=page, seed=500 + i, kv_type=kv_type)
    out = run(dev, gpu, pt, q, n_cached, kv_lo)
    ref = host.attention(q[None], Hq, pt, np.array([n_kv], np.int32), np.array([kv_lo], np.int32),
                         T=T, mode=oracle_mod.GGML)[0].reshape(T, -1)
    assert_close(out, ref, what=f"case {i}: shape {(Hq, Hkv, hd)} type {kv_type} cached {n_cached} T {T} "
                                f"page {page} lo {kv_lo}")
