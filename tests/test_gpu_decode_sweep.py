"""Seeded random decode cases through sfa_attn_decode against the ggml-semantics
oracle (max-abs <= 2e-3, rel-L2 <= 1e-3): KV type (F32, F16, Q8_0), head shape
(g = 1..8, head_dim 32/64/128), batch (1..70; Q8_0 batches of two or more with
>= 1024 tiles take the column layout), page size, lengths including empty
sequences, window starts, and a max_seq_len below or above the longest span."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import Case, assert_close

pytestmark = pytest.mark.gpu

SHAPES = [(32, 8, 128), (8, 2, 128), (8, 4, 64), (8, 8, 128), (12, 6, 64), (4, 1, 128), (16, 2, 128),
          (16, 16, 64), (8, 4, 32)]


def _cases(n=40, seed=11):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        Hq, Hkv, hd = SHAPES[rng.integers(len(SHAPES))]
        kv_type = int(rng.choice([0, 1, 8])) if hd >= 64 else int(rng.choice([0, 1]))
        B = int(rng.choice([1, 2, 3, 8, 33, 40, 70]))
        page = int(rng.choice([32, 64, 256]))
        mx = int(rng.choice([40, 300, 1000, 1200]))
        seq = rng.integers(0, mx + 1, B)
        if rng.random() < 0.5:
            seq[rng.integers(B)] = mx
        lo = None
        if rng.random() < 0.3:
            lo = np.where(rng.random(B) < 0.5, rng.integers(0, max(mx // 2, 1), B), 0)
            lo = np.minimum(lo, np.maximum(seq - 1, 0)).astype(np.int32)
        msl = max(int(max(int(seq.max()), 1) * rng.choice([1.0, 1.0, 0.5, 2.0])), 1)
        out.append((i, (Hq, Hkv, hd), kv_type, seq, lo, page, msl))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"case{c[0]}")
def test_decode_random_case(gpu, oracle_mod, case):
    i, (Hq, Hkv, hd), kv_type, seq, lo, page, msl = case
    c = Case(oracle_mod, seq_lens=seq, kv_lo=lo, n_head=Hq, n_head_kv=Hkv, head_dim=hd, kv_type=kv_type,
             page_size=page, seed=1000 + i)
    out = c.decode(max_seq_len=msl)
    assert_close(out, c.oracle(oracle_mod.GGML),
                 what=f"case {i}: shape {(Hq, Hkv, hd)} type {kv_type} B {len(seq)} page {page} msl {msl}")
    assert np.all(out[np.asarray(seq) == 0] == 0)
