"""The decode node with its consumer fused in (sfa_attn_decode_wo): y = wo * attn
+ residual (src/model/engine/engine.cpp:1904-1906), through the C ABI.

References, both in float64 on the host:
- ggml semantics: the oracle's attention (ggml mode), converted as ggml's mul_mat
  converts src1 for the weight type (F16 weights: rounded to f16), times the
  weights, plus the residual: the projection (y - residual) within the parity
  bar (max-abs 2e-3, rel-L2 1e-3);
- the same projection of the GPU's own sfa_attn_decode output: only the f32
  summation order of the dot products differs (rel-L2 1e-5), which pins the
  fused merge to the two-pass decode's arithmetic.
Replays of a captured call rewrite seq_len in place and must equal eager calls
bit for bit (the arrival counters reset themselves)."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import Case, assert_close

pytestmark = pytest.mark.gpu


def _f16_round(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def _weights(rng, n_embd, k, wdtype):
    w = (rng.standard_normal((n_embd, k)) / np.sqrt(k)).astype(np.float32)
    return w.astype(np.float16) if wdtype == "f16" else w


def _project(attn, w, x, wdtype):
    a = _f16_round(attn) if wdtype == "f16" else np.asarray(attn, np.float64)
    return a @ np.asarray(w, np.float64).T + np.asarray(x, np.float64)


@pytest.mark.parametrize("wdtype", ["f16", "f32"])
@pytest.mark.parametrize("shape,n_embd,lens,kv_type", [
    ((32, 8, 128), 4096, [4096], 1),            # the decode workload's shape, B = 1
    ((32, 8, 128), 4096, [3000, 0, 777], 1),    # a batch with an empty sequence
    ((32, 8, 128), 1000, [9000, 1], 8),         # Q8_0 cache; n_embd not a multiple of 64
    ((8, 4, 32), 256, [96, 40], 1),             # the tiny-MoE attention shape
    ((32, 4, 128), 1024, [2000, 333, 5], 0),    # g = 8, the F32 cache
])
def test_decode_wo_vs_float64(gpu, oracle_mod, shape, n_embd, lens, kv_type, wdtype):
    import torch
    Hq, Hkv, hd = shape
    c = Case(oracle_mod, seq_lens=lens, n_head=Hq, n_head_kv=Hkv, head_dim=hd, kv_type=kv_type,
             seed=sum(lens) + n_embd)
    rng = np.random.default_rng(n_embd + hd)
    w = _weights(rng, n_embd, Hq * hd, wdtype)
    x = rng.standard_normal((c.B, n_embd)).astype(np.float32)
    tw, tx = torch.from_numpy(w).to(gpu), torch.from_numpy(x).to(gpu)
    M = max(max(lens), 1)
    y = c.dev.decode_wo(0, c.t_q, c.t_pt, c.t_sl, M, tw, tx).cpu().numpy()
    # against ggml semantics (the oracle's attention)
    ref = _project(c.oracle(oracle_mod.GGML), w, x, wdtype)
    ma, rl = assert_close(y - x, ref - x, what=f"{shape} {wdtype} projection vs ggml")
    # against the GPU's own two-pass decode output: summation order only (the
    # merge passes add split groups, the fused one splits in order); with f16
    # weights both round O to f16 first, so a last-ulp order difference can
    # move one rounding by 2^-11 of that value
    attn = c.decode(max_seq_len=M)
    own = _project(attn, w, x, wdtype)
    assert_close(y - x, own - x, max_abs=1e-5, rel_l2=5e-5 if wdtype == "f16" else 1e-5,
                 what="projection vs own decode")
    assert np.all(np.isfinite(y))
    # deterministic: a second call gives the same bits
    y2 = c.dev.decode_wo(0, c.t_q, c.t_pt, c.t_sl, M, tw, tx).cpu().numpy()
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    print(f"{shape} {wdtype} B={c.B}: projection vs ggml max_abs {ma:.2e} rel_l2 {rl:.2e}")


def test_decode_wo_graph_replay(gpu, oracle_mod):
    import torch
    lens = np.array([2500, 900], np.int32)
    c = Case(oracle_mod, seq_lens=lens, seed=501)
    rng = np.random.default_rng(502)
    n_embd = 4096
    w = torch.from_numpy(_weights(rng, n_embd, 32 * 128, "f16")).to(gpu)
    x = torch.from_numpy(rng.standard_normal((2, n_embd)).astype(np.float32)).to(gpu)
    sl = c.t_sl.clone()
    y = torch.empty((2, n_embd), device=gpu)

    def call(out):
        c.dev.decode_wo(0, c.t_q, c.t_pt, sl, 2500, w, x, y=out)

    call(y)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(y)
    for n in ([2500, 900], [1, 899], [2400, 0], [2500, 900]):
        sl.copy_(torch.tensor(n, dtype=torch.int32))
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        e = torch.empty_like(y)
        call(e)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), e.view(torch.int32)), n


def test_decode_wo_rejects(gpu, oracle_mod):
    import ctypes
    import torch
    from strataflow_amd import _lib
    lib = _lib.load()
    c = Case(oracle_mod, seq_lens=[100], seed=503)
    d = c.dev.desc(0)
    s = torch.cuda.current_stream().cuda_stream
    y = torch.empty((1, 64), device=gpu)
    w = torch.empty((64, 4096), device=gpu)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=gpu)
    args = lambda wt, n_embd, wsb: (ctypes.byref(d), c.t_q.data_ptr(), c.t_pt.data_ptr(), c.max_pages,
                                    c.t_sl.data_ptr(), None, 1, 100, 0.088, w.data_ptr(), wt, n_embd,
                                    y.data_ptr(), y.data_ptr(), ws.data_ptr(), wsb, s)
    assert lib.sfa_attn_decode_wo(*args(8, 64, ws.numel())) == _lib.SFA_ERR_UNSUPPORTED   # Q8_0 weights
    assert lib.sfa_attn_decode_wo(*args(1, 0, ws.numel())) == _lib.SFA_ERR_INVALID_ARGUMENT
    assert lib.sfa_attn_decode_wo(*args(1, 64, 16)) == _lib.SFA_ERR_INVALID_ARGUMENT    # small workspace
    assert lib.sfa_decode_wo_workspace_bytes(ctypes.byref(d), 1, 100, 64) <= ws.numel()
