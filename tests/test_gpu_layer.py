"""The decode layer's non-attention ops on the GPU (include/sfa_layer.h), each
against a float64 numpy restatement of ggml's CPU arithmetic for it
(build_router_segment / build_expert_segment, src/model/engine/engine.cpp:
1877-1925, 1945-1986), plus closed forms that a wrong index, operand or
order would fail:
- rms_norm: a constant row normalises to +-weight / sqrt(1 + eps/c^2);
- mul_mat_vec: a one-hot activation returns a weight column exactly (f32
  weights) or its f16 value (f16 weights);
- routing: the top-k ids exactly, ties to the lower id, weights that sum to 1;
- experts: one slot of weight 1 equals the plain SwiGLU FFN; an id outside
  the stack adds nothing.
Tolerances: f32 products summed in f32 over n_in terms (1e-5 of the row's
RMS); f16 weights take the activation rounded to f16 as ggml does, and the
reference rounds it the same way.  The SwiGLU activations feed the down
product rounded to f16 with f16 weights, where an f32 last-ulp difference can
move a rounding: 2e-4 there, 2e-5 with f32 weights."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def _rms_ref(x, w, eps):
    x = x.astype(np.float32)
    ss = np.sum((x * x).astype(np.float64), axis=-1, keepdims=True)   # f32 squares, double sum
    mean = (ss / x.shape[-1]).astype(np.float32)
    scale = (np.float32(1.0) / np.sqrt(mean + np.float32(eps))).astype(np.float32)
    return ((x * scale).astype(np.float32) * w).astype(np.float32)


def _mm_ref(w, x, f16):
    xx = x.astype(np.float16).astype(np.float64) if f16 else x.astype(np.float64)
    return xx @ np.asarray(w, np.float64).T


@pytest.mark.parametrize("n_rows,n", [(1, 256), (3, 4096), (2, 100)])
def test_rms_norm(gpu, n_rows, n):
    from strataflow_amd import layer
    rng = np.random.default_rng(n + n_rows)
    x = (rng.standard_normal((n_rows, n)) * 3).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    y = layer.rms_norm(_t(x, gpu), _t(w, gpu), 1e-5).cpu().numpy()
    ref = _rms_ref(x, w, 1e-5)
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-6)) < 2e-6
    # a constant row c: y = w * c / sqrt(c^2 + eps)
    c = np.full((1, n), -2.5, np.float32)
    yc = layer.rms_norm(_t(c, gpu), _t(w, gpu), 1e-5).cpu().numpy()[0]
    assert np.allclose(yc, -w / np.sqrt(1 + 1e-5 / 6.25), rtol=1e-6, atol=0)
    # in place
    tx = _t(x, gpu)
    layer.rms_norm(tx, _t(w, gpu), 1e-5, out=tx)
    assert np.array_equal(tx.cpu().numpy(), y)


@pytest.mark.parametrize("wdtype", ["f32", "f16"])
@pytest.mark.parametrize("n_rows,n_in,n_out", [(1, 256, 512), (1, 4096, 1000), (3, 512, 8),
                                               (8, 256, 4096), (13, 1024, 256), (1, 14336, 64),
                                               (1, 2056, 300)])  # whole load batches + one chunk more
def test_mul_mat_vec(gpu, wdtype, n_rows, n_in, n_out):
    import torch
    from strataflow_amd import layer
    rng = np.random.default_rng(n_in * 7 + n_out + n_rows)
    w = (rng.standard_normal((n_out, n_in)) / np.sqrt(n_in)).astype(np.float32)
    if wdtype == "f16":
        w = w.astype(np.float16)
    x = rng.standard_normal((n_rows, n_in)).astype(np.float32)
    r = rng.standard_normal((n_rows, n_out)).astype(np.float32)
    tw, tx = _t(w, gpu), _t(x, gpu)
    y = layer.mul_mat_vec(tw, tx).cpu().numpy()
    ref = _mm_ref(w, x, wdtype == "f16")
    scale = np.sqrt(np.sum(np.square(ref), axis=-1, keepdims=True) / n_out) + 1e-30
    assert np.max(np.abs(y - ref) / scale) < 1e-5, wdtype
    # with the residual (ggml_add after the product), in place on the residual
    tr = _t(r, gpu)
    layer.mul_mat_vec(tw, tx, residual=tr, out=tr)
    yr = tr.cpu().numpy()
    assert np.array_equal(yr, (y + r).astype(np.float32))
    # one-hot activations pick weight columns exactly
    cols = rng.integers(0, n_in, n_rows)
    oh = np.zeros((n_rows, n_in), np.float32)
    oh[np.arange(n_rows), cols] = 1.0
    yo = layer.mul_mat_vec(tw, _t(oh, gpu)).cpu().numpy()
    assert np.array_equal(yo, np.asarray(w, np.float32)[:, cols].T)
    torch.cuda.synchronize()


def _route_ref(logits, k):
    m = logits.max(-1, keepdims=True)
    e = np.exp((logits - m).astype(np.float64))
    p = (e / e.sum(-1, keepdims=True)).astype(np.float32)
    sel = np.argsort(-p, axis=-1, kind="stable")[:, :k]
    ws = np.take_along_axis(p, sel, -1).astype(np.float64)
    s = np.maximum(ws.sum(-1, keepdims=True), 6.103515625e-5)
    return sel, (ws / s).astype(np.float32)


@pytest.mark.parametrize("n_rows,n_expert,k", [(1, 8, 2), (5, 8, 2), (4, 64, 6), (3, 3, 3), (2, 16, 1)])
def test_moe_route(gpu, n_rows, n_expert, k):
    from strataflow_amd import layer
    rng = np.random.default_rng(n_expert * 10 + k)
    logits = (rng.standard_normal((n_rows, n_expert)) * 2).astype(np.float32)
    ids, w = layer.moe_route(_t(logits, gpu), k)
    ids, w = ids.cpu().numpy(), w.cpu().numpy()
    sel, wref = _route_ref(logits, k)
    assert np.array_equal(ids, sel)
    assert np.allclose(w, wref, rtol=2e-6, atol=1e-7)
    assert np.allclose(w.sum(-1), 1.0, atol=2e-6)
    assert np.all(np.diff(w, axis=-1) <= 0)  # descending


def test_moe_route_ties(gpu):
    from strataflow_amd import layer
    logits = np.array([[0.5, 2.0, 2.0, -1.0, 2.0, 0.0, 0.0, 0.0]], np.float32)
    ids, w = layer.moe_route(_t(logits, gpu), 3)
    assert ids.cpu().numpy().tolist() == [[1, 2, 4]]
    assert np.allclose(w.cpu().numpy(), 1.0 / 3.0, rtol=1e-6)


def _silu(x):
    return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def _moe_ref(x, res, ids, wts, g, u, d, f16):
    """ggml order: act = silu(gate*x) * (up*x) per slot; the down products times
    their weights, added in slot order; + residual.  F16 weights take x and act
    rounded to f16."""
    out = np.zeros_like(res, dtype=np.float64)
    for t in range(x.shape[0]):
        acc = None
        for j in range(ids.shape[1]):
            e = int(ids[t, j])
            if not 0 <= e < g.shape[0]:
                v = np.zeros(res.shape[1])
            else:
                gv = _mm_ref(g[e], x[t:t + 1], f16)[0].astype(np.float32)
                uv = _mm_ref(u[e], x[t:t + 1], f16)[0].astype(np.float32)
                act = (_silu(gv) * uv).astype(np.float32)
                v = _mm_ref(d[e], act[None], f16)[0] * float(wts[t, j])
            acc = v if acc is None else acc + v
        out[t] = acc + res[t]
    return out


@pytest.mark.parametrize("wdtype", ["f32", "f16"])
@pytest.mark.parametrize("n_rows,n_embd,n_ff,n_expert,k", [(1, 256, 512, 8, 2), (3, 512, 1024, 8, 2),
                                                            (2, 4096, 1024, 4, 4), (1, 128, 2048, 16, 1),
                                                            (1, 4160, 2560, 8, 2)])  # batches + chunks left
def test_moe_ffn(gpu, wdtype, n_rows, n_embd, n_ff, n_expert, k):
    from strataflow_amd import layer
    rng = np.random.default_rng(n_embd + n_ff + k)
    g = (rng.standard_normal((n_expert, n_ff, n_embd)) / np.sqrt(n_embd)).astype(np.float32)
    u = (rng.standard_normal((n_expert, n_ff, n_embd)) / np.sqrt(n_embd)).astype(np.float32)
    d = (rng.standard_normal((n_expert, n_embd, n_ff)) / np.sqrt(n_ff)).astype(np.float32)
    if wdtype == "f16":
        g, u, d = g.astype(np.float16), u.astype(np.float16), d.astype(np.float16)
    x = rng.standard_normal((n_rows, n_embd)).astype(np.float32)
    res = rng.standard_normal((n_rows, n_embd)).astype(np.float32)
    ids = np.stack([rng.permutation(n_expert)[:k] for _ in range(n_rows)]).astype(np.int32)
    wts = rng.dirichlet(np.ones(k), n_rows).astype(np.float32)
    tg, tu, td = _t(g, gpu), _t(u, gpu), _t(d, gpu)
    y = layer.moe_ffn(_t(x, gpu), _t(res, gpu), _t(ids, gpu), _t(wts, gpu), tg, tu, td).cpu().numpy()
    ref = _moe_ref(x, res, ids, wts, g, u, d, wdtype == "f16")
    # f16 weights: the activations are rounded to f16 before the down product
    # on both sides, and a one-ulp difference in an f32 activation can move that
    # rounding by one f16 ulp (5e-4 relative) for a few elements
    tol = (2e-4 if wdtype == "f16" else 2e-5)
    assert np.max(np.abs(y - ref)) < tol * max(1.0, float(np.max(np.abs(ref)))), wdtype
    # one slot of weight 1 is the plain SwiGLU FFN
    one = layer.moe_ffn(_t(x, gpu), _t(np.zeros_like(res), gpu), _t(ids[:, :1].copy(), gpu),
                        _t(np.ones((n_rows, 1), np.float32), gpu), tg, tu, td).cpu().numpy()
    ref1 = _moe_ref(x, np.zeros_like(res), ids[:, :1], np.ones((n_rows, 1)), g, u, d, wdtype == "f16")
    assert np.max(np.abs(one - ref1)) < tol * max(1.0, float(np.max(np.abs(ref1))))
    # an id outside the stack adds nothing (the other slots are unchanged)
    bad = ids.copy()
    bad[:, 0] = n_expert + 5
    yb = layer.moe_ffn(_t(x, gpu), _t(res, gpu), _t(bad, gpu), _t(wts, gpu), tg, tu, td).cpu().numpy()
    refb = _moe_ref(x, res, bad, wts, g, u, d, wdtype == "f16")
    assert np.max(np.abs(yb - refb)) < tol * max(1.0, float(np.max(np.abs(refb))))


def test_layer_ops_in_a_graph(gpu):
    """The ops replay from a captured HIP graph with the same bits as eager calls."""
    import torch
    from strataflow_amd import layer
    rng = np.random.default_rng(77)
    n_embd, n_ff, E, k = 256, 512, 8, 2
    w_in = _t((rng.standard_normal((E, n_embd)) * 0.1).astype(np.float32), gpu)
    g = _t((rng.standard_normal((E, n_ff, n_embd)) * 0.05).astype(np.float32), gpu)
    u = _t((rng.standard_normal((E, n_ff, n_embd)) * 0.05).astype(np.float32), gpu)
    d = _t((rng.standard_normal((E, n_embd, n_ff)) * 0.05).astype(np.float32), gpu)
    nw = _t(np.ones(n_embd, np.float32), gpu)
    x = _t(rng.standard_normal((1, n_embd)).astype(np.float32), gpu)
    ws = torch.empty(4 * k * n_ff, dtype=torch.uint8, device=gpu)
    cur, logits, y = (torch.empty((1, n_embd), device=gpu), torch.empty((1, E), device=gpu),
                      torch.empty((1, n_embd), device=gpu))
    ids = torch.empty((1, k), dtype=torch.int32, device=gpu)
    wts = torch.empty((1, k), device=gpu)

    def step():
        layer.rms_norm(x, nw, 1e-5, out=cur)
        layer.mul_mat_vec(w_in, cur, out=logits)
        layer.moe_route(logits, k, ids=ids, weights=wts)
        layer.moe_ffn(cur, x, ids, wts, g, u, d, out=y, workspace=ws)

    step()
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        step()
    for s in range(3):
        x.copy_(torch.from_numpy(rng.standard_normal((1, n_embd)).astype(np.float32)))
        y.fill_(float("nan"))
        gr.replay()
        torch.cuda.synchronize()
        got = y.clone()
        step()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), y.view(torch.int32)), s


@pytest.mark.parametrize("wdtype", ["f32", "f16"])
@pytest.mark.parametrize("n_rows,n_embd,n_expert,k", [(1, 4096, 8, 2), (3, 256, 8, 2), (2, 512, 64, 6),
                                                      (1, 128, 3, 3), (2, 8192, 8, 2)])
def test_moe_norm_gate_equals_norm_then_gate(gpu, wdtype, n_rows, n_embd, n_expert, k):
    """ffn_norm + router + routing in one launch gives the bits of sfa_rms_norm
    then sfa_moe_gate: the normed rows, the ids and the weights; and the normed
    rows match the float64 restatement of ggml's rms_norm."""
    from strataflow_amd import layer
    rng = np.random.default_rng(7 * n_embd + n_expert)
    w = (rng.standard_normal((n_expert, n_embd)) / np.sqrt(n_embd)).astype(np.float32)
    if wdtype == "f16":
        w = w.astype(np.float16)
    x = (3.0 * rng.standard_normal((n_rows, n_embd))).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(n_embd)).astype(np.float32)
    tw, tx, tnw = _t(w, gpu), _t(x, gpu), _t(nw, gpu)
    y, ids, wts = layer.moe_norm_gate(tx, tnw, 1e-5, tw, k)
    y2 = layer.rms_norm(tx, tnw, 1e-5)
    ids2, wts2 = layer.moe_gate(tw, y2, k)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))
    assert np.array_equal(ids.cpu().numpy(), ids2.cpu().numpy())
    assert np.array_equal(wts.cpu().numpy().view(np.uint32), wts2.cpu().numpy().view(np.uint32))
    np.testing.assert_allclose(y.cpu().numpy(), _rms_ref(x, nw, 1e-5), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("wdtype", ["f32", "f16"])
@pytest.mark.parametrize("n_rows,n_embd,n_expert,k", [(1, 4096, 8, 2), (3, 256, 8, 2), (2, 512, 64, 6), (1, 128, 3, 3)])
def test_moe_gate_equals_product_then_route(gpu, wdtype, n_rows, n_embd, n_expert, k):
    """The fused router product + routing gives the bits of sfa_mul_mat_vec then
    sfa_moe_route (the same dot arithmetic)."""
    from strataflow_amd import layer
    rng = np.random.default_rng(n_embd + n_expert)
    w = (rng.standard_normal((n_expert, n_embd)) / np.sqrt(n_embd)).astype(np.float32)
    if wdtype == "f16":
        w = w.astype(np.float16)
    x = rng.standard_normal((n_rows, n_embd)).astype(np.float32)
    tw, tx = _t(w, gpu), _t(x, gpu)
    ids, wts = layer.moe_gate(tw, tx, k)
    ids2, wts2 = layer.moe_route(layer.mul_mat_vec(tw, tx), k)
    assert np.array_equal(ids.cpu().numpy(), ids2.cpu().numpy())
    assert np.array_equal(wts.cpu().numpy().view(np.uint32), wts2.cpu().numpy().view(np.uint32))
    sel, _ = _route_ref(_mm_ref(w, x, wdtype == "f16").astype(np.float32), k)
    assert np.array_equal(ids.cpu().numpy(), sel)
