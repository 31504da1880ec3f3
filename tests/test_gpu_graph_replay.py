"""HIP-graph capture of the decode node and of a pager step (append + attend,
or the two in one call), replayed with changing inputs.

A captured decode is valid across steps only because every launch argument
stays fixed: q, seq_len, kv_lo and the page table are device buffers the
caller rewrites in place, and the split plan is computed on the device from
seq_len / kv_lo at every replay.  Each replay here is compared bit for bit with
an eager call on the same inputs and, for the single node, with the oracle.
Replays are interleaved with eager work and synchronisations (the graph holds
no memset node: the decode passes clear nothing)."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import Case, assert_close

pytestmark = pytest.mark.gpu

F32_MAX_ABS, F32_REL = 4e-5, 2e-5


@pytest.mark.parametrize("kv_type", [1, 8, 0])
def test_decode_graph_replay_rewritten_inputs(gpu, oracle_mod, kv_type):
    import torch
    lens = np.array([3000, 1100, 2000, 520], np.int32)
    c = Case(oracle_mod, seq_lens=lens, kv_type=kv_type, seed=81 + kv_type, extra_pages=5)
    B, M = c.B, int(lens.max())
    t_q = c.t_q.clone()
    t_sl = c.t_sl.clone()
    t_lo = torch.zeros(B, dtype=torch.int32, device=gpu)
    t_pt = c.t_pt.clone()
    out = torch.empty((B, c.n_head * c.head_dim), device=gpu)

    def call(o):
        c.dev.decode(0, t_q, t_pt, t_sl, M, kv_lo=t_lo, out=o)

    call(out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(out)
    torch.cuda.synchronize()

    rng = np.random.default_rng(90 + kv_type)
    steps = [
        (lens, [0, 0, 0, 0], None),                      # the captured inputs
        ([2999, 1, 2000, 0], [0, 0, 1500, 0], None),     # one empty, one single token, a window
        ([32, 1100, 17, 520], [0, 1099, 0, 500], 1),     # short spans; pages moved
        ([3000, 1000, 1999, 519], [2500, 0, 0, 3], 2),   # pages moved again
    ]
    pt_now = c.page_table.copy()
    for i, (sl, lo, perm_seed) in enumerate(steps):
        sl = np.asarray(sl, np.int32)
        lo = np.asarray(lo, np.int32)
        q = rng.standard_normal((B, c.n_head, c.head_dim)).astype(np.float32)
        t_q.copy_(torch.from_numpy(q))
        t_sl.copy_(torch.from_numpy(sl))
        t_lo.copy_(torch.from_numpy(lo))
        if perm_seed is not None:
            # move every physical page p to perm[p] and rewrite the table in place
            perm = np.random.default_rng(perm_seed).permutation(c.n_pages).astype(np.int32)
            idx = torch.from_numpy(perm).long().to(gpu)
            k2 = torch.empty_like(c.dev.k[0])
            v2 = torch.empty_like(c.dev.v[0])
            k2[idx] = c.dev.k[0]
            v2[idx] = c.dev.v[0]
            c.dev.k[0].copy_(k2)
            c.dev.v[0].copy_(v2)
            valid = pt_now >= 0
            pt_now[valid] = perm[pt_now[valid]]
            t_pt.copy_(torch.from_numpy(pt_now))
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        eager = torch.empty_like(out)
        call(eager)
        torch.cuda.synchronize()
        assert np.array_equal(got.view(np.uint32), eager.cpu().numpy().view(np.uint32)), f"replay {i}"
        # the logical cache is unchanged by the page moves: the original table
        # and host pools describe it
        ref = c.host.attention(q, c.n_head, c.page_table, sl, lo, mode=oracle_mod.GGML).reshape(B, -1)
        if kv_type == 0:
            assert_close(got, ref, max_abs=F32_MAX_ABS, rel_l2=F32_REL, what=f"replay {i} vs ggml")
        else:
            assert_close(got, ref, what=f"replay {i} vs ggml")
        assert np.all(got[sl <= lo] == 0)


def test_decode_32_layer_step_graph_replay(gpu, oracle_mod):
    # the timed step of the decode workload: 32 layers with distinct caches
    # captured once and replayed; every replay equals the eager step bitwise
    import torch
    from strataflow_amd import synth
    from strataflow_amd.paged_kv import PagedKV
    L, Hq, Hkv, hd, ps, n_kv = 32, 32, 8, 128, 256, 1300
    rng = np.random.default_rng(95)
    n_pages = (n_kv + ps - 1) // ps + 3
    kv = PagedKV(L, Hq, Hkv, hd, 1, ps, n_pages, device=gpu)
    pt = torch.from_numpy(synth.page_tables(rng, [n_kv], ps, n_pages)).to(gpu)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(95)
    pos = torch.arange(n_kv, dtype=torch.int32, device=gpu)
    seq = torch.zeros(n_kv, dtype=torch.int32, device=gpu)
    for layer in range(L):
        kv.append(layer, torch.randn((n_kv, Hkv, hd), device=gpu, generator=gen),
                  torch.randn((n_kv, Hkv, hd), device=gpu, generator=gen), seq, pos, pt)
    q = torch.randn((L, 1, Hq, hd), device=gpu, generator=gen)
    sl = torch.tensor([n_kv], dtype=torch.int32, device=gpu)
    out = torch.empty((L, 1, Hq * hd), device=gpu)

    def step(o):
        for layer in range(L):
            kv.decode(layer, q[layer], pt, sl, n_kv, out=o[layer])

    step(out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(out)
    for n in (n_kv, 700, 1, n_kv - 33):
        sl.fill_(n)
        q.copy_(torch.randn(q.shape, device=gpu, generator=gen))
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        eager = torch.empty_like(out)
        step(eager)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), eager.view(torch.int32)), f"seq_len {n}"


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("attend", [0, 1])
def test_pager_step_graph_replay(gpu, attend, fused):
    # two pagers fed the same stream: one runs every step eagerly, the other
    # replays one captured step (append + attend of every layer, or the fused
    # append_attend) over fixed input buffers after its host-side begin();
    # pages are evicted (lossless) or released (window) during the replayed
    # steps
    import torch
    from strataflow_amd import synth
    from strataflow_amd.pager import KvPager
    L, Hq, Hkv, hd, ps, B, W, fill = 2, 32, 8, 128, 64, 2, 256, 512
    mk = lambda: KvPager(n_layer=L, n_head=Hq, n_head_kv=Hkv, head_dim=hd, kv_type=1, page_size=ps,
                         n_seq=B, n_ctx=2048, window=W, attend=attend, seed=7)
    eager_p, graph_p = mk(), mk()
    gen = torch.Generator(device=gpu)
    gen.manual_seed(96)
    for c0 in range(0, fill, ps):
        n_tok = np.full(B, ps, np.int32)
        pos = (c0 + torch.arange(ps, device=gpu, dtype=torch.int32)).repeat(B)
        for p in (eager_p, graph_p):
            assert p.begin(n_tok) == 0
        for layer in range(L):
            k = synth.rope_normal_torch(torch.randn((B * ps, Hkv, hd), device=gpu, generator=gen), pos, 1e6)
            k = k.contiguous()
            v = torch.randn((B * ps, Hkv, hd), device=gpu, generator=gen)
            for p in (eager_p, graph_p):
                p.append(layer, k, v)
    ones = np.ones(B, np.int32)
    qb = torch.empty((L, B, Hq, hd), device=gpu)
    kb = torch.empty((L, B, Hkv, hd), device=gpu)
    vb = torch.empty((L, B, Hkv, hd), device=gpu)
    out_g = torch.empty((L, B, Hq * hd), device=gpu)

    def layers(p, q, k, v, out):
        for layer in range(L):
            p.append(layer, k[layer], v[layer])
            p.attend(layer, q[layer], out[layer])

    def layers_g(p, q, k, v, out):
        if not fused:
            layers(p, q, k, v, out)
            return
        for layer in range(L):
            p.append_attend(layer, k[layer], v[layer], q[layer], out[layer])

    def inputs():
        return (torch.randn(qb.shape, device=gpu, generator=gen),
                torch.randn(kb.shape, device=gpu, generator=gen),
                torch.randn(vb.shape, device=gpu, generator=gen))

    st0 = graph_p.stats()
    n_steps = 150  # crosses two page boundaries of every sequence
    for s in range(n_steps):
        q, k, v = inputs()
        out_e = torch.empty_like(out_g)
        assert eager_p.begin(ones) == 0
        layers(eager_p, q, k, v, out_e)
        assert graph_p.begin(ones) == 0
        qb.copy_(q)
        kb.copy_(k)
        vb.copy_(v)
        if s == 0:
            layers_g(graph_p, qb, kb, vb, out_g)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                layers_g(graph_p, qb, kb, vb, out_g)
        else:
            out_g.fill_(float("nan"))
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g.view(torch.int32), out_e.view(torch.int32)), f"step {s}"
    st = graph_p.stats()
    assert st == eager_p.stats()
    key = "pages_evicted" if attend == 0 else "pages_dropped"
    assert st[key] - st0[key] >= 2 * B  # pages left the window during the replayed steps
    eager_p.close()
    graph_p.close()


def test_decode_layer_graph_replay(gpu):
    """A whole decode layer (two layers, small shape, f16 weights and cache)
    through the fused launches: attn_norm, Q/K/V + RoPE + append, decode, wo +
    residual, ffn_norm + gate, experts.  Captured once, replayed for several
    tokens with the position rewritten in place, interleaved with the same
    step run eagerly on a twin cache: the layer output and both pools equal
    the eager ones bit for bit at every step."""
    import torch
    from strataflow_amd import layer as ops
    from strataflow_amd import synth
    from strataflow_amd.paged_kv import PagedKV
    L, D, Hq, Hkv, hd, E, K, F, ps = 2, 512, 8, 4, 64, 4, 2, 1024, 64
    n_ctx = 4 * ps
    rng = np.random.default_rng(33)
    n_pages = n_ctx // ps + 2
    gen = torch.Generator(device=gpu)
    gen.manual_seed(33)

    def w(*shape):
        return (torch.randn(shape, device=gpu, generator=gen) * 0.05).half().contiguous()

    layers = [dict(attn_norm=1 + 0.1 * torch.randn(D, device=gpu, generator=gen),
                   ffn_norm=1 + 0.1 * torch.randn(D, device=gpu, generator=gen),
                   wqkv=w((Hq + 2 * Hkv) * hd, D), wo=w(D, Hq * hd), gate_inp=w(E, D),
                   gate=w(E, F, D), up=w(E, F, D), down=w(E, D, F)) for _ in range(L)]
    pt = torch.from_numpy(synth.page_tables(rng, [n_ctx], ps, n_pages)).to(gpu)
    caches = [PagedKV(L, Hq, Hkv, hd, 1, ps, n_pages, device=gpu) for _ in range(2)]
    # a shared history of 100 positions in both caches
    hist = 100
    hpos = torch.arange(hist, dtype=torch.int32, device=gpu)
    hseq = torch.zeros(hist, dtype=torch.int32, device=gpu)
    for il in range(L):
        k = torch.randn((hist, Hkv, hd), device=gpu, generator=gen)
        v = torch.randn((hist, Hkv, hd), device=gpu, generator=gen)
        for kv in caches:
            kv.append(il, k, v, hseq, hpos, pt)
    x0 = torch.empty((1, D), device=gpu)
    pos = torch.zeros(1, dtype=torch.int32, device=gpu)
    seq = torch.zeros(1, dtype=torch.int32, device=gpu)
    sl = torch.zeros(1, dtype=torch.int32, device=gpu)

    def buffers():
        return dict(x=torch.empty((1, D), device=gpu), cur=torch.empty((1, D), device=gpu),
                    ffn=torch.empty((1, D), device=gpu), q=torch.empty((1, Hq, hd), device=gpu),
                    attn=torch.empty((1, Hq * hd), device=gpu),
                    ids=torch.empty((1, K), dtype=torch.int32, device=gpu), wts=torch.empty((1, K), device=gpu),
                    ws=torch.empty(K * F * 4, dtype=torch.uint8, device=gpu))

    def step(kv, b):
        b["x"].copy_(x0)
        for il, Ly in enumerate(layers):
            ops.rms_norm(b["x"], Ly["attn_norm"], 1e-5, out=b["cur"])
            kv.qkv_rope_append(il, Ly["wqkv"], b["cur"], seq, pos, pt, 1e4, q=b["q"])
            kv.decode(il, b["q"], pt, sl, n_ctx, out=b["attn"])
            ops.mul_mat_vec(Ly["wo"], b["attn"], residual=b["x"], out=b["ffn"])
            ops.moe_norm_gate(b["ffn"], Ly["ffn_norm"], 1e-5, Ly["gate_inp"], K, out=b["cur"], ids=b["ids"],
                              weights=b["wts"])
            ops.moe_ffn(b["cur"], b["ffn"], b["ids"], b["wts"], Ly["gate"], Ly["up"], Ly["down"], out=b["x"],
                        workspace=b["ws"])

    bg, be = buffers(), buffers()
    x0.copy_(torch.randn((1, D), device=gpu, generator=gen))
    pos.fill_(hist)
    sl.fill_(hist + 1)
    step(caches[0], bg)  # warm-up (also the first token, in both caches)
    step(caches[1], be)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(caches[0], bg)
    torch.cuda.synchronize()
    # the capture recorded without running: the next replay writes position hist + 1
    for p in range(hist + 1, hist + 6):
        x0.copy_(torch.randn((1, D), device=gpu, generator=gen))
        pos.fill_(p)
        sl.fill_(p + 1)
        bg["x"].fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        step(caches[1], be)
        torch.cuda.synchronize()
        assert torch.equal(bg["x"].view(torch.int32), be["x"].view(torch.int32)), f"position {p}"
        assert torch.isfinite(bg["x"]).all()
        assert torch.equal(caches[0].k, caches[1].k) and torch.equal(caches[0].v, caches[1].v), f"position {p}"
