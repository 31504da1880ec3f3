#!/usr/bin/env python3
"""Benchmark of the paged-KV attention path on one MI355X.

Headline workload (one "step" = one decode token through all 32 layers of
attention): Mixtral-8x7B attention shape (32 query heads, 8 kv heads,
head_dim 128), batch 1, context 4096, f16 KV in 256-token pages placed by a
seeded permutation, a distinct KV cache per layer (537 MB in all, larger than
the 256 MB Infinity Cache).  Inputs are resident in HBM before timing.

Also reported: chunked causal prefill (2048-token chunk on 2048 cached
positions, same shape), its MFMA rate, and the CPU oracle (ggml semantics) on
the host cores as a baseline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode-attn µs/layer-token + HBM GB/s % peak; prefill MFMA util (Mixtral GQA)"
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2516.6  # MI355X dense f16/bf16
MFMA_F32_PEAK_TFLOPS = 157.3   # MI355X dense f32 matrix

N_LAYER, HQ, HKV, HD, PAGE = 32, 32, 8, 128, 256


def build_decode_workload(torch, ctx, seed: int, kv_type: int = 1):
    """N_LAYER distinct paged caches holding sequences of lengths `ctx` (an int
    or a list, one entry per sequence), pages of all sequences drawn from one
    shuffled pool per layer; K/V ~ N(0,1) with RoPE theta 1e6 on K, written
    through sfa_kv_append (f16 rounding or Q8_0 quantisation on write)."""
    from strataflow_amd import synth
    from strataflow_amd.paged_kv import PagedKV
    dev = torch.device("cuda:0")
    lens = [ctx] if isinstance(ctx, int) else [int(x) for x in ctx]
    B = len(lens)
    need = sum((n + PAGE - 1) // PAGE for n in lens)
    pool_pages = need + 4
    kv = PagedKV(N_LAYER, HQ, HKV, HD, kv_type, PAGE, pool_pages, device=dev)
    rng = np.random.default_rng(seed)
    pt = synth.page_tables(rng, lens, PAGE, pool_pages)
    t_pt = torch.from_numpy(pt).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    for layer in range(N_LAYER):
        for b, n in enumerate(lens):
            pos = torch.arange(n, device=dev, dtype=torch.int32)
            seq = torch.full((n,), b, device=dev, dtype=torch.int32)
            k = torch.randn((n, HKV, HD), device=dev, generator=gen)
            v = torch.randn((n, HKV, HD), device=dev, generator=gen)
            k = synth.rope_normal_torch(k, pos, 1e6).contiguous()
            kv.append(layer, k, v, seq, pos, t_pt)
            del k, v
    q = torch.randn((N_LAYER, B, HQ, HD), device=dev, generator=gen)
    qpos = torch.tensor([n - 1 for n in lens], device=dev, dtype=torch.int32)
    q = torch.stack([synth.rope_normal_torch(q[i], qpos, 1e6) for i in range(N_LAYER)]).contiguous()
    seq_len = torch.tensor(lens, device=dev, dtype=torch.int32)
    torch.cuda.synchronize()
    return kv, pt, t_pt, q, seq_len


def gpu_backlog(torch, ms: float) -> None:
    """Queues a bounded spin kernel of about `ms` so that the launches queued
    behind it run back to back (host launch cost is then off the GPU clock)."""
    torch.cuda._sleep(int(ms * 1e-3 * gpu_backlog.cycles_per_s))


gpu_backlog.cycles_per_s = 1e8


def calibrate_backlog(torch) -> None:
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    torch.cuda._sleep(1_000_000)
    b.record()
    torch.cuda.synchronize()
    gpu_backlog.cycles_per_s = 1_000_000 / max(a.elapsed_time(b) * 1e-3, 1e-6)


def _lib_mod():
    from strataflow_amd import _lib
    return _lib


def time_decode(torch, kv, t_pt, q, seq_len, ctx, steps, warmup):
    """Step timing: the 32-layer loop captured once as a HIP graph and
    replayed `steps` times between two events.  Kernel timing: the split-K
    passes of the 32 layers back to back between two events."""
    B = int(seq_len.numel())
    out = torch.empty((N_LAYER, B, HQ * HD), device=q.device)
    kv.workspace(B, ctx)

    def step():
        for layer in range(N_LAYER):
            kv.decode(layer, q[layer], t_pt, seq_len, ctx, out=out[layer])

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / steps
    # eager loop for comparison (host launch cost included)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    ms_eager = t0.elapsed_time(t1) / steps

    # split-K kernel time: the split passes of all layers back to back between
    # two events (queued behind a backlog, so host launch cost is hidden),
    # divided by the launch count; repeated `steps` times
    calibrate_backlog(torch)
    lib = _lib_mod().load()
    ws = kv.workspace(B, ctx)
    stream = torch.cuda.current_stream().cuda_stream
    args = [(ctypes.byref(kv.desc(layer)), q[layer].data_ptr(), out[layer].data_ptr(), t_pt.data_ptr(),
             int(t_pt.shape[1]), seq_len.data_ptr(), None, B, int(ctx), float(kv.scale), ws.data_ptr(),
             ws.numel(), stream) for layer in range(N_LAYER)]
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    torch.cuda.synchronize()
    gpu_backlog(torch, 0.05 * N_LAYER * steps + 5)
    for a, b in evs:
        a.record()
        for layer in range(N_LAYER):
            lib.sfa_attn_decode_split(*args[layer])
        b.record()
    torch.cuda.synchronize()
    durs = np.array([a.elapsed_time(b) for a, b in evs]) * 1e3 / N_LAYER  # us per launch
    for layer in range(N_LAYER):  # leave complete outputs behind
        kv.decode(layer, q[layer], t_pt, seq_len, ctx, out=out[layer])
    torch.cuda.synchronize()
    return ms_per_step, ms_eager, float(np.mean(durs)), float(np.median(durs)), out


def load_traffic() -> dict:
    """HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE (scaled by a plain copy's readings), recorded per workload in
    profiles/traffic.json by the profiling runs quoted in profiles/*.txt."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def with_traffic(roofline: dict, key: str) -> dict:
    t = load_traffic().get(key)
    if t:
        roofline["traffic"] = t["bytes_per_launch"]
        roofline["traffic_source"] = f"profiles/traffic.json[{key}] (rocprofv3 FETCH_SIZE+WRITE_SIZE)"
    return roofline


KV_NAMES = {0: "f32", 1: "f16", 8: "Q8_0"}


def decode_leg(torch, key, lens, kv_type, steps, warmup, seed):
    """One decode workload: lens (one entry per sequence), f32, f16 or Q8_0."""
    kv, pt, t_pt, q, seq_len = build_decode_workload(torch, lens, seed, kv_type=kv_type)
    mx = int(max(lens))
    ms, _, k_mean, _, _ = time_decode(torch, kv, t_pt, q, seq_len, mx, steps, warmup)
    row = {0: HD * 4, 1: HD * 2, 8: HD // 32 * 34}[kv_type]
    alg = 2 * sum(lens) * HKV * row + len(lens) * HQ * HD * 4 * 2
    us_layer = ms * 1e3 / N_LAYER
    ach = alg / (k_mean * 1e-6) / 1e9
    # Q8_0 batches of two or more with >= 1024 tiles in all run the column layout
    cols = kv_type == 8 and len(lens) >= 2 and len(lens) * ((mx + 31) // 32) >= 1024
    kname = {0: "decode_f32_kernel<128,4>", 1: "decode_f16_kernel<128,4>",
             8: f"decode_q8_kernel<128,4,{'true' if cols else 'false'}>"}[kv_type]
    res = {
        "workload": f"decode-attn {KV_NAMES[kv_type]} KV, Mixtral GQA 32q/8kv hd128, "
                    f"B={len(lens)}, context {lens if len(lens) > 1 else lens[0]}, 256-token pages "
                    f"shuffled, {N_LAYER} layers with distinct caches",
        "us_per_layer_step": round(us_layer, 3),
        "us_per_layer_token": round(us_layer / len(lens), 3),
        "tokens_per_s": round(len(lens) * 1e3 / ms, 1),
        "roofline": with_traffic({
            "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": f"{kname} (split-K pass)", "kernel_us_mean": round(k_mean, 3),
            "bytes_per_launch": alg}, key),
    }
    del kv, q
    torch.cuda.empty_cache()
    return res


def q8_bench(torch, steps, warmup, seed):
    """Q8_0 KV decode: (a) batch 1 at context 32768; (b) batch 8 with lengths
    uniform in [8192, 32768] sharing one page pool; and the 2048-on-2048 chunked
    prefill over a Q8_0 cache."""
    lens_b8 = [int(x) for x in np.random.default_rng(seed).integers(8192, 32769, 8)]
    return {
        "ctx32k_b1": decode_leg(torch, "decode_q8_0_ctx32k_b1", [32768], 8, steps, warmup, seed),
        "b8_varlen_8k_32k": decode_leg(torch, "decode_q8_0_b8", lens_b8, 8, steps, warmup, seed),
        "prefill_2048_on_2048": prefill_bench(torch, max(steps // 3, 3), 2, seed + 1, kv_type=8),
    }


def copy_ceiling(torch) -> dict:
    """A plain 2 GiB device-to-device copy (read + write): the practical HBM
    rate on this part, next to the nominal peak."""
    n = 2 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(5):
        b.copy_(a)
    t1.record()
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / 5
    del a, b
    torch.cuda.empty_cache()
    return {"bytes": 2 * n, "us": round(us, 1), "gbs": round(2 * n / us / 1e3, 1),
            "what": "2 GiB device copy (read + write bytes), torch"}


def prefill_bench(torch, steps: int, warmup: int, seed: int, kv_type: int = 1):
    """Chunked causal prefill: 2048 tokens at positions 2048..4095 over a
    4096-position paged f16 (or f32) cache, 8 layers with distinct caches."""
    from strataflow_amd import synth
    from strataflow_amd.paged_kv import PagedKV
    dev = torch.device("cuda:0")
    n_cached, T = 2048, 2048
    n_kv = n_cached + T
    n_layer = 8  # distinct caches per step (8 x 16.8 MB at f16)
    pool_pages = n_kv // PAGE + 4
    kv = PagedKV(n_layer, HQ, HKV, HD, kv_type, PAGE, pool_pages, device=dev)
    rng = np.random.default_rng(seed)
    pt = torch.from_numpy(synth.page_tables(rng, [n_kv], PAGE, pool_pages)[0]).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    pos = torch.arange(n_kv, device=dev, dtype=torch.int32)
    seq = torch.zeros(n_kv, device=dev, dtype=torch.int32)
    qs = []
    for layer in range(n_layer):
        k = synth.rope_normal_torch(torch.randn((n_kv, HKV, HD), device=dev, generator=gen), pos, 1e6)
        v = torch.randn((n_kv, HKV, HD), device=dev, generator=gen)
        kv.append(layer, k.bfloat16().float().contiguous(), v.bfloat16().float().contiguous(), seq, pos,
                  pt[None])
        q = synth.rope_normal_torch(torch.randn((T, HQ, HD), device=dev, generator=gen), pos[n_cached:], 1e6)
        qs.append(q.bfloat16().float().contiguous())
    out = torch.empty((T, HQ * HD), device=dev)

    def step():
        for layer in range(n_layer):
            kv.prefill(layer, qs[layer], pt, n_cached, out=out)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n_layer * steps)]
    i = 0
    for _ in range(steps):
        for layer in range(n_layer):
            evs[i][0].record()
            kv.prefill(layer, qs[layer], pt, n_cached, out=out)
            evs[i][1].record()
            i += 1
    torch.cuda.synchronize()
    us = float(np.mean([a.elapsed_time(b) for a, b in evs]) * 1e3)
    pairs = sum(n_cached + i + 1 for i in range(T))          # causal (q, k) pairs per head
    flops = 4.0 * HD * pairs * HQ                            # QK^T + PV
    tflops = flops / (us * 1e-6) / 1e12
    # f32: the f32 MFMA peak; Q8_0 (int8 QK, f16 PV): the f16 peak, the slower of its two
    peak = MFMA_F32_PEAK_TFLOPS if kv_type == 0 else MFMA_F16_PEAK_TFLOPS
    name = KV_NAMES[kv_type]
    return {
        "workload": f"causal prefill {name} KV, 2048-token chunk on 2048 cached, Mixtral GQA 32q/8kv hd128",
        "us_per_layer_chunk": round(us, 2),
        "us_per_layer_token": round(us / T, 5),
        "tflops": round(tflops, 1),
        "roofline": with_traffic({"bound": "mfma", "achieved": round(tflops, 1),
                                  "peak": peak, "unit": "TFLOP/s",
                                  "frac": round(tflops / peak, 4), "traffic": None,
                                  "kernel": {0: "prefill_f32_kernel<128,4>", 1: "prefill_f16_kernel<128,4>",
                                             8: "prefill_q8_kernel<128,4>"}[kv_type]},
                                 {1: "prefill_2048_on_2048", 0: "prefill_f32_2048_on_2048",
                                  8: "prefill_q8_0_2048_on_2048"}[kv_type]),
        "flop_per_layer_chunk": flops,
    }


def f32_bench(torch, steps: int, warmup: int, seed: int):
    """F32 KV, the reference's own cache type: decode at context 4096 (B=1,
    32 layers) and the 2048-on-2048 chunked prefill, both on f32 MFMA."""
    return {
        "decode_ctx4096": decode_leg(torch, "decode_f32_ctx4096", [4096], 0, steps, warmup, seed),
        "prefill_2048_on_2048": prefill_bench(torch, max(steps // 10, 3), 2, seed + 1, kv_type=0),
    }


def window_bench(torch, seed: int, steps: int = 128, lossless_steps: int = 4):
    """KV-window decode under paging pressure: 4 sequences with 65536-token
    histories, a 4096-position window, the device pool sized to the window
    (4 x 17 pages per layer), pages evicted and reused by the host page
    manager every 256 steps of a sequence.  (a) the opt-in sliding window over
    all 32 layers for `steps` decode steps; (b) the reference's lossless
    semantics (every position attended, the 61440 evicted positions read from
    the host-pinned cold pool in place) on one layer."""
    from strataflow_amd import synth
    from strataflow_amd.pager import SFA_ATTEND_LOSSLESS, SFA_ATTEND_WINDOW, SFA_KV_F16, KvPager
    dev = torch.device("cuda:0")
    B, hist, W = 4, 65536, 4096
    res = {}
    for name, attend, n_layer, n_steps in (("sliding_window", SFA_ATTEND_WINDOW, N_LAYER, steps),
                                           ("lossless", SFA_ATTEND_LOSSLESS, 1, lossless_steps)):
        pager = KvPager(n_layer=n_layer, n_head=HQ, n_head_kv=HKV, head_dim=HD, kv_type=SFA_KV_F16,
                        page_size=PAGE, n_seq=B, n_ctx=hist + n_steps, window=W, attend=attend,
                        seed=seed)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        for c0 in range(0, hist, PAGE):
            assert pager.begin(np.full(B, PAGE, np.int32)) == 0
            pos = (c0 + torch.arange(PAGE, device=dev, dtype=torch.int32)).repeat(B)
            for layer in range(n_layer):
                k = synth.rope_normal_torch(torch.randn((B * PAGE, HKV, HD), device=dev, generator=gen),
                                            pos, 1e6).contiguous()
                v = torch.randn((B * PAGE, HKV, HD), device=dev, generator=gen)
                pager.append(layer, k, v)
        pos = torch.arange(hist, hist + n_steps, device=dev, dtype=torch.int32)
        qs = synth.rope_normal_torch(
            torch.randn((n_steps * n_layer * B, HQ, HD), device=dev, generator=gen),
            pos.repeat_interleave(n_layer * B), 1e6).view(n_steps, n_layer, B, HQ, HD).contiguous()
        ks = synth.rope_normal_torch(
            torch.randn((n_steps * n_layer * B, HKV, HD), device=dev, generator=gen),
            pos.repeat_interleave(n_layer * B), 1e6).view(n_steps, n_layer, B, HKV, HD).contiguous()
        vs = torch.randn((n_steps, n_layer, B, HKV, HD), device=dev, generator=gen)
        out = torch.empty((n_layer, B, HQ * HD), device=dev)
        ones = np.ones(B, np.int32)
        # a decode step's per-layer calls take the same arguments every step
        # (the pager's device tables change, not their addresses), so the
        # layer loop is one HIP graph over fixed input buffers; each step is
        # the pager's host planning + table-update kernel, the copy of that
        # step's Q/K/V into the buffers, and a replay
        qb, kb, vb = qs[0].clone(), ks[0].clone(), vs[0].clone()

        def layers():
            for layer in range(n_layer):
                pager.append(layer, kb[layer], vb[layer])
                pager.attend(layer, qb[layer], out[layer])

        assert pager.begin(ones) == 0  # one warm step (not timed) opens a step
        layers()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            layers()
        # the capture recorded but did not run the warm step's calls again;
        # the pager is one position ahead of the histories from here on
        torch.cuda.synchronize()
        calibrate_backlog(torch)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        gpu_backlog(torch, 20)
        t0.record()
        for s in range(n_steps - 1):
            assert pager.begin(ones) == 0
            qb.copy_(qs[s + 1])
            kb.copy_(ks[s + 1])
            vb.copy_(vs[s + 1])
            graph.replay()
        t1.record()
        torch.cuda.synchronize()
        n_steps -= 1
        us = t0.elapsed_time(t1) * 1e3 / (n_steps * n_layer)
        st = pager.stats()
        hbm = B * W * HKV * HD * 2 * 2
        entry = {
            "workload": f"decode-attn f16 KV, Mixtral GQA 32q/8kv hd128, B={B}, history {hist}, "
                        f"window {W}, device pool {B * (W // PAGE + 1)} pages/layer, "
                        f"{n_steps} consecutive steps, {n_layer} layer(s)",
            "semantics": ("sliding window: attends the last 4096 positions (opt-in kv_lo)"
                          if attend == SFA_ATTEND_WINDOW else
                          "lossless (reference): attends every position; evicted pages read "
                          "from the host-pinned cold pool"),
            "us_per_layer_step": round(us, 3),
            "us_per_layer_token": round(us / B, 3),
            "includes": "paging (plan + table update), KV append, split-K decode and merge",
            "pages_evicted": st["pages_evicted"], "pages_dropped": st["pages_dropped"],
            "hbm_bytes_per_layer_step": hbm,
            "hbm_gbs": round(hbm / (us * 1e-6) / 1e9, 1),
        }
        if attend == SFA_ATTEND_LOSSLESS:
            cold = sum(hist + s - W for s in range(n_steps)) // n_steps * B * HKV * HD * 2 * 2
            entry["host_link_bytes_per_layer_step"] = cold
            entry["host_link_gbs"] = round(cold / (us * 1e-6) / 1e9, 1)
        res[name] = entry
        pager.close()
        del qs, ks, vs
        torch.cuda.empty_cache()
    return res


def rope_bench(torch, steps: int, seed: int):
    """Fused RoPE + KV append (sfa_rope_kv_append): a decode step (B=1, one
    token per layer, 32 layers in a HIP graph) and a 2048-token prefill chunk
    at positions 2048..4095 (8 layers with distinct caches), f16 cache,
    RoPE base 1e6."""
    from strataflow_amd import synth
    from strataflow_amd.paged_kv import PagedKV, SFA_KV_F16
    dev = torch.device("cuda:0")
    res = {}
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)

    # decode step: one token at position 4095 per layer
    n_kv = 4096
    pool = n_kv // PAGE + 1
    kv = PagedKV(N_LAYER, HQ, HKV, HD, SFA_KV_F16, PAGE, pool, device=dev)
    pt = torch.from_numpy(synth.page_tables(rng, [n_kv], PAGE, pool)).to(dev)
    seq = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.full((1,), n_kv - 1, dtype=torch.int32, device=dev)
    qs = torch.randn((N_LAYER, 1, HQ, HD), device=dev, generator=gen)
    ks = torch.randn((N_LAYER, 1, HKV, HD), device=dev, generator=gen)
    vs = torch.randn((N_LAYER, 1, HKV, HD), device=dev, generator=gen)

    def step():
        for layer in range(N_LAYER):
            kv.rope_append(layer, qs[layer], ks[layer], vs[layer], seq, pos, pt, 1e6)

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / steps / N_LAYER
    res["decode_b1"] = {
        "workload": "fused RoPE (base 1e6) of Q [1,32,128] and K [1,8,128] + append of K, V into an "
                    "f16 paged cache at position 4095, 32 layers in a HIP graph",
        "us_per_layer_token": round(us, 3),
    }
    del kv, qs, ks, vs, g
    torch.cuda.empty_cache()

    # prefill chunk: 2048 tokens at positions 2048..4095
    T, n_layer = 2048, 8
    kv = PagedKV(n_layer, HQ, HKV, HD, SFA_KV_F16, PAGE, pool, device=dev)
    pos = torch.arange(n_kv - T, n_kv, dtype=torch.int32, device=dev)
    seq = torch.zeros(T, dtype=torch.int32, device=dev)
    qs = torch.randn((n_layer, T, HQ, HD), device=dev, generator=gen)
    ks = torch.randn((n_layer, T, HKV, HD), device=dev, generator=gen)
    vs = torch.randn((n_layer, T, HKV, HD), device=dev, generator=gen)
    for layer in range(n_layer):
        kv.rope_append(layer, qs[layer], ks[layer], vs[layer], seq, pos, pt, 1e6)
    torch.cuda.synchronize()
    a.record()
    for _ in range(steps):
        for layer in range(n_layer):
            kv.rope_append(layer, qs[layer], ks[layer], vs[layer], seq, pos, pt, 1e6)
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / steps / n_layer
    # Q read + written, K and V read, K and V f16 rows written, each once
    alg = 2 * T * HQ * HD * 4 + 2 * T * HKV * HD * 4 + 2 * T * HKV * HD * 2
    gbs = alg / (us * 1e-6) / 1e9
    res["prefill_2048"] = {
        "workload": "fused RoPE (base 1e6) of Q [2048,32,128] and K [2048,8,128] + append of K, V "
                    "into an f16 paged cache at positions 2048..4095, 8 layers with distinct caches",
        "us_per_layer_chunk": round(us, 3),
        "roofline": with_traffic({"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                                  "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                                  "kernel": "rope_append_kernel<f16>", "bytes_per_launch": alg},
                                 "rope_append_2048"),
    }
    del kv, qs, ks, vs
    torch.cuda.empty_cache()
    return res


def cpu_baseline(kv, pt, q_layer0, ctx, budget_s=12.0):
    """The oracle (ggml semantics, the reference's op sequence with its three
    history copies) on the host cores, layer 0 of the same workload."""
    import torch
    from oracle import oracle
    host = oracle.HostPagedKv(HKV, HD, PAGE, oracle.KV_F16, kv.n_pages)
    host.k[:] = kv.k[0].cpu().numpy()
    host.v[:] = kv.v[0].cpu().numpy()
    q = q_layer0.cpu().numpy().reshape(1, HQ, HD)
    sl = np.array([ctx], np.int32)
    threads = min(os.cpu_count() or 1, 16)
    res = {}
    for nt in (threads, 1):
        host.attention(q, HQ, pt, sl, n_threads=nt)  # warm
        ts = []
        t_start = time.perf_counter()
        while time.perf_counter() - t_start < budget_s / 2 and len(ts) < 200:
            t0 = time.perf_counter()
            out = host.attention(q, HQ, pt, sl, n_threads=nt)
            ts.append(time.perf_counter() - t0)
        res[nt] = (float(np.median(ts)) * 1e6, len(ts), out)
    return threads, res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-q8", action="store_true", help="skip the Q8_0 decode legs")
    ap.add_argument("--no-window", action="store_true", help="skip the KV-window paging legs")
    ap.add_argument("--no-32k", action="store_true", help="skip the f16 context-32768 decode leg")
    ap.add_argument("--no-rope", action="store_true", help="skip the fused RoPE + append leg")
    ap.add_argument("--no-f32", action="store_true", help="skip the F32-cache legs")
    ap.add_argument("--only", choices=["decode4k", "decode32k", "q8", "prefill", "window", "rope", "f32"],
                    help="run one leg only and print its JSON (profiling runs)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MB",
                    help="only run a plain device copy of MB megabytes (HBM counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: there is no multi-GPU path "
              "(decode would shard by kv head, with no exchange between GPUs)", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from strataflow_amd import _lib
    _lib.load()

    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20)
        a = torch.empty(n, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n, "reps": 5}))
        return

    if args.only == "decode4k":
        args.no_prefill = args.no_q8 = args.no_window = args.no_32k = args.no_cpu = args.no_rope = True
        args.no_f32 = True
    if args.only and args.only != "decode4k":
        if args.only == "decode32k":
            r = decode_leg(torch, "decode_f16_ctx32k", [32768], 1, max(args.steps // 4, 5), 3, args.seed + 4)
        elif args.only == "q8":
            r = q8_bench(torch, max(args.steps // 4, 5), 3, args.seed + 2)
        elif args.only == "prefill":
            r = prefill_bench(torch, max(args.steps // 10, 3), 2, args.seed + 1)
        elif args.only == "rope":
            r = rope_bench(torch, max(args.steps // 5, 5), args.seed + 5)
        elif args.only == "f32":
            r = f32_bench(torch, max(args.steps // 4, 5), 3, args.seed + 6)
        else:
            r = window_bench(torch, args.seed + 3)
        print(json.dumps({args.only: r}))
        return

    ctx = args.ctx
    kv, pt, t_pt, q, seq_len = build_decode_workload(torch, ctx, args.seed)
    ms_step, ms_eager, k_mean, k_med, out = time_decode(torch, kv, t_pt, q, seq_len, ctx, args.steps,
                                                        args.warmup)
    us_layer = ms_step * 1e3 / N_LAYER
    kv_bytes = 2 * ctx * HKV * HD * 2
    alg_bytes = kv_bytes + HQ * HD * 4 * 2  # K + V + Q + O, each once
    achieved = alg_bytes / (k_mean * 1e-6) / 1e9

    result = {
        "metric": METRIC,
        "value": round(us_layer, 3),
        "unit": "us/layer-token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": f"decode-attn f16 KV, Mixtral GQA 32q/8kv hd128, B=1, ctx {ctx}, "
                        f"256-token pages shuffled, {N_LAYER} layers with distinct caches",
            "batch": 1, "context": ctx, "n_layer": N_LAYER, "page_size": PAGE,
        },
        "tokens_per_s": round(1e3 / ms_step, 1),
        "timing": "32-layer step captured as a HIP graph, replayed; eager (per-call host "
                  "launch) step also reported",
        "ms_per_step_eager": round(ms_eager, 4),
        "roofline": with_traffic({
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "decode_f16_kernel<128,4> (split-K pass)", "kernel_us_mean": round(k_mean, 3),
            "kernel_us_median": round(k_med, 3), "bytes_per_launch": alg_bytes,
        }, "decode_f16_ctx4096"),
    }
    if not args.no_32k:
        result["f16_ctx32k"] = decode_leg(torch, "decode_f16_ctx32k", [32768], 1,
                                          max(args.steps // 4, 5), 3, args.seed + 4)
    if not args.no_prefill:
        result["prefill"] = prefill_bench(torch, max(args.steps // 10, 3), 2, args.seed + 1)
    if not args.no_q8:
        result["q8_0"] = q8_bench(torch, max(args.steps // 4, 5), 3, args.seed + 2)
    if not args.no_window:
        result["window"] = window_bench(torch, args.seed + 3)
    if not args.no_rope:
        result["rope_append"] = rope_bench(torch, max(args.steps // 5, 5), args.seed + 5)
    if not args.no_f32:
        result["f32"] = f32_bench(torch, max(args.steps // 4, 5), 3, args.seed + 6)
    result["hbm_copy_ceiling"] = copy_ceiling(torch)
    if not args.no_cpu:
        threads, res = cpu_baseline(kv, pt, q[0], ctx)
        us_all, n_all, cpu_out = res[threads]
        us_one, n_one, _ = res[1]
        gpu0 = out[0].cpu().numpy().reshape(-1).astype(np.float64)
        ref = cpu_out.reshape(-1).astype(np.float64)
        ma = float(np.max(np.abs(gpu0 - ref)))
        rl = float(np.linalg.norm(gpu0 - ref) / np.linalg.norm(ref))
        result["cpu_baseline"] = {
            "value": round(us_all, 1), "unit": "us/layer-token", "cores": threads, "kind": "port",
            "sample": f"layer 0 of the same workload (ctx {ctx}), ggml-semantics oracle, "
                      f"median of {n_all} calls",
            "value_1_thread": round(us_one, 1),
            "parity_vs_gpu": {"max_abs": ma, "rel_l2": rl},
        }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
