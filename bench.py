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


def time_split_launches(torch, lib, args, reps: int):
    """Mean and median duration (us) of one split-K pass launch: the launches
    of all layers back to back between two events on the launching stream,
    queued behind a backlog so host launch cost stays off the GPU clock;
    `reps` such batches.  (Events around every single launch would add the
    command processor's marker latency, about 1.7 us, to each; the profiler's
    per-dispatch durations sit a few percent above this back-to-back figure.)"""
    from strataflow_amd import _lib
    n = len(args)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]
    calibrate_backlog(torch)
    torch.cuda.synchronize()
    gpu_backlog(torch, 0.05 * n * reps + 5)
    for a, b in evs:
        a.record()
        for x in args:
            _lib.check(lib.sfa_attn_decode_split(*x), "sfa_attn_decode_split")
        b.record()
    torch.cuda.synchronize()
    d = np.array([a.elapsed_time(b) for a, b in evs]) * 1e3 / n
    return float(np.mean(d)), float(np.median(d))


def time_decode(torch, kv, t_pt, q, seq_len, ctx, steps, warmup):
    """Step timing: the 32-layer loop captured once as a HIP graph and
    replayed `steps` times between two events.  Kernel timing: every split-K
    pass launch of the 32 layers between its own two events."""
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

    lib = _lib_mod().load()
    ws = kv.workspace(B, ctx)
    stream = torch.cuda.current_stream().cuda_stream
    args = [(ctypes.byref(kv.desc(layer)), q[layer].data_ptr(), out[layer].data_ptr(), t_pt.data_ptr(),
             int(t_pt.shape[1]), seq_len.data_ptr(), None, B, int(ctx), float(kv.scale), ws.data_ptr(),
             ws.numel(), stream) for layer in range(N_LAYER)]
    k_mean, k_med = time_split_launches(torch, lib, args, max(steps // 2, 4))
    for layer in range(N_LAYER):  # leave complete outputs behind
        kv.decode(layer, q[layer], t_pt, seq_len, ctx, out=out[layer])
    torch.cuda.synchronize()
    return ms_per_step, ms_eager, k_mean, k_med, out


def hbm_roofline(alg_bytes: int, k_mean_us: float, node_us: float, kernel: str, key: str) -> dict:
    """The split-K kernel's HBM roofline (algorithmic bytes over its mean
    launch duration) with the node's (split + merge + launch gaps) beside it."""
    ach = alg_bytes / (k_mean_us * 1e-6) / 1e9
    node = alg_bytes / (node_us * 1e-6) / 1e9
    return with_traffic({
        "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None, "kernel": kernel,
        "kernel_us_mean": round(k_mean_us, 3), "bytes_per_launch": alg_bytes,
        # the whole attention node per layer (split pass, merge pass, launch
        # gaps) from the graph-replayed step
        "node_us": round(node_us, 3), "node_achieved": round(node, 1),
        "node_frac": round(node / HBM_PEAK_GBS, 4)}, key)


def flat(prefix: str, d: dict) -> dict:
    """d's fields under prefix + name, nested objects flattened the same way."""
    out = {}
    for k, v in d.items():
        if isinstance(v, dict):
            out.update(flat(f"{prefix}{k}_", v))
        else:
            out[prefix + k] = v
    return out


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
    """Adds the profiled HBM bytes per launch and the rocprofv3 mean duration
    of the same kernel on the same workload, with the achieved rate and frac
    computed from that mean, beside the live figures (HIP events around
    back-to-back launches).  For a decode split pass the profile splits its
    dispatches into the back-to-back launches the live figure times (the
    rocprof_* figures, like with like) and those inside the decode steps,
    each followed by its merge pass (rocprof_*_in_step)."""
    t = load_traffic().get(key)
    if t:
        roofline["traffic"] = t.get("bytes_per_launch")
        roofline["traffic_source"] = f"profiles/traffic.json[{key}] (rocprofv3 FETCH_SIZE+WRITE_SIZE)"
        work = roofline.get("bytes_per_launch") or roofline.get("flop_per_launch")
        scale = 1e9 if roofline["unit"] == "GB/s" else 1e12
        us = t.get("kernel_us_mean_back_to_back") or t.get("kernel_us_mean")
        if work and us:
            ach = work / (us * 1e-6) / scale
            roofline["rocprof_kernel_us_mean"] = us
            roofline["rocprof_achieved"] = round(ach, 1)
            roofline["rocprof_frac"] = round(ach / roofline["peak"], 4)
            roofline["rocprof_source"] = t.get("profile") or "profiles/"
            if t.get("kernel_us_mean_in_step"):
                us_s = t["kernel_us_mean_in_step"]
                roofline["rocprof_kernel_us_mean_in_step"] = us_s
                roofline["rocprof_frac_in_step"] = round(work / (us_s * 1e-6) / scale / roofline["peak"], 4)
        for k in ("mfma_busy", "valu_busy", "lds_bank_conflict_frac"):
            if t.get(k) is not None:
                roofline[f"rocprof_{k}"] = t[k]
    return roofline


KV_NAMES = {0: "f32", 1: "f16", 8: "Q8_0"}


def decode_cpu_leg(kv, pt, q_layer0, lens, gpu_out0, budget_s: float) -> dict:
    """The oracle on layer 0 of a decode workload (all sequences of the step):
    the same seeded bytes, the same Q."""
    from oracle import oracle
    host = host_kv_from_device(kv, 0)
    q = q_layer0.cpu().numpy().reshape(len(lens), HQ, HD)
    sl = np.asarray(lens, np.int32)
    return cpu_leg(lambda nt: host.attention(q, HQ, pt, sl, n_threads=nt, mode=oracle.GGML),
                   "us/layer-step", 1e6,
                   f"layer 0 of the same workload ({len(lens)} sequence(s), "
                   f"{int(sl.sum())} positions), ggml-semantics oracle", budget_s,
                   gpu_out=gpu_out0)


def decode_leg(torch, key, lens, kv_type, steps, warmup, seed, cpu_budget_s: float = 0.0):
    """One decode workload: lens (one entry per sequence), f32, f16 or Q8_0."""
    kv, pt, t_pt, q, seq_len = build_decode_workload(torch, lens, seed, kv_type=kv_type)
    mx = int(max(lens))
    ms, _, k_mean, _, out = time_decode(torch, kv, t_pt, q, seq_len, mx, steps, warmup)
    row = {0: HD * 4, 1: HD * 2, 8: HD // 32 * 34}[kv_type]
    alg = 2 * sum(lens) * HKV * row + len(lens) * HQ * HD * 4 * 2
    us_layer = ms * 1e3 / N_LAYER
    # Q8_0 batches of two or more with >= 1024 tiles in all run the staged
    # kernel (8 kv heads: whole position columns per workgroup)
    staged = kv_type == 8 and len(lens) >= 2 and len(lens) * ((mx + 31) // 32) >= 1024
    one = "true" if len(lens) == 1 else "false"
    kname = {0: "decode_f32_kernel<128,4>", 1: f"decode_f16_kernel<128,4,{one}>",
             8: "decode_q8_staged_kernel<128,4,8>" if staged else f"decode_q8_kernel<128,4,false,{one}>"}[kv_type]
    res = {
        "workload": f"decode-attn {KV_NAMES[kv_type]} KV, Mixtral GQA 32q/8kv hd128, "
                    f"B={len(lens)}, context {lens if len(lens) > 1 else lens[0]}, 256-token pages "
                    f"shuffled, {N_LAYER} layers with distinct caches",
        "us_per_layer_step": round(us_layer, 3),
        "us_per_layer_token": round(us_layer / len(lens), 3),
        "tokens_per_s": round(len(lens) * 1e3 / ms, 1),
        "roofline": hbm_roofline(alg, k_mean, us_layer, f"{kname} (split-K pass)", key),
    }
    if cpu_budget_s > 0:
        res["cpu_baseline"] = decode_cpu_leg(kv, pt, q[0], lens, out[0].cpu().numpy(), cpu_budget_s)
    del kv, q, out
    torch.cuda.empty_cache()
    return res


def q8_bench(torch, steps, warmup, seed, cpu_budget_s: float = 0.0):
    """Q8_0 KV decode: (a) batch 1 at context 32768; (b) batch 8 with lengths
    uniform in [8192, 32768] sharing one page pool; and the 2048-on-2048 chunked
    prefill over a Q8_0 cache."""
    lens_b8 = [int(x) for x in np.random.default_rng(seed).integers(8192, 32769, 8)]
    return {
        "ctx32k_b1": decode_leg(torch, "decode_q8_0_ctx32k_b1", [32768], 8, steps, warmup, seed,
                                cpu_budget_s),
        "b8_varlen_8k_32k": decode_leg(torch, "decode_q8_0_b8", lens_b8, 8, steps, warmup, seed,
                                       cpu_budget_s),
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


def prefill_bench(torch, steps: int, warmup: int, seed: int, kv_type: int = 1, cpu_budget_s: float = 0.0):
    """Chunked causal prefill: 2048 tokens at positions 2048..4095 over a
    4096-position paged f16 (Q8_0, f32) cache, 8 layers with distinct caches."""
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
    cpu = None
    if cpu_budget_s > 0:
        from oracle import oracle
        out0 = kv.prefill(0, qs[0], pt, n_cached).cpu().numpy()
        host = host_kv_from_device(kv, 0)
        q0 = qs[0].cpu().numpy()
        pt_h = pt.cpu().numpy()[None]
        nkv = np.array([n_kv], np.int32)
        one = kv_head_sample(host, 1)
        q_one = np.ascontiguousarray(q0[:, : HQ // HKV])
        cpu = cpu_leg(lambda nt: host.attention(q0[None], HQ, pt_h, nkv, T=T, n_threads=nt,
                                                mode=oracle.GGML),
                      "us/layer-chunk", 1e6,
                      "layer 0 of the same workload (the whole 2048-token chunk, all 32 heads), "
                      "ggml-semantics oracle with the causal mask", cpu_budget_s,
                      run_1t=lambda nt: one.attention(q_one[None], HQ // HKV, pt_h, nkv, T=T, n_threads=nt,
                                                      mode=oracle.GGML),
                      scale_1t=1e6 * HKV,
                      sample_1t="kv head 0 of layer 0 (its 4 query heads, the whole chunk), times 8 "
                                "kv heads; ggml-semantics oracle with the causal mask",
                      gpu_out=out0)
    # one flat object (roofline and CPU baseline fields side by side) so that
    # every figure survives a reader that keeps scalar fields only
    res = {
        "workload": f"causal prefill {name} KV, 2048-token chunk on 2048 cached, Mixtral GQA 32q/8kv hd128",
        "us_per_layer_chunk": round(us, 2),
        "us_per_layer_token": round(us / T, 5),
        "tflops": round(tflops, 1),
        "flop_per_layer_chunk": flops,
    }
    res.update(with_traffic({"bound": "mfma", "achieved": round(tflops, 1),
                             "peak": peak, "unit": "TFLOP/s",
                             "frac": round(tflops / peak, 4), "traffic": None,
                             "kernel": {0: "prefill_f32_kernel<128,4>", 1: "prefill_f16_kernel<128,4>",
                                        8: "prefill_q8_kernel<128,4>"}[kv_type],
                             "flop_per_launch": flops},
                            {1: "prefill_2048_on_2048", 0: "prefill_f32_2048_on_2048",
                             8: "prefill_q8_0_2048_on_2048"}[kv_type]))
    if cpu is not None:
        res.update(flat("cpu_", cpu))
    del kv, qs, out
    torch.cuda.empty_cache()
    return res


def layer_bench(torch, steps: int, warmup: int, seed: int, n_layer: int = 8) -> dict:
    """The whole decode layer on the GPU: n_layer Mixtral-shaped layers (n_embd
    4096, 32 q / 8 kv heads of 128, 8 experts top-2, n_ff 14336; f16 weights
    N(0,1)*0.02, distinct per layer) over distinct f16 caches at context 4096,
    B = 1, one token per step through every layer, the step captured as one HIP
    graph: rms_norm, the Q/K/V product (the three weights stacked) with RoPE
    and the KV append in the same launch, attention, the wo product with the residual added in the same
    pass, rms_norm with the router product and the routing (one launch), the
    two routed experts' SwiGLU FFN and the residual.
    The roofline counts the bytes a layer-token reads once: the Q/K/V, wo and
    router weights, the two routed experts' gate, up and down rows, the KV
    history (activations are a few KB)."""
    from strataflow_amd import layer as ops
    from strataflow_amd import synth
    from strataflow_amd.paged_kv import SFA_KV_F16, PagedKV
    dev = torch.device("cuda:0")
    D, F, E, K, ctx = 4096, 14336, 8, 2, 4096
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)

    def w(*shape):
        return (torch.randn(shape, device=dev, generator=gen, dtype=torch.float16) * 0.02).contiguous()

    layers = [dict(attn_norm=torch.ones(D, device=dev), ffn_norm=torch.ones(D, device=dev),
                   wqkv=w((HQ + 2 * HKV) * HD, D), wo=w(D, HQ * HD), gate_inp=w(E, D),
                   gate=w(E, F, D), up=w(E, F, D), down=w(E, D, F)) for _ in range(n_layer)]
    pages = ctx // PAGE + 2
    kv = PagedKV(n_layer, HQ, HKV, HD, SFA_KV_F16, PAGE, pages, device=dev)
    rng = np.random.default_rng(seed)
    pt = torch.from_numpy(synth.page_tables(rng, [ctx], PAGE, pages)).to(dev)
    hist = ctx - 1
    for il in range(n_layer):
        pos = torch.arange(hist, device=dev, dtype=torch.int32)
        kk = synth.rope_normal_torch(torch.randn((hist, HKV, HD), device=dev, generator=gen), pos, 1e6)
        kv.append(il, kk.contiguous(), torch.randn((hist, HKV, HD), device=dev, generator=gen),
                  torch.zeros(hist, device=dev, dtype=torch.int32), pos, pt)
    x0 = torch.randn((1, D), device=dev, generator=gen)
    x = torch.empty_like(x0)
    cur, ffn_inp = torch.empty_like(x0), torch.empty_like(x0)
    q = torch.empty((1, HQ, HD), device=dev)
    ids, wts = torch.empty((1, K), dtype=torch.int32, device=dev), torch.empty((1, K), device=dev)
    moe_ws = torch.empty(K * F * 4, dtype=torch.uint8, device=dev)
    pos1 = torch.tensor([hist], dtype=torch.int32, device=dev)
    seq1 = torch.zeros(1, dtype=torch.int32, device=dev)
    sl = torch.tensor([ctx], dtype=torch.int32, device=dev)
    attn = torch.empty((1, HQ * HD), device=dev)

    def step():
        x.copy_(x0)
        for il, L in enumerate(layers):
            ops.rms_norm(x, L["attn_norm"], 1e-5, out=cur)
            kv.qkv_rope_append(il, L["wqkv"], cur, seq1, pos1, pt, 1e6, q=q)
            kv.decode(il, q, pt, sl, ctx, out=attn)
            ops.mul_mat_vec(L["wo"], attn, residual=x, out=ffn_inp)
            ops.moe_norm_gate(ffn_inp, L["ffn_norm"], 1e-5, L["gate_inp"], K, out=cur, ids=ids, weights=wts)
            ops.moe_ffn(cur, ffn_inp, ids, wts, L["gate"], L["up"], L["down"], out=x, workspace=moe_ws)

    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    step()
    torch.cuda.synchronize()
    a.record()
    for _ in range(3):
        step()
    b.record()
    torch.cuda.synchronize()
    eager_us = a.elapsed_time(b) * 1e3 / (3 * n_layer)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    a.record()
    for _ in range(steps):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / (steps * n_layer)
    del g
    out_ok = bool(torch.isfinite(x).all().item())
    routed = ids.cpu().numpy().tolist()
    alg = (2 * ((HQ + 2 * HKV) * HD * D + D * HQ * HD + E * D)      # Q/K/V, wo, router weights (f16)
           + K * 3 * F * D * 2                                        # the routed experts' gate, up, down
           + 2 * ctx * HKV * HD * 2                                   # K + V history (f16)
           + 2 * D * 4)                                               # the two norm weights
    ach = alg / (us * 1e-6) / 1e9
    del layers, kv
    torch.cuda.empty_cache()
    return {
        "workload": f"whole decode layer on the GPU, Mixtral shape (n_embd 4096, 32q/8kv hd128, 8 experts "
                    f"top-2, n_ff 14336), f16 weights, f16 KV at context 4096, B=1, {n_layer} layers with "
                    f"distinct weights and caches, one HIP graph per token",
        "us_per_layer_token": round(us, 2),
        "us_per_layer_token_eager": round(eager_us, 2),
        "tokens_per_s_32_layers": round(1e6 / (us * 32), 1),
        "routed_experts_last_layer": routed,
        "finite": out_ok,
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_launch": alg,
                     "kernel": "the layer's launches (graph-replayed)",
                     "what": "weights a layer-token reads (Q/K/V, wo, router, two experts) + KV history, once"},
    }


def f32_bench(torch, steps: int, warmup: int, seed: int):
    """F32 KV, the reference's own cache type: decode at context 4096 (B=1,
    32 layers) and the 2048-on-2048 chunked prefill, both on f32 MFMA."""
    return {
        "decode_ctx4096": decode_leg(torch, "decode_f32_ctx4096", [4096], 0, steps, warmup, seed),
        "prefill_2048_on_2048": prefill_bench(torch, max(steps // 10, 3), 2, seed + 1, kv_type=0),
    }


HOST_LINK_PEAK_GBS = 64.0  # PCIe 5.0 x16, one direction (the GPU reading host memory)


def window_cpu_leg(B: int, hist: int, W: int, lossless: bool, budget_s: float, seed: int) -> dict:
    """The oracle on one layer-step of the window workload's shape: B sequences
    of `hist` positions (f16), attending all of them (lossless) or the last W.
    The cache holds seeded f16 values of the same shape (the oracle's cost does
    not depend on them); parity of this workload is the tests' business."""
    from oracle import oracle
    n_pages = B * hist // PAGE
    host = oracle.HostPagedKv(HKV, HD, PAGE, oracle.KV_F16, n_pages)
    rng = np.random.default_rng(seed)
    tile = rng.standard_normal((8, host.page_bytes // 2)).astype(np.float16).view(np.uint8)
    host.k[:] = np.tile(tile, (n_pages // 8, 1))
    host.v[:] = np.tile(tile[::-1], (n_pages // 8, 1))
    pt = rng.permutation(n_pages).astype(np.int32).reshape(B, -1)
    q = rng.standard_normal((B, HQ, HD)).astype(np.float32)
    sl = np.full(B, hist, np.int32)
    lo = None if lossless else sl - W
    what = (f"one layer-step: {B} sequences of {hist} positions, every position attended (lossless)"
            if lossless else f"one layer-step: {B} sequences, the last {W} of {hist} positions attended")
    return cpu_leg(lambda nt: host.attention(q, HQ, pt, sl, lo, n_threads=nt, mode=oracle.GGML),
                   "us/layer-step", 1e6, what + ", ggml-semantics oracle, seeded f16 values", budget_s)


def window_bench(torch, seed: int, steps: int = 128, lossless_steps: int = 128, cpu_budget_s: float = 0.0,
                 lossless_layers: int = 4):
    """KV-window decode under paging pressure: 4 sequences with 65536-token
    histories, a 4096-position window, the device pool sized to the window
    (4 x 17 pages per layer), pages evicted and reused by the host page
    manager every 256 steps of a sequence.  (a) the opt-in sliding window for
    `steps` decode steps over all 32 layers; (b) the reference's lossless
    semantics (every position attended, the evicted positions read from the
    host-pinned cold pool in place) for `lossless_steps` steps over
    `lossless_layers` layers: a lossless layer-step reads 1 GB of cold pages
    over the host link (about 20 ms), so 128 steps of 32 layers would hold
    the GPU for 80 s; the per-layer-step cost does not depend on the layer
    count."""
    from strataflow_amd import _lib, synth
    from strataflow_amd.pager import SFA_ATTEND_LOSSLESS, SFA_ATTEND_WINDOW, SFA_KV_F16, KvPager
    dev = torch.device("cuda:0")
    B, hist, W = 4, 65536, 4096
    pos_bytes = HKV * HD * 2 * 2  # K and V of one position, all kv heads (f16)
    res = {}
    for name, attend, n_steps in (("sliding_window", SFA_ATTEND_WINDOW, steps),
                                  ("lossless", SFA_ATTEND_LOSSLESS, lossless_steps)):
        n_layer = N_LAYER if attend == SFA_ATTEND_WINDOW else lossless_layers
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
                # the attention node with its append (one token per sequence,
                # F16: fused into the split pass)
                pager.append_attend(layer, kb[layer], vb[layer], qb[layer], out[layer])

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
        timed = n_steps - 1
        us = t0.elapsed_time(t1) * 1e3 / (timed * n_layer)

        # bytes of the last step: resident positions from HBM, cold ones over
        # the host link (every attended position once, K and V)
        pt_h, used = pager.tables()
        hbm = link = 0
        for b in range(B):
            n = int(used[b])
            lo = n - W if attend == SFA_ATTEND_WINDOW else 0
            for lp in range(lo // PAGE, (n - 1) // PAGE + 1):
                cnt = min(n, (lp + 1) * PAGE) - max(lo, lp * PAGE)
                if pt_h[b, lp] >= 0:
                    hbm += cnt * pos_bytes
                elif pt_h[b, lp] <= -2:
                    link += cnt * pos_bytes
        qo = B * HQ * HD * 4 * 2
        # the split pass alone, over the pager's pools and tables, per launch
        lib = _lib.load()
        d_pt, d_sl, d_lo = pager.device_tables()
        d0 = pager.desc(0)
        ws_n = lib.sfa_decode_workspace_bytes(ctypes.byref(d0), B, pager.max_span)
        ws = torch.empty(ws_n, dtype=torch.uint8, device=dev)
        descs = [pager.desc(layer) for layer in range(n_layer)]
        stream = torch.cuda.current_stream().cuda_stream
        args = [(ctypes.byref(descs[layer]), qb[layer].data_ptr(), out[layer].data_ptr(), d_pt,
                 pager.max_pages, d_sl, d_lo if attend == SFA_ATTEND_WINDOW else None, B,
                 pager.max_span, 1.0 / math.sqrt(HD), ws.data_ptr(), ws_n, stream)
                for layer in range(n_layer)]
        k_mean, _ = time_split_launches(torch, lib, args, 4 if attend == SFA_ATTEND_WINDOW else 1)
        st = pager.stats()
        entry = {
            "workload": f"decode-attn f16 KV, Mixtral GQA 32q/8kv hd128, B={B}, history {hist}, "
                        f"window {W}, device pool {B * (W // PAGE + 1)} pages/layer, "
                        f"{timed} consecutive timed steps (+1 warm), {n_layer} layers",
            "semantics": ("sliding window: attends the last 4096 positions (opt-in kv_lo)"
                          if attend == SFA_ATTEND_WINDOW else
                          "lossless (reference): attends every position; evicted pages read "
                          "from the host-pinned cold pool"),
            "steps": timed,
            "us_per_layer_step": round(us, 3),
            "us_per_layer_token": round(us / B, 3),
            "tokens_per_s": round(B * 1e6 / (us * n_layer), 1),
            "includes": "paging (plan + table update), KV append (fused into the split-K pass), "
                        "split-K decode and merge",
            "pages_evicted": st["pages_evicted"], "pages_dropped": st["pages_dropped"],
            "hbm_bytes_per_layer_step": hbm + qo,
            "host_link_bytes_per_layer_step": link,
        }
        kname = "decode_f16_kernel<128,4,false> (split-K pass)"
        if attend == SFA_ATTEND_WINDOW:
            entry["roofline"] = hbm_roofline(hbm + qo, k_mean, us, kname, "window_sliding")
        else:
            ach = link / (k_mean * 1e-6) / 1e9
            node = link / (us * 1e-6) / 1e9
            entry["roofline"] = with_traffic({
                "bound": "host_link", "achieved": round(ach, 1), "peak": HOST_LINK_PEAK_GBS,
                "unit": "GB/s", "frac": round(ach / HOST_LINK_PEAK_GBS, 4), "traffic": None,
                "kernel": kname, "kernel_us_mean": round(k_mean, 3), "bytes_per_launch": link,
                "what": "cold-page bytes read over the host link (PCIe 5.0 x16, 64 GB/s a direction)",
                "node_us": round(us, 3), "node_achieved": round(node, 1),
                "node_frac": round(node / HOST_LINK_PEAK_GBS, 4)}, "window_lossless")
            hb = (hbm + qo) / (k_mean * 1e-6) / 1e9
            entry["roofline_hbm"] = {"bound": "hbm", "achieved": round(hb, 1), "peak": HBM_PEAK_GBS,
                                     "unit": "GB/s", "frac": round(hb / HBM_PEAK_GBS, 4),
                                     "bytes_per_launch": hbm + qo,
                                     "what": "window-resident bytes read from HBM by the same launches"}
        if cpu_budget_s > 0:
            entry["cpu_baseline"] = window_cpu_leg(B, hist, W, attend == SFA_ATTEND_LOSSLESS,
                                                   cpu_budget_s, seed)
        res[name] = entry
        pager.close()
        del qs, ks, vs, graph
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


# ---- CPU baseline: the oracle (ggml semantics) on the host cores ------------------
#
# The oracle restates the reference's op sequence (engine.cpp:1751-1761) with its
# cost structure: the gather into the column layout, the two cont(permute) copies
# and the cont(transpose) of V, then mul_mat -> soft_max_ext -> mul_mat.  It runs
# at one thread (the reference's determinism setting, engine.cpp:1013-1019) and
# at every host thread the process may use; each leg states its sample.

def host_info() -> dict:
    """CPU model, logical CPUs, the CPUs this process may run on and the
    thread count the CPU legs use (the affinity set, capped by OMP_NUM_THREADS
    when the environment sets it: a machine with several GPUs may give each
    GPU's process a share of its cores)."""
    aff = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(aff, int(omp)) if omp.isdigit() and int(omp) > 0 else aff
    model, phys = "", None
    try:
        with open("/proc/cpuinfo") as f:
            info = f.read()
        for line in info.splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
        cores = {(blk.split("physical id")[1].split(":")[1].split()[0],
                  blk.split("core id")[1].split(":")[1].split()[0])
                 for blk in info.split("\n\n") if "core id" in blk and "physical id" in blk}
        phys = len(cores) or None
    except (OSError, IndexError):
        pass
    return {"model": model, "nproc": os.cpu_count(), "physical_cores": phys, "affinity_cpus": aff,
            "omp_num_threads": omp or None, "threads_used": threads}


def cpu_median(fn, budget_s: float, max_calls: int = 200):
    """Median seconds of fn() over about budget_s (a call slower than a third
    of the budget is timed once, without a warm-up call)."""
    t0 = time.perf_counter()
    out = fn()
    first = time.perf_counter() - t0
    if first > budget_s / 3:
        return first, 1, out
    ts = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s and len(ts) < max_calls:
        t0 = time.perf_counter()
        out = fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), len(ts), out


def host_kv_from_device(kv, layer: int):
    """The oracle's host pools holding a copy of one layer of a PagedKV."""
    from oracle import oracle
    host = oracle.HostPagedKv(kv.n_head_kv, kv.head_dim, kv.page_size, kv.kv_type, kv.n_pages)
    host.k[:] = kv.k[layer].cpu().numpy()
    host.v[:] = kv.v[layer].cpu().numpy()
    return host


def kv_head_sample(host, n_keep: int = 1):
    """The first n_keep kv heads of a host cache as a cache of their own (the
    oracle's work scales linearly with kv heads)."""
    from oracle import oracle
    Hkv, rb = host.n_head_kv, host.page_bytes // (host.page_size * host.n_head_kv)
    small = oracle.HostPagedKv(n_keep, host.head_dim, host.page_size, host.kv_type, host.n_pages)
    for src, dst in ((host.k, small.k), (host.v, small.v)):
        dst[:] = src.reshape(src.shape[0], host.page_size, Hkv, rb)[:, :, :n_keep].reshape(dst.shape)
    return small


def parity(gpu_out, ref) -> dict:
    g = np.asarray(gpu_out, np.float64).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    return {"max_abs": float(np.max(np.abs(g - r))),
            "rel_l2": float(np.linalg.norm(g - r) / np.linalg.norm(r))}


def cpu_leg(run, unit: str, scale_us: float, sample: str, budget_s: float, run_1t=None,
            scale_1t: float | None = None, sample_1t: str | None = None, gpu_out=None) -> dict:
    """The oracle at every allotted thread and at one thread.  run(n_threads)
    performs one sampled call; scale_us turns its seconds into the leg's unit.
    run_1t / scale_1t / sample_1t give a smaller one-thread sample (the same
    work per unit, fewer units) when the full one would take too long."""
    hi = host_info()
    nt = hi["threads_used"]
    s_all, n_all, out = cpu_median(lambda: run(nt), budget_s)
    r1 = run_1t or run
    s_one, n_one, _ = cpu_median(lambda: r1(1), budget_s)
    res = {"value": round(s_all * scale_us, 1), "unit": unit, "cores": nt, "kind": "port",
           "sample": f"{sample}; median of {n_all} call(s)",
           "value_1_thread": round(s_one * (scale_1t if scale_1t is not None else scale_us), 1),
           "sample_1_thread": f"{sample_1t or sample}; median of {n_one} call(s)"}
    if gpu_out is not None:
        res["parity_vs_gpu"] = parity(gpu_out, out)
    return res


def _g(d, *path):
    for p in path:
        if not isinstance(d, dict) or p not in d:
            return None
        d = d[p]
    return d


def _traffic_x(roof):
    """HBM traffic per launch over the algorithmic bytes (or None)."""
    t, b = _g(roof, "traffic"), _g(roof, "bytes_per_launch")
    return round(t / b, 3) if t and b else None


def decode_fields(prefix: str, leg: dict, per: str = "us_per_layer_token") -> dict:
    roof = _g(leg, "roofline") or {}
    return {f"{prefix}_us": _g(leg, per), f"{prefix}_kernel_us": roof.get("kernel_us_mean"),
            f"{prefix}_frac": roof.get("frac"), f"{prefix}_rocprof_frac": roof.get("rocprof_frac"),
            f"{prefix}_rocprof_frac_in_step": roof.get("rocprof_frac_in_step"),
            f"{prefix}_node_frac": roof.get("node_frac"), f"{prefix}_traffic_x": _traffic_x(roof),
            f"{prefix}_cpu_us": _g(leg, "cpu_baseline", "value"),
            f"{prefix}_cpu_us_1t": _g(leg, "cpu_baseline", "value_1_thread")}


def legs_summary(r: dict) -> dict:
    """Every workload's headline figures in one flat object (printed last on
    the line): µs, roofline fractions (live HIP events / rocprof mean / whole
    node), HBM traffic over algorithmic bytes, and the CPU oracle at all
    allotted threads and at one thread."""
    s = {"decode_f16_4k_us": r.get("value"), "decode_f16_4k_kernel_us": _g(r, "roofline", "kernel_us_mean"),
         "decode_f16_4k_frac": _g(r, "roofline", "frac"),
         "decode_f16_4k_rocprof_frac": _g(r, "roofline", "rocprof_frac"),
         "decode_f16_4k_rocprof_frac_in_step": _g(r, "roofline", "rocprof_frac_in_step"),
         "decode_f16_4k_node_frac": _g(r, "roofline", "node_frac"),
         "decode_f16_4k_traffic_x": _traffic_x(r.get("roofline")),
         "decode_f16_4k_cpu_us": _g(r, "cpu_baseline", "value"),
         "decode_f16_4k_cpu_us_1t": _g(r, "cpu_baseline", "value_1_thread")}
    if "f16_ctx32k" in r:
        s.update(decode_fields("decode_f16_32k", r["f16_ctx32k"]))
    q8 = r.get("q8_0") or {}
    if q8:
        s.update(decode_fields("decode_q8_0_32k_b1", q8.get("ctx32k_b1")))
        s.update(decode_fields("decode_q8_0_b8", q8.get("b8_varlen_8k_32k"), per="us_per_layer_step"))
    pf = r.get("prefill") or {}
    if pf:
        s.update({"prefill_f16_us": pf.get("us_per_layer_chunk"), "prefill_f16_frac": pf.get("frac"),
                  "prefill_f16_rocprof_frac": pf.get("rocprof_frac"),
                  "prefill_f16_mfma_busy": pf.get("rocprof_mfma_busy"),
                  "prefill_f16_cpu_us": pf.get("cpu_value"), "prefill_f16_cpu_us_1t": pf.get("cpu_value_1_thread")})
    for name, leg in (("prefill_q8_0", _g(q8, "prefill_2048_on_2048")),
                      ("prefill_f32", _g(r, "f32", "prefill_2048_on_2048"))):
        if leg:
            s.update({f"{name}_us": leg.get("us_per_layer_chunk"), f"{name}_frac": leg.get("frac"),
                      f"{name}_rocprof_frac": leg.get("rocprof_frac")})
    if _g(r, "f32", "decode_ctx4096"):
        s.update(decode_fields("decode_f32_4k", r["f32"]["decode_ctx4096"]))
    w = r.get("window") or {}
    if w.get("sliding_window"):
        s.update(decode_fields("window_sliding_b4", w["sliding_window"], per="us_per_layer_step"))
        s["window_sliding_b4_steps"] = w["sliding_window"].get("steps")
    if w.get("lossless"):
        s.update(decode_fields("window_lossless_b4", w["lossless"], per="us_per_layer_step"))
        s["window_lossless_b4_steps"] = w["lossless"].get("steps")
        s["window_lossless_b4_bound"] = _g(w, "lossless", "roofline", "bound")
    ra = r.get("rope_append") or {}
    if ra:
        s.update({"rope_append_b1_us": _g(ra, "decode_b1", "us_per_layer_token"),
                  "rope_append_2048_us": _g(ra, "prefill_2048", "us_per_layer_chunk"),
                  "rope_append_2048_frac": _g(ra, "prefill_2048", "roofline", "frac")})
    ly = r.get("decode_layer") or {}
    if ly:
        s.update({"layer_us": ly.get("us_per_layer_token"), "layer_frac": _g(ly, "roofline", "frac")})
    return {k: v for k, v in s.items() if v is not None}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--cpu-budget", type=float, default=4.0, metavar="S",
                    help="seconds of timed CPU work per thread count and CPU leg")
    ap.add_argument("--window-lossless-steps", type=int, default=128, metavar="N",
                    help="decode steps of the lossless window leg (N-1 timed)")
    ap.add_argument("--window-lossless-layers", type=int, default=4, metavar="L",
                    help="layers of the lossless window leg")
    ap.add_argument("--window-steps", type=int, default=128, metavar="N",
                    help="decode steps of the sliding-window leg (N-1 timed)")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-q8", action="store_true", help="skip the Q8_0 decode legs")
    ap.add_argument("--no-window", action="store_true", help="skip the KV-window paging legs")
    ap.add_argument("--no-32k", action="store_true", help="skip the f16 context-32768 decode leg")
    ap.add_argument("--no-rope", action="store_true", help="skip the fused RoPE + append leg")
    ap.add_argument("--no-f32", action="store_true", help="skip the F32-cache legs")
    ap.add_argument("--no-layer", action="store_true", help="skip the whole-decode-layer leg")
    ap.add_argument("--only", choices=["decode4k", "decode32k", "q8", "prefill", "window", "rope", "f32", "layer"],
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
        args.no_f32 = args.no_layer = True
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
        elif args.only == "layer":
            r = layer_bench(torch, max(args.steps // 5, 5), 2, args.seed + 8)
        else:
            r = window_bench(torch, args.seed + 3, steps=args.window_steps,
                             lossless_steps=args.window_lossless_steps,
                             lossless_layers=args.window_lossless_layers)
        print(json.dumps({args.only: r}))
        return

    ctx = args.ctx
    cpu_s = 0.0 if args.no_cpu else args.cpu_budget
    kv, pt, t_pt, q, seq_len = build_decode_workload(torch, ctx, args.seed)
    ms_step, ms_eager, k_mean, k_med, out = time_decode(torch, kv, t_pt, q, seq_len, ctx, args.steps,
                                                        args.warmup)
    us_layer = ms_step * 1e3 / N_LAYER
    kv_bytes = 2 * ctx * HKV * HD * 2
    alg_bytes = kv_bytes + HQ * HD * 4 * 2  # K + V + Q + O, each once
    roof = hbm_roofline(alg_bytes, k_mean, us_layer, "decode_f16_kernel<128,4,true> (split-K pass)",
                        "decode_f16_ctx4096")
    roof["kernel_us_median"] = round(k_med, 3)

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
        "roofline": roof,
    }
    if cpu_s > 0:
        cb = decode_cpu_leg(kv, pt, q[0], [ctx], out[0].cpu().numpy(), cpu_s)
        cb["unit"] = "us/layer-token"
        result["cpu_baseline"] = cb
        result["host"] = host_info()
    del kv, q, out
    torch.cuda.empty_cache()
    if not args.no_32k:
        result["f16_ctx32k"] = decode_leg(torch, "decode_f16_ctx32k", [32768], 1,
                                          max(args.steps // 4, 5), 3, args.seed + 4)
    if not args.no_prefill:
        result["prefill"] = prefill_bench(torch, max(args.steps // 10, 3), 2, args.seed + 1,
                                          cpu_budget_s=cpu_s)
    if not args.no_q8:
        result["q8_0"] = q8_bench(torch, max(args.steps // 4, 5), 3, args.seed + 2, cpu_budget_s=cpu_s)
    if not args.no_window:
        result["window"] = window_bench(torch, args.seed + 3, steps=args.window_steps,
                                        lossless_steps=args.window_lossless_steps,
                                        lossless_layers=args.window_lossless_layers,
                                        cpu_budget_s=cpu_s)
    if not args.no_rope:
        result["rope_append"] = rope_bench(torch, max(args.steps // 5, 5), args.seed + 5)
    if not args.no_f32:
        result["f32"] = f32_bench(torch, max(args.steps // 4, 5), 3, args.seed + 6)
    if not args.no_layer:
        result["decode_layer"] = layer_bench(torch, max(args.steps // 5, 5), 2, args.seed + 8)
    result["hbm_copy_ceiling"] = copy_ceiling(torch)
    # the decode legs at 32k beside the headline roofline, the other prefill
    # caches beside the f16 prefill (flat fields)
    roof = result["roofline"]
    for prefix, leg in (("f16_ctx32k", result.get("f16_ctx32k")),
                        ("q8_0_ctx32k_b1", _g(result, "q8_0", "ctx32k_b1")),
                        ("q8_0_b8", _g(result, "q8_0", "b8_varlen_8k_32k"))):
        if leg:
            roof[f"{prefix}_frac"] = _g(leg, "roofline", "frac")
            roof[f"{prefix}_rocprof_frac"] = _g(leg, "roofline", "rocprof_frac")
            roof[f"{prefix}_kernel_us"] = _g(leg, "roofline", "kernel_us_mean")
    pf = result.get("prefill")
    if pf:
        for prefix, leg in (("q8_0", _g(result, "q8_0", "prefill_2048_on_2048")),
                            ("f32", _g(result, "f32", "prefill_2048_on_2048"))):
            if leg:
                pf[f"{prefix}_us_per_layer_chunk"] = leg.get("us_per_layer_chunk")
                pf[f"{prefix}_frac"] = leg.get("frac")
    result["legs"] = legs_summary(result)
    # every leg's figures also as scalar fields of the headline's roofline
    # object (a record that keeps only the contract's objects keeps them)
    for k, v in result["legs"].items():
        if not k.startswith("decode_f16_4k"):
            roof[k] = v
    print(json.dumps(result))


if __name__ == "__main__":
    main()
