"""The tiny llama-arch MoE decode loop around the attention node.

A host restatement (numpy, float32) of the reference engine's per-token graph,
used to check that swapping the attention node leaves greedy decoding intact:

  embedding      get_rows(token_embd, tok)                         engine.cpp:2712
  per layer      rms_norm * attn_norm; Q/K/V = W * cur; RoPE NORMAL on Q, K
                                                                   engine.cpp:1877-1897
                 attention node (KV append + attention)            engine.cpp:1901 -> 1633-1762
                 wo * attn + residual                              engine.cpp:1905-1906
                 rms_norm * ffn_norm; router softmax; top-k; weights / clamp(sum)
                                                                   engine.cpp:1908-1925
                 experts: down * (silu(gate * cur) * (up * cur)), weighted sum
                 + residual                                        engine.cpp:1964-1986
  head           rms_norm * output_norm; logits = output * x       engine.cpp:2991-2994

Weights follow the reference's tiny-MoE generator (spike/stream_decode/
make_tiny_moe_gguf.py:57-75): N(0,1) * 0.02 from one seeded generator in
tensor order, norms 1.  The attention node is a callable, so the same loop
runs with the HIP library (``HipAttention``) or with any other implementation
of the node; everything else is bit-for-bit the same code on both sides.
The prompt is fed one token at a time, as the reference engine does
(tests/test_engine_oracle.cpp:180-187), or as one chunk (prefill kernel).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import synth


@dataclass(frozen=True)
class TinyMoeConfig:
    n_layer: int = 4
    n_embd: int = 256
    n_head: int = 8
    n_head_kv: int = 4
    head_dim: int = 32
    n_expert: int = 8
    n_expert_used: int = 2
    n_ff: int = 512
    n_vocab: int = 4096
    rms_eps: float = 1e-5
    freq_base: float = 10000.0
    page_size: int = 256


class TinyMoeWeights:
    def __init__(self, cfg: TinyMoeConfig, seed: int = 0):
        rng = np.random.default_rng(seed)

        def tt(*shape):
            return (rng.standard_normal(shape).astype(np.float32) * np.float32(0.02))

        E, F, D = cfg.n_expert, cfg.n_ff, cfg.n_embd
        kv = cfg.n_head_kv * cfg.head_dim
        self.token_embd = tt(cfg.n_vocab, D)
        self.output_norm = np.ones(D, np.float32)
        self.output = tt(cfg.n_vocab, D)
        self.layers = []
        for _ in range(cfg.n_layer):
            self.layers.append(dict(
                attn_norm=np.ones(D, np.float32),
                wq=tt(cfg.n_head * cfg.head_dim, D), wk=tt(kv, D), wv=tt(kv, D),
                wo=tt(D, cfg.n_head * cfg.head_dim),
                ffn_norm=np.ones(D, np.float32),
                gate_inp=tt(E, D), gate_exps=tt(E, F, D), down_exps=tt(E, D, F), up_exps=tt(E, F, D),
            ))


def rms_norm(x: np.ndarray, eps: float) -> np.ndarray:
    # mean of squares accumulated in double, as ggml's rms_norm does
    ms = np.mean(np.square(x.astype(np.float64)), axis=-1, keepdims=True)
    return (x * (1.0 / np.sqrt(ms + eps)).astype(np.float32)).astype(np.float32)


def softmax(x: np.ndarray) -> np.ndarray:
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp((x - m).astype(np.float32))
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def silu(x: np.ndarray) -> np.ndarray:
    return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def moe_ffn(w: dict, cur: np.ndarray, cfg: TinyMoeConfig) -> np.ndarray:
    """cur [T, D] -> [T, D]: softmax gating, top-k by probability, weights
    renormalised by their sum clamped at 2^-14 (engine.cpp:1912-1925)."""
    probs = softmax(cur @ w["gate_inp"].T)                         # [T, E]
    sel = np.argsort(-probs, axis=-1, kind="stable")[:, :cfg.n_expert_used]
    wsel = np.take_along_axis(probs, sel, axis=-1)
    wsel = wsel / np.maximum(wsel.sum(axis=-1, keepdims=True), np.float32(6.103515625e-5))
    out = np.zeros_like(cur)
    for t in range(cur.shape[0]):
        for j in range(cfg.n_expert_used):
            e = int(sel[t, j])
            up = w["up_exps"][e] @ cur[t]
            gate = w["gate_exps"][e] @ cur[t]
            out[t] += wsel[t, j] * (w["down_exps"][e] @ (silu(gate) * up))
    return out


class TinyMoe:
    """Decode loop; ``attention(layer, q, k, v, pos0)`` appends k/v at
    positions pos0.. and returns the attention output [T, Hq*hd]."""

    def __init__(self, cfg: TinyMoeConfig, weights: TinyMoeWeights, attention):
        self.cfg, self.w, self.attention = cfg, weights, attention

    def forward(self, tokens, pos0: int) -> np.ndarray:
        """tokens [T] at positions pos0..pos0+T-1 -> logits of the last [n_vocab]."""
        cfg, w = self.cfg, self.w
        tokens = np.asarray(tokens, np.int64)
        T = tokens.size
        pos = np.arange(pos0, pos0 + T, dtype=np.int32)
        x = w.token_embd[tokens].astype(np.float32)                # [T, D]
        for il, L in enumerate(w.layers):
            cur = rms_norm(x, cfg.rms_eps) * L["attn_norm"]
            q = (cur @ L["wq"].T).reshape(T, cfg.n_head, cfg.head_dim)
            k = (cur @ L["wk"].T).reshape(T, cfg.n_head_kv, cfg.head_dim)
            v = (cur @ L["wv"].T).reshape(T, cfg.n_head_kv, cfg.head_dim)
            if not getattr(self.attention, "applies_rope", False):
                q = synth.rope_normal(q, pos, cfg.freq_base)
                k = synth.rope_normal(k, pos, cfg.freq_base)
            attn = self.attention(il, np.ascontiguousarray(q), np.ascontiguousarray(k),
                                  np.ascontiguousarray(v), pos0)
            ffn_inp = (attn @ L["wo"].T + x).astype(np.float32)
            cur = rms_norm(ffn_inp, cfg.rms_eps) * L["ffn_norm"]
            x = (moe_ffn(L, cur, cfg) + ffn_inp).astype(np.float32)
        h = rms_norm(x[-1:], cfg.rms_eps) * w.output_norm
        return (h @ w.output.T)[0].astype(np.float32)

    def generate(self, prompt, n_generate: int, chunked_prompt: bool = False):
        """Greedy decode: returns (tokens, per-step logits)."""
        logits = None
        if chunked_prompt:
            logits = self.forward(prompt, 0)
        else:
            for i, tok in enumerate(prompt):
                logits = self.forward([tok], i)
        pos = len(prompt)
        toks, steps = [], []
        for _ in range(n_generate):
            steps.append(logits)
            nxt = int(np.argmax(logits))
            toks.append(nxt)
            logits = self.forward([nxt], pos)
            pos += 1
        return toks, steps


class HipAttention:
    """The attention node on the GPU through libsfa.so: per layer a paged cache
    (f16 by default, or f32 as the reference keeps it; one 256-token page per
    sequence here), sfa_kv_append, then sfa_attn_decode (one token) or
    sfa_attn_prefill (a chunk).  With ``fused_rope`` it receives Q and K before
    RoPE and runs sfa_rope_kv_append (RoPE of Q and K fused with the append)
    instead."""

    def __init__(self, cfg: TinyMoeConfig, n_ctx: int, device: str = "cuda", seed: int = 0,
                 fused_rope: bool = False, kv_type: int | None = None):
        self.applies_rope = fused_rope
        import torch

        from .paged_kv import SFA_KV_F16, PagedKV
        self.torch, self.cfg, self.n_ctx = torch, cfg, n_ctx
        max_pages = (n_ctx + cfg.page_size - 1) // cfg.page_size
        n_pages = max_pages + 3
        self.kv = PagedKV(cfg.n_layer, cfg.n_head, cfg.n_head_kv, cfg.head_dim,
                          SFA_KV_F16 if kv_type is None else kv_type, cfg.page_size, n_pages,
                          device=device)
        rng = np.random.default_rng(seed)
        self.pt = torch.from_numpy(synth.page_tables(rng, [n_ctx], cfg.page_size, n_pages,
                                                     max_pages)).to(device)
        self.device = device

    def __call__(self, layer, q, k, v, pos0):
        torch = self.torch
        T = q.shape[0]
        dev = self.device
        pos = torch.arange(pos0, pos0 + T, dtype=torch.int32, device=dev)
        seq = torch.zeros(T, dtype=torch.int32, device=dev)
        tk = torch.from_numpy(np.ascontiguousarray(k)).to(dev)
        tv = torch.from_numpy(np.ascontiguousarray(v)).to(dev)
        tq = torch.from_numpy(np.ascontiguousarray(q)).to(dev)
        if self.applies_rope:
            self.kv.rope_append(layer, tq, tk, tv, seq, pos, self.pt, self.cfg.freq_base)
        else:
            self.kv.append(layer, tk, tv, seq, pos, self.pt)
        if T == 1:
            sl = torch.tensor([pos0 + 1], dtype=torch.int32, device=dev)
            out = self.kv.decode(layer, tq, self.pt, sl, self.n_ctx)
        else:
            out = self.kv.prefill(layer, tq, self.pt[0], pos0)
        return out.cpu().numpy()


class TinyMoeGpu(TinyMoe):
    """The whole forward on the GPU through libsfa.so, the decode layer of
    build_router_segment + build_expert_segment (engine.cpp:1877-1986) op by
    op: rms_norm * attn_norm; one product for Q, K and V (the three weights
    stacked row-wise: the same dot products, one launch) with RoPE of Q and K
    and the KV append in the same launch (Q8_0 caches: the product, then RoPE
    fused with the append); the decode (one token) or the causal prefill (a
    chunk), then the wo product with the residual added in the same pass;
    rms_norm * ffn_norm with the router product and the softmax top-k
    routing (one launch); the SwiGLU experts with their weighted sum and the residual; the
    output head.  Token ids go in and the last row's logits come out; nothing
    else crosses the host link.  ``weight_dtype`` float16 rounds the weights
    (a different model, for timing); float32 is the reference's."""

    def __init__(self, cfg: TinyMoeConfig, weights: TinyMoeWeights, n_ctx: int, device: str = "cuda",
                 seed: int = 0, kv_type: int | None = None, weight_dtype=None):
        import torch

        from .paged_kv import SFA_KV_F16, PagedKV
        super().__init__(cfg, weights, attention=None)
        self.torch, self.n_ctx, self.device = torch, n_ctx, device
        wd = torch.float32 if weight_dtype is None else weight_dtype

        def dev(a, dtype=torch.float32):
            return torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dtype)

        self.embd = dev(weights.token_embd)
        self.output_norm = dev(weights.output_norm)
        self.output = dev(weights.output, wd)
        self.layers = []
        for L in weights.layers:
            self.layers.append(dict(
                attn_norm=dev(L["attn_norm"]), ffn_norm=dev(L["ffn_norm"]),
                wqkv=dev(np.concatenate([L["wq"], L["wk"], L["wv"]], axis=0), wd), wo=dev(L["wo"], wd),
                gate_inp=dev(L["gate_inp"], wd), gate_exps=dev(L["gate_exps"], wd),
                up_exps=dev(L["up_exps"], wd), down_exps=dev(L["down_exps"], wd)))
        max_pages = (n_ctx + cfg.page_size - 1) // cfg.page_size
        n_pages = max_pages + 3
        self.kv = PagedKV(cfg.n_layer, cfg.n_head, cfg.n_head_kv, cfg.head_dim,
                          SFA_KV_F16 if kv_type is None else kv_type, cfg.page_size, n_pages, device=device)
        rng = np.random.default_rng(seed)
        self.pt = torch.from_numpy(synth.page_tables(rng, [n_ctx], cfg.page_size, n_pages, max_pages)).to(device)
        self._moe_ws = None

    def forward(self, tokens, pos0: int) -> np.ndarray:
        from . import layer as ops
        from .paged_kv import SFA_KV_F16, SFA_KV_F32
        torch, cfg = self.torch, self.cfg
        dev = self.device
        tok = torch.as_tensor(np.asarray(tokens, np.int64), device=dev)
        T = int(tok.numel())
        Hq, Hkv, hd = cfg.n_head, cfg.n_head_kv, cfg.head_dim
        pos = torch.arange(pos0, pos0 + T, dtype=torch.int32, device=dev)
        seq = torch.zeros(T, dtype=torch.int32, device=dev)
        sl = torch.tensor([pos0 + T], dtype=torch.int32, device=dev)
        x = self.embd.index_select(0, tok)                                  # get_rows (engine.cpp:2712)
        for il, L in enumerate(self.layers):
            cur = ops.rms_norm(x, L["attn_norm"], cfg.rms_eps)
            if self.kv.kv_type in (SFA_KV_F16, SFA_KV_F32):
                # the product, RoPE and the append in one launch
                q = self.kv.qkv_rope_append(il, L["wqkv"], cur, seq, pos, self.pt, cfg.freq_base)
            else:  # Q8_0: a block spans 16 RoPE pairs, so the product and the append are separate
                qkv = ops.mul_mat_vec(L["wqkv"], cur)
                q = qkv[:, :Hq * hd].contiguous().view(T, Hq, hd)
                k = qkv[:, Hq * hd:(Hq + Hkv) * hd].contiguous().view(T, Hkv, hd)
                v = qkv[:, (Hq + Hkv) * hd:].contiguous().view(T, Hkv, hd)
                self.kv.rope_append(il, q, k, v, seq, pos, self.pt, cfg.freq_base)
            if T == 1:
                attn = self.kv.decode(il, q, self.pt, sl, self.n_ctx)
            else:
                attn = self.kv.prefill(il, q, self.pt[0], pos0)
            ffn_inp = ops.mul_mat_vec(L["wo"], attn, residual=x)
            cur, ids, wts = ops.moe_norm_gate(ffn_inp, L["ffn_norm"], cfg.rms_eps, L["gate_inp"],
                                              cfg.n_expert_used)
            need = T * cfg.n_expert_used * cfg.n_ff * 4
            if self._moe_ws is None or self._moe_ws.numel() < need:
                self._moe_ws = torch.empty(need, dtype=torch.uint8, device=dev)
            x = ops.moe_ffn(cur, ffn_inp, ids, wts, L["gate_exps"], L["up_exps"], L["down_exps"],
                            workspace=self._moe_ws)
        h = ops.rms_norm(x[-1:].contiguous(), self.output_norm, cfg.rms_eps)
        return ops.mul_mat_vec(self.output, h)[0].cpu().numpy()
