"""Config 1: the tiny llama-arch MoE (4 layers, n_embd 256, 8 q / 4 kv heads of
32, 8 experts top-2, ff 512, vocab 4096, f16 KV in 256-token pages), a seeded
32-token prompt and 64 greedy steps.  The gate is the reference's
(tests/test_engine_oracle.cpp:200-236): identical greedy token sequences and a
per-step max |delta logit| below 1e-3, here between the attention node on the
GPU (libsfa) and on the oracle, with the rest of the graph shared."""
import numpy as np
import pytest

from strataflow_amd.tiny_moe import HipAttention, TinyMoe, TinyMoeConfig, TinyMoeWeights

from .helpers import OracleAttention

N_PROMPT, N_GEN = 32, 64


def _prompt(cfg):
    return np.random.default_rng(1).integers(0, cfg.n_vocab, N_PROMPT)


def _compare(ref, got):
    (rt, rl), (gt, gl) = ref, got
    dl = max(float(np.max(np.abs(a - b))) for a, b in zip(rl, gl))
    margins = [float(np.sort(x)[-1] - np.sort(x)[-2]) for x in rl]
    return rt == gt, dl, min(margins)


def test_tiny_moe_oracle_modes_agree(oracle_mod):
    # CPU: ggml-semantics and float64 attention give the same greedy run
    cfg = TinyMoeConfig()
    w = TinyMoeWeights(cfg, seed=0)
    n_ctx = N_PROMPT + N_GEN
    ref = TinyMoe(cfg, w, OracleAttention(oracle_mod, cfg, n_ctx, oracle_mod.GGML)).generate(
        _prompt(cfg), N_GEN)
    ex = TinyMoe(cfg, w, OracleAttention(oracle_mod, cfg, n_ctx, oracle_mod.EXACT)).generate(
        _prompt(cfg), N_GEN)
    same, dl, margin = _compare(ref, ex)
    assert same and dl < 1e-3, (dl, margin)
    assert len(set(ref[0])) > 4  # the run is not degenerate


@pytest.mark.gpu
@pytest.mark.parametrize("kv_type", [1, 0], ids=["f16_cache", "f32_cache"])
@pytest.mark.parametrize("fused_rope", [False, True], ids=["host_rope", "fused_rope_append"])
@pytest.mark.parametrize("chunked", [False, True], ids=["per_token_prompt", "chunked_prompt"])
def test_tiny_moe_greedy_identical(gpu, oracle_mod, chunked, fused_rope, kv_type):
    # the f16 cache is the config's; f32 is the reference engine's own cache type
    cfg = TinyMoeConfig()
    w = TinyMoeWeights(cfg, seed=0)
    n_ctx = N_PROMPT + N_GEN
    ref = TinyMoe(cfg, w, OracleAttention(oracle_mod, cfg, n_ctx, oracle_mod.GGML, kv_type=kv_type)).generate(
        _prompt(cfg), N_GEN, chunked_prompt=chunked)
    got = TinyMoe(cfg, w, HipAttention(cfg, n_ctx, device=gpu, fused_rope=fused_rope, kv_type=kv_type)).generate(
        _prompt(cfg), N_GEN, chunked_prompt=chunked)
    same, dl, margin = _compare(ref, got)
    print(f"\n[tiny-moe kv_type={kv_type} chunked={chunked} fused_rope={fused_rope}] seq match={same} "
          f"max per-step |dlogit|={dl:.3e} min top-2 margin={margin:.3e} tokens={got[0]}")
    assert same, (ref[0], got[0])
    assert dl < 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("chunked", [False, True], ids=["per_token_prompt", "chunked_prompt"])
def test_tiny_moe_whole_layer_on_gpu(gpu, oracle_mod, chunked):
    """Every op of the layer on the GPU (TinyMoeGpu: rms_norm, the Q/K/V product,
    fused RoPE + append, attention with wo + residual fused, routing, SwiGLU
    experts, the output head) against the host graph with the oracle's
    attention: the same greedy sequence and the same per-step logit bar."""
    from strataflow_amd.tiny_moe import TinyMoeGpu
    cfg = TinyMoeConfig()
    w = TinyMoeWeights(cfg, seed=0)
    n_ctx = N_PROMPT + N_GEN
    ref = TinyMoe(cfg, w, OracleAttention(oracle_mod, cfg, n_ctx, oracle_mod.GGML)).generate(
        _prompt(cfg), N_GEN, chunked_prompt=chunked)
    got = TinyMoeGpu(cfg, w, n_ctx, device=gpu).generate(_prompt(cfg), N_GEN, chunked_prompt=chunked)
    same, dl, margin = _compare(ref, got)
    print(f"\n[tiny-moe whole layer on GPU chunked={chunked}] seq match={same} "
          f"max per-step |dlogit|={dl:.3e} min top-2 margin={margin:.3e}")
    assert same, (ref[0], got[0])
    assert dl < 1e-3
