"""Parity at the workloads' full sizes, against the oracle on every output row.

- f16 decode at context 32768 (the long-context workload on an f16 cache),
  against both oracle modes.  The kernel rounds the unnormalised exponentials
  (at most 2^8 after the lazy rescale) to f16 before P*V, ggml rounds the
  normalised P; at 32k positions ggml's P sits among f16 subnormals, so the two
  roundings part most here.  Both deltas are printed.
- the 2048-token chunk on 2048 cached positions, every one of the 2048 rows, for
  the f16, Q8_0 and F32 caches, against the oracle's T = 2048 causal attention.
- Q8_0 caches written by ggml's SIMD quantisers (the x86 form: id = 127/amax,
  ties to even; the Arm form: ties to even): the device appends with the scalar
  form, and its decode and prefill outputs stay inside the parity bar against
  the oracle run entirely in either SIMD form (cache bytes and the Q8_0
  conversion of Q).
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import Case, assert_close, errors

pytestmark = pytest.mark.gpu

F32_MAX_ABS, F32_REL = 4e-5, 2e-5  # f32 cache: f32 accumulation rounding only


def test_decode_f16_ctx32768_both_modes(gpu, oracle_mod):
    c = Case(oracle_mod, seq_lens=[32768], seed=51)
    out = c.decode()
    ma, rl = assert_close(out, c.oracle(oracle_mod.GGML), what="f16 ctx32768 vs ggml")
    ma2, rl2 = assert_close(out, c.oracle(oracle_mod.EXACT), what="f16 ctx32768 vs exact")
    print(f"f16 ctx32768: vs ggml max_abs {ma:.2e} rel_l2 {rl:.2e}; "
          f"vs exact max_abs {ma2:.2e} rel_l2 {rl2:.2e}")


def test_decode_f16_batch_long_contexts(gpu, oracle_mod):
    # four sequences of 16k..32k sharing one pool, two with window starts
    c = Case(oracle_mod, seq_lens=[32768, 16384, 24001, 30000], kv_lo=[0, 0, 20000, 1], seed=52)
    out = c.decode(max_seq_len=32768)
    ma, rl = assert_close(out, c.oracle(oracle_mod.GGML), what="f16 long batch vs ggml")
    print(f"f16 long batch: vs ggml max_abs {ma:.2e} rel_l2 {rl:.2e}")


def _chunk(oracle_mod, gpu, kv_type, seed):
    from tests.test_gpu_prefill import build, run
    Hq, Hkv, hd, n_cached, T = 32, 8, 128, 2048, 2048
    host, dev, pt, q, n_kv = build(oracle_mod, gpu, Hq=Hq, Hkv=Hkv, hd=hd, n_cached=n_cached, T=T,
                                   seed=seed, bf16=True, kv_type=kv_type)
    out = run(dev, gpu, pt, q, n_cached)
    ref = host.attention(q[None], Hq, pt, np.array([n_kv], np.int32), T=T,
                         mode=oracle_mod.GGML)[0].reshape(T, -1)
    return host, pt, q, n_kv, out, ref


def test_prefill_f16_chunk_2048_on_2048_all_rows(gpu, oracle_mod):
    host, pt, q, n_kv, out, ref = _chunk(oracle_mod, gpu, 1, 61)
    ma, rl = assert_close(out, ref, what="f16 chunk vs ggml")
    ex = host.attention(q[None], 32, pt, np.array([n_kv], np.int32), T=2048,
                        mode=oracle_mod.EXACT)[0].reshape(2048, -1)
    ma2, rl2 = assert_close(out, ex, what="f16 chunk vs exact")
    # the bar holds row by row, not only over the whole chunk
    worst = max(errors(out[t], ref[t])[1] for t in range(0, 2048, 1))
    assert worst <= 1e-3, worst
    print(f"f16 chunk: vs ggml max_abs {ma:.2e} rel_l2 {rl:.2e} (worst row {worst:.2e}); "
          f"vs exact max_abs {ma2:.2e} rel_l2 {rl2:.2e}")


def test_prefill_q8_chunk_2048_on_2048_all_rows(gpu, oracle_mod):
    host, pt, q, n_kv, out, ref = _chunk(oracle_mod, gpu, 8, 62)
    ma, rl = assert_close(out, ref, what="q8 chunk vs ggml")
    worst = max(errors(out[t], ref[t])[1] for t in range(2048))
    assert worst <= 1e-3, worst
    print(f"q8 chunk: vs ggml max_abs {ma:.2e} rel_l2 {rl:.2e} (worst row {worst:.2e})")


def test_prefill_f32_chunk_2048_on_2048_all_rows(gpu, oracle_mod):
    host, pt, q, n_kv, out, ref = _chunk(oracle_mod, gpu, 0, 63)
    ma, rl = assert_close(out, ref, max_abs=F32_MAX_ABS, rel_l2=F32_REL, what="f32 chunk vs ggml")
    print(f"f32 chunk: vs ggml max_abs {ma:.2e} rel_l2 {rl:.2e}")


# ---- ggml's SIMD Q8_0 quantisers -------------------------------------------------

def _q8_forms_case(oracle_mod, gpu, form, *, lens, T=1, seed):
    """One cache written twice from the same f32 K/V: on the device by
    sfa_kv_append (scalar form) and on the host by the oracle in `form`."""
    import torch
    from strataflow_amd import synth
    from strataflow_amd.paged_kv import PagedKV
    Hq, Hkv, hd, ps = 32, 8, 128, 256
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    B = lens.size
    n_pages = int(sum((int(n) + ps - 1) // ps for n in lens)) + 2
    max_pages = int(max((int(n) + ps - 1) // ps for n in lens))
    pt = synth.page_tables(rng, lens, ps, n_pages, max_pages)
    host = oracle_mod.HostPagedKv(Hkv, hd, ps, oracle_mod.KV_Q8_0, n_pages)
    host_scalar = oracle_mod.HostPagedKv(Hkv, hd, ps, oracle_mod.KV_Q8_0, n_pages)
    dev = PagedKV(1, Hq, Hkv, hd, 8, ps, n_pages, device=gpu)
    t_pt = torch.from_numpy(pt).to(gpu)
    qs = []
    for b in range(B):
        n = int(lens[b])
        pos = np.arange(n, dtype=np.int32)
        _, k, v = synth.qkv(rng, n, 1, Hkv, hd, pos, 1e6)
        q = synth.qkv(rng, T, Hq, Hkv, hd, pos[n - T:], 1e6)[0]
        seq = np.full(n, b, np.int32)
        with oracle_mod.q8_variant(form):
            assert host.append(k, v, seq, pos, pt) == 0
        assert host_scalar.append(k, v, seq, pos, pt) == 0
        dev.append(0, torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu), torch.from_numpy(seq).to(gpu),
                   torch.from_numpy(pos).to(gpu), t_pt)
        qs.append(q)
    torch.cuda.synchronize()
    # the device wrote the scalar form's bytes
    assert np.array_equal(dev.k[0].cpu().numpy(), host_scalar.k[:n_pages])
    assert np.array_equal(dev.v[0].cpu().numpy(), host_scalar.v[:n_pages])
    n_diff = int(np.count_nonzero(host.k[:n_pages] != host_scalar.k[:n_pages]) +
                 np.count_nonzero(host.v[:n_pages] != host_scalar.v[:n_pages]))
    return host, dev, pt, t_pt, np.stack(qs).astype(np.float32), n_diff


@pytest.mark.parametrize("form", ["avx2", "neon"])
def test_q8_decode_vs_simd_quantiser_forms(gpu, oracle_mod, form):
    import torch
    f = {"avx2": oracle_mod.Q8_AVX2, "neon": oracle_mod.Q8_NEON}[form]
    lens = [32768, 9000, 20000]
    host, dev, pt, t_pt, q, n_diff = _q8_forms_case(oracle_mod, gpu, f, lens=lens, seed=71)
    q = q[:, 0]
    out = dev.decode(0, torch.from_numpy(q).to(gpu), t_pt,
                     torch.tensor(lens, dtype=torch.int32, device=gpu), 32768).cpu().numpy()
    with oracle_mod.q8_variant(f):
        ref = host.attention(q, 32, pt, np.array(lens, np.int32), mode=oracle_mod.GGML).reshape(len(lens), -1)
    ma, rl = assert_close(out, ref, what=f"q8 decode vs ggml ({form} quantiser)")
    print(f"q8 decode vs ggml ({form} form): max_abs {ma:.2e} rel_l2 {rl:.2e}; "
          f"cache bytes differing from the scalar form: {n_diff}")


@pytest.mark.parametrize("form", ["avx2", "neon"])
def test_q8_prefill_vs_simd_quantiser_forms(gpu, oracle_mod, form):
    import torch
    f = {"avx2": oracle_mod.Q8_AVX2, "neon": oracle_mod.Q8_NEON}[form]
    T, n_kv = 512, 2560
    host, dev, pt, t_pt, q, n_diff = _q8_forms_case(oracle_mod, gpu, f, lens=[n_kv], T=T, seed=72)
    out = dev.prefill(0, torch.from_numpy(q[0]).to(gpu), t_pt[0], n_kv - T).cpu().numpy()
    with oracle_mod.q8_variant(f):
        ref = host.attention(q, 32, pt, np.array([n_kv], np.int32), T=T,
                             mode=oracle_mod.GGML)[0].reshape(T, -1)
    ma, rl = assert_close(out, ref, what=f"q8 prefill vs ggml ({form} quantiser)")
    print(f"q8 prefill vs ggml ({form} form): max_abs {ma:.2e} rel_l2 {rl:.2e}; "
          f"cache bytes differing from the scalar form: {n_diff}")
