"""KV append on the GPU (sfa_kv_append) writes the same bytes as the oracle's
ggml_cpy restatement: f32 as is, f16 round-to-nearest-even and Q8_0
quantisation."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kv_type", [0, 1, 8])
@pytest.mark.parametrize("hd", [32, 128])
def test_append_bit_exact(gpu, oracle_mod, kv_type, hd):
    import torch
    from strataflow_amd.paged_kv import PagedKV
    rng = np.random.default_rng(hd + kv_type)
    Hkv, ps, n_pages, n_tok = 4, 32, 12, 150
    # two sequences, interleaved tokens, shuffled pages; include an exact
    # zero block and large values
    seq = (np.arange(n_tok) % 2).astype(np.int32)
    pos = (np.arange(n_tok) // 2).astype(np.int32)
    pt = rng.permutation(n_pages).astype(np.int32)[:6].reshape(2, 3)
    k = (rng.standard_normal((n_tok, Hkv, hd)) * 3).astype(np.float32)
    v = rng.standard_normal((n_tok, Hkv, hd)).astype(np.float32)
    k[5, 1, :32] = 0.0
    v[7, 0, :32] = 1e4
    if kv_type == 8 and hd < 64:
        # a Q8_0 cache of head_dim 32 is refused for every entry point
        from strataflow_amd import _lib
        with pytest.raises(_lib.SfaError) as e:
            PagedKV(1, Hkv, Hkv, hd, kv_type, ps, n_pages, device=gpu)
        assert e.value.status == _lib.SFA_ERR_UNSUPPORTED
        return
    host = oracle_mod.HostPagedKv(Hkv, hd, ps, kv_type, n_pages)
    assert host.append(k, v, seq, pos, pt) == 0
    dev = PagedKV(1, Hkv, Hkv, hd, kv_type, ps, n_pages, device=gpu)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    dev.append(0, t(k), t(v), t(seq), t(pos), t(pt))
    torch.cuda.synchronize()
    assert np.array_equal(dev.k[0].cpu().numpy(), host.k)
    assert np.array_equal(dev.v[0].cpu().numpy(), host.v)


def test_append_skips_missing_page(gpu, oracle_mod):
    import torch
    from strataflow_amd.paged_kv import PagedKV
    dev = PagedKV(1, 2, 2, 32, 1, 32, 2, device=gpu)
    k = torch.ones((2, 2, 32), device=gpu)
    seq = torch.zeros(2, dtype=torch.int32, device=gpu)
    pos = torch.tensor([0, 40], dtype=torch.int32, device=gpu)  # page 1 is -1
    pt = torch.tensor([[1, -1]], dtype=torch.int32, device=gpu)
    dev.append(0, k, k, seq, pos, pt)
    torch.cuda.synchronize()
    assert int(dev.k[0, 0].count_nonzero()) == 0
    # token 0 wrote two rows (2 kv heads) of 32 halves 0x3c00: 64 nonzero bytes
    assert int(dev.k[0, 1].count_nonzero()) == 64
