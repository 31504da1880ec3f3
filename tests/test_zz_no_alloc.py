"""sfa_attn_decode_noalloc (the allocation-free decode entry point) against
sfa_attn_decode with a caller workspace: bit-identical outputs on two calls
in a row, the second with a smaller input, through the C ABI."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tests.helpers import Case, assert_close

pytestmark = pytest.mark.gpu


def _noalloc(c: Case, max_seq_len: int):
    import torch
    from strataflow_amd import _lib
    lib = _lib.load()
    out = torch.full((c.B, c.n_head * c.head_dim), float("nan"), device=c.t_q.device)
    d = c.dev.desc(0)
    rc = lib.sfa_attn_decode_noalloc(ctypes.byref(d), c.t_q.data_ptr(), out.data_ptr(), c.t_pt.data_ptr(),
                                     c.max_pages, c.t_sl.data_ptr(),
                                     None if c.t_lo is None else c.t_lo.data_ptr(), c.B, max_seq_len,
                                     float(c.dev.scale), torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.SFA_OK, _lib.status_str(rc)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("kv_type", [1, 8, 0])
def test_noalloc_matches_workspace_decode(gpu, oracle_mod, kv_type):
    # a long batch first, then a smaller one on the same scratch: the second
    # call must not see the first call's partials
    big = Case(oracle_mod, seq_lens=[4096, 1500, 3000], kv_lo=[0, 200, 0], kv_type=kv_type,
               seed=31 + kv_type)
    small = Case(oracle_mod, seq_lens=[700], kv_type=kv_type, seed=32 + kv_type)
    for c, msl in ((big, 4096), (small, 700)):
        ref = c.decode(max_seq_len=msl)
        got = _noalloc(c, msl)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"type {kv_type} B={c.B}"
        assert_close(got, c.oracle(oracle_mod.GGML), what=f"noalloc type {kv_type} B={c.B} vs ggml")


def test_noalloc_rejects_oversized_shape(gpu, oracle_mod):
    # a batch whose split partials exceed the fixed scratch is refused on the
    # host (nothing is launched)
    import torch
    from strataflow_amd import _lib
    lib = _lib.load()
    c = Case(oracle_mod, seq_lens=[64], seed=33)
    d = c.dev.desc(0)
    B = 4096
    need = lib.sfa_decode_workspace_bytes(ctypes.byref(d), B, 32768)
    assert need > _lib.SFA_NOALLOC_SCRATCH_BYTES
    rc = lib.sfa_attn_decode_noalloc(ctypes.byref(d), c.t_q.data_ptr(), c.t_q.data_ptr(), c.t_pt.data_ptr(),
                                     c.max_pages, c.t_sl.data_ptr(), None, B, 32768, 0.088,
                                     torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.SFA_ERR_OUT_OF_MEMORY
