"""GPU tests of the host page manager (libsfa_host.so) driving libsfa.so.

The reference's paging gate (tests/test_kv_paging.cpp:242-248) is that decoding
with a resident window W smaller than the sequence is bit-identical to the
full-resident cache, that paging really engaged (positions left the window,
cold bytes were written, cold bytes bounded by what was evicted) and that the
result matches the oracle.  Here the same three checks run per decode step
against a full-resident PagedKV holding the same appended K/V under a
different seeded page placement, for lossless paging (evicted pages read in
place from the host-pinned cold pool) and for the opt-in sliding window.
"""
import numpy as np
import pytest
import torch

from strataflow_amd import synth
from strataflow_amd.pager import (SFA_ATTEND_LOSSLESS, SFA_ATTEND_WINDOW, SFA_KV_F16, SFA_KV_F32,
                                  SFA_KV_Q8_0, KvPager)
from strataflow_amd.paged_kv import PagedKV

from .helpers import assert_close

pytestmark = pytest.mark.gpu


class Mirror:
    """A KvPager and a full-resident PagedKV fed the same K/V stream."""

    def __init__(self, *, n_seq, n_ctx, window, attend, kv_type=SFA_KV_F16, n_layer=1, n_head=32,
                 n_head_kv=8, head_dim=128, page_size=256, seed=0, oracle=None):
        self.n_seq, self.n_ctx, self.window, self.attend = n_seq, n_ctx, window, attend
        self.n_layer, self.n_head, self.n_head_kv, self.head_dim = n_layer, n_head, n_head_kv, head_dim
        self.P = page_size
        self.pager = KvPager(n_layer=n_layer, n_head=n_head, n_head_kv=n_head_kv, head_dim=head_dim,
                             kv_type=kv_type, page_size=page_size, n_seq=n_seq, n_ctx=n_ctx,
                             window=window, attend=attend, seed=seed + 11)
        rng = np.random.default_rng(seed)
        max_pages = (n_ctx + page_size - 1) // page_size
        n_pages = n_seq * max_pages + 2
        self.full = PagedKV(n_layer, n_head, n_head_kv, head_dim, kv_type, page_size, n_pages)
        self.pt = torch.from_numpy(synth.page_tables(rng, [n_ctx] * n_seq, page_size, n_pages,
                                                     max_pages)).cuda()
        self.gen = torch.Generator(device="cuda")
        self.gen.manual_seed(seed)
        self.used = np.zeros(n_seq, np.int64)
        self.oracle = oracle  # optional host mirror of layer 0 (HostPagedKv, same table)
        self.host_pt = self.pt.cpu().numpy()

    def _tokens(self, n_tok):
        seq = np.concatenate([np.full(n, b, np.int32) for b, n in enumerate(n_tok)])
        pos = np.concatenate([self.used[b] + np.arange(n, dtype=np.int32) for b, n in enumerate(n_tok)])
        return seq.astype(np.int32), pos.astype(np.int32)

    def step(self, n_tok, with_q=True):
        n_tok = np.asarray(n_tok, np.int32)
        assert self.pager.begin(n_tok) == 0
        seq, pos = self._tokens(n_tok)
        t_seq = torch.from_numpy(seq).cuda()
        t_pos = torch.from_numpy(pos).cuda()
        n = int(n_tok.sum())
        outs = []
        for layer in range(self.n_layer):
            k = torch.randn((n, self.n_head_kv, self.head_dim), generator=self.gen, device="cuda")
            v = torch.randn((n, self.n_head_kv, self.head_dim), generator=self.gen, device="cuda")
            k = synth.rope_normal_torch(k, t_pos, 1e6).contiguous()
            self.pager.append(layer, k, v)
            self.full.append(layer, k, v, t_seq, t_pos, self.pt)
            if layer == 0 and self.oracle is not None:
                assert self.oracle.append(k.cpu().numpy(), v.cpu().numpy(), seq, pos, self.host_pt) == 0
            if with_q:
                q = torch.randn((n, self.n_head, self.head_dim), generator=self.gen, device="cuda")
                q = synth.rope_normal_torch(q, t_pos, 1e6).contiguous()
                outs.append((q, self.pager.attend(layer, q)))
        self.used += n_tok
        return outs

    def fill(self, lens):
        """Appends histories of the given lengths, page_size tokens per step."""
        lens = np.asarray(lens, np.int64)
        while True:
            n_tok = np.minimum(lens - self.used, self.P).clip(min=0).astype(np.int32)
            if not n_tok.any():
                break
            self.step(n_tok, with_q=False)

    def full_decode(self, layer, q):
        seq_len = torch.from_numpy((self.used).astype(np.int32)).cuda()
        if self.attend == SFA_ATTEND_WINDOW:
            lo = torch.from_numpy(np.maximum(self.used - self.window, 0).astype(np.int32)).cuda()
            span = self.window
        else:
            lo, span = None, self.n_ctx
        return self.full.decode(layer, q.view(self.n_seq, self.n_head, self.head_dim), self.pt,
                                seq_len, span, kv_lo=lo)


def _decode_and_compare(m, n_steps, check_every=1):
    for s in range(n_steps):
        outs = m.step(np.ones(m.n_seq, np.int32))
        if s % check_every and s != n_steps - 1:
            continue
        for layer, (q, out) in enumerate(outs):
            ref = m.full_decode(layer, q)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"step {s} layer {layer}: paged != full-resident"
    return outs


@pytest.mark.parametrize("kv_type", [SFA_KV_F32, SFA_KV_F16, SFA_KV_Q8_0])
def test_pager_lossless_bit_identical(gpu, oracle_mod, kv_type):
    # 4 sequences of different lengths, window of 4 pages, ragged first fill
    host = oracle_mod.HostPagedKv(8, 128, 256, kv_type, 4 * 32 + 2)
    m = Mirror(n_seq=4, n_ctx=8192, window=1024, attend=SFA_ATTEND_LOSSLESS, kv_type=kv_type,
               n_layer=2, seed=1, oracle=host)
    m.fill([3000, 2500, 4000, 1100])
    outs = _decode_and_compare(m, 300, check_every=7)
    st = m.pager.stats()
    # paging engaged: pages left the window and the cold pool holds exactly them
    lens = m.used
    evicted_pages = sum(max(0, (int(n) - 1024) // 256) for n in lens)
    assert st["pages_evicted"] == evicted_pages > 0
    assert st["cold_pages_in_use"] == evicted_pages
    assert st["pages_dropped"] == 0
    row = {SFA_KV_F32: 512, SFA_KV_F16: 256, SFA_KV_Q8_0: 136}[kv_type]
    assert st["bytes_evicted"] == evicted_pages * 2 * 2 * 256 * 8 * row
    assert st["dev_pages_in_use"] <= 4 * 5
    pt, used = m.pager.tables()
    # pages whose copy was not yet seen complete still name their device page
    assert (used == lens).all() and (pt <= -2).sum() + st["pages_in_flight"] == evicted_pages
    # and the paged result is the reference attention over every position
    q, out = outs[0]
    ref = host.attention(q.cpu().numpy(), 32, m.host_pt, lens.astype(np.int32), None,
                         mode=oracle_mod.GGML).reshape(4, -1)
    assert_close(out.cpu().numpy(), ref, what="lossless paged vs oracle")


def test_pager_window_matches_oracle(gpu, oracle_mod):
    host = oracle_mod.HostPagedKv(8, 128, 256, SFA_KV_F16, 4 * 24 + 2)
    m = Mirror(n_seq=4, n_ctx=6144, window=1000, attend=SFA_ATTEND_WINDOW, n_layer=1, seed=2,
               oracle=host)
    m.fill([1500, 3000, 999, 4100])
    outs = _decode_and_compare(m, 260, check_every=5)
    st = m.pager.stats()
    assert st["pages_dropped"] > 0 and st["pages_evicted"] == 0 and st["cold_pages_in_use"] == 0
    pt, _ = m.pager.tables()
    assert (pt <= -2).sum() == 0
    q, out = outs[0]
    lo = np.maximum(m.used - 1000, 0).astype(np.int32)
    ref = host.attention(q.cpu().numpy(), 32, m.host_pt, m.used.astype(np.int32), lo,
                         mode=oracle_mod.GGML).reshape(4, -1)
    assert_close(out.cpu().numpy(), ref, what="window paged vs oracle")


@pytest.mark.parametrize("kv_type", [SFA_KV_F32, SFA_KV_F16, SFA_KV_Q8_0])
def test_pager_prefill_chunk_over_cold_pages(gpu, oracle_mod, kv_type):
    # a 200-token chunk whose history is partly in the cold pool
    host = oracle_mod.HostPagedKv(8, 128, 256, kv_type, 2 * 16 + 2)
    m = Mirror(n_seq=2, n_ctx=4096, window=512, attend=SFA_ATTEND_LOSSLESS, seed=3, oracle=host,
               kv_type=kv_type)
    m.fill([1800, 700])
    pos0 = m.used.copy()
    outs = m.step(np.array([200, 0], np.int32))
    q, out = outs[0]
    assert m.pager.stats()["pages_evicted"] > 0
    assert m.used[0] == pos0[0] + 200
    # query t sits at position seq_len - 200 + t
    ref = host.attention(q.cpu().numpy()[None], 32, m.host_pt[:1], m.used[:1].astype(np.int32),
                         None, T=200, mode=oracle_mod.GGML)
    assert_close(out.cpu().numpy(), ref.reshape(200, -1), what="prefill over cold pages")


def test_pager_out_of_pages_and_reset(gpu):
    p = KvPager(n_layer=1, n_head=32, n_head_kv=8, head_dim=128, kv_type=SFA_KV_F16, page_size=256,
                n_seq=2, n_ctx=4096, window=512, attend=SFA_ATTEND_WINDOW, n_pages=4, seed=0)
    assert p.begin(np.array([256, 256], np.int32)) == 0
    assert p.begin(np.array([256, 256], np.int32)) == 0   # pool full (2 pages each)
    before = p.tables()
    assert p.begin(np.array([1, 0], np.int32)) == 4       # needs a fifth page
    after = p.tables()
    assert (before[0] == after[0]).all() and (before[1] == after[1]).all()
    p.reset(1)
    assert p.begin(np.array([1, 0], np.int32)) == 0
    pt, used = p.tables()
    assert used.tolist() == [513, 0] and (pt[1] == -1).all()
    p.close()


@pytest.mark.parametrize("attend", [SFA_ATTEND_WINDOW, SFA_ATTEND_LOSSLESS])
def test_pager_window_4096_history_65536(gpu, attend):
    # the KV-window workload: 4 sequences, 65536-token histories, W = 4096,
    # device pool sized to the window (4 * 17 pages), then 128 decode steps
    # (two layers); paged == full-resident bit for bit (test_kv_paging.cpp:242-248)
    steps = 128
    m = Mirror(n_seq=4, n_ctx=65536 + 256, window=4096, attend=attend, n_layer=2, seed=4)
    m.fill([65536 - 37, 65536 - 300, 65536 - 1, 65536 - 129])
    _decode_and_compare(m, steps, check_every=16)
    st = m.pager.stats()
    assert st["dev_pages_in_use"] <= 4 * 17
    if attend == SFA_ATTEND_LOSSLESS:
        assert st["cold_pages_in_use"] == st["pages_evicted"] > 4 * 230
    else:
        assert st["pages_dropped"] > 4 * 230 and st["cold_pages_in_use"] == 0


def test_pager_rope_append_matches_full(gpu):
    """sfa_pager_rope_append (pre-RoPE Q and K) against the full-resident cache
    fed through sfa_rope_kv_append: the rotated Q rows and the attention
    outputs are bit-identical while pages leave the window."""
    n_seq, n_ctx, window, P, Hq, Hkv, hd = 2, 2048, 512, 256, 32, 8, 128
    pager = KvPager(n_layer=1, n_head=Hq, n_head_kv=Hkv, head_dim=hd, kv_type=SFA_KV_F16,
                    page_size=P, n_seq=n_seq, n_ctx=n_ctx, window=window,
                    attend=SFA_ATTEND_LOSSLESS, seed=5)
    rng = np.random.default_rng(5)
    max_pages = n_ctx // P
    n_pages = n_seq * max_pages + 2
    full = PagedKV(1, Hq, Hkv, hd, SFA_KV_F16, P, n_pages)
    pt = torch.from_numpy(synth.page_tables(rng, [n_ctx] * n_seq, P, n_pages, max_pages)).cuda()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    used = np.zeros(n_seq, np.int64)
    for step in range(12):
        n_tok = np.array([P, P // 2], np.int32) if step < 5 else np.ones(n_seq, np.int32)
        assert pager.begin(n_tok) == 0
        seq = np.concatenate([np.full(n, b, np.int32) for b, n in enumerate(n_tok)])
        pos = np.concatenate([used[b] + np.arange(n) for b, n in enumerate(n_tok)]).astype(np.int32)
        n = int(n_tok.sum())
        k = torch.randn((n, Hkv, hd), generator=gen, device="cuda")
        v = torch.randn((n, Hkv, hd), generator=gen, device="cuda")
        q = torch.randn((n, Hq, hd), generator=gen, device="cuda")
        q_pager, q_full = q.clone(), q.clone()
        pager.rope_append(0, q_pager, k, v, 1e6)
        full.rope_append(0, q_full, k, v, torch.from_numpy(seq).cuda(), torch.from_numpy(pos).cuda(), pt, 1e6)
        used += n_tok
        assert torch.equal(q_pager, q_full)
        if step >= 5:
            out = pager.attend(0, q_pager)
            ref = full.decode(0, q_full.view(n_seq, Hq, hd), pt, torch.from_numpy(used.astype(np.int32)).cuda(),
                              n_ctx)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"step {step}: paged != full-resident"
    assert pager.stats()["pages_evicted"] > 0


def test_pager_deferred_eviction_serves_pages_in_flight(gpu):
    # an evicted page keeps serving reads from HBM until its copy is seen
    # complete; a pool with no spare page retires in-flight pages at once
    # (the stream waits for the copy); both stay bit-identical to full residency
    for n_pages, seed in ((0, 21), (4 * 5 + 6, 22)):  # the default (tight) pool, then 6 spare pages
        m = Mirror(n_seq=4, n_ctx=4096, window=1024, attend=SFA_ATTEND_LOSSLESS, n_layer=2, seed=seed)
        if n_pages:
            m.pager.close()
            m.pager = KvPager(n_layer=2, n_head=32, n_head_kv=8, head_dim=128, kv_type=SFA_KV_F16,
                              page_size=256, n_seq=4, n_ctx=4096, window=1024,
                              attend=SFA_ATTEND_LOSSLESS, n_pages=n_pages, seed=seed)
        m.fill([1200, 1279, 1500, 1023])
        seen_in_flight = 0
        for s in range(300):
            outs = m.step(np.ones(4, np.int32))
            st = m.pager.stats()
            pt, used = m.pager.tables()
            assert (pt <= -2).sum() + st["pages_in_flight"] == st["pages_evicted"]
            seen_in_flight = max(seen_in_flight, st["pages_in_flight"])
            if s % 13 == 0 or s == 299:
                for layer, (q, out) in enumerate(outs):
                    ref = m.full_decode(layer, q)
                    torch.cuda.synchronize()
                    assert torch.equal(out, ref), f"pool {n_pages} step {s} layer {layer}"
        assert st["pages_evicted"] > 0 and seen_in_flight > 0
        m.pager.close()


def test_pager_page_size_64(gpu, oracle_mod):
    # 64-position pages (the smallest the pager takes): decode steps and a
    # multi-token step (the chunked prefill, one 64-position tile per page)
    # against the oracle
    host = oracle_mod.HostPagedKv(8, 128, 64, SFA_KV_F16, 2 * 32 + 2)
    m = Mirror(n_seq=2, n_ctx=2048, window=300, attend=SFA_ATTEND_LOSSLESS, page_size=64, seed=23,
               oracle=host)
    m.fill([500, 333])
    outs = _decode_and_compare(m, 40, check_every=9)
    q, out = outs[0]
    ref = host.attention(q.cpu().numpy(), 32, m.host_pt, m.used.astype(np.int32), None,
                         mode=oracle_mod.GGML).reshape(2, -1)
    assert_close(out.cpu().numpy(), ref, what="page size 64 vs oracle")


def test_pager_window_idle_sequence(gpu, oracle_mod):
    # sliding window with an idle sequence in the step: the active ones attend
    # their own window (one token each, through the causal prefill)
    host = oracle_mod.HostPagedKv(8, 128, 256, SFA_KV_F16, 3 * 16 + 2)
    m = Mirror(n_seq=3, n_ctx=4096, window=700, attend=SFA_ATTEND_WINDOW, seed=24, oracle=host)
    m.fill([1500, 900, 2000])
    for s in range(5):
        n_tok = np.array([1, 0, 1] if s % 2 == 0 else [0, 1, 1], np.int32)
        outs = m.step(n_tok)
        q, out = outs[0]
        act = np.nonzero(n_tok)[0]
        used = m.used.astype(np.int32)
        lo = np.maximum(used - 700, 0).astype(np.int32)
        qa = q.cpu().numpy()
        ref = host.attention(qa, 32, m.host_pt[act], used[act], lo[act],
                             mode=oracle_mod.GGML).reshape(len(act), -1)
        assert_close(out.cpu().numpy(), ref, what=f"idle step {s}")
