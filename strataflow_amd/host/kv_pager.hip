// kv_pager.hip - host-side paged KV manager over libsfa.so (sfa_pager.h).
//
// Owns the device pool of every layer's K and V pages, the host-pinned cold
// pool and the device page tables; PagePlanner decides residency and this file
// carries its decisions out: eviction copies (one strided device-to-host copy
// moves a page of every layer, K and V) run on a copy stream of the pager's
// own, after an event marking the caller's stream at the step's start, so the
// step's attention and appends do not wait for them.  An evicted page keeps
// serving reads from HBM until its copy is seen complete (an event query at a
// later step); then its table slot moves to the cold page and the device page
// is reused.  Only an allocation that finds no other free page makes the
// caller's stream wait for a copy.  One small kernel per step applies the
// page-table edits and writes seq_len, kv_lo and the step's (seq, pos) token
// arrays.  Step metadata travels as kernel arguments, so a step needs no host
// staging buffer and no synchronisation.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <deque>
#include <map>
#include <new>
#include <utility>
#include <vector>

#include "page_planner.h"
#include "sfa.h"
#include "sfa_pager.h"

namespace {

constexpr int kUpdSeqs = 32;    // sequences per update launch
constexpr int kUpdEdits = 128;  // page-table edits per update launch

struct StepArgs {
    int32_t *table;
    int32_t *seq_len;
    int32_t *kv_lo;
    int32_t *tok_seq;
    int32_t *tok_pos;
    int32_t n_seq;
    int32_t n_edit;
    int32_t seq[kUpdSeqs];
    int32_t tok_off[kUpdSeqs];
    int32_t pos0[kUpdSeqs];
    int32_t n_tok[kUpdSeqs];
    int32_t len[kUpdSeqs];
    int32_t lo[kUpdSeqs];
    int32_t edit_idx[kUpdEdits];
    int32_t edit_val[kUpdEdits];
};

__global__ __launch_bounds__(256) void step_update_kernel(StepArgs a) {
    const int t = threadIdx.x;
    for (int i = t; i < a.n_edit; i += blockDim.x) a.table[a.edit_idx[i]] = a.edit_val[i];
    for (int s = 0; s < a.n_seq; ++s) {
        if (t == 0) {
            a.seq_len[a.seq[s]] = a.len[s];
            a.kv_lo[a.seq[s]] = a.lo[s];
        }
        for (int i = t; i < a.n_tok[s]; i += blockDim.x) {
            a.tok_seq[a.tok_off[s] + i] = a.seq[s];
            a.tok_pos[a.tok_off[s] + i] = a.pos0[s] + i;
        }
    }
}

inline hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

}  // namespace

struct sfa_pager {
    sfa_pager_config cfg{};
    sfa::PagePlanner planner;
    size_t page_bytes = 0;
    int max_pages = 0;
    int32_t max_span = 0;
    uint8_t *dev_pool = nullptr;   // [layer][K|V][n_pages][page_bytes]
    uint8_t *cold_pool = nullptr;  // [layer][K|V][n_cold][page_bytes], host-pinned
    int32_t *d_table = nullptr;    // [n_seq][max_pages]
    int32_t *d_seq_len = nullptr;  // [n_seq]
    int32_t *d_kv_lo = nullptr;    // [n_seq]
    int32_t *d_tok_seq = nullptr;  // [n_seq * page_size]
    int32_t *d_tok_pos = nullptr;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    std::vector<sfa_kv_desc> descs;
    // deferred eviction: copies on copy_stream; one event per eviction in
    // flight, in eviction order (the planner's in-flight order)
    hipStream_t copy_stream = nullptr;
    hipEvent_t step_ready = nullptr;
    std::deque<std::pair<uint64_t, hipEvent_t>> ev_flight;
    std::vector<hipEvent_t> ev_free;
    // the current step
    std::vector<int32_t> step_ntok, step_pos0, step_off;
    int32_t step_tokens = 0;
    bool step_open = false;
    int64_t bytes_evicted = 0;

    sfa_pager(const sfa_pager_config &c, int n_pages, int n_cold)
        : cfg(c),
          planner(c.n_seq, c.page_size, (uint32_t)c.n_ctx, (uint32_t)c.window, n_pages, n_cold,
                  c.attend == SFA_ATTEND_LOSSLESS, c.seed, /*async_evict=*/true) {}

    ~sfa_pager() {
        for (auto &e : ev_flight) (void)hipEventDestroy(e.second);
        for (hipEvent_t e : ev_free) (void)hipEventDestroy(e);
        if (step_ready) (void)hipEventDestroy(step_ready);
        if (copy_stream) (void)hipStreamDestroy(copy_stream);
        if (dev_pool) (void)hipFree(dev_pool);
        if (cold_pool) (void)hipHostFree(cold_pool);
        for (int32_t *p : {d_table, d_seq_len, d_kv_lo, d_tok_seq, d_tok_pos})
            if (p) (void)hipFree(p);
        if (ws) (void)hipFree(ws);
    }

    int n_pages() const { return cfg.n_pages; }
    int n_cold() const { return cfg.n_cold_pages; }

    int launch_updates(const std::vector<std::pair<int32_t, int32_t>> &edits, hipStream_t s) {
        const int n_seq = cfg.n_seq;
        size_t e = 0;
        int b = 0;
        do {
            StepArgs a{};
            a.table = d_table;
            a.seq_len = d_seq_len;
            a.kv_lo = d_kv_lo;
            a.tok_seq = d_tok_seq;
            a.tok_pos = d_tok_pos;
            for (; a.n_seq < kUpdSeqs && b < n_seq; ++b, ++a.n_seq) {
                const int i = a.n_seq;
                a.seq[i] = b;
                a.tok_off[i] = step_off[b];
                a.pos0[i] = step_pos0[b];
                a.n_tok[i] = step_ntok[b];
                a.len[i] = (int32_t)planner.store(b).used();
                a.lo[i] = (int32_t)planner.attend_lo(b);
            }
            for (; a.n_edit < kUpdEdits && e < edits.size(); ++e, ++a.n_edit) {
                a.edit_idx[a.n_edit] = edits[e].first;
                a.edit_val[a.n_edit] = edits[e].second;
            }
            hipLaunchKernelGGL(step_update_kernel, dim3(1), dim3(256), 0, s, a);
            if (hipGetLastError() != hipSuccess) return SFA_ERR_RUNTIME;
        } while (b < n_seq || e < edits.size());
        return SFA_OK;
    }

    // Evictions whose copies have completed, counted from the oldest (the
    // planner retires in the same order); -1 on a runtime error.
    int completed_evictions() const {
        int done = 0;
        for (const auto &e : ev_flight) {
            const hipError_t q = hipEventQuery(e.second);
            if (q == hipErrorNotReady) break;
            if (q != hipSuccess) return -1;
            ++done;
        }
        return done;
    }

    // Carries out a step's actions on stream s (copies on copy_stream).  The
    // event bookkeeping changes only when every call succeeded.
    int apply(const std::vector<sfa::PageAction> &actions, hipStream_t s) {
        const size_t slab = (size_t)2 * cfg.n_layer;  // (layer, K|V) rows of a page
        std::map<int32_t, int32_t> edits;              // table slot -> final id
        std::deque<std::pair<uint64_t, hipEvent_t>> flight = ev_flight;
        std::vector<hipEvent_t> spare = ev_free, created, released;
        bool marked = false;
        int64_t copied = 0;
        auto fail = [&](int rc) {
            for (hipEvent_t e : created) (void)hipEventDestroy(e);
            return rc;
        };
        for (const sfa::PageAction &a : actions) {
            if (a.kind == sfa::PageAction::kEvict) {
                // the copy follows everything issued on s so far (the page's
                // writes included): s marks the step, copy_stream waits for it
                if (!marked) {
                    if (hipEventRecord(step_ready, s) != hipSuccess ||
                        hipStreamWaitEvent(copy_stream, step_ready, 0) != hipSuccess)
                        return fail(SFA_ERR_RUNTIME);
                    marked = true;
                }
                // page `dev` of every (layer, K|V) pool -> cold page `cold`
                if (hipMemcpy2DAsync(cold_pool + (size_t)a.cold * page_bytes,
                                     (size_t)n_cold() * page_bytes,
                                     dev_pool + (size_t)a.dev * page_bytes,
                                     (size_t)n_pages() * page_bytes, page_bytes, slab,
                                     hipMemcpyDeviceToHost, copy_stream) != hipSuccess)
                    return fail(SFA_ERR_RUNTIME);
                hipEvent_t ev = nullptr;
                if (!spare.empty()) {
                    ev = spare.back();
                    spare.pop_back();
                } else {
                    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess)
                        return fail(SFA_ERR_RUNTIME);
                    created.push_back(ev);
                }
                if (hipEventRecord(ev, copy_stream) != hipSuccess) return fail(SFA_ERR_RUNTIME);
                flight.emplace_back(a.evict, ev);
                copied += (int64_t)(page_bytes * slab);
            } else if (a.kind == sfa::PageAction::kRetire) {
                // retirements pop the oldest eviction in flight
                if (flight.empty() || flight.front().first != a.evict) return fail(SFA_ERR_RUNTIME);
                if (a.wait && hipStreamWaitEvent(s, flight.front().second, 0) != hipSuccess)
                    return fail(SFA_ERR_RUNTIME);
                released.push_back(flight.front().second);
                flight.pop_front();
            }
            if (a.edit) {
                const int32_t slot = a.seq * max_pages + a.lpage;
                edits[slot] = planner.table()[slot];
            }
        }
        std::vector<std::pair<int32_t, int32_t>> list(edits.begin(), edits.end());
        if (const int rc = launch_updates(list, s); rc != SFA_OK) return fail(rc);
        // commit: an event released here may be re-recorded later, after the
        // waits already enqueued on it
        spare.insert(spare.end(), released.begin(), released.end());
        ev_flight.swap(flight);
        ev_free.swap(spare);
        bytes_evicted += copied;
        return SFA_OK;
    }
};

extern "C" {

SFA_API int sfa_pager_create(const sfa_pager_config *cfg_in, sfa_pager **out) {
    if (cfg_in == nullptr || out == nullptr) return SFA_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    sfa_pager_config c = *cfg_in;
    if (c.n_layer <= 0 || c.n_seq <= 0 || c.n_ctx <= 0 || c.page_size <= 0 || c.window < 0)
        return SFA_ERR_INVALID_ARGUMENT;
    // a multi-token step is attended by the chunked prefill, whose 64-position
    // tiles must not straddle a page: refused here, before any step is begun
    if (c.page_size % 64 != 0) return SFA_ERR_UNSUPPORTED;
    if (c.attend != SFA_ATTEND_LOSSLESS && c.attend != SFA_ATTEND_WINDOW)
        return SFA_ERR_INVALID_ARGUMENT;
    if (c.window == 0 || c.window > c.n_ctx) c.window = c.n_ctx;
    const int max_pages = (c.n_ctx + c.page_size - 1) / c.page_size;
    const int win_pages = (c.window + c.page_size - 1) / c.page_size + 1;
    if (c.n_pages <= 0) c.n_pages = c.n_seq * std::min(win_pages, max_pages);
    const bool paging = c.window < c.n_ctx;
    if (c.attend == SFA_ATTEND_LOSSLESS && paging) {
        if (c.n_cold_pages <= 0) c.n_cold_pages = c.n_seq * max_pages;
    } else {
        c.n_cold_pages = 0;
    }

    sfa_kv_desc d{};
    d.n_head = c.n_head;
    d.n_head_kv = c.n_head_kv;
    d.head_dim = c.head_dim;
    d.page_size = c.page_size;
    d.kv_type = c.kv_type;
    if (int rc = sfa_kv_desc_check(&d); rc != SFA_OK) return rc;  // shapes (no pools yet)
    d.n_pages = c.n_pages;

    sfa_pager *p = nullptr;
    try {
        p = new sfa_pager(c, c.n_pages, c.n_cold_pages);
        p->page_bytes = sfa_page_bytes(&d);
        p->max_pages = max_pages;
        p->max_span = c.attend == SFA_ATTEND_WINDOW ? c.window : c.n_ctx;
        p->step_ntok.assign(c.n_seq, 0);
        p->step_pos0.assign(c.n_seq, 0);
        p->step_off.assign(c.n_seq, 0);
    } catch (const std::bad_alloc &) {
        delete p;
        return SFA_ERR_OUT_OF_MEMORY;
    }
    auto fail = [&](int rc) {
        delete p;
        return rc;
    };
    const size_t slab = (size_t)2 * c.n_layer;
    if (hipMalloc(&p->dev_pool, slab * c.n_pages * p->page_bytes) != hipSuccess)
        return fail(SFA_ERR_OUT_OF_MEMORY);
    if (c.n_cold_pages > 0 &&
        hipHostMalloc(reinterpret_cast<void **>(&p->cold_pool), slab * c.n_cold_pages * p->page_bytes,
                      hipHostMallocDefault) != hipSuccess)
        return fail(SFA_ERR_OUT_OF_MEMORY);
    const size_t n_table = (size_t)c.n_seq * max_pages;
    const size_t n_tok = (size_t)c.n_seq * c.page_size;
    if (hipMalloc(&p->d_table, n_table * 4) != hipSuccess ||
        hipMalloc(&p->d_seq_len, (size_t)c.n_seq * 4) != hipSuccess ||
        hipMalloc(&p->d_kv_lo, (size_t)c.n_seq * 4) != hipSuccess ||
        hipMalloc(&p->d_tok_seq, n_tok * 4) != hipSuccess ||
        hipMalloc(&p->d_tok_pos, n_tok * 4) != hipSuccess)
        return fail(SFA_ERR_OUT_OF_MEMORY);
    // empty tables (-1), zero lengths; the pools need no initial contents
    if (hipMemset(p->d_table, 0xFF, n_table * 4) != hipSuccess ||
        hipMemset(p->d_seq_len, 0, (size_t)c.n_seq * 4) != hipSuccess ||
        hipMemset(p->d_kv_lo, 0, (size_t)c.n_seq * 4) != hipSuccess)
        return fail(SFA_ERR_RUNTIME);

    p->descs.resize(c.n_layer);
    for (int l = 0; l < c.n_layer; ++l) {
        sfa_kv_desc &L = p->descs[l];
        L = d;
        L.k_pages = p->dev_pool + (size_t)(2 * l) * c.n_pages * p->page_bytes;
        L.v_pages = p->dev_pool + (size_t)(2 * l + 1) * c.n_pages * p->page_bytes;
        L.n_cold_pages = c.n_cold_pages;
        if (c.n_cold_pages > 0) {
            L.k_cold = p->cold_pool + (size_t)(2 * l) * c.n_cold_pages * p->page_bytes;
            L.v_cold = p->cold_pool + (size_t)(2 * l + 1) * c.n_cold_pages * p->page_bytes;
        }
    }
    p->ws_bytes = sfa_decode_workspace_bytes(&p->descs[0], c.n_seq, p->max_span);
    if (p->ws_bytes == 0) return fail(SFA_ERR_INVALID_ARGUMENT);
    if (hipMalloc(&p->ws, p->ws_bytes) != hipSuccess) return fail(SFA_ERR_OUT_OF_MEMORY);
    // default-priority copy stream and the step marker of deferred eviction
    if (hipStreamCreateWithFlags(&p->copy_stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&p->step_ready, hipEventDisableTiming) != hipSuccess)
        return fail(SFA_ERR_RUNTIME);
    if (sfa_workspace_init(p->ws, p->ws_bytes, nullptr) != SFA_OK) return fail(SFA_ERR_RUNTIME);
    if (hipDeviceSynchronize() != hipSuccess) return fail(SFA_ERR_RUNTIME);
    *out = p;
    return SFA_OK;
}

SFA_API void sfa_pager_destroy(sfa_pager *p) {
    if (p == nullptr) return;
    (void)hipDeviceSynchronize();  // no copy or kernel may still use the pools
    delete p;
}

SFA_API int sfa_pager_begin(sfa_pager *p, const int32_t *n_tok, void *stream) {
    if (p == nullptr || n_tok == nullptr) return SFA_ERR_INVALID_ARGUMENT;
    const int n_seq = p->cfg.n_seq;
    for (int b = 0; b < n_seq; ++b)
        if (n_tok[b] < 0 || n_tok[b] > p->cfg.page_size) return SFA_ERR_INVALID_ARGUMENT;
    const int done = p->completed_evictions();
    if (done < 0) return SFA_ERR_RUNTIME;
    try {
        // everything below is undone on any error: the planner is restored
        // from this copy and the step metadata is committed last
        sfa::PagePlanner saved = p->planner;
        std::vector<int32_t> pos0(n_seq), off(n_seq);
        int32_t total = 0;
        for (int b = 0; b < n_seq; ++b) {
            pos0[b] = (int32_t)p->planner.store(b).used();
            off[b] = total;
            total += n_tok[b];
        }
        std::vector<sfa::PageAction> actions;
        int rc = SFA_OK;
        try {
            p->planner.retire_completed(done, &actions);
        } catch (const std::bad_alloc &) {
            rc = SFA_ERR_OUT_OF_MEMORY;
        }
        if (rc == SFA_OK) rc = p->planner.plan_step(n_tok, &actions);
        if (rc == SFA_OK) {
            // apply() reads the step metadata for the update kernel
            std::vector<int32_t> old_ntok(n_tok, n_tok + n_seq);
            p->step_ntok.swap(old_ntok);
            p->step_pos0.swap(pos0);
            p->step_off.swap(off);
            rc = p->apply(actions, as_stream(stream));
            if (rc != SFA_OK) {
                p->step_ntok.swap(old_ntok);
                p->step_pos0.swap(pos0);
                p->step_off.swap(off);
            }
        }
        if (rc != SFA_OK) {
            p->planner = std::move(saved);
            p->step_open = false;
            return rc;
        }
        p->step_tokens = total;
        p->step_open = true;
        return SFA_OK;
    } catch (const std::bad_alloc &) {  // no exception leaves the C ABI
        return SFA_ERR_OUT_OF_MEMORY;
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API int sfa_pager_append(sfa_pager *p, int32_t layer, const float *k, const float *v,
                             void *stream) {
    if (p == nullptr || !p->step_open || layer < 0 || layer >= p->cfg.n_layer)
        return SFA_ERR_INVALID_ARGUMENT;
    if (p->step_tokens == 0) return SFA_OK;
    return sfa_kv_append(&p->descs[layer], k, v, p->d_tok_seq, p->d_tok_pos, p->step_tokens,
                         p->d_table, p->max_pages, stream);
}

SFA_API int sfa_pager_rope_append(sfa_pager *p, int32_t layer, float *q, const float *k,
                                  const float *v, float freq_base, void *stream) {
    if (p == nullptr || !p->step_open || layer < 0 || layer >= p->cfg.n_layer)
        return SFA_ERR_INVALID_ARGUMENT;
    if (p->step_tokens == 0) return SFA_OK;
    return sfa_rope_kv_append(&p->descs[layer], q, k, v, p->d_tok_seq, p->d_tok_pos, p->step_tokens,
                              p->d_table, p->max_pages, freq_base, stream);
}

SFA_API int sfa_pager_attend(sfa_pager *p, int32_t layer, const float *q, float *out,
                             void *stream) {
    if (p == nullptr || !p->step_open || layer < 0 || layer >= p->cfg.n_layer)
        return SFA_ERR_INVALID_ARGUMENT;
    const sfa_kv_desc *d = &p->descs[layer];
    const float scale = 1.0f / std::sqrt((float)p->cfg.head_dim);
    const bool windowed = p->cfg.attend == SFA_ATTEND_WINDOW;
    const bool one_each = std::all_of(p->step_ntok.begin(), p->step_ntok.end(),
                                      [](int32_t n) { return n == 1; });
    if (one_each)
        return sfa_attn_decode(d, q, out, p->d_table, p->max_pages, p->d_seq_len,
                               windowed ? p->d_kv_lo : nullptr, p->cfg.n_seq, p->max_span, scale,
                               p->ws, p->ws_bytes, stream);
    // a chunk (or a batch with idle sequences): the causal prefill per active
    // sequence.  Under the sliding window one token attends [attend_lo, pos];
    // the tokens of a longer chunk would each need their own window start.
    const size_t row = (size_t)p->cfg.n_head * p->cfg.head_dim;
    for (int b = 0; b < p->cfg.n_seq; ++b)
        if (windowed && p->step_ntok[b] > 1) return SFA_ERR_UNSUPPORTED;
    for (int b = 0; b < p->cfg.n_seq; ++b) {
        if (p->step_ntok[b] == 0) continue;
        const size_t off = (size_t)p->step_off[b] * row;
        const int32_t lo = windowed ? (int32_t)p->planner.attend_lo(b) : 0;
        const int rc = sfa_attn_prefill(d, q + off, out + off, p->d_table + (size_t)b * p->max_pages,
                                        p->max_pages, p->step_pos0[b], p->step_ntok[b], lo, scale,
                                        stream);
        if (rc != SFA_OK) return rc;
    }
    return SFA_OK;
}

SFA_API int sfa_pager_append_attend(sfa_pager *p, int32_t layer, const float *k, const float *v,
                                    const float *q, float *out, void *stream) {
    if (p == nullptr || !p->step_open || layer < 0 || layer >= p->cfg.n_layer)
        return SFA_ERR_INVALID_ARGUMENT;
    const bool one_each = std::all_of(p->step_ntok.begin(), p->step_ntok.end(),
                                      [](int32_t n) { return n == 1; });
    if (!one_each || p->cfg.kv_type == SFA_KV_Q8_0) {
        const int rc = sfa_pager_append(p, layer, k, v, stream);
        return rc != SFA_OK ? rc : sfa_pager_attend(p, layer, q, out, stream);
    }
    // one token per sequence, token b of sequence b at position seq_len[b] - 1
    const sfa_kv_desc *d = &p->descs[layer];
    const float scale = 1.0f / std::sqrt((float)p->cfg.head_dim);
    const bool windowed = p->cfg.attend == SFA_ATTEND_WINDOW;
    return sfa_attn_decode_append(d, k, v, q, out, p->d_table, p->max_pages, p->d_seq_len,
                                  windowed ? p->d_kv_lo : nullptr, p->cfg.n_seq, p->max_span, scale,
                                  p->ws, p->ws_bytes, stream);
}

SFA_API int sfa_pager_reset(sfa_pager *p, int32_t seq, void *stream) {
    if (p == nullptr || seq < 0 || seq >= p->cfg.n_seq) return SFA_ERR_INVALID_ARGUMENT;
    std::vector<sfa::PageAction> actions;
    try {
        p->planner.reset(seq, &actions);
    } catch (const std::bad_alloc &) {
        return SFA_ERR_OUT_OF_MEMORY;
    }
    std::fill(p->step_ntok.begin(), p->step_ntok.end(), 0);
    for (int b = 0; b < p->cfg.n_seq; ++b) p->step_pos0[b] = (int32_t)p->planner.store(b).used();
    p->step_tokens = 0;
    p->step_open = false;
    // the table slots of the released pages go back to -1
    try {
        std::vector<std::pair<int32_t, int32_t>> edits;
        for (int lp = 0; lp < p->max_pages; ++lp) edits.emplace_back(seq * p->max_pages + lp, -1);
        return p->launch_updates(edits, as_stream(stream));
    } catch (const std::bad_alloc &) {  // no exception leaves the C ABI
        return SFA_ERR_OUT_OF_MEMORY;
    }
}

SFA_API int sfa_pager_stats_get(const sfa_pager *p, sfa_pager_stats *out) {
    if (p == nullptr || out == nullptr) return SFA_ERR_INVALID_ARGUMENT;
    const sfa::PlannerStats &s = p->planner.stats();
    out->pages_allocated = s.allocated;
    out->pages_evicted = s.evicted;
    out->pages_dropped = s.dropped;
    out->dev_pages_in_use = s.dev_in_use;
    out->cold_pages_in_use = s.cold_in_use;
    out->bytes_evicted = p->bytes_evicted;
    out->pages_in_flight = s.in_flight;
    return SFA_OK;
}

SFA_API int sfa_pager_desc(const sfa_pager *p, int32_t layer, sfa_kv_desc *out) {
    if (p == nullptr || out == nullptr || layer < 0 || layer >= p->cfg.n_layer)
        return SFA_ERR_INVALID_ARGUMENT;
    *out = p->descs[layer];
    return SFA_OK;
}

SFA_API int32_t sfa_pager_max_pages(const sfa_pager *p) { return p ? p->max_pages : 0; }

SFA_API int sfa_pager_device_tables(const sfa_pager *p, const int32_t **page_table,
                                    const int32_t **seq_len, const int32_t **kv_lo) {
    if (p == nullptr) return SFA_ERR_INVALID_ARGUMENT;
    if (page_table) *page_table = p->d_table;
    if (seq_len) *seq_len = p->d_seq_len;
    if (kv_lo) *kv_lo = p->d_kv_lo;
    return SFA_OK;
}

SFA_API int sfa_pager_tables(const sfa_pager *p, int32_t *page_table, int32_t *used) {
    if (p == nullptr) return SFA_ERR_INVALID_ARGUMENT;
    if (page_table) std::copy(p->planner.table().begin(), p->planner.table().end(), page_table);
    if (used)
        for (int b = 0; b < p->cfg.n_seq; ++b) used[b] = (int32_t)p->planner.store(b).used();
    return SFA_OK;
}

}  // extern "C"
