/*
 * sfa_pager.h - C ABI of the host-side paged KV manager (libsfa_host.so).
 *
 * This is the engine side of the attention node: the KV ownership and lossless
 * window paging that the reference keeps in Engine::Impl and KvStore, driving
 * libsfa.so (sfa.h) for the device work.
 *
 *   KV ownership   : per-layer K/V caches owned for the engine's lifetime
 *                    (src/model/engine/engine.cpp:1253-1286, freed in ~Impl :521-522)
 *   window paging  : KvStore (src/kv/kv_store.h:30-95) bounds residency to W
 *                    positions; before a write pushes a position out of the
 *                    window its bytes go to a RAM cold store (engine.cpp:2620-2661)
 *                    and attention still covers 0..pos (engine.cpp:1669-1749).
 *
 * Here residency is per page: a sequence keeps the pages overlapping its last
 * W positions in one device pool shared by all sequences (pages handed out in a
 * seeded order), and a page whose last position leaves the window is copied to
 * a host-pinned cold pool that the decode kernels read in place
 * (SFA_ATTEND_LOSSLESS, the reference semantics), or released
 * (SFA_ATTEND_WINDOW, an opt-in sliding attention window of W positions).
 *
 * A step is sfa_pager_begin (plan pages, evict, update device tables), then per
 * layer sfa_pager_append and sfa_pager_attend, all ordered on one stream.
 * Calls return sf_status codes (sfa.h) and never throw.  A pager is used from
 * one thread (Engine::forward is not thread-safe, engine.h:97-101).
 */
#ifndef SFA_PAGER_H
#define SFA_PAGER_H

#include "sfa.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SFA_ATTEND_LOSSLESS 0 /* attend 0..pos; evicted pages live in the cold pool */
#define SFA_ATTEND_WINDOW   1 /* attend the last `window` positions; evicted pages are freed */

typedef struct sfa_pager sfa_pager;

typedef struct sfa_pager_config {
    int32_t n_layer;
    int32_t n_head, n_head_kv, head_dim;
    int32_t kv_type;       /* SFA_KV_F32, SFA_KV_F16 or SFA_KV_Q8_0                  */
    int32_t page_size;     /* positions per page, a multiple of 64 (a multi-token    */
                           /* step is attended by the prefill's 64-position tiles); */
                           /* other sizes: SFA_ERR_UNSUPPORTED from create          */
    int32_t n_seq;         /* sequences decoded together                             */
    int32_t n_ctx;         /* positions per sequence (KvStore capacity)              */
    int32_t window;        /* resident positions per sequence; 0 = n_ctx (no paging) */
    int32_t attend;        /* SFA_ATTEND_LOSSLESS or SFA_ATTEND_WINDOW               */
    int32_t n_pages;       /* device pool pages; 0 = n_seq * (ceil(window/page_size) + 1) */
    int32_t n_cold_pages;  /* cold pool pages (lossless); 0 = n_seq * ceil(n_ctx/page_size) */
    uint64_t seed;         /* order in which free device pages are handed out        */
} sfa_pager_config;

typedef struct sfa_pager_stats {
    int64_t pages_allocated;  /* device pages handed out                      */
    int64_t pages_evicted;    /* pages copied to the cold pool                */
    int64_t pages_dropped;    /* pages released without a copy                */
    int64_t dev_pages_in_use;
    int64_t cold_pages_in_use;
    int64_t bytes_evicted;    /* device-to-host bytes of the eviction copies  */
    int64_t pages_in_flight;  /* evicted pages still served from the device   */
} sfa_pager_stats;

/* Allocates the device pool (all layers, K and V), the host-pinned cold pool,
 * the device page tables and the decode workspace.  Synchronises the device. */
SFA_API int sfa_pager_create(const sfa_pager_config *cfg, sfa_pager **out);
SFA_API void sfa_pager_destroy(sfa_pager *pager);

/* Starts a step: sequence b gets the next n_tok[b] positions (0 <= n_tok[b] <=
 * page_size; host array).  Pages whose last position leaves the window are
 * released (SFA_ATTEND_WINDOW) or evicted (lossless): a device-to-host copy of
 * every layer's K and V runs on a copy stream of the pager's own, ordered after
 * the work already on `stream`, and the page keeps serving reads from HBM until
 * a later step sees the copy complete; only then does its table entry move to
 * the cold page and the device page return to the pool.  An allocation that
 * finds no other free page takes the oldest such page and makes `stream` wait
 * for its copy.  New pages are taken from the pool, and the device page tables,
 * seq_len, kv_lo and the step's (seq, pos) token arrays are updated by a kernel
 * on `stream` (no host synchronisation).  Tokens of the step are ordered by
 * sequence, then position.  On error the pager is unchanged.  Host code: not
 * for HIP graph capture (the per-layer calls below are). */
SFA_API int sfa_pager_begin(sfa_pager *pager, const int32_t *n_tok, void *stream);

/* Appends the step's tokens to one layer: k, v [n_tokens][n_head_kv][head_dim]
 * f32 device, post-RoPE K (engine.cpp:1646-1656). */
SFA_API int sfa_pager_append(sfa_pager *pager, int32_t layer, const float *k, const float *v,
                             void *stream);

/* sfa_pager_append with the RoPE of Qcur and Kcur fused in (sfa_rope_kv_append,
 * engine.cpp:1892-1897 then :1646-1656): q [n_tokens][n_head][head_dim] f32
 * device pre-RoPE, rotated in place for sfa_pager_attend (may be NULL); k
 * pre-RoPE, v raw. */
SFA_API int sfa_pager_rope_append(sfa_pager *pager, int32_t layer, float *q, const float *k,
                                  const float *v, float freq_base, void *stream);

/* Attention of the step's tokens over one layer: q [n_tokens][n_head][head_dim]
 * f32 device, out [n_tokens][n_head * head_dim] f32 device.  A step with one
 * token per sequence runs sfa_attn_decode over the batch (split plan sized for
 * n_ctx when lossless, `window` when windowed); other steps run
 * sfa_attn_prefill per sequence with tokens (its page-size and Q8_0 head_dim
 * limits are checked by sfa_pager_create already).  Under
 * SFA_ATTEND_WINDOW a sequence may take at most one token in such a step (each
 * token of a chunk would need its own window start): SFA_ERR_UNSUPPORTED. */
SFA_API int sfa_pager_attend(sfa_pager *pager, int32_t layer, const float *q, float *out,
                             void *stream);

/* sfa_pager_append then sfa_pager_attend for one layer, in one call: the
 * reference's attention node with its append (engine.cpp:1633-1762).  A step
 * with one token per sequence over an F16 or F32 cache runs them fused
 * (sfa_attn_decode_append: one launch fewer, the same bytes and results);
 * other steps issue the two calls. */
SFA_API int sfa_pager_append_attend(sfa_pager *pager, int32_t layer, const float *k, const float *v,
                                    const float *q, float *out, void *stream);

/* Releases every page of sequence `seq` and rewinds it to position 0. */
SFA_API int sfa_pager_reset(sfa_pager *pager, int32_t seq, void *stream);

SFA_API int sfa_pager_stats_get(const sfa_pager *pager, sfa_pager_stats *out);

/* The per-layer descriptor the pager passes to libsfa. */
SFA_API int sfa_pager_desc(const sfa_pager *pager, int32_t layer, sfa_kv_desc *out);

/* Pages per sequence table row (ceil(n_ctx / page_size)). */
SFA_API int32_t sfa_pager_max_pages(const sfa_pager *pager);

/* The device arrays the pager keeps for libsfa: page tables [n_seq][max_pages],
 * seq_len [n_seq] and kv_lo [n_seq] (int32, device memory owned by the pager,
 * valid until sfa_pager_destroy; rewritten at every sfa_pager_begin on that
 * call's stream).  For callers that run sfa.h entry points over the pager's
 * pools themselves (sfa_attn_decode_split to time the split pass alone,
 * sfa_attn_decode_noalloc).  Any pointer may be NULL. */
SFA_API int sfa_pager_device_tables(const sfa_pager *pager, const int32_t **page_table,
                                    const int32_t **seq_len, const int32_t **kv_lo);

/* Host mirror of the page tables [n_seq][max_pages] and fill positions [n_seq];
 * either pointer may be NULL. */
SFA_API int sfa_pager_tables(const sfa_pager *pager, int32_t *page_table, int32_t *used);

#ifdef __cplusplus
}
#endif

#endif /* SFA_PAGER_H */
