/*
 * sfa.h - C ABI of the MI355X (gfx950) paged-KV attention library (libsfa.so).
 *
 * This ABI replaces the attention node of StrataFlow's per-layer forward graph:
 *
 *   ggml_tensor *build_kv_attention(gctx, hp, Qcur, Kcur, Vcur, k_cache, v_cache,
 *                                   kq_mask, pos, n_kv, pg, graph_stores, cold_fills)
 *   (src/model/engine/engine.cpp:1633-1762)
 *
 * which appends this step's K/V into the KV cache column (engine.cpp:1646-1656),
 * assembles the history (engine.cpp:1658-1749) and computes
 *   kq = mul_mat(k, q) -> soft_max_ext(kq, mask, 1/sqrt(head_dim), 0) -> mul_mat(vt, kq)
 * (engine.cpp:1751-1761).  Here the append is sfa_kv_append() and the attention is
 * sfa_attn_decode() (one query token per sequence, the only shape the reference
 * engine issues, engine.cpp:2498, 2796) or sfa_attn_prefill() (a causal chunk).
 *
 * Layouts are the reference's:
 *   Q    : [n_tok][n_head][head_dim] f32, post-RoPE   (Qcur [hd, Hq, T], engine.cpp:1887,1892)
 *   K, V : [n_tok][n_head_kv][head_dim] f32, K post-RoPE, V raw (engine.cpp:1888-1897)
 *   out  : [n_tok][n_head * head_dim] f32              (cont_2d, engine.cpp:1761)
 *   cache: one "column" per position = n_head_kv rows of head_dim elements
 *          (k_cache [hd, Hkv, W], engine.cpp:1264-1275).  A page is page_size
 *          consecutive columns: byte offset of (pos_in_page, kv_head) is
 *          (pos_in_page * n_head_kv + kv_head) * row_bytes.  F32 rows are head_dim
 *          floats (the reference's own cache type); F16 rows are head_dim IEEE
 *          halves; Q8_0 rows are head_dim/32 ggml block_q8_0 records
 *          {fp16 d; int8 qs[32]} (34 bytes each).
 *   GQA  : query head h reads kv head h / (n_head / n_head_kv).
 *
 * Page tables map logical page i of a sequence (positions i*page_size ..) to a
 * physical page:  id >= 0  -> page id of the device pool (k_pages / v_pages);
 *                 id <= -2 -> page (-2 - id) of the cold pool (k_cold / v_cold),
 *                             host memory the GPU can read (hipHostMalloc);
 *                 id == -1 -> no page (an error if a read needs it).
 *
 * Every call is ordered on the given stream, allocates nothing, keeps no global
 * state and never throws.  Concurrent calls on distinct streams are safe when
 * they use distinct workspaces.  All pointer arguments except the cold pools
 * are device pointers.  Status codes reuse sf_status (include/strataflow/
 * strataflow.h:46-55 of the reference).
 */
#ifndef SFA_H
#define SFA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SFA_API __attribute__((visibility("default")))

/* status codes: same values as sf_status (strataflow.h:46-55) */
#define SFA_OK                   0
#define SFA_ERR_INVALID_ARGUMENT 1
#define SFA_ERR_UNSUPPORTED      3
#define SFA_ERR_OUT_OF_MEMORY    4
#define SFA_ERR_RUNTIME          7

/* KV element types: ggml type ids (GGML_TYPE_F32 = 0, F16 = 1, Q8_0 = 8) */
#define SFA_KV_F32  0
#define SFA_KV_F16  1
#define SFA_KV_Q8_0 8

/* Paged KV cache of ONE layer (the reference keeps a k_cache/v_cache pair per
 * layer, engine.cpp:1264-1275; a caller with one pool for all layers passes
 * per-layer pointers). */
typedef struct sfa_kv_desc {
    int32_t n_head;        /* Hq (query heads)                                  */
    int32_t n_head_kv;     /* Hkv; n_head % n_head_kv == 0                      */
    int32_t head_dim;      /* 32, 64 or 128 (64 or 128 for SFA_KV_Q8_0)         */
    int32_t page_size;     /* positions per page, a multiple of 32              */
    int32_t kv_type;       /* SFA_KV_F32, SFA_KV_F16 or SFA_KV_Q8_0             */
    int32_t n_pages;       /* pages in k_pages / v_pages                        */
    void   *k_pages;       /* device, n_pages * sfa_page_bytes()                */
    void   *v_pages;
    int32_t n_cold_pages;  /* pages in k_cold / v_cold (0 if none)              */
    int32_t reserved;
    void   *k_cold;        /* host-pinned cold pool readable by the GPU, or NULL */
    void   *v_cold;
} sfa_kv_desc;

/* Human-readable message for a status code. Never NULL. (sf_status_str,
 * strataflow.h:58) */
SFA_API const char *sfa_status_str(int status);

/* Library version string. */
SFA_API const char *sfa_version(void);

/* Bytes of one row (one position, one kv head) and of one page of K (or V).
 * Returns 0 for an invalid descriptor. */
SFA_API size_t sfa_row_bytes(const sfa_kv_desc *kv);
SFA_API size_t sfa_page_bytes(const sfa_kv_desc *kv);

/* Validates a descriptor on the host (shapes, type, alignment). */
SFA_API int sfa_kv_desc_check(const sfa_kv_desc *kv);

/* KV append: the ggml_cpy of Kcur/Vcur into the cache column of each token
 * (engine.cpp:1646-1656).  k, v: [n_tok][n_head_kv][head_dim] f32; token i
 * belongs to sequence seq[i] at absolute position pos[i]; its row lands in
 * page page_table[seq[i] * max_pages + pos[i] / page_size].  F32 caches store
 * the values as they are; F16 caches round to nearest even; Q8_0 caches
 * quantise each 32-block with d = amax/127 (fp16) and q = round(x / d).  The kernel writes nothing for a token whose page id
 * is -1 or outside its pool (it cannot report that back without a sync), so
 * callers validate host page tables with sfa_page_table_check(). */
SFA_API int sfa_kv_append(const sfa_kv_desc *kv, const float *k, const float *v,
                          const int32_t *seq, const int32_t *pos, int32_t n_tok,
                          const int32_t *page_table, int32_t max_pages,
                          void *stream);

/* Fused RoPE + KV append: the rope_ext of Qcur and Kcur (engine.cpp:1892-1897:
 * ggml_rope_ext mode NORMAL, n_dims = head_dim, freq_base, freq_scale 1,
 * ext_factor 0, attn_factor 1) followed by the append of sfa_kv_append
 * (engine.cpp:1646-1656), in one pass.  q: [n_tok][n_head][head_dim] f32 pre-RoPE,
 * rotated in place (may be NULL: K and V only); k: [n_tok][n_head_kv][head_dim]
 * f32 pre-RoPE (not modified; its rotation goes only into the cache, as Kcur's
 * does in the reference); v: raw V.  Pair (x[2i], x[2i+1]) rotates by theta_i,
 * theta_0 = pos and theta_{i+1} = theta_i * powf(freq_base, -2/head_dim) in f32
 * (ggml's recurrence), with cosf/sinf.  The rotated K is converted exactly as
 * sfa_kv_append converts.  A token with seq < 0 or pos < 0 is skipped (its Q
 * row untouched).  head_dim <= 128. */
SFA_API int sfa_rope_kv_append(const sfa_kv_desc *kv, float *q, const float *k, const float *v,
                               const int32_t *seq, const int32_t *pos, int32_t n_tok,
                               const int32_t *page_table, int32_t max_pages, float freq_base,
                               void *stream);

/* Workspace bytes needed by sfa_attn_decode for B sequences with the given
 * max_seq_len (the bound on the attended span, see sfa_attn_decode). */
SFA_API size_t sfa_decode_workspace_bytes(const sfa_kv_desc *kv, int32_t B,
                                          int32_t max_seq_len);

/* Zeroes a workspace with a fill kernel (safe under stream capture).  The
 * decode passes do not need a zeroed workspace; this is for callers that want
 * deterministic contents before first use. */
SFA_API int sfa_workspace_init(void *workspace, size_t ws_bytes, void *stream);

/* Decode attention: one query token per sequence (engine.cpp:1751-1761 with
 * n_tokens == 1 and an all-zero mask, engine.cpp:2796, 2820-2822).
 *   q   : [B][n_head][head_dim] f32 post-RoPE;  out: [B][n_head * head_dim] f32
 *   page_table : [B][max_pages] int32;  seq_len : [B] int32 = n_kv = pos + 1
 *   kv_lo : [B] int32 first attended position, or NULL for 0.  NULL (or 0) is
 *           the reference semantics: every position 0..n_kv-1 is attended
 *           (the KV window bounds residency only, src/kv/kv_store.h:1-22).  A
 *           positive kv_lo is an opt-in sliding attention window.
 *   max_seq_len : host bound on every attended span seq_len[b] - kv_lo[b]
 *           (seq_len[b] when kv_lo is NULL); sizes the split grid and the
 *           workspace.  A longer span is still attended in full, by fewer,
 *           longer splits.
 *   scale : 1/sqrt(head_dim) in the reference (engine.cpp:1756)
 * Split-K over logical positions, then a merge pass in split order: results
 * do not depend on where pages live (paged == contiguous, bit for bit).
 * Sequences with seq_len <= kv_lo produce zeros.  The kernels read seq_len on
 * the device and never past the table: positions at or beyond
 * max_pages * page_size are not attended (seq_len is clamped to the table's
 * capacity without an error, which a device-side call cannot report);
 * sfa_page_table_check() rejects such a table on the host. */
SFA_API int sfa_attn_decode(const sfa_kv_desc *kv, const float *q, float *out,
                            const int32_t *page_table, int32_t max_pages,
                            const int32_t *seq_len, const int32_t *kv_lo,
                            int32_t B, int32_t max_seq_len, float scale,
                            void *workspace, size_t ws_bytes, void *stream);

/* The whole attention node of one decode step, the append included
 * (build_kv_attention, engine.cpp:1633-1762: ggml_cpy of Kcur/Vcur into the
 * cache column at engine.cpp:1646-1656, then the attention): appends each
 * sequence's new token and attends, in the same two passes as
 * sfa_attn_decode.
 *   k, v : [B][n_head_kv][head_dim] f32, K post-RoPE; token b goes to position
 *          seq_len[b] - 1 of sequence b (no token where seq_len[b] is 0)
 *   the rest as sfa_attn_decode; the pools are written (kv->k_pages / v_pages
 *   and the cold pools, through the page table).
 * Equals sfa_kv_append(k, v, seq = b, pos = seq_len[b] - 1) followed by
 * sfa_attn_decode, bit for bit, pool bytes included (a position past the
 * table, or on a page id that is not there, is skipped as the append skips
 * it).  F16 and F32 caches: SFA_ERR_UNSUPPORTED for Q8_0, whose callers issue
 * the two calls. */
SFA_API int sfa_attn_decode_append(const sfa_kv_desc *kv, const float *k, const float *v,
                                   const float *q, float *out, const int32_t *page_table,
                                   int32_t max_pages, const int32_t *seq_len, const int32_t *kv_lo,
                                   int32_t B, int32_t max_seq_len, float scale, void *workspace,
                                   size_t ws_bytes, void *stream);

/* The two passes of sfa_attn_decode, for callers that schedule them apart
 * (e.g. to overlap the merge with other work, or to time the split-K pass):
 * sfa_attn_decode == sfa_attn_decode_split then sfa_attn_decode_merge on the
 * same stream with the same arguments.  The split pass writes per-split
 * (m, l, o) partials to the workspace (and the final output directly when a
 * sequence needs one split); the merge pass combines them.  No counterpart in
 * the reference: its attention is one ggml graph. */
SFA_API int sfa_attn_decode_split(const sfa_kv_desc *kv, const float *q, float *out,
                                  const int32_t *page_table, int32_t max_pages,
                                  const int32_t *seq_len, const int32_t *kv_lo,
                                  int32_t B, int32_t max_seq_len, float scale,
                                  void *workspace, size_t ws_bytes, void *stream);
SFA_API int sfa_attn_decode_merge(const sfa_kv_desc *kv, const float *q, float *out,
                                  const int32_t *page_table, int32_t max_pages,
                                  const int32_t *seq_len, const int32_t *kv_lo,
                                  int32_t B, int32_t max_seq_len, float scale,
                                  void *workspace, size_t ws_bytes, void *stream);

/* Allocation-free decode: sfa_attn_decode without a workspace argument, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
 * the reference (its attention is one ggml graph whose allocator owns every
 * buffer).  The split partials live in a library-owned device array of
 * SFA_NOALLOC_SCRATCH_BYTES per GPU: a global of libsfa's code object, so
 * every process that loads libsfa's kernels on a GPU holds it there until the
 * process ends, whether or not it calls this entry point; its address is
 * looked up once per device, at the first call on that device.  The call
 * makes no allocation.  Returns SFA_ERR_OUT_OF_MEMORY when the shape needs
 * more than SFA_NOALLOC_SCRATCH_BYTES (sfa_decode_workspace_bytes tells the
 * need).  Every call on one GPU shares that GPU's array: calls that overlap
 * in time on one GPU (distinct streams, or concurrent host threads) race, so
 * a caller orders them on one stream.  The passes read only what the same
 * call wrote, so nothing needs clearing between calls.  Results are bit
 * identical to sfa_attn_decode's. */
#define SFA_NOALLOC_SCRATCH_BYTES (8u << 20)
SFA_API int sfa_attn_decode_noalloc(const sfa_kv_desc *kv, const float *q, float *out,
                                    const int32_t *page_table, int32_t max_pages,
                                    const int32_t *seq_len, const int32_t *kv_lo,
                                    int32_t B, int32_t max_seq_len, float scale, void *stream);

/* Chunked causal prefill of ONE sequence: T query tokens at absolute positions
 * q_pos0 .. q_pos0+T-1, whose K/V are already appended.  Token t attends kv
 * positions kv_lo .. q_pos0+t (causal -INF mask above the diagonal, the
 * llama.cpp kq_mask convention).  q: [T][n_head][head_dim] f32,
 * out: [T][n_head * head_dim] f32.  F32, F16 and Q8_0 caches (Q8_0 with
 * head_dim >= 64, as in decode).  The 64-position K/V tiles must each lie in
 * one page: page_size must be a multiple of 64 (SFA_ERR_UNSUPPORTED
 * otherwise). */
SFA_API int sfa_attn_prefill(const sfa_kv_desc *kv, const float *q, float *out,
                             const int32_t *page_table, int32_t max_pages,
                             int32_t q_pos0, int32_t T, int32_t kv_lo,
                             float scale, void *stream);

/* Host-side page-table validation (host arrays): every page a read of
 * positions [kv_lo[b], seq_len[b]) needs must be a valid id.  Returns SFA_OK or
 * SFA_ERR_INVALID_ARGUMENT. */
SFA_API int sfa_page_table_check(const sfa_kv_desc *kv, const int32_t *page_table,
                                 int32_t max_pages, const int32_t *seq_len,
                                 const int32_t *kv_lo, int32_t B);

#ifdef __cplusplus
}
#endif

#endif /* SFA_H */
