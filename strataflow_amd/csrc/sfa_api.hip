// sfa_api.hip - extern "C" entry points of libsfa.so (declared in include/sfa.h).
// Every entry point validates its arguments on the host, returns an sf_status
// value and never lets an exception escape (the reference's C ABI rule,
// src/model/ggml_model.cpp:121-124).
#include <exception>

#include "sfa_common.h"

namespace sfa {
int decode_launch(const sfa_kv_desc *kv, const float *q, float *out, const int32_t *page_table,
                  int32_t max_pages, const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                  int32_t max_seq_len, float scale, void *workspace, size_t ws_bytes,
                  int passes, hipStream_t stream);
size_t decode_workspace_bytes(int B, int Hkv, int G, int HD, int max_seq_len);
int prefill_launch(const sfa_kv_desc *kv, const float *q, float *out, const int32_t *page_table,
                   int32_t max_pages, int32_t q_pos0, int32_t T, int32_t kv_lo, float scale,
                   hipStream_t stream);
int append_launch(const sfa_kv_desc *kv, const float *k, const float *v, const int32_t *seq,
                  const int32_t *pos, int32_t n_tok, const int32_t *page_table, int32_t max_pages,
                  hipStream_t stream);
int rope_append_launch(const sfa_kv_desc *kv, float *q, const float *k, const float *v,
                       const int32_t *seq, const int32_t *pos, int32_t n_tok,
                       const int32_t *page_table, int32_t max_pages, float freq_base,
                       hipStream_t stream);
int workspace_init_launch(void *ws, size_t bytes, hipStream_t stream);
int decode_noalloc_launch(const sfa_kv_desc *kv, const float *q, float *out, const int32_t *page_table,
                          int32_t max_pages, const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                          int32_t max_seq_len, float scale, hipStream_t stream);
int decode_append_launch(const sfa_kv_desc *kv, const float *k, const float *v, const float *q,
                         float *out, const int32_t *page_table, int32_t max_pages,
                         const int32_t *seq_len, const int32_t *kv_lo, int32_t B, int32_t max_seq_len,
                         float scale, void *workspace, size_t ws_bytes, hipStream_t stream);
}  // namespace sfa

namespace {

int check_desc(const sfa_kv_desc *kv) {
    if (kv == nullptr) return SFA_ERR_INVALID_ARGUMENT;
    if (kv->n_head <= 0 || kv->n_head_kv <= 0 || kv->n_head % kv->n_head_kv != 0)
        return SFA_ERR_INVALID_ARGUMENT;
    if (kv->head_dim != 32 && kv->head_dim != 64 && kv->head_dim != 128) return SFA_ERR_UNSUPPORTED;
    if (kv->page_size <= 0 || kv->page_size % sfa::kTile != 0) return SFA_ERR_INVALID_ARGUMENT;
    if (kv->kv_type != SFA_KV_F32 && kv->kv_type != SFA_KV_F16 && kv->kv_type != SFA_KV_Q8_0)
        return SFA_ERR_UNSUPPORTED;
    // the Q8_0 attention kernels take two or four 32-element blocks per row
    // (one per lane half); a one-block row (head_dim 32) is refused for every
    // entry point, the append included, so no cache is written that nothing
    // could attend over
    if (kv->kv_type == SFA_KV_Q8_0 && kv->head_dim < 64) return SFA_ERR_UNSUPPORTED;
    if (kv->n_pages < 0 || kv->n_cold_pages < 0) return SFA_ERR_INVALID_ARGUMENT;
    if (kv->n_pages > 0 && (kv->k_pages == nullptr || kv->v_pages == nullptr))
        return SFA_ERR_INVALID_ARGUMENT;
    if (kv->n_cold_pages > 0 && (kv->k_cold == nullptr || kv->v_cold == nullptr))
        return SFA_ERR_INVALID_ARGUMENT;
    const int g = kv->n_head / kv->n_head_kv;
    if (g != 1 && g != 2 && g != 4 && g != 8) return SFA_ERR_UNSUPPORTED;
    return SFA_OK;
}

}  // namespace

extern "C" {

SFA_API const char *sfa_status_str(int status) {
    switch (status) {
    case SFA_OK: return "ok";
    case SFA_ERR_INVALID_ARGUMENT: return "invalid argument";
    case SFA_ERR_UNSUPPORTED: return "unsupported";
    case SFA_ERR_OUT_OF_MEMORY: return "out of memory";
    case SFA_ERR_RUNTIME: return "runtime error";
    default: return "unknown status";
    }
}

SFA_API const char *sfa_version(void) { return "0.1.0-gfx950"; }

SFA_API size_t sfa_row_bytes(const sfa_kv_desc *kv) {
    if (kv == nullptr) return 0;
    return (size_t)sfa::row_bytes_of(kv->kv_type, kv->head_dim);
}

SFA_API size_t sfa_page_bytes(const sfa_kv_desc *kv) {
    if (kv == nullptr || kv->page_size <= 0 || kv->n_head_kv <= 0) return 0;
    return sfa_row_bytes(kv) * (size_t)kv->n_head_kv * (size_t)kv->page_size;
}

SFA_API int sfa_kv_desc_check(const sfa_kv_desc *kv) { return check_desc(kv); }

SFA_API int sfa_kv_append(const sfa_kv_desc *kv, const float *k, const float *v,
                          const int32_t *seq, const int32_t *pos, int32_t n_tok,
                          const int32_t *page_table, int32_t max_pages, void *stream) {
    try {
        const int rc = check_desc(kv);
        if (rc != SFA_OK) return rc;
        return sfa::append_launch(kv, k, v, seq, pos, n_tok, page_table, max_pages,
                                  static_cast<hipStream_t>(stream));
    } catch (const std::exception &) {
        return SFA_ERR_RUNTIME;
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API int sfa_rope_kv_append(const sfa_kv_desc *kv, float *q, const float *k, const float *v,
                               const int32_t *seq, const int32_t *pos, int32_t n_tok,
                               const int32_t *page_table, int32_t max_pages, float freq_base,
                               void *stream) {
    try {
        const int rc = check_desc(kv);
        if (rc != SFA_OK) return rc;
        return sfa::rope_append_launch(kv, q, k, v, seq, pos, n_tok, page_table, max_pages, freq_base,
                                       static_cast<hipStream_t>(stream));
    } catch (const std::exception &) {
        return SFA_ERR_RUNTIME;
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API size_t sfa_decode_workspace_bytes(const sfa_kv_desc *kv, int32_t B, int32_t max_seq_len) {
    if (check_desc(kv) != SFA_OK || B <= 0 || max_seq_len <= 0) return 0;
    return sfa::decode_workspace_bytes(B, kv->n_head_kv, kv->n_head / kv->n_head_kv, kv->head_dim,
                                       max_seq_len);
}

SFA_API int sfa_workspace_init(void *workspace, size_t ws_bytes, void *stream) {
    try {
        return sfa::workspace_init_launch(workspace, ws_bytes, static_cast<hipStream_t>(stream));
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

static int decode_entry(const sfa_kv_desc *kv, const float *q, float *out, const int32_t *page_table,
                        int32_t max_pages, const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                        int32_t max_seq_len, float scale, void *workspace, size_t ws_bytes,
                        void *stream, int passes) {
    try {
        const int rc = check_desc(kv);
        if (rc != SFA_OK) return rc;
        if (!(scale > 0.0f)) return SFA_ERR_INVALID_ARGUMENT;
        return sfa::decode_launch(kv, q, out, page_table, max_pages, seq_len, kv_lo, B, max_seq_len,
                                  scale, workspace, ws_bytes, passes, static_cast<hipStream_t>(stream));
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API int sfa_attn_decode(const sfa_kv_desc *kv, const float *q, float *out,
                            const int32_t *page_table, int32_t max_pages,
                            const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                            int32_t max_seq_len, float scale, void *workspace, size_t ws_bytes,
                            void *stream) {
    return decode_entry(kv, q, out, page_table, max_pages, seq_len, kv_lo, B, max_seq_len, scale,
                        workspace, ws_bytes, stream, 3);
}

SFA_API int sfa_attn_decode_append(const sfa_kv_desc *kv, const float *k, const float *v,
                                   const float *q, float *out, const int32_t *page_table,
                                   int32_t max_pages, const int32_t *seq_len, const int32_t *kv_lo,
                                   int32_t B, int32_t max_seq_len, float scale, void *workspace,
                                   size_t ws_bytes, void *stream) {
    try {
        const int rc = check_desc(kv);
        if (rc != SFA_OK) return rc;
        if (!(scale > 0.0f)) return SFA_ERR_INVALID_ARGUMENT;
        return sfa::decode_append_launch(kv, k, v, q, out, page_table, max_pages, seq_len, kv_lo, B,
                                         max_seq_len, scale, workspace, ws_bytes,
                                         static_cast<hipStream_t>(stream));
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API int sfa_attn_decode_split(const sfa_kv_desc *kv, const float *q, float *out,
                                  const int32_t *page_table, int32_t max_pages,
                                  const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                                  int32_t max_seq_len, float scale, void *workspace,
                                  size_t ws_bytes, void *stream) {
    return decode_entry(kv, q, out, page_table, max_pages, seq_len, kv_lo, B, max_seq_len, scale,
                        workspace, ws_bytes, stream, 1);
}

SFA_API int sfa_attn_decode_merge(const sfa_kv_desc *kv, const float *q, float *out,
                                  const int32_t *page_table, int32_t max_pages,
                                  const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                                  int32_t max_seq_len, float scale, void *workspace,
                                  size_t ws_bytes, void *stream) {
    return decode_entry(kv, q, out, page_table, max_pages, seq_len, kv_lo, B, max_seq_len, scale,
                        workspace, ws_bytes, stream, 2);
}

SFA_API int sfa_attn_decode_noalloc(const sfa_kv_desc *kv, const float *q, float *out,
                                    const int32_t *page_table, int32_t max_pages,
                                    const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                                    int32_t max_seq_len, float scale, void *stream) {
    try {
        const int rc = check_desc(kv);
        if (rc != SFA_OK) return rc;
        if (!(scale > 0.0f)) return SFA_ERR_INVALID_ARGUMENT;
        return sfa::decode_noalloc_launch(kv, q, out, page_table, max_pages, seq_len, kv_lo, B,
                                          max_seq_len, scale, static_cast<hipStream_t>(stream));
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API int sfa_attn_prefill(const sfa_kv_desc *kv, const float *q, float *out,
                             const int32_t *page_table, int32_t max_pages, int32_t q_pos0,
                             int32_t T, int32_t kv_lo, float scale, void *stream) {
    try {
        const int rc = check_desc(kv);
        if (rc != SFA_OK) return rc;
        if (!(scale > 0.0f)) return SFA_ERR_INVALID_ARGUMENT;
        return sfa::prefill_launch(kv, q, out, page_table, max_pages, q_pos0, T, kv_lo, scale,
                                   static_cast<hipStream_t>(stream));
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API int sfa_page_table_check(const sfa_kv_desc *kv, const int32_t *page_table,
                                 int32_t max_pages, const int32_t *seq_len, const int32_t *kv_lo,
                                 int32_t B) {
    const int rc = check_desc(kv);
    if (rc != SFA_OK) return rc;
    if (page_table == nullptr || seq_len == nullptr || B < 0 || max_pages <= 0)
        return SFA_ERR_INVALID_ARGUMENT;
    for (int32_t b = 0; b < B; ++b) {
        const int32_t n = seq_len[b];
        int32_t lo = kv_lo ? kv_lo[b] : 0;
        if (lo < 0) lo = 0;
        if (n < 0) return SFA_ERR_INVALID_ARGUMENT;
        if (n <= lo) continue;
        if ((int64_t)(n - 1) / kv->page_size >= max_pages) return SFA_ERR_INVALID_ARGUMENT;
        for (int32_t lp = lo / kv->page_size; lp <= (n - 1) / kv->page_size; ++lp) {
            const int32_t id = page_table[(int64_t)b * max_pages + lp];
            if (id >= 0) {
                if (id >= kv->n_pages) return SFA_ERR_INVALID_ARGUMENT;
            } else if (id <= -2) {
                if (-2 - (int64_t)id >= kv->n_cold_pages) return SFA_ERR_INVALID_ARGUMENT;
            } else {
                return SFA_ERR_INVALID_ARGUMENT;
            }
        }
    }
    return SFA_OK;
}

}  // extern "C"
