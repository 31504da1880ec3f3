// sfa_kv.hip - KV append into the paged cache and workspace fill.
//
// The append is the ggml_cpy of Kcur/Vcur into the cache column of each token
// (src/model/engine/engine.cpp:1646-1656), with the conversion a cpy into the
// cache type performs: F32 copies (the reference's own cache type); F16 rounds
// to nearest even; Q8_0 quantises each 32-block
// with d = amax/127 (stored fp16) and q = round(x * (1/d)).  Division and
// reciprocal are IEEE-correct here (no fast-math), so the bytes written equal a
// CPU quantiser's bit for bit.
#include "sfa_append.h"

namespace sfa {

// One thread per 8 elements of a row: f32 -> f16 (RNE) or f32 as is.
template <int KVT>
__global__ __launch_bounds__(256) void append_e8_kernel(AppendParams p) {
    const int chunks = p.head_dim / 8;
    const int64_t total = (int64_t)p.n_tok * p.n_head_kv * chunks * 2;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int which = (int)(idx & 1);
    int64_t r = idx >> 1;
    const int c = (int)(r % chunks);
    r /= chunks;
    const int kvh = (int)(r % p.n_head_kv);
    const int tok = (int)(r / p.n_head_kv);
    uint8_t *dst = row_ptr(p, which, tok, kvh);
    if (dst == nullptr) return;
    float x[8];
    load_f32<8>((which ? p.v : p.k) + ((int64_t)tok * p.n_head_kv + kvh) * p.head_dim + 8 * c, x);
    if constexpr (KVT == SFA_KV_F16)
        store_f16x8(dst + 16 * c, x);
    else
        store_f32x8(dst + 32 * c, x);
}

// One thread per 32-element block: quantize_row_q8_0 semantics.
__global__ __launch_bounds__(256) void append_q8_0_kernel(AppendParams p) {
    const int nb = p.head_dim / kQK;
    const int64_t total = (int64_t)p.n_tok * p.n_head_kv * nb * 2;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int which = (int)(idx & 1);
    int64_t r = idx >> 1;
    const int blk = (int)(r % nb);
    r /= nb;
    const int kvh = (int)(r % p.n_head_kv);
    const int tok = (int)(r / p.n_head_kv);
    uint8_t *dst = row_ptr(p, which, tok, kvh);
    if (dst == nullptr) return;
    float x[kQK];
    load_f32<kQK>((which ? p.v : p.k) + ((int64_t)tok * p.n_head_kv + kvh) * p.head_dim + kQK * blk, x);
    store_q8_block(dst + kQ8Bytes * blk, x);
}

// Fused RoPE NORMAL + KV append (engine.cpp:1892-1897, then :1646-1656), one
// workgroup per token.  ggml_rope_ext mode 0 with n_dims = head_dim,
// freq_scale 1, ext_factor 0, attn_factor 1: pair (x[2i], x[2i+1]) rotates by
// theta_i, where theta_0 = pos and theta_{i+1} = theta_i * theta_scale in f32
// (ggml's recurrence, theta_scale = powf(freq_base, -2/n_dims) computed on the
// host), with cosf / sinf of theta_i.  Q rotates in place; K rotates on its
// way into the cache (converted as the append converts); V is appended raw.
// A token with seq < 0 or pos < 0 is skipped entirely (Q untouched).
// Each thread's first Q pairs and K/V unit, and its unit's page-table entry,
// are loaded before the cos/sin table is built, so a one-token call's memory
// waits overlap the table's math.
constexpr int kMaxHalfDim = 64;
constexpr int kRopeQPairs = 8;  // Q pairs per thread loaded ahead (32 heads x 64 pairs / 256)
template <int KVT>
__global__ __launch_bounds__(256) void rope_append_kernel(AppendParams p, float *q, int n_head,
                                                          float theta_scale) {
    constexpr int E = KVT == SFA_KV_Q8_0 ? kQK : 8;  // elements per K/V unit of work
    __shared__ float cs[kMaxHalfDim][2];
    const int tok = blockIdx.x;
    const int ps = p.pos[tok];
    const bool valid = ps >= 0 && p.seq[tok] >= 0;  // workgroup-uniform
    const int tid = threadIdx.x;
    const int half = p.head_dim / 2;
    const int n_qp = q != nullptr ? n_head * half : 0;
    const int units = p.head_dim / E;
    const int n_units = 2 * p.n_head_kv * units;

    float2 qv[kRopeQPairs];
    float2 *qrow = q != nullptr ? reinterpret_cast<float2 *>(q + (int64_t)tok * n_head * p.head_dim) : nullptr;
#pragma unroll
    for (int j = 0; j < kRopeQPairs; ++j) {
        const int idx = tid + j * (int)blockDim.x;
        if (idx < n_qp) qv[j] = qrow[idx];
    }
    float x[E];
    const bool has_unit = tid < n_units;
    int which = 0, kvh = 0, u = 0;
    if (has_unit) {
        which = tid / (p.n_head_kv * units);
        const int r = tid % (p.n_head_kv * units);
        kvh = r / units;
        u = r % units;
        load_f32<E>((which ? p.v : p.k) + ((int64_t)tok * p.n_head_kv + kvh) * p.head_dim + E * u, x);
    }
    // the unit's destination row (a page-table read) while the loads fly
    uint8_t *dst0 = valid && has_unit ? row_ptr(p, which, tok, kvh) : nullptr;

    if (valid && tid < half) {
        float sn, c;
        rope_cos_sin(ps, tid, theta_scale, c, sn);
        cs[tid][0] = c;
        cs[tid][1] = sn;
    }
    __syncthreads();
    if (!valid) return;  // after the barrier every thread of the workgroup reaches
    auto rot = [&](float &x0, float &x1, int i) { rope_rotate(x0, x1, cs[i][0], cs[i][1]); };
    // Q: pair idx of the token's row is head idx / half, pair idx % half
#pragma unroll
    for (int j = 0; j < kRopeQPairs; ++j) {
        const int idx = tid + j * (int)blockDim.x;
        if (idx < n_qp) {
            float2 v = qv[j];
            rot(v.x, v.y, idx % half);
            qrow[idx] = v;
        }
    }
    for (int idx = tid + kRopeQPairs * (int)blockDim.x; idx < n_qp; idx += blockDim.x) {
        float2 v = qrow[idx];
        rot(v.x, v.y, idx % half);
        qrow[idx] = v;
    }
    auto put = [&](uint8_t *dst, int w, int un, float (&xs)[E]) {
        if (dst == nullptr) return;
        if (w == 0) {
#pragma unroll
            for (int j = 0; j < E; j += 2) rot(xs[j], xs[j + 1], (E * un + j) / 2);
        }
        if constexpr (KVT == SFA_KV_F16)
            store_f16x8(dst + 16 * un, xs);
        else if constexpr (KVT == SFA_KV_F32)
            store_f32x8(dst + 32 * un, xs);
        else
            store_q8_block(dst + kQ8Bytes * un, xs);
    };
    if (has_unit) put(dst0, which, u, x);
    for (int idx = tid + (int)blockDim.x; idx < n_units; idx += blockDim.x) {
        const int w = idx / (p.n_head_kv * units);
        const int r = idx % (p.n_head_kv * units);
        const int h = r / units, un = r % units;
        float xs[E];
        load_f32<E>((w ? p.v : p.k) + ((int64_t)tok * p.n_head_kv + h) * p.head_dim + E * un, xs);
        put(row_ptr(p, w, tok, h), w, un, xs);
    }
}

__global__ void fill_zero_kernel(uint32_t *p, size_t n_words) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n_words) p[i] = 0u;
}

static AppendParams append_params(const sfa_kv_desc *kv, const float *k, const float *v,
                                  const int32_t *seq, const int32_t *pos, int32_t n_tok,
                                  const int32_t *page_table, int32_t max_pages) {
    AppendParams p;
    p.k_pages = static_cast<uint8_t *>(kv->k_pages);
    p.v_pages = static_cast<uint8_t *>(kv->v_pages);
    p.k_cold = static_cast<uint8_t *>(kv->k_cold);
    p.v_cold = static_cast<uint8_t *>(kv->v_cold);
    p.row_bytes = row_bytes_of(kv->kv_type, kv->head_dim);
    p.page_bytes = (int64_t)p.row_bytes * kv->n_head_kv * kv->page_size;
    p.n_pages = kv->n_pages;
    p.n_cold = kv->n_cold_pages;
    p.page_size = kv->page_size;
    p.n_head_kv = kv->n_head_kv;
    p.head_dim = kv->head_dim;
    p.k = k;
    p.v = v;
    p.seq = seq;
    p.pos = pos;
    p.n_tok = n_tok;
    p.page_table = page_table;
    p.max_pages = max_pages;
    return p;
}

int append_launch(const sfa_kv_desc *kv, const float *k, const float *v, const int32_t *seq,
                  const int32_t *pos, int32_t n_tok, const int32_t *page_table, int32_t max_pages,
                  hipStream_t stream) {
    if (n_tok < 0 || max_pages <= 0) return SFA_ERR_INVALID_ARGUMENT;
    if (n_tok == 0) return SFA_OK;
    if (k == nullptr || v == nullptr || seq == nullptr || pos == nullptr || page_table == nullptr)
        return SFA_ERR_INVALID_ARGUMENT;
    AppendParams p = append_params(kv, k, v, seq, pos, n_tok, page_table, max_pages);
    int64_t total;
    if (kv->kv_type == SFA_KV_F16 || kv->kv_type == SFA_KV_F32) {
        total = (int64_t)n_tok * kv->n_head_kv * (kv->head_dim / 8) * 2;
        const dim3 grid((unsigned)((total + 255) / 256));
        if (kv->kv_type == SFA_KV_F16)
            hipLaunchKernelGGL(append_e8_kernel<SFA_KV_F16>, grid, dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL(append_e8_kernel<SFA_KV_F32>, grid, dim3(256), 0, stream, p);
    } else if (kv->kv_type == SFA_KV_Q8_0) {
        total = (int64_t)n_tok * kv->n_head_kv * (kv->head_dim / kQK) * 2;
        hipLaunchKernelGGL(append_q8_0_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                           stream, p);
    } else {
        return SFA_ERR_UNSUPPORTED;
    }
    return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
}

int workspace_init_launch(void *ws, size_t bytes, hipStream_t stream) {
    if (ws == nullptr || (bytes & 3) != 0) return SFA_ERR_INVALID_ARGUMENT;
    const size_t words = bytes / 4;
    if (words == 0) return SFA_OK;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream,
                       static_cast<uint32_t *>(ws), words);
    return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
}

int rope_append_launch(const sfa_kv_desc *kv, float *q, const float *k, const float *v,
                       const int32_t *seq, const int32_t *pos, int32_t n_tok,
                       const int32_t *page_table, int32_t max_pages, float freq_base,
                       hipStream_t stream) {
    if (n_tok < 0 || max_pages <= 0 || !(freq_base > 0.0f)) return SFA_ERR_INVALID_ARGUMENT;
    if (n_tok == 0) return SFA_OK;
    if (k == nullptr || v == nullptr || seq == nullptr || pos == nullptr || page_table == nullptr)
        return SFA_ERR_INVALID_ARGUMENT;
    if (kv->head_dim / 2 > kMaxHalfDim) return SFA_ERR_UNSUPPORTED;
    AppendParams p = append_params(kv, k, v, seq, pos, n_tok, page_table, max_pages);
    // ggml: theta_scale = powf(freq_base, -2.0f/n_dims)
    const float theta_scale = powf(freq_base, -2.0f / (float)kv->head_dim);
    if (kv->kv_type == SFA_KV_F16) {
        hipLaunchKernelGGL(rope_append_kernel<SFA_KV_F16>, dim3((unsigned)n_tok), dim3(256), 0, stream, p, q,
                           kv->n_head, theta_scale);
    } else if (kv->kv_type == SFA_KV_F32) {
        hipLaunchKernelGGL(rope_append_kernel<SFA_KV_F32>, dim3((unsigned)n_tok), dim3(256), 0, stream, p, q,
                           kv->n_head, theta_scale);
    } else if (kv->kv_type == SFA_KV_Q8_0) {
        hipLaunchKernelGGL(rope_append_kernel<SFA_KV_Q8_0>, dim3((unsigned)n_tok), dim3(256), 0, stream, p, q,
                           kv->n_head, theta_scale);
    } else {
        return SFA_ERR_UNSUPPORTED;
    }
    return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
}

}  // namespace sfa
