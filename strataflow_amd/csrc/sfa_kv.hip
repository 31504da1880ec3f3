// sfa_kv.hip - KV append into the paged cache and workspace fill.
//
// The append is the ggml_cpy of Kcur/Vcur into the cache column of each token
// (src/model/engine/engine.cpp:1646-1656), with the conversion a cpy into the
// cache type performs: F16 rounds to nearest even; Q8_0 quantises each 32-block
// with d = amax/127 (stored fp16) and q = round(x * (1/d)).  Division and
// reciprocal are IEEE-correct here (no fast-math), so the bytes written equal a
// CPU quantiser's bit for bit.
#include "sfa_common.h"

namespace sfa {

struct AppendParams {
    uint8_t *k_pages;
    uint8_t *v_pages;
    uint8_t *k_cold;
    uint8_t *v_cold;
    int64_t page_bytes;
    int n_pages;
    int n_cold;
    int page_size;
    int n_head_kv;
    int head_dim;
    int row_bytes;
    const float *k;
    const float *v;
    const int32_t *seq;
    const int32_t *pos;
    int n_tok;
    const int32_t *page_table;
    int max_pages;
};

__device__ inline uint8_t *page_base_rw(int32_t id, uint8_t *pool, int n_pages, uint8_t *cold,
                                        int n_cold, int64_t page_bytes) {
    return const_cast<uint8_t *>(page_base(id, pool, n_pages, cold, n_cold, page_bytes));
}

__device__ inline uint8_t *row_ptr(const AppendParams &p, int which, int tok, int kvh) {
    const int ps = p.pos[tok];
    const int sq = p.seq[tok];
    if (ps < 0 || sq < 0) return nullptr;
    const int lp = ps / p.page_size;
    if (lp >= p.max_pages) return nullptr;
    const int32_t id = p.page_table[(int64_t)sq * p.max_pages + lp];
    uint8_t *base = which ? page_base_rw(id, p.v_pages, p.n_pages, p.v_cold, p.n_cold, p.page_bytes)
                          : page_base_rw(id, p.k_pages, p.n_pages, p.k_cold, p.n_cold, p.page_bytes);
    if (base == nullptr) return nullptr;
    return base + ((int64_t)(ps - lp * p.page_size) * p.n_head_kv + kvh) * p.row_bytes;
}

// One thread per 8 elements of a row: f32 -> f16 (RNE), 16-byte store.
__global__ __launch_bounds__(256) void append_f16_kernel(AppendParams p) {
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
    const float *src = (which ? p.v : p.k) + ((int64_t)tok * p.n_head_kv + kvh) * p.head_dim + 8 * c;
    const floatx4 a = reinterpret_cast<const floatx4 *>(src)[0];
    const floatx4 bq = reinterpret_cast<const floatx4 *>(src)[1];
    half8 h;
    h[0] = (_Float16)a[0]; h[1] = (_Float16)a[1]; h[2] = (_Float16)a[2]; h[3] = (_Float16)a[3];
    h[4] = (_Float16)bq[0]; h[5] = (_Float16)bq[1]; h[6] = (_Float16)bq[2]; h[7] = (_Float16)bq[3];
    *reinterpret_cast<half8 *>(dst + 16 * c) = h;
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
    const float *src = (which ? p.v : p.k) + ((int64_t)tok * p.n_head_kv + kvh) * p.head_dim + kQK * blk;
    float x[kQK];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < kQK; j += 4) {
        const floatx4 v4 = reinterpret_cast<const floatx4 *>(src + j)[0];
        x[j] = v4[0]; x[j + 1] = v4[1]; x[j + 2] = v4[2]; x[j + 3] = v4[3];
    }
#pragma unroll
    for (int j = 0; j < kQK; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t *blkp = dst + kQ8Bytes * blk;
    const _Float16 dh = (_Float16)d;
    uint16_t dbits;
    __builtin_memcpy(&dbits, &dh, 2);
    // the block starts 2-byte aligned: store d and the quants as 16-bit words
    uint16_t *w = reinterpret_cast<uint16_t *>(blkp);
    w[0] = dbits;
#pragma unroll
    for (int j = 0; j < kQK; j += 2) {
        const int q0 = (int)roundf(x[j] * id);
        const int q1 = (int)roundf(x[j + 1] * id);
        w[1 + j / 2] = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
    }
}

__global__ void fill_zero_kernel(uint32_t *p, size_t n_words) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n_words) p[i] = 0u;
}

int append_launch(const sfa_kv_desc *kv, const float *k, const float *v, const int32_t *seq,
                  const int32_t *pos, int32_t n_tok, const int32_t *page_table, int32_t max_pages,
                  hipStream_t stream) {
    if (n_tok < 0 || max_pages <= 0) return SFA_ERR_INVALID_ARGUMENT;
    if (n_tok == 0) return SFA_OK;
    if (k == nullptr || v == nullptr || seq == nullptr || pos == nullptr || page_table == nullptr)
        return SFA_ERR_INVALID_ARGUMENT;
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
    int64_t total;
    if (kv->kv_type == SFA_KV_F16) {
        total = (int64_t)n_tok * kv->n_head_kv * (kv->head_dim / 8) * 2;
        hipLaunchKernelGGL(append_f16_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                           stream, p);
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

}  // namespace sfa
