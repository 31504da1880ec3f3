// sfa_append.h - writing K/V rows into the paged cache (the ggml_cpy of
// Kcur/Vcur into the cache column, src/model/engine/engine.cpp:1646-1656) and
// RoPE NORMAL's rotation (ggml_rope_ext mode 0, engine.cpp:1892-1897), shared
// by the append kernels and the fused Q/K/V product + RoPE + append.
#pragma once
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

// 8 consecutive elements of a row -> f16 (RNE), one 16-byte store.
__device__ inline void store_f16x8(uint8_t *dst, const float (&x)[8]) {
    half8 h;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = (_Float16)x[j];
    *reinterpret_cast<half8 *>(dst) = h;
}

// 8 consecutive elements of a row stored as f32, two 16-byte stores.
__device__ inline void store_f32x8(uint8_t *dst, const float (&x)[8]) {
    reinterpret_cast<floatx4 *>(dst)[0] = floatx4{x[0], x[1], x[2], x[3]};
    reinterpret_cast<floatx4 *>(dst)[1] = floatx4{x[4], x[5], x[6], x[7]};
}

// One 32-element block -> block_q8_0 (quantize_row_q8_0 semantics): d =
// amax / 127 stored fp16, q = round(x * (1/d)).  The block starts 2-byte
// aligned: d and the quants are stored as 16-bit words.
__device__ inline void store_q8_block(uint8_t *blkp, const float (&x)[kQK]) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < kQK; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const _Float16 dh = (_Float16)d;
    uint16_t dbits;
    __builtin_memcpy(&dbits, &dh, 2);
    uint16_t *w = reinterpret_cast<uint16_t *>(blkp);
    w[0] = dbits;
#pragma unroll
    for (int j = 0; j < kQK; j += 2) {
        const int q0 = (int)roundf(x[j] * id);
        const int q1 = (int)roundf(x[j + 1] * id);
        w[1 + j / 2] = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
    }
}

template <int N>
__device__ inline void load_f32(const float *src, float (&x)[N]) {
#pragma unroll
    for (int j = 0; j < N; j += 4) {
        const floatx4 v4 = reinterpret_cast<const floatx4 *>(src + j)[0];
        x[j] = v4[0]; x[j + 1] = v4[1]; x[j + 2] = v4[2]; x[j + 3] = v4[3];
    }
}

// ggml_rope_ext mode 0 (n_dims = head_dim, freq_scale 1, ext_factor 0,
// attn_factor 1): pair i rotates by theta_i, theta_0 = pos and theta_{j+1} =
// theta_j * theta_scale in f32 (ggml's recurrence), with cosf / sinf of
// theta_i (one sincosf: one argument reduction for both).
__device__ inline void rope_cos_sin(int pos, int i, float theta_scale, float &c, float &sn) {
    float theta = (float)pos;
    for (int j = 0; j < i; ++j) theta *= theta_scale;
    sincosf(theta, &sn, &c);
}

// (x0, x1) -> (x0 c - x1 s, x0 s + x1 c), each product rounded, then the sum
// (no fused multiply-add, as ggml's scalar rope computes it)
__device__ inline void rope_rotate(float &x0, float &x1, float c, float sn) {
    const float a0 = x0, a1 = x1;
    x0 = __fsub_rn(__fmul_rn(a0, c), __fmul_rn(a1, sn));
    x1 = __fadd_rn(__fmul_rn(a0, sn), __fmul_rn(a1, c));
}

}  // namespace sfa
