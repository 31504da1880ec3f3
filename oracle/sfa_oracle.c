/*
 * sfa_oracle.c - CPU restatement of StrataFlow's attention node over the KV
 * cache.  TEST INFRASTRUCTURE ONLY: tests/, the smoke check and the bench's
 * CPU-baseline leg load this library to check results against.  The product path (the HIP
 * library) never links, loads or calls it.
 *
 * What it restates (reference files under StrataFlow's tree):
 *   - KV append: ggml_cpy of Kcur/Vcur into cache column `pos`
 *     (src/model/engine/engine.cpp:1646-1656).  A cpy into F16 rounds to
 *     nearest even; a cpy into Q8_0 runs ggml's quantize_row_q8_0 (ggml, tag
 *     b11379, not vendored in the reference: d = amax/127 stored as fp16,
 *     q = round(x * (1/d))).
 *   - history assembly in absolute position order (engine.cpp:1658-1749): here
 *     a gather of pages through the page table into the column layout
 *     [n_kv][n_head_kv][head_dim].
 *   - the op sequence (engine.cpp:1751-1761):
 *       k  = cont(permute(k_hist))  [hd, n_kv, Hkv]
 *       v  = cont(permute(v_hist))
 *       kq = mul_mat(k, q)          GQA by batch broadcast: q head h -> kv h/g
 *       kq = soft_max_ext(kq, mask, 1/sqrt(hd), 0)
 *       vt = cont(transpose(v))     [n_kv, hd, Hkv]
 *       kqv = mul_mat(vt, kq) -> permute -> cont_2d
 *     with ggml's CPU operand conversions (mul_mat converts src1 to the
 *     vec_dot_type of src0): F16 K -> Q rounded to F16; Q8_0 K -> Q quantised
 *     to Q8_0 and an integer dot scaled by d_k*d_q per 32-block; F16 V -> P
 *     rounded to F16.  A Q8_0 V cannot be transposed as Q8_0, so it is
 *     dequantised to F32 before the transpose.  soft_max_ext: w = x*scale +
 *     mask, max, e = exp(w - max), sum in double, e * (float)(1/sum).
 *     (ORC_GGML mode.)
 *   - ORC_EXACT mode: float64 arithmetic on the exactly dequantised K/V and
 *     the unrounded Q (the "exact-dequant" reading).
 *
 * Summation order inside dot products follows no particular SIMD schedule;
 * it affects the last ulps only.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_KV_F32 0
#define ORC_KV_F16 1
#define ORC_KV_Q8_0 8

#define ORC_GGML 0
#define ORC_EXACT 1

#define QK8_0 32

typedef struct {
    uint16_t d;
    int8_t qs[QK8_0];
} __attribute__((packed)) orc_block_q8_0;

_Static_assert(sizeof(orc_block_q8_0) == 34, "block_q8_0 is 34 bytes");

/* ---- IEEE half conversion ------------------------------------------------ */

/* f32 -> f16, round to nearest even, with subnormals, inf and nan.  This is the
 * conversion ggml's cpy / from_float applies (F16C or its software twin). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) { /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
    }
    if (absx >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (absx < 0x38800000u) { /* below the smallest normal half (2^-14) */
        /* subnormal half: value = m * 2^-24, m = round(|f| * 2^24) (RNE) */
        if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25 -> 0 */
        uint32_t e = absx >> 23;                       /* biased exponent */
        uint32_t mant = (absx & 0x7fffffu) | 0x800000u; /* 24-bit significand */
        /* value = mant * 2^(e-127-23); want mant * 2^(e-150+24) = mant >> (126-e) */
        uint32_t shift = 126u - e; /* 14..24 */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    /* normal half */
    uint32_t e = (absx >> 23) - 127u + 15u;
    uint32_t mant = absx & 0x7fffffu;
    uint32_t q = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u; /* may carry into exp */
    return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24 */
            float v = (float)m * (1.0f / 16777216.0f);
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_f32_to_f16_row(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_f16(x[i]);
}

/* f16 -> f32 lookup table for the hot loops (ggml's CPU backend keeps the same
 * kind of table); filled once at library load. */
static float orc_f16_table[65536];

__attribute__((constructor)) static void orc_init_table(void) {
    for (uint32_t i = 0; i < 65536u; ++i) orc_f16_table[i] = orc_f16_to_f32((uint16_t)i);
}

void orc_f16_to_f32_row(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f16_table[x[i]];
}

/* ---- Q8_0 ------------------------------------------------------------------ */

/* ggml's quantize_row_q8_0 comes in three forms (ggml, tag b11379; all store
 * d = amax / 127 as fp16 and q = round(x * id) per block of 32):
 *   ORC_Q8_SCALAR (0): the portable reference form quantize_row_q8_0_ref:
 *                      id = d ? 1/d : 0, roundf (ties away from zero);
 *   ORC_Q8_AVX2   (1): the x86 SIMD form: id = amax ? 127/amax : 0, rounded
 *                      to nearest even (_mm256_round_ps, _MM_ROUND_NEAREST);
 *   ORC_Q8_NEON   (2): the Arm SIMD form: id = d ? 1/d : 0, nearest even
 *                      (vcvtnq_s32_f32).
 * ggml's CPU backend runs the SIMD form of the host it was built for, both for
 * a cpy into a Q8_0 cache and for the Q8_0 conversion of src1 in mul_mat.  The
 * form is process-wide (orc_set_q8_variant); the default is the scalar one,
 * which is what the GPU append writes. */
#define ORC_Q8_SCALAR 0
#define ORC_Q8_AVX2 1
#define ORC_Q8_NEON 2
static int orc_q8_variant = ORC_Q8_SCALAR;

int orc_set_q8_variant(int v) {
    if (v < ORC_Q8_SCALAR || v > ORC_Q8_NEON) return 1;
    orc_q8_variant = v;
    return 0;
}

void orc_quantize_row_q8_0(const float *x, void *vy, int64_t k) {
    orc_block_q8_0 *y = (orc_block_q8_0 *)vy;
    const int64_t nb = k / QK8_0;
    const int var = orc_q8_variant;
    for (int64_t i = 0; i < nb; ++i) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; ++j) {
            const float v = fabsf(x[i * QK8_0 + j]);
            if (v > amax) amax = v;
        }
        const float d = amax / 127.0f;
        float id;
        if (var == ORC_Q8_AVX2) id = amax != 0.0f ? 127.0f / amax : 0.0f;
        else id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = orc_f32_to_f16(d);
        for (int j = 0; j < QK8_0; ++j) {
            const float v = x[i * QK8_0 + j] * id;
            /* nearbyintf rounds to nearest even in the default rounding mode */
            y[i].qs[j] = (int8_t)(var == ORC_Q8_SCALAR ? roundf(v) : nearbyintf(v));
        }
    }
}

void orc_dequantize_row_q8_0(const void *vx, float *y, int64_t k) {
    const orc_block_q8_0 *x = (const orc_block_q8_0 *)vx;
    const int64_t nb = k / QK8_0;
    for (int64_t i = 0; i < nb; ++i) {
        const float d = orc_f16_table[x[i].d];
        for (int j = 0; j < QK8_0; ++j) y[i * QK8_0 + j] = (float)x[i].qs[j] * d;
    }
}

/* ---- paged KV --------------------------------------------------------------- */

typedef struct orc_paged_kv {
    int32_t n_head_kv;
    int32_t head_dim;
    int32_t page_size;
    int32_t kv_type;
    int32_t n_pages;
    int32_t n_cold_pages;
    void *k_pages; /* host memory, page-major */
    void *v_pages;
    void *k_cold;
    void *v_cold;
} orc_paged_kv;

int64_t orc_row_bytes(const orc_paged_kv *kv) {
    switch (kv->kv_type) {
    case ORC_KV_F32: return (int64_t)kv->head_dim * 4;
    case ORC_KV_F16: return (int64_t)kv->head_dim * 2;
    case ORC_KV_Q8_0: return (int64_t)(kv->head_dim / QK8_0) * 34;
    default: return 0;
    }
}

int64_t orc_page_bytes(const orc_paged_kv *kv) {
    return orc_row_bytes(kv) * kv->n_head_kv * kv->page_size;
}

/* Address of the row (pos, kv_head) of the K (which=0) or V (which=1) cache of
 * a sequence whose page table is `pt`; NULL if the page is missing. */
static uint8_t *orc_row_ptr(const orc_paged_kv *kv, int which, const int32_t *pt,
                            int32_t max_pages, int64_t pos, int kvh) {
    const int64_t lp = pos / kv->page_size;
    if (lp < 0 || lp >= max_pages) return NULL;
    const int32_t id = pt[lp];
    uint8_t *base;
    int64_t page;
    if (id >= 0) {
        if (id >= kv->n_pages) return NULL;
        base = (uint8_t *)(which ? kv->v_pages : kv->k_pages);
        page = id;
    } else if (id <= -2) {
        page = -2 - (int64_t)id;
        if (page >= kv->n_cold_pages) return NULL;
        base = (uint8_t *)(which ? kv->v_cold : kv->k_cold);
    } else {
        return NULL;
    }
    if (base == NULL) return NULL;
    const int64_t rb = orc_row_bytes(kv);
    return base + page * orc_page_bytes(kv) +
           ((pos % kv->page_size) * kv->n_head_kv + kvh) * rb;
}

/* KV append (engine.cpp:1646-1656): token i of sequence seq[i] at position
 * pos[i]; k, v are [n_tok][n_head_kv][head_dim] f32.  Returns 0, or 1 if a
 * token's page is missing (nothing is written for it). */
int orc_kv_append(const orc_paged_kv *kv, const float *k, const float *v,
                  const int32_t *seq, const int32_t *pos, int32_t n_tok,
                  const int32_t *page_table, int32_t max_pages) {
    const int hd = kv->head_dim;
    int rc = 0;
    for (int32_t i = 0; i < n_tok; ++i) {
        const int32_t *pt = page_table + (int64_t)seq[i] * max_pages;
        for (int kvh = 0; kvh < kv->n_head_kv; ++kvh) {
            for (int which = 0; which < 2; ++which) {
                uint8_t *dst = orc_row_ptr(kv, which, pt, max_pages, pos[i], kvh);
                if (dst == NULL) { rc = 1; continue; }
                const float *src = (which ? v : k) + ((int64_t)i * kv->n_head_kv + kvh) * hd;
                switch (kv->kv_type) {
                case ORC_KV_F32: memcpy(dst, src, (size_t)hd * 4); break;
                case ORC_KV_F16: orc_f32_to_f16_row(src, (uint16_t *)dst, hd); break;
                case ORC_KV_Q8_0: orc_quantize_row_q8_0(src, dst, hd); break;
                }
            }
        }
    }
    return rc;
}

/* ---- attention ---------------------------------------------------------------- */

/* f32 dot with 8 independent partial sums (the shape of ggml's SIMD f32
 * accumulators; vectorises under -O3). */
static float orc_dot_f32(const float *a, const float *b, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        for (int j = 0; j < 8; ++j) acc[j] += a[i + j] * b[i + j];
    }
    float s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}

/* ggml_vec_dot_q8_0_q8_0: per block sumi (exact int) * (d_x * d_y), summed in f32. */
static float orc_dot_q8_0(const orc_block_q8_0 *x, const orc_block_q8_0 *y, int nb) {
    float sumf = 0.0f;
    for (int b = 0; b < nb; ++b) {
        int sumi = 0;
        for (int j = 0; j < QK8_0; ++j) sumi += (int)x[b].qs[j] * (int)y[b].qs[j];
        sumf += (float)sumi * (orc_f16_table[x[b].d] * orc_f16_table[y[b].d]);
    }
    return sumf;
}

/* Decodes one cache row into f32. */
static void orc_row_to_f32(const orc_paged_kv *kv, const uint8_t *row, float *out) {
    switch (kv->kv_type) {
    case ORC_KV_F32: memcpy(out, row, (size_t)kv->head_dim * 4); break;
    case ORC_KV_F16: orc_f16_to_f32_row((const uint16_t *)row, out, kv->head_dim); break;
    case ORC_KV_Q8_0: orc_dequantize_row_q8_0(row, out, kv->head_dim); break;
    }
}

/*
 * Attention over the paged cache for B sequences, T query tokens each.
 *   q   [B][T][n_head][hd] f32, out [B][T][n_head][hd] f32
 *   page_table [B][max_pages], seq_len[B] = n_kv (position of the last query
 *   token + 1), kv_lo[B] or NULL.  Query t of sequence b sits at position
 *   seq_len[b] - T + t and attends kv positions kv_lo[b] .. that position
 *   (the causal -INF mask; for T == 1 the mask is all zeros, engine.cpp:2796).
 *   Positions below kv_lo are masked with -INF, which ggml's soft_max_ext maps
 *   to an exact 0 weight, so skipping them is the same arithmetic.
 * mode ORC_GGML follows ggml's operand conversions; ORC_EXACT is float64.
 * Returns 0, 1 on a missing page, 2 on a bad argument.
 */
int orc_attention(const orc_paged_kv *kv, const float *q, float *out, int32_t n_head,
                  const int32_t *page_table, int32_t max_pages, const int32_t *seq_len,
                  const int32_t *kv_lo, int32_t B, int32_t T, float scale, int mode,
                  int n_threads) {
    const int hd = kv->head_dim;
    const int Hkv = kv->n_head_kv;
    if (hd <= 0 || Hkv <= 0 || n_head % Hkv != 0 || T <= 0) return 2;
    if (kv->kv_type == ORC_KV_Q8_0 && hd % QK8_0 != 0) return 2;
    const int g = n_head / Hkv;
    int rc = 0;
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#else
    (void)n_threads;
#endif

    for (int32_t b = 0; b < B; ++b) {
        const int64_t n_kv = seq_len[b];
        const int64_t lo = kv_lo ? (kv_lo[b] > 0 ? kv_lo[b] : 0) : 0;
        const int32_t *pt = page_table + (int64_t)b * max_pages;
        const float *qb = q + (int64_t)b * T * n_head * hd;
        float *ob = out + (int64_t)b * T * n_head * hd;
        if (n_kv == 0) { /* empty sequence: nothing attended */
            memset(ob, 0, sizeof(float) * (size_t)T * n_head * hd);
            continue;
        }
        if (n_kv - T < 0) return 2;
        const int64_t n = n_kv > lo ? n_kv - lo : 0; /* attended history length */
        if (n == 0) {
            memset(ob, 0, sizeof(float) * (size_t)T * n_head * hd);
            continue;
        }

        /* 1. gather: history [n][Hkv][hd] decoded to f32 (ggml views / assembly
         *    keep the typed bytes; decoding here is exact).  For the ggml mode
         *    the typed K is kept as well for the Q8_0 integer dot. */
        float *kh = (float *)malloc(sizeof(float) * (size_t)n * Hkv * hd);
        float *vh = (float *)malloc(sizeof(float) * (size_t)n * Hkv * hd);
        orc_block_q8_0 *kq8 = NULL;
        const int nb = hd / QK8_0;
        if (kv->kv_type == ORC_KV_Q8_0)
            kq8 = (orc_block_q8_0 *)malloc(sizeof(orc_block_q8_0) * (size_t)n * Hkv * nb);
        /* the copies run on all threads, as ggml's cpy / cont ops do */
        int missing = 0;
#pragma omp parallel for schedule(static) reduction(|| : missing)
        for (int64_t j = 0; j < n; ++j) {
            for (int kvh = 0; kvh < Hkv; ++kvh) {
                const uint8_t *kr = orc_row_ptr(kv, 0, pt, max_pages, lo + j, kvh);
                const uint8_t *vr = orc_row_ptr(kv, 1, pt, max_pages, lo + j, kvh);
                float *kd = kh + (j * Hkv + kvh) * hd;
                float *vd = vh + (j * Hkv + kvh) * hd;
                if (kr == NULL || vr == NULL) {
                    missing = 1;
                    memset(kd, 0, sizeof(float) * hd);
                    memset(vd, 0, sizeof(float) * hd);
                    continue;
                }
                orc_row_to_f32(kv, kr, kd);
                orc_row_to_f32(kv, vr, vd);
                if (kq8) memcpy(kq8 + (j * Hkv + kvh) * nb, kr, sizeof(orc_block_q8_0) * nb);
            }
        }
        if (missing) rc = 1;
        if (rc) {
            free(kh); free(vh); free(kq8);
            return rc;
        }

        if (mode == ORC_EXACT) {
#pragma omp parallel for collapse(2) schedule(static)
            for (int32_t t = 0; t < T; ++t) {
                for (int h = 0; h < n_head; ++h) {
                    const int kvh = h / g;
                    const int64_t qpos = n_kv - T + t;
                    const int64_t nt = qpos - lo + 1; /* causal: kv <= qpos */
                    const float *qr = qb + ((int64_t)t * n_head + h) * hd;
                    float *orow = ob + ((int64_t)t * n_head + h) * hd;
                    if (nt <= 0) {
                        memset(orow, 0, sizeof(float) * hd);
                        continue;
                    }
                    double *s = (double *)malloc(sizeof(double) * (size_t)nt);
                    double mx = -INFINITY;
                    for (int64_t j = 0; j < nt; ++j) {
                        const float *kr = kh + (j * Hkv + kvh) * hd;
                        double acc = 0.0;
                        for (int d = 0; d < hd; ++d) acc += (double)qr[d] * (double)kr[d];
                        s[j] = acc * (double)scale;
                        if (s[j] > mx) mx = s[j];
                    }
                    double sum = 0.0;
                    for (int64_t j = 0; j < nt; ++j) {
                        s[j] = exp(s[j] - mx);
                        sum += s[j];
                    }
                    for (int d = 0; d < hd; ++d) {
                        double acc = 0.0;
                        for (int64_t j = 0; j < nt; ++j) acc += s[j] * (double)vh[(j * Hkv + kvh) * hd + d];
                        orow[d] = (float)(acc / sum);
                    }
                    free(s);
                }
            }
        } else {
            /* 2. k = cont(permute(k_hist)) -> [Hkv][n][hd];
             *    v = cont(permute(v_hist)); vt = cont(transpose(v)) -> [Hkv][hd][n].
             *    Values keep the cache type (F16 values are F16-exact in f32). */
            float *kp = (float *)malloc(sizeof(float) * (size_t)n * Hkv * hd);
            float *vt = (float *)malloc(sizeof(float) * (size_t)n * Hkv * hd);
            orc_block_q8_0 *kp8 = NULL;
#pragma omp parallel for collapse(2) schedule(static)
            for (int kvh = 0; kvh < Hkv; ++kvh)
                for (int64_t j = 0; j < n; ++j)
                    memcpy(kp + ((int64_t)kvh * n + j) * hd, kh + (j * Hkv + kvh) * hd, sizeof(float) * hd);
            if (kq8) {
                kp8 = (orc_block_q8_0 *)malloc(sizeof(orc_block_q8_0) * (size_t)n * Hkv * nb);
#pragma omp parallel for collapse(2) schedule(static)
                for (int kvh = 0; kvh < Hkv; ++kvh)
                    for (int64_t j = 0; j < n; ++j)
                        memcpy(kp8 + ((int64_t)kvh * n + j) * nb, kq8 + (j * Hkv + kvh) * nb,
                               sizeof(orc_block_q8_0) * nb);
            }
#pragma omp parallel for collapse(2) schedule(static)
            for (int kvh = 0; kvh < Hkv; ++kvh)
                for (int d = 0; d < hd; ++d)
                    for (int64_t j = 0; j < n; ++j)
                        vt[((int64_t)kvh * hd + d) * n + j] = vh[(j * Hkv + kvh) * hd + d];

#pragma omp parallel for collapse(2) schedule(static)
            for (int32_t t = 0; t < T; ++t) {
                for (int h = 0; h < n_head; ++h) {
                    const int kvh = h / g;
                    const int64_t qpos = n_kv - T + t;
                    const int64_t nt = qpos - lo + 1;
                    const float *qr = qb + ((int64_t)t * n_head + h) * hd;
                    float *orow = ob + ((int64_t)t * n_head + h) * hd;
                    if (nt <= 0) {
                        memset(orow, 0, sizeof(float) * hd);
                        continue;
                    }
                    /* 3. kq = mul_mat(k, q): q converted to the vec_dot_type of k */
                    float *qc = (float *)malloc(sizeof(float) * hd);
                    orc_block_q8_0 *q8 = NULL;
                    if (kv->kv_type == ORC_KV_F16) {
                        for (int d = 0; d < hd; ++d) qc[d] = orc_f16_to_f32(orc_f32_to_f16(qr[d]));
                    } else {
                        memcpy(qc, qr, sizeof(float) * hd);
                    }
                    if (kv->kv_type == ORC_KV_Q8_0) {
                        q8 = (orc_block_q8_0 *)malloc(sizeof(orc_block_q8_0) * nb);
                        orc_quantize_row_q8_0(qr, q8, hd);
                    }
                    /* the row covers the full history; masked columns get -INF */
                    float *w = (float *)malloc(sizeof(float) * (size_t)n);
                    for (int64_t j = 0; j < n; ++j) {
                        float kqv;
                        if (q8) kqv = orc_dot_q8_0(kp8 + ((int64_t)kvh * n + j) * nb, q8, nb);
                        else kqv = orc_dot_f32(kp + ((int64_t)kvh * n + j) * hd, qc, hd);
                        /* 4. soft_max_ext: w = x*scale + mask (slope 1) */
                        const float mask = j < nt ? 0.0f : -INFINITY;
                        w[j] = kqv * scale + mask;
                    }
                    float mx = -INFINITY;
                    for (int64_t j = 0; j < n; ++j) if (w[j] > mx) mx = w[j];
                    double sum = 0.0;
                    for (int64_t j = 0; j < n; ++j) {
                        const float e = expf(w[j] - mx);
                        w[j] = e;
                        sum += (double)e;
                    }
                    const float inv = (float)(1.0 / sum);
                    for (int64_t j = 0; j < n; ++j) w[j] *= inv;
                    /* 5. kqv = mul_mat(vt, kq): kq converted to the vec_dot_type of vt */
                    if (kv->kv_type == ORC_KV_F16) {
                        for (int64_t j = 0; j < n; ++j) w[j] = orc_f16_to_f32(orc_f32_to_f16(w[j]));
                    }
                    for (int d = 0; d < hd; ++d) {
                        orow[d] = orc_dot_f32(vt + ((int64_t)kvh * hd + d) * n, w, (int)n);
                    }
                    free(w);
                    free(qc);
                    free(q8);
                }
            }
            free(kp);
            free(vt);
            free(kp8);
        }
        free(kh);
        free(vh);
        free(kq8);
    }
    return rc;
}

/* RoPE NORMAL (ggml_rope_ext mode 0, freq_scale 1, ext_factor 0, attn_factor 1;
 * engine.cpp:1892-1897): for each head, pairs (x[2i], x[2i+1]) rotate by
 * theta_i = pos * base^(-2i/n_dims).  theta follows ggml's float recurrence
 * theta *= powf(base, -2/n_dims).  x: [n_tok][n_heads][head_dim], in place. */
void orc_rope_normal(float *x, const int32_t *pos, int32_t n_tok, int32_t n_heads,
                     int32_t head_dim, float freq_base) {
    const float theta_scale = powf(freq_base, -2.0f / (float)head_dim);
    for (int32_t t = 0; t < n_tok; ++t) {
        for (int32_t h = 0; h < n_heads; ++h) {
            float *r = x + ((int64_t)t * n_heads + h) * head_dim;
            float theta = (float)pos[t];
            for (int32_t i0 = 0; i0 < head_dim; i0 += 2) {
                const float c = cosf(theta), s = sinf(theta);
                const float x0 = r[i0], x1 = r[i0 + 1];
                r[i0] = x0 * c - x1 * s;
                r[i0 + 1] = x0 * s + x1 * c;
                theta *= theta_scale;
            }
        }
    }
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
