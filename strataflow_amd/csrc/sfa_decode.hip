// sfa_decode.hip - split-K paged decode attention for gfx950 (f16 KV).
//
// Replaces kq = mul_mat(k, q) -> soft_max_ext(kq, 0-mask, scale) -> mul_mat(vt, kq)
// of build_kv_attention (src/model/engine/engine.cpp:1751-1761) for one query
// token per sequence.  One workgroup = (sequence b, kv head, split s); its four
// waves walk 32-position tiles of the split.  Per tile a wave
//   - loads the 32 K rows straight into the A operand of v_mfma_f32_32x32x16_f16
//     (lane = position, 8 consecutive dims per lane, 16-byte loads),
//   - computes S^T = K * Q^T on MFMA.  Q^T's 32 columns hold the g query heads of
//     this kv head replicated (column n is head n % g), so every lane owns the
//     scores of its column's head for 16 positions and the softmax needs no
//     cross-lane traffic except one lane^32 max,
//   - runs an fp32 online softmax in the log2 domain,
//   - keeps P in registers as the B operand of O^T = V^T * P^T (the MFMA output
//     layout of S^T is exactly the B layout P^T needs),
//   - stages the V tile through LDS (coalesced 16-byte loads in, transposed
//     2-byte gathers out) to build the V^T operand.
// Waves merge through LDS; each workgroup stores its (m, l, o) to the
// workspace and a second kernel merges the splits of each (sequence, head) in
// split order, so the result does not depend on scheduling or page placement.
// The kernel boundary is what makes the partials of all eight XCDs visible to
// the merge (no device-scope fences inside a kernel: on this part each one
// writes back a whole XCD L2).
#include "sfa_common.h"

namespace sfa {

struct DecodeParams {
    const uint8_t *k_pages;
    const uint8_t *v_pages;
    const uint8_t *k_cold;
    const uint8_t *v_cold;
    int64_t page_bytes;
    int n_pages;
    int n_cold;
    int page_size;
    int n_head_kv;
    int n_head;
    int row_bytes;
    const float *q;
    float *out;
    const int32_t *page_table;
    int max_pages;
    const int32_t *seq_len;
    const int32_t *kv_lo;
    int n_splits;         // grid.x
    int tiles_per_split;  // minimum tiles per split (host heuristic)
    float scale_log2;     // scale * log2(e)
    float *part;          // [B][Hkv][n_splits][G][HD + 4]
};

constexpr int kDecodeWaves = 4;
// merge kernel block: one thread per dim, at least one full wave
template <int HD>
constexpr int kMergeThreads = HD < 64 ? 64 : HD;

// Active tile range of sequence b: tiles are 32-aligned absolute position
// blocks [32t, 32t+32) intersecting [lo, n_kv).
__device__ inline void seq_tiles(const DecodeParams &p, int b, int &lo, int &n_kv, int &t0,
                                 int &n_tiles, int &tps, int &n_active) {
    n_kv = p.seq_len[b];
    const int cap = p.max_pages * p.page_size;
    if (n_kv > cap) n_kv = cap;
    lo = p.kv_lo ? p.kv_lo[b] : 0;
    if (lo < 0) lo = 0;
    if (n_kv <= lo) {
        t0 = 0; n_tiles = 0; tps = 1; n_active = 0;
        return;
    }
    t0 = lo / kTile;
    n_tiles = (n_kv + kTile - 1) / kTile - t0;
    tps = p.tiles_per_split;
    const int need = (n_tiles + p.n_splits - 1) / p.n_splits;
    if (tps < need) tps = need;
    n_active = (n_tiles + tps - 1) / tps;
}

template <int HD, int G>
__global__ __launch_bounds__(256) void decode_f16_kernel(DecodeParams p) {
    static_assert(HD == 32 || HD == 64 || HD == 128, "head_dim");
    static_assert(G >= 1 && G <= 32 && (32 % G) == 0, "group size");
    constexpr int KC = HD / 16;          // 16-dim k chunks of the QK MFMA
    constexpr int DB = HD / 32;          // 32-dim blocks of the PV MFMA output
    constexpr int VROW = HD * 2 + 16;    // padded LDS row of the V tile (bytes)
    constexpr int CPR = HD / 8;          // 16-byte chunks per row
    constexpr int RPI = kWave / CPR;     // rows per coalesced V load
    constexpr int VIT = kTile / RPI;     // V loads per lane per tile

    __shared__ __attribute__((aligned(16))) uint8_t lds_v[kDecodeWaves][kTile * VROW];
    __shared__ float lds_m[kDecodeWaves][G];
    __shared__ float lds_l[kDecodeWaves][G];
    __shared__ float lds_o[kDecodeWaves][G][HD];

    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 31;   // MFMA column (head replica) / A-operand row
    const int hh = lane >> 5;  // k half
    const int32_t *pt = p.page_table + (int64_t)b * p.max_pages;

    const int Hkv = p.n_head_kv;
    const int64_t col_bytes = (int64_t)Hkv * p.row_bytes;
    uint8_t *vt = lds_v[wave];
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);

    // Issues the K (A operand: row n, dims 16c + 8hh) and V (coalesced: row
    // i*RPI + lane/CPR, chunk lane%CPR) loads of tile t.  The loads do not
    // depend on seq_len: every row of a tile lies in one existing page, and
    // rows outside [lo, n_kv) are masked after arrival (score -inf, V zeroed).
    // Returns false (wave-uniform) when the tile's page id is invalid.
    half8 kf[KC];
    half8 vr[VIT];
    auto issue = [&](int t) -> bool {
        const int pos0 = t * kTile;
        const int lpage = pos0 / p.page_size;
        if (lpage >= p.max_pages) return false;
        const int32_t pid = __builtin_amdgcn_readfirstlane(pt[lpage]);
        const uint8_t *kb = page_base(pid, p.k_pages, p.n_pages, p.k_cold, p.n_cold, p.page_bytes);
        const uint8_t *vb = page_base(pid, p.v_pages, p.n_pages, p.v_cold, p.n_cold, p.page_bytes);
        if (kb == nullptr || vb == nullptr) return false;
        const int64_t off0 = (int64_t)(pos0 - lpage * p.page_size) * col_bytes + (int64_t)kvh * p.row_bytes;
        const uint8_t *kr = kb + off0 + (int64_t)n * col_bytes + 16 * hh;
#pragma unroll
        for (int c = 0; c < KC; ++c) kf[c] = *reinterpret_cast<const half8 *>(kr + 32 * c);
#pragma unroll
        for (int i = 0; i < VIT; ++i) {
            const int r = i * RPI + lane / CPR;
            vr[i] = *reinterpret_cast<const half8 *>(vb + off0 + (int64_t)r * col_bytes + 16 * (lane % CPR));
        }
        return true;
    };

    // The first tile as the host plan places it (kv_lo 0, seq_len within the
    // plan) is fetched before seq_len is known; re-issued below if the guess
    // was wrong.
    const int t_guess = __builtin_amdgcn_readfirstlane(split * p.tiles_per_split + wave);
    bool tile_ok = issue(t_guess);

    int lo, n_kv, t0, n_tiles, tps, n_active;
    seq_tiles(p, b, lo, n_kv, t0, n_tiles, tps, n_active);
    float *out_b = p.out + ((int64_t)b * p.n_head + (int64_t)kvh * G) * HD;
    if (split >= n_active) {
        if (split == 0 && n_active == 0) {
            for (int i = threadIdx.x; i < G * HD; i += blockDim.x) out_b[i] = 0.0f;
        }
        return;
    }
    const int tile_lo = t0 + split * tps;
    int tile_hi = tile_lo + tps;
    if (tile_hi > t0 + n_tiles) tile_hi = t0 + n_tiles;
    int t = tile_lo + wave_u;
    if (t != t_guess) tile_ok = t < tile_hi ? issue(t) : false;

    // Q^T operand: column n -> head kvh*G + n%G, dims 16c + 8hh .. +8, f16
    // (the F16 vec_dot_type conversion ggml applies to src1).  Loaded after
    // the first tile's K/V so both latencies overlap.
    half8 qf[KC];
    {
        const float *qr = p.q + ((int64_t)b * p.n_head + (int64_t)kvh * G + (n % G)) * HD;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const floatx4 *src = reinterpret_cast<const floatx4 *>(qr + 16 * c + 8 * hh);
            const floatx4 x0 = src[0], x1 = src[1];
            half8 h;
            h[0] = (_Float16)x0[0]; h[1] = (_Float16)x0[1]; h[2] = (_Float16)x0[2]; h[3] = (_Float16)x0[3];
            h[4] = (_Float16)x1[0]; h[5] = (_Float16)x1[1]; h[6] = (_Float16)x1[2]; h[7] = (_Float16)x1[3];
            qf[c] = h;
        }
    }

    floatx16 o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) o[d] = floatx16{};
    float m_run = -INFINITY;
    float l_run = 0.0f;

    bool first = true;
    for (; t < tile_hi; t += kDecodeWaves) {
        const int pos0 = t * kTile;
        if (!tile_ok) {  // invalid page id: this tile contributes nothing
            tile_ok = t + kDecodeWaves < tile_hi ? issue(t + kDecodeWaves) : false;
            continue;
        }
        // S^T = K * Q^T, two accumulation chains
        floatx16 s0 = floatx16{}, s1 = floatx16{};
#pragma unroll
        for (int c = 0; c < KC; c += 2) {
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c], qf[c], s0, 0, 0, 0);
            if (c + 1 < KC) s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c + 1], qf[c + 1], s1, 0, 0, 0);
        }
        // V tile into the wave's LDS region; rows outside [lo, n_kv) zeroed
        // (they may hold stale bytes of a page's unused tail)
#pragma unroll
        for (int i = 0; i < VIT; ++i) {
            const int r = i * RPI + lane / CPR;
            const bool ok = pos0 + r >= lo && pos0 + r < n_kv;
            *reinterpret_cast<half8 *>(vt + r * VROW + 16 * (lane % CPR)) = ok ? vr[i] : half8{};
        }
        // registers are free: start the next tile's loads now
        const bool next_ok = t + kDecodeWaves < tile_hi ? issue(t + kDecodeWaves) : false;

        // online softmax (log2 domain); row of register i is tile position
        // 8(i/4) + 4hh + i%4
        float sv[16];
        float mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = 8 * (i >> 2) + 4 * hh + (i & 3);
            const int pp = pos0 + r;
            const bool ok = pp >= lo && pp < n_kv;
            sv[i] = ok ? (s0[i] + s1[i]) * p.scale_log2 : -INFINITY;
            mt = fmaxf(mt, sv[i]);
        }
        mt = fmaxf(mt, xor32(mt));
        const float m_new = fmaxf(m_run, mt);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = exp2f(m_run - m_use);
        float ls = 0.0f;
        half8 pb[2];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float e = exp2f(sv[i] - m_use);
            ls += e;
            pb[i >> 3][i & 7] = (_Float16)e;
        }
        l_run = l_run * alpha + ls;
        m_run = m_new;
        if (!first) {  // o is still zero on the first tile
#pragma unroll
            for (int d = 0; d < DB; ++d) o[d] *= alpha;
        }
        first = false;

        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // V^T operands: k index 8hh + j of chunk kk is tile position
        // 16kk + 8(j/4) + 4hh + j%4 (the rows this lane holds in pb[kk]).
        // ds_read_b64_tr_b16 hands lane i of each 16-lane group column i%4 of
        // the 8-byte chunks addressed by lanes i/4 + 4j (j = 0..3), so lane
        // r of group gq supplies chunk (position 16kk + 8u + 4(gq/2) + r/4,
        // dims 32d + 16(gq%2) + 4(r%4)) and receives its own dim n at the four
        // positions of half u.
        half8 va[2][DB];
        {
            const int gq = lane >> 4, rr = lane & 15;
            const uint8_t *vsrc = vt + (4 * (gq >> 1) + (rr >> 2)) * VROW + 2 * (16 * (gq & 1) + 4 * (rr & 3));
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
                for (int d = 0; d < DB; ++d) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const half4 h = tr16_read(vsrc + (16 * kk + 8 * u) * VROW + 64 * d);
                        va[kk][d][4 * u + 0] = h[0];
                        va[kk][d][4 * u + 1] = h[1];
                        va[kk][d][4 * u + 2] = h[2];
                        va[kk][d][4 * u + 3] = h[3];
                    }
                }
            }
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
            for (int d = 0; d < DB; ++d)
                o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[kk][d], pb[kk], o[d], 0, 0, 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        tile_ok = next_ok;
    }

    // wave partial -> LDS (column n < G is head n; dims of register i of block
    // d are 32d + 8(i/4) + 4hh + i%4)
    l_run += xor32(l_run);
    if (n < G) {
        if (hh == 0) {
            lds_m[wave][n] = m_run;
            lds_l[wave][n] = l_run;
        }
#pragma unroll
        for (int d = 0; d < DB; ++d) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                lds_o[wave][n][32 * d + 8 * (i >> 2) + 4 * hh + (i & 3)] = o[d][i];
            }
        }
    }
    __syncthreads();

    // merge the waves; the workgroup's (m, l, o) per head
    const int64_t head_base = (int64_t)b * Hkv + kvh;
    float *part = p.part + (head_base * p.n_splits + split) * G * (HD + 4);
    for (int idx = threadIdx.x; idx < G * HD; idx += blockDim.x) {
        const int g = idx / HD, d = idx % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) M = fmaxf(M, lds_m[w][g]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) {
            const float mw = lds_m[w][g];
            const float wt = mw == -INFINITY ? 0.0f : exp2f(mw - M);
            L += lds_l[w][g] * wt;
            O += lds_o[w][g][d] * wt;
        }
        if (n_active == 1) {
            out_b[g * HD + d] = L > 0.0f ? O / L : 0.0f;
        } else {
            part[g * (HD + 4) + d] = O;
            if (d == 0) {
                part[g * (HD + 4) + HD] = M;
                part[g * (HD + 4) + HD + 1] = L;
            }
        }
    }
}

// Second pass: out = sum_s o_s * 2^(m_s - M) / sum_s l_s * 2^(m_s - M) over
// the active splits of each (sequence, kv head), in split order.  One
// workgroup per (b, kv head, group head), one thread per dim.
template <int HD, int G>
__global__ __launch_bounds__(kMergeThreads<HD>) void decode_merge_kernel(DecodeParams p) {
    constexpr int CH = 32;  // splits whose loads are in flight together
    const int g = blockIdx.x % G;
    const int kvh = (blockIdx.x / G) % p.n_head_kv;
    const int b = blockIdx.x / (G * p.n_head_kv);
    const int tid = threadIdx.x;
    int lo, n_kv, t0, n_tiles, tps, n_active;
    seq_tiles(p, b, lo, n_kv, t0, n_tiles, tps, n_active);
    if (n_active <= 1 || tid >= HD) return;  // one split: written by the split pass
    const int64_t head_base = (int64_t)b * p.n_head_kv + kvh;
    const float *pbase = p.part + head_base * p.n_splits * G * (HD + 4) + g * (HD + 4);
    const int64_t sstride = (int64_t)G * (HD + 4);
    // log-sum-exp merge in split order, CH splits per round: every load of a
    // round is issued before any is used
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    for (int s0 = 0; s0 < n_active; s0 += CH) {
        float m[CH], l[CH], o[CH];
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int s = s0 + u < n_active ? s0 + u : n_active - 1;
            const float *ps = pbase + s * sstride;
            m[u] = ps[HD];
            l[u] = ps[HD + 1];
            o[u] = ps[tid];
        }
        float mc = M;
#pragma unroll
        for (int u = 0; u < CH; ++u)
            if (s0 + u < n_active) mc = fmaxf(mc, m[u]);
        if (mc == -INFINITY) continue;
        const float a = exp2f(M - mc);  // M == -inf -> 0
        L *= a;
        O *= a;
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const float w = (s0 + u < n_active && m[u] != -INFINITY) ? exp2f(m[u] - mc) : 0.0f;
            L += l[u] * w;
            O += o[u] * w;
        }
        M = mc;
    }
    float *out = p.out + ((int64_t)b * p.n_head + (int64_t)kvh * G + g) * HD;
    out[tid] = L > 0.0f ? O / L : 0.0f;
}

// ---- host side -------------------------------------------------------------

struct SplitPlan {
    int n_splits;
    int tiles_per_split;
};

SplitPlan plan_splits(int B, int Hkv, int max_seq_len) {
    const int tiles = (max_seq_len + kTile - 1) / kTile;
    const int heads = B * Hkv;
    const int wg_target = 1024;
    int S = (wg_target + heads - 1) / heads;
    if (S < 1) S = 1;
    if (S > 256) S = 256;
    int tps = (tiles + S - 1) / S;
    if (tps < kDecodeWaves) tps = kDecodeWaves;
    S = (tiles + tps - 1) / tps;
    if (S < 1) S = 1;
    return SplitPlan{S, tps};
}

size_t decode_workspace_bytes(int B, int Hkv, int G, int HD, int max_seq_len) {
    const SplitPlan sp = plan_splits(B, Hkv, max_seq_len);
    return (size_t)B * Hkv * sp.n_splits * G * (HD + 4) * sizeof(float);
}

// pass bit 1: split-K pass, bit 2: merge pass
template <int HD, int G>
static void launch_f16(const DecodeParams &p, int B, int Hkv, int passes, hipStream_t s) {
    if (passes & 1) {
        dim3 grid(p.n_splits, Hkv, B);
        hipLaunchKernelGGL((decode_f16_kernel<HD, G>), grid, dim3(256), 0, s, p);
    }
    if ((passes & 2) && p.n_splits > 1)
        hipLaunchKernelGGL((decode_merge_kernel<HD, G>), dim3(B * Hkv * G), dim3(kMergeThreads<HD>), 0,
                           s, p);
}

template <int HD>
static int launch_f16_g(const DecodeParams &p, int G, int B, int Hkv, int passes, hipStream_t s) {
    switch (G) {
    case 1: launch_f16<HD, 1>(p, B, Hkv, passes, s); return SFA_OK;
    case 2: launch_f16<HD, 2>(p, B, Hkv, passes, s); return SFA_OK;
    case 4: launch_f16<HD, 4>(p, B, Hkv, passes, s); return SFA_OK;
    case 8: launch_f16<HD, 8>(p, B, Hkv, passes, s); return SFA_OK;
    default: return SFA_ERR_UNSUPPORTED;
    }
}

int decode_launch(const sfa_kv_desc *kv, const float *q, float *out, const int32_t *page_table,
                  int32_t max_pages, const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                  int32_t max_seq_len, float scale, void *workspace, size_t ws_bytes,
                  int passes, hipStream_t stream) {
    const int Hkv = kv->n_head_kv, HD = kv->head_dim, G = kv->n_head / kv->n_head_kv;
    if (B <= 0 || max_seq_len <= 0 || max_pages <= 0) return SFA_ERR_INVALID_ARGUMENT;
    if (q == nullptr || out == nullptr || page_table == nullptr || seq_len == nullptr)
        return SFA_ERR_INVALID_ARGUMENT;
    const size_t need = decode_workspace_bytes(B, Hkv, G, HD, max_seq_len);
    if (workspace == nullptr || ws_bytes < need) return SFA_ERR_INVALID_ARGUMENT;
    const SplitPlan sp = plan_splits(B, Hkv, max_seq_len);

    DecodeParams p;
    p.k_pages = static_cast<const uint8_t *>(kv->k_pages);
    p.v_pages = static_cast<const uint8_t *>(kv->v_pages);
    p.k_cold = static_cast<const uint8_t *>(kv->k_cold);
    p.v_cold = static_cast<const uint8_t *>(kv->v_cold);
    p.row_bytes = row_bytes_of(kv->kv_type, HD);
    p.page_bytes = (int64_t)p.row_bytes * Hkv * kv->page_size;
    p.n_pages = kv->n_pages;
    p.n_cold = kv->n_cold_pages;
    p.page_size = kv->page_size;
    p.n_head_kv = Hkv;
    p.n_head = kv->n_head;
    p.q = q;
    p.out = out;
    p.page_table = page_table;
    p.max_pages = max_pages;
    p.seq_len = seq_len;
    p.kv_lo = kv_lo;
    p.n_splits = sp.n_splits;
    p.tiles_per_split = sp.tiles_per_split;
    p.scale_log2 = scale * 1.4426950408889634f;
    p.part = static_cast<float *>(workspace);

    if (kv->kv_type != SFA_KV_F16) return SFA_ERR_UNSUPPORTED;
    int rc;
    switch (HD) {
    case 32: rc = launch_f16_g<32>(p, G, B, Hkv, passes, stream); break;
    case 64: rc = launch_f16_g<64>(p, G, B, Hkv, passes, stream); break;
    case 128: rc = launch_f16_g<128>(p, G, B, Hkv, passes, stream); break;
    default: return SFA_ERR_UNSUPPORTED;
    }
    if (rc != SFA_OK) return rc;
    return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
}

}  // namespace sfa
