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
    int kv_type;
    const float *q;
    float *out;
    const int32_t *page_table;
    int max_pages;
    const int32_t *seq_len;
    const int32_t *kv_lo;
    int n_splits;         // splits per (sequence, kv head)
    int n_seq;            // B
    int split_row;        // B * n_splits rounded up to a multiple of 8
    int tiles_per_split;  // minimum tiles per split (host heuristic)
    float scale_log2;     // scale * log2(e)
    float *part;          // [B][Hkv][n_splits][G][HD + 4]
};

constexpr int kDecodeWaves = 4;
constexpr int kMaxSplits = 256;  // splits per (sequence, kv head)
constexpr float kRescaleLog2 = 8.0f;  // lazy rescale threshold: P <= 2^8
// merge kernel block: one thread per dim, at least one full wave
template <int HD>
constexpr int kMergeThreads = HD < 64 ? 64 : HD;

// Head of MFMA output register i (rows 8(i/4) + 4hh + i%4, row m is head
// m % g) for the Q8_0 kernel's S = Q * K^T: (4hh + i) % g, a compile-time
// value for g <= 4.
template <int G>
__device__ inline int head_of(int i, int hh) {
    return G <= 4 ? (i % G) : ((4 * hh + i) % G);
}
template <int G>
__device__ inline float head_val(const float (&arr)[G], int i, int hh) {
    if constexpr (G <= 4) {
        return arr[i % G];
    } else {
        return hh ? arr[(4 + i) % G] : arr[i % G];
    }
}

// Workgroup -> (split, kv head, sequence).  The grid is 1-D with rows of
// `split_row` = B * n_splits rounded up to a multiple of 8; workgroup L serves
// kv head L / split_row and (sequence, split) L % split_row.  Workgroups go to
// the eight XCDs round-robin (XCD = L % 8), so every kv head of one (sequence,
// split) lands on the same XCD and shares its L2: Q8_0 rows (136 bytes) of
// neighbouring kv heads share cache lines.  Returns false for padding slots.
__device__ inline bool split_coords(const DecodeParams &p, int &split, int &kvh, int &b) {
    const int L = blockIdx.x;
    kvh = L / p.split_row;
    const int j = L - kvh * p.split_row;
    b = j / p.n_splits;
    split = j - b * p.n_splits;
    return b < p.n_seq;
}

// Active tile range of sequence b: tiles are 32-aligned absolute position
// blocks [32t, 32t+32) intersecting [lo, n_kv).
__device__ inline void seq_tiles_from(const DecodeParams &p, int n_kv_raw, int lo_raw, int &lo,
                                      int &n_kv, int &t0, int &n_tiles, int &tps, int &n_active) {
    n_kv = n_kv_raw;
    const int cap = p.max_pages * p.page_size;
    if (n_kv > cap) n_kv = cap;
    lo = lo_raw;
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
__device__ inline void seq_tiles(const DecodeParams &p, int b, int &lo, int &n_kv, int &t0,
                                 int &n_tiles, int &tps, int &n_active) {
    seq_tiles_from(p, p.seq_len[b], p.kv_lo ? p.kv_lo[b] : 0, lo, n_kv, t0, n_tiles, tps, n_active);
}

// Workgroup epilogue of a split: the four waves' (m, l, O^T) for the g heads
// (MFMA column n < g is head n; register i of dim block d holds dim
// 32d + 8(i/4) + 4hh + i%4) merge through LDS into the split's (m, l, o),
// written to the workspace, or straight to the output when the sequence has
// one split.  `l_run` is the lane's full sum over its tiles.
template <int HD, int G>
__device__ inline void split_epilogue(const floatx16 (&o)[HD / 32], float m_run, float l_run,
                                      float (*lds_m)[G], float (*lds_l)[G], float (*lds_o)[G][HD],
                                      const DecodeParams &p, int b, int kvh, int split, int n_active,
                                      float *out_b, int wave, int n, int hh) {
    constexpr int DB = HD / 32;
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
    const int64_t head_base = (int64_t)b * p.n_head_kv + kvh;
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
            const float wt = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
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

template <int HD, int G>
__global__ __launch_bounds__(256, 2) void decode_f16_kernel(DecodeParams p) {
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
    __shared__ __attribute__((aligned(16))) _Float16 lds_q[G * HD];
    __shared__ float lds_o[kDecodeWaves][G][HD];

    int split, kvh, b;
    if (!split_coords(p, split, kvh, b)) return;
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
    PageWindow pages;
    auto issue = [&](int t) -> bool {
        const int pos0 = t * kTile;
        const int lpage = pos0 / p.page_size;
        if (lpage >= p.max_pages) return false;
        const int32_t pid = pages.get(pt, p.max_pages, lpage, lane);
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

    // Prologue order matters: loads complete in issue order (one vmcnt), so
    // the small loads a wave waits on first (its page-id window, seq_len /
    // kv_lo, its Q chunk) are issued before the first tile's K/V burst; the
    // first tile, as the host plan places it (kv_lo 0, seq_len within the
    // plan), is fetched before seq_len is known and re-issued below if the
    // guess was wrong.
    const int t_guess = __builtin_amdgcn_readfirstlane(split * p.tiles_per_split + wave);
    pages.load(pt, p.max_pages, t_guess * kTile / p.page_size, lane);
    const int n_kv_raw = p.seq_len[b];
    const int lo_raw = p.kv_lo ? p.kv_lo[b] : 0;
    // Q of the g heads rounded to f16 (the F16 vec_dot_type conversion ggml
    // applies to src1), staged once per workgroup in LDS; the Q^T operand of
    // column n (head n % g, dims 16c + 8hh .. +8) is re-read per tile, which
    // keeps 32 registers free.  One 8-element chunk per thread.
    static_assert(G * HD / 8 <= 256, "one Q chunk per thread");
    const bool q_thread = threadIdx.x < G * HD / 8;
    floatx4 qx0 = floatx4{}, qx1 = floatx4{};
    if (q_thread) {
        const floatx4 *qr = reinterpret_cast<const floatx4 *>(
            p.q + ((int64_t)b * p.n_head + (int64_t)kvh * G) * HD);
        qx0 = qr[2 * threadIdx.x];
        qx1 = qr[2 * threadIdx.x + 1];
    }
    bool tile_ok = issue(t_guess);
    if (q_thread) {
        half8 h;
        h[0] = (_Float16)qx0[0]; h[1] = (_Float16)qx0[1]; h[2] = (_Float16)qx0[2]; h[3] = (_Float16)qx0[3];
        h[4] = (_Float16)qx1[0]; h[5] = (_Float16)qx1[1]; h[6] = (_Float16)qx1[2]; h[7] = (_Float16)qx1[3];
        reinterpret_cast<half8 *>(lds_q)[threadIdx.x] = h;
    }

    int lo, n_kv, t0, n_tiles, tps, n_active;
    seq_tiles_from(p, n_kv_raw, lo_raw, lo, n_kv, t0, n_tiles, tps, n_active);
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
    __syncthreads();
    const half8 *qrow = reinterpret_cast<const half8 *>(lds_q) + (n % G) * (HD / 8) + hh;

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
        // S^T = K * Q^T
        floatx16 s0 = floatx16{};
#pragma unroll
        for (int c = 0; c < KC; ++c) s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c], qrow[2 * c], s0, 0, 0, 0);
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
        // 8(i/4) + 4hh + i%4.  Interior tiles need no mask.  The reference
        // max moves only when a score exceeds it by 2^8 (a wave-uniform
        // ballot), so most tiles skip the max exchange and the O rescale;
        // P <= 256 and O, l share the reference, so the result is unchanged.
        const bool interior = pos0 >= lo && pos0 + kTile <= n_kv;
        float sv[16];
        float mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float v = s0[i] * p.scale_log2;
            if (!interior) {
                const int pp = pos0 + 8 * (i >> 2) + 4 * hh + (i & 3);
                v = (pp >= lo && pp < n_kv) ? v : -INFINITY;
            }
            sv[i] = v;
            mt = fmaxf(mt, v);
        }
        if (__any(mt > m_run + kRescaleLog2)) {
            mt = fmaxf(mt, xor32(mt));
            const float m_new = fmaxf(m_run, mt);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // m_run == -inf -> 0
            l_run *= alpha;
            if (!first) {
#pragma unroll
                for (int d = 0; d < DB; ++d) o[d] *= alpha;
            }
            m_run = m_new;
        }
        first = false;
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        float ls = 0.0f;
        half8 pb[2];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float e = __builtin_amdgcn_exp2f(sv[i] - m_use);
            ls += e;
            pb[i >> 3][i & 7] = (_Float16)e;
        }
        l_run += ls;

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
        {
            const int gq = lane >> 4, rr = lane & 15;
            const uint8_t *vsrc = vt + (4 * (gq >> 1) + (rr >> 2)) * VROW + 2 * (16 * (gq & 1) + 4 * (rr & 3));
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                half8 va[DB];
#pragma unroll
                for (int d = 0; d < DB; ++d) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const half4 h = tr16_read(vsrc + (16 * kk + 8 * u) * VROW + 64 * d);
                        va[d][4 * u + 0] = h[0];
                        va[d][4 * u + 1] = h[1];
                        va[d][4 * u + 2] = h[2];
                        va[d][4 * u + 3] = h[3];
                    }
                }
#pragma unroll
                for (int d = 0; d < DB; ++d)
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[d], pb[kk], o[d], 0, 0, 0);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        tile_ok = next_ok;
    }

    l_run += xor32(l_run);
    split_epilogue<HD, G>(o, m_run, l_run, lds_m, lds_l, lds_o, p, b, kvh, split, n_active, out_b,
                          wave, n, hh);
}

// Q8_0 decode (head_dim 64 or 128).  A row is head_dim/32 ggml block_q8_0
// records {fp16 d; int8 q[32]} of 34 bytes; rows start 4-byte aligned (the
// row is 68 or 136 bytes), so block c starts at 2c mod 4 and every byte
// offset below is a compile-time constant modulo 4.
//   - Q is quantised to Q8_0 in the prologue exactly as ggml's mul_mat does
//     for a Q8_0 src0 (vec_dot_type Q8_0: d = amax/127 stored fp16,
//     q = round(x/d)), and S = Q * K^T runs on v_mfma_i32_32x32x32_i8, one
//     MFMA per block, then s += float(sumi) * (d_k * d_q) per block in block
//     order: ggml_vec_dot_q8_0_q8_0's arithmetic.  Rows of the MFMA are the
//     query heads (row m is head m % g), columns are the 32 tile positions,
//     so each lane owns one position and its d_k.
//   - V is dequantised in registers (q * d, rounded to f16) into the same
//     LDS tile layout as the f16 path, and P goes through LDS to the P^T
//     operand; PV is the f16 path's O^T = V^T * P^T.
template <int HD, int G>
__global__ __launch_bounds__(256, G <= 4 ? 2 : 1) void decode_q8_kernel(DecodeParams p) {
    static_assert(HD == 64 || HD == 128, "head_dim");
    static_assert(G >= 1 && G <= 8 && (8 % G) == 0, "group size");
    constexpr int NB = HD / 32;          // blocks per row
    constexpr int DB = HD / 32;          // 32-dim blocks of the PV output
    constexpr int VROW = HD * 2 + 16;    // padded LDS row of the f16 V tile
    constexpr int VBL = NB / 2;          // V blocks dequantised per lane

    __shared__ __attribute__((aligned(16))) uint8_t lds_v[kDecodeWaves][kTile * VROW];
    __shared__ __attribute__((aligned(16))) _Float16 lds_p[kDecodeWaves][G][kTile];
    __shared__ float lds_dq[G][NB];
    __shared__ intx4 lds_qa[G][NB][2];
    __shared__ float lds_m[kDecodeWaves][G];
    __shared__ float lds_l[kDecodeWaves][G];
    __shared__ float lds_o[kDecodeWaves][G][HD];

    int split, kvh, b;
    if (!split_coords(p, split, kvh, b)) return;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 31;   // tile position (QK) / MFMA column (PV)
    const int hh = lane >> 5;
    const int32_t *pt = p.page_table + (int64_t)b * p.max_pages;
    const int Hkv = p.n_head_kv;
    const int64_t col_bytes = (int64_t)Hkv * p.row_bytes;
    uint8_t *vt = lds_v[wave];
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);

    // K operand of block c for lane (row n, half hh): quants 16hh..16hh+15 of
    // block c and the block scale; V: blocks VBL*hh .. of row n.  All kept
    // as loaded (arithmetic on them at issue time would make the wave wait
    // for the prefetched tile right where it issues it); the byte alignment
    // of even K blocks happens when the tile is consumed.  Two such register
    // sets (tiles A and B) alternate: the loop is unrolled by two so each set
    // is loaded and consumed in place, never copied (a copy of a register
    // still being loaded would wait for the load).
    struct Raw {
        intx4 kw[NB];                // 16 bytes at 34c + 16hh (c even) or 34c + 2 + 16hh (c odd)
        uint32_t kx[NB / 2 > 0 ? NB / 2 : 1];  // the dword after them (even c)
        uint32_t kd[NB];             // dword holding d_k of block c
        uint32_t vw[VBL][9];         // the 36 bytes around each V block
    };
    PageWindow pages;
    auto issue = [&](int t, Raw &r) -> bool {
        const int pos0 = t * kTile;
        const int lpage = pos0 / p.page_size;
        if (lpage >= p.max_pages) return false;
        const int32_t pid = pages.get(pt, p.max_pages, lpage, lane);
        const uint8_t *kb = page_base(pid, p.k_pages, p.n_pages, p.k_cold, p.n_cold, p.page_bytes);
        const uint8_t *vb = page_base(pid, p.v_pages, p.n_pages, p.v_cold, p.n_cold, p.page_bytes);
        if (kb == nullptr || vb == nullptr) return false;
        const int64_t off = (int64_t)(pos0 - lpage * p.page_size + n) * col_bytes + (int64_t)kvh * p.row_bytes;
        const uint8_t *kr = kb + off;
        const uint8_t *vr = vb + off;
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            if ((c & 1) == 0) {
                // block at 34c (4-aligned): quants of half hh start 2 bytes
                // into the dword at 34c + 16hh; d is the low half at 34c
                const uint8_t *w = kr + 34 * c + 16 * hh;
                r.kw[c] = load16_a4(w);
                r.kx[c / 2] = load4_a4(w + 16);
                r.kd[c] = load4_a4(kr + 34 * c);
            } else {
                // block at 34c (2 mod 4): quants 4-aligned; d is the high half
                // of the dword at 34c - 2
                r.kw[c] = load16_a4(kr + 34 * c + 2 + 16 * hh);
                r.kd[c] = load4_a4(kr + 34 * c - 2);
            }
        }
#pragma unroll
        for (int u = 0; u < VBL; ++u) {
            const int c = VBL * hh + u;
            // 9 dwords from the 4-aligned address at or 2 bytes below the block
            const uint8_t *w = vr + 34 * c - (c & 1) * 2;
            const intx4 a0 = load16_a4(w), a1 = load16_a4(w + 16);
#pragma unroll
            for (int j = 0; j < 4; ++j) { r.vw[u][j] = (uint32_t)a0[j]; r.vw[u][4 + j] = (uint32_t)a1[j]; }
            r.vw[u][8] = load4_a4(w + 32);
        }
        return true;
    };

    // Prologue order as in the f16 kernel: page-id window, seq_len / kv_lo
    // and the lane's Q values are issued before the first tile's K/V burst.
    const int t_guess = __builtin_amdgcn_readfirstlane(split * p.tiles_per_split + wave);
    pages.load(pt, p.max_pages, t_guess * kTile / p.page_size, lane);
    const int n_kv_raw = p.seq_len[b];
    const int lo_raw = p.kv_lo ? p.kv_lo[b] : 0;
    const int hq = n % G;
    floatx4 qraw[NB][4];
    {
        const float *qr = p.q + ((int64_t)b * p.n_head + (int64_t)kvh * G + hq) * HD;
#pragma unroll
        for (int c = 0; c < NB; ++c)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                qraw[c][j] = reinterpret_cast<const floatx4 *>(qr + 32 * c + 16 * hh)[j];
    }
    Raw ra, rb;
    bool ok_a = issue(t_guess, ra);

    // Q8_0 of Q, the MFMA A operand: lane row m = n is head n % G, block c,
    // elements 16hh .. 16hh+15; staged in LDS (read per tile, which keeps 16
    // registers for the tile pipeline).
    {
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            float x[16];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const floatx4 v4 = qraw[c][j];
                x[4 * j] = v4[0]; x[4 * j + 1] = v4[1]; x[4 * j + 2] = v4[2]; x[4 * j + 3] = v4[3];
            }
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) amax = fmaxf(amax, fabsf(x[j]));
            amax = fmaxf(amax, xor32(amax));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int q0 = (int)roundf(x[4 * j] * id), q1 = (int)roundf(x[4 * j + 1] * id);
                const int q2 = (int)roundf(x[4 * j + 2] * id), q3 = (int)roundf(x[4 * j + 3] * id);
                const int w4 = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | ((int)((unsigned)q3 << 24));
                if (wave == 0 && n < G) lds_qa[n][c][hh][j] = w4;
            }
            if (wave == 0 && hh == 0 && n < G) lds_dq[n][c] = (float)(_Float16)d;
        }
    }

    int lo, n_kv, t0, n_tiles, tps, n_active;
    seq_tiles_from(p, n_kv_raw, lo_raw, lo, n_kv, t0, n_tiles, tps, n_active);
    float *out_b = p.out + ((int64_t)b * p.n_head + (int64_t)kvh * G) * HD;
    if (split >= n_active) {
        if (split == 0 && n_active == 0) {
            for (int i = threadIdx.x; i < G * HD; i += blockDim.x) out_b[i] = 0.0f;
        }
        return;
    }
    __syncthreads();  // lds_qa, lds_dq (d_q of the heads of output rows i = 0..3,
                      // i.e. rows 4hh + i, head (4hh + i) % G, read per tile)

    const int tile_lo = t0 + split * tps;
    int tile_hi = tile_lo + tps;
    if (tile_hi > t0 + n_tiles) tile_hi = t0 + n_tiles;
    int t = tile_lo + wave_u;
    if (t != t_guess) ok_a = t < tile_hi ? issue(t, ra) : false;

    floatx16 o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) o[d] = floatx16{};
    float m_run[G], l_run[G], alpha_h[G];
#pragma unroll
    for (int h = 0; h < G; ++h) { m_run[h] = -INFINITY; l_run[h] = 0.0f; alpha_h[h] = 1.0f; }
    bool first = true;

    // part 1 of a tile: the scores and the V tile (the raw registers are dead
    // after it); part 2: softmax and PV
    auto consume1 = [&](int t, const Raw &r, float (&sv)[4]) {
        const int pos0 = t * kTile;
        const bool row_ok = pos0 + n >= lo && pos0 + n < n_kv;
        const bool interior = pos0 >= lo && pos0 + kTile <= n_kv;
        // S = Q8 * K8^T per block, scaled in block order
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = 0.0f;
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            intx4 kq = r.kw[c];
            if ((c & 1) == 0) {
                const uint32_t *x = reinterpret_cast<const uint32_t *>(&r.kw[c]);
                kq[0] = (int)__builtin_amdgcn_alignbyte(x[1], x[0], 2);
                kq[1] = (int)__builtin_amdgcn_alignbyte(x[2], x[1], 2);
                kq[2] = (int)__builtin_amdgcn_alignbyte(x[3], x[2], 2);
                kq[3] = (int)__builtin_amdgcn_alignbyte(r.kx[c / 2], x[3], 2);
            }
            const intx16 acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(lds_qa[n % G][c][hh], kq, intx16{}, 0, 0, 0);
            const uint32_t dbits = (c & 1) ? (r.kd[c] >> 16) : (r.kd[c] & 0xffffu);
            const float dk = (float)__builtin_bit_cast(_Float16, (uint16_t)dbits);
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[i] += (float)acc[i] * (dk * lds_dq[(4 * hh + i) % G][c]);
            // one block's 16-register accumulator live at a time
            __builtin_amdgcn_sched_barrier(0);
        }
        // V blocks: dequantise into the f16 LDS tile (rows outside [lo, n_kv) zeroed)
#pragma unroll
        for (int u = 0; u < VBL; ++u) {
            const int c = VBL * hh + u;
            uint32_t q[8];
            uint32_t dbits;
            if ((c & 1) == 0) {
                dbits = r.vw[u][0] & 0xffffu;
#pragma unroll
                for (int j = 0; j < 8; ++j) q[j] = __builtin_amdgcn_alignbyte(r.vw[u][j + 1], r.vw[u][j], 2);
            } else {
                dbits = r.vw[u][0] >> 16;
#pragma unroll
                for (int j = 0; j < 8; ++j) q[j] = r.vw[u][j + 1];
            }
            // q * d rounded to f16 on packed halves: byte b of a dword becomes
            // the f16 1024 + (b ^ 0x80) (exponent byte 0x64 above it), minus
            // 1152 gives q exactly, and one f16 multiply rounds q * d once,
            // the same value as rounding the (exact) f32 product.  Rows
            // outside [lo, n_kv) use d = 0 (their bytes may be anything).
            const _Float16 dv = (interior || row_ok) ? __builtin_bit_cast(_Float16, (uint16_t)dbits) : (_Float16)0.0f;
            const half2v dv2 = {dv, dv};
            const half2v bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
            half8 h[4];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t x = q[j] ^ 0x80808080u;
                const half2v lo = (__builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)) + bias) * dv2;
                const half2v hi = (__builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)) + bias) * dv2;
                h[j >> 1][4 * (j & 1) + 0] = lo[0];
                h[j >> 1][4 * (j & 1) + 1] = lo[1];
                h[j >> 1][4 * (j & 1) + 2] = hi[0];
                h[j >> 1][4 * (j & 1) + 3] = hi[1];
            }
#pragma unroll
            for (int k = 0; k < 4; ++k)
                *reinterpret_cast<half8 *>(vt + n * VROW + 64 * c + 16 * k) = h[k];
        }
    };
    auto consume2 = [&](int t, float (&sv)[4]) {
        const int pos0 = t * kTile;
        const bool row_ok = pos0 + n >= lo && pos0 + n < n_kv;
        const bool interior = pos0 >= lo && pos0 + kTile <= n_kv;

        // online softmax per head (log2 domain); this lane holds position n
        // for the heads (4hh + i) % G of registers i = 0..3 (i % G when
        // g <= 4).  Lazy reference max as in the f16 path.
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = (interior || row_ok) ? sv[i] * p.scale_log2 : -INFINITY;
        bool exceed = false;
#pragma unroll
        for (int i = 0; i < 4; ++i) exceed |= sv[i] > head_val(m_run, i, hh) + kRescaleLog2;
        if (__any(exceed)) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float mt = -INFINITY;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (head_of<G>(i, hh) == h) mt = fmaxf(mt, sv[i]);
#pragma unroll
                for (int off = 1; off < 64; off <<= 1) mt = fmaxf(mt, __shfl_xor(mt, off, 64));
                const float m_new = fmaxf(m_run[h], mt);
                const float alpha = __builtin_amdgcn_exp2f(m_run[h] - m_new);  // m_run == -inf -> 0
                l_run[h] *= alpha;
                alpha_h[h] = alpha;
                m_run[h] = m_new;
            }
            if (!first) {
                float a = alpha_h[0];
#pragma unroll
                for (int h = 1; h < G; ++h) a = (n % G == h) ? alpha_h[h] : a;
#pragma unroll
                for (int d = 0; d < DB; ++d) o[d] *= a;
            }
        }
        first = false;
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float mr = head_val(m_run, i, hh);
            pv[i] = __builtin_amdgcn_exp2f(sv[i] - (mr == -INFINITY ? 0.0f : mr));
        }
        // each (head, position) counted once over the wave: for g <= 4 both
        // halves hold every head, so only half 0 and i < g count
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (G == 8) {
                if (hh) l_run[4 + i] += pv[i]; else l_run[i] += pv[i];
            } else if (i < G && hh == 0) {
                l_run[i] += pv[i];
            }
        }
        // P -> LDS [head][position]
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i < G || G == 8) lds_p[wave][head_of<G>(i, hh)][n] = (_Float16)pv[i];
        }

        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // P^T operand (column n -> head n % G): positions 16kk + 4hh + 0..3
        // and 16kk + 8 + 4hh + 0..3, the k order the V^T operand uses
        half8 pb[2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const _Float16 *pr = &lds_p[wave][n % G][16 * kk + 4 * hh];
            const half4 a0 = *reinterpret_cast<const half4 *>(pr);
            const half4 a1 = *reinterpret_cast<const half4 *>(pr + 8);
#pragma unroll
            for (int j = 0; j < 4; ++j) { pb[kk][j] = a0[j]; pb[kk][4 + j] = a1[j]; }
        }
        {
            const int gq = lane >> 4, rr = lane & 15;
            const uint8_t *vsrc = vt + (4 * (gq >> 1) + (rr >> 2)) * VROW + 2 * (16 * (gq & 1) + 4 * (rr & 3));
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                half8 va[DB];
#pragma unroll
                for (int d = 0; d < DB; ++d) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const half4 h = tr16_read(vsrc + (16 * kk + 8 * u) * VROW + 64 * d);
                        va[d][4 * u + 0] = h[0];
                        va[d][4 * u + 1] = h[1];
                        va[d][4 * u + 2] = h[2];
                        va[d][4 * u + 3] = h[3];
                    }
                }
#pragma unroll
                for (int d = 0; d < DB; ++d)
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[d], pb[kk], o[d], 0, 0, 0);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    // tiles t (set A) and t + 4 (set B) per trip; the next tile is issued
    // into the other set as soon as a tile's raw registers are consumed, so
    // one tile is in flight while the current one finishes
    float sv[4];
    for (; t < tile_hi; t += 2 * kDecodeWaves) {
        const int t1 = t + kDecodeWaves;
        if (ok_a) consume1(t, ra, sv);
        const bool ok_b = t1 < tile_hi ? issue(t1, rb) : false;
        if (ok_a) consume2(t, sv);
        if (t1 >= tile_hi) break;
        if (ok_b) consume1(t1, rb, sv);
        ok_a = t1 + kDecodeWaves < tile_hi ? issue(t1 + kDecodeWaves, ra) : false;
        if (ok_b) consume2(t1, sv);
    }

    // per-head sums over all 64 lanes (each position counted once per head)
    float Lh[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float v = l_run[h];
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
        Lh[h] = v;
    }
    float m_col = m_run[0], l_col = Lh[0];
#pragma unroll
    for (int h = 1; h < G; ++h)
        if (n % G == h) { m_col = m_run[h]; l_col = Lh[h]; }
    split_epilogue<HD, G>(o, m_col, l_col, lds_m, lds_l, lds_o, p, b, kvh, split, n_active, out_b,
                          wave, n, hh);
}

// Second pass: out = sum_s o_s * 2^(m_s - M) / sum_s l_s * 2^(m_s - M) over
// the active splits of each (sequence, kv head), M the largest m_s.  One
// workgroup per (b, kv head, group head), one thread per dim.  Every load of
// the first 64 splits (the lane-parallel (m, l) of all splits and this dim's
// o_s) is issued before seq_len is read, so the kernel waits on memory once
// for up to 64 splits; split indices past n_splits are clamped (the loads
// stay inside the workspace) and their weights are zero.  The code is
// branch-free straight-line work: the pass is latency-bound and each taken
// branch or instruction-cache miss adds to it.
template <int HD, int G>
__global__ __launch_bounds__(kMergeThreads<HD>) void decode_merge_kernel(DecodeParams p) {
    constexpr int CH = kWave;                       // splits per round
    constexpr int RMAX = (kMaxSplits + CH - 1) / CH;  // (m, l) registers per lane
    const int g = blockIdx.x % G;
    const int kvh = (blockIdx.x / G) % p.n_head_kv;
    const int b = blockIdx.x / (G * p.n_head_kv);
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int d = tid < HD ? tid : HD - 1;  // threads past HD (HD < 64) only load (m, l)
    const int64_t head_base = (int64_t)b * p.n_head_kv + kvh;
    const float *pg = p.part + head_base * p.n_splits * G * (HD + 4) + g * (HD + 4);
    const int sstride = G * (HD + 4);
    const int S = p.n_splits;

    float o[CH];
    auto load_round = [&](int s0) {
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const float *row = pg + (int64_t)min(s0 + u, S - 1) * sstride;  // wave-uniform
            o[u] = row[d];
        }
    };
    load_round(0);
    float mv[RMAX], lv[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
        const int s = min(CH * r + lane, S - 1);
        mv[r] = pg[s * sstride + HD];
        lv[r] = pg[s * sstride + HD + 1];
    }
    int lo, n_kv, t0, n_tiles, tps, n_active;
    seq_tiles(p, b, lo, n_kv, t0, n_tiles, tps, n_active);
    if (n_active <= 1) return;  // one split: written by the split pass

    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
        mv[r] = CH * r + lane < n_active ? mv[r] : -INFINITY;
        mx = fmaxf(mx, mv[r]);
    }
    const float M = wave_max(mx);
    float w[RMAX], lsum = 0.0f;
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
        w[r] = mv[r] != -INFINITY ? __builtin_amdgcn_exp2f(mv[r] - M) : 0.0f;
        lsum += w[r] != 0.0f ? lv[r] * w[r] : 0.0f;
    }
    const float L = wave_sum(lsum);

    // rows of splits >= n_active are not written by this call: their weight
    // is zero and their (possibly stale) values are never multiplied
    float O = 0.0f;
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
        if (CH * r >= n_active) break;
        if (r > 0) load_round(CH * r);
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const float wt = lane_val(w[r], u);
            O = wt != 0.0f ? fmaf(o[u], wt, O) : O;
        }
    }
    if (tid < HD) {
        float *out = p.out + ((int64_t)b * p.n_head + (int64_t)kvh * G + g) * HD;
        out[tid] = L > 0.0f ? O / L : 0.0f;
    }
}

// ---- host side -------------------------------------------------------------

struct SplitPlan {
    int n_splits;
    int tiles_per_split;
};

SplitPlan plan_splits(int B, int Hkv, int max_seq_len) {
    const int tiles = (max_seq_len + kTile - 1) / kTile;
    const int heads = B * Hkv;
    // one round of workgroups: two 4-wave workgroups per CU (two waves per
    // SIMD at these register footprints) over 256 CUs; longer contexts give
    // each wave more tiles, whose loads the tile loop prefetches one ahead
    const int wg_target = 512;
    int S = (wg_target + heads - 1) / heads;
    if (S < 1) S = 1;
    if (S > kMaxSplits) S = kMaxSplits;
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
        dim3 grid(p.split_row * Hkv);
        if (p.kv_type == SFA_KV_Q8_0) {
            if constexpr (HD >= 64 && G <= 8)
                hipLaunchKernelGGL((decode_q8_kernel<HD, G>), grid, dim3(256), 0, s, p);
        } else {
            hipLaunchKernelGGL((decode_f16_kernel<HD, G>), grid, dim3(256), 0, s, p);
        }
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
    p.n_seq = B;
    p.split_row = (B * sp.n_splits + 7) / 8 * 8;
    p.tiles_per_split = sp.tiles_per_split;
    p.scale_log2 = scale * 1.4426950408889634f;
    p.part = static_cast<float *>(workspace);

    p.kv_type = kv->kv_type;
    if (kv->kv_type != SFA_KV_F16 && kv->kv_type != SFA_KV_Q8_0) return SFA_ERR_UNSUPPORTED;
    if (kv->kv_type == SFA_KV_Q8_0 && HD < 64) return SFA_ERR_UNSUPPORTED;
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
