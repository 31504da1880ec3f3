// sfa_prefill.hip - chunked causal prefill attention over the paged f16 cache.
//
// The same op sequence as build_kv_attention (src/model/engine/engine.cpp:
// 1751-1761) for T query tokens of one sequence, with llama.cpp's causal mask
// (-INF where kv position > query position).  The reference engine itself only
// issues T == 1 (engine.cpp:2796); this is the chunked extension.
//
// One workgroup = (query block, kv head); its 128 MFMA rows are the g query
// heads of that kv head times 128/g query tokens, so every K/V tile read from
// the cache serves all g heads.  Per 64-position tile the four waves share a K
// tile and a V tile in LDS; each wave computes S^T = K * Q^T on
// v_mfma_f32_32x32x16_f16 (K rows from LDS, Q^T in registers), runs an fp32
// online softmax in the log2 domain with the lane owning its query row, and
// accumulates O^T += V^T * P^T (P^T straight from the S^T accumulator layout).
// Tiles above the block's last query position are never visited.
#include "sfa_common.h"

namespace sfa {

struct PrefillParams {
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
    const float *q;
    float *out;
    const int32_t *page_table;
    int max_pages;
    int q_pos0;
    int T;
    int kv_lo;
    int n_qblk;
    float scale_log2;
};

constexpr int kPBN = 64;           // positions per prefill tile
constexpr float kRescaleLog2 = 8.0f;  // lazy rescale threshold (P <= 2^8)
template <int N>
struct IntC {  // a compile-time int passed to a generic lambda
    static constexpr int value = N;
};
struct HalfPairs {
    half2v v[4];  // the four dwords of a half8
};

// The workgroup's query block and this lane's query row.  Workgroup L serves
// kv head L % Hkv and query block n_qblk - 1 - L / Hkv (heaviest blocks first);
// its 128 MFMA columns (4 waves x 32) are the g heads of that kv head times
// 128/g tokens, column n of wave w being row 32w + n.
struct PrefillRows {
    int kvh, tq, h, qp;   // this lane's row: token, query head, absolute position
    bool row_ok;          // tq < T
    int q_lo, kv_hi, lo;  // block's first query position, last attended position, window start
    int tile0, tile1;     // 64-position tiles of the block's kv range (inclusive)
    bool block_full;      // every row of the block is < T
};
template <int G>
__device__ __attribute__((always_inline)) inline PrefillRows prefill_rows(const PrefillParams &p, int wave, int n) {
    constexpr int QB = 128 / G;  // query tokens per workgroup
    PrefillRows r;
    r.kvh = (int)blockIdx.x % p.n_head_kv;
    const int qblk = p.n_qblk - 1 - (int)blockIdx.x / p.n_head_kv;
    const int rho = wave * 32 + n;
    r.tq = qblk * QB + rho % QB;
    r.row_ok = r.tq < p.T;
    r.h = r.kvh * G + rho / QB;
    r.qp = p.q_pos0 + r.tq;
    const int first_tok = qblk * QB;
    int last_tok = first_tok + QB - 1;
    if (last_tok > p.T - 1) last_tok = p.T - 1;
    r.kv_hi = p.q_pos0 + last_tok;
    r.q_lo = p.q_pos0 + first_tok;
    r.lo = p.kv_lo > 0 ? p.kv_lo : 0;
    r.tile0 = r.lo / kPBN;
    r.tile1 = r.kv_hi / kPBN;
    r.block_full = (qblk + 1) * QB <= p.T;
    return r;
}

// A tile needs masking where it meets the window start, the diagonal or rows
// past T, or when its page was invalid (wave-uniform).
__device__ __attribute__((always_inline)) inline bool prefill_edge(const PrefillRows &r, int pos0, bool dead) {
    return dead || pos0 < r.lo || pos0 + kPBN - 1 > r.q_lo || !r.block_full;
}

// Scores of positions outside [lo, qp] (all of them for a dead tile or a row
// past T) -> -inf; register i of block pb is position pos0 + 32pb + 8(i/4) +
// 4hh + i%4.
__device__ __attribute__((always_inline)) inline void prefill_mask(floatx16 (&s)[2], const PrefillRows &r, int pos0, int hh, bool dead) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int kp = pos0 + 32 * pb + 8 * (i >> 2) + 4 * hh + (i & 3);
            s[pb][i] = (!dead && r.row_ok && kp >= r.lo && kp <= r.qp) ? s[pb][i] : -INFINITY;
        }
    }
}

// Row max of the tile (both 32-position blocks, both lane halves) in the log2
// domain, with the lazy reference: m_run moves only when the tile max exceeds
// it by 2^8 (P stays <= 256; exact since O and l share the reference).
// Returns the factor O and l are rescaled by (1 when the reference stays).
__device__ __attribute__((always_inline)) inline float prefill_rescale(const floatx16 (&s)[2], float scale_log2, float &m_run) {
    // a v_max3 tree (4 levels, 16 instructions) rather than a 32-long chain
    float a[11], b[4];
#pragma unroll
    for (int i = 0; i < 10; ++i) {
        const int k = 3 * i;
        a[i] = max3_raw(s[k >> 4][k & 15], s[(k + 1) >> 4][(k + 1) & 15], s[(k + 2) >> 4][(k + 2) & 15]);
    }
    a[10] = max3_raw(s[1][14], s[1][15], s[1][15]);
#pragma unroll
    for (int i = 0; i < 3; ++i) b[i] = max3_raw(a[3 * i], a[3 * i + 1], a[3 * i + 2]);
    b[3] = max3_raw(a[9], a[10], a[10]);
    const float lane_max = max3_raw(max3_raw(b[0], b[1], b[2]), b[3], b[3]);
    // the other half of the row: lanes l and l ^ 32 hold the same query row
    float lo, hi;
    swap_halves(lane_max, lo, hi);
    const float mt = max3_raw(lo, hi, hi) * scale_log2;
    float alpha = 1.0f;
    if (mt > m_run + kRescaleLog2) {
        alpha = __builtin_amdgcn_exp2f(m_run - mt);  // m_run == -inf -> 0
        m_run = mt;
    }
    return alpha;
}

// O^T / l to the output row of this lane (register i of dim block d is dim
// 32d + 8(i/4) + 4hh + i%4); l is the lane's half of the row sum.
template <int HD>
__device__ __attribute__((always_inline)) inline void prefill_write(const floatx16 (&o)[HD / 32], float l_run, const PrefillRows &r,
                                     const PrefillParams &p, int hh) {
    l_run += xor32(l_run);
    if (!r.row_ok) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    float *orow = p.out + ((int64_t)r.tq * p.n_head + r.h) * HD;
#pragma unroll
    for (int d = 0; d < HD / 32; ++d) {
#pragma unroll
        for (int i = 0; i < 16; ++i) orow[32 * d + 8 * (i >> 2) + 4 * hh + (i & 3)] = o[d][i] * inv;
    }
}

// LDS address (32 bits) of a pointer into shared memory.
__device__ inline uint32_t lds_u32(const void *ptr) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)(ptr);
}

// One 16-byte chunk per lane from a buffer resource straight into LDS
// (buffer_load_dwordx4 ... lds): the instruction fills the 1 KB block at
// lds_addr (wave-uniform), lane l its chunk l, from byte voff of the resource
// (past num_records a lane reads zeros).  Issued from asm, so the compiler
// does not count these loads: its own LDS reads of the other buffers do not
// wait for them, and the caller waits with s_waitcnt vmcnt before the
// barrier that publishes the tile.  M0 holds the instruction's LDS base; it
// is declared clobbered (the kernels that call this use M0 for nothing else,
// and the compiler sets M0 itself before any use of its own).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // "m0 is reserved": intended, as above
__device__ inline void dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_addr, int voff) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen lds"
        :
        : "s"(lds_addr), "v"(voff), "s"(rsrc)
        : "memory", "m0");
}
#pragma clang diagnostic pop

// Buffer resources of one 64-position tile's rows of one kv head in the K and
// V pools.  A resource starts at the tile's first row and ends after its row
// at kv_hi, so rows past kv_hi (a page's unwritten tail may hold any bytes),
// tiles of an invalid page and tiles past the block's range read as zeros.
struct TileSrc {
    __amdgpu_buffer_rsrc_t k, v;
    bool ok;  // a valid page (wave-uniform)
};

template <int HD, int G>
__global__ __launch_bounds__(256, 2) void prefill_f16_kernel(PrefillParams p) {
    constexpr int KC = HD / 16;          // 16-dim K operand steps per row
    constexpr int DB = HD / 32;          // 32-dim output blocks
    constexpr int RB = HD * 2;           // f16 row bytes
    constexpr int CPR = RB / 16;         // 16-byte chunks per row
    constexpr int TB = kPBN * RB;        // tile bytes (K or V)
    constexpr int IPW = TB / 4096;       // 1 KB DMA instructions per wave per tile and tensor
    constexpr int RPI = 1024 / RB;       // rows per 1 KB block
    constexpr int NG = RB / 64;          // 64-byte groups per row
    constexpr int RP = 256 / RB > 0 ? 256 / RB : 1;  // rows per 256 bytes (all LDS banks)
    static_assert(TB % 4096 == 0 && 1024 % RB == 0, "tile split over four waves");

    // Two K and two V tiles, filled straight from the page.  K's 16-byte chunk
    // c of row r sits at chunk c ^ (r % CPR): the 16 rows one 16-lane slice
    // of an MFMA operand read touches cover all 64 LDS banks.  V's 64-byte
    // group j of row r sits at group j ^ ((r / RP) % NG): the four rows a
    // 32-lane half of a transposed read covers (64 bytes each) fall in
    // disjoint banks.
    __shared__ __attribute__((aligned(16))) uint8_t lds_k[2][TB];
    __shared__ __attribute__((aligned(16))) uint8_t lds_v[2][TB];

    // 1-D grid: workgroup L serves kv head L % Hkv and query block
    // n_qblk - 1 - L / Hkv (heaviest blocks first).  Workgroups go to the
    // eight XCDs round-robin (XCD = L % 8), so with Hkv a multiple of 8 every
    // query block of one kv head runs on one XCD and that head's K/V stays in
    // its L2 (each tile is re-read by every query block of the head).
    const int kvh = (int)blockIdx.x % p.n_head_kv;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31;
    const int hh = lane >> 5;
    const int col_bytes = p.n_head_kv * RB;

    // this lane's query row (MFMA column n): head g of the group, token tq
    const PrefillRows rows = prefill_rows<G>(p, wave, n);
    const bool row_ok = rows.row_ok;
    const int tq = rows.tq, h = rows.h;
    const int kv_hi = rows.kv_hi, tile0 = rows.tile0, tile1 = rows.tile1;

    // DMA lane offsets: block i of this wave holds rows (IPW wave + i) RPI +
    // lane / CPR; the lane fills LDS chunk lane % CPR of its row, which holds
    // the row's chunk (lane % CPR) ^ swizzle.
    int k_off[IPW], v_off[IPW];
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
        const int r = (IPW * wave + i) * RPI + lane / CPR, cp = lane % CPR;
        k_off[i] = r * col_bytes + 16 * (cp ^ (r % CPR));
        v_off[i] = r * col_bytes + 16 * (cp ^ (4 * ((r / RP) % NG)));
    }
    const uint32_t lds_k0 = lds_u32(lds_k[0]) + 1024u * IPW * wave;
    const uint32_t lds_v0 = lds_u32(lds_v[0]) + 1024u * IPW * wave;

    // Page ids of 64 logical pages from the block's first one, one per lane:
    // a tile's id is a v_readlane instead of a dependent scalar load ahead of
    // every tile's loads.  The window moves (one reload) only when the block's
    // kv range spans more than 64 pages.
    PageWindow win;
    win.load(p.page_table, p.max_pages, tile0 * kPBN / p.page_size, lane);
    // Q of this lane's row (rows past T read row 0, zeroed below): its loads
    // go out right after the page-id window's, so they overlap the wait for
    // the window that the first tiles' loads need
    floatx4 qx[KC][2];
    {
        const float *qr = p.q + ((int64_t)(row_ok ? tq : 0) * p.n_head + h) * HD;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const floatx4 *src = reinterpret_cast<const floatx4 *>(qr + 16 * c + 8 * hh);
            qx[c][0] = src[0];
            qx[c][1] = src[1];
        }
    }
    // (logical page, first row in it) of tile t, advanced one tile per call
    // (page_size is a multiple of the tile) instead of a division per tile
    struct TilePos {
        int lp, row;
    };
    auto advance = [&](TilePos &tp) {
        tp.row += kPBN;
        const bool wrap = tp.row == p.page_size;
        tp.lp += wrap ? 1 : 0;
        tp.row = wrap ? 0 : tp.row;
    };
    // the K and V pages of logical page lp (nullptr both for an invalid id),
    // resolved once per page rather than once per tile (the scalar unit is
    // shared by the CU's eight waves)
    struct PageSrc {
        const uint8_t *kb, *vb;
    };
    auto page_src = [&](int lp) -> PageSrc {
        const int32_t pid = lp < p.max_pages ? win.get(p.page_table, p.max_pages, lp, lane) : -1;
        PageSrc ps;
        ps.kb = page_base(pid, p.k_pages, p.n_pages, p.k_cold, p.n_cold, p.page_bytes);
        ps.vb = page_base(pid, p.v_pages, p.n_pages, p.v_cold, p.n_cold, p.page_bytes);
        if (ps.kb == nullptr || ps.vb == nullptr) ps.kb = ps.vb = nullptr;
        return ps;
    };
    auto tile_src = [&](const PageSrc &ps, const TilePos &tp, int t) -> TileSrc {
        const int pos0 = t * kPBN;
        const int r_hi = kv_hi - pos0 < kPBN - 1 ? kv_hi - pos0 : kPBN - 1;
        TileSrc ts;
        ts.ok = ps.kb != nullptr;
        const int n_rec = ts.ok && r_hi >= 0 ? r_hi * col_bytes + RB : 0;
        const int64_t off = (int64_t)tp.row * col_bytes + (int64_t)kvh * RB;
        ts.k = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(ts.ok ? ps.kb + off : p.k_pages), 0, n_rec,
                                                 kBufferRsrcWord3);
        ts.v = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(ts.ok ? ps.vb + off : p.v_pages), 0, n_rec,
                                                 kBufferRsrcWord3);
        return ts;
    };

    // prologue: K and V of the first tile, K of the second (one tile ahead)
    TilePos pos1{tile0 * kPBN / p.page_size, tile0 * kPBN % p.page_size};
    PageSrc page2 = page_src(pos1.lp);
    const TileSrc src0 = tile_src(page2, pos1, tile0);
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
        dma16(src0.k, lds_k0 + 1024u * i, k_off[i]);
        dma16(src0.v, lds_v0 + 1024u * i, v_off[i]);
    }
    advance(pos1);
    if (pos1.row == 0) page2 = page_src(pos1.lp);
    TileSrc src1 = tile_src(page2, pos1, tile0 + 1);  // zeros past tile1
#pragma unroll
    for (int i = 0; i < IPW; ++i) dma16(src1.k, lds_k0 + (uint32_t)TB + 1024u * i, k_off[i]);
    bool dead_cur = !src0.ok;
    TilePos pos2 = pos1;

    // Q^T operand of this lane's row, rounded to f16
    half8 qf[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        half8 hv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            hv[e] = (_Float16)qx[c][0][e];
            hv[4 + e] = (_Float16)qx[c][1][e];
        }
        qf[c] = row_ok ? hv : half8{};
    }

    // S^T = K * Q^T of the tile in K buffer kb (two 32-position blocks)
    auto qk = [&](const uint8_t *kt, floatx16 (&s)[2]) {
        s[0] = floatx16{};
        s[1] = floatx16{};
#pragma unroll
        for (int c = 0; c < KC; ++c) {
#pragma unroll
            for (int pb = 0; pb < 2; ++pb) {
                const int r = 32 * pb + n;
                const half8 a = *reinterpret_cast<const half8 *>(kt + r * RB + 16 * ((2 * c + hh) ^ (r % CPR)));
                s[pb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[c], s[pb], 0, 0, 0);
            }
        }
    };

    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    floatx16 s[2];
    qk(lds_k[0], s);
    float m_run = -INFINITY, l_run = 0.0f;
    if (prefill_edge(rows, tile0 * kPBN, dead_cur)) prefill_mask(s, rows, tile0 * kPBN, hh, dead_cur);
    float alpha = prefill_rescale(s, p.scale_log2, m_run);

    floatx16 o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) o[d] = floatx16{};

    // V^T operand reads: lane rr of 16-lane group gq takes row 4(gq/2) + rr/4
    // (+ the step's row offset, a multiple of 8), logical bytes 64d +
    // 32(gq%2) + 8(rr%4), its 64-byte group swizzled by the row
    const int gq = lane >> 4, rr = lane & 15;
    int tr_off[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) {
        const int r = 4 * (gq >> 1) + (rr >> 2);
        tr_off[d] = r * RB + 64 * (d ^ ((r / RP) % NG)) + 32 * (gq & 1) + 8 * (rr & 3);
    }
    const half2v ones = {(_Float16)1.0f, (_Float16)1.0f};

    // Tile t: K(t+1) and V(t) are in LDS once the barrier at the top has
    // passed; K(t+2) and V(t+1) go into the buffers the previous trip
    // finished with, one load instruction per QK region (issued together,
    // every wave's loads would queue behind each other at the top of the
    // trip), so each has most of a trip to land.  The trip computes P(t)
    // from S(t) while the MFMAs form S(t+1), then O += V(t)^T P(t)^T.  Trips
    // come in pairs (PAR = (t - tile0) % 2) so that the buffers are fixed per
    // trip and S(t) and S(t+1) swap register sets instead of being copied.
    auto trip = [&](int t, auto par, floatx16(&s)[2], floatx16(&sn)[2]) {
        constexpr int PAR = decltype(par)::value;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        advance(pos2);
        if (pos2.row == 0) page2 = page_src(pos2.lp);
        const TileSrc src2 = tile_src(page2, pos2, t + 2);  // zeros past tile1
        const uint32_t k_dst = lds_k0 + (uint32_t)(PAR * TB);
        const uint32_t v_dst = lds_v0 + (uint32_t)((1 - PAR) * TB);
        const bool dead_next = !src1.ok;

        l_run *= alpha;
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int d = 0; d < DB; ++d) o[d] *= alpha;
        }

        // P(t) = exp2(S(t) scale - m) (f16) beside S(t+1) = K(t+1) Q^T, then
        // O^T += V(t)^T P(t)^T beside P's row sum, in short regions the
        // scheduler may not reorder across (sched_barrier), so the MFMA pipe
        // works on one while the VALU computes the other, and each region's
        // LDS reads feed the next region's products.  (On the last tile the
        // QK products read a stale buffer and are discarded.)
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        const uint8_t *kt = lds_k[1 - PAR];
        const uint8_t *vt = lds_v[PAR];
        auto k_read = [&](int c, half8(&a)[2]) {
#pragma unroll
            for (int pb = 0; pb < 2; ++pb) {
                const int r = 32 * pb + n;
                a[pb] = *reinterpret_cast<const half8 *>(kt + r * RB + 16 * ((2 * c + hh) ^ (r % CPR)));
            }
        };
        auto v_read = [&](int step, half8(&va)[DB]) {  // step = 2 pb + kk
#pragma unroll
            for (int d = 0; d < DB; ++d) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const half4 hv = tr16_read(vt + tr_off[d] + (16 * step + 8 * u) * RB);
                    va[d][4 * u + 0] = hv[0];
                    va[d][4 * u + 1] = hv[1];
                    va[d][4 * u + 2] = hv[2];
                    va[d][4 * u + 3] = hv[3];
                }
            }
        };
        constexpr int EPC = 32 / KC;  // exponentials per QK chunk
        half8 pbv[2][2];
        sn[0] = floatx16{};
        sn[1] = floatx16{};
        half8 ka[2], kb[2], va[DB], vb[DB];
        k_read(0, ka);
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            if (c + 1 < KC) k_read(c + 1, kb);
            if (c + 1 == KC) v_read(0, va);
#pragma unroll
            for (int pb = 0; pb < 2; ++pb) sn[pb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[pb], qf[c], sn[pb], 0, 0, 0);
#pragma unroll
            for (int e = 0; e < EPC; ++e) {
                const int i = EPC * c + e;  // score i % 16 of block i / 16
                pbv[i >> 4][(i >> 3) & 1][i & 7] =
                    (_Float16)__builtin_amdgcn_exp2f(fmaf(s[i >> 4][i & 15], p.scale_log2, -m_use));
            }
            if (c < IPW) dma16(src2.k, k_dst + 1024u * c, k_off[c]);
            else if (c < 2 * IPW) dma16(src1.v, v_dst + 1024u * (c - IPW), v_off[c - IPW]);
            __builtin_amdgcn_sched_barrier(0);
            ka[0] = kb[0];
            ka[1] = kb[1];
        }
        float ls = 0.0f;
#pragma unroll
        for (int step = 0; step < 4; ++step) {
            if (step + 1 < 4) v_read(step + 1, vb);
#pragma unroll
            for (int d = 0; d < DB; ++d)
                o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[d], pbv[step >> 1][step & 1], o[d], 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(HalfPairs, pbv[step >> 1][step & 1]).v[e], ones,
                                            ls, false);
            asm volatile("" : "+v"(ls));  // keeps the sums in this region
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int d = 0; d < DB; ++d) va[d] = vb[d];
        }
        l_run += ls;

        // masking of S(t+1) only where it meets the window start, the
        // diagonal or rows past T, or for an invalid page (wave-uniform)
        if (t < tile1 && prefill_edge(rows, (t + 1) * kPBN, dead_next))
            prefill_mask(sn, rows, (t + 1) * kPBN, hh, dead_next);
        alpha = prefill_rescale(sn, p.scale_log2, m_run);
        src1 = src2;
    };
    floatx16 s1[2];
    for (int t = tile0;; t += 2) {
        trip(t, IntC<0>{}, s, s1);
        if (t + 1 > tile1) break;
        trip(t + 1, IntC<1>{}, s1, s);
        if (t + 2 > tile1) break;
    }

    prefill_write<HD>(o, l_run, rows, p, hh);
}

// F32 cache (the reference's own type): ggml converts nothing, so both
// products run on v_mfma_f32_32x32x2_f32 with Q, K, P and V in f32, in the
// layouts of prefill_f16_kernel (S^T with the lane owning its query row, P^T
// step s of a 32-position block = the lane's score register s).  K and V
// tiles go from the page straight into LDS (global_load_lds, 1 KB per
// instruction): K chunks are XOR-swizzled by row so the 16 rows one ds_read_b128
// phase touches cover all 64 banks; V chunks of rows with bit 2 set are
// shifted by 128 bytes so the two lane halves of a V^T read (rows 4 apart)
// use disjoint banks.  Rows outside the attended range (and tiles of an
// invalid page) are masked in the scores and read as 0 for P*V.
template <int HD, int G>
__global__ __launch_bounds__(256, 1) void prefill_f32_kernel(PrefillParams p) {
    constexpr int KH = HD / 2;           // Q / K floats per lane (half a row)
    constexpr int DB = HD / 32;
    constexpr int RB = HD * 4;           // row bytes
    constexpr int CPR = RB / 16;         // 16-byte chunks per row
    constexpr int TB = kPBN * RB;        // tile bytes (K or V)
    constexpr int IPW = TB / 1024 / 4;   // 1 KB load instructions per wave per tile (K or V)
    constexpr int KSW = (CPR < 16 ? CPR : 16) - 1;  // K chunk swizzle mask (row bits)
    constexpr int VSW = CPR >= 16 ? 8 : CPR / 2;    // V chunk shift for rows with bit 2 set
    static_assert(TB % 4096 == 0, "tile split over four waves");
    typedef __attribute__((address_space(3))) void lds_void;
    __shared__ __attribute__((aligned(16))) uint8_t lds_k[2][TB];
    __shared__ __attribute__((aligned(16))) uint8_t lds_v[2][TB];

    const int kvh = (int)blockIdx.x % p.n_head_kv;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 31;
    const int hh = lane >> 5;
    const int64_t col_bytes = (int64_t)p.n_head_kv * RB;

    const PrefillRows rows = prefill_rows<G>(p, wave, n);
    const bool row_ok = rows.row_ok;
    const int tq = rows.tq, h = rows.h;
    const int kv_hi = rows.kv_hi, lo = rows.lo, tile0 = rows.tile0, tile1 = rows.tile1;

    // tile t -> LDS buffer buf; false (workgroup-uniform) for an invalid page
    auto load = [&](int t, int buf) -> bool {
        const int pos0 = t * kPBN;
        const int lp = pos0 / p.page_size;
        const int32_t pid = __builtin_amdgcn_readfirstlane(lp < p.max_pages ? p.page_table[lp] : -1);
        const uint8_t *kb = page_base(pid, p.k_pages, p.n_pages, p.k_cold, p.n_cold, p.page_bytes);
        const uint8_t *vb = page_base(pid, p.v_pages, p.n_pages, p.v_cold, p.n_cold, p.page_bytes);
        if (kb == nullptr || vb == nullptr) return false;
        const int64_t base = (int64_t)(pos0 - lp * p.page_size) * col_bytes + (int64_t)kvh * RB;
#pragma unroll
        for (int i = 0; i < IPW; ++i) {
            const int blk = wave * IPW + i;      // 1 KB block of the tile
            const int cid = blk * 64 + lane;     // LDS chunk this lane fills
            const int r = cid / CPR, cp = cid % CPR;
            const int ck = cp ^ (r & KSW);
            const int cv = cp ^ (((r >> 2) & 1) * VSW);
            __builtin_amdgcn_global_load_lds(kb + base + (int64_t)r * col_bytes + 16 * ck,
                                             (lds_void *)(&lds_k[buf][1024 * blk]), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(vb + base + (int64_t)r * col_bytes + 16 * cv,
                                             (lds_void *)(&lds_v[buf][1024 * blk]), 16, 0, 0);
        }
        return true;
    };

    bool ok_cur = load(tile0, 0);
    // Q of this lane's row, dims KH*hh .. KH*hh + KH - 1 (rows past T read row 0, zeroed)
    float qf[KH];
    {
        const floatx4 *qr = reinterpret_cast<const floatx4 *>(
            p.q + ((int64_t)(row_ok ? tq : 0) * p.n_head + h) * HD + KH * hh);
#pragma unroll
        for (int j = 0; j < KH / 4; ++j) {
            const floatx4 v4 = qr[j];
#pragma unroll
            for (int e = 0; e < 4; ++e) qf[4 * j + e] = row_ok ? v4[e] : 0.0f;
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    floatx16 o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) o[d] = floatx16{};
    float m_run = -INFINITY, l_run = 0.0f;

    for (int t = tile0; t <= tile1; ++t) {
        const int buf = (t - tile0) & 1;
        const int pos0 = t * kPBN;
        const bool ok_next = t < tile1 ? load(t + 1, buf ^ 1) : false;  // in flight meanwhile
        const uint8_t *kt = lds_k[buf];
        const uint8_t *vt = lds_v[buf];
        const bool dead = !ok_cur;

        floatx16 s[2] = {floatx16{}, floatx16{}};
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) {
            const int r = 32 * pb + n;
#pragma unroll
            for (int j = 0; j < KH / 4; ++j) {
                const int ch = (KH * hh) / 4 + j;
                const floatx4 a = *reinterpret_cast<const floatx4 *>(kt + r * RB + 16 * (ch ^ (r & KSW)));
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    s[pb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], qf[4 * j + e], s[pb], 0, 0, 0);
            }
        }
        const bool edge = prefill_edge(rows, pos0, dead);
        if (edge) prefill_mask(s, rows, pos0, hh, dead);
        const float alpha = prefill_rescale(s, p.scale_log2, m_run);
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        float pe[2][16];
        float ls = 0.0f;
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                pe[pb][i] = __builtin_amdgcn_exp2f(fmaf(s[pb][i], p.scale_log2, -m_use));
                ls += pe[pb][i];
            }
        }
        l_run = l_run * alpha + ls;
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int d = 0; d < DB; ++d) o[d] *= alpha;
        }
        // O^T += V^T * P^T: step s of block pb reads row 32pb + 8(s/4) + 4hh + s%4
        // (its chunk shifted by hh * VSW), dim 32d + n
        const uint8_t *vl = vt + (4 * hh) * RB + 4 * (n & 3);
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
            for (int sidx = 0; sidx < 16; ++sidx) {
                const int r = 32 * pb + 8 * (sidx >> 2) + (sidx & 3);  // + 4hh through vl
                const bool vok = !edge || (!dead && pos0 + r + 4 * hh >= lo && pos0 + r + 4 * hh <= kv_hi);
#pragma unroll
                for (int d = 0; d < DB; ++d) {
                    const int ch = (32 * d + n) / 4;
                    float va = *reinterpret_cast<const float *>(vl + r * RB + 16 * (ch ^ (hh * VSW)));
                    va = vok ? va : 0.0f;
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(va, pe[pb][sidx], o[d], 0, 0, 0);
                }
            }
        }
        // the next tile's loads have landed in every wave before anyone reads them
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        ok_cur = ok_next;
    }

    prefill_write<HD>(o, l_run, rows, p, hh);
}

// Q8_0 cache (head_dim 64 or 128), ggml's arithmetic: Q is quantised to Q8_0
// (d = amax/127 stored fp16, q = round(x/d)), S^T = K * Q^T runs on
// v_mfma_i32_32x32x32_i8 one 32-dim block at a time and s += float(sumi) *
// (d_k * d_q) in block order (ggml_vec_dot_q8_0_q8_0); V is dequantised to f16
// (q * d rounded once) into the f16 kernel's V tile, and the softmax and P*V
// are the f16 kernel's.  Tiles are staged through registers: one thread per
// (position, block) loads the 34-byte block (and the V block) as 4-aligned
// dwords, then writes the quants to a 16-byte-aligned K tile (16-byte chunks
// XOR-swizzled by row / (rows per 256 bytes), so the 16 rows of an operand read
// and the 4 x 4 chunks of a staging write each cover all 64 LDS banks), the
// scale to a per-block scale row (f32), and the dequantised V.
template <int HD, int G>
__global__ __launch_bounds__(256, 2) void prefill_q8_kernel(PrefillParams p) {
    static_assert(HD == 64 || HD == 128, "head_dim");
    constexpr int NB = HD / 32;           // blocks per row
    constexpr int DB = HD / 32;
    constexpr int ROW = HD * 2 + 64;      // padded f16 V row (bytes)
    constexpr int QROW = HD;              // int8 K row in LDS (bytes)
    constexpr int SW = QROW / 16 - 1;     // K chunk swizzle mask
    constexpr int RPB = 256 / QROW;       // K rows per 256 bytes (all 64 LDS banks)
    constexpr int RB = NB * kQ8Bytes;     // bytes of one cache row
    __shared__ __attribute__((aligned(16))) uint8_t lds_k[2][kPBN * QROW];
    __shared__ __attribute__((aligned(16))) float lds_dk[2][NB][kPBN];  // d_k as f32 (converted once, at staging)
    __shared__ __attribute__((aligned(16))) uint8_t lds_v[2][kPBN * ROW];

    const int kvh = (int)blockIdx.x % p.n_head_kv;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 31;
    const int hh = lane >> 5;
    const int64_t col_bytes = (int64_t)p.n_head_kv * RB;

    const PrefillRows rows = prefill_rows<G>(p, wave, n);
    const bool row_ok = rows.row_ok;
    const int tq = rows.tq, h = rows.h;
    const int kv_hi = rows.kv_hi, lo = rows.lo, tile0 = rows.tile0, tile1 = rows.tile1;

    // staging unit of this thread: position sp_, block sc (threads past
    // kPBN * NB stage nothing)
    const bool stager = tid < kPBN * NB;
    const int sp_ = tid / NB, sc = tid % NB;
    uint32_t kraw[9], vraw[9];
    bool page_ok = false;
    // page ids of 64 logical pages, one per lane (a tile's id is a
    // v_readlane, not a dependent load ahead of its data loads), and the
    // current page's K and V bases, resolved once per page
    PageWindow win;
    win.load(p.page_table, p.max_pages, tile0 * kPBN / p.page_size, lane);
    int cur_lp = -1;
    const uint8_t *kb = nullptr, *vb = nullptr;
    auto load = [&](int t) {
        const int pos0 = t * kPBN;
        const int lp = pos0 / p.page_size;
        if (lp != cur_lp) {
            cur_lp = lp;
            const int32_t pid = lp < p.max_pages ? win.get(p.page_table, p.max_pages, lp, lane) : -1;
            kb = page_base(pid, p.k_pages, p.n_pages, p.k_cold, p.n_cold, p.page_bytes);
            vb = page_base(pid, p.v_pages, p.n_pages, p.v_cold, p.n_cold, p.page_bytes);
        }
        page_ok = kb != nullptr && vb != nullptr;
        if (!page_ok || !stager) return;
        // the 36 bytes at or 2 below the block (rows are 4-byte aligned)
        const int64_t off = (int64_t)(pos0 - lp * p.page_size + sp_) * col_bytes + (int64_t)kvh * RB +
                            kQ8Bytes * sc - (sc & 1) * 2;
        const intx4 k0 = load16_a4(kb + off), k1 = load16_a4(kb + off + 16);
        const intx4 v0 = load16_a4(vb + off), v1 = load16_a4(vb + off + 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            kraw[j] = (uint32_t)k0[j]; kraw[4 + j] = (uint32_t)k1[j];
            vraw[j] = (uint32_t)v0[j]; vraw[4 + j] = (uint32_t)v1[j];
        }
        kraw[8] = load4_a4(kb + off + 32);
        vraw[8] = load4_a4(vb + off + 32);
    };
    // registers -> LDS buffer: K quants (swizzled 16-byte chunks 2sc, 2sc+1 of
    // row sp_), its scale, and V dequantised (rows outside [lo, kv_hi] zero)
    auto store = [&](int t, int buf) {
        if (!stager) return;
        const int pos0 = t * kPBN;
        uint32_t kq[8], vq[8];
        uint32_t kd, vd;
        if ((sc & 1) == 0) {
            kd = kraw[0] & 0xffffu;
            vd = vraw[0] & 0xffffu;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                kq[j] = __builtin_amdgcn_alignbyte(kraw[j + 1], kraw[j], 2);
                vq[j] = __builtin_amdgcn_alignbyte(vraw[j + 1], vraw[j], 2);
            }
        } else {
            kd = kraw[0] >> 16;
            vd = vraw[0] >> 16;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                kq[j] = kraw[j + 1];
                vq[j] = vraw[j + 1];
            }
        }
        if (!page_ok) {
            kd = 0u;
#pragma unroll
            for (int j = 0; j < 8; ++j) kq[j] = 0u;
        }
        uint8_t *krow = &lds_k[buf][sp_ * QROW];
        *reinterpret_cast<intx4 *>(krow + 16 * ((2 * sc) ^ ((sp_ / RPB) & SW))) =
            intx4{(int)kq[0], (int)kq[1], (int)kq[2], (int)kq[3]};
        *reinterpret_cast<intx4 *>(krow + 16 * ((2 * sc + 1) ^ ((sp_ / RPB) & SW))) =
            intx4{(int)kq[4], (int)kq[5], (int)kq[6], (int)kq[7]};
        lds_dk[buf][sc][sp_] = (float)__builtin_bit_cast(_Float16, (uint16_t)kd);
        // q * d rounded to f16 on packed halves, as in the Q8_0 decode kernel
        const bool ok = page_ok && pos0 + sp_ >= lo && pos0 + sp_ <= kv_hi;
        const _Float16 dv = ok ? __builtin_bit_cast(_Float16, (uint16_t)vd) : (_Float16)0.0f;
        const half2v dv2 = {dv, dv};
        const half2v bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
        half8 hv[4];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t x = vq[j] ^ 0x80808080u;
            const half2v a = (__builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)) + bias) * dv2;
            const half2v b = (__builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)) + bias) * dv2;
            hv[j >> 1][4 * (j & 1) + 0] = a[0];
            hv[j >> 1][4 * (j & 1) + 1] = a[1];
            hv[j >> 1][4 * (j & 1) + 2] = b[0];
            hv[j >> 1][4 * (j & 1) + 3] = b[1];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
            *reinterpret_cast<half8 *>(&lds_v[buf][sp_ * ROW + 64 * sc + 16 * k]) = hv[k];
    };

    load(tile0);

    // Q8_0 of this lane's query row: block c, elements 16hh .. 16hh+15 (the
    // B operand), d_q = fp16(amax / 127) as f32; rows past T quantise zeros
    intx4 qa[NB];
    float dq[NB];
    {
        const float *qr = p.q + ((int64_t)(row_ok ? tq : 0) * p.n_head + h) * HD;
        floatx4 xr[NB][4];
#pragma unroll
        for (int c = 0; c < NB; ++c)
#pragma unroll
            for (int j = 0; j < 4; ++j) xr[c][j] = reinterpret_cast<const floatx4 *>(qr + 32 * c + 16 * hh)[j];
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            float x[16];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[4 * j] = row_ok ? xr[c][j][0] : 0.0f;
                x[4 * j + 1] = row_ok ? xr[c][j][1] : 0.0f;
                x[4 * j + 2] = row_ok ? xr[c][j][2] : 0.0f;
                x[4 * j + 3] = row_ok ? xr[c][j][3] : 0.0f;
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
                qa[c][j] = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | ((int)((unsigned)q3 << 24));
            }
            dq[c] = (float)(_Float16)d;
        }
    }

    store(tile0, 0);
    __syncthreads();

    floatx16 o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) o[d] = floatx16{};
    float m_run = -INFINITY, l_run = 0.0f;
    const int gq = lane >> 4, rr = lane & 15;
    const int tr_off = (4 * (gq >> 1) + (rr >> 2)) * ROW + 2 * (16 * (gq & 1) + 4 * (rr & 3));
    const half2v ones = {(_Float16)1.0f, (_Float16)1.0f};

    bool ok_cur = page_ok;
    for (int t = tile0; t <= tile1; ++t) {
        const int buf = (t - tile0) & 1;
        const int pos0 = t * kPBN;
        const bool dead = !ok_cur;
        if (t < tile1) load(t + 1);  // in flight while this tile computes
        const uint8_t *kt = lds_k[buf];
        const uint8_t *vt = lds_v[buf];

        // S^T = K * Q^T block by block, scaled in block order
        floatx16 s[2] = {floatx16{}, floatx16{}};
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) {
            const int r = 32 * pb + n;
#pragma unroll
            for (int c = 0; c < NB; ++c) {
                const intx4 a = *reinterpret_cast<const intx4 *>(kt + r * QROW + 16 * ((2 * c + hh) ^ ((r / RPB) & SW)));
                const intx16 acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, qa[c], intx16{}, 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // d_k of positions 32pb + 8j + 4hh + 0..3
                    const floatx4 dk4 = *reinterpret_cast<const floatx4 *>(&lds_dk[buf][c][32 * pb + 8 * j + 4 * hh]);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        s[pb][4 * j + e] += (float)acc[4 * j + e] * ((float)dk4[e] * dq[c]);
                }
            }
        }
        // prefill_edge and prefill_mask spelled out: with the helper calls the
        // register allocator spills 296 bytes in this kernel at head_dim 128
        const bool edge = dead || pos0 < lo || pos0 + kPBN - 1 > rows.q_lo || !rows.block_full;
        if (edge) {
#pragma unroll
            for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kp = pos0 + 32 * pb + 8 * (i >> 2) + 4 * hh + (i & 3);
                    s[pb][i] = (!dead && row_ok && kp >= lo && kp <= rows.qp) ? s[pb][i] : -INFINITY;
                }
            }
        }
        const float alpha = prefill_rescale(s, p.scale_log2, m_run);
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        half8 pbv[2][2];
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                pbv[pb][i >> 3][i & 7] = (_Float16)__builtin_amdgcn_exp2f(fmaf(s[pb][i], p.scale_log2, -m_use));
        }
        float ls = 0.0f;
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(HalfPairs, pbv[pb][kk]).v[j], ones, ls, false);
        l_run = l_run * alpha + ls;
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int d = 0; d < DB; ++d) o[d] *= alpha;
        }
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                half8 va[DB];
#pragma unroll
                for (int d = 0; d < DB; ++d) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const half4 hv = tr16_read(vt + tr_off + (32 * pb + 16 * kk + 8 * u) * ROW + 64 * d);
                        va[d][4 * u + 0] = hv[0];
                        va[d][4 * u + 1] = hv[1];
                        va[d][4 * u + 2] = hv[2];
                        va[d][4 * u + 3] = hv[3];
                    }
                }
#pragma unroll
                for (int d = 0; d < DB; ++d)
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[d], pbv[pb][kk], o[d], 0, 0, 0);
            }
        }
        ok_cur = page_ok;  // the loaded (next) tile's page status
        if (t < tile1) store(t + 1, buf ^ 1);
        __syncthreads();
    }

    prefill_write<HD>(o, l_run, rows, p, hh);
}

template <int HD, int G>
static void launch_prefill(const PrefillParams &p, int kv_type, hipStream_t s) {
    if (kv_type == SFA_KV_F32) {
        hipLaunchKernelGGL((prefill_f32_kernel<HD, G>), dim3(p.n_qblk * p.n_head_kv), dim3(256), 0, s, p);
    } else if (kv_type == SFA_KV_Q8_0) {
        if constexpr (HD >= 64)
            hipLaunchKernelGGL((prefill_q8_kernel<HD, G>), dim3(p.n_qblk * p.n_head_kv), dim3(256), 0, s, p);
    } else
        hipLaunchKernelGGL((prefill_f16_kernel<HD, G>), dim3(p.n_qblk * p.n_head_kv), dim3(256), 0, s, p);
}

template <int HD>
static int launch_prefill_g(const PrefillParams &p, int G, int kv_type, hipStream_t s) {
    switch (G) {
    case 1: launch_prefill<HD, 1>(p, kv_type, s); return SFA_OK;
    case 2: launch_prefill<HD, 2>(p, kv_type, s); return SFA_OK;
    case 4: launch_prefill<HD, 4>(p, kv_type, s); return SFA_OK;
    case 8: launch_prefill<HD, 8>(p, kv_type, s); return SFA_OK;
    default: return SFA_ERR_UNSUPPORTED;
    }
}

int prefill_launch(const sfa_kv_desc *kv, const float *q, float *out, const int32_t *page_table,
                   int32_t max_pages, int32_t q_pos0, int32_t T, int32_t kv_lo, float scale,
                   hipStream_t stream) {
    if (kv->kv_type != SFA_KV_F16 && kv->kv_type != SFA_KV_F32 && kv->kv_type != SFA_KV_Q8_0)
        return SFA_ERR_UNSUPPORTED;
    if (kv->kv_type == SFA_KV_Q8_0 && kv->head_dim < 64) return SFA_ERR_UNSUPPORTED;
    if (kv->page_size % kPBN != 0) return SFA_ERR_UNSUPPORTED;
    if (q == nullptr || out == nullptr || page_table == nullptr) return SFA_ERR_INVALID_ARGUMENT;
    if (T < 0 || q_pos0 < 0 || max_pages <= 0) return SFA_ERR_INVALID_ARGUMENT;
    if (T == 0) return SFA_OK;
    if ((int64_t)q_pos0 + T > (int64_t)max_pages * kv->page_size) return SFA_ERR_INVALID_ARGUMENT;
    const int G = kv->n_head / kv->n_head_kv;
    PrefillParams p;
    p.k_pages = static_cast<const uint8_t *>(kv->k_pages);
    p.v_pages = static_cast<const uint8_t *>(kv->v_pages);
    p.k_cold = static_cast<const uint8_t *>(kv->k_cold);
    p.v_cold = static_cast<const uint8_t *>(kv->v_cold);
    p.page_bytes = (int64_t)row_bytes_of(kv->kv_type, kv->head_dim) * kv->n_head_kv * kv->page_size;
    p.n_pages = kv->n_pages;
    p.n_cold = kv->n_cold_pages;
    p.page_size = kv->page_size;
    p.n_head_kv = kv->n_head_kv;
    p.n_head = kv->n_head;
    p.q = q;
    p.out = out;
    p.page_table = page_table;
    p.max_pages = max_pages;
    p.q_pos0 = q_pos0;
    p.T = T;
    p.kv_lo = kv_lo;
    const int QB = 128 / G;
    p.n_qblk = (T + QB - 1) / QB;
    p.scale_log2 = scale * 1.4426950408889634f;
    int rc;
    switch (kv->head_dim) {
    case 32: rc = launch_prefill_g<32>(p, G, kv->kv_type, stream); break;
    case 64: rc = launch_prefill_g<64>(p, G, kv->kv_type, stream); break;
    case 128: rc = launch_prefill_g<128>(p, G, kv->kv_type, stream); break;
    default: return SFA_ERR_UNSUPPORTED;
    }
    if (rc != SFA_OK) return rc;
    return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
}

}  // namespace sfa
