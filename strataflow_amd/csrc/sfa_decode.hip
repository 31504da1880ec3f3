// sfa_decode.hip - split-K paged decode attention for gfx950 (f16 and Q8_0 KV).
//
// Replaces kq = mul_mat(k, q) -> soft_max_ext(kq, 0-mask, scale) -> mul_mat(vt, kq)
// of build_kv_attention (src/model/engine/engine.cpp:1751-1761) for one query
// token per sequence.  One workgroup = one slot of a kv head's row, which the
// split plan below maps to a (sequence, split); its four waves walk the
// split's 32-position tiles.  Per tile a wave of the f16 kernel
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
#include <mutex>

#include "sfa_decode.h"

namespace sfa {

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


// Workgroup epilogue of a split: the four waves' (m, l, O^T) for the g heads
// (MFMA column n < g is head n; register i of dim block d holds dim
// 32d + 8(i/4) + 4hh + i%4) merge through LDS into the split's (m, l, o),
// written to the workspace, or straight to the output when the sequence has
// one split.  `l_run` is the lane's full sum over its tiles.
template <int HD, int G>
__device__ inline void split_merge(float (*lds_m)[G], float (*lds_l)[G], float (*lds_o)[G][HD],
                                   const DecodeParams &p, int kvh, int slot, int n_b, float *out_b);

template <int HD, int G>
__device__ inline void split_epilogue(const floatx16 (&o)[HD / 32], float m_run, float l_run,
                                      float (*lds_m)[G], float (*lds_l)[G], float (*lds_o)[G][HD],
                                      const DecodeParams &p, int kvh, int slot, int n_b,
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
    split_merge<HD, G>(lds_m, lds_l, lds_o, p, kvh, slot, n_b, out_b);
}

// The four waves' staged (m, l, o) -> the split's record, or the output when
// the sequence has one split.
template <int HD, int G>
__device__ inline void split_merge(float (*lds_m)[G], float (*lds_l)[G], float (*lds_o)[G][HD],
                                   const DecodeParams &p, int kvh, int slot, int n_b, float *out_b) {
    float *part = p.part + ((int64_t)kvh * p.split_row + slot) * G * (HD + 4);
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
        if (n_b == 1) {
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

// ONE: a single sequence.  Its plan then comes from seq_len[0] / kv_lo[0]
// through scalar loads, and the prologue is straight-line code, so the one
// wait before the first tile's K/V requests is for the page-id load alone
// (the Q loads stay in flight): a load inside a branch would make the
// compiler's wait at the join count every later load.
// APP: the fused append (sfa_attn_decode_append).  Sequence b's new token
// (app_k / app_v [B][Hkv][HD] f32, at position seq_len[b] - 1) is written to
// its page rounded to f16 by wave 0 of row slot b (every sequence has a slot
// of that number: the row holds at least B), with loads issued in the
// prologue and stores at the end; the wave that owns the token's tile reads
// the page row before that store may have landed, so it takes the row from
// its own copy of the token instead (the K operand rows and the V tile row
// of that position).  Both round as the append kernel does, so the result
// equals sfa_kv_append then sfa_attn_decode bit for bit.
template <int HD, int G, bool ONE, bool APP = false>
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
    // APP: the owner wave's new K and V rows (f16), staged for its operand
    __shared__ __attribute__((aligned(16))) _Float16 lds_new[APP ? kDecodeWaves : 1][2][APP ? HD : 8];

    // slot j of kv head kvh's row; (b_g, split_g) is the host's guess of its
    // sequence and split, used to start the first tile's loads before the
    // plan (which needs seq_len) is known
    const int kvh = (int)blockIdx.x / p.split_row;
    const int slot = (int)blockIdx.x - kvh * p.split_row;
    int b_g = slot / p.guess_splits;
    if (b_g >= p.n_seq) b_g = p.n_seq - 1;
    const int split_g = slot - b_g * p.guess_splits;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 31;   // MFMA column (head replica) / A-operand row
    const int hh = lane >> 5;  // k half
    const int32_t *pt = p.page_table + (int64_t)b_g * p.max_pages;

    const int Hkv = p.n_head_kv;
    const int64_t col_bytes = (int64_t)Hkv * p.row_bytes;
    uint8_t *vt = lds_v[wave];
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);

    // Issues the K (A operand: row n, dims 16c + 8hh) and V (coalesced: row
    // i*RPI + lane/CPR, chunk lane%CPR) loads of tile t, whose page id is pid
    // (wave-uniform).  The loads do not depend on seq_len: every row of a tile
    // lies in one existing page, and rows outside [lo, n_kv) are masked after
    // arrival (score -inf, V zeroed).  Returns false (wave-uniform), loading
    // nothing, for an invalid page.  Plain global loads: buffer loads over the
    // tile's rows (a zero-byte descriptor for an invalid page, no branch) made
    // the prologue no faster and the loop slower (B = 1, context 32768: split
    // pass 28.9 -> 30.0 us).
    half8 kf[KC];
    half8 vr[VIT];
    PageWindow pages;
    auto issue = [&](int t, int32_t pid) -> bool {
        const int pos0 = t * kTile;
        const int lpage = pos0 / p.page_size;
        if (lpage >= p.max_pages) return false;
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
    auto page_of = [&](int t) -> int32_t {
        const int lpage = t * kTile / p.page_size;
        return lpage < p.max_pages ? pages.get(pt, p.max_pages, lpage, lane) : -1;
    };

    // Prologue order matters: loads complete in issue order (one vmcnt), so
    // the small loads a wave waits on first (its page-id window, seq_len /
    // kv_lo, its Q chunk) are issued before the first tile's K/V burst; the
    // first tile, as the host plan places it (kv_lo 0, seq_len within the
    // plan), is fetched before seq_len is known and re-issued below if the
    // guess was wrong.
    int t_guess, t_guess_hi;
    split_tiles(0, p.guess_tiles, p.guess_splits, split_g, t_guess, t_guess_hi);
    t_guess = __builtin_amdgcn_readfirstlane(t_guess + wave);
    pages.load(pt, p.max_pages, t_guess * kTile / p.page_size, lane);
    // one sequence: seq_len / kv_lo through scalar loads (a counter of their
    // own); a batch: per-lane loads
    int one_n_kv = 0, one_lo = 0;
    PlanRaw raw{0, 0};
    if constexpr (ONE) {
        one_n_kv = p.seq_len[0];
        one_lo = p.kv_lo ? p.kv_lo[0] : 0;
    } else {
        raw = plan_load(p, lane);
    }
    // Q of the g heads rounded to f16 (the F16 vec_dot_type conversion ggml
    // applies to src1), staged once per workgroup in LDS; the Q^T operand of
    // column n (head n % g, dims 16c + 8hh .. +8) is re-read per tile, which
    // keeps 32 registers free.  One 8-element chunk per thread.
    static_assert(G * HD / 8 <= 256, "one Q chunk per thread");
    const bool q_thread = threadIdx.x < G * HD / 8;
    floatx4 qx0 = floatx4{}, qx1 = floatx4{};
    // every thread loads (the spare ones re-read chunk 0): no branch around it
    auto load_q = [&](int bq) {
        const floatx4 *qr = reinterpret_cast<const floatx4 *>(
            p.q + ((int64_t)bq * p.n_head + (int64_t)kvh * G) * HD);
        const int c = q_thread ? (int)threadIdx.x : 0;
        qx0 = qr[2 * c];
        qx1 = qr[2 * c + 1];
    };
    load_q(b_g);
    // the window starts at the guessed tile's page: its id is lane 0's
    bool tile_ok = issue(t_guess, __builtin_amdgcn_readlane(pages.ids, 0));

    // APP writer: sequence `slot`'s new row, two elements per lane (lanes
    // past head_dim / 2 repeat the last pair); loads unconditional, behind
    // the first tile's
    constexpr int APL = HD / 2;  // lanes carrying a new row's element pairs
    const int app_e = 2 * (lane < APL ? lane : APL - 1);
    const int app_ws = slot < p.n_seq ? slot : p.n_seq - 1;
    float2 app_wk{}, app_wv{};
    if constexpr (APP) {
        const int64_t o = ((int64_t)app_ws * Hkv + kvh) * HD + app_e;
        app_wk = *reinterpret_cast<const float2 *>(p.app_k + o);
        app_wv = *reinterpret_cast<const float2 *>(p.app_v + o);
    }

    SlotPlan sp;
    bool active;
    if constexpr (ONE) {
        sp.g = seq_geom(one_n_kv, one_lo, p.max_pages * p.page_size);
        sp.n_b = splits_of(sp.g.n_tiles, p.one_split ? 0 : p.split_row - 1, sp.g.n_tiles);
        sp.b = 0;
        sp.rec0 = 0;
        sp.split = slot;
        active = slot < sp.n_b;
    } else {
        active = plan(p, raw, slot, -1, lane, sp);
    }
    // raw seq_len of sequence j (wave-uniform): lane j of the plan's loads
    // holds it when the batch has at most 64 sequences
    auto seq_len_of = [&](int j) -> int {
        if constexpr (ONE) return one_n_kv;
        else return p.n_seq <= kWave ? __builtin_amdgcn_readlane(raw.n_kv, j) : p.seq_len[j];
    };
    // the writer's row: position seq_len - 1 of sequence `slot`, skipped past
    // the table or for a page that is not there, as the append kernel skips
    // them; its page id is loaded now and the stores go out at the end
    int app_pn = -1;
    int32_t app_wid = -1;
    if constexpr (APP) {
        const int pn = seq_len_of(app_ws) - 1;
        const int lp = pn < 0 ? 0 : pn / p.page_size;
        app_pn = slot < p.n_seq && wave_u == 0 && pn >= 0 && lp < p.max_pages ? pn : -1;
        app_wid = p.page_table[(int64_t)app_ws * p.max_pages + (lp < p.max_pages ? lp : p.max_pages - 1)];
    }
    auto app_write = [&]() {
        if constexpr (APP) {
            if (app_pn < 0) return;
            uint8_t *kb = const_cast<uint8_t *>(
                page_base(app_wid, p.app_k_pages, p.n_pages, p.app_k_cold, p.n_cold, p.page_bytes));
            uint8_t *vb = const_cast<uint8_t *>(
                page_base(app_wid, p.app_v_pages, p.n_pages, p.app_v_cold, p.n_cold, p.page_bytes));
            if (kb == nullptr || vb == nullptr || lane >= APL) return;
            const int lp = app_pn / p.page_size;
            const int64_t off = ((int64_t)(app_pn - lp * p.page_size) * Hkv + kvh) * p.row_bytes + 2 * app_e;
            *reinterpret_cast<half2v *>(kb + off) = half2v{(_Float16)app_wk.x, (_Float16)app_wk.y};
            *reinterpret_cast<half2v *>(vb + off) = half2v{(_Float16)app_wv.x, (_Float16)app_wv.y};
        }
    };
    if (!active) {
        // an idle slot; the merge pass writes the output of a sequence
        // without tiles, or, for one sequence, the slot that would own it
        if (p.n_seq == 1 && slot == 0 && sp.n_b == 0) {
            float *out0 = p.out + (int64_t)kvh * G * HD;
            for (int i = threadIdx.x; i < G * HD; i += blockDim.x) out0[i] = 0.0f;
        }
        app_write();
        return;
    }
    const int b = sp.b;
    int tile_lo, tile_hi;
    split_tiles(sp.g.t0, sp.g.n_tiles, sp.n_b, sp.split, tile_lo, tile_hi);
    if (b != b_g) {  // a wrong guess: this slot serves another sequence
        pt = p.page_table + (int64_t)b * p.max_pages;
        pages.load(pt, p.max_pages, tile_lo * kTile / p.page_size, lane);
        load_q(b);
    }
    if (q_thread) {
        half8 h;
        h[0] = (_Float16)qx0[0]; h[1] = (_Float16)qx0[1]; h[2] = (_Float16)qx0[2]; h[3] = (_Float16)qx0[3];
        h[4] = (_Float16)qx1[0]; h[5] = (_Float16)qx1[1]; h[6] = (_Float16)qx1[2]; h[7] = (_Float16)qx1[3];
        reinterpret_cast<half8 *>(lds_q)[threadIdx.x] = h;
    }

    const int lo = sp.g.lo, n_kv = sp.g.n_kv;
    float *out_b = p.out + ((int64_t)b * p.n_head + (int64_t)kvh * G) * HD;
    int t = tile_lo + wave_u;
    if (t != t_guess || b != b_g) tile_ok = t < tile_hi ? issue(t, page_of(t)) : false;
    // APP owner: the wave whose tiles include sequence b's new position (its
    // last tile) keeps the token's row (two elements per lane) to put in place
    // of the page row it loads
    int t_new = -1, r_new = 0;
    float2 app_ok{}, app_ov{};
    if constexpr (APP) {
        const int64_t o = ((int64_t)b * Hkv + kvh) * HD + app_e;
        app_ok = *reinterpret_cast<const float2 *>(p.app_k + o);
        app_ov = *reinterpret_cast<const float2 *>(p.app_v + o);
        const int pn = seq_len_of(b) - 1;
        if (pn >= 0 && pn < p.max_pages * p.page_size) {
            const int tn = pn / kTile;
            if (tn >= tile_lo && tn < tile_hi && (tn - tile_lo) % kDecodeWaves == wave_u) {
                t_new = tn;
                r_new = pn - tn * kTile;
            }
        }
    }
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
        // an invalid page id (tile_ok false) leaves the registers stale: the
        // tile then runs fully masked and contributes nothing
        const bool dead = !tile_ok;
        if constexpr (APP) {
            if (t == t_new) {
                // the new token's rows through the wave's LDS: K dims 16c + 8hh
                // of row r_new into the operand, V after the V tile below
                _Float16 *nk = &lds_new[wave_u][0][0];
                _Float16 *nv = &lds_new[wave_u][1][0];
                if (lane < APL) {
                    *reinterpret_cast<half2v *>(nk + app_e) = half2v{(_Float16)app_ok.x, (_Float16)app_ok.y};
                    *reinterpret_cast<half2v *>(nv + app_e) = half2v{(_Float16)app_ov.x, (_Float16)app_ov.y};
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                for (int c = 0; c < KC; ++c) {
                    const half8 h = *reinterpret_cast<const half8 *>(nk + 16 * c + 8 * hh);
                    kf[c] = n == r_new ? h : kf[c];
                }
            }
        }
        // S^T = K * Q^T
        floatx16 s0 = floatx16{};
#pragma unroll
        for (int c = 0; c < KC; ++c) s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[c], qrow[2 * c], s0, 0, 0, 0);
        // V tile into the wave's LDS region; rows outside [lo, n_kv) zeroed
        // (they may hold stale bytes of a page's unused tail).  Interior
        // tiles (a scalar test) store unmasked.
        const bool interior = !dead && pos0 >= lo && pos0 + kTile <= n_kv;
        if (interior) {
#pragma unroll
            for (int i = 0; i < VIT; ++i) {
                const int r = i * RPI + lane / CPR;
                *reinterpret_cast<half8 *>(vt + r * VROW + 16 * (lane % CPR)) = vr[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < VIT; ++i) {
                const int r = i * RPI + lane / CPR;
                const bool ok = !dead && pos0 + r >= lo && pos0 + r < n_kv;
                *reinterpret_cast<half8 *>(vt + r * VROW + 16 * (lane % CPR)) = ok ? vr[i] : half8{};
            }
        }
        if constexpr (APP) {
            // row r_new of the V tile (after every lane's tile stores: a
            // wave's LDS operations complete in order)
            if (t == t_new && !dead && lane < CPR)
                *reinterpret_cast<half8 *>(vt + r_new * VROW + 16 * lane) =
                    *reinterpret_cast<const half8 *>(&lds_new[wave_u][1][8 * lane]);
        }
        // registers are free: start the next tile's loads now
        const bool next_ok = t + kDecodeWaves < tile_hi ? issue(t + kDecodeWaves, page_of(t + kDecodeWaves)) : false;

        // online softmax (log2 domain); row of register i is tile position
        // 8(i/4) + 4hh + i%4.  Interior tiles need no mask.  The reference
        // max moves only when a score exceeds it by 2^8 (a wave-uniform
        // ballot), so most tiles skip the max exchange and the O rescale;
        // P <= 256 and O, l share the reference, so the result is unchanged.
        float sv[16];
        float mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float v = s0[i] * p.scale_log2;
            if (!interior) {
                const int pp = pos0 + 8 * (i >> 2) + 4 * hh + (i & 3);
                v = (!dead && pp >= lo && pp < n_kv) ? v : -INFINITY;
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
    app_write();
    split_epilogue<HD, G>(o, m_run, l_run, lds_m, lds_l, lds_o, p, kvh, sp.rec0 + sp.split, sp.n_b, out_b,
                          wave, n, hh);
}

// F32 decode: the reference's own cache type.  ggml's F32 path keeps Q, K,
// P and V in f32 (the vec_dot_type of F32 is F32), so both products run on
// v_mfma_f32_16x16x4_f32: 16 columns hold the g heads of the kv head (4x
// replication at g = 4, against 8x on the 32-column f32 MFMA, which halves the
// MFMA work).  Lane l serves column c = l % 16 (head c % g) and quarter
// q = l / 16.  S^T = K * Q^T per 16-position row block rb: quarter q brings
// dims q*HD/4 .. of K row 16rb + c (contiguous 16-byte loads) and of Q, so
// the k order of the product is a permutation of the dims; S^T lands with
// register r of block rb at position 16rb + 4q + r.  O^T += V^T * P^T takes
// step (rb, r) with quarter q supplying position 16rb + 4q + r, so its P^T
// operand is the lane's own score register: P never moves.  V tiles go
// straight from the page into the wave's LDS region (global_load_lds, 1 KB
// per instruction, no registers) with the 16-byte chunks of row r XORed by
// 4 * ((r / 4) % 4), so the four quarters' V^T reads (rows 4 apart) fall in
// different LDS banks.  At 4 bytes per element the kernel stays bound by HBM
// at long contexts.  APP: the fused append, as in decode_f16_kernel (rows
// stored as f32, as the append stores them).
template <int HD, int G, bool APP = false>
__global__ __launch_bounds__(256, G <= 4 ? 2 : 1) void decode_f32_kernel(DecodeParams p) {
    static_assert(HD == 32 || HD == 64 || HD == 128, "head_dim");
    static_assert(G >= 1 && G <= 16 && (16 % G) == 0, "group size");
    constexpr int QD = HD / 4;           // dims per quarter (k steps per row block)
    constexpr int KQ4 = QD / 4;          // 16-byte K loads per lane and row block
    constexpr int KV4 = 2 * KQ4;         // K load instructions per tile
    constexpr int DB = HD / 16;          // 16-dim blocks of the PV output
    constexpr int VRB = HD * 4;          // V row bytes in LDS (unpadded)
    constexpr int CPR = VRB / 16;        // 16-byte chunks per V row
    constexpr int RPI = kWave / CPR;     // V rows per global_load_lds instruction
    constexpr int VIT = kTile / RPI;     // V instructions per tile
    typedef __attribute__((address_space(3))) void lds_void;

    __shared__ __attribute__((aligned(16))) uint8_t lds_v[kDecodeWaves][kTile * VRB];
    __shared__ float lds_m[kDecodeWaves][G];
    __shared__ float lds_l[kDecodeWaves][G];
    __shared__ __attribute__((aligned(16))) float lds_q[G * HD];
    __shared__ float lds_o[kDecodeWaves][G][HD];
    // APP: the owner wave's new K row, staged for its operand
    __shared__ __attribute__((aligned(16))) float lds_newk[APP ? kDecodeWaves : 1][APP ? HD : 4];

    const int kvh = (int)blockIdx.x / p.split_row;
    const int slot = (int)blockIdx.x - kvh * p.split_row;
    int b_g = slot / p.guess_splits;
    if (b_g >= p.n_seq) b_g = p.n_seq - 1;
    const int split_g = slot - b_g * p.guess_splits;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c16 = lane & 15;  // MFMA column (head c16 % g) / A-operand row
    const int qt = lane >> 4;   // quarter: k slot of the MFMA operands
    const int32_t *pt = p.page_table + (int64_t)b_g * p.max_pages;

    const int Hkv = p.n_head_kv;
    const int64_t col_bytes = (int64_t)Hkv * p.row_bytes;
    uint8_t *vt = lds_v[wave];
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);

    // K of tile t into registers (rows 16rb + c16, dims QD*qt ..), V of tile
    // t into the wave's LDS tile (instruction i: row r = i*RPI + lane/CPR,
    // LDS chunk lane%CPR holding the row's chunk (lane%CPR) ^ vswz(r), lane l
    // at byte 16 l of the instruction's 1 KB run).  Both return false
    // (wave-uniform) for an invalid page id and then load nothing.
    floatx4 kf[2][KQ4];
    PageWindow pages;
    const uint8_t *vsrc_next = nullptr;
    auto issue_k = [&](int t) -> bool {
        const int pos0 = t * kTile;
        const int lpage = pos0 / p.page_size;
        vsrc_next = nullptr;
        if (lpage >= p.max_pages) return false;
        const int32_t pid = pages.get(pt, p.max_pages, lpage, lane);
        const uint8_t *kb = page_base(pid, p.k_pages, p.n_pages, p.k_cold, p.n_cold, p.page_bytes);
        const uint8_t *vb = page_base(pid, p.v_pages, p.n_pages, p.v_cold, p.n_cold, p.page_bytes);
        if (kb == nullptr || vb == nullptr) return false;
        const int64_t off0 = (int64_t)(pos0 - lpage * p.page_size) * col_bytes + (int64_t)kvh * p.row_bytes;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const uint8_t *kr = kb + off0 + (int64_t)(16 * rb + c16) * col_bytes + QD * 4 * qt;
#pragma unroll
            for (int j = 0; j < KQ4; ++j) kf[rb][j] = *reinterpret_cast<const floatx4 *>(kr + 16 * j);
        }
        vsrc_next = vb + off0;
        return true;
    };
    // the V half of the tile issue_k last resolved (nothing for an invalid page)
    auto issue_v = [&]() {
        if (vsrc_next == nullptr) return;
#pragma unroll
        for (int i = 0; i < VIT; ++i) {
            const int r = i * RPI + lane / CPR;
            __builtin_amdgcn_global_load_lds(vsrc_next + (int64_t)r * col_bytes + 16 * ((lane % CPR) ^ ((4 * ((r >> 2) & 3)) & (CPR - 1))),
                                             (lds_void *)(vt + 1024 * i), 16, 0, 0);
        }
    };

    int t_guess, t_guess_hi;
    split_tiles(0, p.guess_tiles, p.guess_splits, split_g, t_guess, t_guess_hi);
    t_guess = __builtin_amdgcn_readfirstlane(t_guess + wave);
    pages.load(pt, p.max_pages, t_guess * kTile / p.page_size, lane);
    const PlanRaw raw = plan_load(p, lane);
    // Q of the g heads in f32, staged once per workgroup in LDS
    floatx4 qx[(G * HD / 4 + 255) / 256];
    auto load_q = [&](int bq) {
        const floatx4 *qr = reinterpret_cast<const floatx4 *>(p.q + ((int64_t)bq * p.n_head + (int64_t)kvh * G) * HD);
#pragma unroll
        for (int j = 0; j < (G * HD / 4 + 255) / 256; ++j) {
            const int idx = j * 256 + (int)threadIdx.x;
            if (idx < G * HD / 4) qx[j] = qr[idx];
        }
    };
    load_q(b_g);
    bool tile_ok = issue_k(t_guess);
    bool v_pending = tile_ok;  // the guessed tile's V loads are in flight into vt
    issue_v();

    // APP writer (wave 0 of slot j < B writes sequence j's new row): two
    // elements per lane, loaded behind the first tile
    constexpr int APL = HD / 2;
    const int app_e = 2 * (lane < APL ? lane : APL - 1);
    const int app_ws = slot < p.n_seq ? slot : p.n_seq - 1;
    float2 app_wk{}, app_wv{};
    if constexpr (APP) {
        const int64_t o = ((int64_t)app_ws * Hkv + kvh) * HD + app_e;
        app_wk = *reinterpret_cast<const float2 *>(p.app_k + o);
        app_wv = *reinterpret_cast<const float2 *>(p.app_v + o);
    }

    SlotPlan sp;
    const bool active = plan(p, raw, slot, -1, lane, sp);
    // raw seq_len of sequence j: lane j of the plan's loads (up to 64 sequences)
    auto seq_len_of = [&](int j) -> int {
        return p.n_seq <= kWave ? __builtin_amdgcn_readlane(raw.n_kv, j) : p.seq_len[j];
    };
    int app_pn = -1;
    int32_t app_wid = -1;
    if constexpr (APP) {
        const int pn = seq_len_of(app_ws) - 1;
        const int lp = pn < 0 ? 0 : pn / p.page_size;
        app_pn = slot < p.n_seq && wave_u == 0 && pn >= 0 && lp < p.max_pages ? pn : -1;
        app_wid = p.page_table[(int64_t)app_ws * p.max_pages + (lp < p.max_pages ? lp : p.max_pages - 1)];
    }
    auto app_write = [&]() {
        if constexpr (APP) {
            if (app_pn < 0) return;
            uint8_t *kb = const_cast<uint8_t *>(
                page_base(app_wid, p.app_k_pages, p.n_pages, p.app_k_cold, p.n_cold, p.page_bytes));
            uint8_t *vb = const_cast<uint8_t *>(
                page_base(app_wid, p.app_v_pages, p.n_pages, p.app_v_cold, p.n_cold, p.page_bytes));
            if (kb == nullptr || vb == nullptr || lane >= APL) return;
            const int lp = app_pn / p.page_size;
            const int64_t off = ((int64_t)(app_pn - lp * p.page_size) * Hkv + kvh) * p.row_bytes + 4 * app_e;
            *reinterpret_cast<float2 *>(kb + off) = app_wk;
            *reinterpret_cast<float2 *>(vb + off) = app_wv;
        }
    };
    if (!active) {
        if (p.n_seq == 1 && slot == 0 && sp.n_b == 0) {
            float *out0 = p.out + (int64_t)kvh * G * HD;
            for (int i = threadIdx.x; i < G * HD; i += blockDim.x) out0[i] = 0.0f;
        }
        app_write();
        // the wave's LDS loads must land before the workgroup ends
        __builtin_amdgcn_s_waitcnt(0);
        return;
    }
    const int b = sp.b;
    int tile_lo, tile_hi;
    split_tiles(sp.g.t0, sp.g.n_tiles, sp.n_b, sp.split, tile_lo, tile_hi);
    if (b != b_g) {
        pt = p.page_table + (int64_t)b * p.max_pages;
        pages.load(pt, p.max_pages, tile_lo * kTile / p.page_size, lane);
        load_q(b);
    }
#pragma unroll
    for (int j = 0; j < (G * HD / 4 + 255) / 256; ++j) {
        const int idx = j * 256 + (int)threadIdx.x;
        if (idx < G * HD / 4) reinterpret_cast<floatx4 *>(lds_q)[idx] = qx[j];
    }

    const int lo = sp.g.lo, n_kv = sp.g.n_kv;
    float *out_b = p.out + ((int64_t)b * p.n_head + (int64_t)kvh * G) * HD;
    int t = tile_lo + wave_u;
    if (t != t_guess || b != b_g) {
        // the guessed V loads write vt: let them land before the real ones
        if (v_pending) __builtin_amdgcn_s_waitcnt(0);
        if (t < tile_hi) {
            tile_ok = issue_k(t);
        } else {
            tile_ok = false;
            vsrc_next = nullptr;
        }
        issue_v();
    }
    // APP owner: the wave whose tiles include sequence b's new position
    int t_new = -1, r_new = 0;
    float2 app_ok{}, app_ov{};
    if constexpr (APP) {
        const int64_t o = ((int64_t)b * Hkv + kvh) * HD + app_e;
        app_ok = *reinterpret_cast<const float2 *>(p.app_k + o);
        app_ov = *reinterpret_cast<const float2 *>(p.app_v + o);
        const int pn = seq_len_of(b) - 1;
        if (pn >= 0 && pn < p.max_pages * p.page_size) {
            const int tn = pn / kTile;
            if (tn >= tile_lo && tn < tile_hi && (tn - tile_lo) % kDecodeWaves == wave_u) {
                t_new = tn;
                r_new = pn - tn * kTile;
            }
        }
    }
    __syncthreads();
    const float *qcol = lds_q + (c16 % G) * HD + QD * qt;

    floatx4 o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) o[d] = floatx4{};
    float m_run = -INFINITY;
    float l_run = 0.0f;

    bool first = true;
    for (; t < tile_hi; t += kDecodeWaves) {
        const int pos0 = t * kTile;
        const bool dead = !tile_ok;
        if constexpr (APP) {
            if (t == t_new) {
                // the new K row through the wave's LDS into the operand of
                // lanes c16 == r_new % 16, row block r_new / 16
                if (lane < APL) *reinterpret_cast<float2 *>(&lds_newk[wave_u][app_e]) = app_ok;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const bool mine = c16 == (r_new & 15);
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
                    for (int j = 0; j < KQ4; ++j) {
                        const floatx4 nk = *reinterpret_cast<const floatx4 *>(&lds_newk[wave_u][QD * qt + 4 * j]);
                        kf[rb][j] = (mine && rb == (r_new >> 4)) ? nk : kf[rb][j];
                    }
                }
            }
        }
        // S^T = K * Q^T: row block rb, k step 4j + e is dim QD*qt + 4j + e
        floatx4 s[2] = {floatx4{}, floatx4{}};
#pragma unroll
        for (int j = 0; j < KQ4; ++j) {
            const floatx4 qv = *reinterpret_cast<const floatx4 *>(qcol + 4 * j);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
                    s[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[rb][j][e], qv[e], s[rb], 0, 0, 0);
            }
        }
        // registers are free: fetch the next tile's K (its V follows the P*V)
        const bool next_ok = t + kDecodeWaves < tile_hi ? issue_k(t + kDecodeWaves) : false;

        // score register 4rb + r is position 16rb + 4qt + r of column c16
        const bool interior = !dead && pos0 >= lo && pos0 + kTile <= n_kv;
        float sv[8];
        float mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float v = s[i >> 2][i & 3] * p.scale_log2;
            if (!interior) {
                const int pp = pos0 + 16 * (i >> 2) + 4 * qt + (i & 3);
                v = (!dead && pp >= lo && pp < n_kv) ? v : -INFINITY;
            }
            sv[i] = v;
            mt = fmaxf(mt, v);
        }
        if (__any(mt > m_run + kRescaleLog2)) {
            // the column's max over the four quarters (lanes c16 + 16q)
            mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
            mt = fmaxf(mt, xor32(mt));
            const float m_new = fmaxf(m_run, mt);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
            if (!first) {
#pragma unroll
                for (int d = 0; d < DB; ++d) o[d] *= alpha;
            }
            m_run = m_new;
        }
        first = false;
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        float pe[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            pe[i] = __builtin_amdgcn_exp2f(sv[i] - m_use);
            l_run += pe[i];
        }

        // this tile's V has landed in vt (the next tile's K loads, issued after
        // it, may still fly: loads complete in order); then O^T += V^T * P^T,
        // rows outside [lo, n_kv) read as 0 (a page's unused tail may hold any
        // bytes).  Step (rb, r): quarter qt supplies row 16rb + 4qt + r, dim
        // 16d + c16 of the A operand and its own score register as B.
        if (next_ok)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(KV4) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if constexpr (APP) {
            // row r_new of the landed V tile (logical chunk c at chunk c ^ the
            // row's swizzle), before any lane reads it
            if (t == t_new && !dead && lane < APL) {
                const int sw = (4 * ((r_new >> 2) & 3)) & (CPR - 1);
                *reinterpret_cast<float2 *>(vt + r_new * VRB + 16 * ((lane >> 1) ^ sw) + 8 * (lane & 1)) = app_ov;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 16 * (i >> 2) + 4 * qt + (i & 3);
            const bool row_ok = interior || (!dead && pos0 + r >= lo && pos0 + r < n_kv);
            const uint8_t *vrow = vt + r * VRB + 4 * (c16 & 3);
            const int sw = (4 * ((r >> 2) & 3)) & (CPR - 1);  // the chunk XOR of row r
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                float va = *reinterpret_cast<const float *>(vrow + 16 * ((4 * d + (c16 >> 2)) ^ sw));
                va = row_ok ? va : 0.0f;
                o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(va, pe[i], o[d], 0, 0, 0);
            }
        }
        // every V^T read of this tile has returned before the next tile's V
        // overwrites vt
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (next_ok) issue_v();
        tile_ok = next_ok;
    }
    __builtin_amdgcn_s_waitcnt(0);
    app_write();

    // the column's sum over the four quarters; one replica of each head
    // (columns c16 < g) stages its (m, l, O^T): register r of block d is dim
    // 16d + 4qt + r
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += xor32(l_run);
    if (c16 < G) {
        if (qt == 0) {
            lds_m[wave][c16] = m_run;
            lds_l[wave][c16] = l_run;
        }
#pragma unroll
        for (int d = 0; d < DB; ++d) {
#pragma unroll
            for (int r = 0; r < 4; ++r) lds_o[wave][c16][16 * d + 4 * qt + r] = o[d][r];
        }
    }
    __syncthreads();
    split_merge<HD, G>(lds_m, lds_l, lds_o, p, kvh, sp.rec0 + sp.split, sp.n_b, out_b);
}

// One lane's half of a Q8_0 row of K and of V, kept as loaded: head_dim 128,
// row bytes 68hh .. 68hh + 67 (blocks 2hh and 2hh + 1, 17 dwords); head_dim
// 64, bytes 32hh .. 32hh + 35 (block hh and two bytes beside it, 9 dwords).
template <int HD>
struct Q8Raw {
    intx4 k4[HD / 32];
    uint32_t k1;
    intx4 v4[HD / 32];
    uint32_t v1;
};

// The K operand of S = Q8 * K8^T for the lane's row (MFMA column n, quants
// 16hh .. 16hh + 15 of every block) and the row's block scales, from the two
// halves' raw pieces.  Half-row dwords D (local byte 0 = row byte 68hh or
// 32hh).  head_dim 128: the half's first block (2hh) has d at local bytes 0-1
// and quants 0-15 / 16-31 at 2-17 / 18-33, its second (2hh + 1) d at 34-35
// and quants at 36-51 / 52-67 (dwords 9-12 / 13-16).  head_dim 64: half 0
// holds block 0 as the first block above; half 1 (from row byte 32) block 1
// with d at local 2-3 and quants at dwords 1-4 / 5-8.  Per pair of blocks the
// lane forms X = its block's quants 0-15 and Y = quants 16-31; swapping X's
// upper 32 lanes with Y's lower 32 leaves X = the first block of half 0
// (lanes of half hh holding quants 16hh ..) and Y = that of half 1.
template <int HD>
__device__ inline void q8_k_operand(const Q8Raw<HD> &r, int hh, intx4 (&kop)[HD / 32], uint32_t (&kdb)[HD / 32]) {
    constexpr int KQ = HD / 32, NB = HD / 32;
    uint32_t D[4 * KQ + 1];
#pragma unroll
    for (int j = 0; j < KQ; ++j) {
#pragma unroll
        for (int e = 0; e < 4; ++e) D[4 * j + e] = (uint32_t)r.k4[j][e];
    }
    D[4 * KQ] = r.k1;
    // bytes 2.. of dwords j, j+1 (head_dim 128, and half 0 of 64); dword
    // j + 1 itself for half 1 of head_dim 64
    const uint32_t sel = (HD == 64 && hh) ? 0x07060504u : 0x05040302u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t x = __builtin_amdgcn_perm(D[j + 1], D[j], sel);
        const uint32_t y = __builtin_amdgcn_perm(D[j + 5], D[j + 4], sel);
        const auto s = __builtin_amdgcn_permlane32_swap(x, y, false, false);
        kop[0][j] = (int)s[0];
        kop[NB / 2][j] = (int)s[1];
    }
    if constexpr (HD == 128) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const auto s = __builtin_amdgcn_permlane32_swap(D[9 + j], D[13 + j], false, false);
            kop[1][j] = (int)s[0];
            kop[3][j] = (int)s[1];
        }
        // d of the half's two blocks (low half of dword 0, high half of dword
        // 8), then both halves' pairs to every lane
        const uint32_t dd = __builtin_amdgcn_perm(D[8], D[0], 0x07060100u);
        const auto s = __builtin_amdgcn_permlane32_swap(dd, dd, false, false);
        kdb[0] = s[0] & 0xffffu;
        kdb[1] = s[0] >> 16;
        kdb[2] = s[1] & 0xffffu;
        kdb[3] = s[1] >> 16;
    } else {
        const uint32_t dd = hh ? D[0] >> 16 : D[0] & 0xffffu;
        const auto s = __builtin_amdgcn_permlane32_swap(dd, dd, false, false);
        kdb[0] = s[0];
        kdb[1] = s[1];
    }
}

// The lane's V blocks (VBL = head_dim / 64 of them: blocks VBL*hh ..)
// dequantised into its row of the f16 LDS tile (`row`, dims 32c .. at byte
// 64c), or zeros when !keep (a row outside [lo, n_kv): its bytes may be
// anything).  Block u of the lane's piece spans dwords 8u .. 8u + 8; an even
// block has d at the low half of its first dword.
template <int HD>
__device__ inline void q8_v_row(const Q8Raw<HD> &r, int hh, bool keep, uint8_t *row) {
    constexpr int KQ = HD / 32, VBL = HD / 64;
    uint32_t Dv[4 * KQ + 1];
#pragma unroll
    for (int j = 0; j < KQ; ++j) {
#pragma unroll
        for (int e = 0; e < 4; ++e) Dv[4 * j + e] = (uint32_t)r.v4[j][e];
    }
    Dv[4 * KQ] = r.v1;
#pragma unroll
    for (int u = 0; u < VBL; ++u) {
        const int c = VBL * hh + u;
        const uint32_t *w = Dv + 8 * u;
        uint32_t q[8];
        uint32_t dbits;
        if ((c & 1) == 0) {
            dbits = w[0] & 0xffffu;
#pragma unroll
            for (int j = 0; j < 8; ++j) q[j] = __builtin_amdgcn_alignbyte(w[j + 1], w[j], 2);
        } else {
            dbits = w[0] >> 16;
#pragma unroll
            for (int j = 0; j < 8; ++j) q[j] = w[j + 1];
        }
        // q * d rounded to f16 on packed halves: byte b of a dword becomes the
        // f16 1024 + (b ^ 0x80) (exponent byte 0x64 above it), minus 1152
        // gives q exactly, and one f16 multiply rounds q * d once, the same
        // value as rounding the (exact) f32 product.
        const _Float16 dv = keep ? __builtin_bit_cast(_Float16, (uint16_t)dbits) : (_Float16)0.0f;
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
        for (int k = 0; k < 4; ++k) *reinterpret_cast<half8 *>(row + 64 * c + 16 * k) = h[k];
    }
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
// COLS = false: one workgroup per (kv head, row slot), its four waves take
// every fourth tile of the split and merge through LDS.  COLS = true (long
// batches): one workgroup per (row slot, group of up to kColsWaves kv heads),
// wave w serves kv head group * waves + w over every tile of the split and
// writes its own record.  The waves of a workgroup then read whole position
// columns together and the split epilogue needs no workgroup merge.  The
// 136-byte rows of neighbouring kv heads share cache lines, fetched once only
// while the sharers stay close in time: over a long split unsynchronised waves
// drift apart, so a barrier every other loop trip (four tiles) keeps them in
// step (B = 8 over 8k..32k: 452 -> 392 MiB read per layer; a barrier every
// trip reads 377 MiB but waits longer than it saves).
// ONE (per-kv-head layout only): a single sequence, planned from seq_len[0] /
// kv_lo[0] through scalar loads, with a straight-line prologue (see the f16
// kernel).
template <int HD, int G, bool COLS, bool ONE>
__global__ __launch_bounds__(COLS ? 64 * kColsWaves : 256, (COLS || G <= 4) ? 2 : 1)
void decode_q8_kernel(DecodeParams p) {
    static_assert(HD == 64 || HD == 128, "head_dim");
    static_assert(G >= 1 && G <= 8 && (8 % G) == 0, "group size");
    constexpr int NB = HD / 32;          // blocks per row
    constexpr int DB = HD / 32;          // 32-dim blocks of the PV output
    constexpr int VROW = HD * 2 + 16;    // padded LDS row of the f16 V tile
    constexpr int NW = COLS ? kColsWaves : kDecodeWaves;  // most waves per workgroup
    constexpr int QW = COLS ? kColsWaves : 1;             // Q copies (one per kv head)
    constexpr int MW = COLS ? 1 : kDecodeWaves;           // wave records merged in LDS
    constexpr int TS = COLS ? 1 : kDecodeWaves;           // tile stride of a wave

    __shared__ __attribute__((aligned(16))) uint8_t lds_v[NW][kTile * VROW];
    __shared__ __attribute__((aligned(16))) _Float16 lds_p[NW][G][kTile];
    __shared__ float lds_dq[QW][G][NB];
    __shared__ intx4 lds_qa[QW][G][NB][2];
    __shared__ float lds_m[MW][G];
    __shared__ float lds_l[MW][G];
    __shared__ float lds_o[MW][G][HD];

    // slot of kv head kvh's row and the host's guess of its sequence / split
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 31;   // tile position (QK) / MFMA column (PV)
    const int hh = lane >> 5;
    const int grp = (int)blockIdx.x / p.split_row;
    const int slot = (int)blockIdx.x - grp * p.split_row;
    const int kvh = COLS ? grp * ((int)blockDim.x >> 6) + wave : grp;
    const int qw = COLS ? wave : 0;
    int b_g = slot / p.guess_splits;
    if (b_g >= p.n_seq) b_g = p.n_seq - 1;
    const int split_g = slot - b_g * p.guess_splits;
    const int32_t *pt = p.page_table + (int64_t)b_g * p.max_pages;
    const int Hkv = p.n_head_kv;
    const int64_t col_bytes = (int64_t)Hkv * p.row_bytes;
    uint8_t *vt = lds_v[wave];
    const int wave_u = __builtin_amdgcn_readfirstlane(COLS ? 0 : wave);

    // Lane (row n, half hh) loads one contiguous, 4-aligned piece of row n of
    // K and of V: head_dim 128, bytes 68hh .. 68hh + 67 (blocks 2hh and
    // 2hh + 1, 17 dwords); head_dim 64, bytes 32hh .. 32hh + 35 (block hh
    // and two bytes beside it, 9 dwords): five (three) loads per row and
    // tensor.  The V blocks are the ones the lane dequantises; the K operand
    // of block c (quants 16hh .. 16hh + 15) is put together when the tile is
    // consumed, the halves trading their quants across the 32-lane boundary
    // (v_permlane32_swap).  All kept as loaded (arithmetic on them at issue
    // time would make the wave wait for the prefetched tile right where it
    // issues it).  Two such register sets (tiles A and B) alternate: the loop
    // is unrolled by two so each set is loaded and consumed in place, never
    // copied (a copy of a register still being loaded would wait for the
    // load).
    constexpr int KQ = HD / 32;          // 16-byte loads per piece
    using Raw = Q8Raw<HD>;
    PageWindow pages;
    // Tile t's loads (page id pid, wave-uniform) are buffer loads over the
    // kv head's rows of the tile, issued unconditionally: an invalid page gets
    // a zero-byte descriptor (loads return zeros, nothing is read) and false.
    // Every offset is 4-byte aligned (rows are 136 or 68 bytes, columns a
    // multiple of 4, pieces at 68hh or 32hh).
    const int row_lane = n * (int)col_bytes + (HD == 128 ? 68 : 32) * hh;
    auto issue = [&](int t, Raw &r, int32_t pid) -> bool {
        const int pos0 = t * kTile;
        const int lpage = pos0 / p.page_size;
        const uint8_t *kb = page_base(pid, p.k_pages, p.n_pages, p.k_cold, p.n_cold, p.page_bytes);
        const uint8_t *vb = page_base(pid, p.v_pages, p.n_pages, p.v_cold, p.n_cold, p.page_bytes);
        const bool ok = lpage < p.max_pages && kb != nullptr && vb != nullptr;
        const int64_t off = (int64_t)(pos0 - lpage * p.page_size) * col_bytes + (int64_t)kvh * p.row_bytes;
        if constexpr (COLS) {
            // the column layout keeps plain global loads after one page check
            // (with the buffer loads below, or a check per load, the compiler's
            // waits drain the other register set: 104 -> 130 us per B = 8 step)
            if (!ok) return false;
            const uint8_t *kr = kb + off + row_lane;
            const uint8_t *vr = vb + off + row_lane;
#pragma unroll
            for (int j = 0; j < KQ; ++j) r.k4[j] = load16_a4(kr + 16 * j);
            r.k1 = load4_a4(kr + 16 * KQ);
#pragma unroll
            for (int j = 0; j < KQ; ++j) r.v4[j] = load16_a4(vr + 16 * j);
            r.v1 = load4_a4(vr + 16 * KQ);
            return true;
        }
        const int n_rec = ok ? (kTile - 1) * (int)col_bytes + p.row_bytes : 0;
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(ok ? kb + off : p.k_pages), 0, n_rec, kBufferRsrcWord3);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(ok ? vb + off : p.v_pages), 0, n_rec, kBufferRsrcWord3);
        auto ld16 = [&](__amdgpu_buffer_rsrc_t rs, int o) {
            return __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(rs, row_lane + o, 0, 0));
        };
        auto ld4 = [&](__amdgpu_buffer_rsrc_t rs, int o) {
            return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, row_lane + o, 0, 0);
        };
#pragma unroll
        for (int j = 0; j < KQ; ++j) r.k4[j] = ld16(rk, 16 * j);
        r.k1 = ld4(rk, 16 * KQ);
#pragma unroll
        for (int j = 0; j < KQ; ++j) r.v4[j] = ld16(rv, 16 * j);
        r.v1 = ld4(rv, 16 * KQ);
        return ok;
    };
    auto page_of = [&](int t) -> int32_t {
        const int lpage = t * kTile / p.page_size;
        return lpage < p.max_pages ? pages.get(pt, p.max_pages, lpage, lane) : -1;
    };

    // Prologue order as in the f16 kernel: page-id window, seq_len / kv_lo
    // and the lane's Q values are issued before the first tile's K/V burst.
    int t_guess, t_guess_hi;
    split_tiles(0, p.guess_tiles, p.guess_splits, split_g, t_guess, t_guess_hi);
    t_guess = __builtin_amdgcn_readfirstlane(t_guess + wave_u);
    pages.load(pt, p.max_pages, t_guess * kTile / p.page_size, lane);
    int one_n_kv = 0, one_lo = 0;
    PlanRaw raw{0, 0};
    if constexpr (ONE) {
        one_n_kv = p.seq_len[0];
        one_lo = p.kv_lo ? p.kv_lo[0] : 0;
    } else {
        raw = plan_load(p, lane);
    }
    // Q of the g heads of a kv head, one 8-element chunk per thread (one load
    // of each Q value per workgroup: per-lane copies would queue ahead of the
    // first tile's K/V requests); COLS: each wave its own kv head's chunks.
    // Spare threads re-read the last chunk (no branch around the loads).
    static_assert(G * HD / 8 <= 256, "one Q chunk per thread");
    constexpr int QCH = COLS ? (G * HD / 8 + 63) / 64 : 1;  // chunks per thread
    const int q_idx0 = COLS ? lane : (int)threadIdx.x;
    floatx4 qx0[QCH], qx1[QCH];
    auto load_q = [&](int bq) {
        const floatx4 *qr = reinterpret_cast<const floatx4 *>(
            p.q + ((int64_t)bq * p.n_head + (int64_t)kvh * G) * HD);
#pragma unroll
        for (int k = 0; k < QCH; ++k) {
            const int idx = min(q_idx0 + 64 * k, G * HD / 8 - 1);
            qx0[k] = qr[2 * idx];
            qx1[k] = qr[2 * idx + 1];
        }
    };
    load_q(b_g);
    Raw ra, rb;
    // the window starts at the guessed tile's page: its id is lane 0's
    bool ok_a = issue(t_guess, ra, __builtin_amdgcn_readlane(pages.ids, 0));

    SlotPlan sp;
    bool active;
    if constexpr (ONE) {
        sp.g = seq_geom(one_n_kv, one_lo, p.max_pages * p.page_size);
        sp.n_b = splits_of(sp.g.n_tiles, p.one_split ? 0 : p.split_row - 1, sp.g.n_tiles);
        sp.b = 0;
        sp.rec0 = 0;
        sp.split = slot;
        active = slot < sp.n_b;
    } else {
        active = plan(p, raw, slot, -1, lane, sp);
    }
    if (!active) {
        // an idle slot; the merge pass writes the output of a sequence
        // without tiles, or, for one sequence, the slot that would own it
        if (p.n_seq == 1 && slot == 0 && sp.n_b == 0) {
            float *out0 = p.out + (int64_t)kvh * G * HD;
            for (int i = COLS ? lane : (int)threadIdx.x; i < G * HD; i += COLS ? 64 : (int)blockDim.x)
                out0[i] = 0.0f;
        }
        return;
    }
    const int b = sp.b;
    int tile_lo, tile_hi;
    split_tiles(sp.g.t0, sp.g.n_tiles, sp.n_b, sp.split, tile_lo, tile_hi);
    if (b != b_g) {  // a wrong guess: this slot serves another sequence
        pt = p.page_table + (int64_t)b * p.max_pages;
        pages.load(pt, p.max_pages, tile_lo * kTile / p.page_size, lane);
        load_q(b);
    }

    // Q8_0 of Q, the MFMA A operand (lane row n is head n % G, block c,
    // elements 16hh .. 16hh+15), staged in LDS and read per tile.  Chunk i
    // holds dims 8k .. 8k+7 (k = i % (HD/8)) of head i / (HD/8), a quarter of
    // block k / 4; the block's amax is taken over the 4 adjacent lanes.
#pragma unroll
    for (int kq = 0; kq < QCH; ++kq) {
        const floatx4 qa0 = qx0[kq], qa1 = qx1[kq];
        const float x[8] = {qa0[0], qa0[1], qa0[2], qa0[3], qa1[0], qa1[1], qa1[2], qa1[3]};
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(x[j]));
        amax = fmaxf(amax, dpp_row<0xB1>(amax));  // lane ^ 1
        amax = fmaxf(amax, dpp_row<0x4E>(amax));  // lane ^ 2
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        int w[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int q0 = (int)roundf(x[4 * j] * id), q1 = (int)roundf(x[4 * j + 1] * id);
            const int q2 = (int)roundf(x[4 * j + 2] * id), q3 = (int)roundf(x[4 * j + 3] * id);
            w[j] = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | ((int)((unsigned)q3 << 24));
        }
        const int idx = q_idx0 + 64 * kq;
        if (idx < G * HD / 8) {
            const int hq = idx / (HD / 8), k = idx % (HD / 8);
            int *dst = reinterpret_cast<int *>(&lds_qa[qw][hq][k >> 2][(k >> 1) & 1]) + 2 * (k & 1);
            dst[0] = w[0];
            dst[1] = w[1];
            if ((k & 3) == 0) lds_dq[qw][hq][k >> 2] = (float)(_Float16)d;
        }
    }

    const int lo = sp.g.lo, n_kv = sp.g.n_kv;
    float *out_b = p.out + ((int64_t)b * p.n_head + (int64_t)kvh * G) * HD;
    __syncthreads();  // lds_qa, lds_dq (d_q of the heads of output rows i = 0..3,
                      // i.e. rows 4hh + i, head (4hh + i) % G, read per tile)

    int t = tile_lo + wave_u;
    if (t != t_guess || b != b_g) ok_a = t < tile_hi ? issue(t, ra, page_of(t)) : false;

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
        // K operands of the row pair (n, both halves)
        intx4 kop[NB];
        uint32_t kdb[NB];
        q8_k_operand<HD>(r, hh, kop, kdb);
        // S = Q8 * K8^T per block, scaled in block order
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = 0.0f;
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            const intx16 acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(lds_qa[qw][n % G][c][hh], kop[c], intx16{}, 0, 0, 0);
            const float dk = (float)__builtin_bit_cast(_Float16, (uint16_t)kdb[c]);
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[i] += (float)acc[i] * (dk * lds_dq[qw][(4 * hh + i) % G][c]);
            // one block's 16-register accumulator live at a time
            __builtin_amdgcn_sched_barrier(0);
        }
        // V blocks: dequantise into the f16 LDS tile (rows outside [lo, n_kv)
        // zeroed)
        q8_v_row<HD>(r, hh, interior || row_ok, vt + n * VROW);
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
            if (G == 8) {  // selects, not l_run[4hh + i]: a per-lane index puts l_run in scratch
                l_run[i] += hh ? 0.0f : pv[i];
                l_run[4 + i] += hh ? pv[i] : 0.0f;
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
    int trip = 0;
    for (; t < tile_hi; t += 2 * TS) {
        const int t1 = t + TS;
        if (ok_a) consume1(t, ra, sv);
        const bool ok_b = t1 < tile_hi ? issue(t1, rb, page_of(t1)) : false;
        if (ok_a) consume2(t, sv);
        if (t1 >= tile_hi) break;
        if (ok_b) consume1(t1, rb, sv);
        ok_a = t1 + TS < tile_hi ? issue(t1 + TS, ra, page_of(t1 + TS)) : false;
        if (ok_b) consume2(t1, sv);
        // column layout: every wave has the same tiles; keep them in step so
        // the cache lines that neighbouring kv heads share are fetched once
        if constexpr (COLS) {
            if ((++trip & 1) == 0) __syncthreads();
        }
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
    if constexpr (COLS) {
        // this wave's record: column n < g holds head n
        if (n < G) {
            const float inv = l_col > 0.0f ? 1.0f / l_col : 0.0f;
            float *part = p.part + ((int64_t)kvh * p.split_row + sp.rec0 + sp.split) * G * (HD + 4) + n * (HD + 4);
#pragma unroll
            for (int d = 0; d < DB; ++d) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int dim = 32 * d + 8 * (i >> 2) + 4 * hh + (i & 3);
                    if (sp.n_b == 1) out_b[n * HD + dim] = o[d][i] * inv;
                    else part[dim] = o[d][i];
                }
            }
            if (sp.n_b != 1 && hh == 0) {
                part[HD] = m_col;
                part[HD + 1] = l_col;
            }
        }
    } else {
        split_epilogue<HD, G>(o, m_col, l_col, lds_m, lds_l, lds_o, p, kvh, sp.rec0 + sp.split, sp.n_b, out_b,
                              wave, n, hh);
    }
}

// LDS written by some lanes of a wave and then read by others: a wave's LDS
// operations complete in order, so only code motion has to be stopped.  (A
// wavefront-scope fence would also wait for the wave's stage loads into LDS,
// which are counted with the memory loads.)
__device__ inline void wave_lds_sync() {
    __builtin_amdgcn_wave_barrier();
}

// 32-bit LDS address of a pointer into shared memory
__device__ inline uint32_t lds_addr32(const uint8_t *ptr) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)(ptr);
}

// The P^T operand of both PV steps from the lane's row of the wave's P tile
// (address a = positions 4hh ..): halves 16kk + 0..3 and 16kk + 8..11 into
// h[2kk] and h[2kk + 1], then the wait for them (asm for the reason below).
__device__ inline void p_tile_read(uint32_t a, half4 (&h)[4]) {
    asm volatile(
        "ds_read_b64 %0, %4\n"
        "ds_read_b64 %1, %4 offset:16\n"
        "ds_read_b64 %2, %4 offset:32\n"
        "ds_read_b64 %3, %4 offset:48\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(h[0]), "=&v"(h[1]), "=&v"(h[2]), "=&v"(h[3])
        : "v"(a)
        : "memory");
}

// The V^T operand reads of one PV step (k block KK) from the f16 V tile at
// LDS address a: for 32-dim block d and half v, ds_read_b64_tr_b16 at
// a + (16 KK + 8v) * VROW + 64d into h[2d + v], then the wait for them, in
// one asm block.  As the builtin, each read would make the compiler wait for
// every stage load into LDS in flight (it cannot tell the V tile from the
// stage), which would serialise the next tile's loads with this compute.
template <int HD, int VROW, int KK>
__device__ inline void v_tile_tr16(uint32_t a, half4 (&h)[HD / 16]) {
    constexpr int R0 = 16 * KK * VROW, R1 = (16 * KK + 8) * VROW;
    if constexpr (HD == 128) {
        asm volatile(
            "ds_read_b64_tr_b16 %0, %8 offset:%9\n"
            "ds_read_b64_tr_b16 %1, %8 offset:%10\n"
            "ds_read_b64_tr_b16 %2, %8 offset:%11\n"
            "ds_read_b64_tr_b16 %3, %8 offset:%12\n"
            "ds_read_b64_tr_b16 %4, %8 offset:%13\n"
            "ds_read_b64_tr_b16 %5, %8 offset:%14\n"
            "ds_read_b64_tr_b16 %6, %8 offset:%15\n"
            "ds_read_b64_tr_b16 %7, %8 offset:%16\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(h[0]), "=&v"(h[1]), "=&v"(h[2]), "=&v"(h[3]), "=&v"(h[4]), "=&v"(h[5]), "=&v"(h[6]),
              "=&v"(h[7])
            : "v"(a), "n"(R0), "n"(R1), "n"(R0 + 64), "n"(R1 + 64), "n"(R0 + 128), "n"(R1 + 128),
              "n"(R0 + 192), "n"(R1 + 192)
            : "memory");
    } else {
        asm volatile(
            "ds_read_b64_tr_b16 %0, %4 offset:%5\n"
            "ds_read_b64_tr_b16 %1, %4 offset:%6\n"
            "ds_read_b64_tr_b16 %2, %4 offset:%7\n"
            "ds_read_b64_tr_b16 %3, %4 offset:%8\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(h[0]), "=&v"(h[1]), "=&v"(h[2]), "=&v"(h[3])
            : "v"(a), "n"(R0), "n"(R1), "n"(R0 + 64), "n"(R1 + 64)
            : "memory");
    }
}

// Q8_0 decode, batches: R = 4 neighbouring kv heads per wave.  Row n of a
// 32-row tile is position n / R of the tile's P = 8 positions and kv head
// kvh0 + n % R of the workgroup's group, so a tile is P runs of R * row_bytes
// contiguous bytes per tensor.  The wave streams them into its own LDS stage
// in memory order (global_load_lds, 16 bytes per lane, so every load
// instruction covers about 1 KB of consecutive bytes), then each lane reads
// its row piece back from LDS in the layout decode_q8_kernel loads from
// memory.  Lanes loading row pieces straight from memory touch every cache
// line of a tile once per load instruction (five per piece), and that cache
// traffic, not HBM, sets decode_q8_kernel's read rate (3.2 TB/s against about
// 6 for this loop once it runs).  The kernel's fixed prologue and epilogue are
// longer, so it serves batches, whose splits give every wave many tiles.
//   - S = Q8 * K8^T: MFMA rows 8j .. 8j + 7 hold the g heads of kv head j
//     (row 8j + r is head r % g), so tile row n takes output rows
//     8(n % R) + 4hh + i, accumulator registers 4(n % R) + i.
//   - PV: column c of O^T is head c / R of kv head c % R, and the P^T operand
//     is block diagonal: its row n is zero for the columns of other kv heads
//     (those entries are cleared once and never written), so one MFMA
//     sequence per tile serves all R kv heads.
// The split plan is the per-kv-head layout's (32-position tiles, split_row
// slots per kv head, the same records), so the merge passes are shared; the
// 32-position tiles [tile_lo, tile_hi) of a split are R times as many tiles
// of P positions, which the four waves take in turn.  A tile's stage is read
// out before the next tile's loads are issued into it, so one tile is in
// flight while one is computed.
template <int HD, int G, int R>
__global__ __launch_bounds__(64 * (R == 8 ? 8 : 4), R == 8 ? 1 : 2) void decode_q8_staged_kernel(DecodeParams p) {
    static_assert(HD == 64 || HD == 128, "head_dim");
    static_assert(R == 4 || R == 8, "kv heads per workgroup");
    static_assert(G >= 1 && G <= 4, "group size");
    constexpr int NB = HD / 32;        // blocks per row
    constexpr int DB = HD / 32;        // 32-dim blocks of the PV output
    constexpr int VROW = HD * 2 + 16;  // padded LDS row of the f16 V tile
    constexpr int P = kTile / R;       // positions per tile
    constexpr int C = R * G;           // query heads of the workgroup
    constexpr int W = R == 8 ? 8 : 4;  // waves, taking the split's tiles in turn
    constexpr int RB = NB * 34;                       // row bytes
    constexpr int CR = R * RB / 16;                   // 16-byte chunks per position run
    constexpr int CT = P * CR;                        // chunks per tensor and tile
    constexpr int NI = (2 * CT + kWave - 1) / kWave;  // stage load instructions per tile
    constexpr int SB = 2 * CT * 16;                   // stage bytes (K, then V)
    constexpr int PD = HD / 32 * 4 + 1;               // dwords of a lane's row piece
    static_assert(R * RB % 16 == 0, "runs of whole 16-byte chunks");
    static_assert(C * HD * 4 <= SB + kTile * VROW, "the wave's O^T fits its stage and V tile");
    static_assert(C * HD / 8 <= 64 * W, "one Q chunk per thread");
    using Raw = Q8Raw<HD>;
    typedef __attribute__((address_space(3))) void lds_void;

    // per wave: the stage (K chunks 0 .. CT-1 then V chunks, 16 bytes each in
    // memory order), then the f16 V tile; the epilogue reuses both for O^T
    __shared__ __attribute__((aligned(16))) uint8_t lds_sv[W][SB + kTile * VROW];
    __shared__ __attribute__((aligned(16))) _Float16 lds_p[W][C][kTile];
    __shared__ float lds_dq[C][NB];
    __shared__ intx4 lds_qa[C][NB][2];
    __shared__ float lds_m[W][C];
    __shared__ float lds_l[W][C];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 31;  // tile row (QK) / MFMA column (PV)
    const int hh = lane >> 5;
    const int kr = n % R;     // kv head of tile row n and of PV column n
    const int hc = (n / R) % G;  // head of PV column n
    // R = 4: both lane halves hold the scores of tile row n (MFMA rows
    // 8kr + 4hh + i are heads (4hh + i) % g of kv head kr).  R = 8: MFMA rows
    // 4j .. 4j + 3 are kv head j's heads, so output register group jj, half
    // hh holds kv head 2jj + hh: row n's scores are in half kr % 2 only.
    const bool valid = R == 4 || hh == (kr & 1);
    const int jj = R == 4 ? kr : kr >> 1;  // the lane's accumulator register group
    const int grp = (int)blockIdx.x / p.split_row;
    const int slot = (int)blockIdx.x - grp * p.split_row;
    const int kvh0 = grp * R;
    int b_g = slot / p.guess_splits;  // the host's guess of the slot's sequence / split
    if (b_g >= p.n_seq) b_g = p.n_seq - 1;
    const int split_g = slot - b_g * p.guess_splits;
    const int32_t *pt = p.page_table + (int64_t)b_g * p.max_pages;
    const int64_t col_bytes = (int64_t)p.n_head_kv * p.row_bytes;
    uint8_t *stage = lds_sv[wave];
    uint8_t *vt = lds_sv[wave] + SB;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);

    // Chunk q = 64j + lane of a tile (instruction j): tensor q / CT, position
    // run (q % CT) / CR, byte 16 ((q % CT) % CR) of the run.  The last
    // instruction runs only for the lanes of the tile's last chunks.
    int coff[NI];
    bool cvt[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        int q = kWave * j + lane;
        if (q >= 2 * CT) q = 2 * CT - 1;
        const bool v = q >= CT;
        const int rq = v ? q - CT : q;
        coff[j] = (rq / CR) * (int)col_bytes + 16 * (rq % CR);
        cvt[j] = v;
    }
    // Tile u (positions Pu .. Pu + P - 1) of kv heads kvh0 .. kvh0 + R - 1 into
    // the stage; nothing is issued for an invalid page (false)
    PageWindow pages;
    auto issue = [&](int u, int32_t pid) -> bool {
        const int pos0 = u * P;
        const int lpage = pos0 / p.page_size;
        const uint8_t *kb = page_base(pid, p.k_pages, p.n_pages, p.k_cold, p.n_cold, p.page_bytes);
        const uint8_t *vb = page_base(pid, p.v_pages, p.n_pages, p.v_cold, p.n_cold, p.page_bytes);
        const bool ok = lpage < p.max_pages && kb != nullptr && vb != nullptr;
        if (ok) {
            const int64_t off = (int64_t)(pos0 - lpage * p.page_size) * col_bytes + (int64_t)kvh0 * p.row_bytes;
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                const uint8_t *src = (cvt[j] ? vb : kb) + off + coff[j];
                if (kWave * j + kWave <= 2 * CT || lane < 2 * CT - kWave * j)
                    __builtin_amdgcn_global_load_lds(src, (lds_void *)(stage + 1024 * j), 16, 0, 0);
            }
        }
        return ok;
    };
    // lane (n, hh)'s row piece from the stage (the bytes decode_q8_kernel
    // loads: head_dim 128, row bytes 68hh ..; 64, row bytes 32hh ..)
    const uint8_t *piece = stage + (n / R) * (R * RB) + kr * RB + (HD == 128 ? 68 : 32) * hh;
    auto read_stage = [&](Raw &r) {
        const uint32_t *pk = reinterpret_cast<const uint32_t *>(piece);
        const uint32_t *pv = reinterpret_cast<const uint32_t *>(piece + CT * 16);
        uint32_t dk[PD], dv[PD];
#pragma unroll
        for (int w = 0; w < PD; ++w) { dk[w] = pk[w]; dv[w] = pv[w]; }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
#pragma unroll
            for (int e = 0; e < 4; ++e) { r.k4[j][e] = (int)dk[4 * j + e]; r.v4[j][e] = (int)dv[4 * j + e]; }
        }
        r.k1 = dk[PD - 1];
        r.v1 = dv[PD - 1];
    };
    auto page_of = [&](int u) -> int32_t {
        const int lpage = u * P / p.page_size;
        return lpage < p.max_pages ? pages.get(pt, p.max_pages, lpage, lane) : -1;
    };

    // prologue as in decode_q8_kernel: page-id window, seq_len / kv_lo and Q
    // issued before the guessed first tile's K/V burst
    int t_guess, t_guess_hi;
    split_tiles(0, p.guess_tiles, p.guess_splits, split_g, t_guess, t_guess_hi);
    const int u_guess = __builtin_amdgcn_readfirstlane(R * t_guess + wave_u);
    pages.load(pt, p.max_pages, u_guess * P / p.page_size, lane);
    const PlanRaw raw = plan_load(p, lane);
    // Q of the C heads kvh0 * g .. of a sequence (one 8-element chunk per
    // thread)
    const int q_idx = min((int)threadIdx.x, C * HD / 8 - 1);
    floatx4 qa0, qa1;
    auto load_q = [&](int bq) {
        const floatx4 *qr = reinterpret_cast<const floatx4 *>(p.q + ((int64_t)bq * p.n_head + (int64_t)kvh0 * G) * HD);
        qa0 = qr[2 * q_idx];
        qa1 = qr[2 * q_idx + 1];
    };
    load_q(b_g);
    bool ok = issue(u_guess, __builtin_amdgcn_readlane(pages.ids, 0));

    SlotPlan sp;
    if (!plan(p, raw, slot, -1, lane, sp)) {
        // an idle slot (the merge pass writes the output of a sequence
        // without tiles); the stage loads land before the workgroup ends
        __builtin_amdgcn_s_waitcnt(0);
        return;
    }
    const int b = sp.b;
    int tile_lo, tile_hi;
    split_tiles(sp.g.t0, sp.g.n_tiles, sp.n_b, sp.split, tile_lo, tile_hi);
    if (b != b_g) {  // a wrong guess: this slot serves another sequence
        pt = p.page_table + (int64_t)b * p.max_pages;
        pages.load(pt, p.max_pages, tile_lo * kTile / p.page_size, lane);
        load_q(b);
    }
    const int u_hi = R * tile_hi;
    const int lo = sp.g.lo, n_kv = sp.g.n_kv;
    // Q8_0 of Q (as in the per-kv-head kernel), head hq = chunk / (HD / 8)
    {
        const float x[8] = {qa0[0], qa0[1], qa0[2], qa0[3], qa1[0], qa1[1], qa1[2], qa1[3]};
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(x[j]));
        amax = fmaxf(amax, dpp_row<0xB1>(amax));  // lane ^ 1
        amax = fmaxf(amax, dpp_row<0x4E>(amax));  // lane ^ 2
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        int w[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int q0 = (int)roundf(x[4 * j] * id), q1 = (int)roundf(x[4 * j + 1] * id);
            const int q2 = (int)roundf(x[4 * j + 2] * id), q3 = (int)roundf(x[4 * j + 3] * id);
            w[j] = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | ((int)((unsigned)q3 << 24));
        }
        const int idx = threadIdx.x;
        if (idx < C * HD / 8) {
            const int hq = idx / (HD / 8), k = idx % (HD / 8);
            int *dst = reinterpret_cast<int *>(&lds_qa[hq][k >> 2][(k >> 1) & 1]) + 2 * (k & 1);
            dst[0] = w[0];
            dst[1] = w[1];
            if ((k & 3) == 0) lds_dq[hq][k >> 2] = (float)(_Float16)d;
        }
    }
    // the wave's P^T tile starts all zero: entries of another kv head stay so
    for (int i = lane; i < C * kTile / 8; i += kWave) reinterpret_cast<half8 *>(&lds_p[wave][0][0])[i] = half8{};
    __syncthreads();

    // A operand row n: R = 4: head (n % 8) % g of kv head n / 8 (rows past
    // the group repeat its last kv head; their outputs are not read); R = 8:
    // head (n % 4) % g of kv head n / 4.  d_q of the lane's output rows.
    const int hq_a = R == 4 ? min(n / 8, R - 1) * G + (n % 8) % G : (n / 4) * G + (n % 4) % G;
    float dqr[NB][4];
#pragma unroll
    for (int c = 0; c < NB; ++c) {
#pragma unroll
        for (int i = 0; i < 4; ++i) dqr[c][i] = lds_dq[kr * G + (R == 4 ? (4 * hh + i) : i) % G][c];
    }


    // the lane's accumulator group (registers 4jj .. 4jj + 3) is picked with
    // all-ones / zero masks that the optimiser cannot see through: written as
    // selects between elements of one vector, the choice becomes a
    // variable-index extract, a compare and select per element
    int gmask[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int m = jj == j ? -1 : 0;
        asm volatile("" : "+v"(m));
        gmask[j] = m;
    }
    // head of the lane's score register i (valid lanes)
    auto head_i = [&](int i) { return R == 4 ? head_of<G>(i, hh) : i % G; };

    int u = R * tile_lo + wave_u;
    if (u != u_guess || b != b_g) {
        // the guessed tile's loads land before the real ones overwrite the stage
        __builtin_amdgcn_s_waitcnt(0);
        ok = u < u_hi ? issue(u, page_of(u)) : false;
    }

    floatx16 o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) o[d] = floatx16{};
    float m_run[G], l_run[G], alpha_h[G];  // of kv head kr (valid lanes)
#pragma unroll
    for (int h = 0; h < G; ++h) { m_run[h] = -INFINITY; l_run[h] = 0.0f; alpha_h[h] = 1.0f; }
    bool first = true;

    auto consume1 = [&](int u, const Raw &r, float (&sv)[4]) {
        const int pos0 = u * P;
        const bool row_ok = pos0 + n / R >= lo && pos0 + n / R < n_kv;
        const bool interior = pos0 >= lo && pos0 + P <= n_kv;
        intx4 kop[NB];
        uint32_t kdb[NB];
        q8_k_operand<HD>(r, hh, kop, kdb);
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = 0.0f;
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            const intx16 acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(lds_qa[hq_a][c][hh], kop[c], intx16{}, 0, 0, 0);
            const float dk = (float)__builtin_bit_cast(_Float16, (uint16_t)kdb[c]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int a = acc[i] & gmask[0];
#pragma unroll
                for (int j = 1; j < 4; ++j) a |= acc[4 * j + i] & gmask[j];
                sv[i] += (float)a * (dk * dqr[c][i]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        q8_v_row<HD>(r, hh, interior || row_ok, vt + n * VROW);
    };
    auto consume2 = [&](int u, float (&sv)[4]) {
        const int pos0 = u * P;
        const bool row_ok = pos0 + n / R >= lo && pos0 + n / R < n_kv;
        const bool interior = pos0 >= lo && pos0 + P <= n_kv;
        // online softmax of kv head kr's heads over the lanes holding that kv
        // head (R = 4: lanes n' = n mod 4, both halves; R = 8: n' = n mod 8 in
        // half kr % 2)
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = (valid && (interior || row_ok)) ? sv[i] * p.scale_log2 : -INFINITY;
        bool exceed = false;
#pragma unroll
        for (int i = 0; i < 4; ++i) exceed |= sv[i] > m_run[head_i(i)] + kRescaleLog2;
        if (__any(exceed)) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float mt = -INFINITY;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (head_i(i) == h) mt = fmaxf(mt, sv[i]);
#pragma unroll
                for (int off = R; off < (R == 4 ? 64 : 32); off <<= 1) mt = fmaxf(mt, __shfl_xor(mt, off, 64));
                const float m_new = fmaxf(m_run[h], mt);
                // m_run == -inf -> 0; a lane without this kv head's scores
                // keeps factor 1
                const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run[h] - m_new);
                l_run[h] *= alpha;
                alpha_h[h] = alpha;
                m_run[h] = m_new;
            }
            if (!first) {
                float a = alpha_h[0];
#pragma unroll
                for (int h = 1; h < G; ++h) a = hc == h ? alpha_h[h] : a;
                // R = 8: PV column n's factor is in the lane holding its scores.
                // Every lane takes part in the exchange: written as
                // valid ? a : xor32(a), the compiler ran the lane exchange
                // only in the lanes that use it, with their partner lanes
                // switched off, so it read nothing from them.  The empty asm
                // keeps the exchange in the uniform code.
                if constexpr (R == 8) {
                    float ax = xor32(a);
                    asm volatile("" : "+v"(ax));
                    a = valid ? a : ax;
                }
#pragma unroll
                for (int d = 0; d < DB; ++d) o[d] *= a;
            }
        }
        first = false;
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float mr = m_run[head_i(i)];
            pv[i] = __builtin_amdgcn_exp2f(sv[i] - (mr == -INFINITY ? 0.0f : mr));
        }
        // each (kv head, head, position) counted once: R = 4 half 0, R = 8 the
        // valid half
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i < G && (R == 8 ? valid : hh == 0)) l_run[i] += pv[i];
        }
        // P -> LDS [PV column of (kv head kr, head)][tile row]
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i < G && valid) lds_p[wave][kr + R * head_i(i)][n] = (_Float16)pv[i];
        }

        wave_lds_sync();

        half8 pb[2];
        {
            half4 a[4];
            p_tile_read(lds_addr32(reinterpret_cast<const uint8_t *>(&lds_p[wave][kr + R * hc][4 * hh])), a);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
                for (int j = 0; j < 4; ++j) { pb[kk][j] = a[2 * kk][j]; pb[kk][4 + j] = a[2 * kk + 1][j]; }
            }
        }
        {
            const int gq = lane >> 4, rr = lane & 15;
            const uint8_t *vsrc = vt + (4 * (gq >> 1) + (rr >> 2)) * VROW + 2 * (16 * (gq & 1) + 4 * (rr & 3));
            const uint32_t va_base = lds_addr32(vsrc);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                half4 h[2 * DB];
                if (kk == 0)
                    v_tile_tr16<HD, VROW, 0>(va_base, h);
                else
                    v_tile_tr16<HD, VROW, 1>(va_base, h);
#pragma unroll
                for (int d = 0; d < DB; ++d) {
                    half8 va;
#pragma unroll
                    for (int e = 0; e < 4; ++e) { va[e] = h[2 * d][e]; va[4 + e] = h[2 * d + 1][e]; }
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[kk], o[d], 0, 0, 0);
                }
            }
        }
        wave_lds_sync();
    };

    // per tile: wait for the stage, read it out, issue the next tile into it,
    // then compute
    float sv[4];
    for (; u < u_hi; u += W) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        Raw r;
        read_stage(r);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int un = u + W;
        const bool ok_n = un < u_hi ? issue(un, page_of(un)) : false;
        if (ok) {
            consume1(u, r, sv);
            consume2(u, sv);
        }
        ok = ok_n;
    }
    // no stage load in flight once the loop ends (the last issue was for a
    // tile past the split): stage and V tile now take the waves' O^T

    // per-(kv head, head) sums over the lanes holding the kv head
    float Lh[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float v = l_run[h];
#pragma unroll
        for (int off = R; off < (R == 4 ? 64 : 32); off <<= 1) v += __shfl_xor(v, off, 64);
        Lh[h] = v;
    }
    auto lds_o = [&](int w) { return reinterpret_cast<float (*)[HD]>(lds_sv[w]); };
    float m_col = m_run[0], l_col = Lh[0];
#pragma unroll
    for (int h = 1; h < G; ++h)
        if (hc == h) { m_col = m_run[h]; l_col = Lh[h]; }
    if (n < C) {
        if (R == 8 ? valid : hh == 0) {
            lds_m[wave][n] = m_col;
            lds_l[wave][n] = l_col;
        }
#pragma unroll
        for (int d = 0; d < DB; ++d) {
#pragma unroll
            for (int i = 0; i < 16; ++i) lds_o(wave)[n][32 * d + 8 * (i >> 2) + 4 * hh + (i & 3)] = o[d][i];
        }
    }
    __syncthreads();
    // each column's wave weights once, one thread per column, in place:
    // lds_m[w][c] <- wave w's weight 2^(m_w - M), lds_l[0][c] <- L, lds_l[1][c] <- M
    if ((int)threadIdx.x < C) {
        const int c = threadIdx.x;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, lds_m[w][c]);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float mw = lds_m[w][c];
            const float wt = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
            L += lds_l[w][c] * wt;
            lds_m[w][c] = wt;
        }
        lds_l[0][c] = L;
        lds_l[1][c] = M;
    }
    __syncthreads();
    // the waves' (m, l, o) -> the split's record of each (kv head, head), or
    // the output when the sequence has one split
    for (int idx = threadIdx.x; idx < C * HD; idx += blockDim.x) {
        const int c = idx / HD, d = idx % HD;
        const int kvh = kvh0 + c % R, h = c / R;
        float O = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) O += lds_o(w)[c][d] * lds_m[w][c];
        const float L = lds_l[0][c], M = lds_l[1][c];
        if (sp.n_b == 1) {
            p.out[((int64_t)b * p.n_head + (int64_t)kvh * G + h) * HD + d] = L > 0.0f ? O / L : 0.0f;
        } else {
            float *part = p.part + ((int64_t)kvh * p.split_row + sp.rec0 + sp.split) * G * (HD + 4) + h * (HD + 4);
            part[d] = O;
            if (d == 0) {
                part[HD] = M;
                part[HD + 1] = L;
            }
        }
    }
}

// Second pass: out = sum_s o_s * 2^(m_s - M) / sum_s l_s * 2^(m_s - M) over
// the active splits of each (sequence, kv head), M the largest m_s.  One
// workgroup per (b, kv head, group head), one thread per dim.  For one
// sequence every load of the first 64 splits (the lane-parallel (m, l) of all
// splits and this dim's o_s) is issued before seq_len is read, so the kernel
// waits on memory once; in a batch the plan (from every seq_len) first places
// the sequence's records in the row.  Split indices past the sequence's are
// clamped (the loads stay inside the workspace) and their weights are zero.
// A batch sequence without tiles gets a zero output here.  The code is
// branch-free straight-line work: the pass is latency-bound and each taken
// branch or instruction-cache miss adds to it.  CH partial rows are loaded
// per round (64; 32 would suit a row of at most 32 slots, which the small
// merges below serve); the (m, l) of split s sit in lane s % 64 of register
// s / 64.  Rows of at most 64 slots take the small merges.
template <int HD, int G, bool ONE, int CH>
__global__ __launch_bounds__(kMergeThreads<HD>) void decode_merge_kernel(DecodeParams p) {
    static_assert(CH == 32 || CH == 64, "round size");
    // (m, l) registers per lane: one when the row has at most 32 slots
    constexpr int RMAX = CH == 32 ? 1 : (kMaxSplits + kWave - 1) / kWave;
    const int g = blockIdx.x % G;
    const int kvh = (blockIdx.x / G) % p.n_head_kv;
    const int b = blockIdx.x / (G * p.n_head_kv);
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int d = tid < HD ? tid : HD - 1;  // threads past HD (HD < 64) only load (m, l)
    const int sstride = G * (HD + 4);
    const float *row0 = p.part + (int64_t)kvh * p.split_row * sstride + g * (HD + 4);

    float o[CH];
    float mv[RMAX], lv[RMAX];
    // the rows of splits s0 .. s0 + CH - 1 of the sequence's records at pg,
    // indices clamped to the S records (wave-uniform, always in bounds)
    auto load_round = [&](const float *pg, int s0, int S) {
#pragma unroll
        for (int u = 0; u < CH; ++u) o[u] = pg[(int64_t)min(s0 + u, S - 1) * sstride + d];
    };
    auto load_ml = [&](const float *pg, int S) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            const int s = min(kWave * r + lane, S - 1);
            mv[r] = pg[(int64_t)s * sstride + HD];
            lv[r] = pg[(int64_t)s * sstride + HD + 1];
        }
    };
    int n_active, rec0 = 0, S;
    if constexpr (ONE) {
        // one sequence owns the row from slot 0: every load of the first CH
        // splits and the (m, l) of all goes out before seq_len (scalar loads,
        // their own counter) is known
        S = p.split_row;
        load_round(row0, 0, S);
        load_ml(row0, S);
        const SeqGeom sg = seq_geom(p.seq_len[0], p.kv_lo ? p.kv_lo[0] : 0, p.max_pages * p.page_size);
        n_active = splits_of(sg.n_tiles, p.one_split ? 0 : p.split_row - 1, sg.n_tiles);
    } else {
        // in a batch the plan (from every seq_len) places the sequence's
        // records in the row first
        const PlanRaw raw = plan_load(p, lane);
        SlotPlan sp;
        plan_lanes(p, raw, 0, b, lane, sp);  // per-lane selects below; no scalar copy needed
        rec0 = sp.rec0;
        S = sp.n_b > 0 ? sp.n_b : 1;
        n_active = sp.n_b;
        load_round(row0 + (int64_t)rec0 * sstride, 0, S);
        load_ml(row0 + (int64_t)rec0 * sstride, S);
    }
    const float *pg = row0 + (int64_t)rec0 * sstride;
    if (n_active <= 1) {
        // one split: written by the split pass; none (a batch sequence with
        // no tiles): the output is zero
        if (!ONE && n_active == 0 && tid < HD)
            p.out[((int64_t)b * p.n_head + (int64_t)kvh * G + g) * HD + tid] = 0.0f;
        return;
    }

    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
        mv[r] = kWave * r + lane < n_active ? mv[r] : -INFINITY;
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
    for (int r = 0; r < kMaxSplits / CH; ++r) {
        if (CH * r >= n_active) break;
        if (r > 0) load_round(pg, CH * r, S);
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int sp = CH * r + u;  // compile-time
            const float wt = lane_val(w[sp / kWave], sp % kWave);
            O = wt != 0.0f ? fmaf(o[u], wt, O) : O;
        }
    }
    if (tid < HD) {
        float *out = p.out + ((int64_t)b * p.n_head + (int64_t)kvh * G + g) * HD;
        out[tid] = L > 0.0f ? O / L : 0.0f;
    }
}

// The merge pass of one sequence whose kv-head rows have at most SM = 32 or
// 64 slots (the B = 1 decode up to 16k positions, or 32k at 64 splits): the
// pass waits on one round of loads, so it is the number of load instructions
// per wave that sets its length.  Thread t takes dims 4(t % (HD/4)) .. + 3 of
// the splits t / (HD/4) + NG*i (16-byte loads, NG split groups), every lane
// the (m, l) of split lane % SM; each group's weighted rows are summed in LDS
// in group order.  At HD = 128, 6 loads per thread for 32 slots and 10 for 64
// (the general merge issues 34 and 66).
template <int HD, int G, int SM>
__global__ __launch_bounds__(256) void decode_merge_small_kernel(DecodeParams p) {
    static_assert(SM == 32 || SM == 64, "slots");
    constexpr int TPG = HD / 4;             // threads per split group
    constexpr int NG = 256 / TPG;           // split groups
    constexpr int SPT = (SM + NG - 1) / NG; // splits per thread
    __shared__ floatx4 acc_g[NG][TPG];
    const int g = (int)blockIdx.x % G;
    const int kvh = (int)blockIdx.x / G;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int dc = tid % TPG, grp = tid / TPG;
    const int sstride = G * (HD + 4);
    const int S = p.split_row;  // <= SM
    const float *row0 = p.part + (int64_t)kvh * S * sstride + g * (HD + 4);
    // every load before seq_len (scalar loads, their own counter) is known
    const int sl = min(lane & (SM - 1), S - 1);
    const float m_raw = row0[(int64_t)sl * sstride + HD];
    const float l_raw = row0[(int64_t)sl * sstride + HD + 1];
    floatx4 o[SPT];
#pragma unroll
    for (int i = 0; i < SPT; ++i)
        o[i] = *reinterpret_cast<const floatx4 *>(row0 + (int64_t)min(grp + NG * i, S - 1) * sstride + 4 * dc);
    const SeqGeom sg = seq_geom(p.seq_len[0], p.kv_lo ? p.kv_lo[0] : 0, p.max_pages * p.page_size);
    const int n_active = splits_of(sg.n_tiles, p.one_split ? 0 : S - 1, sg.n_tiles);
    if (n_active <= 1) return;  // the split pass wrote the output

    const bool act = (lane & (SM - 1)) < n_active && lane < SM;
    const float m = act ? m_raw : -INFINITY;
    const float M = wave_max(m);
    const float w = m != -INFINITY ? __builtin_amdgcn_exp2f(m - M) : 0.0f;  // lane s: split s
    const float L = wave_sum(w != 0.0f ? l_raw * w : 0.0f);
    floatx4 acc = floatx4{};
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
        const int s = grp + NG * i;
        const float wt = __shfl(w, s & (SM - 1), 64);
        if (s < SM && wt != 0.0f) {
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = fmaf(o[i][e], wt, acc[e]);
        }
    }
    acc_g[grp][dc] = acc;
    __syncthreads();
    if (tid < TPG) {
        floatx4 O = acc_g[0][tid];
#pragma unroll
        for (int k = 1; k < NG; ++k) O += acc_g[k][tid];
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        floatx4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = L > 0.0f ? O[e] * inv : 0.0f;
        *reinterpret_cast<floatx4 *>(p.out + ((int64_t)kvh * G + g) * HD + 4 * tid) = r;
    }
}

// The merge pass of one sequence whose kv-head rows have 65 .. 256 slots (B =
// 1 at long context with few kv heads, or many splits per kv head): one
// workgroup per (kv head, group head, 32 dims), so the rows' bytes spread over
// Hkv * g * HD / 32 workgroups and every load goes out in one round.  Thread
// t takes 4 dims (t % 8) of the splits t / 8 + 32 i; lane s holds the (m, l)
// of splits s + 64 r; the 32 split groups' weighted sums are added in LDS in
// group order.
template <int HD, int G>
__global__ __launch_bounds__(256) void decode_merge_wide_kernel(DecodeParams p) {
    constexpr int DQ = HD / 32;                        // 32-dim slices
    constexpr int RM = kMaxSplits / kWave;             // (m, l) registers per lane
    constexpr int SPT = kMaxSplits / 32;               // splits per thread
    static_assert(HD % 32 == 0, "32-dim slices");
    __shared__ floatx4 acc_g[32][8];
    const int q4 = (int)blockIdx.x % DQ;
    const int g = ((int)blockIdx.x / DQ) % G;
    const int kvh = (int)blockIdx.x / (DQ * G);
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int dc = tid & 7, sg = tid >> 3;
    const int sstride = G * (HD + 4);
    const int S = p.split_row;  // <= kMaxSplits
    const float *row0 = p.part + (int64_t)kvh * S * sstride + g * (HD + 4);
    // every load before seq_len (scalar loads, their own counter) is known
    float mv[RM], lv[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        const int sl = min(lane + kWave * r, S - 1);
        mv[r] = row0[(int64_t)sl * sstride + HD];
        lv[r] = row0[(int64_t)sl * sstride + HD + 1];
    }
    floatx4 o[SPT];
#pragma unroll
    for (int i = 0; i < SPT; ++i)
        o[i] = *reinterpret_cast<const floatx4 *>(row0 + (int64_t)min(sg + 32 * i, S - 1) * sstride + 32 * q4 + 4 * dc);
    const SeqGeom sgeo = seq_geom(p.seq_len[0], p.kv_lo ? p.kv_lo[0] : 0, p.max_pages * p.page_size);
    const int n_active = splits_of(sgeo.n_tiles, p.one_split ? 0 : S - 1, sgeo.n_tiles);
    if (n_active <= 1) return;  // the split pass wrote the output

    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        mv[r] = lane + kWave * r < n_active ? mv[r] : -INFINITY;
        mx = fmaxf(mx, mv[r]);
    }
    const float M = wave_max(mx);
    float w[RM], lsum = 0.0f;
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        w[r] = mv[r] != -INFINITY ? __builtin_amdgcn_exp2f(mv[r] - M) : 0.0f;  // lane s: split s + 64 r
        lsum += w[r] != 0.0f ? lv[r] * w[r] : 0.0f;
    }
    const float L = wave_sum(lsum);
    floatx4 acc = floatx4{};
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
        // split sg + 32 i sits in lane sg + 32 (i % 2) of register i / 2
        const float wt = __shfl(w[i / 2], sg + 32 * (i % 2), kWave);
        if (wt != 0.0f) {
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = fmaf(o[i][e], wt, acc[e]);
        }
    }
    acc_g[sg][dc] = acc;
    __syncthreads();
    if (tid < 8) {
        floatx4 O = acc_g[0][tid];
#pragma unroll
        for (int k = 1; k < 32; ++k) O += acc_g[k][tid];
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        floatx4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = L > 0.0f ? O[e] * inv : 0.0f;
        *reinterpret_cast<floatx4 *>(p.out + ((int64_t)kvh * G + g) * HD + 32 * q4 + 4 * tid) = r;
    }
}

// The merge pass of a batch whose kv-head rows have at most 64 slots (f16 and
// F32 batches with 8 or more kv heads): the small single-sequence merge's
// loads (16-byte loads of split groups, every lane the (m, l) of one split).
// They go out from the host's guess of the sequence's records (every sequence
// at max_seq_len: slots b * guess_splits ..) before the plan is known, and
// again from the planned slots only when the guess was wrong.  A sequence
// without tiles gets a zero output; one with a single split was written by
// the split pass.
template <int HD, int G>
__global__ __launch_bounds__(256) void decode_merge_batch_small_kernel(DecodeParams p) {
    constexpr int TPG = HD / 4;             // threads per split group
    constexpr int NG = 256 / TPG;           // split groups
    constexpr int SPT = (kWave + NG - 1) / NG;  // splits per thread
    __shared__ floatx4 acc_g[NG][TPG];
    const int g = blockIdx.x % G;
    const int kvh = (blockIdx.x / G) % p.n_head_kv;
    const int b = blockIdx.x / (G * p.n_head_kv);
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int dc = tid % TPG, grp = tid / TPG;
    const int sstride = G * (HD + 4);
    const float *row0 = p.part + (int64_t)kvh * p.split_row * sstride + g * (HD + 4);
    float m_raw, l_raw;
    floatx4 o[SPT];
    // records rec .. rec + S - 1 (indices clamped into them)
    auto load = [&](int rec, int S) {
        const float *pg = row0 + (int64_t)rec * sstride;
        const int sl = min(lane, S - 1);
        m_raw = pg[(int64_t)sl * sstride + HD];
        l_raw = pg[(int64_t)sl * sstride + HD + 1];
#pragma unroll
        for (int i = 0; i < SPT; ++i)
            o[i] = *reinterpret_cast<const floatx4 *>(pg + (int64_t)min(grp + NG * i, S - 1) * sstride + 4 * dc);
    };
    // the plan's inputs first: the plan is worked out while the guessed
    // records are in flight
    const PlanRaw raw = plan_load(p, lane);
    const int rec_g = b * p.guess_splits;  // the guess stays inside the row
    load(rec_g, p.guess_splits);
    SlotPlan sp;
    plan_lanes(p, raw, 0, b, lane, sp);
    const int n_active = __builtin_amdgcn_readfirstlane(sp.n_b);
    const int rec0 = __builtin_amdgcn_readfirstlane(sp.rec0);
    // records past n_active get weight zero, so the guess serves when it
    // starts at rec0 and covers n_active of them
    if (n_active > 1 && (rec0 != rec_g || n_active > p.guess_splits)) load(rec0, n_active);
    float *out = p.out + ((int64_t)b * p.n_head + (int64_t)kvh * G + g) * HD;
    if (n_active <= 1) {
        if (n_active == 0 && tid < HD) out[tid] = 0.0f;
        return;
    }

    const bool act = lane < n_active;
    const float m = act ? m_raw : -INFINITY;
    const float M = wave_max(m);
    const float w = m != -INFINITY ? __builtin_amdgcn_exp2f(m - M) : 0.0f;  // lane s: split s
    const float L = wave_sum(w != 0.0f ? l_raw * w : 0.0f);
    floatx4 acc = floatx4{};
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
        const int s = grp + NG * i;
        const float wt = __shfl(w, s & (kWave - 1), kWave);
        if (s < kWave && wt != 0.0f) {
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = fmaf(o[i][e], wt, acc[e]);
        }
    }
    acc_g[grp][dc] = acc;
    __syncthreads();
    if (tid < TPG) {
        floatx4 O = acc_g[0][tid];
#pragma unroll
        for (int k = 1; k < NG; ++k) O += acc_g[k][tid];
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        floatx4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = L > 0.0f ? O[e] * inv : 0.0f;
        *reinterpret_cast<floatx4 *>(out + 4 * tid) = r;
    }
}

// ---- host side -------------------------------------------------------------

struct SplitPlan {
    int split_row;     // slots per kv head
    int guess_splits;  // splits per sequence if every sequence had max_seq_len from 0
    int guess_tiles;
};

// About 2048 waves (two per SIMD at these register footprints, over 256 CUs):
// the row of each kv head gets 2048 / (Hkv * waves per slot) slots (512 four-
// wave workgroups; with the column layout one wave per (slot, kv head)), at
// most kMaxSplits, no more than the batch could use (every sequence's widest
// span of max_seq_len positions, which covers one tile more when a window start
// is not tile-aligned, cut into kDecodeWaves-tile splits), at least B, rounded
// up to a multiple of 8.  The device plan deals the slots out by length.
// One sequence over a Q8_0 cache (`one_q8`) takes half the slots: one
// workgroup per CU with twice the tiles per wave (Mixtral shape, per layer:
// 32k 25.0 -> 24.2 us, 8k 13.0 -> 12.4 us; f16 at 32k gains nothing, and a
// quarter of the slots leaves CUs idle: 35.0 us).
SplitPlan plan_splits(int B, int Hkv, int max_seq_len, bool windowed, bool cols, bool one_q8) {
    const int slot_target = cols ? 2048 : (one_q8 ? 1024 : 2048) / kDecodeWaves;
    const int tiles = ceil_div(max_seq_len, kTile);
    const int span_tiles = windowed ? ceil_div(max_seq_len - 1, kTile) + 1 : tiles;
    int row = (slot_target + Hkv - 1) / Hkv;
    if (row > kMaxSplits) row = kMaxSplits;
    const long long most = (long long)B * ceil_div(span_tiles, kDecodeWaves);
    if (row > most) row = (int)most;
    if (row < B) row = B;
    row = (row + 7) / 8 * 8;
    // the guess, with the device's rule: every sequence max_seq_len from 0
    const int avail = row - B;
    const int g = splits_of(tiles, avail / B, tiles);
    return SplitPlan{row, g > 0 ? g : 1, tiles};
}

// The column layout of the Q8_0 kernel (g <= 4) serves batches of two or more
// sequences with at least kColsMinTiles tiles in all (B times the widest span).
// One sequence keeps the per-kv-head layout: its merge pass then reads 4x the
// records over only Hkv * g workgroups (B = 1 at 32k: 27.6 -> 33.2 us per
// layer with the column layout, B = 8 over 8k..32k: 107.6 -> 103.6 us).
constexpr long long kColsMinTiles = 1024;
bool use_cols(int kv_type, int HD, int G, int B, int max_seq_len, bool windowed) {
    if (kv_type != SFA_KV_Q8_0 || HD < 64 || G > 4 || B < 2) return false;
    const int tiles = ceil_div(max_seq_len, kTile);
    const int span_tiles = windowed ? ceil_div(max_seq_len - 1, kTile) + 1 : tiles;
    return (long long)B * span_tiles >= kColsMinTiles;
}

// The staged Q8_0 kernel takes the column layout's batches when its workgroup
// of kStagedKv kv heads divides the kv heads (g <= 4 already holds there).  It
// plans the column layout's row: 2048 / Hkv slots, kStagedKv kv heads per
// four-wave workgroup.
bool use_staged(int Hkv) { return Hkv % kStagedKv == 0; }

// kv heads per column-layout workgroup: the largest of 8, 4, 2, 1 dividing Hkv
int cols_waves_of(int Hkv) {
    for (int w = kColsWaves; w > 1; w /= 2)
        if (Hkv % w == 0) return w;
    return 1;
}

size_t decode_workspace_bytes(int B, int Hkv, int G, int HD, int max_seq_len) {
    // the larger row of both layouts, windowed (one tile more)
    const SplitPlan a = plan_splits(B, Hkv, max_seq_len, true, false, false);
    const SplitPlan c = plan_splits(B, Hkv, max_seq_len, true, true, false);
    const int row = a.split_row > c.split_row ? a.split_row : c.split_row;
    return (size_t)Hkv * row * G * (HD + 4) * sizeof(float);
}

template <int HD, int G>
static void launch_merge(const DecodeParams &p, int B, int Hkv, int passes, hipStream_t s) {
    if ((passes & 2) && !p.one_split) {
        const bool small = p.split_row <= 32;
        if (B == 1) {
            if (small)
                hipLaunchKernelGGL((decode_merge_small_kernel<HD, G, 32>), dim3(Hkv * G), dim3(256), 0, s, p);
            else if (p.split_row <= 64)
                hipLaunchKernelGGL((decode_merge_small_kernel<HD, G, 64>), dim3(Hkv * G), dim3(256), 0, s, p);
            else if constexpr (HD % 32 == 0)
                hipLaunchKernelGGL((decode_merge_wide_kernel<HD, G>), dim3(Hkv * G * (HD / 32)), dim3(256), 0, s,
                                   p);
        } else {
            if (p.split_row <= kWave)
                hipLaunchKernelGGL((decode_merge_batch_small_kernel<HD, G>), dim3(B * Hkv * G), dim3(256), 0, s, p);
            else
                hipLaunchKernelGGL((decode_merge_kernel<HD, G, false, 64>), dim3(B * Hkv * G),
                                   dim3(kMergeThreads<HD>), 0, s, p);
        }
    }
}

// pass bit 1: split-K pass, bit 2: merge pass
template <int HD, int G>
static void launch_f16(const DecodeParams &p, int B, int Hkv, int passes, hipStream_t s) {
    if (passes & 1) {
        dim3 grid(p.split_row * Hkv);
        if (p.kv_type == SFA_KV_Q8_0) {
            if constexpr (HD >= 64 && G <= 4) {
                if (p.staged) {
                    // eight kv heads (whole position columns) per workgroup
                    // when 8 | Hkv, else four
                    if (Hkv % 8 == 0)
                        hipLaunchKernelGGL((decode_q8_staged_kernel<HD, G, 8>), dim3(p.split_row * (Hkv / 8)),
                                           dim3(512), 0, s, p);
                    else
                        hipLaunchKernelGGL((decode_q8_staged_kernel<HD, G, 4>), dim3(p.split_row * (Hkv / 4)),
                                           dim3(256), 0, s, p);
                    return launch_merge<HD, G>(p, B, Hkv, passes, s);
                }
                if (p.cols_waves > 0) {
                    hipLaunchKernelGGL((decode_q8_kernel<HD, G, true, false>), dim3(p.split_row * (Hkv / p.cols_waves)),
                                       dim3(64 * p.cols_waves), 0, s, p);
                    return launch_merge<HD, G>(p, B, Hkv, passes, s);
                }
            }
            if constexpr (HD >= 64 && G <= 8)
            {
                if (B == 1)
                    hipLaunchKernelGGL((decode_q8_kernel<HD, G, false, true>), grid, dim3(256), 0, s, p);
                else
                    hipLaunchKernelGGL((decode_q8_kernel<HD, G, false, false>), grid, dim3(256), 0, s, p);
            }
        } else if (p.kv_type == SFA_KV_F32) {
            if (p.app_k != nullptr)
                hipLaunchKernelGGL((decode_f32_kernel<HD, G, true>), grid, dim3(256), 0, s, p);
            else
                hipLaunchKernelGGL((decode_f32_kernel<HD, G>), grid, dim3(256), 0, s, p);
        } else if (p.app_k != nullptr) {
            if (B == 1)
                hipLaunchKernelGGL((decode_f16_kernel<HD, G, true, true>), grid, dim3(256), 0, s, p);
            else
                hipLaunchKernelGGL((decode_f16_kernel<HD, G, false, true>), grid, dim3(256), 0, s, p);
        } else {
            if (B == 1)
                hipLaunchKernelGGL((decode_f16_kernel<HD, G, true>), grid, dim3(256), 0, s, p);
            else
                hipLaunchKernelGGL((decode_f16_kernel<HD, G, false>), grid, dim3(256), 0, s, p);
        }
    }
    launch_merge<HD, G>(p, B, Hkv, passes, s);
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

int decode_setup(const sfa_kv_desc *kv, const float *q, float *out, const int32_t *page_table,
                 int32_t max_pages, const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                 int32_t max_seq_len, float scale, void *workspace, size_t ws_bytes,
                 DecodeParams *out_p) {
    const int Hkv = kv->n_head_kv, HD = kv->head_dim, G = kv->n_head / kv->n_head_kv;
    if (B <= 0 || max_seq_len <= 0 || max_pages <= 0) return SFA_ERR_INVALID_ARGUMENT;
    // the split plan sums tile counts over the batch in 32-bit integers
    const long long cap_tiles = ceil_div((long long)max_pages * kv->page_size, (long long)kTile);
    if ((long long)B * cap_tiles > kMaxPlanTiles)
        return SFA_ERR_INVALID_ARGUMENT;
    if (q == nullptr || out == nullptr || page_table == nullptr || seq_len == nullptr)
        return SFA_ERR_INVALID_ARGUMENT;
    const size_t need = decode_workspace_bytes(B, Hkv, G, HD, max_seq_len);
    if (workspace == nullptr || ws_bytes < need) return SFA_ERR_INVALID_ARGUMENT;
    if (kv->kv_type != SFA_KV_F32 && kv->kv_type != SFA_KV_F16 && kv->kv_type != SFA_KV_Q8_0)
        return SFA_ERR_UNSUPPORTED;
    if (kv->kv_type == SFA_KV_Q8_0 && HD < 64) return SFA_ERR_UNSUPPORTED;
    const bool cols = use_cols(kv->kv_type, HD, G, B, max_seq_len, kv_lo != nullptr);
    const SplitPlan sp = plan_splits(B, Hkv, max_seq_len, kv_lo != nullptr, cols,
                                     kv->kv_type == SFA_KV_Q8_0 && B == 1);

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
    p.n_seq = B;
    p.split_row = sp.split_row;
    p.guess_splits = sp.guess_splits;
    p.guess_tiles = sp.guess_tiles;
    p.one_split = B == 1 && sp.guess_splits == 1;
    p.staged = cols && use_staged(Hkv);
    p.cols_waves = cols && !p.staged ? cols_waves_of(Hkv) : 0;
    p.scale_log2 = scale * 1.4426950408889634f;
    p.part = static_cast<float *>(workspace);
    p.kv_type = kv->kv_type;
    p.app_k = p.app_v = nullptr;
    p.app_k_pages = p.app_v_pages = p.app_k_cold = p.app_v_cold = nullptr;
    *out_p = p;
    return SFA_OK;
}

int decode_run(const DecodeParams &p, int HD, int passes, hipStream_t stream) {
    const int G = p.n_head / p.n_head_kv;
    int rc;
    switch (HD) {
    case 32: rc = launch_f16_g<32>(p, G, p.n_seq, p.n_head_kv, passes, stream); break;
    case 64: rc = launch_f16_g<64>(p, G, p.n_seq, p.n_head_kv, passes, stream); break;
    case 128: rc = launch_f16_g<128>(p, G, p.n_seq, p.n_head_kv, passes, stream); break;
    default: return SFA_ERR_UNSUPPORTED;
    }
    if (rc != SFA_OK) return rc;
    return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
}

int decode_launch(const sfa_kv_desc *kv, const float *q, float *out, const int32_t *page_table,
                  int32_t max_pages, const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                  int32_t max_seq_len, float scale, void *workspace, size_t ws_bytes,
                  int passes, hipStream_t stream) {
    DecodeParams p;
    const int rc = decode_setup(kv, q, out, page_table, max_pages, seq_len, kv_lo, B, max_seq_len, scale,
                                workspace, ws_bytes, &p);
    if (rc != SFA_OK) return rc;
    return decode_run(p, kv->head_dim, passes, stream);
}

// Decode with each sequence's new token appended in the split pass (F16 and
// F32 caches): k, v [B][Hkv][head_dim] f32, token b at position seq_len[b] - 1.
int decode_append_launch(const sfa_kv_desc *kv, const float *k, const float *v, const float *q,
                         float *out, const int32_t *page_table, int32_t max_pages,
                         const int32_t *seq_len, const int32_t *kv_lo, int32_t B, int32_t max_seq_len,
                         float scale, void *workspace, size_t ws_bytes, hipStream_t stream) {
    if (kv->kv_type != SFA_KV_F16 && kv->kv_type != SFA_KV_F32) return SFA_ERR_UNSUPPORTED;
    if (k == nullptr || v == nullptr) return SFA_ERR_INVALID_ARGUMENT;
    DecodeParams p;
    const int rc = decode_setup(kv, q, out, page_table, max_pages, seq_len, kv_lo, B, max_seq_len, scale,
                                workspace, ws_bytes, &p);
    if (rc != SFA_OK) return rc;
    p.app_k = k;
    p.app_v = v;
    p.app_k_pages = static_cast<uint8_t *>(kv->k_pages);
    p.app_v_pages = static_cast<uint8_t *>(kv->v_pages);
    p.app_k_cold = static_cast<uint8_t *>(kv->k_cold);
    p.app_v_cold = static_cast<uint8_t *>(kv->v_cold);
    return decode_run(p, kv->head_dim, 3, stream);
}

// ---- allocation-free decode ----------------------------------------------------
// sfa_attn_decode_noalloc runs the same two passes over a library-owned
// scratch array instead of a caller workspace.  The array is a device global
// of the code object, so every GPU the library runs on holds its own copy
// until the process ends; its device address is looked up once per device
// (with that device current) and cached.  Host code never passes the array's
// name itself to a kernel: on the host that name is only a stand-in.
static __device__ __align__(256) uint8_t scratch[SFA_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the device that owns `stream`.
int scratch_address(hipStream_t stream, void **out) {
    int dev = -1;
    if (stream != nullptr) {
        if (hipStreamGetDevice(stream, &dev) != hipSuccess) return SFA_ERR_RUNTIME;
    } else if (hipGetDevice(&dev) != hipSuccess) {
        return SFA_ERR_RUNTIME;
    }
    if (dev < 0 || dev >= kMaxDevices) return SFA_ERR_RUNTIME;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess) return SFA_ERR_RUNTIME;
        if (cur != dev && hipSetDevice(dev) != hipSuccess) return SFA_ERR_RUNTIME;
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess || p == nullptr) return SFA_ERR_RUNTIME;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return SFA_OK;
}
}  // namespace

int decode_noalloc_launch(const sfa_kv_desc *kv, const float *q, float *out, const int32_t *page_table,
                          int32_t max_pages, const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                          int32_t max_seq_len, float scale, hipStream_t stream) {
    if (B <= 0 || max_seq_len <= 0) return SFA_ERR_INVALID_ARGUMENT;
    const int Hkv = kv->n_head_kv, G = kv->n_head / kv->n_head_kv;
    const size_t need = decode_workspace_bytes(B, Hkv, G, kv->head_dim, max_seq_len);
    if (need > (size_t)SFA_NOALLOC_SCRATCH_BYTES) return SFA_ERR_OUT_OF_MEMORY;
    void *ws = nullptr;
    const int rc = scratch_address(stream, &ws);
    if (rc != SFA_OK) return rc;
    return decode_launch(kv, q, out, page_table, max_pages, seq_len, kv_lo, B, max_seq_len, scale, ws,
                         (size_t)SFA_NOALLOC_SCRATCH_BYTES, 3, stream);
}

}  // namespace sfa
