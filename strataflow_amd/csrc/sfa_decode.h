// sfa_decode.h - the split-K decode's parameters and split plan, shared by
// the decode passes (sfa_decode.hip).  Device helpers are inline; the host side of the plan
// (split-row sizing, workspace size, parameter setup) is declared at the end.
#pragma once

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
    int n_seq;            // B
    int split_row;        // workgroup slots per kv head (a multiple of 8)
    int guess_splits;     // the host's guess of splits per sequence (all at max_seq_len)
    int guess_tiles;      // and of its tiles; the device plan decides
    int one_split;        // 1: no merge pass runs (one sequence, guessed one split)
    int cols_waves;       // Q8_0: kv heads per column-layout workgroup, 0 = per-kv-head layout
    int staged;           // Q8_0 batches: 1 = decode_q8_staged_kernel (kStagedKv kv heads per wave)
    float scale_log2;     // scale * log2(e)
    float *part;          // [Hkv][split_row][G][HD + 4]: one (o, m, l) record per slot
    // fused append (F16 cache): sequence b's new token, [B][Hkv][HD] f32, at
    // position seq_len[b] - 1; nullptr otherwise
    const float *app_k;
    const float *app_v;
    uint8_t *app_k_pages;  // the writable pools (k_pages / v_pages above)
    uint8_t *app_v_pages;
    uint8_t *app_k_cold;
    uint8_t *app_v_cold;
};

constexpr int kDecodeWaves = 4;
constexpr int kColsWaves = 8;    // most waves (kv heads) of a column-layout Q8_0 workgroup
constexpr int kStagedKv = 4;     // kv heads per wave of the staged Q8_0 kernel
constexpr int kMaxSplits = 256;  // splits per (sequence, kv head)
constexpr int kMaxPlanTiles = 1 << 30;  // bound on the tiles of one call (all sequences)
constexpr float kRescaleLog2 = 8.0f;  // lazy rescale threshold: P <= 2^8
// merge kernel block: one thread per dim, at least one full wave
template <int HD>
constexpr int kMergeThreads = HD < 64 ? 64 : HD;

// ---- split plan --------------------------------------------------------------
// Each kv head owns a row of `split_row` workgroup slots (XCD = L % 8 and
// split_row % 8 == 0, so every kv head of one slot shares an XCD and its L2:
// Q8_0 rows of neighbouring kv heads share cache lines).  The slots are dealt
// out to the sequences in proportion to their active tiles: with T the sum of
// the sequences' tiles and Z the number of sequences with any, sequence b of
// n_b tiles takes 1 + floor((split_row - Z) * n_b / T) consecutive slots (at
// most one per kDecodeWaves tiles, at most kMaxSplits), so the shares never
// exceed the row and a short sequence in a batch does not leave slots idle
// that a long one could use.  Inside a sequence the tiles are spread evenly:
// splits differ by at most one tile.  The plan is computed on the device from
// seq_len / kv_lo (device arrays), identically by every workgroup and by the
// merge pass; the host only guesses it (every sequence at max_seq_len, from
// position 0) so the first tile can be fetched before seq_len arrives.

// Tiles of a sequence: 32-aligned absolute position blocks [32t, 32t+32)
// intersecting [lo, n_kv).
struct SeqGeom {
    int lo, n_kv, t0, n_tiles;
};
__host__ __device__ inline SeqGeom seq_geom(int n_kv_raw, int lo_raw, int cap) {
    SeqGeom g;
    g.n_kv = n_kv_raw > cap ? cap : n_kv_raw;
    g.lo = lo_raw < 0 ? 0 : lo_raw;
    if (g.n_kv <= g.lo) {
        g.t0 = 0;
        g.n_tiles = 0;
    } else {
        g.t0 = g.lo / kTile;
        g.n_tiles = (g.n_kv + kTile - 1) / kTile - g.t0;
    }
    return g;
}

__host__ __device__ inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
__host__ inline long long ceil_div(long long a, long long b) { return (a + b - 1) / b; }

// Splits of a sequence with n tiles, given `avail` slots to share beyond one
// per non-empty sequence and T tiles in all (T >= n).
__host__ __device__ inline int splits_of(int n, int avail, int T) {
    if (n <= 0) return 0;
    const unsigned long long prod = (unsigned long long)avail * (unsigned)n;
    const int share = prod <= 0xffffffffull ? (int)((unsigned)prod / (unsigned)T)
                                            : (int)(prod / (unsigned long long)T);
    int s = 1 + share;
    const int most = ceil_div(n, kDecodeWaves);
    if (s > most) s = most;
    if (s > kMaxSplits) s = kMaxSplits;
    return s;
}

// Tiles [lo, hi) of split s of n_s splits over n tiles from t0: the first
// n % n_s splits take one tile more.
__host__ __device__ inline void split_tiles(int t0, int n, int n_s, int s, int &lo, int &hi) {
    const int q = n / n_s, r = n - q * n_s;
    lo = t0 + s * q + (s < r ? s : r);
    hi = lo + q + (s < r ? 1 : 0);
}

// Wave-wide integer sum (every lane gets the result) and inclusive prefix
// sum, on DPP: butterflies or shifts inside each 16-lane row, then the rows
// combined (readlanes for the sum; row_bcast:15 / row_bcast:31 for the scan,
// as the atomic-optimizer scan of the AMDGPU backend does).
template <int CTRL>
__device__ inline int dpp_i(int x) {
    return __builtin_amdgcn_mov_dpp(x, CTRL, 0xf, 0xf, false);
}
template <int CTRL, int ROWS>
__device__ inline int dpp_i0(int x) {  // source lanes outside the row read 0
    return __builtin_amdgcn_update_dpp(0, x, CTRL, ROWS, 0xf, true);
}
__device__ inline int lane_sum_i(int x) {
    x += dpp_i<0xB1>(x);
    x += dpp_i<0x4E>(x);
    x += dpp_i<0x141>(x);
    x += dpp_i<0x140>(x);
    return (__builtin_amdgcn_readlane(x, 0) + __builtin_amdgcn_readlane(x, 16)) +
           (__builtin_amdgcn_readlane(x, 32) + __builtin_amdgcn_readlane(x, 48));
}
__device__ inline int lane_scan_i(int x) {
    x += dpp_i0<0x111, 0xf>(x);  // row_shr:1
    x += dpp_i0<0x112, 0xf>(x);  // row_shr:2
    x += dpp_i0<0x114, 0xf>(x);  // row_shr:4
    x += dpp_i0<0x118, 0xf>(x);  // row_shr:8
    x += dpp_i0<0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
    x += dpp_i0<0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
    return x;
}

// The plan as one slot or one sequence sees it.
struct SlotPlan {
    int b;       // sequence
    int split;   // split index within the sequence
    int n_b;     // splits of the sequence
    int rec0;    // its first slot in the row
    SeqGeom g;   // the sequence's tiles
};

// Per-lane raw inputs of the plan, issued early in a kernel: lane l holds
// sequence l (2 <= B <= 64); for a single sequence every lane holds it.
struct PlanRaw {
    int n_kv, lo;
};
// Branch-free: every lane loads (clamped indices, then selects), so the
// compiler can wait for exactly these loads and not for the ones issued after.
__device__ inline PlanRaw plan_load(const DecodeParams &p, int lane) {
    const int i = p.n_seq <= kWave ? (lane < p.n_seq ? lane : p.n_seq - 1) : 0;
    // kv_lo or, when absent, a harmless re-read of seq_len; both are global
    // memory (a generic-pointer load here would be a flat load, which the
    // compiler's waits cannot count apart from the loads after it)
    typedef const __attribute__((address_space(1))) int32_t *gptr;
    const gptr lo_src = (gptr)(p.kv_lo ? p.kv_lo : p.seq_len);
    const int32_t n = ((gptr)p.seq_len)[i];
    const int32_t lo = lo_src[i];
    const bool mine = p.n_seq == 1 || (p.n_seq <= kWave && lane < p.n_seq);
    return PlanRaw{mine ? n : 0, (mine && p.kv_lo) ? lo : 0};
}

// Sequence b = -1 asks for the owner of row slot j (false: the slot is idle);
// b >= 0 asks for sequence b's splits and first slot (the merge pass).  Every
// lane of the wave must be active.  2 <= B <= 64: lane l computes sequence l;
// larger batches take ceil(B / 64) rounds of the same lane-parallel sums and
// scans (lane l of round r holds sequence 64r + l).
__device__ inline bool plan_lanes(const DecodeParams &p, const PlanRaw &raw, int j, int b, int lane, SlotPlan &sp) {
    sp = SlotPlan{0, 0, 0, 0, SeqGeom{0, 0, 0, 0}};
    const int cap = p.max_pages * p.page_size;
    const int row = p.split_row;
    if (p.n_seq == 1) {
        sp.g = seq_geom(raw.n_kv, raw.lo, cap);
        sp.b = 0;
        sp.n_b = splits_of(sp.g.n_tiles, p.one_split ? 0 : row - 1, sp.g.n_tiles);
        sp.rec0 = 0;
        sp.split = b < 0 ? j : 0;
        return b >= 0 || j < sp.n_b;
    }
    if (p.n_seq <= kWave) {
        const SeqGeom g = lane < p.n_seq ? seq_geom(raw.n_kv, raw.lo, cap) : SeqGeom{0, 0, 0, 0};
        const int T = lane_sum_i(g.n_tiles);
        const int Z = __popcll(__ballot(g.n_tiles > 0));
        const int n_lane = splits_of(g.n_tiles, row - Z, T);
        const int pre_lane = lane_scan_i(n_lane) - n_lane;  // exclusive prefix over the lanes
        if (b < 0) {
            const unsigned long long m = __ballot(n_lane > 0 && pre_lane <= j && j < pre_lane + n_lane);
            if (m == 0) return false;
            b = __builtin_ctzll(m);
        }
        sp.b = b;
        sp.n_b = __shfl(n_lane, b, kWave);
        sp.rec0 = __shfl(pre_lane, b, kWave);
        sp.g.lo = __shfl(g.lo, b, kWave);
        sp.g.n_kv = __shfl(g.n_kv, b, kWave);
        sp.g.t0 = __shfl(g.t0, b, kWave);
        sp.g.n_tiles = __shfl(g.n_tiles, b, kWave);
        sp.split = j - sp.rec0;
        return true;
    }
    // more than 64 sequences: rounds of 64, lane l holding sequence 64r + l
    // (coalesced loads); T and Z first, then the slot prefix round by round
    const int rounds = (p.n_seq + kWave - 1) / kWave;
    auto geom = [&](int r) -> SeqGeom {
        const int bb = r * kWave + lane;
        return bb < p.n_seq ? seq_geom(p.seq_len[bb], p.kv_lo ? p.kv_lo[bb] : 0, cap) : SeqGeom{0, 0, 0, 0};
    };
    int T = 0, Z = 0;
    for (int r = 0; r < rounds; ++r) {
        const SeqGeom g = geom(r);
        T += lane_sum_i(g.n_tiles);
        Z += __popcll(__ballot(g.n_tiles > 0));
    }
    int pre = 0;  // slots of the earlier rounds
    for (int r = 0; r < rounds; ++r) {
        const SeqGeom g = geom(r);
        const int n_lane = splits_of(g.n_tiles, row - Z, T);
        const int incl = lane_scan_i(n_lane);
        const int pre_lane = pre + incl - n_lane;
        int sel = -1;
        if (b < 0) {
            const unsigned long long m = __ballot(n_lane > 0 && pre_lane <= j && j < pre_lane + n_lane);
            if (m != 0) sel = __builtin_ctzll(m);
        } else if (b / kWave == r) {
            sel = b - r * kWave;
        }
        if (sel >= 0) {
            sp.b = r * kWave + sel;
            sp.n_b = __shfl(n_lane, sel, kWave);
            sp.rec0 = __shfl(pre_lane, sel, kWave);
            sp.g.lo = __shfl(g.lo, sel, kWave);
            sp.g.n_kv = __shfl(g.n_kv, sel, kWave);
            sp.g.t0 = __shfl(g.t0, sel, kWave);
            sp.g.n_tiles = __shfl(g.n_tiles, sel, kWave);
            sp.split = j - sp.rec0;
            return true;
        }
        pre += __shfl(incl, kWave - 1, kWave);
    }
    return false;
}

// The plan with every field wave-uniform (scalar registers), so the tile
// bounds and the interior / edge tests derived from it are scalar branches.
__device__ inline bool plan(const DecodeParams &p, const PlanRaw &raw, int j, int b, int lane, SlotPlan &sp) {
    const bool ok = plan_lanes(p, raw, j, b, lane, sp);
    sp.b = __builtin_amdgcn_readfirstlane(sp.b);
    sp.split = __builtin_amdgcn_readfirstlane(sp.split);
    sp.n_b = __builtin_amdgcn_readfirstlane(sp.n_b);
    sp.rec0 = __builtin_amdgcn_readfirstlane(sp.rec0);
    sp.g.lo = __builtin_amdgcn_readfirstlane(sp.g.lo);
    sp.g.n_kv = __builtin_amdgcn_readfirstlane(sp.g.n_kv);
    sp.g.t0 = __builtin_amdgcn_readfirstlane(sp.g.t0);
    sp.g.n_tiles = __builtin_amdgcn_readfirstlane(sp.g.n_tiles);
    return ok;
}

// ---- host side (sfa_decode.hip) ------------------------------------------------

// Fills DecodeParams for a call (validates the arguments, sizes the split row
// and the host's plan guess); `workspace` holds the split partials.
int decode_setup(const sfa_kv_desc *kv, const float *q, float *out, const int32_t *page_table,
                 int32_t max_pages, const int32_t *seq_len, const int32_t *kv_lo, int32_t B,
                 int32_t max_seq_len, float scale, void *workspace, size_t ws_bytes,
                 DecodeParams *p);
// Launches the split-K pass (pass bit 1) and the merge pass (bit 2) for p.
int decode_run(const DecodeParams &p, int head_dim, int passes, hipStream_t stream);
size_t decode_workspace_bytes(int B, int Hkv, int G, int HD, int max_seq_len);

}  // namespace sfa
