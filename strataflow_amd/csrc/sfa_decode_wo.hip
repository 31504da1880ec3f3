// sfa_decode_wo.hip - the attention node's consumer fused into the decode's
// second pass: y = wo * attn + residual, the output projection and residual
// add that follow build_kv_attention (src/model/engine/engine.cpp:1904-1906:
// cur = ggml_mul_mat(wo, attn_out); ffn_inp = ggml_add(cur, inpSA)).
//
// The split-K pass runs unchanged and leaves per-split (m, l, o) records.  One
// workgroup per (kv head, block of 64 output rows) then merges the attention
// output of its kv head's g query heads from those records (the same
// arithmetic, in the same split order, as the stand-alone merge pass, so the
// attention output is bit-identical to sfa_attn_decode's), rounds it as ggml's
// mul_mat converts src1 for the weight type (F16 weights: to f16), and takes the
// dot products of its 64 rows of wo with that slice of the output.  The kv
// heads' partial sums of a row block meet in the workspace: the last of the
// Hkv workgroups to arrive (a device-scope counter) adds them in kv-head order,
// then the residual, so the result does not depend on arrival order.  The
// attention output itself is never written.  Partial sums are stored with
// system-scope stores (written through to memory, not left in an XCD's L2),
// each workgroup waits for its own stores before it counts itself in, and the
// last one reads them back with system-scope loads: the workgroups of a row
// block may sit on different XCDs.
#include "sfa_decode.h"

namespace sfa {

struct WoParams {
    int n_embd;
    int n_rb;                // row blocks
    const uint8_t *wo;       // [n_embd][n_head * head_dim], F32 or F16 (ggml row order)
    const float *residual;   // [B][n_embd]
    float *y;                // [B][n_embd]
    float *ypart;            // [B][Hkv][n_embd]: per-kv-head partial sums
    uint32_t *counters;      // [B][n_rb]: arrivals, reset to 0 by the last arrival
};

constexpr int kWoRows = 64;     // output rows per workgroup
constexpr int kWoThreads = 256;
constexpr int kWoWaves = kWoThreads / kWave;

__device__ inline void store_through(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ inline float load_through(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Raw weights: C consecutive elements of one row as loaded (f16 stays packed
// until used, which halves the registers holding the wave's rows).
template <int WT, int C>
struct WRow {
    static constexpr int kWords = (C * (WT == SFA_KV_F16 ? 2 : 4) + 3) / 4;
    uint32_t u[kWords];
    __device__ inline void load(const uint8_t *src) {
        if constexpr (kWords % 4 == 0) {
#pragma unroll
            for (int i = 0; i < kWords / 4; ++i) {
                const intx4 v = reinterpret_cast<const intx4 *>(src)[i];
#pragma unroll
                for (int j = 0; j < 4; ++j) u[4 * i + j] = (uint32_t)v[j];
            }
        } else if constexpr (WT == SFA_KV_F16 && C == 1) {
            u[0] = *reinterpret_cast<const uint16_t *>(src);
        } else {
#pragma unroll
            for (int i = 0; i < kWords; ++i) u[i] = reinterpret_cast<const uint32_t *>(src)[i];
        }
    }
    __device__ inline float at(int i) const {
        if constexpr (WT == SFA_KV_F16) {
            const uint16_t h = (uint16_t)(u[i / 2] >> (16 * (i % 2)));
            return (float)__builtin_bit_cast(_Float16, h);
        } else {
            return __builtin_bit_cast(float, u[i]);
        }
    }
};

// ONE: a single sequence (no loop over sequences: the loads of its records, its
// plan and the rows of wo then sit in one straight line of code, and the waits
// for each are exact).
template <int HD, int G, int WT, bool ONE>
__global__ __launch_bounds__(kWoThreads, G * HD <= 512 ? 2 : 1) void merge_wo_kernel(DecodeParams p, WoParams w) {
    constexpr int K = G * HD;          // inputs of one kv head's slice of wo
    constexpr int C = K / kWave;       // of them per lane
    constexpr int RW = kWoRows / kWoWaves;  // rows per wave
    constexpr int ES = WT == SFA_KV_F16 ? 2 : 4;
    constexpr int VPT = (K + kWoThreads - 1) / kWoThreads;  // merged values per thread
    constexpr int SB = 16;             // split records loaded per batch
    constexpr int MR = kMaxSplits / kWave;  // (m, l) registers per lane
    static_assert(C >= 1 && K % kWave == 0, "slice of at least one input per lane");
    __shared__ float lds_o[K];
    __shared__ float lds_wt[G][kMaxSplits];
    __shared__ float lds_l[G];
    __shared__ uint32_t lds_last;

    const int Hkv = p.n_head_kv;
    const int kvh = (int)blockIdx.x % Hkv;  // a kv head's row blocks share an XCD and its partials
    const int rb = (int)blockIdx.x / Hkv;
    const int tid = (int)threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int sstride = G * (HD + 4);
    const float *row0 = p.part + (int64_t)kvh * p.split_row * sstride;
    const int64_t in_stride = (int64_t)p.n_head * HD * ES;  // bytes of one wo row
    const uint8_t *wcol = w.wo + (int64_t)kvh * K * ES + (int64_t)lane * C * ES;
    const int wrow0 = rb * kWoRows + wave * RW;  // this wave's first row

    // a sequence's split records: the (m, l) of every split of the wave's
    // heads and the thread's values' first SB partial rows, all loaded before
    // any of them is needed; indices clamp into the row, so every load is in
    // bounds, and records past the sequence's splits get weight zero
    float mv[(G + kWoWaves - 1) / kWoWaves][MR], lv[(G + kWoWaves - 1) / kWoWaves][MR];
    float ob[VPT][SB];
    auto load_records = [&](const float *pg, int n_rec) {
#pragma unroll
        for (int gi = 0; gi * kWoWaves < G; ++gi) {
            const int g = wave + gi * kWoWaves;
            if (g < G) {
#pragma unroll
                for (int r = 0; r < MR; ++r) {
                    const int s = min(kWave * r + lane, n_rec - 1);
                    mv[gi][r] = pg[(int64_t)s * sstride + g * (HD + 4) + HD];
                    lv[gi][r] = pg[(int64_t)s * sstride + g * (HD + 4) + HD + 1];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const int v = min(tid + kWoThreads * k, K - 1);
            const float *col = pg + (v / HD) * (HD + 4) + v % HD;
#pragma unroll
            for (int u = 0; u < SB; ++u) ob[k][u] = col[(int64_t)min(u, n_rec - 1) * sstride];
        }
    };
    // Issue order matters: loads complete in issue order, so the small loads
    // the merge waits on (seq_len, and for one sequence its split records,
    // which it owns from slot 0 of its kv head's row and can fetch before the
    // plan is known) go out before the wave's rows of wo, which stream in
    // from HBM while the merge runs.  The rows (this lane's C inputs of each;
    // rows past n_embd read row 0) are reused for every sequence.
    // one sequence: its plan from seq_len[0] / kv_lo[0] (scalar loads), as
    // plan_lanes computes it for B = 1; a batch: the general plan
    int one_n_kv = 0, one_lo = 0;
    PlanRaw raw{0, 0};
    if constexpr (ONE) {
        one_n_kv = p.seq_len[0];
        one_lo = p.kv_lo ? p.kv_lo[0] : 0;
        load_records(row0, p.split_row);
    } else {
        raw = plan_load(p, lane);
    }
    WRow<WT, C> wv[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) wv[r].load(wcol + (int64_t)(wrow0 + r < w.n_embd ? wrow0 + r : 0) * in_stride);

    for (int b = 0; b < (ONE ? 1 : p.n_seq); ++b) {
        SlotPlan sp;
        if constexpr (ONE) {
            sp.g = seq_geom(one_n_kv, one_lo, p.max_pages * p.page_size);
            sp.n_b = splits_of(sp.g.n_tiles, p.one_split ? 0 : p.split_row - 1, sp.g.n_tiles);
            sp.rec0 = 0;
        } else {
            plan(p, raw, 0, b, lane, sp);
        }
        const int n_b = sp.n_b;
        const float *pg = row0 + (int64_t)sp.rec0 * sstride;
        // ---- the attention output of this kv head's g heads -> lds_o
        if (n_b > 1) {
            if constexpr (!ONE) load_records(pg, n_b);
            // split weights 2^(m_s - M) per head, the merge pass's arithmetic
#pragma unroll
            for (int gi = 0; gi * kWoWaves < G; ++gi) {
                const int g = wave + gi * kWoWaves;
                if (g < G) {
                    float mx = -INFINITY;
#pragma unroll
                    for (int r = 0; r < MR; ++r) {
                        mv[gi][r] = kWave * r + lane < n_b ? mv[gi][r] : -INFINITY;
                        mx = fmaxf(mx, mv[gi][r]);
                    }
                    const float M = wave_max(mx);
                    float lsum = 0.0f;
#pragma unroll
                    for (int r = 0; r < MR; ++r) {
                        const float wt = mv[gi][r] != -INFINITY ? __builtin_amdgcn_exp2f(mv[gi][r] - M) : 0.0f;
                        lsum += wt != 0.0f ? lv[gi][r] * wt : 0.0f;
                        lds_wt[g][kWave * r + lane] = wt;
                    }
                    const float L = wave_sum(lsum);
                    if (lane == 0) lds_l[g] = L;
                }
            }
            __syncthreads();
            // accumulate in split order: the first SB records are in registers,
            // later ones (long sequences) load batch by batch
#pragma unroll
            for (int k = 0; k < VPT; ++k) {
                const int v = tid + kWoThreads * k;
                if (v < K) {
                    const int g = v / HD;
                    const float *col = pg + g * (HD + 4) + v % HD;
                    float O = 0.0f;
#pragma unroll
                    for (int u = 0; u < SB; ++u) {
                        const float wt = lds_wt[g][u];
                        O = wt != 0.0f ? fmaf(ob[k][u], wt, O) : O;
                    }
                    for (int s0 = SB; s0 < n_b; s0 += SB) {
                        float o[SB];
#pragma unroll
                        for (int u = 0; u < SB; ++u) o[u] = col[(int64_t)min(s0 + u, n_b - 1) * sstride];
#pragma unroll
                        for (int u = 0; u < SB; ++u) {
                            const float wt = lds_wt[g][s0 + u];
                            O = wt != 0.0f ? fmaf(o[u], wt, O) : O;
                        }
                    }
                    const float L = lds_l[g];
                    float x = L > 0.0f ? O / L : 0.0f;
                    if constexpr (WT == SFA_KV_F16) x = (float)(_Float16)x;  // vec_dot_type F16
                    lds_o[v] = x;
                }
            }
        } else {
            // one split: the split pass wrote the output; none: zero
            const float *obuf = p.out + ((int64_t)b * p.n_head + (int64_t)kvh * G) * HD;
#pragma unroll
            for (int k = 0; k < VPT; ++k) {
                const int v = tid + kWoThreads * k;
                if (v < K) {
                    float x = n_b == 1 ? obuf[v] : 0.0f;
                    if constexpr (WT == SFA_KV_F16) x = (float)(_Float16)x;
                    lds_o[v] = x;
                }
            }
        }
        __syncthreads();

        // ---- this kv head's partial sums of the wave's rows.  The empty asm
        // keeps the f16 -> f32 conversions of the rows here: hoisted out of
        // the sequence loop they would wait for the rows before the merge.
#pragma unroll
        for (int r = 0; r < RW; ++r) {
#pragma unroll
            for (int j = 0; j < WRow<WT, C>::kWords; ++j) asm volatile("" : "+v"(wv[r].u[j]));
        }
        float ov[C];
#pragma unroll
        for (int i = 0; i < C; ++i) ov[i] = lds_o[lane * C + i];
        float acc[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < C; ++i) a = fmaf(wv[r].at(i), ov[i], a);
            acc[r] = a;
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[r] = wave_sum(acc[r]);
        float *yp = w.ypart + ((int64_t)b * Hkv + kvh) * w.n_embd;
        if (lane < RW && wrow0 + lane < w.n_embd) {
            float a = acc[0];
#pragma unroll
            for (int r = 1; r < RW; ++r) a = lane == r ? acc[r] : a;
            store_through(yp + wrow0 + lane, a);
        }
        // every wave's stores have reached memory before the workgroup counts in
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            uint32_t *cnt = w.counters + (int64_t)b * w.n_rb + rb;
            // performed at system scope, past every XCD's L2
            const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            lds_last = old == (uint32_t)(Hkv - 1);
            if (lds_last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        __syncthreads();
        if (lds_last && tid < kWoRows) {
            const int row = rb * kWoRows + tid;
            if (row < w.n_embd) {
                float a = 0.0f;
                for (int k = 0; k < Hkv; ++k)
                    a += load_through(w.ypart + ((int64_t)b * Hkv + k) * w.n_embd + row);
                w.y[(int64_t)b * w.n_embd + row] = a + w.residual[(int64_t)b * w.n_embd + row];
            }
        }
        __syncthreads();  // lds_o / lds_wt are rewritten for the next sequence
    }
}

// Workspace of the fused node: the decode partials, the outputs of one-split
// sequences, the per-kv-head partial sums and the arrival counters.
struct WoLayout {
    size_t part, one, ypart, counters, total;
};
static WoLayout wo_layout(int B, int Hq, int Hkv, int HD, int max_seq_len, int n_embd) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    WoLayout L;
    L.part = 0;
    L.one = up(decode_workspace_bytes(B, Hkv, Hq / Hkv, HD, max_seq_len));
    L.ypart = L.one + up((size_t)B * Hq * HD * sizeof(float));
    L.counters = L.ypart + up((size_t)B * Hkv * n_embd * sizeof(float));
    const int n_rb = (n_embd + kWoRows - 1) / kWoRows;
    L.total = L.counters + up((size_t)B * n_rb * sizeof(uint32_t));
    return L;
}

size_t decode_wo_workspace_bytes(const sfa_kv_desc *kv, int B, int max_seq_len, int n_embd) {
    return wo_layout(B, kv->n_head, kv->n_head_kv, kv->head_dim, max_seq_len, n_embd).total;
}

template <int HD, int G>
static int launch_wo(const DecodeParams &p, const WoParams &w, int wo_type, hipStream_t s) {
    if constexpr (G * HD < kWave) {
        return SFA_ERR_UNSUPPORTED;
    } else {
        const dim3 grid(p.n_head_kv * w.n_rb), block(kWoThreads);
        const bool one = p.n_seq == 1;
        if (wo_type == SFA_KV_F16) {
            if (one) hipLaunchKernelGGL((merge_wo_kernel<HD, G, SFA_KV_F16, true>), grid, block, 0, s, p, w);
            else hipLaunchKernelGGL((merge_wo_kernel<HD, G, SFA_KV_F16, false>), grid, block, 0, s, p, w);
        } else {
            if (one) hipLaunchKernelGGL((merge_wo_kernel<HD, G, SFA_KV_F32, true>), grid, block, 0, s, p, w);
            else hipLaunchKernelGGL((merge_wo_kernel<HD, G, SFA_KV_F32, false>), grid, block, 0, s, p, w);
        }
        return SFA_OK;
    }
}

template <int HD>
static int launch_wo_g(const DecodeParams &p, const WoParams &w, int wo_type, hipStream_t s) {
    switch (p.n_head / p.n_head_kv) {
    case 1: return launch_wo<HD, 1>(p, w, wo_type, s);
    case 2: return launch_wo<HD, 2>(p, w, wo_type, s);
    case 4: return launch_wo<HD, 4>(p, w, wo_type, s);
    case 8: return launch_wo<HD, 8>(p, w, wo_type, s);
    default: return SFA_ERR_UNSUPPORTED;
    }
}

int decode_wo_launch(const sfa_kv_desc *kv, const float *q, const int32_t *page_table, int32_t max_pages,
                     const int32_t *seq_len, const int32_t *kv_lo, int32_t B, int32_t max_seq_len,
                     float scale, const void *wo, int32_t wo_type, int32_t n_embd, const float *residual,
                     float *y, void *workspace, size_t ws_bytes, hipStream_t stream) {
    if (B <= 0 || max_seq_len <= 0 || n_embd <= 0) return SFA_ERR_INVALID_ARGUMENT;
    if (wo == nullptr || residual == nullptr || y == nullptr || workspace == nullptr)
        return SFA_ERR_INVALID_ARGUMENT;
    if (wo_type != SFA_KV_F32 && wo_type != SFA_KV_F16) return SFA_ERR_UNSUPPORTED;
    const int HD = kv->head_dim, Hq = kv->n_head, Hkv = kv->n_head_kv;
    if ((Hq / Hkv) * HD < kWave) return SFA_ERR_UNSUPPORTED;
    const WoLayout L = wo_layout(B, Hq, Hkv, HD, max_seq_len, n_embd);
    if (ws_bytes < L.total) return SFA_ERR_INVALID_ARGUMENT;
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    DecodeParams p;
    // one-split sequences leave their output in the workspace for the merge
    int rc = decode_setup(kv, q, reinterpret_cast<float *>(ws + L.one), page_table, max_pages, seq_len,
                          kv_lo, B, max_seq_len, scale, ws + L.part, L.one, &p);
    if (rc != SFA_OK) return rc;
    WoParams w;
    w.n_embd = n_embd;
    w.n_rb = (n_embd + kWoRows - 1) / kWoRows;
    w.wo = static_cast<const uint8_t *>(wo);
    w.residual = residual;
    w.y = y;
    w.ypart = reinterpret_cast<float *>(ws + L.ypart);
    w.counters = reinterpret_cast<uint32_t *>(ws + L.counters);
    rc = decode_run(p, HD, 1, stream);  // the split-K pass only
    if (rc != SFA_OK) return rc;
    switch (HD) {
    case 32: rc = launch_wo_g<32>(p, w, wo_type, stream); break;
    case 64: rc = launch_wo_g<64>(p, w, wo_type, stream); break;
    case 128: rc = launch_wo_g<128>(p, w, wo_type, stream); break;
    default: return SFA_ERR_UNSUPPORTED;
    }
    if (rc != SFA_OK) return rc;
    return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
}

}  // namespace sfa
