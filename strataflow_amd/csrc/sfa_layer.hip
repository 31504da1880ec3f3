// sfa_layer.hip - the rest of the decode layer around the attention node, for
// gfx950: build_router_segment and build_expert_segment of the reference
// (src/model/engine/engine.cpp:1877-1925, 1945-1986) as four kernels.
//
//   attn_norm / ffn_norm   rms_norm(x, eps) * weight             engine.cpp:1879-1880, 1908-1909
//   Q/K/V, wo, router      mul_mat(W, x) (+ residual)            engine.cpp:1883-1885, 1905-1906, 1912
//   routing                soft_max, argsort_top_k, get_rows,
//                          sum_rows, clamp, div                  engine.cpp:1913-1925
//   experts                mul_mat_id(up/gate), swiglu_split,
//                          mul_mat_id(down), * weights, sum,
//                          + residual                            engine.cpp:1964-1984
//
// Arithmetic follows ggml's CPU backend, the reference's oracle: rms_norm sums
// the f32 squares in double and scales by 1/sqrtf(mean + eps); mul_mat with F16
// weights first rounds the activation row to f16 (the vec_dot_type of F16) and
// sums f16 x f16 products in f32; soft_max sums exp(x - max) in double and
// scales by (float)(1/sum); sum_rows sums in double; the expert outputs are
// multiplied by their weights, added in slot order, then the residual is added.
//
// Every kernel is HBM-bound at decode (one or a few tokens per weight read):
// a wave owns one to four output rows and its lanes stream each row in
// 16-byte chunks, several chunks in flight per lane; activations (a few KB)
// come from L2.  Weights are row-major [n_out][n_in] (ggml ne =
// [n_in, n_out]); expert stacks are [n_expert][n_out][n_in].
#include <exception>

#include "sfa_append.h"
#include "sfa_layer.h"

namespace sfa {

// expert gate/up rows per wave (one gate and one up row): Mixtral's 2 x 14336
// rows per slot give 28672 waves (2 / 4 / 8 rows per wave were slower: 81 /
// 89 / 104 us against 79 for two experts' 470 MB)
constexpr int kRowsPerWave = 1;
constexpr int kLayerWaves = 4;
constexpr int kRowsPerBlock = kRowsPerWave * kLayerWaves;  // expert gate/up rows per workgroup

// 8 consecutive activations as the f16 operand of F16 weights (RNE, the
// FP32 -> FP16 conversion ggml applies to src1)
__device__ inline half8 to_half8(const floatx4 a, const floatx4 b) {
    half8 h;
    h[0] = (_Float16)a[0]; h[1] = (_Float16)a[1]; h[2] = (_Float16)a[2]; h[3] = (_Float16)a[3];
    h[4] = (_Float16)b[0]; h[5] = (_Float16)b[1]; h[6] = (_Float16)b[2]; h[7] = (_Float16)b[3];
    return h;
}

struct Half2x4 {
    half2v v[4];  // the four dwords of a half8
};

// sum of 8 products: f16 x f16 through v_dot2_f32_f16 (exact products, f32
// accumulation), f32 x f32 by fma
__device__ inline float dot8(const half8 w, const half8 x, float acc) {
    const Half2x4 a = __builtin_bit_cast(Half2x4, w), b = __builtin_bit_cast(Half2x4, x);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_fdot2(a.v[j], b.v[j], acc, false);
    return acc;
}
__device__ inline float dot8(const floatx4 w0, const floatx4 w1, const floatx4 x0, const floatx4 x1, float acc) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = fmaf(w0[j], x0[j], acc);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = fmaf(w1[j], x1[j], acc);
    return acc;
}

// ---- rms_norm * weight --------------------------------------------------------

// One workgroup per row: y = (x * (1/sqrtf(mean(x^2) + eps))) * w, the two
// products rounded separately (ggml_rms_norm, then ggml_mul).  Up to
// kNormRegs * 256 values per row are loaded (x and w) before any is used and
// kept in registers, so the pass waits on memory once; longer rows loop over
// the rest.
constexpr int kNormThreads = 256;
constexpr int kNormRegs = 16;
// The norm of one row by a kNormThreads workgroup, written to yr and, when
// ly is not null, to ly (an LDS copy for a consumer in the same workgroup).
__device__ inline void norm_row(const float *xr, const float *w, float *yr, float *ly, int n, float eps,
                                double *part) {
    const int tid = threadIdx.x;
    float xv[kNormRegs], wv[kNormRegs];
#pragma unroll
    for (int k = 0; k < kNormRegs; ++k) {
        const int i = min(tid + kNormThreads * k, n - 1);  // clamped: every load in bounds
        xv[k] = xr[i];
        wv[k] = w[i];
    }
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < kNormRegs; ++k) {
        const float v = tid + kNormThreads * k < n ? xv[k] : 0.0f;
        s += (double)(v * v);
    }
    for (int i = tid + kNormThreads * kNormRegs; i < n; i += kNormThreads) {
        const float v = xr[i];
        s += (double)(v * v);
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((tid & 63) == 0) part[tid >> 6] = s;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int k = 0; k < kNormThreads / 64; ++k) t += part[k];
    const float mean = (float)(t / n);
    const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int k = 0; k < kNormRegs; ++k) {
        const int i = tid + kNormThreads * k;
        if (i < n) {
            const float v = __fmul_rn(__fmul_rn(xv[k], scale), wv[k]);
            yr[i] = v;
            if (ly != nullptr) ly[i] = v;
        }
    }
    for (int i = tid + kNormThreads * kNormRegs; i < n; i += kNormThreads) {
        const float v = __fmul_rn(__fmul_rn(xr[i], scale), w[i]);
        yr[i] = v;
        if (ly != nullptr) ly[i] = v;
    }
}

__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const float *x, const float *w, float *y, int n,
                                                                float eps) {
    __shared__ double part[kNormThreads / 64];
    norm_row(x + (int64_t)blockIdx.x * n, w, y + (int64_t)blockIdx.x * n, nullptr, n, eps, part);
}

// ---- mul_mat_vec ---------------------------------------------------------------

struct GemvParams {
    const void *w;         // [n_out][n_in], f32 or f16
    const float *x;        // [n_rows][n_in]
    const float *residual; // [n_rows][n_out] or null
    float *y;              // [n_rows][n_out]
    int n_rows, n_in, n_out;
};

// Wave w of block b owns rows RW * (4b + w) .. + RW - 1 (clamped to n_out - 1
// for the loads, not stored) for NT tokens starting at token blockIdx.y * NT.
// RW follows n_out so that a launch has about 4096 waves or more: one row per
// wave for the 4096- and 6144-row products of a decode layer, four for wide
// ones.  One token's F16 row loads kGemvBatch chunks a lane (activations and
// weights) before it uses any: a load-use loop holds fewer in flight
// (`wo` 4096 x 4096 and the Q/K/V stack, layer 165.3 -> 163.2 us).
constexpr int kGemvBatch = 4;
template <bool F16, int NT, int RW>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = ((int)blockIdx.x * kLayerWaves + wave) * RW;
    const int tok0 = (int)blockIdx.y * NT;
    const int nc = p.n_in / 8;  // 8-element chunks per row
    float acc[RW][NT];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[r][t] = 0.0f;
    int rows[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) rows[r] = min(row0 + r, p.n_out - 1);
    int toks[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) toks[t] = min(tok0 + t, p.n_rows - 1);

    int c_rest = lane;
    if constexpr (F16 && RW == 1 && NT == 1) {
        // one token's row (the decode case): whole batches of kGemvBatch
        // chunks a lane, activations then weights, loaded before any is used
        const half8 *W = static_cast<const half8 *>(p.w);
        const floatx4 *xr = reinterpret_cast<const floatx4 *>(p.x + (int64_t)toks[0] * p.n_in);
        constexpr int CB = kGemvBatch;
        const int full = nc / (64 * CB) * (64 * CB);
        for (int c0 = lane; c0 < full; c0 += 64 * CB) {
            half8 wv[CB];
            floatx4 x0[CB], x1[CB];
#pragma unroll
            for (int k = 0; k < CB; ++k) {
                x0[k] = xr[2 * (c0 + 64 * k)];
                x1[k] = xr[2 * (c0 + 64 * k) + 1];
            }
#pragma unroll
            for (int k = 0; k < CB; ++k) wv[k] = W[(int64_t)rows[0] * nc + c0 + 64 * k];
#pragma unroll
            for (int k = 0; k < CB; ++k) acc[0][0] = dot8(wv[k], to_half8(x0[k], x1[k]), acc[0][0]);
        }
        c_rest = full + lane;
    }
    constexpr int kUnroll = RW == 1 ? 8 : 4;
#pragma unroll kUnroll
    for (int c = c_rest; c < nc; c += 64) {
        if constexpr (F16) {
            const half8 *W = static_cast<const half8 *>(p.w);
            half8 wv[RW];
#pragma unroll
            for (int r = 0; r < RW; ++r) wv[r] = W[(int64_t)rows[r] * nc + c];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const floatx4 *xr = reinterpret_cast<const floatx4 *>(p.x + (int64_t)toks[t] * p.n_in) + 2 * c;
                const half8 xh = to_half8(xr[0], xr[1]);
#pragma unroll
                for (int r = 0; r < RW; ++r) acc[r][t] = dot8(wv[r], xh, acc[r][t]);
            }
        } else {
            const floatx4 *W = static_cast<const floatx4 *>(p.w);
            floatx4 w0[RW], w1[RW];
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                w0[r] = W[((int64_t)rows[r] * nc + c) * 2];
                w1[r] = W[((int64_t)rows[r] * nc + c) * 2 + 1];
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const floatx4 *xr = reinterpret_cast<const floatx4 *>(p.x + (int64_t)toks[t] * p.n_in) + 2 * c;
                const floatx4 x0 = xr[0], x1 = xr[1];
#pragma unroll
                for (int r = 0; r < RW; ++r) acc[r][t] = dot8(w0[r], w1[r], x0, x1, acc[r][t]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float v = wave_sum(acc[r][t]);
            if (lane == r * NT + t && row0 + r < p.n_out && tok0 + t < p.n_rows) {
                const int64_t o = (int64_t)(tok0 + t) * p.n_out + row0 + r;
                p.y[o] = p.residual ? __fadd_rn(v, p.residual[o]) : v;
            }
        }
    }
}

// ---- routing --------------------------------------------------------------------

// Routing of one token by one wave, lane e holding logit e (n_expert <= 64):
// probabilities, the n_used largest in descending order (ties: the lower
// expert first, a stable descending argsort), their weights divided by their
// sum clamped at 2^-14.
__device__ inline void route_wave(float x, int lane, int n_expert, int n_used, int32_t *ids, float *weights) {
    const bool live = lane < n_expert;
    x = live ? x : -INFINITY;
    const float mx = wave_max(x);
    const float e = live ? expf(x - mx) : 0.0f;
    double s = (double)e;
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    const float inv = (float)(1.0 / s);
    const float pr = __fmul_rn(e, inv);
    bool taken = !live;
    float wsel = 0.0f;  // lane j < n_used: the j-th selected probability
    int esel = 0;
    for (int j = 0; j < n_used; ++j) {
        const float cand = taken ? -INFINITY : pr;
        const float best = wave_max(cand);
        const uint64_t hit = __ballot(!taken && cand == best);
        const int pick = hit ? __builtin_ctzll(hit) : 0;
        const float pv = __shfl(pr, pick, 64);
        if (lane == j) { wsel = pv; esel = pick; }
        taken = taken || lane == pick;
    }
    double ws = lane < n_used ? (double)wsel : 0.0;
    for (int off = 32; off > 0; off >>= 1) ws += __shfl_xor(ws, off, 64);
    float sum = (float)ws;
    sum = sum < 6.103515625e-5f ? 6.103515625e-5f : sum;
    if (lane < n_used) {
        ids[lane] = esel;
        weights[lane] = __fdiv_rn(wsel, sum);
    }
}

__global__ __launch_bounds__(64) void moe_route_kernel(const float *logits, int n_expert, int n_used,
                                                       int32_t *ids, float *weights) {
    const int lane = threadIdx.x;
    const float x = logits[(int64_t)blockIdx.x * n_expert + min(lane, n_expert - 1)];
    route_wave(x, lane, n_expert, n_used, ids + (int64_t)blockIdx.x * n_used,
               weights + (int64_t)blockIdx.x * n_used);
}

// The router product and the routing in one launch (engine.cpp:1912-1925):
// one workgroup per token; wave w computes the logits of experts w, w + 4, ..
// (the mul_mat_vec arithmetic), wave 0 routes them from LDS.
template <bool F16>
__device__ inline void router_logits(const void *w, const float *x, int n_embd, int n_expert, float *lds_logit) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nc = n_embd / 8;
    const floatx4 *xr = reinterpret_cast<const floatx4 *>(x);
    for (int e0 = wave; e0 < n_expert; e0 += 2 * kLayerWaves) {
        const int e1 = min(e0 + kLayerWaves, n_expert - 1);  // two rows per pass (clamped, stored once)
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll 4
        for (int c = lane; c < nc; c += 64) {
            if constexpr (F16) {
                const half8 *W = static_cast<const half8 *>(w);
                const half8 w0 = W[(int64_t)e0 * nc + c], w1 = W[(int64_t)e1 * nc + c];
                const half8 xh = to_half8(xr[2 * c], xr[2 * c + 1]);
                a0 = dot8(w0, xh, a0);
                a1 = dot8(w1, xh, a1);
            } else {
                const floatx4 *W = static_cast<const floatx4 *>(w);
                const floatx4 x0 = xr[2 * c], x1 = xr[2 * c + 1];
                a0 = dot8(W[((int64_t)e0 * nc + c) * 2], W[((int64_t)e0 * nc + c) * 2 + 1], x0, x1, a0);
                a1 = dot8(W[((int64_t)e1 * nc + c) * 2], W[((int64_t)e1 * nc + c) * 2 + 1], x0, x1, a1);
            }
        }
        a0 = wave_sum(a0);
        a1 = wave_sum(a1);
        if (lane == 0) {
            lds_logit[e0] = a0;
            if (e0 + kLayerWaves < n_expert) lds_logit[e0 + kLayerWaves] = a1;
        }
    }
}

template <bool F16>
__global__ __launch_bounds__(256) void moe_gate_kernel(const void *w, const float *x, int n_embd, int n_expert,
                                                       int n_used, int32_t *ids, float *weights) {
    __shared__ float lds_logit[64];
    const int t = blockIdx.x;
    router_logits<F16>(w, x + (int64_t)t * n_embd, n_embd, n_expert, lds_logit);
    __syncthreads();
    const int lane = threadIdx.x & 63;
    if (threadIdx.x < 64)
        route_wave(lds_logit[min(lane, n_expert - 1)], lane, n_expert, n_used, ids + (int64_t)t * n_used,
                   weights + (int64_t)t * n_used);
}

// ffn_norm, the router product and the routing in one launch
// (engine.cpp:1908-1925): the workgroup normalises its token's row
// (norm_row, written to y for the experts and kept in LDS), then computes the
// logits from the LDS copy and routes them as moe_gate_kernel does.  One
// launch less than rms_norm + gate; bit-identical to that pair.
constexpr int kNormGateMaxEmbd = 8192;
template <bool F16>
__global__ __launch_bounds__(kNormThreads) void moe_norm_gate_kernel(const float *x, const float *nw, float eps,
                                                                     const void *w, int n_embd, int n_expert,
                                                                     int n_used, float *y, int32_t *ids,
                                                                     float *weights) {
    static_assert(kNormThreads == 64 * kLayerWaves, "the router product's waves");
    __shared__ double part[kNormThreads / 64];
    __shared__ __attribute__((aligned(16))) float lds_x[kNormGateMaxEmbd];
    __shared__ float lds_logit[64];
    const int t = blockIdx.x;
    norm_row(x + (int64_t)t * n_embd, nw, y + (int64_t)t * n_embd, lds_x, n_embd, eps, part);
    __syncthreads();
    router_logits<F16>(w, lds_x, n_embd, n_expert, lds_logit);
    __syncthreads();
    const int lane = threadIdx.x & 63;
    if (threadIdx.x < 64)
        route_wave(lds_logit[min(lane, n_expert - 1)], lane, n_expert, n_used, ids + (int64_t)t * n_used,
                   weights + (int64_t)t * n_used);
}

// ---- experts --------------------------------------------------------------------

struct MoeParams {
    const float *x;          // [n_rows][n_embd] (ffn_norm output)
    const float *residual;   // [n_rows][n_embd] (ffn_inp)
    const int32_t *ids;      // [n_rows][n_used]
    const float *weights;    // [n_rows][n_used]
    const void *gate, *up;   // [n_expert][n_ff][n_embd]
    const void *down;        // [n_expert][n_embd][n_ff]
    float *act;              // [n_rows][n_used][n_ff] (halves for F16 weights)
    float *y;                // [n_rows][n_embd]
    int n_rows, n_embd, n_ff, n_expert, n_used;
};

// chunks of 8 a lane loads before it uses any in the F16 gate/up product;
// that kernel may take the registers of four waves per SIMD (it takes those
// of three), so the compiler keeps them all in flight (the launch has 28672
// waves for Mixtral's two slots, so the chip stays full)
constexpr int kGateUpBatch = 8;

// act[t][j][f] = silu(gate[e][f] . x[t]) * (up[e][f] . x[t]), e = ids[t][j];
// an id outside [0, n_expert) gives zeros.  Grid (row blocks of n_ff, n_used,
// n_rows).
template <bool F16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, F16 ? 4 : 8))) void moe_gate_up_kernel(MoeParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int f0 = (int)blockIdx.x * kRowsPerBlock + wave * kRowsPerWave;
    const int j = blockIdx.y, t = blockIdx.z;
    const int e_raw = p.ids[(int64_t)t * p.n_used + j];
    const bool valid = e_raw >= 0 && e_raw < p.n_expert;
    const int e = valid ? e_raw : 0;
    const int nc = p.n_embd / 8;
    float g[kRowsPerWave], u[kRowsPerWave];
    int rows[kRowsPerWave];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        g[r] = u[r] = 0.0f;
        rows[r] = min(f0 + r, p.n_ff - 1);
    }
    const floatx4 *xr = reinterpret_cast<const floatx4 *>(p.x + (int64_t)t * p.n_embd);
    const int64_t mat = (int64_t)e * p.n_ff;
    int c_rest = lane;
    if constexpr (F16 && kRowsPerWave == 1) {
        // whole batches of kGateUpBatch chunks a lane: the activations, then
        // the gate and up rows, all loaded before any is used (a whole
        // 4096-wide row at once), then the products in chunk order
        const half8 *G = static_cast<const half8 *>(p.gate), *U = static_cast<const half8 *>(p.up);
        constexpr int CB = kGateUpBatch;
        const int full = nc / (64 * CB) * (64 * CB);
        for (int c0 = lane; c0 < full; c0 += 64 * CB) {
            half8 gv[CB], uv[CB];
            floatx4 x0[CB], x1[CB];
#pragma unroll
            for (int k = 0; k < CB; ++k) {
                x0[k] = xr[2 * (c0 + 64 * k)];
                x1[k] = xr[2 * (c0 + 64 * k) + 1];
            }
#pragma unroll
            for (int k = 0; k < CB; ++k) {
                gv[k] = G[(mat + rows[0]) * nc + c0 + 64 * k];
                uv[k] = U[(mat + rows[0]) * nc + c0 + 64 * k];
            }
#pragma unroll
            for (int k = 0; k < CB; ++k) {
                const half8 xh = to_half8(x0[k], x1[k]);
                g[0] = dot8(gv[k], xh, g[0]);
                u[0] = dot8(uv[k], xh, u[0]);
            }
        }
        c_rest = full + lane;
    }
#pragma unroll 4
    for (int c = c_rest; c < nc; c += 64) {
        if constexpr (F16) {
            const half8 *G = static_cast<const half8 *>(p.gate), *U = static_cast<const half8 *>(p.up);
            half8 gv[kRowsPerWave], uv[kRowsPerWave];
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) {
                gv[r] = G[(mat + rows[r]) * nc + c];
                uv[r] = U[(mat + rows[r]) * nc + c];
            }
            const half8 xh = to_half8(xr[2 * c], xr[2 * c + 1]);
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) {
                g[r] = dot8(gv[r], xh, g[r]);
                u[r] = dot8(uv[r], xh, u[r]);
            }
        } else {
            const floatx4 *G = static_cast<const floatx4 *>(p.gate), *U = static_cast<const floatx4 *>(p.up);
            floatx4 g0[kRowsPerWave], g1[kRowsPerWave], u0[kRowsPerWave], u1[kRowsPerWave];
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) {
                const int64_t o = ((mat + rows[r]) * nc + c) * 2;
                g0[r] = G[o]; g1[r] = G[o + 1];
                u0[r] = U[o]; u1[r] = U[o + 1];
            }
            const floatx4 x0 = xr[2 * c], x1 = xr[2 * c + 1];
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) {
                g[r] = dot8(g0[r], g1[r], x0, x1, g[r]);
                u[r] = dot8(u0[r], u1[r], x0, x1, u[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        const float gs = wave_sum(g[r]), us = wave_sum(u[r]);
        if (lane == r && f0 + r < p.n_ff) {
            // ggml_silu_f32(x) = x / (1 + expf(-x)), times up (swiglu_split)
            const float a = __fmul_rn(__fdiv_rn(gs, __fadd_rn(1.0f, expf(-gs))), us);
            const int64_t ai = ((int64_t)t * p.n_used + j) * p.n_ff + f0 + r;
            // F16 down weights take the activation rounded to f16 (ggml's
            // vec_dot_type): stored that way, the down pass loads half the bytes
            if constexpr (F16)
                reinterpret_cast<_Float16 *>(p.act)[ai] = valid ? (_Float16)a : (_Float16)0.0f;
            else
                p.act[ai] = valid ? a : 0.0f;
        }
    }
}

// y[t][o] = (sum over slots j in order of (down[e_j][o] . act[t][j]) * w[t][j])
// + residual[t][o]; a slot with an id outside [0, n_expert) adds nothing.
// Every slot's rows stream in the same loop; two rows per wave, so a 4096-row
// output has 2048 waves.  For F16 weights the activations arrive as halves,
// and each lane loads kDownBatch 16-byte pieces (a batch of chunks of every
// slot's two rows and activations) before it uses any; that kernel is built
// for the two waves per SIMD such a launch has, so the compiler keeps the
// batch in flight.  Grid (row blocks of n_embd, n_rows).
constexpr int kDownRows = 2;
constexpr int kDownBatch = 24;
template <bool F16, int NU>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, F16 ? 2 : 8))) void moe_down_kernel(MoeParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int o0 = ((int)blockIdx.x * kLayerWaves + wave) * kDownRows;
    const int t = blockIdx.y;
    const int nc = p.n_ff / 8;
    int rows[kDownRows];
#pragma unroll
    for (int r = 0; r < kDownRows; ++r) rows[r] = min(o0 + r, p.n_embd - 1);
    int64_t mat[NU];
    bool valid[NU];
    float wj[NU];
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        const int e_raw = p.ids[(int64_t)t * NU + j];
        valid[j] = e_raw >= 0 && e_raw < p.n_expert;
        mat[j] = (int64_t)(valid[j] ? e_raw : 0) * p.n_embd;
        wj[j] = p.weights[(int64_t)t * NU + j];
    }
    const floatx4 *act = reinterpret_cast<const floatx4 *>(p.act + (int64_t)t * NU * p.n_ff);
    const half8 *act_h = reinterpret_cast<const half8 *>(reinterpret_cast<const _Float16 *>(p.act) +
                                                         (int64_t)t * NU * p.n_ff);
    float d[NU][kDownRows];
#pragma unroll
    for (int j = 0; j < NU; ++j)
#pragma unroll
        for (int r = 0; r < kDownRows; ++r) d[j][r] = 0.0f;
    if constexpr (F16) {
        // CB chunks of every slot's rows and activations loaded before any is
        // used: 2048 waves are eight a CU, so each keeps a whole batch in
        // flight, not the six loads the compiler holds in a load-use loop.
        // Whole batches first (no lane-dependent test the loads could sink
        // into), then the chunks left, one at a time: products in chunk order.
        const half8 *D = static_cast<const half8 *>(p.down);
        constexpr int CB = kDownBatch / (NU * kDownRows + NU) > 0 ? kDownBatch / (NU * kDownRows + NU) : 1;
        const int full = nc / (64 * CB) * (64 * CB);
        auto chunk = [&](int c, half8 (&dv)[NU][kDownRows], half8 (&ah)[NU]) {
#pragma unroll
            for (int j = 0; j < NU; ++j) {
#pragma unroll
                for (int r = 0; r < kDownRows; ++r) dv[j][r] = D[(mat[j] + rows[r]) * nc + c];
                ah[j] = act_h[(int64_t)j * nc + c];
            }
        };
        auto use = [&](const half8 (&dv)[NU][kDownRows], const half8 (&ah)[NU]) {
#pragma unroll
            for (int j = 0; j < NU; ++j)
#pragma unroll
                for (int r = 0; r < kDownRows; ++r) d[j][r] = dot8(dv[j][r], ah[j], d[j][r]);
        };
        for (int c0 = lane; c0 < full; c0 += 64 * CB) {
            half8 dv[CB][NU][kDownRows], ah[CB][NU];
#pragma unroll
            for (int k = 0; k < CB; ++k) chunk(c0 + 64 * k, dv[k], ah[k]);
#pragma unroll
            for (int k = 0; k < CB; ++k) use(dv[k], ah[k]);
        }
        for (int c = full + lane; c < nc; c += 64) {
            half8 dv[NU][kDownRows], ah[NU];
            chunk(c, dv, ah);
            use(dv, ah);
        }
    } else {
        const floatx4 *D = static_cast<const floatx4 *>(p.down);
#pragma unroll 4
        for (int c = lane; c < nc; c += 64) {
#pragma unroll
            for (int j = 0; j < NU; ++j) {
                const floatx4 *ar = act + (int64_t)j * (p.n_ff / 4);
                floatx4 d0[kDownRows], d1[kDownRows];
#pragma unroll
                for (int r = 0; r < kDownRows; ++r) {
                    d0[r] = D[((mat[j] + rows[r]) * nc + c) * 2];
                    d1[r] = D[((mat[j] + rows[r]) * nc + c) * 2 + 1];
                }
                const floatx4 a0 = ar[2 * c], a1 = ar[2 * c + 1];
#pragma unroll
                for (int r = 0; r < kDownRows; ++r) d[j][r] = dot8(d0[r], d1[r], a0, a1, d[j][r]);
            }
        }
    }
    float out[kDownRows];
#pragma unroll
    for (int r = 0; r < kDownRows; ++r) {
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const float v = valid[j] ? __fmul_rn(wave_sum(d[j][r]), wj[j]) : 0.0f;
            out[r] = j == 0 ? v : __fadd_rn(out[r], v);
        }
    }
    if (lane < kDownRows && o0 + lane < p.n_embd) {
        float v = out[0];
#pragma unroll
        for (int r = 1; r < kDownRows; ++r) v = lane == r ? out[r] : v;
        const int64_t o = (int64_t)t * p.n_embd + o0 + lane;
        p.y[o] = __fadd_rn(v, p.residual[o]);
    }
}

// ---- Q/K/V product + RoPE + KV append ----------------------------------------

// The stacked Q/K/V product (engine.cpp:1883-1885), RoPE NORMAL of Q and K
// (:1892-1897) and the KV append (:1646-1656) in one launch, for decode
// tokens: gemv_kernel's arithmetic for the rows (wave w < 4 of block b owns
// row 4b + w, so a workgroup holds two whole RoPE pairs); a fifth wave
// meanwhile computes the two pairs' cos / sin and destination rows
// (rope_append_kernel's rope_cos_sin and row_ptr), so only the rotation
// (rope_rotate) and the stores follow the products.  Rows [0, n_q) are Q
// (written rotated to q, or as computed for a token with seq or pos < 0,
// which rope_append_kernel leaves alone), then n_kv K rows, then n_kv V rows;
// F16 caches round to nearest even, F32 store as is.  Grid (n_out / 4, n_tok).
struct QkvRopeParams {
    const void *w;     // [n_out][n_in]
    const float *x;    // [n_tok][n_in]
    float *q;          // [n_tok][n_q]
    int n_in, n_out, n_q;
    float theta_scale;
    AppendParams ap;   // k / v unused
};
constexpr int kQkvThreads = 64 * (kLayerWaves + 1);
template <bool F16, int KVT>
__global__ __launch_bounds__(kQkvThreads) void qkv_rope_append_kernel(QkvRopeParams p) {
    __shared__ float lds_y[kLayerWaves];
    __shared__ float lds_cs[2][2];      // per pair: cos, sin
    __shared__ uint8_t *lds_dst[2];     // per pair: the K or V row (null: not written)
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tok = blockIdx.y;
    const int hd = p.ap.head_dim;
    const int n_kv = p.ap.n_head_kv * hd;
    if (wave == kLayerWaves) {
        if (lane < 2) {
            const int row = (int)blockIdx.x * kLayerWaves + 2 * lane;  // the pair's first row
            const bool is_q = row < p.n_q, is_k = !is_q && row < p.n_q + n_kv;
            const int r = is_q ? row : row - p.n_q - (is_k ? 0 : n_kv);
            const int ps = p.ap.pos[tok];
            const bool valid = ps >= 0 && p.ap.seq[tok] >= 0;
            float c = 1.0f, sn = 0.0f;
            if (valid && (is_q || is_k)) rope_cos_sin(ps, (r % hd) / 2, p.theta_scale, c, sn);
            lds_cs[lane][0] = c;
            lds_cs[lane][1] = sn;
            lds_dst[lane] = is_q ? nullptr : row_ptr(p.ap, is_k ? 0 : 1, tok, r / hd);
        }
    } else {
        const int row = (int)blockIdx.x * kLayerWaves + wave;  // < n_out (n_out % 4 == 0)
        const int nc = p.n_in / 8;
        const floatx4 *xr = reinterpret_cast<const floatx4 *>(p.x + (int64_t)tok * p.n_in);
        float acc = 0.0f;
        int c_rest = lane;
        if constexpr (F16) {  // gemv_kernel's batches for one token
            const half8 *W = static_cast<const half8 *>(p.w);
            constexpr int CB = kGemvBatch;
            const int full = nc / (64 * CB) * (64 * CB);
            for (int c0 = lane; c0 < full; c0 += 64 * CB) {
                half8 wv[CB];
                floatx4 x0[CB], x1[CB];
#pragma unroll
                for (int k = 0; k < CB; ++k) {
                    x0[k] = xr[2 * (c0 + 64 * k)];
                    x1[k] = xr[2 * (c0 + 64 * k) + 1];
                }
#pragma unroll
                for (int k = 0; k < CB; ++k) wv[k] = W[(int64_t)row * nc + c0 + 64 * k];
#pragma unroll
                for (int k = 0; k < CB; ++k) acc = dot8(wv[k], to_half8(x0[k], x1[k]), acc);
            }
            c_rest = full + lane;
        }
#pragma unroll 8
        for (int c = c_rest; c < nc; c += 64) {
            if constexpr (F16) {
                const half8 *W = static_cast<const half8 *>(p.w);
                acc = dot8(W[(int64_t)row * nc + c], to_half8(xr[2 * c], xr[2 * c + 1]), acc);
            } else {
                const floatx4 *W = static_cast<const floatx4 *>(p.w);
                acc = dot8(W[((int64_t)row * nc + c) * 2], W[((int64_t)row * nc + c) * 2 + 1], xr[2 * c],
                           xr[2 * c + 1], acc);
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) lds_y[wave] = acc;
    }
    __syncthreads();
    if (wave == kLayerWaves || lane != 0) return;
    const int row = (int)blockIdx.x * kLayerWaves + wave;
    const int pr = wave >> 1;
    const bool is_q = row < p.n_q, is_k = !is_q && row < p.n_q + n_kv;
    const int ps = p.ap.pos[tok];
    const bool valid = ps >= 0 && p.ap.seq[tok] >= 0;
    float y = lds_y[wave];
    if (valid && (is_q || is_k)) {
        float x0 = lds_y[wave & ~1], x1 = lds_y[wave | 1];
        rope_rotate(x0, x1, lds_cs[pr][0], lds_cs[pr][1]);
        y = (wave & 1) ? x1 : x0;
    }
    if (is_q) {
        p.q[(int64_t)tok * p.n_q + row] = y;
        return;
    }
    uint8_t *dst = lds_dst[pr];
    if (dst == nullptr) return;
    const int d = (row - p.n_q - (is_k ? 0 : n_kv)) % hd;
    if constexpr (KVT == SFA_KV_F16)
        reinterpret_cast<_Float16 *>(dst)[d] = (_Float16)y;
    else
        reinterpret_cast<float *>(dst)[d] = y;
}

// ---- host side -------------------------------------------------------------------

static int grid_x(int n) { return (n + kRowsPerBlock - 1) / kRowsPerBlock; }

template <int RW>
static void gemv_launch_rw(const GemvParams &p, bool f16, int nt, hipStream_t s) {
    const dim3 grid((p.n_out + kLayerWaves * RW - 1) / (kLayerWaves * RW), (p.n_rows + nt - 1) / nt);
#define SFA_GEMV(NT)                                                                           \
    case NT:                                                                                   \
        if (f16) hipLaunchKernelGGL((gemv_kernel<true, NT, RW>), grid, dim3(256), 0, s, p);   \
        else hipLaunchKernelGGL((gemv_kernel<false, NT, RW>), grid, dim3(256), 0, s, p);      \
        break;
    switch (nt) {
        SFA_GEMV(1)
        SFA_GEMV(2)
        SFA_GEMV(4)
        SFA_GEMV(8)
    }
#undef SFA_GEMV
}

static int gemv_launch(const GemvParams &p, bool f16, hipStream_t s) {
    const int nt = p.n_rows >= 8 ? 8 : p.n_rows >= 4 ? 4 : p.n_rows >= 2 ? 2 : 1;
    if (p.n_out >= 16384)
        gemv_launch_rw<4>(p, f16, nt, s);
    else if (p.n_out >= 8192)
        gemv_launch_rw<2>(p, f16, nt, s);
    else
        gemv_launch_rw<1>(p, f16, nt, s);
    return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
}

static bool weight_type_ok(int t) { return t == SFA_KV_F32 || t == SFA_KV_F16; }

}  // namespace sfa

extern "C" {

SFA_API int sfa_rms_norm(const float *x, const float *weight, float *y, int32_t n_rows, int32_t n_embd,
                         float eps, void *stream) {
    try {
        if (x == nullptr || weight == nullptr || y == nullptr) return SFA_ERR_INVALID_ARGUMENT;
        if (n_rows < 0 || n_embd <= 0 || !(eps >= 0.0f)) return SFA_ERR_INVALID_ARGUMENT;
        if (n_rows == 0) return SFA_OK;
        hipLaunchKernelGGL(sfa::rms_norm_kernel, dim3(n_rows), dim3(sfa::kNormThreads), 0,
                           static_cast<hipStream_t>(stream),
                           x, weight, y, n_embd, eps);
        return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API int sfa_mul_mat_vec(const void *w, int32_t w_type, const float *x, const float *residual, float *y,
                            int32_t n_rows, int32_t n_in, int32_t n_out, void *stream) {
    try {
        if (w == nullptr || x == nullptr || y == nullptr) return SFA_ERR_INVALID_ARGUMENT;
        if (n_rows < 0 || n_in <= 0 || n_out <= 0) return SFA_ERR_INVALID_ARGUMENT;
        if (!sfa::weight_type_ok(w_type) || n_in % 8 != 0) return SFA_ERR_UNSUPPORTED;
        if ((n_rows + 7) / 8 > 65535) return SFA_ERR_UNSUPPORTED;  // token blocks on grid y
        if (n_rows == 0) return SFA_OK;
        const sfa::GemvParams p{w, x, residual, y, n_rows, n_in, n_out};
        return sfa::gemv_launch(p, w_type == SFA_KV_F16, static_cast<hipStream_t>(stream));
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API int sfa_moe_route(const float *logits, int32_t n_rows, int32_t n_expert, int32_t n_used,
                          int32_t *ids, float *weights, void *stream) {
    try {
        if (logits == nullptr || ids == nullptr || weights == nullptr) return SFA_ERR_INVALID_ARGUMENT;
        if (n_rows < 0 || n_expert <= 0 || n_used <= 0 || n_used > n_expert) return SFA_ERR_INVALID_ARGUMENT;
        if (n_expert > 64) return SFA_ERR_UNSUPPORTED;
        if (n_rows == 0) return SFA_OK;
        hipLaunchKernelGGL(sfa::moe_route_kernel, dim3(n_rows), dim3(64), 0, static_cast<hipStream_t>(stream),
                           logits, n_expert, n_used, ids, weights);
        return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API int sfa_moe_gate(const void *gate_inp, int32_t w_type, const float *x, int32_t n_rows, int32_t n_embd,
                         int32_t n_expert, int32_t n_used, int32_t *ids, float *weights, void *stream) {
    try {
        if (gate_inp == nullptr || x == nullptr || ids == nullptr || weights == nullptr)
            return SFA_ERR_INVALID_ARGUMENT;
        if (n_rows < 0 || n_embd <= 0 || n_expert <= 0 || n_used <= 0 || n_used > n_expert)
            return SFA_ERR_INVALID_ARGUMENT;
        if (!sfa::weight_type_ok(w_type) || n_embd % 8 != 0 || n_expert > 64) return SFA_ERR_UNSUPPORTED;
        if (n_rows == 0) return SFA_OK;
        const hipStream_t s = static_cast<hipStream_t>(stream);
        if (w_type == SFA_KV_F16)
            hipLaunchKernelGGL(sfa::moe_gate_kernel<true>, dim3(n_rows), dim3(256), 0, s, gate_inp, x, n_embd,
                               n_expert, n_used, ids, weights);
        else
            hipLaunchKernelGGL(sfa::moe_gate_kernel<false>, dim3(n_rows), dim3(256), 0, s, gate_inp, x, n_embd,
                               n_expert, n_used, ids, weights);
        return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API int sfa_moe_norm_gate(const float *x, const float *norm_weight, float eps, const void *gate_inp,
                              int32_t w_type, int32_t n_rows, int32_t n_embd, int32_t n_expert, int32_t n_used,
                              float *y, int32_t *ids, float *weights, void *stream) {
    try {
        if (x == nullptr || norm_weight == nullptr || gate_inp == nullptr || y == nullptr || ids == nullptr ||
            weights == nullptr)
            return SFA_ERR_INVALID_ARGUMENT;
        if (n_rows < 0 || n_embd <= 0 || !(eps >= 0.0f) || n_expert <= 0 || n_used <= 0 || n_used > n_expert)
            return SFA_ERR_INVALID_ARGUMENT;
        if (!sfa::weight_type_ok(w_type) || n_embd % 8 != 0 || n_embd > sfa::kNormGateMaxEmbd || n_expert > 64)
            return SFA_ERR_UNSUPPORTED;
        if (n_rows == 0) return SFA_OK;
        const hipStream_t s = static_cast<hipStream_t>(stream);
        if (w_type == SFA_KV_F16)
            hipLaunchKernelGGL(sfa::moe_norm_gate_kernel<true>, dim3(n_rows), dim3(sfa::kNormThreads), 0, s, x,
                               norm_weight, eps, gate_inp, n_embd, n_expert, n_used, y, ids, weights);
        else
            hipLaunchKernelGGL(sfa::moe_norm_gate_kernel<false>, dim3(n_rows), dim3(sfa::kNormThreads), 0, s, x,
                               norm_weight, eps, gate_inp, n_embd, n_expert, n_used, y, ids, weights);
        return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API int sfa_qkv_rope_kv_append(const sfa_kv_desc *kv, const void *w_qkv, int32_t w_type, const float *x,
                                   int32_t n_embd, float *q, const int32_t *seq, const int32_t *pos,
                                   int32_t n_tok, const int32_t *page_table, int32_t max_pages,
                                   float freq_base, void *stream) {
    try {
        if (kv == nullptr || w_qkv == nullptr || x == nullptr || q == nullptr || seq == nullptr ||
            pos == nullptr || page_table == nullptr)
            return SFA_ERR_INVALID_ARGUMENT;
        const int rc = sfa_kv_desc_check(kv);
        if (rc != SFA_OK) return rc;
        if (n_tok < 0 || n_embd <= 0 || max_pages <= 0 || !(freq_base > 0.0f)) return SFA_ERR_INVALID_ARGUMENT;
        if (kv->kv_type != SFA_KV_F16 && kv->kv_type != SFA_KV_F32) return SFA_ERR_UNSUPPORTED;
        if (!sfa::weight_type_ok(w_type) || n_embd % 8 != 0 || n_tok > 65535) return SFA_ERR_UNSUPPORTED;
        if (n_tok == 0) return SFA_OK;
        sfa::QkvRopeParams p;
        p.w = w_qkv;
        p.x = x;
        p.q = q;
        p.n_in = n_embd;
        p.n_q = kv->n_head * kv->head_dim;
        p.n_out = p.n_q + 2 * kv->n_head_kv * kv->head_dim;
        p.theta_scale = powf(freq_base, -2.0f / (float)kv->head_dim);  // ggml: powf(base, -2/n_dims)
        sfa::AppendParams &a = p.ap;
        a.k_pages = static_cast<uint8_t *>(kv->k_pages);
        a.v_pages = static_cast<uint8_t *>(kv->v_pages);
        a.k_cold = static_cast<uint8_t *>(kv->k_cold);
        a.v_cold = static_cast<uint8_t *>(kv->v_cold);
        a.row_bytes = (int)sfa_row_bytes(kv);
        a.page_bytes = (int64_t)a.row_bytes * kv->n_head_kv * kv->page_size;
        a.n_pages = kv->n_pages;
        a.n_cold = kv->n_cold_pages;
        a.page_size = kv->page_size;
        a.n_head_kv = kv->n_head_kv;
        a.head_dim = kv->head_dim;
        a.k = a.v = nullptr;
        a.seq = seq;
        a.pos = pos;
        a.n_tok = n_tok;
        a.page_table = page_table;
        a.max_pages = max_pages;
        const dim3 grid((unsigned)(p.n_out / sfa::kLayerWaves), (unsigned)n_tok);
        const hipStream_t s = static_cast<hipStream_t>(stream);
        const bool f16w = w_type == SFA_KV_F16;
        if (kv->kv_type == SFA_KV_F16) {
            if (f16w) hipLaunchKernelGGL((sfa::qkv_rope_append_kernel<true, SFA_KV_F16>), grid, dim3(sfa::kQkvThreads), 0, s, p);
            else hipLaunchKernelGGL((sfa::qkv_rope_append_kernel<false, SFA_KV_F16>), grid, dim3(sfa::kQkvThreads), 0, s, p);
        } else {
            if (f16w) hipLaunchKernelGGL((sfa::qkv_rope_append_kernel<true, SFA_KV_F32>), grid, dim3(sfa::kQkvThreads), 0, s, p);
            else hipLaunchKernelGGL((sfa::qkv_rope_append_kernel<false, SFA_KV_F32>), grid, dim3(sfa::kQkvThreads), 0, s, p);
        }
        return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

SFA_API size_t sfa_moe_workspace_bytes(int32_t n_rows, int32_t n_used, int32_t n_ff) {
    if (n_rows <= 0 || n_used <= 0 || n_ff <= 0) return 0;
    return (size_t)n_rows * n_used * n_ff * sizeof(float);
}

SFA_API int sfa_moe_ffn(const float *x, const float *residual, const int32_t *ids, const float *weights,
                        const void *gate_exps, const void *up_exps, const void *down_exps, int32_t w_type,
                        int32_t n_rows, int32_t n_embd, int32_t n_ff, int32_t n_expert, int32_t n_used,
                        void *workspace, size_t ws_bytes, float *y, void *stream) {
    try {
        if (x == nullptr || residual == nullptr || ids == nullptr || weights == nullptr || y == nullptr)
            return SFA_ERR_INVALID_ARGUMENT;
        if (gate_exps == nullptr || up_exps == nullptr || down_exps == nullptr) return SFA_ERR_INVALID_ARGUMENT;
        if (n_rows < 0 || n_embd <= 0 || n_ff <= 0 || n_expert <= 0 || n_used <= 0 || n_used > n_expert)
            return SFA_ERR_INVALID_ARGUMENT;
        if (!sfa::weight_type_ok(w_type) || n_embd % 8 != 0 || n_ff % 8 != 0) return SFA_ERR_UNSUPPORTED;
        if (n_rows == 0) return SFA_OK;
        if (workspace == nullptr || ws_bytes < sfa_moe_workspace_bytes(n_rows, n_used, n_ff))
            return SFA_ERR_INVALID_ARGUMENT;
        if (n_rows > 65535 || n_used > 8) return SFA_ERR_UNSUPPORTED;
        sfa::MoeParams p{x, residual, ids, weights, gate_exps, up_exps, down_exps, static_cast<float *>(workspace),
                         y, n_rows, n_embd, n_ff, n_expert, n_used};
        const hipStream_t s = static_cast<hipStream_t>(stream);
        const bool f16 = w_type == SFA_KV_F16;
        const dim3 g1(sfa::grid_x(n_ff), n_used, n_rows);
        const dim3 g2((n_embd + sfa::kLayerWaves * sfa::kDownRows - 1) / (sfa::kLayerWaves * sfa::kDownRows), n_rows);
        if (f16)
            hipLaunchKernelGGL(sfa::moe_gate_up_kernel<true>, g1, dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL(sfa::moe_gate_up_kernel<false>, g1, dim3(256), 0, s, p);
        switch (n_used) {
#define SFA_DOWN(NU)                                                                       \
    case NU:                                                                               \
        if (f16) hipLaunchKernelGGL((sfa::moe_down_kernel<true, NU>), g2, dim3(256), 0, s, p);   \
        else hipLaunchKernelGGL((sfa::moe_down_kernel<false, NU>), g2, dim3(256), 0, s, p);      \
        break;
            SFA_DOWN(1)
            SFA_DOWN(2)
            SFA_DOWN(3)
            SFA_DOWN(4)
            SFA_DOWN(5)
            SFA_DOWN(6)
            SFA_DOWN(7)
            SFA_DOWN(8)
#undef SFA_DOWN
        }
        return hipGetLastError() == hipSuccess ? SFA_OK : SFA_ERR_RUNTIME;
    } catch (...) {
        return SFA_ERR_RUNTIME;
    }
}

}  // extern "C"
