/*
 * sfa_layer.h - C ABI of the rest of the decode layer around the attention
 * node (libsfa.so): the ops of build_router_segment and build_expert_segment
 * (src/model/engine/engine.cpp:1877-1925, 1945-1986 of the reference) on the
 * GPU, so a whole layer runs without a host round trip.  With sfa.h's
 * sfa_rope_kv_append and sfa_attn_decode / sfa_attn_prefill they cover the
 * layer:
 *
 *   cur     = rms_norm(x) * attn_norm         sfa_rms_norm            engine.cpp:1879-1880
 *   Q, K, V = Wq/Wk/Wv * cur                  sfa_mul_mat_vec         engine.cpp:1883-1885
 *   RoPE, KV append, attention                sfa.h                   engine.cpp:1892-1901
 *             (the product, RoPE and the
 *              append in one launch:          sfa_qkv_rope_kv_append)
 *   ffn_inp = Wo * attn + x                   sfa_mul_mat_vec         engine.cpp:1905-1906
 *             (the residual added in the same pass)
 *   cur     = rms_norm(ffn_inp) * ffn_norm    sfa_rms_norm            engine.cpp:1908-1909
 *   logits  = gate_inp * cur                  sfa_mul_mat_vec         engine.cpp:1912
 *   ids, w  = top-k of softmax, renormalised  sfa_moe_route           engine.cpp:1913-1925
 *             (both in one launch:            sfa_moe_gate;
 *              with the ffn_norm too:         sfa_moe_norm_gate)
 *   x'      = sum_j w_j * down_j(silu(gate_j * cur) * (up_j * cur)) + ffn_inp
 *                                             sfa_moe_ffn             engine.cpp:1964-1984
 *
 * Layouts are ggml's: activations [n_rows][n] f32 (one row per token); a
 * weight W with ggml ne = [n_in, n_out] is row-major [n_out][n_in]; expert
 * stacks (ne = [n_in, n_out, n_expert]) are [n_expert][n_out][n_in].  Weight
 * types use the ggml type ids of sfa.h (SFA_KV_F32 = 0, SFA_KV_F16 = 1).  The
 * arithmetic is ggml's CPU backend's: rms_norm sums squares in double; F16
 * weights take the activation rounded to f16 and sum the products in f32;
 * soft_max and sum_rows sum in double.  Every call is ordered on the given
 * stream, allocates nothing and never throws; all pointers are device
 * pointers.
 */
#ifndef SFA_LAYER_H
#define SFA_LAYER_H

#include "sfa.h"

#ifdef __cplusplus
extern "C" {
#endif

/* y = (x * 1/sqrtf(mean(x^2) + eps)) * weight per row of n_embd values
 * (ggml_rms_norm then ggml_mul, engine.cpp:1879-1880 and 1908-1909).  y may
 * alias x. */
SFA_API int sfa_rms_norm(const float *x, const float *weight, float *y, int32_t n_rows,
                         int32_t n_embd, float eps, void *stream);

/* y[t] = W * x[t] (+ residual[t]) for n_rows tokens: ggml_mul_mat(W, x)
 * (engine.cpp:1883-1885, 1912) and, with a residual, the wo projection plus
 * ggml_add (engine.cpp:1905-1906).  W [n_out][n_in] f32 or f16 (w_type);
 * n_in must be a multiple of 8 (SFA_ERR_UNSUPPORTED otherwise).  residual may
 * be null or alias y. */
SFA_API int sfa_mul_mat_vec(const void *w, int32_t w_type, const float *x, const float *residual,
                            float *y, int32_t n_rows, int32_t n_in, int32_t n_out, void *stream);

/* Softmax gating of build_moe_ffn (engine.cpp:1913-1925): per row, probs =
 * soft_max(logits), the n_used most probable experts in descending order
 * (ties: the lower expert id first), their probabilities divided by their sum
 * clamped below at 6.103515625e-5.  logits [n_rows][n_expert], ids and
 * weights [n_rows][n_used].  n_expert <= 64. */
SFA_API int sfa_moe_route(const float *logits, int32_t n_rows, int32_t n_expert, int32_t n_used,
                          int32_t *ids, float *weights, void *stream);

/* The router product and the gating in one launch: logits = gate_inp * x
 * (engine.cpp:1912, the sfa_mul_mat_vec arithmetic), then sfa_moe_route's
 * selection and weights (engine.cpp:1913-1925).  gate_inp [n_expert][n_embd]
 * f32 or f16, x [n_rows][n_embd] (n_embd a multiple of 8), n_expert <= 64. */
SFA_API int sfa_moe_gate(const void *gate_inp, int32_t w_type, const float *x, int32_t n_rows,
                         int32_t n_embd, int32_t n_expert, int32_t n_used, int32_t *ids,
                         float *weights, void *stream);

/* ffn_norm, the router product and the gating in one launch (engine.cpp:
 * 1908-1925): y = rms_norm(x) * norm_weight (sfa_rms_norm's arithmetic; y is
 * the experts' input), then sfa_moe_gate on y.  The results equal those two
 * calls bit for bit, with one launch less.  x, y [n_rows][n_embd] f32,
 * norm_weight [n_embd] f32, gate_inp [n_expert][n_embd] of w_type; n_embd a
 * multiple of 8 and <= 8192, n_expert <= 64 (else SFA_ERR_UNSUPPORTED). */
SFA_API int sfa_moe_norm_gate(const float *x, const float *norm_weight, float eps, const void *gate_inp,
                              int32_t w_type, int32_t n_rows, int32_t n_embd, int32_t n_expert,
                              int32_t n_used, float *y, int32_t *ids, float *weights, void *stream);

/* The stacked Q/K/V product, RoPE NORMAL and the KV append in one launch
 * (engine.cpp:1883-1885, 1892-1897, 1646-1656): the results of
 * sfa_mul_mat_vec(w_qkv, x) followed by sfa_rope_kv_append on its Q, K and V
 * parts, bit for bit, without the intermediate Q/K/V rows.
 *   w_qkv : [(n_head + 2 n_head_kv) * head_dim][n_embd] of w_type (the Q, K
 *           and V weights stacked row-wise), x : [n_tok][n_embd] f32
 *   q     : out, [n_tok][n_head][head_dim] f32, rotated (as computed for a
 *           token with seq or pos < 0, whose K/V are not written)
 *   seq, pos, page_table, max_pages, freq_base : as sfa_rope_kv_append.
 * F16 and F32 caches; SFA_ERR_UNSUPPORTED for Q8_0 (a block spans 16 RoPE
 * pairs: use the two calls) and for n_tok > 65535.  The weight matrix is read
 * once per token, so this is the decode path; a long chunk is better served by
 * sfa_mul_mat_vec + sfa_rope_kv_append. */
SFA_API int sfa_qkv_rope_kv_append(const sfa_kv_desc *kv, const void *w_qkv, int32_t w_type,
                                   const float *x, int32_t n_embd, float *q, const int32_t *seq,
                                   const int32_t *pos, int32_t n_tok, const int32_t *page_table,
                                   int32_t max_pages, float freq_base, void *stream);

/* Workspace bytes of sfa_moe_ffn (the SwiGLU activations, n_rows * n_used *
 * n_ff floats); 0 for an invalid shape. */
SFA_API size_t sfa_moe_workspace_bytes(int32_t n_rows, int32_t n_used, int32_t n_ff);

/* The expert segment (build_expert_segment, engine.cpp:1964-1984): for each
 * row t and slot j, e = ids[t][j]:
 *   act_j = silu(gate_exps[e] * x[t]) * (up_exps[e] * x[t])      (mul_mat_id, swiglu_split)
 *   y[t]  = sum over j in order of (down_exps[e] * act_j) * weights[t][j] + residual[t]
 * gate_exps / up_exps [n_expert][n_ff][n_embd], down_exps [n_expert][n_embd][n_ff],
 * all of w_type; n_embd and n_ff multiples of 8, n_used <= 8 (else
 * SFA_ERR_UNSUPPORTED).  An id outside
 * [0, n_expert) contributes nothing.  y must not alias x; it may alias
 * residual. */
SFA_API int sfa_moe_ffn(const float *x, const float *residual, const int32_t *ids,
                        const float *weights, const void *gate_exps, const void *up_exps,
                        const void *down_exps, int32_t w_type, int32_t n_rows, int32_t n_embd,
                        int32_t n_ff, int32_t n_expert, int32_t n_used, void *workspace,
                        size_t ws_bytes, float *y, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SFA_LAYER_H */
