/*
 * xq_oracle.h — CPU oracle for the attention + gated-delta-net hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * ggml CPU semantics (the ggml sources themselves are not available to build).
 * Only the test suite, the smoke check and the benchmark's CPU-baseline leg may
 * load it, and only as the reference results are compared with; the product
 * library never links it.
 *
 * Each function cites the reference file:line it restates. Functions marked
 * "parity unpinned at bit level" follow upstream ggml's published algorithm
 * whose exact summation order cannot be compiled here; their results are pinned
 * by closed forms and invariants in tests/ to within float rounding.
 */
#ifndef XQ_ORACLE_H
#define XQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/xq_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar codecs ---- */
uint16_t xo_f32_to_f16(float x);
float xo_f16_to_f32(uint16_t h);
uint16_t xo_f32_to_bf16(float x);
float xo_bf16_to_f32(uint16_t h);
uint8_t xo_f16_to_e5m2(uint16_t h);
uint16_t xo_e5m2_to_f16(uint8_t b);

/* ---- row codecs (n elements) ---- */
void xo_f32_to_f16_row(const float* x, uint16_t* y, int64_t n);
void xo_f16_to_f32_row(const uint16_t* x, float* y, int64_t n);
void xo_f32_to_bf16_row(const float* x, uint16_t* y, int64_t n);
void xo_bf16_to_f32_row(const uint16_t* x, float* y, int64_t n);
void xo_f32_to_e5m2_row(const float* x, uint8_t* y, int64_t n);

/* q8 variant: 0 = ggml-cpu x86 quantize_row_q8_0, 1 = quantize_row_q8_0_ref. */
void xo_quantize_row_q8_0(const float* x, void* y, int64_t k, int variant);
void xo_quantize_row_q4_0(const float* x, void* y, int64_t k);
/* Any of F32/F16/BF16/Q8_0/Q4_0/E5M2 -> f32. */
void xo_dequant_row(int type, const void* x, float* y, int64_t k);
size_t xo_row_bytes(int type, int64_t k);

/* ---- flash attention ---- */

/* ggml CPU flash_attn_ext one-chunk loop (tensors hold HOST pointers).
 * qk_policy: enum xq_fa_qk_policy. v_acc_f16: 1 = ggml's f16 V accumulator for
 * F16 V (faithful), 0 = f32 accumulator. lse may be NULL. Returns 0 on success. */
int xo_flash_attn_ext(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                      const xq_tensor* mask, const xq_tensor* sinks, const xq_tensor* dst,
                      float* lse, float scale, float max_bias, float softcap, int qk_policy,
                      int v_acc_f16, int n_threads);

/* float64 closed form softmax(Q K^T * scale (softcapped) + slope*mask) V over
 * the decoded K/V. q_round: 0 = Q as given (f32), 1 = Q converted as the
 * policy's vec-dot does (q8_0 round trip for quantized K, f16 for NATIVE F16 K). */
int xo_flash_attn_f64(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                      const xq_tensor* mask, const xq_tensor* sinks, double* out, double* lse,
                      float scale, float max_bias, float softcap, int qk_policy, int q_round,
                      int n_threads);

/* ALiBi slope for head h of n_head (ggml flash_attn_ext). */
float xo_alibi_slope(float max_bias, int n_head, int h);

/* ---- RKVA range attention (shaders/rkva/rkva_range_attn.hlsl + reducers) ---- */

int32_t xo_ref_split_k(uint32_t active);                         /* rkva-range-profile.h:99-101 */
int32_t xo_opt_split_k(uint32_t active, uint32_t mode);          /* :103-107 (modes 1..3) */
uint32_t xo_split_rows(uint32_t active, uint32_t split_k);       /* :109-111 */
void xo_q4_mq_split(uint32_t active, uint32_t mode, uint32_t* split_k, uint32_t* rows); /* :141-147 */

/* Pass 1 of rkva_range_attn.hlsl:59-106 for every split: partials laid out
 * [split][n_q*n_head][D+2] (acc, max, den). */
int xo_range_attn_partials(const float* q, const int32_t* positions, int32_t n_q, int32_t n_head,
                           const void* k, const void* v, int32_t n_head_kv, int32_t head_dim,
                           int32_t kv_type, int32_t origin, int32_t active, float kq_scale,
                           int32_t split_k, float* partials);
/* rkva_range_reduce.hlsl:12-46 (poison = 0) or rkva_range_reduce_opt.hlsl:25-133
 * (poison = 1): out [n_qh][D] then lse [n_qh]. */
int xo_range_reduce(const float* partials, int32_t n_qh, int32_t head_dim, int32_t split_k,
                    int32_t poison, float* out, float* lse);

/* Merge of position-split range results (OUT [rows][D] + LSE [rows] per part,
 * parts over disjoint KV ranges) in part order, with the reducer's poisoning. */
int xo_lse_merge(const float* parts_out, const float* parts_lse, int32_t n_parts, int64_t rows,
                 int32_t D, float* out, float* lse);

/* ---- gated delta net ---- */

/* Sequential recurrence in the order of d3d12_gdn_emulate
 * (src/bridge/ggml_d3d12.cpp:113-158), batched over ne[3] sequences. q/k/v may
 * be F32 or BF16. dst rows as the op's output. */
int xo_gated_delta_net(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                       const xq_tensor* g, const xq_tensor* beta, const xq_tensor* state,
                       const xq_tensor* dst, int32_t slots, int n_threads);
/* Same recurrence in float64 (y and states in double, dst layout). */
int xo_gated_delta_net_f64(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                           const xq_tensor* g, const xq_tensor* beta, const xq_tensor* state,
                           double* dst, int32_t slots, int n_threads);

/* ---- KV append ---- */
int xo_kv_store(const float* src, const int32_t* positions, int32_t n_tokens, int32_t n_head_kv,
                int32_t head_dim, int32_t kv_type, int32_t q8_variant, void* dst,
                int32_t capacity);

#ifdef __cplusplus
}
#endif

#endif /* XQ_ORACLE_H */
