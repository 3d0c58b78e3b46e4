/*
 * xq_attn.h — C ABI of the MI355X (gfx950) attention hot path for Qwen3.5-style
 * hybrid models: flash-attention decode / short multi-query verify over an
 * f16 / q8_0 / q4_0 / fp8(E5M2) KV cache, and the gated-delta-net recurrence
 * (single-token step and chunked prefill).
 *
 * The ABI keeps ggml's op-level contract so it can sit behind a ggml backend:
 *   - tensors are described by ggml's (type, ne[4], nb[4], data) with ggml type
 *     ids, innermost dimension first, strides in bytes;
 *   - KV block formats are ggml's block_q8_0 {f16 d; int8 qs[32]} (34 B) and
 *     block_q4_0 {f16 d; uint8 qs[16]} (18 B);
 *   - mask / scale / max_bias (ALiBi) / logit_softcap / sinks follow
 *     GGML_OP_FLASH_ATTN_EXT, output permuted to [D, n_head, n_q, n_seq];
 *   - GATED_DELTA_NET keeps the transposed f32 state layout and the output
 *     [4096, T + slots*128] = per-token outputs then rollback state snapshots.
 *
 * All pointers in xq_tensor.data are DEVICE pointers. Calls are asynchronous on
 * the given HIP stream (NULL = the default stream); a caller that needs ggml's
 * synchronous graph_compute contract synchronizes the stream itself. No entry
 * point allocates device memory: scratch comes from a caller-owned workspace
 * whose size is returned by the *_workspace queries. Errors are returned as
 * xq_status codes (never abort); xq_last_error() gives a message for the
 * calling thread. Calls sharing one workspace buffer must be ordered by the
 * caller. xq_flash_attn_ext calls with more than one KV split launch a second
 * kernel (the ascending-order split merge) on the same stream; calls keep no
 * state between them.
 */
#ifndef XQ_ATTN_H
#define XQ_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XQ_ABI_VERSION 1

/* ggml type ids (ggml.h enum ggml_type) for the formats this path reads. */
enum xq_type {
    XQ_TYPE_F32 = 0,
    XQ_TYPE_F16 = 1,
    XQ_TYPE_Q4_0 = 2,
    XQ_TYPE_Q8_0 = 8,
    XQ_TYPE_BF16 = 30,
    /* FP8 E5M2 KV storage: not a ggml type. One byte per element, decoded as
     * the upper byte of an IEEE f16 (value = f16(byte << 8)), encoded from f32
     * via f16 RNE then E5M2 RNE with finite saturation to 0x7b, the codec of
     * shaders/rkva/rkva_range_bulk_f16.hlsl:156-167. Id chosen outside ggml's
     * range. */
    XQ_TYPE_E5M2 = 0x100,
};

typedef enum xq_status {
    XQ_OK = 0,
    XQ_ERR_UNSUPPORTED = 1, /* valid ggml op, but outside what this backend runs */
    XQ_ERR_BAD_SHAPE = 2,   /* inconsistent ne/nb/type combination */
    XQ_ERR_BAD_ARG = 3,     /* null pointer, bad enum, bad scalar */
    XQ_ERR_WORKSPACE = 4,   /* workspace missing or smaller than required */
    XQ_ERR_HIP = 5,         /* a HIP runtime call failed */
} xq_status;

/* ggml_tensor's data-bearing fields (ggml.h struct ggml_tensor: type, ne, nb,
 * data). ne[i] = elements along dim i (innermost first), nb[i] = byte stride. For
 * block types nb[0] is the block size in bytes and ne[0] counts elements. */
typedef struct xq_tensor {
    int32_t type;
    int32_t reserved;
    int64_t ne[4];
    size_t nb[4];
    void* data;
} xq_tensor;

/* ---------------------------------------------------------------------------
 * Flash attention (GGML_OP_FLASH_ATTN_EXT)
 * ------------------------------------------------------------------------- */

/* How Q meets K in the score dot product.
 *  XQ_FA_QK_CONSISTENT (default): the reference's consistent query policy
 *    (GGML_FLASH_ATTN_NO_QUERY_TILING=4 with GGML_FLASH_ATTN_NO_SPLIT_KV=1;
 *    patches/0008-flash-attn-query-consistency.patch:7-9,30-37): F32 Q with
 *    F16 K/V keeps Q in f32 and expands K to f32; quantized K uses the
 *    native vec-dot (Q quantized to q8_0, integer block dots).
 *  XQ_FA_QK_NATIVE: ggml's q_to_vec_dot for every K type (Q rounded to f16 for
 *    F16 K; Q quantized to q8_0 for Q8_0/Q4_0 K).
 * E5M2 K always uses f32 Q against the decoded K. */
enum xq_fa_qk_policy {
    XQ_FA_QK_CONSISTENT = 0,
    XQ_FA_QK_NATIVE = 1,
};

/* KV split (split-K) policy. The partition never depends on the number of
 * queries, and a query tile's kernel variant (wave count, slice-to-wave
 * assignment) depends on the head dim and GQA group only, so a query's result
 * is bitwise independent of how many queries share the call
 * (patches/0008-flash-attn-query-consistency.patch:40-56). Partial states
 * are merged in ascending split order. A split is rows_per_split contiguous
 * rows, except in the matrix-core engine under AUTO and LENGTH (no positions):
 * there the splits take the KV rows in groups of 128 (8 waves x 16-row
 * slices) in turn, split s the groups s, s + n, s + 2n, ... of n splits, so
 * their sizes differ by at most one group whatever the KV length.
 *  XQ_FA_SPLIT_AUTO: MI355X policy, about 256 / (sequences x KV heads) splits
 *    (one workgroup per CU), rows a multiple of 16 and at least 256 per split
 *    (at most ceil(L/256) splits). It depends on the number
 *    of sequences and KV heads of the call: a sequence's bits can change with
 *    the batch it is in.
 *  The other modes depend on the KV length only (as the reference's do,
 *  uwp/rkva/rkva-range-profile.h:99-107): under them a sequence's result is
 *  also bitwise independent of the sequences batched with it.
 *  XQ_FA_SPLIT_REFERENCE: clamp(ceil(L/256), 1, 32) splits
 *    (uwp/rkva/rkva-range-profile.h:99-101).
 *  XQ_FA_SPLIT_BALANCED / FINE / COARSE: the reference's optimized modes
 *    1/2/3 (target rows, max splits) = (128,128) / (32,256) / (512,64)
 *    (uwp/rkva/rkva-range-profile.h:82-107).
 *  XQ_FA_SPLIT_NONE: one split (no reduce pass).
 *  XQ_FA_SPLIT_MQ_BALANCED / MQ_FINE: the reference's multi-query verify split
 *    (q4_mq_split, uwp/rkva/rkva-range-profile.h:141-147): the balanced / fine
 *    mode's rows rounded up to whole 64-row tiles, the count recomputed so no
 *    split is empty (58128 rows: 114 x 512 / 228 x 256).
 *  XQ_FA_SPLIT_LENGTH: MI355X length-only split: AUTO's partition evaluated
 *    for 16 (sequence x KV head) units whatever the call holds, i.e. at most
 *    16 splits of a multiple of 16 rows, at least 256 rows each. A call with
 *    16 such units (4 sequences x 4 KV heads at 32k rows, one workgroup per
 *    CU) runs exactly AUTO's partition; others trade occupancy for results
 *    that do not depend on the batch. */
enum xq_fa_split_mode {
    XQ_FA_SPLIT_AUTO = 0,
    XQ_FA_SPLIT_REFERENCE = 1,
    XQ_FA_SPLIT_BALANCED = 2,
    XQ_FA_SPLIT_FINE = 3,
    XQ_FA_SPLIT_COARSE = 4,
    XQ_FA_SPLIT_NONE = 5,
    XQ_FA_SPLIT_MQ_BALANCED = 6,
    XQ_FA_SPLIT_MQ_FINE = 7,
    XQ_FA_SPLIT_LENGTH = 8,
};

/* Which pass-1 kernel computes the scores and the value product.
 *  XQ_FA_ENGINE_AUTO: the matrix-core kernel where it exists (q8_0/q4_0 K with
 *    integer scores, F16/E5M2 K), else the VALU kernel. Its value products
 *    (quantized V: weight x block scale; F16/E5M2 V: the weight) enter the
 *    matrix cores as f16 hi + lo, about 22 significant bits, against the exact
 *    V values, with f32 accumulation.
 *  XQ_FA_ENGINE_MFMA: the matrix-core kernel (UNSUPPORTED where it does not exist).
 *  XQ_FA_ENGINE_VALU: the vector-ALU kernel (dot4 integer scores, f32 FMA values:
 *    ggml's f32 value products, slower). */
enum xq_fa_engine {
    XQ_FA_ENGINE_AUTO = 0,
    XQ_FA_ENGINE_MFMA = 1,
    XQ_FA_ENGINE_VALU = 2,
};

typedef struct xq_fa_params {
    float scale;         /* op_params[0] */
    float max_bias;      /* op_params[1], ALiBi; 0 = off */
    float logit_softcap; /* op_params[2]; 0 = off */
    int32_t qk_policy;   /* enum xq_fa_qk_policy */
    int32_t split_mode;  /* enum xq_fa_split_mode */
    int32_t engine;      /* enum xq_fa_engine */
    int32_t reserved[2];
} xq_fa_params;

/* Pure predicate mirroring a ggml backend's supports_op for
 * GGML_OP_FLASH_ATTN_EXT (same role as dev_supports_op,
 * src/bridge/ggml_d3d12.cpp:2331-2347). Returns 1 when xq_flash_attn_ext runs
 * the op, 0 otherwise; mask and sinks may be NULL. Shapes follow ggml:
 *   q    F32          [D, n_q, H, B]
 *   k    F16/Q8_0/Q4_0/E5M2 [D, L, Hkv, B]  (rows = KV positions)
 *   v    same type as k     [D, L, Hkv, B]
 *   mask F16 (or NULL)      [L, >= n_q, 1 or H, 1 or B], 0 / -inf / finite bias
 *   sinks F32 (or NULL)     [H]
 *   dst  F32                [D, H, n_q, B]  (ggml's permuted output) */
int xq_supports_flash_attn_ext(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                               const xq_tensor* mask, const xq_tensor* sinks,
                               const xq_tensor* dst, const xq_fa_params* params);

/* Device workspace bytes xq_flash_attn_ext needs for these shapes. */
xq_status xq_flash_attn_ext_workspace(const xq_tensor* q, const xq_tensor* k,
                                      const xq_tensor* v, const xq_tensor* mask,
                                      const xq_tensor* sinks, const xq_tensor* dst,
                                      const xq_fa_params* params, size_t* bytes);

/* GGML_OP_FLASH_ATTN_EXT on the GPU (replaces the CPU op's one-chunk loop,
 * ggml-cpu ops.cpp ggml_compute_forward_flash_attn_ext_f16, as patched by
 * patches/0006-cpu-flash-attn-consistent-kv-reduction.patch:3-14 and
 * patches/0008-flash-attn-query-consistency.patch:3-56). Writes dst and, when
 * lse != NULL, the natural-log softmax normaliser per (q, head, seq) as
 * lse[(b*n_q + iq)*H + h] (-inf for a fully masked row, whose output is 0).
 * stream is a hipStream_t. */
xq_status xq_flash_attn_ext(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                            const xq_tensor* mask, const xq_tensor* sinks, xq_tensor* dst,
                            float* lse, const xq_fa_params* params, void* workspace,
                            size_t workspace_bytes, void* stream);

/* xq_flash_attn_ext without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. It
 * allocates nothing: its workspace is a 32 MiB array in the library's device
 * image, one per GPU, whose address is looked up on the first call on a device
 * (the current device must be the stream's). Calls whose workspace
 * (xq_flash_attn_ext_workspace) exceeds 32 MiB return XQ_ERR_WORKSPACE before
 * any launch. Every call on a GPU shares that GPU's array (nothing in it needs
 * to start zeroed): calls that overlap on one GPU race and must be ordered by
 * the caller. Results equal xq_flash_attn_ext's bit for bit. */
xq_status xq_flash_attn_ext_noalloc(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                                    const xq_tensor* mask, const xq_tensor* sinks, xq_tensor* dst,
                                    float* lse, const xq_fa_params* params, void* stream);

/* Range attention (the remote-KV-attention engine's attend_range,
 * uwp/rkva/remote-attn-engine.h:152-154 and op RKVA_RANGE_ATTN,
 * uwp/rkva/remote-attn-protocol.h:228-237). KV rows are compact: row r holds
 * absolute position origin + r, rows [0, active) are live. Query i at absolute
 * position positions[i] sees rows [0, min(active, positions[i] - origin + 1))
 * (none when positions[i] < origin).
 *   q         F32 [n_q][n_head][D] (device)
 *   positions I32 [n_q] (device)
 *   k, v      cache planes [capacity][n_head_kv][record] of kv_type (device)
 *   out       F32 [n_q][n_head][D], lse F32 [n_q][n_head] (device); an empty
 *             range gives O = 0, LSE = -inf.
 * split_mode as in xq_fa_params. Scores use f32 Q against the decoded K
 * (shaders/rkva/rkva_range_attn.hlsl:74-78); split states merge with the
 * non-finite poisoning of shaders/rkva/rkva_range_reduce_opt.hlsl:39-56. */
xq_status xq_fa_range_workspace(int32_t n_q, int32_t n_head, int32_t n_head_kv,
                                int32_t head_dim, int32_t kv_type, int32_t active,
                                int32_t split_mode, size_t* bytes);
xq_status xq_fa_range(const float* q, const int32_t* positions, int32_t n_q, int32_t n_head,
                      const void* k, const void* v, int32_t n_head_kv, int32_t head_dim,
                      int32_t kv_type, int32_t origin, int32_t active, float kq_scale,
                      int32_t split_mode, float* out, float* lse, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Merge of position-split results: n_parts results of the same rows
 * (query, head) over disjoint KV ranges, each OUT [rows][head_dim] F32 and
 * natural-log LSE [rows] F32 as xq_fa_range or xq_flash_attn_ext return them
 * (an empty range is O = 0, LSE = -inf), into OUT and LSE over the union:
 * M = max LSE_p over the parts with LSE_p != -inf,
 * OUT = sum_p OUT_p e^(LSE_p - M) / sum_p e^(LSE_p - M), LSE = M + ln(sum),
 * accumulated in part order. This is the merge a caller applies after
 * splitting the KV rows between engines or devices (the result contract of
 * uwp/rkva/remote-attn-protocol.h:228-231; poisoning as the split reducer,
 * shaders/rkva/rkva_range_reduce_opt.hlsl:39-56,126-132: a participating
 * NaN or +inf LSE, or a non-finite merged value, makes the row NaN). No
 * participating part gives O = 0, LSE = -inf.
 *   parts_out [n_parts][rows][head_dim], parts_lse [n_parts][rows] (device)
 *   out [rows][head_dim], lse [rows] (device); 1 <= head_dim <= 512. */
xq_status xq_fa_lse_merge(const float* parts_out, const float* parts_lse, int32_t n_parts,
                          int64_t rows, int32_t head_dim, float* out, float* lse, void* stream);

/* The reference's knob semantics for the policy fields (host-side, pure
 * apart from reading the environment). ggml reads two variables, with exact
 * values only:
 *   GGML_FLASH_ATTN_NO_QUERY_TILING=4 -> qk_policy = XQ_FA_QK_CONSISTENT
 *     (patches/0008-flash-attn-query-consistency.patch:7-9: f32 Q with
 *     expanded F16 K, scalar queries); =1 -> XQ_FA_QK_NATIVE (scalar queries
 *     with ggml's own Q conversion, :46-56);
 *   GGML_FLASH_ATTN_NO_SPLIT_KV=1 -> split_mode = XQ_FA_SPLIT_LENGTH
 *     (patches/0006-cpu-flash-attn-consistent-kv-reduction.patch:7-11: no
 *     partition of the KV rows that depends on the batch or the threads;
 *     here a partition by the KV length only).
 * The reference's flashattn.txt=2 sets both (uwp/inference-bridge.cpp:887-893).
 * Absent, empty or other values leave the field as it is. */
xq_status xq_fa_params_from_env(xq_fa_params* params);

/* Split count the policy picks for a KV length (host-side, pure; AUTO is
 * evaluated for one sequence and one KV head). */
int32_t xq_fa_split_count(int64_t kv_len, int32_t split_mode);
/* Rows per split for that policy (the last split may be shorter; the
 * interleaved AUTO / LENGTH splits of the matrix-core engine hold the same
 * count of rows to within one 128-row group). */
int64_t xq_fa_split_rows(int64_t kv_len, int32_t split_mode);

/* ---------------------------------------------------------------------------
 * Gated delta net (GGML_OP_GATED_DELTA_NET)
 * ------------------------------------------------------------------------- */

enum xq_gdn_mode {
    XQ_GDN_AUTO = 0,     /* step for T <= 64, chunked above */
    XQ_GDN_STEP = 1,     /* token-sequential recurrence */
    XQ_GDN_CHUNKED = 2,  /* 64-token chunks in the UT form on the matrix cores (f32
                            operands split into f16 hi + lo, or three bf16 terms
                            against bf16 rows); q/k/v row strides of 2^25 bytes
                            or more run the token-sequential kernel instead, and
                            q/k rows outside the chunk operands' range, decays
                            e^g outside [0, 1], a non-finite beta, or an Inf/NaN
                            in v or the state run the token recurrence for the
                            heads or column blocks concerned */
};

/* Pure predicate mirroring d3d12_gdn_supported (src/bridge/ggml_d3d12.cpp:77-109),
 * widened to any T >= 1 and B >= 1 sequences and to BF16 q/k/v:
 *   q, k  F32|BF16 [128, 16, T, B]  rows contiguous
 *   v     F32|BF16 [128, 32, T, B]  rows contiguous
 *   g, beta F32 [1, 32, T, B] contiguous (activated scalar gates: g = log decay)
 *   state F32 [128, 128, 32, B] contiguous, state(i, c) of head h at
 *         h*16384 + c*128 + i (transposed; shaders/ggml_d3d12_gated_delta_net.hlsl:3)
 *   dst   F32 [4096, T + slots*128, B, 1] contiguous
 * slots in [1, 17]; raw_gates must be 0 (op_params[1]). The reference op is the
 * single-sequence case B == 1. */
int xq_supports_gated_delta_net(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                                const xq_tensor* g, const xq_tensor* beta,
                                const xq_tensor* state, const xq_tensor* dst, int32_t slots,
                                int32_t raw_gates);

xq_status xq_gated_delta_net_workspace(const xq_tensor* q, const xq_tensor* v, int32_t slots,
                                       int32_t mode, size_t* bytes);

/* GGML_OP_GATED_DELTA_NET on the GPU (the work of
 * shaders/ggml_d3d12_gated_delta_net.hlsl:40-85 dispatched at
 * src/bridge/ggml_d3d12.cpp:1905-1942). Per sequence, v-head h reads q/k head
 * h % 16; with S the state column of value index c:
 *   S *= exp(g[t,h]); delta = (v[t,h,c] - S.k) * beta[t,h]; S += k*delta;
 *   y[t,h,c] = (S.q) / sqrt(128).
 * dst rows [0, T) hold y as [T][32][128]; slot j (j < min(T, slots)) at row
 * T + 128*j holds the state j tokens before the end (slot 0 = final); with
 * slots == 1 only the final state is written. Rows of slots >= T are left
 * untouched. Inputs are never written. */
xq_status xq_gated_delta_net(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                             const xq_tensor* g, const xq_tensor* beta, const xq_tensor* state,
                             xq_tensor* dst, int32_t slots, int32_t raw_gates, int32_t mode,
                             void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * KV cache append (the step before the path)
 * ------------------------------------------------------------------------- */

/* Quantize/convert F32 rows src[n_tokens][n_head_kv][head_dim] into a KV cache
 * plane [capacity][n_head_kv][record] of kv_type at row positions[t]
 * (rows with positions outside [0, capacity) are skipped), the scatter of
 * shaders/rkva/rkva_store_f16.hlsl:63-85 widened to every KV type. F16 uses
 * ggml's RNE conversion (NaN -> 0x7e00|sign); Q8_0 and Q4_0 use
 * quantize_row_q8_0 / quantize_row_q4_0_ref; E5M2 uses the f16-then-E5M2 codec.
 * q8_variant: 0 = ggml-cpu x86 quantize_row_q8_0 (id = 127/amax, round half to
 * even), 1 = quantize_row_q8_0_ref (id = 1/d, roundf). */
xq_status xq_kv_store(const float* src, const int32_t* positions, int32_t n_tokens,
                      int32_t n_head_kv, int32_t head_dim, int32_t kv_type, int32_t q8_variant,
                      void* dst, int32_t capacity, void* stream);

/* Bytes of one (row, head) record of head_dim elements of kv_type (0 if unsupported). */
size_t xq_kv_record_bytes(int32_t kv_type, int32_t head_dim);

/* ---------------------------------------------------------------------------
 * Misc
 * ------------------------------------------------------------------------- */

/* Per-kernel device timing (the role of the reference's per-call GPU
 * timestamps, include/xllama/ggml_d3d12.h:253-289). While enabled, each kernel
 * launch of this library is bracketed by two HIP events on its stream.
 * xq_profile_read waits for the recorded events, folds them into per-kernel
 * totals and copies up to max entries: names (32 bytes each, NUL-padded),
 * total device milliseconds and launch counts; it returns the entry count.
 * Off by default; timing adds two event records per launch. */
void xq_profile_enable(int32_t on);
void xq_profile_reset(void);
int32_t xq_profile_read(char* names, double* total_ms, int64_t* launches, int32_t max);

/* Message for the last non-OK status on the calling thread ("" if none). */
const char* xq_last_error(void);
/* XQ_ABI_VERSION of the loaded library. */
int32_t xq_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* XQ_ATTN_H */
