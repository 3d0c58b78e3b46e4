// xq_api.hip — the C ABI of include/xq_attn.h: contract checks (pure
// predicates, as a ggml backend's supports_op), workspace sizing, split policy
// and dispatch to the gfx950 kernels. Nothing here allocates device memory.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <string>

#include "xq_kernels.h"

// ------------------------------------------------------------ no-alloc scratch
// The workspace of xq_flash_attn_ext_noalloc: one array per GPU, part of the
// library's device image (each GPU the library runs on holds it until the
// process ends). Host code reaches it only through the per-device address
// hipGetSymbolAddress returns (the array's name is not a device address).
constexpr size_t kScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

thread_local std::string g_last_error;

xq_status fail(xq_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return st;
}

xq_status ok() {
    g_last_error.clear();
    return XQ_OK;
}

size_t type_size(int t) {  // ggml_type_size: bytes of one element or block
    switch (t) {
    case XQ_TYPE_F32: return 4;
    case XQ_TYPE_F16:
    case XQ_TYPE_BF16: return 2;
    case XQ_TYPE_Q8_0: return 34;
    case XQ_TYPE_Q4_0: return 18;
    case XQ_TYPE_E5M2: return 1;
    default: return 0;
    }
}

bool kv_type_ok(int t) {
    return t == XQ_TYPE_F16 || t == XQ_TYPE_Q8_0 || t == XQ_TYPE_Q4_0 || t == XQ_TYPE_E5M2;
}

size_t record_bytes(int t, int64_t d) {
    switch (t) {
    case XQ_TYPE_F32: return (size_t)d * 4;
    case XQ_TYPE_F16:
    case XQ_TYPE_BF16: return (size_t)d * 2;
    case XQ_TYPE_Q8_0: return (size_t)(d / 32) * 34;
    case XQ_TYPE_Q4_0: return (size_t)(d / 32) * 18;
    case XQ_TYPE_E5M2: return (size_t)d;
    default: return 0;
    }
}

// Copy granularity of the K/V staging loads for a record size.
size_t kv_chunk(size_t rec) { return rec % 16 == 0 ? 16 : rec % 8 == 0 ? 8 : 4; }

// ------------------------------------------------------------ split policy

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Reference optimized modes (uwp/rkva/rkva-range-profile.h:82-107).
int64_t opt_split_k(int64_t active, int mode) {
    int64_t target = 128, max_splits = 128;
    if (mode == 2) {
        target = 32;
        max_splits = 256;
    } else if (mode == 3) {
        target = 512;
        max_splits = 64;
    }
    int64_t k = cdiv(active, target);
    if (k > max_splits) k = max_splits;
    if (k > 256) k = 256;
    return k < 1 ? 1 : k;
}

// n_seq_heads = sequences x KV heads of the call (never the query count, so a
// query's result does not depend on how many queries share the call).
void split_policy(int64_t L, int mode, int64_t n_seq_heads, int32_t* n_splits, int64_t* rows) {
    if (L <= 0) {
        *n_splits = 1;
        *rows = 1;
        return;
    }
    int64_t r = L, k = 1;
    switch (mode) {
    case XQ_FA_SPLIT_AUTO: {
        // about one workgroup per CU (256 on MI355X) over the (sequence, KV
        // head) pairs, rows a multiple of the 16-row wave slice, and at least
        // 256 rows per split (two slices per wave of the 8-wave decode): a
        // short call is bound by latency, and a second slice per wave costs
        // less than the partial states the extra splits write and merge
        // (4096 f16 rows over 8 KV heads: 16 splits 15.9 us per call, 32
        // splits 16.8 us)
        k = cdiv(256, n_seq_heads < 1 ? 1 : n_seq_heads);
        const int64_t kmax = cdiv(L, 256);
        if (k > kmax) k = kmax;
        if (k > 256) k = 256;
        if (k < 1) k = 1;
        r = cdiv(cdiv(L, k), 16) * 16;
        k = cdiv(L, r);
        break;
    }
    // the reference's modes keep their k even when the last split is empty
    // (rows * (k - 1) >= L happens, e.g. 58128 rows in the fine mode)
    case XQ_FA_SPLIT_REFERENCE:
        k = cdiv(L, 256);
        if (k > 32) k = 32;
        if (k < 1) k = 1;
        r = cdiv(L, k);
        break;
    case XQ_FA_SPLIT_BALANCED: k = opt_split_k(L, 1); r = cdiv(L, k); break;
    case XQ_FA_SPLIT_FINE: k = opt_split_k(L, 2); r = cdiv(L, k); break;
    case XQ_FA_SPLIT_COARSE: k = opt_split_k(L, 3); r = cdiv(L, k); break;
    // the reference's multi-query verify split (uwp/rkva/rkva-range-profile.h:
    // 141-147): the mode's rows rounded up to whole 64-row tiles, then the
    // split count recomputed so no split is empty
    case XQ_FA_SPLIT_MQ_BALANCED:
    case XQ_FA_SPLIT_MQ_FINE: {
        const int64_t k0 = opt_split_k(L, mode == XQ_FA_SPLIT_MQ_BALANCED ? 1 : 2);
        r = cdiv(cdiv(L, k0), 64) * 64;
        k = cdiv(L, r);
        break;
    }
    // AUTO's partition for 16 (sequence x KV head) units, whatever the call
    case XQ_FA_SPLIT_LENGTH: split_policy(L, XQ_FA_SPLIT_AUTO, 16, n_splits, rows); return;
    case XQ_FA_SPLIT_NONE:
    default: r = L; k = 1; break;
    }
    *rows = r;
    *n_splits = (int32_t)k;
}

// ------------------------------------------------------------ FA contract

struct FaPlan {
    int D, NQ, H, B, Hkv, G, kt;
    int64_t L;
    int qk_mode, q_round_f16;
    int32_t n_splits;
    int64_t split_rows;
    int interleave;  // this build's split modes (AUTO, LENGTH)
    size_t ws;
};

xq_status fa_check(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                   const xq_tensor* mask, const xq_tensor* sinks, const xq_tensor* dst,
                   const xq_fa_params* p, FaPlan* plan) {
    if (!q || !k || !v || !dst || !p) return fail(XQ_ERR_BAD_ARG, "null tensor or params");
    if (q->type != XQ_TYPE_F32) return fail(XQ_ERR_UNSUPPORTED, "q must be F32");
    if (dst->type != XQ_TYPE_F32) return fail(XQ_ERR_UNSUPPORTED, "dst must be F32");
    if (!kv_type_ok(k->type) || k->type != v->type)
        return fail(XQ_ERR_UNSUPPORTED, "k/v type %d/%d not supported (F16, Q8_0, Q4_0, E5M2; same type)", k->type, v->type);
    if (p->qk_policy != XQ_FA_QK_CONSISTENT && p->qk_policy != XQ_FA_QK_NATIVE)
        return fail(XQ_ERR_BAD_ARG, "bad qk_policy %d", p->qk_policy);
    if (p->split_mode < XQ_FA_SPLIT_AUTO || p->split_mode > XQ_FA_SPLIT_LENGTH)
        return fail(XQ_ERR_BAD_ARG, "bad split_mode %d", p->split_mode);
    if (p->engine < XQ_FA_ENGINE_AUTO || p->engine > XQ_FA_ENGINE_VALU)
        return fail(XQ_ERR_BAD_ARG, "bad engine %d", p->engine);
    for (int i = 0; i < 4; ++i)
        if (q->ne[i] < 1 || k->ne[i] < 0 || v->ne[i] < 0 || dst->ne[i] < 1)
            return fail(XQ_ERR_BAD_SHAPE, "bad ne");
    const int64_t D = q->ne[0];
    if (D != 128 && D != 256) return fail(XQ_ERR_UNSUPPORTED, "head dim %lld not in {128, 256}", (long long)D);
    if (k->ne[0] != D || v->ne[0] != D) return fail(XQ_ERR_UNSUPPORTED, "K/V head dims must equal Q's");
    if (k->ne[1] != v->ne[1]) return fail(XQ_ERR_BAD_SHAPE, "K and V lengths differ");
    if (k->ne[2] != v->ne[2] || k->ne[2] < 1) return fail(XQ_ERR_UNSUPPORTED, "K and V head counts differ");
    const int64_t H = q->ne[2], Hkv = k->ne[2], B = q->ne[3], NQ = q->ne[1];
    if (H % Hkv) return fail(XQ_ERR_BAD_SHAPE, "n_head %% n_head_kv != 0");
    if (H / Hkv > 32) return fail(XQ_ERR_UNSUPPORTED, "GQA group above 32");
    if (k->ne[3] < 1 || v->ne[3] < 1 || B % k->ne[3] || B % v->ne[3])
        return fail(XQ_ERR_BAD_SHAPE, "sequence broadcast");
    if (dst->ne[0] != D || dst->ne[1] != H || dst->ne[2] != NQ || dst->ne[3] != B)
        return fail(XQ_ERR_BAD_SHAPE, "dst must be [D, n_head, n_q, n_seq]");
    if (q->nb[0] != 4 || dst->nb[0] != 4) return fail(XQ_ERR_UNSUPPORTED, "q/dst elements must be contiguous");
    if (k->nb[0] != type_size(k->type) || v->nb[0] != type_size(v->type))
        return fail(XQ_ERR_UNSUPPORTED, "K/V records must be contiguous");
    const size_t rec = record_bytes(k->type, D);
    const size_t ch = kv_chunk(rec);
    for (int i = 1; i < 4; ++i)
        if (k->nb[i] % ch || v->nb[i] % ch)
            return fail(XQ_ERR_UNSUPPORTED, "K/V strides must be multiples of %zu bytes", ch);
    if (q->nb[1] % 4 || q->nb[2] % 4 || q->nb[3] % 4) return fail(XQ_ERR_UNSUPPORTED, "q strides");
    if (dst->nb[1] % 16 || dst->nb[2] % 16 || dst->nb[3] % 16)
        return fail(XQ_ERR_UNSUPPORTED, "dst strides must be multiples of 16 bytes");
    if (mask) {
        if (mask->type != XQ_TYPE_F16 || mask->nb[0] != 2) return fail(XQ_ERR_UNSUPPORTED, "mask must be contiguous F16");
        if (mask->ne[0] < k->ne[1] || mask->ne[1] < NQ) return fail(XQ_ERR_BAD_SHAPE, "mask smaller than [n_kv, n_q]");
        if (mask->ne[2] < 1 || mask->ne[3] < 1 || H % mask->ne[2] || B % mask->ne[3])
            return fail(XQ_ERR_BAD_SHAPE, "mask broadcast");
    }
    if (sinks) {
        if (sinks->type != XQ_TYPE_F32 || sinks->ne[0] != H || sinks->nb[0] != 4)
            return fail(XQ_ERR_UNSUPPORTED, "sinks must be contiguous F32 [n_head]");
    }
    if (!(p->scale == p->scale) || !(p->max_bias >= 0.0f) || !(p->logit_softcap >= 0.0f))
        return fail(XQ_ERR_BAD_ARG, "bad scale / max_bias / softcap");
    FaPlan P{};
    P.D = (int)D;
    P.NQ = (int)NQ;
    P.H = (int)H;
    P.B = (int)B;
    P.Hkv = (int)Hkv;
    P.G = (int)(H / Hkv);
    P.kt = k->type;
    P.L = k->ne[1];
    P.qk_mode = (k->type == XQ_TYPE_Q8_0 || k->type == XQ_TYPE_Q4_0) ? xq::kQkInt8 : xq::kQkFloat;
    P.q_round_f16 = (p->qk_policy == XQ_FA_QK_NATIVE && k->type == XQ_TYPE_F16) ? 1 : 0;
    split_policy(P.L, p->split_mode, B * Hkv, &P.n_splits, &P.split_rows);
    P.interleave = p->split_mode == XQ_FA_SPLIT_AUTO || p->split_mode == XQ_FA_SPLIT_LENGTH;
    if (P.n_splits > 256) return fail(XQ_ERR_UNSUPPORTED, "more than 256 KV splits");
    const int npairs = P.G * xq::fa_query_tile(P.D, P.G, P.NQ);
    if (!xq::fa_kernel_available(P.kt, P.D, P.qk_mode, npairs))
        return fail(XQ_ERR_UNSUPPORTED, "no kernel for this combination");
    if (p->engine == XQ_FA_ENGINE_MFMA && !xq::fa_mma_available(P.kt, P.D, P.qk_mode, npairs))
        return fail(XQ_ERR_UNSUPPORTED, "no matrix-core kernel for this combination");
    P.ws = xq::fa_workspace_bytes((int64_t)B * NQ * H, P.D, P.qk_mode, P.kt, P.n_splits) +
           xq::fa_mask_pack_bytes(mask, P.L, P.NQ);
    if (plan) *plan = P;
    return XQ_OK;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace

namespace xq {

xq_status set_error(xq_status st, const char* msg) {
    g_last_error = msg;
    return st;
}

}  // namespace xq

extern "C" {

int32_t xq_abi_version(void) { return XQ_ABI_VERSION; }

const char* xq_last_error(void) { return g_last_error.c_str(); }

// getenv value equal to want exactly (ggml's strict parse)
static bool env_is(const char* name, const char* want) {
    const char* v = getenv(name);
    return v && strcmp(v, want) == 0;
}

xq_status xq_fa_params_from_env(xq_fa_params* p) {
    if (!p) return fail(XQ_ERR_BAD_ARG, "params is null");
    if (env_is("GGML_FLASH_ATTN_NO_QUERY_TILING", "4"))
        p->qk_policy = XQ_FA_QK_CONSISTENT;
    else if (env_is("GGML_FLASH_ATTN_NO_QUERY_TILING", "1"))
        p->qk_policy = XQ_FA_QK_NATIVE;
    if (env_is("GGML_FLASH_ATTN_NO_SPLIT_KV", "1")) p->split_mode = XQ_FA_SPLIT_LENGTH;
    return ok();
}

int32_t xq_fa_split_count(int64_t kv_len, int32_t split_mode) {
    int32_t n;
    int64_t r;
    split_policy(kv_len, split_mode, 1, &n, &r);
    return n;
}

int64_t xq_fa_split_rows(int64_t kv_len, int32_t split_mode) {
    int32_t n;
    int64_t r;
    split_policy(kv_len, split_mode, 1, &n, &r);
    return r;
}

int xq_supports_flash_attn_ext(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                               const xq_tensor* mask, const xq_tensor* sinks,
                               const xq_tensor* dst, const xq_fa_params* params) {
    xq_fa_params dflt{};
    dflt.scale = 1.0f;
    return fa_check(q, k, v, mask, sinks, dst, params ? params : &dflt, nullptr) == XQ_OK;
}

xq_status xq_flash_attn_ext_workspace(const xq_tensor* q, const xq_tensor* k,
                                      const xq_tensor* v, const xq_tensor* mask,
                                      const xq_tensor* sinks, const xq_tensor* dst,
                                      const xq_fa_params* params, size_t* bytes) {
    if (!bytes) return fail(XQ_ERR_BAD_ARG, "bytes is null");
    FaPlan P;
    const xq_status st = fa_check(q, k, v, mask, sinks, dst, params, &P);
    if (st != XQ_OK) return st;
    *bytes = P.ws;
    return ok();
}

xq_status xq_flash_attn_ext(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                            const xq_tensor* mask, const xq_tensor* sinks, xq_tensor* dst,
                            float* lse, const xq_fa_params* params, void* workspace,
                            size_t workspace_bytes, void* stream) {
    FaPlan P;
    xq_status st = fa_check(q, k, v, mask, sinks, dst, params, &P);
    if (st != XQ_OK) return st;
    if (!q->data || !k->data || !v->data || !dst->data || (mask && !mask->data) || (sinks && !sinks->data))
        return fail(XQ_ERR_BAD_ARG, "null data pointer");
    const size_t ch = kv_chunk(record_bytes(k->type, P.D));
    if (!aligned(k->data, ch) || !aligned(v->data, ch) || !aligned(dst->data, 16) || !aligned(q->data, 4) ||
        (mask && !aligned(mask->data, 2)))
        return fail(XQ_ERR_UNSUPPORTED, "misaligned data pointer");
    if (!workspace || workspace_bytes < P.ws)
        return fail(XQ_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", P.ws, workspace_bytes);
    if (!aligned(workspace, 256)) return fail(XQ_ERR_WORKSPACE, "workspace must be 256-byte aligned");
    xq::FaLaunch L{};
    L.q = q;
    L.k = k;
    L.v = v;
    L.mask = mask;
    L.sinks = sinks;
    L.dst = dst;
    L.lse = lse;
    L.scale = params->scale;
    L.max_bias = params->max_bias;
    L.softcap = params->logit_softcap;
    L.qk_mode = P.qk_mode;
    L.q_round_f16 = P.q_round_f16;
    L.n_splits = P.n_splits;
    L.split_rows = P.split_rows;
    L.interleave = P.interleave;
    L.poison = 0;
    L.engine = params->engine;
    L.positions = nullptr;
    L.origin = 0;
    L.workspace = workspace;
    L.workspace_bytes = workspace_bytes;
    const hipError_t e = xq::fa_launch(L, (hipStream_t)stream);
    if (e != hipSuccess) return fail(XQ_ERR_HIP, "flash_attn_ext launch: %s", hipGetErrorString(e));
    return ok();
}

// The scratch array's address on the current device, looked up once per device
// (with that device current) and kept. The lookup enqueues no work, but it may
// load the library's code object onto the device: it runs with this thread's
// stream-capture mode relaxed, so a first call made while a caller captures a
// HIP graph (the callers this entry point is for) is legal and is not recorded.
static hipError_t scratch_address(void** out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(mu);
    if (!addr[dev]) {
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        e = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        const hipError_t e2 = hipThreadExchangeStreamCaptureMode(&mode);  // restore the caller's mode
        if (e != hipSuccess) return e;
        if (e2 != hipSuccess) return e2;
        addr[dev] = p;
    }
    *out = addr[dev];
    return hipSuccess;
}

xq_status xq_flash_attn_ext_noalloc(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                                    const xq_tensor* mask, const xq_tensor* sinks, xq_tensor* dst,
                                    float* lse, const xq_fa_params* params, void* stream) {
    FaPlan P;
    const xq_status st = fa_check(q, k, v, mask, sinks, dst, params, &P);
    if (st != XQ_OK) return st;
    if (P.ws > kScratchBytes)
        return fail(XQ_ERR_WORKSPACE,
                    "call needs %zu bytes of workspace; the no-alloc entry's scratch holds %zu bytes per GPU "
                    "(use xq_flash_attn_ext with a caller workspace)",
                    P.ws, kScratchBytes);
    void* ws = nullptr;
    const hipError_t e = scratch_address(&ws);
    if (e != hipSuccess) return fail(XQ_ERR_HIP, "scratch address: %s", hipGetErrorString(e));
    xq::NoAllocScope no_events;
    return xq_flash_attn_ext(q, k, v, mask, sinks, dst, lse, params, ws, kScratchBytes, stream);
}

// ------------------------------------------------------------ range attention

static void range_descs(int32_t n_q, int32_t n_head, int32_t n_head_kv, int32_t D, int32_t kv_type,
                        int32_t active, const void* q, const void* k, const void* v, void* out,
                        xq_tensor* tq, xq_tensor* tk, xq_tensor* tv, xq_tensor* td) {
    const size_t rec = record_bytes(kv_type, D);
    *tq = xq_tensor{XQ_TYPE_F32, 0, {D, n_q, n_head, 1},
                    {4, (size_t)n_head * D * 4, (size_t)D * 4, (size_t)n_q * n_head * D * 4}, (void*)q};
    *tk = xq_tensor{kv_type, 0, {D, active, n_head_kv, 1},
                    {type_size(kv_type), (size_t)n_head_kv * rec, rec, (size_t)(active > 0 ? active : 1) * n_head_kv * rec},
                    (void*)k};
    *tv = *tk;
    tv->data = (void*)v;
    *td = xq_tensor{XQ_TYPE_F32, 0, {D, n_head, n_q, 1},
                    {4, (size_t)D * 4, (size_t)n_head * D * 4, (size_t)n_q * n_head * D * 4}, out};
}

xq_status xq_fa_lse_merge(const float* parts_out, const float* parts_lse, int32_t n_parts,
                          int64_t rows, int32_t head_dim, float* out, float* lse, void* stream) {
    if (!parts_out || !parts_lse || !out || !lse) return fail(XQ_ERR_BAD_ARG, "null pointer");
    if (n_parts < 1 || rows < 1 || head_dim < 1) return fail(XQ_ERR_BAD_ARG, "bad merge sizes");
    if (head_dim > 512) return fail(XQ_ERR_UNSUPPORTED, "head dim above 512");
    if (rows > 0x7fffffff) return fail(XQ_ERR_UNSUPPORTED, "more than 2^31 rows");
    for (const void* p : {(const void*)parts_out, (const void*)parts_lse, (const void*)out, (const void*)lse})
        if (!aligned(p, 4)) return fail(XQ_ERR_UNSUPPORTED, "misaligned pointer");
    const hipError_t e =
        xq::fa_lse_merge_launch(parts_out, parts_lse, n_parts, rows, head_dim, out, lse, (hipStream_t)stream);
    if (e != hipSuccess) return fail(XQ_ERR_HIP, "fa_lse_merge launch: %s", hipGetErrorString(e));
    return ok();
}

xq_status xq_fa_range_workspace(int32_t n_q, int32_t n_head, int32_t n_head_kv, int32_t head_dim,
                                int32_t kv_type, int32_t active, int32_t split_mode, size_t* bytes) {
    if (!bytes || n_q < 1 || n_head < 1 || n_head_kv < 1 || active < 0)
        return fail(XQ_ERR_BAD_ARG, "bad range arguments");
    xq_tensor tq, tk, tv, td;
    range_descs(n_q, n_head, n_head_kv, head_dim, kv_type, active, nullptr, nullptr, nullptr, nullptr,
                &tq, &tk, &tv, &td);
    xq_fa_params p{};
    p.scale = 1.0f;
    p.split_mode = split_mode;
    FaPlan P;
    const xq_status st = fa_check(&tq, &tk, &tv, nullptr, nullptr, &td, &p, &P);
    if (st != XQ_OK) return st;
    *bytes = xq::fa_workspace_bytes((int64_t)n_q * n_head, head_dim, xq::kQkFloat, kv_type, P.n_splits);
    return ok();
}

xq_status xq_fa_range(const float* q, const int32_t* positions, int32_t n_q, int32_t n_head,
                      const void* k, const void* v, int32_t n_head_kv, int32_t head_dim,
                      int32_t kv_type, int32_t origin, int32_t active, float kq_scale,
                      int32_t split_mode, float* out, float* lse, void* workspace,
                      size_t workspace_bytes, void* stream) {
    if (!q || !positions || !k || !v || !out || !lse) return fail(XQ_ERR_BAD_ARG, "null pointer");
    if (n_q < 1 || n_head < 1 || n_head_kv < 1 || active < 0) return fail(XQ_ERR_BAD_ARG, "bad range arguments");
    xq_tensor tq, tk, tv, td;
    range_descs(n_q, n_head, n_head_kv, head_dim, kv_type, active, q, k, v, out, &tq, &tk, &tv, &td);
    xq_fa_params p{};
    p.scale = kq_scale;
    p.split_mode = split_mode;
    FaPlan P;
    xq_status st = fa_check(&tq, &tk, &tv, nullptr, nullptr, &td, &p, &P);
    if (st != XQ_OK) return st;
    const size_t need = xq::fa_workspace_bytes((int64_t)n_q * n_head, head_dim, xq::kQkFloat, kv_type, P.n_splits);
    if (!workspace || workspace_bytes < need)
        return fail(XQ_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    const size_t ch = kv_chunk(record_bytes(kv_type, head_dim));
    if (!aligned(k, ch) || !aligned(v, ch) || !aligned(out, 16) || !aligned(workspace, 256))
        return fail(XQ_ERR_UNSUPPORTED, "misaligned pointer");
    xq::FaLaunch L{};
    L.q = &tq;
    L.k = &tk;
    L.v = &tv;
    L.dst = &td;
    L.lse = lse;
    L.scale = kq_scale;
    L.qk_mode = xq::kQkFloat;  // f32 Q against the decoded K (shaders/rkva/rkva_range_attn.hlsl:74-78)
    L.n_splits = P.n_splits;
    L.split_rows = P.split_rows;
    L.poison = 1;
    L.engine = XQ_FA_ENGINE_AUTO;
    L.positions = positions;
    L.origin = origin;
    L.workspace = workspace;
    L.workspace_bytes = workspace_bytes;
    const hipError_t e = xq::fa_launch(L, (hipStream_t)stream);
    if (e != hipSuccess) return fail(XQ_ERR_HIP, "fa_range launch: %s", hipGetErrorString(e));
    return ok();
}

// ------------------------------------------------------------ gated delta net

static xq_status gdn_check(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                           const xq_tensor* g, const xq_tensor* beta, const xq_tensor* state,
                           const xq_tensor* dst, int32_t slots, int32_t raw_gates) {
    if (!q || !k || !v || !g || !beta || !state || !dst) return fail(XQ_ERR_BAD_ARG, "null tensor");
    if (raw_gates != 0) return fail(XQ_ERR_UNSUPPORTED, "raw gates (op_params[1] != 0) not supported");
    if (slots < 1 || slots > 17) return fail(XQ_ERR_UNSUPPORTED, "slots must be in [1, 17]");
    const int qt = q->type;
    if ((qt != XQ_TYPE_F32 && qt != XQ_TYPE_BF16) || k->type != qt || v->type != qt)
        return fail(XQ_ERR_UNSUPPORTED, "q/k/v must share type F32 or BF16");
    if (g->type != XQ_TYPE_F32 || beta->type != XQ_TYPE_F32 || state->type != XQ_TYPE_F32 || dst->type != XQ_TYPE_F32)
        return fail(XQ_ERR_UNSUPPORTED, "g/beta/state/dst must be F32");
    const int64_t T = v->ne[2], B = v->ne[3];
    if (T < 1 || B < 1) return fail(XQ_ERR_BAD_SHAPE, "T and B must be >= 1");
    for (const xq_tensor* t : {q, k})
        if (t->ne[0] != 128 || t->ne[1] != 16 || t->ne[2] != T || t->ne[3] != B)
            return fail(XQ_ERR_UNSUPPORTED, "q/k must be [128, 16, T, B]");
    if (v->ne[0] != 128 || v->ne[1] != 32) return fail(XQ_ERR_UNSUPPORTED, "v must be [128, 32, T, B]");
    const size_t es = qt == XQ_TYPE_F32 ? 4 : 2;
    for (const xq_tensor* t : {q, k, v}) {
        if (t->nb[0] != es) return fail(XQ_ERR_UNSUPPORTED, "q/k/v rows must be contiguous");
        for (int j = 1; j < 4; ++j)
            if (t->nb[j] % es) return fail(XQ_ERR_UNSUPPORTED, "q/k/v strides must be element-aligned");
    }
    for (const xq_tensor* t : {g, beta}) {
        if (t->ne[0] != 1 || t->ne[1] != 32 || t->ne[2] != T || t->ne[3] != B)
            return fail(XQ_ERR_UNSUPPORTED, "g/beta must be [1, 32, T, B] (scalar gates)");
        if (t->nb[0] != 4 || t->nb[1] != 4 || t->nb[2] != 128 || t->nb[3] != (size_t)128 * T)
            return fail(XQ_ERR_UNSUPPORTED, "g/beta must be contiguous");
    }
    if (state->ne[0] != 128 || state->ne[1] != 128 || state->ne[2] != 32 || state->ne[3] != B)
        return fail(XQ_ERR_UNSUPPORTED, "state must be [128, 128, 32, B]");
    if (state->nb[0] != 4 || state->nb[1] != 512 || state->nb[2] != 65536 || state->nb[3] != (size_t)65536 * 32)
        return fail(XQ_ERR_UNSUPPORTED, "state must be contiguous");
    if (dst->ne[0] != 4096 || dst->ne[1] != T + (int64_t)slots * 128 || dst->ne[2] != B || dst->ne[3] != 1)
        return fail(XQ_ERR_UNSUPPORTED, "dst must be [4096, T + slots*128, B, 1]");
    if (dst->nb[0] != 4 || dst->nb[1] != 16384 || dst->nb[2] != (size_t)16384 * dst->ne[1])
        return fail(XQ_ERR_UNSUPPORTED, "dst must be contiguous");
    return XQ_OK;
}

int xq_supports_gated_delta_net(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                                const xq_tensor* g, const xq_tensor* beta,
                                const xq_tensor* state, const xq_tensor* dst, int32_t slots,
                                int32_t raw_gates) {
    return gdn_check(q, k, v, g, beta, state, dst, slots, raw_gates) == XQ_OK;
}

static int gdn_pick(int32_t mode, int64_t T) {
    if (mode == XQ_GDN_STEP) return XQ_GDN_STEP;
    if (mode == XQ_GDN_CHUNKED) return XQ_GDN_CHUNKED;
    return (T <= 64 || !xq::gdn_chunked_available()) ? XQ_GDN_STEP : XQ_GDN_CHUNKED;
}

xq_status xq_gated_delta_net_workspace(const xq_tensor* q, const xq_tensor* v, int32_t slots,
                                       int32_t mode, size_t* bytes) {
    if (!q || !v || !bytes) return fail(XQ_ERR_BAD_ARG, "null argument");
    if (mode < XQ_GDN_AUTO || mode > XQ_GDN_CHUNKED) return fail(XQ_ERR_BAD_ARG, "bad mode");
    const int64_t T = v->ne[2], B = v->ne[3];
    *bytes = gdn_pick(mode, T) == XQ_GDN_CHUNKED
                 ? xq::gdn_chunked_workspace_bytes(T, B, slots, q->type == XQ_TYPE_BF16)
                 : 0;
    return ok();
}

xq_status xq_gated_delta_net(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                             const xq_tensor* g, const xq_tensor* beta, const xq_tensor* state,
                             xq_tensor* dst, int32_t slots, int32_t raw_gates, int32_t mode,
                             void* workspace, size_t workspace_bytes, void* stream) {
    xq_status st = gdn_check(q, k, v, g, beta, state, dst, slots, raw_gates);
    if (st != XQ_OK) return st;
    if (mode < XQ_GDN_AUTO || mode > XQ_GDN_CHUNKED) return fail(XQ_ERR_BAD_ARG, "bad mode");
    if (mode == XQ_GDN_CHUNKED && !xq::gdn_chunked_available())
        return fail(XQ_ERR_UNSUPPORTED, "chunked mode not available in this library");
    for (const xq_tensor* t : {q, k, v, g, beta, state, (const xq_tensor*)dst})
        if (!t->data) return fail(XQ_ERR_BAD_ARG, "null data pointer");
    if (!aligned(state->data, 16) || !aligned(dst->data, 16))
        return fail(XQ_ERR_UNSUPPORTED, "state/dst must be 16-byte aligned");
    xq::GdnLaunch L{q, k, v, g, beta, state, dst, slots, workspace, workspace_bytes};
    const int64_t T = v->ne[2], B = v->ne[3];
    hipError_t e;
    if (gdn_pick(mode, T) == XQ_GDN_CHUNKED) {
        const size_t need = xq::gdn_chunked_workspace_bytes(T, B, slots, q->type == XQ_TYPE_BF16);
        if (need && (!workspace || workspace_bytes < need))
            return fail(XQ_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        e = xq::gdn_chunked_launch(L, (hipStream_t)stream);
    } else {
        e = xq::gdn_step_launch(L, (hipStream_t)stream);
    }
    if (e != hipSuccess) return fail(XQ_ERR_HIP, "gated_delta_net launch: %s", hipGetErrorString(e));
    return ok();
}

// ------------------------------------------------------------ KV append

size_t xq_kv_record_bytes(int32_t kv_type, int32_t head_dim) {
    if (head_dim < 32 || head_dim % 32) return 0;
    if (kv_type != XQ_TYPE_F32 && kv_type != XQ_TYPE_BF16 && !kv_type_ok(kv_type)) return 0;
    return record_bytes(kv_type, head_dim);
}

xq_status xq_kv_store(const float* src, const int32_t* positions, int32_t n_tokens,
                      int32_t n_head_kv, int32_t head_dim, int32_t kv_type, int32_t q8_variant,
                      void* dst, int32_t capacity, void* stream) {
    if (!src || !positions || !dst) return fail(XQ_ERR_BAD_ARG, "null pointer");
    if (n_tokens < 0 || n_head_kv < 1 || capacity < 0) return fail(XQ_ERR_BAD_ARG, "bad sizes");
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return fail(XQ_ERR_UNSUPPORTED, "head_dim must be 64, 128 or 256");
    if (!xq_kv_record_bytes(kv_type, head_dim)) return fail(XQ_ERR_UNSUPPORTED, "kv_type %d", kv_type);
    if (q8_variant != 0 && q8_variant != 1) return fail(XQ_ERR_BAD_ARG, "q8_variant must be 0 or 1");
    const hipError_t e = xq::kv_store_launch(src, positions, n_tokens, n_head_kv, head_dim, kv_type,
                                             q8_variant, dst, capacity, (hipStream_t)stream);
    if (e != hipSuccess) return fail(XQ_ERR_HIP, "kv_store launch: %s", hipGetErrorString(e));
    return ok();
}

}  // extern "C"
