// xq_ggml_backend.hip — the ggml-backend face of the library (include/xq_ggml_backend.h):
// a pure supports_op predicate over ggml node descriptors and a synchronous
// graph_compute that runs the flash-attention and gated-delta-net nodes of a
// graph, in graph order, on the backend's own stream through the C ABI of
// xq_attn.h. The backend object owns one grow-only device workspace: a graph
// allocates only when it needs more room than any graph before it.
#include <stdarg.h>
#include <stddef.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "xq_ggml_backend.h"
#include "xq_kernels.h"

// the node layout the bindings build (ctypes mirror in xqattn/__init__.py)
static_assert(sizeof(xq_tensor) == 80, "xq_tensor layout");
static_assert(sizeof(xq_ggml_backend_params) == 32, "xq_ggml_backend_params layout");
static_assert(offsetof(xq_ggml_node, dst) == 72 && offsetof(xq_ggml_node, src) == 152 &&
                  sizeof(xq_ggml_node) == 232,
              "xq_ggml_node layout");

struct xq_ggml_backend {
    int32_t device = 0;
    hipStream_t stream = nullptr;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    xq_ggml_backend_params params{};
    std::mutex mu;  // one graph at a time per backend (ggml_d3d12.cpp:1893)
};

namespace {

xq_status err(xq_status st, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
xq_status err(xq_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return xq::set_error(st, buf);
}

bool is_empty(const xq_tensor& t) {  // ggml_is_empty
    for (int i = 0; i < 4; ++i)
        if (t.ne[i] == 0) return true;
    return false;
}

float param_f32(const xq_ggml_node* n, int i) {
    float f;
    memcpy(&f, &n->op_params[i], sizeof(f));
    return f;
}

// ggml_flash_attn_ext's op_params (scale, max_bias, logit_softcap as float
// bits) with the backend-wide policy choices; the automatic split under the
// consistent query policy is the length-only partition (batch-invariant bits).
xq_fa_params fa_params_of(const xq_ggml_node* n, const xq_ggml_backend_params& bp) {
    xq_fa_params p{};
    p.scale = param_f32(n, 0);
    p.max_bias = param_f32(n, 1);
    p.logit_softcap = param_f32(n, 2);
    p.qk_policy = bp.fa_qk_policy;
    p.split_mode = bp.fa_split_mode == XQ_FA_SPLIT_AUTO && bp.fa_qk_policy == XQ_FA_QK_CONSISTENT
                       ? XQ_FA_SPLIT_LENGTH
                       : bp.fa_split_mode;
    p.engine = bp.fa_engine;
    return p;
}

bool srcs_absent_from(const xq_ggml_node* n, int first) {
    for (int i = first; i < XQ_GGML_MAX_SRC; ++i)
        if (n->src[i]) return false;
    return true;
}

bool fa_supported(const xq_ggml_node* n, const xq_ggml_backend_params& bp) {
    if (!n->src[0] || !n->src[1] || !n->src[2] || !srcs_absent_from(n, 5)) return false;
    const xq_fa_params p = fa_params_of(n, bp);
    return xq_supports_flash_attn_ext(n->src[0], n->src[1], n->src[2], n->src[3], n->src[4],
                                      &n->dst, &p) != 0;
}

// the reference's rule for min_tokens: 2 stays 2, anything else is 1
// (d3d12_set_gdn_enabled, ggml_d3d12.cpp:68-71)
int gdn_min_tokens_of(const xq_ggml_backend_params& bp) { return bp.gdn_min_tokens == 2 ? 2 : 1; }

// d3d12_gdn_supported's operand rules (ggml_d3d12.cpp:77-109): six sources,
// src[6..8] (the rows-indexed mode) absent, activated gates, 1..17 slots, and
// at least the backend's minimum token count (:89).
bool gdn_supported(const xq_ggml_node* n, const xq_ggml_backend_params& bp) {
    for (int i = 0; i < 6; ++i)
        if (!n->src[i]) return false;
    if (!srcs_absent_from(n, 6)) return false;
    if (n->src[2]->ne[2] < gdn_min_tokens_of(bp)) return false;
    return xq_supports_gated_delta_net(n->src[0], n->src[1], n->src[2], n->src[3], n->src[4],
                                       n->src[5], &n->dst, n->op_params[0],
                                       n->op_params[1]) != 0;
}

bool runs_work(const xq_ggml_node* n) {
    return (n->flags & XQ_GGML_FLAG_COMPUTE) && !is_empty(n->dst) && n->op != XQ_GGML_OP_NOOP;
}

const xq_ggml_backend_params kDefaults = {XQ_FA_QK_CONSISTENT, XQ_FA_SPLIT_AUTO, XQ_FA_ENGINE_AUTO,
                                          XQ_GDN_AUTO, 1, {0, 0, 0}};

// the one predicate the scheduler-facing supports_op and graph_compute share
bool node_supported(const xq_ggml_node* n, const xq_ggml_backend_params& bp) {
    switch (n->op) {
    case XQ_GGML_OP_NOOP: return true;
    case XQ_GGML_OP_FLASH_ATTN_EXT: return fa_supported(n, bp);
    case XQ_GGML_OP_GATED_DELTA_NET: return gdn_supported(n, bp);
    default: return false;
    }
}

bool params_ok(const xq_ggml_backend_params& bp) {
    return bp.fa_qk_policy >= XQ_FA_QK_CONSISTENT && bp.fa_qk_policy <= XQ_FA_QK_NATIVE &&
           bp.fa_split_mode >= XQ_FA_SPLIT_AUTO && bp.fa_split_mode <= XQ_FA_SPLIT_LENGTH &&
           bp.fa_engine >= XQ_FA_ENGINE_AUTO && bp.fa_engine <= XQ_FA_ENGINE_VALU &&
           bp.gdn_mode >= XQ_GDN_AUTO && bp.gdn_mode <= XQ_GDN_CHUNKED;
}

struct DeviceGuard {  // restores the caller's current device
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

}  // namespace

extern "C" {

xq_ggml_backend* xq_ggml_backend_init(int32_t device, const xq_ggml_backend_params* params) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) {
        err(XQ_ERR_HIP, "no HIP device %d (%d present)", device, count);
        return nullptr;
    }
    xq_ggml_backend_params bp = params ? *params : kDefaults;
    if (!params) {  // the defaults take the environment's ggml knobs, as ggml's op does
        xq_fa_params fp{};
        fp.qk_policy = bp.fa_qk_policy;
        fp.split_mode = bp.fa_split_mode;
        (void)xq_fa_params_from_env(&fp);
        bp.fa_qk_policy = fp.qk_policy;
        bp.fa_split_mode = fp.split_mode;
    }
    if (!params_ok(bp)) {
        err(XQ_ERR_BAD_ARG, "bad backend params");
        return nullptr;
    }
    DeviceGuard g(device);
    hipStream_t s = nullptr;
    const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) {
        err(XQ_ERR_HIP, "hipStreamCreateWithFlags: %s", hipGetErrorString(e));
        return nullptr;
    }
    xq_ggml_backend* be = new xq_ggml_backend;
    be->device = device;
    be->stream = s;
    be->params = bp;
    xq::set_error(XQ_OK, "");
    return be;
}

void xq_ggml_backend_free(xq_ggml_backend* be) {
    if (!be) return;
    {
        std::lock_guard<std::mutex> lock(be->mu);
        DeviceGuard g(be->device);
        (void)hipStreamSynchronize(be->stream);
        if (be->ws) (void)hipFree(be->ws);
        (void)hipStreamDestroy(be->stream);
    }
    delete be;
}

const char* xq_ggml_backend_name(const xq_ggml_backend*) { return "XQ-MI355X"; }

void* xq_ggml_backend_stream(const xq_ggml_backend* be) { return be ? (void*)be->stream : nullptr; }

size_t xq_ggml_backend_workspace_bytes(const xq_ggml_backend* be) { return be ? be->ws_bytes : 0; }

int xq_ggml_supports_op(const xq_ggml_node* n) { return n && node_supported(n, kDefaults) ? 1 : 0; }

int xq_ggml_supports_op_params(const xq_ggml_node* n, const xq_ggml_backend_params* params) {
    if (!n || (params && !params_ok(*params))) return 0;
    return node_supported(n, params ? *params : kDefaults) ? 1 : 0;
}

xq_status xq_ggml_graph_compute(xq_ggml_backend* be, const xq_ggml_node* nodes, int32_t n_nodes) {
    if (!be) return err(XQ_ERR_BAD_ARG, "backend is null");
    if (n_nodes < 0 || (n_nodes > 0 && !nodes)) return err(XQ_ERR_BAD_ARG, "bad node list");

    // collect: every compute node must pass the predicate before anything runs
    std::vector<int32_t> work;
    size_t need = 0;
    for (int32_t i = 0; i < n_nodes; ++i) {
        const xq_ggml_node* n = &nodes[i];
        if (!runs_work(n)) continue;
        size_t bytes = 0;
        if (n->op == XQ_GGML_OP_FLASH_ATTN_EXT) {
            if (!fa_supported(n, be->params))
                return err(XQ_ERR_UNSUPPORTED, "node %d: FLASH_ATTN_EXT outside the supported contract", i);
            const xq_fa_params p = fa_params_of(n, be->params);
            const xq_status st = xq_flash_attn_ext_workspace(n->src[0], n->src[1], n->src[2], n->src[3],
                                                             n->src[4], &n->dst, &p, &bytes);
            if (st != XQ_OK) return st;
        } else if (n->op == XQ_GGML_OP_GATED_DELTA_NET) {
            if (!gdn_supported(n, be->params))
                return err(XQ_ERR_UNSUPPORTED, "node %d: GATED_DELTA_NET outside the supported contract", i);
            const xq_status st = xq_gated_delta_net_workspace(n->src[0], n->src[2], n->op_params[0],
                                                              be->params.gdn_mode, &bytes);
            if (st != XQ_OK) return st;
        } else {
            return err(XQ_ERR_UNSUPPORTED, "node %d: op kind %d is not run by this backend", i, n->op);
        }
        if (bytes > need) need = bytes;
        work.push_back(i);
    }
    if (work.empty()) return xq::set_error(XQ_OK, "");

    std::lock_guard<std::mutex> lock(be->mu);
    DeviceGuard g(be->device);
    if (need > be->ws_bytes) {  // grow: the previous graph has completed (synchronous contract)
        if (be->ws) (void)hipFree(be->ws);
        be->ws = nullptr;
        be->ws_bytes = 0;
        const hipError_t e = hipMalloc(&be->ws, need);
        if (e != hipSuccess) return err(XQ_ERR_HIP, "workspace of %zu bytes: %s", need, hipGetErrorString(e));
        be->ws_bytes = need;
    }

    xq_status st = XQ_OK;
    for (const int32_t i : work) {
        const xq_ggml_node* n = &nodes[i];
        xq_tensor dst = n->dst;
        if (n->op == XQ_GGML_OP_FLASH_ATTN_EXT) {
            const xq_fa_params p = fa_params_of(n, be->params);
            st = xq_flash_attn_ext(n->src[0], n->src[1], n->src[2], n->src[3], n->src[4], &dst, nullptr,
                                   &p, be->ws, be->ws_bytes, be->stream);
        } else {
            st = xq_gated_delta_net(n->src[0], n->src[1], n->src[2], n->src[3], n->src[4], n->src[5],
                                    &dst, n->op_params[0], n->op_params[1], be->params.gdn_mode, be->ws,
                                    be->ws_bytes, be->stream);
        }
        if (st != XQ_OK) break;
    }
    // graph_compute returns after completion (the reference has no synchronize hook)
    const hipError_t e = hipStreamSynchronize(be->stream);
    if (st != XQ_OK) return st;
    if (e != hipSuccess) return err(XQ_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
    return xq::set_error(XQ_OK, "");
}

}  // extern "C"
