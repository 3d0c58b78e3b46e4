/* xq_ggml_backend.h — the ggml-backend face of the MI355X attention +
 * gated-delta-net library: what a thin ggml_backend_i / ggml_backend_device_i
 * binding calls to place GGML_OP_FLASH_ATTN_EXT and GGML_OP_GATED_DELTA_NET
 * nodes of a llama.cpp graph on the GPU.
 *
 * It has the shape of the reference's D3D12 backend
 * (src/bridge/ggml_d3d12.cpp:1836-1942 graph_compute, :2268-2285 the backend
 * interface, :2331-2420 supports_op):
 *   - xq_ggml_supports_op is a pure predicate; the same predicate gates
 *     graph_compute's node collection, so a node the scheduler placed here is
 *     always one that runs (ggml_d3d12.cpp:1862-1866);
 *   - graph_compute walks the nodes in graph order, skips empty nodes, nodes
 *     without the compute flag and the view-like no-ops (NONE, RESHAPE, VIEW,
 *     PERMUTE, TRANSPOSE), runs the rest in order on the backend's stream and
 *     returns after the work has completed (the reference sets
 *     synchronize = nullptr for the same reason, ggml_d3d12.cpp:2277);
 *   - calls on one backend are serialized by a mutex (ggml_d3d12.cpp:1893).
 * Where the reference aborts on an unsupported node (GGML_ABORT,
 * ggml_d3d12.cpp:1886), graph_compute validates every node first and returns
 * XQ_ERR_UNSUPPORTED without launching anything.
 *
 * ggml's headers are not part of this library: the binding copies each node's
 * type / ne / nb / data / op_params / src into xq_ggml_node (with ggml's type
 * ids, which xq_tensor shares) and maps enum ggml_op onto enum xq_ggml_op. */
#ifndef XQ_GGML_BACKEND_H
#define XQ_GGML_BACKEND_H

#include "xq_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define XQ_GGML_MAX_SRC 10        /* GGML_MAX_SRC */
#define XQ_GGML_MAX_OP_PARAMS 16  /* GGML_MAX_OP_PARAMS / sizeof(int32_t) */
#define XQ_GGML_FLAG_COMPUTE 1    /* the node's GGML_TENSOR_FLAG_COMPUTE bit */

enum xq_ggml_op {
    XQ_GGML_OP_NOOP = 0,            /* GGML_OP_NONE / RESHAPE / VIEW / PERMUTE / TRANSPOSE */
    XQ_GGML_OP_FLASH_ATTN_EXT = 1,  /* GGML_OP_FLASH_ATTN_EXT */
    XQ_GGML_OP_GATED_DELTA_NET = 2, /* GGML_OP_GATED_DELTA_NET */
    XQ_GGML_OP_OTHER = 3,           /* any other ggml op: not supported here */
};

/* One ggml graph node, as the binding copies it out of a ggml_tensor.
 *   FLASH_ATTN_EXT: src = {q, k, v, mask|NULL, sinks|NULL};
 *     op_params[0..2] = scale, max_bias, logit_softcap as float bits
 *     (ggml_flash_attn_ext), op_params[3] = precision (ggml_flash_attn_ext_set_prec:
 *     accepted, the kernels accumulate in f32 whatever it asks).
 *   GATED_DELTA_NET: src = {q, k, v, g, beta, state}, src[6..9] NULL;
 *     op_params[0] = snapshot slots, op_params[1] = raw-gate flag (must be 0)
 *     (ggml_d3d12.cpp:77-83). */
typedef struct xq_ggml_node {
    int32_t op;    /* enum xq_ggml_op */
    int32_t flags; /* XQ_GGML_FLAG_COMPUTE when ggml marks the node for compute */
    int32_t op_params[XQ_GGML_MAX_OP_PARAMS];
    xq_tensor dst;                          /* the node tensor itself (device data) */
    const xq_tensor* src[XQ_GGML_MAX_SRC];  /* NULL where ggml's src[i] is NULL */
} xq_ggml_node;

/* Backend-wide choices. NULL = the defaults (the reference's consistent query
 * policy, the automatic split, engine and GDN modes, GDN from one token) with
 * the environment's ggml flash-attention knobs applied on top
 * (xq_fa_params_from_env: GGML_FLASH_ATTN_NO_QUERY_TILING,
 * GGML_FLASH_ATTN_NO_SPLIT_KV, read once at init).
 *   fa_split_mode: XQ_FA_SPLIT_AUTO under XQ_FA_QK_CONSISTENT runs
 *     XQ_FA_SPLIT_LENGTH, a partition by the KV length only, so a sequence's
 *     bits do not depend on the sequences batched with it, as ggml's CPU loop
 *     under the reference's consistent mode (flashattn.txt=2 sets
 *     GGML_FLASH_ATTN_NO_SPLIT_KV=1 with it, uwp/inference-bridge.cpp:887-893).
 *     Under XQ_FA_QK_NATIVE it is the batch-sized AUTO partition.
 *   gdn_min_tokens: the fewest tokens a GATED_DELTA_NET node needs to run
 *     here; 2 leaves single-token decode nodes to the CPU and runs T >= 2 on
 *     the GPU (the reference's hybrid d3d12_set_gdn_enabled(true, 2),
 *     src/bridge/ggml_d3d12.cpp:68-71,89, set by d3d12gdn.txt=2,
 *     uwp/inference-bridge.cpp:901-906); any other value means 1, as there. */
typedef struct xq_ggml_backend_params {
    int32_t fa_qk_policy;   /* enum xq_fa_qk_policy */
    int32_t fa_split_mode;  /* enum xq_fa_split_mode */
    int32_t fa_engine;      /* enum xq_fa_engine */
    int32_t gdn_mode;       /* enum xq_gdn_mode */
    int32_t gdn_min_tokens; /* 1 or 2 */
    int32_t reserved[3];
} xq_ggml_backend_params;

typedef struct xq_ggml_backend xq_ggml_backend;

/* dev_init_backend (ggml_d3d12.cpp:2318-2322): a backend on HIP device
 * `device` with its own stream (default priority) and a workspace that grows
 * to the largest node it has run. NULL on failure (xq_last_error says why). */
xq_ggml_backend* xq_ggml_backend_init(int32_t device, const xq_ggml_backend_params* params);
/* backend_free: waits for the stream, frees the workspace and the stream. */
void xq_ggml_backend_free(xq_ggml_backend* backend);
/* get_name: "XQ-MI355X". */
const char* xq_ggml_backend_name(const xq_ggml_backend* backend);
/* The backend's hipStream_t (for a binding that orders its buffer copies). */
void* xq_ggml_backend_stream(const xq_ggml_backend* backend);
/* Workspace bytes the backend holds now. */
size_t xq_ggml_backend_workspace_bytes(const xq_ggml_backend* backend);

/* dev_supports_op (ggml_d3d12.cpp:2331-2353): 1 when graph_compute runs the
 * node (no-op kinds included), 0 otherwise. Pure; needs no GPU.
 * xq_ggml_supports_op_params answers for a backend created with these params
 * (gdn_min_tokens, the FA policy fields; NULL = the defaults without the
 * environment): the predicate its graph_compute applies, as the reference's
 * supports_op reads the mode d3d12_set_gdn_enabled set
 * (ggml_d3d12.cpp:77-109). xq_ggml_supports_op(node) answers for the
 * defaults. */
int xq_ggml_supports_op(const xq_ggml_node* node);
int xq_ggml_supports_op_params(const xq_ggml_node* node, const xq_ggml_backend_params* params);

/* graph_compute (ggml_d3d12.cpp:1836-1942): runs nodes[0 .. n_nodes) in order
 * and returns once they have completed on the device. XQ_ERR_UNSUPPORTED
 * (nothing launched) when a compute node fails xq_ggml_supports_op. */
xq_status xq_ggml_graph_compute(xq_ggml_backend* backend, const xq_ggml_node* nodes,
                                int32_t n_nodes);

#ifdef __cplusplus
}
#endif

#endif /* XQ_GGML_BACKEND_H */
