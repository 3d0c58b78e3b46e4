// xq_kernels.h — internal launch interface between the C-ABI layer (xq_api.hip)
// and the gfx950 kernels. Shapes arrive here already validated.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "xq_attn.h"
#include "xq_device.h"

namespace xq {

// Sets the calling thread's xq_last_error message and returns st.
xq_status set_error(xq_status st, const char* msg);

// Per-kernel device timing. While profiling is enabled (and the stream is not
// being captured into a graph), launch() hands the kernel a start/stop HIP
// event pair that the dispatch itself records at the kernel's first wave and
// at its completion (hipExtLaunchKernelGGL), so the elapsed time is the
// kernel's own execution interval, without the host's launch latency.
bool prof_events(hipStream_t stream, hipEvent_t* start, hipEvent_t* stop);
void prof_commit(const char* name, hipEvent_t start, hipEvent_t stop);

// While one is alive on a thread, launches on that thread record no timing
// events (the no-allocation entry point creates no HIP objects).
struct NoAllocScope {
    NoAllocScope();
    ~NoAllocScope();
};

template <typename F, typename... Args>
inline void launch(const char* name, F kernel, dim3 grid, dim3 block, hipStream_t stream, Args... args) {
    hipEvent_t start, stop;
    if (prof_events(stream, &start, &stop)) {
        hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0, args...);
        prof_commit(name, start, stop);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
    }
}

// ---------------------------------------------------------------- storage

constexpr int kQK = 32;  // elements per q8_0 / q4_0 block

constexpr int rec_bytes(int kt, int d) {
    return kt == XQ_TYPE_F16 ? 2 * d
         : kt == XQ_TYPE_Q8_0 ? d / kQK * 34
         : kt == XQ_TYPE_Q4_0 ? d / kQK * 18
         : kt == XQ_TYPE_E5M2 ? d
         : kt == XQ_TYPE_F32 ? 4 * d
         : 0;
}

// ---------------------------------------------------------------- flash attn

// Score mode: float image (f32 Q, or Q rounded to f16) against decoded K, or
// q8_0 image against quantized K with integer block dots.
enum QkMode { kQkFloat = 0, kQkInt8 = 1 };

// 32-bit words of one Q image row (one query x head).
constexpr int qimg_words(int qkm, int kt, int d) {
    return qkm == kQkFloat ? d
         : kt == XQ_TYPE_Q8_0 ? (d / 64) * 17 + d / kQK         // pair images + d_q
         : (d / 64) * 18 + 2 * (d / kQK);                        // lo/hi images + d_q + sum_q
}

// (query, head) pairs of a query tile: 32, except 16 at head dim 256 when the
// GQA group fits in 16. Every tile of a head-dim-256 call then runs the same
// 16-pair kernel variant (one wave count, one slice-to-wave assignment), so a
// query's bits do not depend on how many queries share the call.
constexpr int fa_max_pairs(int d, int g) { return d == 256 && g <= 16 ? 16 : 32; }
// Queries per tile for a call with n_q queries and GQA group g.
constexpr int fa_query_tile(int d, int g, int n_q) {
    return g >= fa_max_pairs(d, g) ? 1 : (fa_max_pairs(d, g) / g < n_q ? fa_max_pairs(d, g) / g : n_q);
}

struct FaLaunch {
    const xq_tensor* q;
    const xq_tensor* k;
    const xq_tensor* v;
    const xq_tensor* mask;   // may be null
    const xq_tensor* sinks;  // may be null
    const xq_tensor* dst;
    float* lse;              // may be null
    float scale, max_bias, softcap;
    int qk_mode;             // QkMode
    int q_round_f16;         // float image rounded to f16 (NATIVE policy, F16 K)
    int n_splits;
    int64_t split_rows;
    // matrix-core engine, no positions: the splits take the 16 x 8-row slice
    // groups in turn instead of split_rows contiguous rows each
    int interleave;
    int poison;              // reduce poisons non-finite partial states
    int engine;              // xq_fa_engine
    // range mode (positions != null): row r visible to query i iff
    // r < min(active, positions[i] - origin + 1); kv_len == active.
    const int32_t* positions;
    int32_t origin;
    void* workspace;
    size_t workspace_bytes;
};

size_t fa_workspace_bytes(int64_t n_rows, int d, int qk_mode, int kt, int n_splits);
hipError_t fa_lse_merge_launch(const float* parts_out, const float* parts_lse, int n_parts, int64_t rows, int d,
                               float* out, float* lse, hipStream_t stream);
// Extra workspace after fa_workspace_bytes for a mask whose rows the
// matrix-core engine must re-lay (reserved whenever a mask is given).
size_t fa_mask_pack_bytes(const xq_tensor* mask, int64_t L, int n_q);
hipError_t fa_launch(const FaLaunch& L, hipStream_t stream);
// Whether a compiled kernel exists for this combination.
bool fa_kernel_available(int kt, int d, int qk_mode, int n_pairs);
bool fa_mma_available(int kt, int d, int qk_mode, int n_pairs);

// ---------------------------------------------------------------- gdn

struct GdnLaunch {
    const xq_tensor* q;
    const xq_tensor* k;
    const xq_tensor* v;
    const xq_tensor* g;
    const xq_tensor* beta;
    const xq_tensor* state;
    const xq_tensor* dst;
    int32_t slots;
    void* workspace;
    size_t workspace_bytes;
};

hipError_t gdn_step_launch(const GdnLaunch& L, hipStream_t stream);
// Chunked prefill: tokens [0, T - (slots - 1)) in 64-token chunks, the last
// slots - 1 tokens on the step kernel so each keeps its snapshot.
size_t gdn_chunked_workspace_bytes(int64_t T, int64_t B, int32_t slots, bool bf16_rows);
hipError_t gdn_chunked_launch(const GdnLaunch& L, hipStream_t stream);
bool gdn_chunked_available();

// ---------------------------------------------------------------- kv append

hipError_t kv_store_launch(const float* src, const int32_t* positions, int32_t n_tokens,
                           int32_t n_head_kv, int32_t head_dim, int32_t kv_type,
                           int32_t q8_variant, void* dst, int32_t capacity, hipStream_t stream);

}  // namespace xq
