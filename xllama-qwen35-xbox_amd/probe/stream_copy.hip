// stream_copy.hip — HBM ceiling probe for the benchmark (not part of the
// library's ABI): a streaming device copy with the gated-delta-net step
// kernel's launch shape (256-thread workgroups, up to 24 16-byte non-temporal
// loads per thread issued before their stores), so the step's time can be set
// against a plain copy of the same bytes on the same GPU.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMaxPer = 24;  // 16-byte words per thread (up to 96 KiB per workgroup)

// 256 workgroups (one per CU, as the step kernel's 8 x 32), each copying a
// contiguous 1/256 of the words: every thread issues its loads, then its stores.
__global__ __launch_bounds__(kThreads) void stream_copy(const f4v* __restrict__ src, f4v* __restrict__ dst,
                                                        size_t n_words, size_t per_wg) {
    const size_t w0 = (size_t)blockIdx.x * per_wg;
    const size_t w1 = w0 + per_wg < n_words ? w0 + per_wg : n_words;
    f4v r[kMaxPer];
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const size_t w = w0 + (size_t)i * kThreads + threadIdx.x;
        r[i] = w < w1 ? __builtin_nontemporal_load(src + w) : f4v{};
    }
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const size_t w = w0 + (size_t)i * kThreads + threadIdx.x;
        if (w < w1) __builtin_nontemporal_store(r[i], dst + w);
    }
}

extern "C" {

// Copies `bytes` (a multiple of 16, at most 24 MiB; both pointers 16-byte
// aligned) from src to dst on `stream`. Returns 0 on success, 1 on a bad argument, 2 on a launch error.
int xqp_stream_copy(const void* src, void* dst, size_t bytes, void* stream) {
    if (!src || !dst || bytes % 16 || (uintptr_t)src % 16 || (uintptr_t)dst % 16) return 1;
    const size_t n_words = bytes / 16;
    if (n_words == 0) return 0;
    const size_t per_wg = (n_words + 255) / 256;
    if (per_wg > (size_t)kMaxPer * kThreads) return 1;  // above 256 x 96 KiB
    hipLaunchKernelGGL(stream_copy, dim3(256), dim3(kThreads), 0, (hipStream_t)stream, (const f4v*)src, (f4v*)dst,
                       n_words, per_wg);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
