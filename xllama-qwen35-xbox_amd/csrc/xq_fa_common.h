// xq_fa_common.h — definitions shared by the two flash-attention pass-1
// engines (VALU in xq_fa.hip, matrix cores in xq_fa_mma.hip) and the split
// reduce: launch arguments, the sinks/normalisation tail, helpers.
#pragma once

#include <math.h>

#include "xq_kernels.h"

namespace xq {

constexpr int kTile = 64;
constexpr int kThreads = 256;
constexpr int kMaxSplits = 256;

// LDS record stride: a multiple of 16 bytes with an odd number of 16-byte
// units, so 16 lanes reading 16 bytes from consecutive records hit distinct
// bank groups.
constexpr int pad_rec(int rec) {
    int u = (rec + 15) / 16;
    if ((u & 1) == 0) ++u;
    return u * 16;
}
constexpr int chunk_bytes(int rec) { return rec % 16 == 0 ? 16 : rec % 8 == 0 ? 8 : 4; }

template <int CH> struct ChunkT;
template <> struct ChunkT<16> { using T = uint4; };
template <> struct ChunkT<8> { using T = uint2; };
template <> struct ChunkT<4> { using T = uint32_t; };

struct FaArgs {
    const uint8_t* k;
    const uint8_t* v;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t v_nb1, v_nb2, v_nb3;
    const uint8_t* mask;
    int64_t m_nb1, m_nb2, m_nb3;
    int32_t m_ne2, m_ne3;
    const int32_t* positions;
    int32_t origin;
    const float* sinks;
    uint8_t* dst;
    int64_t d_nb1, d_nb2, d_nb3;
    float* lse;
    float* part_o;
    float2* part_ml;
    int64_t L;
    int64_t split_rows;
    int32_t interleave;  // fa_dec: split s takes the slice groups s, s + n_splits, ...
    int32_t H, Hkv, G, NQ, B, QT, n_qtiles, n_splits, rk3, rv3;
    float scale, softcap, max_bias, m0, m1;
    int32_t n_head_log2;
    int32_t poison;
    // matrix-core engine: f32 Q rows (quantised inside the kernel), hi-only
    // f16 Q for the NATIVE policy
    const uint8_t* q;
    int64_t q_nb1, q_nb2, q_nb3;
    int32_t hi_only;
};

XQ_DEV float alibi_slope(const FaArgs& a, int h) {
    if (!(a.max_bias > 0.0f)) return 1.0f;
    return h < a.n_head_log2 ? powf(a.m0, (float)(h + 1))
                             : powf(a.m1, (float)(2 * (h - a.n_head_log2) + 1));
}

// Sinks and 1/S exactly as ggml's tail of the one-chunk loop: a sink above the
// running maximum rescales the accumulator by exp(M - sink) and adds 1 to S,
// otherwise S += exp(sink - M); then out = acc * (S == 0 ? 0 : 1/S).
XQ_DEV void fa_finalize(float M, float S, bool has_sink, float sink, float& a1, float& inv,
                        float& lse) {
    a1 = 1.0f;
    float meff = M;
    if (has_sink) {
        if (sink > M) {
            const float ms = expf(M - sink);
            a1 = ms;
            S = fmaf(S, ms, 1.0f);
            meff = sink;
        } else {
            S = S + expf(sink - M);
        }
    }
    inv = S == 0.0f ? 0.0f : 1.0f / S;
    lse = S > 0.0f ? meff + logf(S) : -INFINITY;
}

// e^x through the hardware base-2 exponential (v_exp_f32, 1 ulp) on x*log2(e);
// exact 0 for x = -inf. Used for the online-softmax weights (arguments <= 0).
XQ_DEV float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

XQ_DEV uint32_t lds_u32(const uint8_t* p) { return *(const uint32_t*)p; }
XQ_DEV uint32_t lds_u16(const uint8_t* p) { return *(const uint16_t*)p; }


struct FaLaunch;
hipError_t fa_mma_launch(FaArgs a, const FaLaunch& L, hipStream_t stream);
// Mask layout the matrix-core engine can read (4-byte aligned rows).
bool fa_mma_mask_ok(const FaArgs& a);
// Separate split-merge kernel (used when the merge cannot run inside pass 1).
hipError_t fa_reduce_launch(const FaArgs& a, int d, hipStream_t stream);

}  // namespace xq
