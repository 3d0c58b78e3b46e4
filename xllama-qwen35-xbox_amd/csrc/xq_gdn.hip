// xq_gdn.hip — GATED_DELTA_NET on gfx950: the token-sequential step kernel.
//
// Work of shaders/ggml_d3d12_gated_delta_net.hlsl:40-85 (one group per
// (v-head, 8 value columns), 8 lanes x 16 registers per column) re-laid for
// wave64 and HBM: a 16-lane DPP row owns one state column (128 f32 = 512 B),
// each lane holds 8 elements as two float4 at i = 4*li + 64*r (r = 0, 1), so a
// row's state read/write is two fully coalesced 256-byte transactions. Both
// column dot products reduce inside the DPP row (4 steps, no LDS, no barrier).
// A 256-thread workgroup covers 16 columns of one (sequence, v-head); tokens
// run chronologically with the state in registers, so the state is read once
// and each kept snapshot written once.
#include "xq_kernels.h"

namespace xq {

struct GdnStepArgs {
    const uint8_t* q;
    const uint8_t* k;
    const uint8_t* v;
    const uint8_t* g;
    const uint8_t* beta;
    const float* state;
    float* dst;
    int64_t q_nb1, q_nb2, q_nb3;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t v_nb1, v_nb2, v_nb3;
    int64_t g_nb1, g_nb2, g_nb3;
    int64_t b_nb1, b_nb2, b_nb3;
    int64_t s_nb3;    // state bytes per sequence
    int64_t dst_nb2;  // dst bytes per sequence
    int32_t T;
    int32_t slots;
    int32_t B;
    float scale;
};

template <bool BF16>
XQ_DEV float ld_elem(const uint8_t* p, int i) {
    if constexpr (BF16)
        return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    else
        return ((const float*)p)[i];
}

constexpr int kGdnColsPerWg = 16;

template <bool BF16>
__global__ __launch_bounds__(256) void gdn_step_kernel(GdnStepArgs a) {
    const int n_wg = a.B * 32 * (128 / kGdnColsPerWg);
    const int wg = (int)xcd_remap(blockIdx.x, (uint32_t)n_wg);
    const int cblk = wg % (128 / kGdnColsPerWg);
    const int bh = wg / (128 / kGdnColsPerWg);
    const int b = bh / 32, h = bh % 32, kh = h % 16;
    const int lane = lane_id();
    const int li = lane & 15;
    const int col = cblk * kGdnColsPerWg + (int)(threadIdx.x >> 4);

    const float* s_in = (const float*)((const char*)a.state + (int64_t)b * a.s_nb3) +
                        ((int64_t)h * 128 + col) * 128;
    float4 s0 = *(const float4*)(s_in + 4 * li);
    float4 s1 = *(const float4*)(s_in + 64 + 4 * li);

    float* out = (float*)((char*)a.dst + (int64_t)b * a.dst_nb2);
    const int64_t s_off = (int64_t)4096 * a.T;

    for (int t = 0; t < a.T; ++t) {
        const uint8_t* qp = a.q + (int64_t)b * a.q_nb3 + (int64_t)t * a.q_nb2 + (int64_t)kh * a.q_nb1;
        const uint8_t* kp = a.k + (int64_t)b * a.k_nb3 + (int64_t)t * a.k_nb2 + (int64_t)kh * a.k_nb1;
        float qv[8], kv[8];
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                qv[4 * r + j] = ld_elem<BF16>(qp, 64 * r + 4 * li + j);
                kv[4 * r + j] = ld_elem<BF16>(kp, 64 * r + 4 * li + j);
            }
        const float gt = *(const float*)(a.g + (int64_t)b * a.g_nb3 + (int64_t)t * a.g_nb2 + (int64_t)h * a.g_nb1);
        const float bt = *(const float*)(a.beta + (int64_t)b * a.b_nb3 + (int64_t)t * a.b_nb2 + (int64_t)h * a.b_nb1);
        const float vt = ld_elem<BF16>(a.v + (int64_t)b * a.v_nb3 + (int64_t)t * a.v_nb2 + (int64_t)h * a.v_nb1, col);
        const float decay = expf(gt);

        float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        float part = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            s[e] = s[e] * decay;
            part = fmaf(s[e], kv[e], part);
        }
        const float dot_sk = row16_sum(part);
        const float delta = (vt - dot_sk) * bt;
        float att = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            s[e] = fmaf(kv[e], delta, s[e]);
            att = fmaf(s[e], qv[e], att);
        }
        const float y = row16_sum(att);
        if (li == 0) out[((int64_t)t * 32 + h) * 128 + col] = y * a.scale;
        s0 = make_float4(s[0], s[1], s[2], s[3]);
        s1 = make_float4(s[4], s[5], s[6], s[7]);

        const int slot = a.T - 1 - t;
        if ((a.slots > 1 && slot < a.slots) || (a.slots == 1 && t + 1 == a.T)) {
            float* snap = out + s_off + (int64_t)(a.slots == 1 ? 0 : slot) * 524288 +
                          ((int64_t)h * 128 + col) * 128;
            *(float4*)(snap + 4 * li) = s0;
            *(float4*)(snap + 64 + 4 * li) = s1;
        }
    }
}

hipError_t gdn_step_launch(const GdnLaunch& L, hipStream_t stream) {
    GdnStepArgs a;
    a.q = (const uint8_t*)L.q->data;
    a.k = (const uint8_t*)L.k->data;
    a.v = (const uint8_t*)L.v->data;
    a.g = (const uint8_t*)L.g->data;
    a.beta = (const uint8_t*)L.beta->data;
    a.state = (const float*)L.state->data;
    a.dst = (float*)L.dst->data;
    a.q_nb1 = L.q->nb[1]; a.q_nb2 = L.q->nb[2]; a.q_nb3 = L.q->nb[3];
    a.k_nb1 = L.k->nb[1]; a.k_nb2 = L.k->nb[2]; a.k_nb3 = L.k->nb[3];
    a.v_nb1 = L.v->nb[1]; a.v_nb2 = L.v->nb[2]; a.v_nb3 = L.v->nb[3];
    a.g_nb1 = L.g->nb[1]; a.g_nb2 = L.g->nb[2]; a.g_nb3 = L.g->nb[3];
    a.b_nb1 = L.beta->nb[1]; a.b_nb2 = L.beta->nb[2]; a.b_nb3 = L.beta->nb[3];
    a.s_nb3 = L.state->nb[3];
    a.dst_nb2 = L.dst->nb[2];
    a.T = (int32_t)L.v->ne[2];
    a.B = (int32_t)L.v->ne[3];
    a.slots = L.slots;
    a.scale = 1.0f / sqrtf(128.0f);
    const int n_wg = a.B * 32 * (128 / kGdnColsPerWg);
    ProfScope ps("gdn_step", stream);
    if (L.q->type == XQ_TYPE_BF16)
        hipLaunchKernelGGL(gdn_step_kernel<true>, dim3(n_wg), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(gdn_step_kernel<false>, dim3(n_wg), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace xq

namespace xq {

// The chunked (WY/UT, bf16 MFMA) prefill lives in xq_gdn_chunked.hip once
// built; until then CHUNKED mode is reported as unsupported.
size_t gdn_chunked_workspace_bytes(int64_t, int64_t) { return 0; }
hipError_t gdn_chunked_launch(const GdnLaunch&, hipStream_t) { return hipErrorNotSupported; }
bool gdn_chunked_available() { return false; }

}  // namespace xq
