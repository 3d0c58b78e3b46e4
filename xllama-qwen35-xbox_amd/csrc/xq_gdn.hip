// xq_gdn.hip — GATED_DELTA_NET on gfx950: the token-sequential step kernel.
//
// Work of shaders/ggml_d3d12_gated_delta_net.hlsl:40-85 (one group per
// (v-head, 8 value columns), 8 lanes x 16 registers per column) re-laid for
// wave64 and HBM: a 16-lane DPP row owns one state column (128 f32 = 512 B),
// each lane holds 8 elements as two float4 at i = 4*li + 64*r (r = 0, 1), so a
// row's state read/write is two fully coalesced 256-byte transactions. Both
// column dot products reduce inside the DPP row (4 steps, no LDS, no barrier).
// A 256-thread workgroup covers 128 columns of one (sequence, v-head); tokens
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

typedef float f4v __attribute__((ext_vector_type(4)));

// State columns are read once and written once per call: they stream past
// the caches with non-temporal accesses (measured 7.1 us against 8.2 us per
// call with ordinary loads and stores at 8 sequences x 32 heads).
XQ_DEV float4 ld_state(const float* p) {
    const f4v v = __builtin_nontemporal_load((const f4v*)p);
    return make_float4(v[0], v[1], v[2], v[3]);
}
XQ_DEV void st_state(float* p, float4 x) { __builtin_nontemporal_store(f4v{x.x, x.y, x.z, x.w}, (f4v*)p); }

template <bool BF16>
XQ_DEV float ld_elem(const uint8_t* p, int i) {
    if constexpr (BF16)
        return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    else
        return ((const float*)p)[i];
}

// Eight elements i = 64*r + 4*li + j (r, j in 0..1, 0..3) of a q/k row.
template <bool BF16, bool VEC>
XQ_DEV void ld_row8(const uint8_t* p, int li, float (&x)[8]) {
    if constexpr (VEC && !BF16) {
        const float4 a = *(const float4*)(p + 16 * li);
        const float4 b = *(const float4*)(p + 256 + 16 * li);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else if constexpr (VEC && BF16) {
        const uint2 a = *(const uint2*)(p + 8 * li);
        const uint2 b = *(const uint2*)(p + 128 + 8 * li);
        const uint32_t w[4] = {a.x, a.y, b.x, b.y};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = bf16_bits_to_f32(w[e] & 0xffffu);
            x[2 * e + 1] = bf16_bits_to_f32(w[e] >> 16);
        }
    } else {
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j) x[4 * r + j] = ld_elem<BF16>(p, 64 * r + 4 * li + j);
    }
}

// Inputs of one token as one row of a workgroup needs them.
template <int CPT>
struct StepIn {
    float q[8], k[8], v[CPT], g, beta;
};

template <bool BF16, bool VEC, int CPT>
XQ_DEV void load_token(const GdnStepArgs& a, int b, int h, int kh, int li, int col0, int t, StepIn<CPT>& in) {
    ld_row8<BF16, VEC>(a.q + (int64_t)b * a.q_nb3 + (int64_t)t * a.q_nb2 + (int64_t)kh * a.q_nb1, li, in.q);
    ld_row8<BF16, VEC>(a.k + (int64_t)b * a.k_nb3 + (int64_t)t * a.k_nb2 + (int64_t)kh * a.k_nb1, li, in.k);
    const uint8_t* vrow = a.v + (int64_t)b * a.v_nb3 + (int64_t)t * a.v_nb2 + (int64_t)h * a.v_nb1;
#pragma unroll
    for (int j = 0; j < CPT; ++j) in.v[j] = ld_elem<BF16>(vrow, col0 + 16 * j);
    in.g = *(const float*)(a.g + (int64_t)b * a.g_nb3 + (int64_t)t * a.g_nb2 + (int64_t)h * a.g_nb1);
    in.beta = *(const float*)(a.beta + (int64_t)b * a.b_nb3 + (int64_t)t * a.b_nb2 + (int64_t)h * a.b_nb1);
}

// One token through CPT state columns of a row (column c_j = col0 + 16*j):
// decay, delta rule, output, and the snapshot when the token keeps one. A
// single token (ONE) always keeps its state, in slot 0.
template <int CPT, bool ONE>
XQ_DEV void step_token(const GdnStepArgs& a, const StepIn<CPT>& in, float4 (&s0)[CPT], float4 (&s1)[CPT],
                       float* out, int h, int li, int col0, int t) {
    const float decay = expf(in.g);
    const int slot = a.T - 1 - t;
    const bool keep = ONE || (a.slots > 1 && slot < a.slots) || (a.slots == 1 && t + 1 == a.T);
    const int64_t s_off = (int64_t)4096 * a.T;
    const int64_t slot_off = ONE || a.slots == 1 ? 0 : (int64_t)slot * 524288;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int col = col0 + 16 * j;
        float s[8] = {s0[j].x, s0[j].y, s0[j].z, s0[j].w, s1[j].x, s1[j].y, s1[j].z, s1[j].w};
        float part = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            s[e] = s[e] * decay;
            part = fmaf(s[e], in.k[e], part);
        }
        const float dot_sk = row16_sum(part);
        const float delta = (in.v[j] - dot_sk) * in.beta;
        float att = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            s[e] = fmaf(in.k[e], delta, s[e]);
            att = fmaf(s[e], in.q[e], att);
        }
        const float y = row16_sum(att);
        if (li == 0) out[((int64_t)t * 32 + h) * 128 + col] = y * a.scale;
        s0[j] = make_float4(s[0], s[1], s[2], s[3]);
        s1[j] = make_float4(s[4], s[5], s[6], s[7]);
        if (keep) {
            float* snap = out + s_off + slot_off + ((int64_t)h * 128 + col) * 128;
            st_state(snap + 4 * li, s0[j]);
            st_state(snap + 64 + 4 * li, s1[j]);
        }
    }
}

// CPT state columns per 16-lane row. The state loads are all issued at the
// start. ONE (a single token, the decode step) has no prefetch; otherwise each
// token's inputs are loaded while the previous token computes, into two
// alternating buffers, so that every load is issued ahead of the previous
// token's stores (on gfx9 a wait for a load also waits for the stores issued
// before it).
template <bool BF16, bool VEC, int CPT, bool ONE>
__global__ __launch_bounds__(256) void gdn_step_kernel(GdnStepArgs a) {
    constexpr int COLS = 16 * CPT;  // columns per workgroup
    const int n_wg = a.B * 32 * (128 / COLS);
    const int wg = (int)xcd_remap(blockIdx.x, (uint32_t)n_wg);
    const int cblk = wg % (128 / COLS);
    const int bh = wg / (128 / COLS);
    const int b = bh / 32, h = bh % 32, kh = h % 16;
    const int li = threadIdx.x & 15;
    const int col0 = cblk * COLS + (int)(threadIdx.x >> 4);

    // the state first, in column order, then the first token's inputs
    // (6.51-6.55 us per call at 8 sequences, against 6.55-6.59 us with the
    // inputs first); column j computes and stores as soon as its own state
    // has arrived
    const float* s_in = (const float*)((const char*)a.state + (int64_t)b * a.s_nb3) + (int64_t)h * 16384;
    float4 s0[CPT], s1[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const float* sc = s_in + (int64_t)(col0 + 16 * j) * 128;
        s0[j] = ld_state(sc + 4 * li);
        s1[j] = ld_state(sc + 64 + 4 * li);
    }
    StepIn<CPT> ia;
    load_token<BF16, VEC, CPT>(a, b, h, kh, li, col0, 0, ia);
    float* out = (float*)((char*)a.dst + (int64_t)b * a.dst_nb2);
    if constexpr (ONE) {
        step_token<CPT, true>(a, ia, s0, s1, out, h, li, col0, 0);
    } else {
        StepIn<CPT> ib;
        for (int t = 0; t < a.T; t += 2) {
            if (t + 1 < a.T) load_token<BF16, VEC, CPT>(a, b, h, kh, li, col0, t + 1, ib);
            step_token<CPT, false>(a, ia, s0, s1, out, h, li, col0, t);
            if (t + 1 >= a.T) break;
            if (t + 2 < a.T) load_token<BF16, VEC, CPT>(a, b, h, kh, li, col0, t + 2, ia);
            step_token<CPT, false>(a, ib, s0, s1, out, h, li, col0, t + 1);
        }
    }
}

// Eight columns per row: one 256-thread workgroup owns all 128 columns (64 KB
// of state) of one (sequence, v-head), so the whole state read is in flight at
// once; with 8 sequences x 32 heads that is one workgroup per CU. Measured
// against one, two and four columns per row at 8 sequences x 32 heads, eight
// was fastest (6.5 us per call against 7.1 us for four).
constexpr int kStepCpt = 8;

template <bool BF16, bool VEC>
static void step_dispatch(const GdnStepArgs& a, hipStream_t stream) {
    const dim3 grid(a.B * 32 * (128 / (16 * kStepCpt)));
    if (a.T == 1)
        launch("gdn_step", gdn_step_kernel<BF16, VEC, kStepCpt, true>, grid, dim3(256), stream, a);
    else
        launch("gdn_step", gdn_step_kernel<BF16, VEC, kStepCpt, false>, grid, dim3(256), stream, a);
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
    const bool bf16 = L.q->type == XQ_TYPE_BF16;
    const size_t al = bf16 ? 8 : 16;  // q/k rows read as 16- (f32) or 8-byte (bf16) vectors
    bool vec = true;
    for (const xq_tensor* t : {L.q, L.k}) {
        vec = vec && ((uintptr_t)t->data % al == 0);
        for (int i = 1; i < 4; ++i) vec = vec && (t->nb[i] % al == 0);
    }
    if (bf16) {
        if (vec) step_dispatch<true, true>(a, stream);
        else step_dispatch<true, false>(a, stream);
    } else {
        if (vec) step_dispatch<false, true>(a, stream);
        else step_dispatch<false, false>(a, stream);
    }
    return hipGetLastError();
}

}  // namespace xq

