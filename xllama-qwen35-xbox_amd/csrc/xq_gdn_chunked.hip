// xq_gdn_chunked.hip — GATED_DELTA_NET chunked prefill on the gfx950 matrix cores.
//
// The recurrence of shaders/ggml_d3d12_gated_delta_net.hlsl:40-85, per v-head
// and value column c (state column s in R^128, k-head = v-head % 16):
//   s *= e^{g_t};  u_t = beta_t (v_t[c] - s . k_t);  s += k_t u_t;  y_t[c] = scale * s . q_t
// is computed 64 tokens at a time in the WY / UT form of the delta rule.
// With G_t = g_1 + ... + g_t inside the chunk (cumulative log-decay) and S_0
// the state entering the chunk (S[i][c], key dim i, value column c):
//   L[t][j] = beta_t e^{G_t - G_j} (k_t . k_j)  (j < t),   T = (I + L)^{-1} diag(beta)
//   U = W_v - W_k S_0,  W_v = T V,  W_k = T diag(e^G) K
//   Y = scale (diag(e^G) Q S_0 + P U),  P[t][j] = (q_t . k_j) e^{G_t - G_j}  (j <= t)
//   S_C = e^{G_C} S_0 + K^T diag(e^{G_C - G}) U
// which equals the token-by-token recurrence in exact arithmetic.
//
// Two kernels:
//   gdn_chunk_prep  one workgroup per (sequence, v-head, chunk), all chunks in
//                   parallel: K K^T and Q K^T on f16 MFMA (products of the
//                   f16-converted bf16/f32 inputs, f32 accumulation), the unit
//                   lower-triangular solve for T in f32, W_k, W_v on f16 MFMA
//                   with T split into f16 hi + lo parts, P with its decays;
//                   stores W_k, W_v, P (f16 hi + lo planes), Q and K^T (f16) and
//                   the decay vectors in the workspace;
//   gdn_chunk_scan  one workgroup per (sequence, v-head, 32-column block) runs
//                   the chunks in order with its 128 x 32 state block in
//                   registers (f32): U, Y and the next state on f16 MFMA, f32
//                   operands split into hi + lo (about 22 significant bits), so
//                   the result stays within f32-recurrence tolerances.
// MFMA operand layouts (v_mfma_f32_16x16x16_f16): A lane (m = l % 16,
// k = 4 (l / 16) .. +3), B lane (n = l % 16, same k), C lane (rows
// 4 (l / 16) + r, column l % 16). An output tile whose rows are the next
// product's contraction index is that product's B operand as it stands.
#include "xq_kernels.h"

namespace xq {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;
constexpr int kCols = 32;  // value columns per scan workgroup

// Workspace record of one (sequence, v-head, chunk), byte offsets.
constexpr int kRecWkHi = 0;                      // f16 [64][128]
constexpr int kRecWkLo = kRecWkHi + 64 * 128 * 2;
constexpr int kRecWvHi = kRecWkLo + 64 * 128 * 2;  // f16 [64][128]
constexpr int kRecWvLo = kRecWvHi + 64 * 128 * 2;
constexpr int kRecPHi = kRecWvLo + 64 * 128 * 2;   // f16 [64][64]
constexpr int kRecPLo = kRecPHi + 64 * 64 * 2;
constexpr int kRecQ = kRecPLo + 64 * 64 * 2;       // f16 [64][128]
constexpr int kRecKT = kRecQ + 64 * 128 * 2;       // f16 [128][64]
constexpr int kRecDec = kRecKT + 128 * 64 * 2;     // f32 eG[64], eGCG[64], eGC
constexpr int kRecBytes = kRecDec + 1024;

struct GdnChunkArgs {
    const uint8_t* q;
    const uint8_t* k;
    const uint8_t* v;
    const uint8_t* g;
    const uint8_t* beta;
    const float* state;
    float* dst;        // per-token outputs [T][4096] of sequence 0 (+ b * dst_nb2)
    float* state_out;  // final state [32][128][128] of sequence 0 (+ b * so_nb3)
    uint8_t* ws;
    int64_t q_nb1, q_nb2, q_nb3;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t v_nb1, v_nb2, v_nb3;
    int64_t g_nb1, g_nb2, g_nb3;
    int64_t b_nb1, b_nb2, b_nb3;
    int64_t s_nb3, dst_nb2, so_nb3;
    int32_t T;  // tokens processed here (multiple chunks, last one partial)
    int32_t n_chunks;
    float scale;
};

// x = hi + lo with hi = f16(x), lo = f16(x - hi)
XQ_DEV _Float16 f16_hi(float x) { return (_Float16)x; }
XQ_DEV _Float16 f16_lo(float x) { return (_Float16)(x - (float)(_Float16)x); }

template <bool BF16>
XQ_DEV float in_elem(const uint8_t* row, int i) {
    if constexpr (BF16)
        return bf16_bits_to_f32(((const uint16_t*)row)[i]);
    else
        return ((const float*)row)[i];
}

// ---------------------------------------------------------------- prep

template <bool BF16>
__global__ __launch_bounds__(256) void gdn_chunk_prep(GdnChunkArgs a) {
    constexpr int KP = 136;  // padded f16 row strides
    constexpr int TP = 72;
    constexpr int FP = 65;   // padded f32 row stride
    __shared__ __attribute__((aligned(16))) _Float16 sK[64 * KP];    // K [t][i]
    __shared__ __attribute__((aligned(16))) _Float16 sKT[128 * TP];  // K^T [i][t]
    __shared__ __attribute__((aligned(16))) _Float16 sQ[64 * KP];    // Q [t][i]
    __shared__ __attribute__((aligned(16))) _Float16 sVT[128 * TP];  // V^T [c][t]
    __shared__ float sKK[64 * FP];  // K K^T, then L
    __shared__ float sQK[64 * FP];  // Q K^T
    __shared__ float sT[64 * FP];   // T [t][j]
    __shared__ float sG[64], sBeta[64], sEG[64];

    const int n = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int kh = h % 16;
    const int tid = threadIdx.x;
    const int wave = wave_id(), lane = lane_id(), lr = lane & 15, lg = lane >> 4;
    const int t0 = n * kChunk;

    // ---- chunk rows -> LDS as f16 (tokens past T are zero, with g = beta = 0)
    {
        const int t = tid >> 2, qtr = tid & 3;  // 64 tokens x 4 quarters of 32 elements
        const int tg = t0 + t;
        const bool ok = tg < a.T;
        const uint8_t* kr = a.k + (int64_t)b * a.k_nb3 + (int64_t)tg * a.k_nb2 + (int64_t)kh * a.k_nb1;
        const uint8_t* qr = a.q + (int64_t)b * a.q_nb3 + (int64_t)tg * a.q_nb2 + (int64_t)kh * a.q_nb1;
        const uint8_t* vr = a.v + (int64_t)b * a.v_nb3 + (int64_t)tg * a.v_nb2 + (int64_t)h * a.v_nb1;
#pragma unroll 8
        for (int e = 0; e < 32; ++e) {
            const int i = qtr * 32 + e;
            const _Float16 kv = ok ? (_Float16)in_elem<BF16>(kr, i) : (_Float16)0.0f;
            const _Float16 qv = ok ? (_Float16)in_elem<BF16>(qr, i) : (_Float16)0.0f;
            const _Float16 vv = ok ? (_Float16)in_elem<BF16>(vr, i) : (_Float16)0.0f;
            sK[t * KP + i] = kv;
            sKT[i * TP + t] = kv;
            sQ[t * KP + i] = qv;
            sVT[i * TP + t] = vv;
        }
        if (tid < 64) {
            const int tt = t0 + tid;
            const bool ok2 = tt < a.T;
            sG[tid] = ok2 ? *(const float*)(a.g + (int64_t)b * a.g_nb3 + (int64_t)tt * a.g_nb2 + (int64_t)h * a.g_nb1) : 0.0f;
            sBeta[tid] = ok2 ? *(const float*)(a.beta + (int64_t)b * a.b_nb3 + (int64_t)tt * a.b_nb2 + (int64_t)h * a.b_nb1) : 0.0f;
        }
    }
    __syncthreads();
    // cumulative log-decay (sequential sum, as the recurrence applies the decays)
    if (tid < 64) {
        float G = 0.0f;
        for (int s = 0; s <= tid; ++s) G += sG[s];
        sEG[tid] = G;  // G for now, exponentiated below
    }
    // ---- K K^T and Q K^T: 16 tiles each, 4 per wave, contraction over 128 key dims
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        const int tile = wave * 4 + tt;
        const int mt = tile >> 2, nt = tile & 3;
        f4 kk = f4{0.0f, 0.0f, 0.0f, 0.0f}, qk = kk;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const h4 bk = *(const h4*)(sK + (nt * 16 + lr) * KP + ks * 16 + 4 * lg);
            const h4 ak = *(const h4*)(sK + (mt * 16 + lr) * KP + ks * 16 + 4 * lg);
            const h4 aq = *(const h4*)(sQ + (mt * 16 + lr) * KP + ks * 16 + 4 * lg);
            kk = __builtin_amdgcn_mfma_f32_16x16x16f16(ak, bk, kk, 0, 0, 0);
            qk = __builtin_amdgcn_mfma_f32_16x16x16f16(aq, bk, qk, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = mt * 16 + 4 * lg + r, col = nt * 16 + lr;
            sKK[row * FP + col] = kk[r];
            sQK[row * FP + col] = qk[r];
        }
    }
    __syncthreads();
    // ---- L (strictly lower, in place of K K^T); decays e^{G}
    for (int e = tid; e < 64 * 64; e += 256) {
        const int t = e >> 6, j = e & 63;
        const float L = j < t ? sBeta[t] * __expf(sEG[t] - sEG[j]) * sKK[t * FP + j] : 0.0f;
        sKK[t * FP + j] = L;
    }
    __syncthreads();
    // ---- T = (I + L)^{-1} diag(beta): column j by a quad of lanes; lane part p
    //      keeps x_s for s in [16p, 16p + 16) and the quad sums the dot products
    {
        const int j = wave * 16 + (lane >> 2), p = lane & 3;
        float x[16];
#pragma unroll
        for (int m = 0; m < 16; ++m) x[m] = 0.0f;
        const float bj = sBeta[j];
#pragma unroll
        for (int t = 0; t < 64; ++t) {
            float part = 0.0f;
            if (t > 0) {
                const float* Lr = sKK + t * FP + 16 * p;
#pragma unroll
                for (int m = 0; m < 16; ++m) part = fmaf(Lr[m], x[m], part);  // L[t][s >= t] = 0
            }
            part += dpp<0xB1>(part);  // quad: lanes p ^ 1
            part += dpp<0x4E>(part);  // quad: lanes p ^ 2
            const float xt = t < j ? 0.0f : (t == j ? bj : -part);
            if ((t >> 4) == p) x[t & 15] = xt;
        }
#pragma unroll
        for (int m = 0; m < 16; ++m) sT[(16 * p + m) * FP + j] = x[m];
    }
    if (tid < 64) {
        const float GC = sEG[63];
        const float G = sEG[tid];
        float* dec = (float*)(a.ws + (((int64_t)b * 32 + h) * a.n_chunks + n) * kRecBytes + kRecDec);
        dec[tid] = __expf(G);
        dec[64 + tid] = __expf(GC - G);
        if (tid == 0) dec[128] = __expf(GC);
    }
    __syncthreads();

    uint8_t* rec = a.ws + (((int64_t)b * 32 + h) * a.n_chunks + n) * kRecBytes;
    // ---- W_k = T diag(e^G) K and W_v = T V: 32 tiles each (64 x 128), 8 per wave
#pragma unroll 2
    for (int tt = 0; tt < 8; ++tt) {
        const int tile = wave * 8 + tt;
        const int mt = tile >> 3, nt = tile & 7;
        f4 wk = f4{0.0f, 0.0f, 0.0f, 0.0f}, wv = wk;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int j0 = ks * 16 + 4 * lg;
            h4 th, tl, tph, tpl;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float tv = sT[(mt * 16 + lr) * FP + j0 + e];
                th[e] = f16_hi(tv), tl[e] = f16_lo(tv);
                tph[e] = f16_hi(tv * __expf(sEG[j0 + e])), tpl[e] = f16_lo(tv * __expf(sEG[j0 + e]));
            }
            const h4 bk = *(const h4*)(sKT + (nt * 16 + lr) * TP + j0);
            const h4 bv = *(const h4*)(sVT + (nt * 16 + lr) * TP + j0);
            wk = __builtin_amdgcn_mfma_f32_16x16x16f16(tph, bk, wk, 0, 0, 0);
            wk = __builtin_amdgcn_mfma_f32_16x16x16f16(tpl, bk, wk, 0, 0, 0);
            wv = __builtin_amdgcn_mfma_f32_16x16x16f16(th, bv, wv, 0, 0, 0);
            wv = __builtin_amdgcn_mfma_f32_16x16x16f16(tl, bv, wv, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = mt * 16 + 4 * lg + r, col = nt * 16 + lr;
            _Float16 hi, lo;
            hi = f16_hi(wk[r]), lo = f16_lo(wk[r]);
            ((_Float16*)(rec + kRecWkHi))[row * 128 + col] = hi;
            ((_Float16*)(rec + kRecWkLo))[row * 128 + col] = lo;
            hi = f16_hi(wv[r]), lo = f16_lo(wv[r]);
            ((_Float16*)(rec + kRecWvHi))[row * 128 + col] = hi;
            ((_Float16*)(rec + kRecWvLo))[row * 128 + col] = lo;
        }
    }
    // ---- P (with the diagonal), Q and K^T copies
    for (int e = tid; e < 64 * 64; e += 256) {
        const int t = e >> 6, j = e & 63;
        const float pv = j <= t ? sQK[t * FP + j] * __expf(sEG[t] - sEG[j]) : 0.0f;
        _Float16 hi, lo;
        hi = f16_hi(pv), lo = f16_lo(pv);
        ((_Float16*)(rec + kRecPHi))[e] = hi;
        ((_Float16*)(rec + kRecPLo))[e] = lo;
    }
    for (int e = tid; e < 64 * 128; e += 256) {
        const int t = e >> 7, i = e & 127;
        ((_Float16*)(rec + kRecQ))[e] = sQ[t * KP + i];
        const int ii = e >> 6, tt = e & 63;
        ((_Float16*)(rec + kRecKT))[e] = sKT[ii * TP + tt];
    }
}

// ---------------------------------------------------------------- scan

__global__ __launch_bounds__(256) void gdn_chunk_scan(GdnChunkArgs a) {
    constexpr int SP = 136;  // S^T row stride (halves): [c][i]
    constexpr int UP = 72;   // U^T row stride: [c][t]
    __shared__ __attribute__((aligned(16))) _Float16 sSh[kCols * SP], sSl[kCols * SP];
    __shared__ __attribute__((aligned(16))) _Float16 sUh[kCols * UP], sUl[kCols * UP];
    __shared__ __attribute__((aligned(16))) _Float16 sVh[kCols * UP], sVl[kCols * UP];  // U' = e^{G_C - G} U

    const int cb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int wave = wave_id(), lane = lane_id(), lr = lane & 15, lg = lane >> 4;
    const float* st = a.state + (int64_t)b * (a.s_nb3 / 4) + (int64_t)h * 16384;

    // state tiles owned by this wave: key-dim tiles 2w, 2w + 1, column tiles 0, 1;
    // lane holds S[i = 16 it + 4 lg + r][c = 32 cb + 16 ct + lr]
    f4 S[2][2];
#pragma unroll
    for (int a2 = 0; a2 < 2; ++a2)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int it = 2 * wave + a2;
            const int c = kCols * cb + 16 * ct + lr;
            const float4 v = *(const float4*)(st + (int64_t)c * 128 + 16 * it + 4 * lg);
            S[a2][ct] = f4{v.x, v.y, v.z, v.w};
        }
    float* out = a.dst + (int64_t)b * (a.dst_nb2 / 4);

    for (int n = 0; n < a.n_chunks; ++n) {
        const uint8_t* rec = a.ws + (((int64_t)b * 32 + h) * a.n_chunks + n) * kRecBytes;
        const _Float16* Wkh = (const _Float16*)(rec + kRecWkHi);
        const _Float16* Wkl = (const _Float16*)(rec + kRecWkLo);
        const _Float16* Wvh = (const _Float16*)(rec + kRecWvHi);
        const _Float16* Wvl = (const _Float16*)(rec + kRecWvLo);
        const _Float16* Ph = (const _Float16*)(rec + kRecPHi);
        const _Float16* Pl = (const _Float16*)(rec + kRecPLo);
        const _Float16* Qh = (const _Float16*)(rec + kRecQ);
        const _Float16* KT = (const _Float16*)(rec + kRecKT);
        const float* dec = (const float*)(rec + kRecDec);

        // ---- S (hi, lo) -> LDS as S^T [c][i]: B operand rows
#pragma unroll
        for (int a2 = 0; a2 < 2; ++a2)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const int it = 2 * wave + a2;
                h4 hi, lo;
#pragma unroll
                for (int r = 0; r < 4; ++r) hi[r] = f16_hi(S[a2][ct][r]), lo[r] = f16_lo(S[a2][ct][r]);
                *(h4*)(sSh + (16 * ct + lr) * SP + 16 * it + 4 * lg) = hi;
                *(h4*)(sSl + (16 * ct + lr) * SP + 16 * it + 4 * lg) = lo;
            }
        __syncthreads();

        // ---- U = W_v - W_k S and Q S for token tile w (16 tokens), both column tiles
        f4 U[2], QS[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            f4 acc = f4{0.0f, 0.0f, 0.0f, 0.0f}, accq = acc;
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const int arow = (16 * wave + lr) * 128 + 16 * ks + 4 * lg;
                const h4 ah = *(const h4*)(Wkh + arow), al = *(const h4*)(Wkl + arow), aq = *(const h4*)(Qh + arow);
                const h4 bh = *(const h4*)(sSh + (16 * ct + lr) * SP + 16 * ks + 4 * lg);
                const h4 bl = *(const h4*)(sSl + (16 * ct + lr) * SP + 16 * ks + 4 * lg);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bh, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bl, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bh, acc, 0, 0, 0);
                accq = __builtin_amdgcn_mfma_f32_16x16x16f16(aq, bh, accq, 0, 0, 0);
                accq = __builtin_amdgcn_mfma_f32_16x16x16f16(aq, bl, accq, 0, 0, 0);
            }
            QS[ct] = accq;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * wave + 4 * lg + r, c = kCols * cb + 16 * ct + lr;
                U[ct][r] = ((float)Wvh[t * 128 + c] + (float)Wvl[t * 128 + c]) - acc[r];
            }
            // U and U' = e^{G_C - G_t} U (hi, lo) -> LDS as U^T [c][t]
            h4 uh, ul, vh, vl;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * wave + 4 * lg + r;
                uh[r] = f16_hi(U[ct][r]), ul[r] = f16_lo(U[ct][r]);
                vh[r] = f16_hi(U[ct][r] * dec[64 + t]), vl[r] = f16_lo(U[ct][r] * dec[64 + t]);
            }
            const int o = (16 * ct + lr) * UP + 16 * wave + 4 * lg;
            *(h4*)(sUh + o) = uh;
            *(h4*)(sUl + o) = ul;
            *(h4*)(sVh + o) = vh;
            *(h4*)(sVl + o) = vl;
        }
        __syncthreads();

        // ---- Y = scale (diag(e^G) Q S + P U) for token tile w
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            f4 acc;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] = QS[ct][r] * dec[16 * wave + 4 * lg + r];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int arow = (16 * wave + lr) * 64 + 16 * ks + 4 * lg;
                const h4 ah = *(const h4*)(Ph + arow), al = *(const h4*)(Pl + arow);
                const int bo = (16 * ct + lr) * UP + 16 * ks + 4 * lg;
                const h4 bh = *(const h4*)(sUh + bo), bl = *(const h4*)(sUl + bo);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bh, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bl, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bh, acc, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = n * kChunk + 16 * wave + 4 * lg + r;
                if (t < a.T) out[(int64_t)t * 4096 + h * 128 + kCols * cb + 16 * ct + lr] = acc[r] * a.scale;
            }
        }

        // ---- S = e^{G_C} S + K^T U' for this wave's state tiles
        const float eGC = dec[128];
#pragma unroll
        for (int a2 = 0; a2 < 2; ++a2) {
            const int it = 2 * wave + a2;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                f4 acc = S[a2][ct] * eGC;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const h4 ak = *(const h4*)(KT + (16 * it + lr) * 64 + 16 * ks + 4 * lg);
                    const int bo = (16 * ct + lr) * UP + 16 * ks + 4 * lg;
                    const h4 bh = *(const h4*)(sVh + bo), bl = *(const h4*)(sVl + bo);
                    acc = __builtin_amdgcn_mfma_f32_16x16x16f16(ak, bh, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x16f16(ak, bl, acc, 0, 0, 0);
                }
                S[a2][ct] = acc;
            }
        }
    }

    // ---- final state (transposed layout: element (i, c) of head h at h*16384 + c*128 + i)
    float* so = a.state_out + (int64_t)b * (a.so_nb3 / 4) + (int64_t)h * 16384;
#pragma unroll
    for (int a2 = 0; a2 < 2; ++a2)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int it = 2 * wave + a2;
            const int c = kCols * cb + 16 * ct + lr;
            *(float4*)(so + (int64_t)c * 128 + 16 * it + 4 * lg) =
                make_float4(S[a2][ct][0], S[a2][ct][1], S[a2][ct][2], S[a2][ct][3]);
        }
}

// ---------------------------------------------------------------- host

static int64_t chunked_tokens(int64_t T, int32_t slots) { return slots > 1 ? T - (slots - 1) : T; }

size_t gdn_chunked_workspace_bytes(int64_t T, int64_t B, int32_t slots) {
    const int64_t Tc = chunked_tokens(T, slots);
    if (Tc < 1) return 0;
    const int64_t nch = (Tc + kChunk - 1) / kChunk;
    return (size_t)B * 32 * nch * kRecBytes;
}

bool gdn_chunked_available() { return true; }

hipError_t gdn_chunked_launch(const GdnLaunch& L, hipStream_t stream) {
    const int64_t T = L.v->ne[2], B = L.v->ne[3];
    const int64_t Tc = chunked_tokens(T, L.slots);
    if (Tc < 1) return gdn_step_launch(L, stream);  // every token needs its own snapshot
    if (L.workspace_bytes < gdn_chunked_workspace_bytes(T, B, L.slots)) return hipErrorInvalidValue;
    GdnChunkArgs a{};
    a.q = (const uint8_t*)L.q->data;
    a.k = (const uint8_t*)L.k->data;
    a.v = (const uint8_t*)L.v->data;
    a.g = (const uint8_t*)L.g->data;
    a.beta = (const uint8_t*)L.beta->data;
    a.state = (const float*)L.state->data;
    a.dst = (float*)L.dst->data;
    a.ws = (uint8_t*)L.workspace;
    a.q_nb1 = L.q->nb[1]; a.q_nb2 = L.q->nb[2]; a.q_nb3 = L.q->nb[3];
    a.k_nb1 = L.k->nb[1]; a.k_nb2 = L.k->nb[2]; a.k_nb3 = L.k->nb[3];
    a.v_nb1 = L.v->nb[1]; a.v_nb2 = L.v->nb[2]; a.v_nb3 = L.v->nb[3];
    a.g_nb1 = L.g->nb[1]; a.g_nb2 = L.g->nb[2]; a.g_nb3 = L.g->nb[3];
    a.b_nb1 = L.beta->nb[1]; a.b_nb2 = L.beta->nb[2]; a.b_nb3 = L.beta->nb[3];
    a.s_nb3 = L.state->nb[3];
    a.dst_nb2 = L.dst->nb[2];
    // the chunked part's final state is the snapshot slot (slots - 1): slot j holds
    // the state j tokens before the end (slot 0, the final state, when slots == 1)
    a.state_out = (float*)((uint8_t*)L.dst->data + (T + 128 * (int64_t)(L.slots - 1)) * 16384);
    a.so_nb3 = L.dst->nb[2];
    a.T = (int32_t)Tc;
    a.n_chunks = (int32_t)((Tc + kChunk - 1) / kChunk);
    a.scale = 1.0f / sqrtf(128.0f);
    const bool bf16 = L.q->type == XQ_TYPE_BF16;
    {
        ProfScope ps("gdn_chunk_prep", stream);
        if (bf16)
            hipLaunchKernelGGL(gdn_chunk_prep<true>, dim3(a.n_chunks, 32, (uint32_t)B), dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL(gdn_chunk_prep<false>, dim3(a.n_chunks, 32, (uint32_t)B), dim3(256), 0, stream, a);
    }
    {
        ProfScope ps("gdn_chunk_scan", stream);
        hipLaunchKernelGGL(gdn_chunk_scan, dim3(128 / kCols, 32, (uint32_t)B), dim3(256), 0, stream, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || L.slots == 1) return e;
    // the last slots - 1 tokens run on the step kernel, starting from the chunked
    // part's final state, writing their outputs and the remaining snapshots
    xq_tensor q = *L.q, k = *L.k, v = *L.v, g = *L.g, be = *L.beta, s = *L.state, d = *L.dst;
    for (xq_tensor* t : {&q, &k, &v, &g, &be}) {
        t->data = (uint8_t*)t->data + Tc * t->nb[2];
        t->ne[2] = T - Tc;
    }
    s.data = a.state_out;
    s.nb[3] = L.dst->nb[2];
    d.data = (uint8_t*)L.dst->data + Tc * 16384;
    d.ne[1] = (T - Tc) + 128 * (L.slots - 1);
    GdnLaunch tail = L;
    tail.q = &q; tail.k = &k; tail.v = &v; tail.g = &g; tail.beta = &be; tail.state = &s; tail.dst = &d;
    tail.slots = L.slots - 1;
    return gdn_step_launch(tail, stream);
}

}  // namespace xq
