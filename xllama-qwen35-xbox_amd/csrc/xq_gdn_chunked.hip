// xq_gdn_chunked.hip — GATED_DELTA_NET chunked prefill on the gfx950 matrix cores.
//
// The recurrence of shaders/ggml_d3d12_gated_delta_net.hlsl:40-85, per v-head
// and value column c (state column s in R^128, k-head = v-head % 16):
//   s *= e^{g_t};  u_t = beta_t (v_t[c] - s . k_t);  s += k_t u_t;  y_t[c] = scale * s . q_t
// is computed 64 tokens at a time in the UT form of the delta rule. With
// G_t = g_1 + ... + g_t inside the chunk (cumulative log-decay), S the state
// entering the chunk (S[i][c], key dim i, value column c), K, Q, V the chunk's
// rows and
//   L[t][j] = beta_t e^{G_t - G_j} (k_t . k_j)  (j < t),   T = (I + L)^{-1} diag(beta)
//   P[t][j] = (q_t . k_j) e^{G_t - G_j}  (j <= t)
// the chunk is
//   U  = T (V - diag(e^G) K S)
//   Y  = scale (diag(e^G) Q S + P U)
//   S' = e^{G_C} S + K^T diag(e^{G_C - G}) U
// which equals the token-by-token recurrence in exact arithmetic.
//
// Two kernels:
//   gdn_chunk_prep  one workgroup per (sequence, k-head, chunk), all chunks in
//                   parallel, for the two v-heads that share the k-head: K K^T on
//                   f16 MFMA once (f32 accumulation) and, per v-head, the unit
//                   lower-triangular inverse for T in f32 (by 16 x 16 blocks,
//                   the products on f32 MFMA); stores T as f16 hi + lo
//                   planes, the decay vectors, the cumulative log-decays G,
//                   the chunk's largest |v| per 16-column block and, for bf16
//                   rows read as 16-byte words, the P tiles (f16 hi + lo; 27 KB
//                   per chunk) in the workspace. f32 k rows enter as f16 hi + lo
//                   (the products take hi*hi + hi*lo + lo*hi); bf16 rows enter
//                   as f16 (their 8 significant bits fit; a bf16 value below
//                   2^-14 keeps an absolute precision of 2^-25 there, not its
//                   relative one), or as bf16 on bf16 MFMA when read as
//                   16-byte words (exact).
//   gdn_chunk_scan  one workgroup per (sequence, v-head, 16 value columns) runs
//                   the chunks in order with its 128 x 16 state block in
//                   registers (f32). Every MFMA operand that does not depend on
//                   the state (K and Q rows straight from the inputs, as f16,
//                   or f16 hi + lo for f32 rows; T rows from the workspace; V,
//                   the decays and G) is loaded into registers a chunk ahead,
//                   in four parts spread over the chunk's phases. K^T is formed
//                   in the scan from the K rows it already holds (the waves
//                   share them through LDS: written transposed, or for bf16
//                   rows read as 16-byte words written as loaded and read
//                   with gfx950's transposing LDS read), which keeps 16 KB per
//                   chunk out of every workgroup's operand fetch. P is formed
//                   by the prep for bf16 rows read as 16-byte words (10 KB per
//                   chunk, off the scan's chain; its products and decays are
//                   the scan's own), and by the scan from its K and Q rows
//                   (shared through LDS) otherwise. LDS otherwise
//                   carries the state-dependent exchanges (S^T, X^T, U^T). The products run
//                   on f16 MFMA with f32 operands split into f16 hi + lo (about
//                   22 significant bits), so the result stays within
//                   f32-recurrence tolerances. bf16 rows read as 16-byte words
//                   skip the f16 conversion: they are the operands of bf16
//                   MFMAs as loaded, and the f32 operands that meet them (the
//                   state, e^{G_C - G} U) enter as three bf16 terms hi + mid + lo,
//                   which hold the f32 value exactly; 30 % fewer VALU
//                   instructions and 6 % less time per scan than the f16 form.
// The 8 column blocks of a head run on one XCD (consecutive logical workgroups)
// so the chunk rows and T, P they share are read from HBM once.
//
// Range. The recurrence is linear in (V, S): the scan runs on V and S times a
// power of two 2^a per (sequence, v-head, column block), chosen from the largest
// |v| of the column block over the prefill and the largest |S| entering it so
// that they lie in [1, 2), and divides Y and the final state by 2^a (exact). V
// and the state may so have any finite f32 magnitude: f16's range holds a state
// that grows 2^15-fold beyond them. q and k rows enter as f16 (or hi + lo) and
// meet in f16 planes (the P tiles): the prep records per chunk whether they
// lie in the range those operands hold (qk_in_range: |k| < 16, |q| < 2^15,
// |q| |k| < 256 per element, finite; L2-normalised rows lie far inside) and
// whether every decay e^g lies in [0, 1] and beta is finite (g finite and at
// most 0, as the model's g = -softplus(..) is), and a (sequence, v-head) with
// any chunk outside it runs the token-by-token f32 recurrence in the scan
// instead (the sequential form's results, NaN / Inf included). So does a
// column block whose v or entering state holds an Inf or NaN. Inside the range
// each f16 element keeps an absolute precision of about 2^-25 (in the scan's
// bf16 form the q and k rows are exact).
#include <type_traits>

#include "xq_kernels.h"

namespace xq {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;
constexpr int kCols = 16;            // value columns per scan workgroup
constexpr int kColBlocks = 128 / kCols;

// Workspace record of one (sequence, v-head, chunk), byte offsets. Records are
// ordered (sequence, chunk, v-head): the prep's workgroups running at a time
// write neighbouring records.
constexpr int kRecTHi = 0;                       // f16 [64][64]
constexpr int kRecTLo = kRecTHi + 64 * 64 * 2;
constexpr int kRecDec = kRecTLo + 64 * 64 * 2;  // f32 e^G[64], e^{G_C - G}[64], e^{G_C}, range flag at 129, max|v|[8] at 136, G[64] at 192
constexpr int kRecG = 192;                      // G offset in floats within the decays
constexpr int kRecVmax = 136;                   // largest |v| of the chunk per 16-column block (floats)
constexpr int kRecRange = 129;                  // 1.0f when the chunk's q / k leave the operands' range, else 0
// P tiles (bf16 rows with 16-byte loads): tile (w, jt), jt <= w, of scan wave w
// is 1 KB at kRecP + (w (w + 1) / 2 + jt) KB; lane l's 16 bytes at 16 l are its
// four values of P[16w + l % 16][16jt + 4(l / 16) + i] as f16 hi, then f16 lo
constexpr int kRecP = kRecDec + 1024;
constexpr int kRecBytes = kRecP + 10 * 1024;
XQ_DEV constexpr int p_tile(int w, int jt) { return kRecP + (w * (w + 1) / 2 + jt) * 1024; }

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
    int32_t T;  // tokens processed here (several chunks, the last one partial)
    int32_t n_chunks;
    int32_t B;
    float scale;
};

// x = hi + lo with hi = f16(x), lo = f16(x - hi)
XQ_DEV _Float16 f16_hi(float x) { return (_Float16)x; }
XQ_DEV _Float16 f16_lo(float x) { return (_Float16)(x - (float)(_Float16)x); }

// Eight consecutive elements of an input row (bf16 or f32) as f32; VEC reads
// them with 16-byte loads (the host checks the alignment).
template <bool BF16, bool VEC>
XQ_DEV void load8(const uint8_t* row, int i0, float (&x)[8]) {
    if constexpr (VEC && BF16) {
        const uint4 w = *(const uint4*)(row + 2 * i0);
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = bf16_bits_to_f32(u[e] & 0xffffu);
            x[2 * e + 1] = bf16_bits_to_f32(u[e] >> 16);
        }
    } else if constexpr (VEC) {
        const float4 a = *(const float4*)(row + 4 * i0);
        const float4 b = *(const float4*)(row + 4 * i0 + 16);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            x[e] = BF16 ? bf16_bits_to_f32(((const uint16_t*)row)[i0 + e]) : ((const float*)row)[i0 + e];
    }
}

XQ_DEV h8 to_h8(const float (&x)[8]) {
    h8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (_Float16)x[e];
    return r;
}

// the f16 remainders x - hi of eight values whose f16 parts are hi
XQ_DEV h8 lo_h8(const float (&x)[8], h8 hi) {
    h8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (_Float16)(x[e] - (float)hi[e]);
    return r;
}

XQ_DEV f4 mfma32(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
XQ_DEV f4 mfma16(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
XQ_DEV f4 mfma_bf(uint4 a, uint4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0, 0);
}

// x = hi + mid + lo exactly with three bf16 values (truncations; the bits sit in
// the high halves of the returned words)
XQ_DEV void bf16_split3(float x, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
    hi = __float_as_uint(x) & 0xffff0000u;
    const float r = x - __uint_as_float(hi);
    mid = __float_as_uint(r) & 0xffff0000u;
    lo = __float_as_uint(r - __uint_as_float(mid));  // at most 8 significant bits: its low half is zero
}

// the high halves of a and b as one word (a low)
XQ_DEV uint32_t hi_halves(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// four consecutive f32 values as 3 x 4 bf16 terms (hi, mid, lo), one uint2 each
XQ_DEV void split3_x4(const f4& v, uint2 (&t)[3]) {
    uint32_t h[4], m[4], l[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) bf16_split3(v[r], h[r], m[r], l[r]);
    t[0] = make_uint2(hi_halves(h[0], h[1]), hi_halves(h[2], h[3]));
    t[1] = make_uint2(hi_halves(m[0], m[1]), hi_halves(m[2], m[3]));
    t[2] = make_uint2(hi_halves(l[0], l[1]), hi_halves(l[2], l[3]));
}

// Whether a chunk's q and k rows lie in the range the chunked form's operands
// hold, from the largest |element| of each (f32 bits): k below 16 and q below
// 2^15 with |q| |k| below 256 per element pair, all finite. Then every f16
// operand (k, q as f16 or hi + lo; K K^T, q . k <= 128 |q| |k| in the f16 P
// tiles) stays below 2^15; L2-normalised rows (|element| <= 1) lie far
// inside. A NaN compares false, so non-finite rows fall outside.
XQ_DEV bool qk_in_range(uint32_t kbits, uint32_t qbits) {
    const float km = __uint_as_float(kbits), qm = __uint_as_float(qbits);
    return km < 16.0f && qm < 32768.0f && km * qm < 256.0f;
}

// Running maximum of |x| over bf16 pairs: m holds two 16-bit magnitude fields
// (the bf16 bits without sign), updated by one packed unsigned maximum
XQ_DEV uint32_t bf16x2_absmax(uint32_t m, uint32_t w) {
    typedef unsigned short u16x2v __attribute__((ext_vector_type(2)));
    const u16x2v a = __builtin_bit_cast(u16x2v, m), b = __builtin_bit_cast(u16x2v, w & 0x7fff7fffu);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(a, b));
}
// f32 bits of the larger magnitude field of bf16x2_absmax's result
XQ_DEV uint32_t bf16x2_max_bits(uint32_t m) { return max(m & 0xffffu, m >> 16) << 16; }

// the largest of v over the wave (unsigned)
XQ_DEV uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp_i<0xB1>((int)v));
    v = max(v, (uint32_t)dpp_i<0x4E>((int)v));
    v = max(v, (uint32_t)dpp_i<0x141>((int)v));
    v = max(v, (uint32_t)dpp_i<0x140>((int)v));  // the 16-lane row's maximum in every lane
    v = max(v, (uint32_t)__shfl_xor((int)v, 16));
    return max(v, (uint32_t)__shfl_xor((int)v, 32));
}

// ---------------------------------------------------------------- prep

template <bool BF16, bool VEC>
__global__ __launch_bounds__(256, BF16 ? 2 : 1) void gdn_chunk_prep(GdnChunkArgs a) {
    constexpr int KP = 136;  // padded f16 row stride (halves)
    constexpr int FP = 68;   // padded f32 row stride (16-byte rows, conflict-free MFMA stores)
    // 36 KB for bf16 rows (53 KB for f32 rows); after the products sK becomes M.
    __shared__ __attribute__((aligned(16))) _Float16 sK[64 * KP];    // K [t][i], then M f32 [64][FP]
    __shared__ __attribute__((aligned(16))) float sKK[64 * FP];  // L of one v-head
    __shared__ __attribute__((aligned(16))) float sG[2][64], sBeta[2][64], sEG[2][64];
    __shared__ uint32_t sVmax[2][kColBlocks];  // bits of the largest |v| per column block
    __shared__ uint32_t sQKmax[2];              // bits of the chunk's largest |k|, |q|
    __shared__ uint32_t sGBout[2];              // per v-head: some g not finite or above 0, or beta not finite
    // f32 rows: the f16 remainders of K
    constexpr int NKL = BF16 ? 8 : 64 * KP;
    __shared__ __attribute__((aligned(16))) _Float16 sKl[NKL];
    static_assert(64 * FP * 4 <= 64 * KP * 2, "LDS aliases");

    // bf16 rows read as 16-byte words (RAW): K and Q stay bf16 in LDS and the
    // products run on bf16 MFMA (exact operands); the P tiles are formed here
    constexpr bool RAW = BF16 && VEC;
    _Float16* sQ = (_Float16*)sKK;  // RAW: Q [t][i] until the products are done
    static_assert(64 * FP * 4 >= 64 * KP * 2, "Q rows fit the L buffer");

    // v-heads kh and kh + 16 share k-head kh: K K^T is formed once for both.
    // The k-heads of a chunk are consecutive workgroups: they read the
    // neighbouring parts of the same rows at about the same time.
    const int n = blockIdx.y, kh = blockIdx.x, b = blockIdx.z;
    const int tid = threadIdx.x;
    const int wave = wave_id(), lane = lane_id(), lr = lane & 15, lg = lane >> 4;
    const int t0 = n * kChunk;

    // ---- chunk rows -> LDS as f16 (tokens past T are zero, with g = beta = 0):
    //      thread = (token, quarter of 32 elements), 8 elements per load
    {
        const int t = tid >> 2, qt = tid & 3;
        const int tg = t0 + t;
        const bool ok = tg < a.T;
        const uint8_t* kr = a.k + (int64_t)b * a.k_nb3 + (int64_t)tg * a.k_nb2 + (int64_t)kh * a.k_nb1;
        uint32_t kmx = 0, qmx = 0;  // the largest |k|, |q| of the thread's elements (f32 bits)
        if constexpr (RAW) {
            // rows past T: loads of row T - 1, zeroed (no conditional loads)
            const int tc = min(tg, a.T - 1);
            const uint8_t* kc = a.k + (int64_t)b * a.k_nb3 + (int64_t)tc * a.k_nb2 + (int64_t)kh * a.k_nb1;
            const uint8_t* qc = a.q + (int64_t)b * a.q_nb3 + (int64_t)tc * a.q_nb2 + (int64_t)kh * a.q_nb1;
            uint4 wk[4], wq[4];
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                wk[gi] = *(const uint4*)(kc + 2 * (32 * qt + 8 * gi));
                wq[gi] = *(const uint4*)(qc + 2 * (32 * qt + 8 * gi));
            }
            const uint32_t m = ok ? ~0u : 0u;  // a mask, not a select of the arrays
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const uint4 x = wk[gi], y = wq[gi];
                *(uint4*)(sK + t * KP + 32 * qt + 8 * gi) = make_uint4(x.x & m, x.y & m, x.z & m, x.w & m);
                *(uint4*)(sQ + t * KP + 32 * qt + 8 * gi) = make_uint4(y.x & m, y.y & m, y.z & m, y.w & m);
                kmx = bf16x2_absmax(bf16x2_absmax(bf16x2_absmax(bf16x2_absmax(kmx, x.x & m), x.y & m), x.z & m), x.w & m);
                qmx = bf16x2_absmax(bf16x2_absmax(bf16x2_absmax(bf16x2_absmax(qmx, y.x & m), y.y & m), y.z & m), y.w & m);
            }
            kmx = bf16x2_max_bits(kmx);
            qmx = bf16x2_max_bits(qmx);
        }
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
            if constexpr (RAW) break;
            const int i0 = 32 * qt + 8 * gi;
            float xk[8];
            if (ok) {
                load8<BF16, VEC>(kr, i0, xk);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) xk[e] = 0.0f;
            }
            const h8 hk = to_h8(xk);
            *(h8*)(sK + t * KP + i0) = hk;
            if constexpr (!BF16) *(h8*)(sKl + t * KP + i0) = lo_h8(xk, hk);
            // q rows, read here for their range only (the scan forms P from them)
            float xq[8];
            if (ok) {
                load8<BF16, VEC>(a.q + (int64_t)b * a.q_nb3 + (int64_t)tg * a.q_nb2 + (int64_t)kh * a.q_nb1, i0, xq);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) xq[e] = 0.0f;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                kmx = max(kmx, __float_as_uint(xk[e]) & 0x7fffffffu);
                qmx = max(qmx, __float_as_uint(xq[e]) & 0x7fffffffu);
            }
        }
        // largest |v| of the token's 32 columns 32qt.. (two column blocks) for
        // each v-head; Inf and NaN compare as the largest bits, so they reach
        // the scan's choice (which runs such a column block token by token)
        if (tid < 2 * kColBlocks) sVmax[tid / kColBlocks][tid % kColBlocks] = 0;
        if (tid < 2) sQKmax[tid] = 0, sGBout[tid] = 0;
        uint32_t vm[2][2] = {{0, 0}, {0, 0}};
        if (ok) {
#pragma unroll
            for (int e2 = 0; e2 < 2; ++e2) {
                const uint8_t* vr = a.v + (int64_t)b * a.v_nb3 + (int64_t)tg * a.v_nb2 + (int64_t)(kh + 16 * e2) * a.v_nb1;
#pragma unroll
                for (int gi = 0; gi < 4; ++gi) {
                    float xv[8];
                    load8<BF16, false>(vr, 32 * qt + 8 * gi, xv);
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        vm[e2][gi >> 1] = max(vm[e2][gi >> 1], __float_as_uint(xv[e]) & 0x7fffffffu);
                }
            }
        }
        __syncthreads();  // sVmax cleared
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2) {
            atomicMax(&sVmax[e2][2 * qt], vm[e2][0]);
            atomicMax(&sVmax[e2][2 * qt + 1], vm[e2][1]);
        }
        kmx = wave_max_u32(kmx);
        qmx = wave_max_u32(qmx);
        if (lane == 0) {
            atomicMax(&sQKmax[0], kmx);
            atomicMax(&sQKmax[1], qmx);
        }
        if (tid < 128) {
            const int e2 = tid >> 6, tt = t0 + (tid & 63), h = kh + 16 * e2;
            const bool ok2 = tt < a.T;
            const float gv = ok2 ? *(const float*)(a.g + (int64_t)b * a.g_nb3 + (int64_t)tt * a.g_nb2 + (int64_t)h * a.g_nb1) : 0.0f;
            const float bv = ok2 ? *(const float*)(a.beta + (int64_t)b * a.b_nb3 + (int64_t)tt * a.b_nb2 + (int64_t)h * a.b_nb1) : 0.0f;
            sG[e2][tid & 63] = gv;
            sBeta[e2][tid & 63] = bv;
            // the chunked form takes decays e^g in [0, 1]: g finite and <= 0
            // (differences of cumulative log-decays stay finite and the
            // factors e^{G_t - G_j} at most 1), beta finite
            if (!(gv <= 0.0f && gv > -INFINITY && __builtin_isfinite(bv))) atomicOr(&sGBout[e2], 1u);
        }
    }
    __syncthreads();
    // cumulative log-decays (sequential sums, as the recurrence applies the decays)
    if (tid < 128) {
        const int e2 = tid >> 6, t = tid & 63;
        float G = 0.0f;
        for (int s = 0; s <= t; ++s) G += sG[e2][s];
        sEG[e2][t] = G;
    }
    // ---- K K^T: 16 tiles, 4 per wave, contraction over 128 key dims; kept in
    //      registers for the L of both v-heads
    f4 kk[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        const int tile = wave * 4 + tt;
        const int mt = tile >> 2, nt = tile & 3;
        kk[tt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (RAW) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                kk[tt] = mfma_bf(*(const uint4*)(sK + (mt * 16 + lr) * KP + ks * 32 + 8 * lg),
                                 *(const uint4*)(sK + (nt * 16 + lr) * KP + ks * 32 + 8 * lg), kk[tt]);
            continue;
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const h8 bk = *(const h8*)(sK + (nt * 16 + lr) * KP + ks * 32 + 8 * lg);
            const h8 ak = *(const h8*)(sK + (mt * 16 + lr) * KP + ks * 32 + 8 * lg);
            kk[tt] = mfma32(ak, bk, kk[tt]);
            if constexpr (!BF16) {
                const h8 bkl = *(const h8*)(sKl + (nt * 16 + lr) * KP + ks * 32 + 8 * lg);
                const h8 akl = *(const h8*)(sKl + (mt * 16 + lr) * KP + ks * 32 + 8 * lg);
                kk[tt] = mfma32(ak, bkl, kk[tt]);
                kk[tt] = mfma32(akl, bk, kk[tt]);
            }
        }
    }
    // RAW: P^T = K Q^T for the scan wave w's tiles (token tile w of q, tiles
    // jt <= w of k), the products the scan would form: lane (lr, lg) holds
    // q_t . k_j for t = 16w + lr, j = 16jt + 4lg + i
    f4 pq[4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
        pq[jt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if (RAW && jt <= wave) {  // wave-uniform
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                pq[jt] = mfma_bf(*(const uint4*)(sK + (16 * jt + lr) * KP + 32 * ks + 8 * lg),
                                 *(const uint4*)(sQ + (16 * wave + lr) * KP + 32 * ks + 8 * lg), pq[jt]);
        }
    }
    __syncthreads();  // K and Q no longer read; G ready

    // ---- per v-head: M = (I + L)^{-1} by blocks of 16 (T = M diag(beta) is
    //      formed at the record). With D_i = I + L_ii the unit lower-triangular
    //      diagonal blocks:
    //        1. M_ii = D_i^{-1}, one wave per block, a 16-step substitution;
    //        2. the 32 x 32 diagonal blocks: M_10 = -M_11 L_10 M_00 and
    //           M_32 = -M_33 L_32 M_22;
    //        3. the lower-left 32 x 32 block: -M_B C M_A with C = L[32..64)[0..32)
    //           and M_A, M_B the 32 x 32 inverses of step 2.
    //      The products run on f32 MFMA. The dependent chain is 16 substitution
    //      steps and six 16 x 16 x 16 products, against 64 steps for a column-wise
    //      substitution. The upper-triangular blocks of L (zero, never read
    //      again) hold the intermediate products.
    float* sT = (float*)sK;  // M [t][j], f32
    auto blk = [&](float* base, int bi, int bj) { return base + 16 * bi * FP + 16 * bj; };
    // acc += A B for 16 x 16 blocks A, B (row stride FP), on f32 MFMA
    auto mm16 = [&](const float* A, const float* B, f4 acc) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[lr * FP + 4 * kb + lg], B[(4 * kb + lg) * FP + lr], acc, 0, 0, 0);
        return acc;
    };
    auto st16 = [&](float* C, const f4& v, float sgn) {
#pragma unroll
        for (int r = 0; r < 4; ++r) C[(4 * lg + r) * FP + lr] = sgn * v[r];
    };
    for (int e2 = 0; e2 < 2; ++e2) {
        const int h = kh + 16 * e2;
        // L (strictly lower) from the K K^T tiles. The previous v-head's last
        // reads of sKK sit before the barrier that ends its inverse, its reads
        // of M before the barrier below.
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            const int tile = wave * 4 + tt;
            const int mt = tile >> 2, nt = tile & 3;
            const int j = nt * 16 + lr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = mt * 16 + 4 * lg + r;
                sKK[t * FP + j] = j < t ? sBeta[e2][t] * __expf(sEG[e2][t] - sEG[e2][j]) * kk[tt][r] : 0.0f;
            }
        }
        __syncthreads();
        {
            // 1. D_w^{-1}: column c by a quad of lanes, lane part p keeps rows
            //    4p..4p+3 and the quad sums the dot products; the rows of L are
            //    read two steps ahead so the LDS latency stays off the chain
            const int c = lane >> 2, p = lane & 3, o = 16 * wave;
            float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            f4 Lq[3];
            auto ldrow = [&](int t) { return *(const f4*)(sKK + (o + t) * FP + o + 4 * p); };
            Lq[1] = ldrow(1);
            Lq[2] = ldrow(2);
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                float part = 0.0f;
                if (t > 0) {
                    if (t + 2 < 16) Lq[(t + 2) % 3] = ldrow(t + 2);
                    const f4 Lr = Lq[t % 3];  // L[t][s >= t] = 0
                    part = fmaf(Lr[1], x[1], Lr[0] * x[0]) + fmaf(Lr[3], x[3], Lr[2] * x[2]);
                }
                part += dpp<0xB1>(part);  // quad: lanes p ^ 1
                part += dpp<0x4E>(part);  // quad: lanes p ^ 2
                const float xt = t < c ? 0.0f : (t == c ? 1.0f : -part);
                if ((t >> 2) == p) x[t & 3] = xt;
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) sT[(o + 4 * p + m) * FP + o + c] = x[m];
            // the upper-triangular blocks of M are zero
            for (int bj = wave + 1; bj < 4; ++bj) st16(blk(sT, wave, bj), f4{0.0f, 0.0f, 0.0f, 0.0f}, 1.0f);
        }
        __syncthreads();
        if (wave < 2) {  // 2. wave 0: M_10, wave 1: M_32 (scratch: L blocks (0, 1), (2, 3))
            const int i = 2 * wave + 1, j = 2 * wave;
            float* P = blk(sKK, j, i);
            st16(P, mm16(blk(sKK, i, j), blk(sT, j, j), f4{0.0f, 0.0f, 0.0f, 0.0f}), 1.0f);
            st16(blk(sT, i, j), mm16(blk(sT, i, i), P, f4{0.0f, 0.0f, 0.0f, 0.0f}), -1.0f);
        }
        __syncthreads();
        {  // 3. wave w: block (i, j) = (2 + w / 2, w % 2); Q = C M_A in L blocks (j, i)
            const int i = 2 + (wave >> 1), j = wave & 1;
            f4 q = mm16(blk(sKK, i, 1), blk(sT, 1, j), f4{0.0f, 0.0f, 0.0f, 0.0f});
            if (j == 0) q = mm16(blk(sKK, i, 0), blk(sT, 0, 0), q);
            st16(blk(sKK, j, i), q, 1.0f);
            __syncthreads();
            f4 r = mm16(blk(sT, i, 2), blk(sKK, j, 2), f4{0.0f, 0.0f, 0.0f, 0.0f});
            if (i == 3) r = mm16(blk(sT, 3, 3), blk(sKK, j, 3), r);
            st16(blk(sT, i, j), r, -1.0f);
        }
        __syncthreads();

        // ---- the record: T (f16 hi + lo) with 16-byte stores, the decays and G
        uint8_t* rec = a.ws + (((int64_t)b * a.n_chunks + n) * 32 + h) * kRecBytes;
        {
            const int t = tid >> 2, j0 = 16 * (tid & 3);
            h8 th[2], tl[2];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float tv = sT[t * FP + j0 + e] * sBeta[e2][j0 + e];  // T = M diag(beta)
                th[e >> 3][e & 7] = f16_hi(tv), tl[e >> 3][e & 7] = f16_lo(tv);
            }
            const int o = (t * 64 + j0) * 2;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                *(h8*)(rec + kRecTHi + o + 16 * u) = th[u];
                *(h8*)(rec + kRecTLo + o + 16 * u) = tl[u];
            }
        }
        if (tid < 64) {
            const float GC = sEG[e2][63];
            const float G = sEG[e2][tid];
            float* dec = (float*)(rec + kRecDec);
            dec[tid] = __expf(G);
            dec[64 + tid] = __expf(GC - G);
            dec[kRecG + tid] = G;
            if (tid == 0) dec[128] = __expf(GC);
            if (tid == 1) dec[kRecRange] = qk_in_range(sQKmax[0], sQKmax[1]) && !sGBout[e2] ? 0.0f : 1.0f;
            if (tid < kColBlocks) dec[kRecVmax + tid] = __uint_as_float(sVmax[e2][tid]);
        }
        if constexpr (RAW) {  // P[t][j] = (q_t . k_j) e^{G_t - G_j} (j <= t), f16 hi + lo
            uint8_t* pr = rec + 16 * lane;
            const float gt = sEG[e2][16 * wave + lr];
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                if (jt <= wave) {  // wave-uniform
                    const f4 gj = *(const f4*)&sEG[e2][16 * jt + 4 * lg];
                    h4 ph, pl;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const bool causal = jt < wave || 4 * lg + i <= lr;
                        const float pv = causal ? pq[jt][i] * __expf(gt - gj[i]) : 0.0f;
                        ph[i] = f16_hi(pv), pl[i] = f16_lo(pv);
                    }
                    const uint2 bh = __builtin_bit_cast(uint2, ph), bl = __builtin_bit_cast(uint2, pl);
                    *(uint4*)(pr + p_tile(wave, jt)) = make_uint4(bh.x, bh.y, bl.x, bl.y);
                }
            }
        }
    }
}

// ---------------------------------------------------------------- scan

// Operands of one chunk for one wave of a scan workgroup, loaded a chunk ahead:
// A operands (row 16w + lr of the wave's token tile, k = 32 ks + 8 lg .. +7) of
// K and Q (raw input words, decoded when used) and of T (hi, lo); the raw V
// values and e^G, e^{G_C - G} of the lane's four tokens 16w + 4lg + r (column
// 16cb + lr), e^{G_C}; for bf16 rows read as 16-byte words the wave's P tiles
// from the record, otherwise the G values the scan's P needs (token 16w + lr,
// tokens 16jt + 4lg + i). The loads are unconditional but for the P tiles (one
// per tile jt <= w, a count fixed per wave): token and chunk indices are
// clamped into range and out-of-range tokens masked at use, so the compiler's
// waits for a chunk's operands never include the next chunk's loads.
template <bool BF16, bool VEC>
struct ScanOps {
    static constexpr int KW = VEC ? (BF16 ? 1 : 2) : 4;  // 16-byte words per 8 elements (VEC), else raw dwords
    uint4 kw[4][KW], qw[4][KW];
    uint4 pw[4];  // bf16 rows with 16-byte loads: the wave's P tiles (w, jt <= w) from the record
    h8 th[2], tl[2];
    // raw V words, in the input's width: a 16-bit load widened at use (widened
    // here, the compiler copies the value at the loop edge and waits for it)
    std::conditional_t<BF16, uint16_t, uint32_t> vw[4];
    float4 eg, egc;
    float eGC;
    float gt;       // G of token 16w + lr
    f4 gj[4];       // G of tokens 16jt + 4lg + i
    bool ok;        // the A-operand token is in range
    uint32_t vok;   // bit r: token 16w + 4lg + r is in range
};

// 8 elements of a K / Q row: raw words at element i0
template <bool BF16, bool VEC, int KW>
XQ_DEV void load_raw8(const uint8_t* row, int i0, uint4 (&w)[KW]) {
    if constexpr (VEC) {
        const uint8_t* p = row + (BF16 ? 2 : 4) * i0;
#pragma unroll
        for (int u = 0; u < KW; ++u) w[u] = *(const uint4*)(p + 16 * u);
    } else {
        uint32_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            e[j] = BF16 ? (uint32_t)((const uint16_t*)row)[i0 + j] : ((const uint32_t*)row)[i0 + j];
        w[0] = make_uint4(e[0], e[1], e[2], e[3]);
        w[1] = make_uint4(e[4], e[5], e[6], e[7]);
        w[2] = w[3] = make_uint4(0, 0, 0, 0);
    }
}

// f32 rows: the f16 remainder x - f16(x) of the same eight elements
template <int KW>
XQ_DEV h8 decode8_lo(const uint4 (&w)[KW], bool ok) {
    const uint32_t u[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
    h8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float x = __uint_as_float(u[e]);
        r[e] = ok ? (_Float16)(x - (float)(_Float16)x) : (_Float16)0.0f;
    }
    return r;
}

template <bool BF16, bool VEC, int KW>
XQ_DEV h8 decode8(const uint4 (&w)[KW], bool ok) {
    float x[8];
    if constexpr (VEC && BF16) {
        const uint32_t u[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = bf16_bits_to_f32(u[e] & 0xffffu);
            x[2 * e + 1] = bf16_bits_to_f32(u[e] >> 16);
        }
    } else {
        const uint32_t u[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = BF16 ? bf16_bits_to_f32(u[e] & 0xffffu) : __uint_as_float(u[e]);
    }
    h8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = ok ? (_Float16)x[e] : (_Float16)0.0f;
    return r;
}

// Four 16-bit elements read transposed from LDS (gfx950 ds_read_b64_tr_b16):
// in each group of 16 lanes, lane 4j + q addresses 4 consecutive elements of
// row j of a 4 x 16 block (columns 4q .. 4q + 3), and lane m of the group
// receives column m of that block, rows 0..3, in order.
XQ_DEV uint2 lds_read_tr16(const _Float16* p) {
    typedef short s4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s4 lds_s4;
    const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(__attribute__((address_space(3))) short*)p);
    return __builtin_bit_cast(uint2, v);
}

// A buffer resource over one workspace record (raw: byte offsets, no stride;
// the record is far below the 2^31-byte range it allows).
XQ_DEV __amdgpu_buffer_rsrc_t rec_rsrc(const uint8_t* rec) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)rec, (short)0, 0x7fffffff, 0x00020000);
}

// The operands of chunk n in four parts, each issued in its own phase of the
// previous chunk's step (between its barriers), in the order the step uses
// them: a burst of all of them at the start of a step stalls the wave while
// the loads queue. Part 0: K and Q rows; 1: T; 2: the decays and G; 3: V.
template <int PART, bool BF16, bool VEC>
XQ_DEV void scan_load(const GdnChunkArgs& a, int b, int h, int cb, int n, int wave, int lr, int lg,
                      ScanOps<BF16, VEC>& L) {
    const int kh = h % 16;
    n = min(n, a.n_chunks - 1);  // the prefetch past the last chunk re-reads it
    const int row0 = n * kChunk;      // the chunk's first token
    const int last = a.T - 1 - row0;  // the chunk's rows past T read row T - 1 instead
    const uint8_t* rec = a.ws + (((int64_t)b * a.n_chunks + n) * 32 + h) * kRecBytes;
    // Row addresses are a wave-uniform base (sequence, head, chunk: scalar
    // registers) plus a 32-bit per-lane offset (the host keeps the row strides
    // below 2^25 bytes), so the loads take their base from SGPRs and the
    // per-chunk address arithmetic stays off the vector ALU.
    if constexpr (PART == 0) {
        const int r = 16 * wave + lr;  // A-operand row of the chunk
        L.ok = r <= last;
        const uint32_t rc = (uint32_t)min(r, last);
        const uint8_t* kb = a.k + (int64_t)b * a.k_nb3 + (int64_t)row0 * a.k_nb2 + (int64_t)kh * a.k_nb1;
        const uint8_t* qb = a.q + (int64_t)b * a.q_nb3 + (int64_t)row0 * a.q_nb2 + (int64_t)kh * a.q_nb1;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if constexpr (VEC) {  // the lane's part of the offset in one 32-bit word
                const uint32_t eo = (BF16 ? 2u : 4u) * (8u * (uint32_t)lg);
                const uint32_t ko = rc * (uint32_t)a.k_nb2 + eo, qo = rc * (uint32_t)a.q_nb2 + eo;
#pragma unroll
                for (int u = 0; u < ScanOps<BF16, VEC>::KW; ++u) {
                    L.kw[ks][u] = *(const uint4*)(kb + (BF16 ? 64 : 128) * ks + 16 * u + ko);
                    L.qw[ks][u] = *(const uint4*)(qb + (BF16 ? 64 : 128) * ks + 16 * u + qo);
                }
            } else {
                load_raw8<BF16, VEC>(kb + rc * (uint32_t)a.k_nb2, 32 * ks + 8 * lg, L.kw[ks]);
                load_raw8<BF16, VEC>(qb + rc * (uint32_t)a.q_nb2, 32 * ks + 8 * lg, L.qw[ks]);
            }
        }
    } else if constexpr (PART == 1) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const uint32_t o = ((uint32_t)(16 * wave + lr) * 64u + 32u * ks + 8u * lg) * 2u;
            if constexpr (BF16 && VEC) {
                const __amdgpu_buffer_rsrc_t r = rec_rsrc(rec);
                L.th[ks] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(r, o, kRecTHi, 0));
                L.tl[ks] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(r, o, kRecTLo, 0));
            } else {
                L.th[ks] = *(const h8*)(rec + kRecTHi + o);
                L.tl[ks] = *(const h8*)(rec + kRecTLo + o);
            }
        }
    } else if constexpr (PART == 2 && BF16 && VEC) {
        // the record through a buffer resource: uniform parts of the offsets in
        // SGPRs, the lane's part in one VGPR, no per-load address arithmetic
        const __amdgpu_buffer_rsrc_t r = rec_rsrc(rec);
        const uint32_t eo = 4u * (uint32_t)(16 * wave + 4 * lg);
        L.eg = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, eo, kRecDec, 0));
        L.egc = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, eo, kRecDec + 256, 0));
        L.eGC = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, 0u, kRecDec + 512, 0));
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
            if (jt <= wave)  // wave-uniform
                L.pw[jt] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, 16u * (uint32_t)(lr + 16 * lg), p_tile(wave, jt), 0));
    } else if constexpr (PART == 2) {
        const uint8_t* dec = rec + kRecDec;  // f32 values, byte offsets below
        L.eg = *(const float4*)(dec + 4u * (uint32_t)(16 * wave + 4 * lg));
        L.egc = *(const float4*)(dec + 4u * (uint32_t)(64 + 16 * wave + 4 * lg));
        L.eGC = *(const float*)(dec + 4u * 128u);
        L.gt = *(const float*)(dec + 4u * (uint32_t)(kRecG + 16 * wave + lr));
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) L.gj[jt] = *(const f4*)(dec + 4u * (uint32_t)(kRecG + 16 * jt + 4 * lg));
    } else if constexpr (BF16 && VEC) {
        // the chunk's V rows through a buffer resource whose range ends after
        // row `last` (row offsets below 2^25 bytes): a row past it reads 0
        // without touching memory (and is masked at use), so the lane offsets
        // need no clamp and stay the same for every chunk
        L.vok = 0;
        const uint8_t* vb = a.v + (int64_t)b * a.v_nb3 + (int64_t)row0 * a.v_nb2 + (int64_t)h * a.v_nb1;
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc((void*)vb, (short)0, (int)((uint32_t)min(last, kChunk - 1) * (uint32_t)a.v_nb2 + 256u), 0x00020000);
        const uint32_t co = (uint32_t)(kCols * cb + lr) * 2u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int rr = 16 * wave + 4 * lg + q;
            L.vok |= (rr <= last ? 1u : 0u) << q;
            L.vw[q] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, (uint32_t)rr * (uint32_t)a.v_nb2 + co, 0, 0);
        }
    } else {
        L.vok = 0;
        const uint8_t* vb = a.v + (int64_t)b * a.v_nb3 + (int64_t)row0 * a.v_nb2 + (int64_t)h * a.v_nb1;
        const uint32_t co = (uint32_t)(kCols * cb + lr) * (BF16 ? 2u : 4u);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rr = 16 * wave + 4 * lg + r;
            L.vok |= (rr <= last ? 1u : 0u) << r;
            const uint8_t* vr = vb + ((uint32_t)min(rr, last) * (uint32_t)a.v_nb2 + co);
            if constexpr (BF16)
                L.vw[r] = *(const uint16_t*)vr;
            else
                L.vw[r] = *(const uint32_t*)vr;
        }
    }
}

template <bool BF16, bool VEC>
XQ_DEV void scan_load_all(const GdnChunkArgs& a, int b, int h, int cb, int n, int wave, int lr, int lg,
                          ScanOps<BF16, VEC>& L) {
    scan_load<0>(a, b, h, cb, n, wave, lr, lg, L);
    scan_load<1>(a, b, h, cb, n, wave, lr, lg, L);
    scan_load<2>(a, b, h, cb, n, wave, lr, lg, L);
    scan_load<3>(a, b, h, cb, n, wave, lr, lg, L);
}

// The token-by-token recurrence for a scan workgroup's 16 columns, in f32: the
// chunked form's fallback for a (sequence, v-head) whose q or k rows leave
// the range its operands hold in some chunk (qk_in_range). Lanes 16j .. 16j +
// 15 of wave w own column 16 cb + 4w + j, lane part r its key dims 8r .. 8r +
// 7; each token's dot products reduce over the 16 lanes.
template <bool BF16>
XQ_DEV void scan_sequential(const GdnChunkArgs& a, int b, int h, int cb, int wave, int lane) {
    const int kh = h % 16, r = lane & 15, c = kCols * cb + 4 * wave + (lane >> 4);
    const float* st = a.state + (int64_t)b * (a.s_nb3 / 4) + (int64_t)h * 16384 + (int64_t)c * 128 + 8 * r;
    float s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = st[e];
    float* out = a.dst + (int64_t)b * (a.dst_nb2 / 4);
    for (int t = 0; t < a.T; ++t) {
        float kx[8], qx[8];
        load8<BF16, false>(a.k + (int64_t)b * a.k_nb3 + (int64_t)t * a.k_nb2 + (int64_t)kh * a.k_nb1, 8 * r, kx);
        load8<BF16, false>(a.q + (int64_t)b * a.q_nb3 + (int64_t)t * a.q_nb2 + (int64_t)kh * a.q_nb1, 8 * r, qx);
        const float g = *(const float*)(a.g + (int64_t)b * a.g_nb3 + (int64_t)t * a.g_nb2 + (int64_t)h * a.g_nb1);
        const float be = *(const float*)(a.beta + (int64_t)b * a.b_nb3 + (int64_t)t * a.b_nb2 + (int64_t)h * a.b_nb1);
        const uint8_t* vr = a.v + (int64_t)b * a.v_nb3 + (int64_t)t * a.v_nb2 + (int64_t)h * a.v_nb1;
        const float vv = BF16 ? bf16_bits_to_f32(((const uint16_t*)vr)[c]) : ((const float*)vr)[c];
        const float dk = expf(g);
        float kv = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            s[e] *= dk;
            kv = fmaf(s[e], kx[e], kv);
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) kv += __shfl_xor(kv, o);
        const float d = (vv - kv) * be;
        float y = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            s[e] = fmaf(kx[e], d, s[e]);
            y = fmaf(s[e], qx[e], y);
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) y += __shfl_xor(y, o);
        if (r == 0) out[(int64_t)t * 4096 + h * 128 + c] = y * a.scale;
    }
    float* so = a.state_out + (int64_t)b * (a.so_nb3 / 4) + (int64_t)h * 16384 + (int64_t)c * 128 + 8 * r;
#pragma unroll
    for (int e = 0; e < 8; ++e) so[e] = s[e];
}

// NTY: the outputs Y are stored non-temporally (one workgroup per CU; see the
// stores)
template <bool BF16, bool VEC, bool NTY>
__global__ __launch_bounds__(256) void gdn_chunk_scan(GdnChunkArgs a) {
    constexpr int TP = 72;   // X^T, U^T rows [c][t] (halves)
    constexpr int SP = 136;  // S^T rows [c][i] (halves)
    // bf16 rows with 16-byte row loads (RAW): the raw rows are the operands of
    // bf16 products (exact), the state and e^{G_C - G} U enter as three bf16
    // terms (hi, mid, lo; the f32 value exactly); otherwise f16 hi + lo
    constexpr bool RAW = BF16 && VEC;
    __shared__ __attribute__((aligned(16))) _Float16 sSh[kCols * SP], sSl[kCols * SP];  // S^T hi, lo
    __shared__ __attribute__((aligned(16))) _Float16 sSm[RAW ? kCols * SP : 8];        // S^T mid (RAW)
    __shared__ __attribute__((aligned(16))) _Float16 sXh[kCols * TP], sXl[kCols * TP];  // X^T
    __shared__ __attribute__((aligned(16))) _Float16 sUh[kCols * TP], sUl[kCols * TP];  // U^T
    __shared__ __attribute__((aligned(16))) _Float16 sWh[kCols * TP], sWl[kCols * TP];  // (e^{G_C - G} U)^T
    __shared__ __attribute__((aligned(16))) _Float16 sWm[RAW ? kCols * TP : 8];
    // K rows of the chunk [t][i] (f16 hi, and lo for f32 rows): the A operands of P^T = K Q^T
    __shared__ __attribute__((aligned(16))) _Float16 sKh[RAW ? 8 : 64 * SP], sKl[BF16 ? 8 : 64 * SP];
    // The state update's A operands K^T, by chunk parity (read after the step's
    // last barrier, so the next chunk writes the other one): K^T [i][t] (f16
    // hi, and lo for f32 rows), or in the bf16 operand form (RAW) the chunk's K
    // rows [t][i] as loaded, pitch KRP, which the update reads transposed
    // (lds_read_tr16). Both layouts take 128 x KTP = 64 x KRP halves.
    constexpr int KTP = 72;   // K^T rows (halves)
    constexpr int KRP = 144;  // RAW: K rows (halves; 288 bytes, rows 8 banks apart)
    static_assert(128 * KTP == 64 * KRP, "one buffer for both layouts");
    __shared__ __attribute__((aligned(16))) _Float16 sKTh[2][128 * KTP], sKTl[2][BF16 ? 8 : 128 * KTP];

    const uint32_t n_wg = (uint32_t)a.B * 32 * kColBlocks;
    // column blocks of a head adjacent, then the two v-heads kh, kh + 16 that
    // read the same K and Q rows: the 16 workgroups on one XCD (shared L2)
    const uint32_t wg = xcd_remap(blockIdx.x, n_wg);
    const int cb = (int)(wg % kColBlocks);
    const int h = (int)((wg / (2 * kColBlocks)) % 16) + 16 * (int)((wg / kColBlocks) % 2);
    const int b = (int)(wg / (kColBlocks * 32));
    const int wave = wave_id(), lane = lane_id(), lr = lane & 15, lg = lane >> 4;

    // state tiles of this wave: key-dim tiles 2w, 2w + 1 of the 128 x 16 block;
    // lane holds S[i = 16 it + 4 lg + r][c = 16 cb + lr]
    const float* st = a.state + (int64_t)b * (a.s_nb3 / 4) + (int64_t)h * 16384;
    f4 S[2];
#pragma unroll
    for (int a2 = 0; a2 < 2; ++a2) {
        const int it = 2 * wave + a2;
        const float4 v = *(const float4*)(st + (int64_t)(kCols * cb + lr) * 128 + 16 * it + 4 * lg);
        S[a2] = f4{v.x, v.y, v.z, v.w};
    }
    float* out = a.dst + (int64_t)b * (a.dst_nb2 / 4);
    // the first chunk's operands do not depend on 2^a (V is scaled at use): their
    // loads go out with the state's and the maxima's
    ScanOps<BF16, VEC> ops[2];
    scan_load_all<BF16, VEC>(a, b, h, cb, 0, wave, lr, lg, ops[0]);

    // ---- 2^a: the largest |S| entering the block and |v| of its columns over
    //      the prefill (the chunks' maxima from the prep) brought into [1, 2)
    //      (and whether some chunk's q / k leave the operands' range)
    __shared__ uint32_t sAm[4], sOut[4];
    {
        uint32_t am = 0;
        bool out_of_range = false;
#pragma unroll
        for (int a2 = 0; a2 < 2; ++a2)
#pragma unroll
            for (int r = 0; r < 4; ++r) am = max(am, __float_as_uint(S[a2][r]) & 0x7fffffffu);
        for (int n = lane; n < a.n_chunks; n += 64) {
            const float* dec = (const float*)(a.ws + (((int64_t)b * a.n_chunks + n) * 32 + h) * kRecBytes + kRecDec);
            am = max(am, __float_as_uint(dec[kRecVmax + cb]) & 0x7fffffffu);
            out_of_range |= dec[kRecRange] != 0.0f;
        }
        const bool wave_out = __builtin_amdgcn_ballot_w64(out_of_range) != 0;  // every lane of the wave
        if (lane == 0) sOut[wave] = wave_out ? 1u : 0u;
        am = max(am, (uint32_t)dpp_i<0xB1>((int)am));
        am = max(am, (uint32_t)dpp_i<0x4E>((int)am));
        am = max(am, (uint32_t)dpp_i<0x141>((int)am));
        am = max(am, (uint32_t)dpp_i<0x140>((int)am));
        am = max(am, (uint32_t)__shfl_xor((int)am, 16));
        am = max(am, (uint32_t)__shfl_xor((int)am, 32));
        if (lane == 0) sAm[wave] = am;
    }
    __syncthreads();
    // an Inf or NaN among the column block's v or entering state: the chunked
    // products would carry it into earlier tokens of its chunk (a zero of T
    // times it is NaN), so the block runs token by token, as the recurrence
    // spreads it
    const uint32_t am_all = max(max(sAm[0], sAm[1]), max(sAm[2], sAm[3]));
    if ((sOut[0] | sOut[1] | sOut[2] | sOut[3]) || am_all >= 0x7f800000u) {  // workgroup-uniform
        scan_sequential<BF16>(a, b, h, cb, wave, lane);
        return;
    }
    int pa = 0;  // the power a
    {
        const float m = __uint_as_float(am_all);
        if (m > 0.0f) {
            int ex;
            (void)frexpf(m, &ex);  // m = f 2^ex, f in [0.5, 1)
            pa = min(max(1 - ex, -100), 100);
        }
    }
    const float vscale = __builtin_ldexpf(1.0f, pa), unscale = __builtin_ldexpf(1.0f, -pa);
    const float yscale = a.scale * unscale;
#pragma unroll
    for (int a2 = 0; a2 < 2; ++a2) S[a2] *= vscale;

    // One chunk: C holds its operands (loaded a chunk ahead), the next chunk's
    // operands are loaded into Nx part by part.
    auto chunk = [&](const int nn, ScanOps<BF16, VEC>& C, ScanOps<BF16, VEC>& Nx, _Float16* kth, _Float16* ktl) {
        scan_load<0>(a, b, h, cb, nn + 1, wave, lr, lg, Nx);

        // ---- the wave's K rows -> LDS transposed (the state update's
        //      operands) and, when the scan forms P, as rows (every wave forms
        //      its P from all of them)
        h8 ak[4], aq[4];
        uint4 rk[4], rq[4];  // RAW: the rows as loaded
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if constexpr (RAW) {
                // rows past T are real rows (clamped loads): every product they
                // enter meets a zero T row or column, so they add nothing
                rk[ks] = C.kw[ks][0];
                rq[ks] = C.qw[ks][0];
                *(uint4*)(kth + (16 * wave + lr) * KRP + 32 * ks + 8 * lg) = rk[ks];
                continue;
            }
            ak[ks] = decode8<BF16, VEC>(C.kw[ks], C.ok);
            aq[ks] = decode8<BF16, VEC>(C.qw[ks], C.ok);
            const int ko = (16 * wave + lr) * SP + 32 * ks + 8 * lg;
            *(h8*)(sKh + ko) = ak[ks];
#pragma unroll
            for (int e = 0; e < 8; ++e) kth[(32 * ks + 8 * lg + e) * KTP + 16 * wave + lr] = ak[ks][e];
            if constexpr (!BF16) {
                const h8 al = decode8_lo(C.kw[ks], C.ok);
                *(h8*)(sKl + ko) = al;
#pragma unroll
                for (int e = 0; e < 8; ++e) ktl[(32 * ks + 8 * lg + e) * KTP + 16 * wave + lr] = al[e];
            }
        }

        // ---- S (hi, lo) -> LDS as S^T [c][i]: the B operand rows of K S and Q S
#pragma unroll
        for (int a2 = 0; a2 < 2; ++a2) {
            const int it = 2 * wave + a2;
            if constexpr (RAW) {
                uint2 t3[3];
                split3_x4(S[a2], t3);
                *(uint2*)(sSh + lr * SP + 16 * it + 4 * lg) = t3[0];
                *(uint2*)(sSm + lr * SP + 16 * it + 4 * lg) = t3[1];
                *(uint2*)(sSl + lr * SP + 16 * it + 4 * lg) = t3[2];
                continue;
            }
            h4 sh, sl;
#pragma unroll
            for (int r = 0; r < 4; ++r) sh[r] = f16_hi(S[a2][r]), sl[r] = f16_lo(S[a2][r]);
            *(h4*)(sSh + lr * SP + 16 * it + 4 * lg) = sh;
            *(h4*)(sSl + lr * SP + 16 * it + 4 * lg) = sl;
        }
        __syncthreads();
        scan_load<1>(a, b, h, cb, nn + 1, wave, lr, lg, Nx);

        // ---- K S and Q S for token tile w (16 tokens x 16 columns)
        f4 ksh = f4{0.0f, 0.0f, 0.0f, 0.0f}, ksl = ksh, qsh = ksh, qsl = ksh;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int bo = lr * SP + 32 * ks + 8 * lg;
            if constexpr (RAW) {
                const uint4 b0 = *(const uint4*)(sSh + bo), b1 = *(const uint4*)(sSm + bo),
                            b2 = *(const uint4*)(sSl + bo);
                ksh = mfma_bf(rk[ks], b0, ksh);
                qsh = mfma_bf(rq[ks], b0, qsh);
                ksl = mfma_bf(rk[ks], b1, ksl);
                qsl = mfma_bf(rq[ks], b1, qsl);
                ksl = mfma_bf(rk[ks], b2, ksl);
                qsl = mfma_bf(rq[ks], b2, qsl);
                continue;
            }
            const h8 bh = *(const h8*)(sSh + bo), bl = *(const h8*)(sSl + bo);
            ksh = mfma32(ak[ks], bh, ksh);
            ksl = mfma32(ak[ks], bl, ksl);
            qsh = mfma32(aq[ks], bh, qsh);
            qsl = mfma32(aq[ks], bl, qsl);
            if constexpr (!BF16) {
                ksl = mfma32(decode8_lo(C.kw[ks], C.ok), bh, ksl);
                qsl = mfma32(decode8_lo(C.qw[ks], C.ok), bh, qsl);
            }
        }
        // ---- X = V - e^G (K S) -> LDS as X^T [c][t] (hi, lo); lane: column lr,
        //      tokens 16w + 4lg + r
        f4 QS;
        h4 xh, xl;
        const float egr[4] = {C.eg.x, C.eg.y, C.eg.z, C.eg.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float vv =
                (C.vok >> r) & 1 ? (BF16 ? bf16_bits_to_f32(C.vw[r]) : __uint_as_float(C.vw[r])) * vscale : 0.0f;
            const float x = vv - egr[r] * (ksh[r] + ksl[r]);
            QS[r] = egr[r] * (qsh[r] + qsl[r]);
            xh[r] = f16_hi(x), xl[r] = f16_lo(x);
        }
        *(h4*)(sXh + lr * TP + 16 * wave + 4 * lg) = xh;
        *(h4*)(sXl + lr * TP + 16 * wave + 4 * lg) = xl;

        // ---- P[t][j] = (q_t . k_j) e^{G_t - G_j} (j <= t) for t in the wave's
        //      tile, as P^T = K Q^T per token tile jt <= w: lane (lr, lg) gets
        //      t = 16w + lr, j = 16jt + 4lg + i, which is the A operand layout of
        //      the 16x16x16 product Y += P U below. RAW: the prep formed them
        //      (the same products), so they stay off the step's chain
        h4 ph[4], pl[4];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            ph[jt] = h4{0, 0, 0, 0};
            pl[jt] = ph[jt];
            if constexpr (RAW) {  // the prep's tiles, loaded a chunk ahead
                if (jt > wave) continue;  // wave-uniform
                ph[jt] = __builtin_bit_cast(h4, make_uint2(C.pw[jt].x, C.pw[jt].y));
                pl[jt] = __builtin_bit_cast(h4, make_uint2(C.pw[jt].z, C.pw[jt].w));
            } else {
                if (jt > wave) continue;  // wave-uniform
                f4 pt = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int ko = (16 * jt + lr) * SP + 32 * ks + 8 * lg;
                    const h8 kj = *(const h8*)(sKh + ko);
                    pt = mfma32(kj, aq[ks], pt);
                    if constexpr (!BF16) {
                        pt = mfma32(kj, decode8_lo(C.qw[ks], C.ok), pt);
                        pt = mfma32(*(const h8*)(sKl + ko), aq[ks], pt);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool causal = jt < wave || 4 * lg + i <= lr;
                    const float pv = causal ? pt[i] * __expf(C.gt - C.gj[jt][i]) : 0.0f;
                    ph[jt][i] = f16_hi(pv), pl[jt][i] = f16_lo(pv);
                }
            }
        }
        __syncthreads();
        scan_load<2>(a, b, h, cb, nn + 1, wave, lr, lg, Nx);

        // ---- U = T X for token tile w; U and e^{G_C - G} U -> LDS as [c][t]
        f4 u = f4{0.0f, 0.0f, 0.0f, 0.0f}, u2 = u;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int bo = lr * TP + 32 * ks + 8 * lg;
            const h8 bh = *(const h8*)(sXh + bo), bl = *(const h8*)(sXl + bo);
            u = mfma32(C.th[ks], bh, u);
            u2 = mfma32(C.th[ks], bl, u2);
            u2 = mfma32(C.tl[ks], bh, u2);
        }
        u += u2;
        {
            const float egcr[4] = {C.egc.x, C.egc.y, C.egc.z, C.egc.w};
            h4 uh, ul, wh, wl;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float w = u[r] * egcr[r];
                uh[r] = f16_hi(u[r]), ul[r] = f16_lo(u[r]);
                wh[r] = f16_hi(w), wl[r] = f16_lo(w);
            }
            const int o = lr * TP + 16 * wave + 4 * lg;
            *(h4*)(sUh + o) = uh;
            *(h4*)(sUl + o) = ul;
            if constexpr (RAW) {
                uint2 w3[3];
                split3_x4(f4{u[0] * egcr[0], u[1] * egcr[1], u[2] * egcr[2], u[3] * egcr[3]}, w3);
                *(uint2*)(sWh + o) = w3[0];
                *(uint2*)(sWm + o) = w3[1];
                *(uint2*)(sWl + o) = w3[2];
            } else {
                *(h4*)(sWh + o) = wh;
                *(h4*)(sWl + o) = wl;
            }
        }
        __syncthreads();
        scan_load<3>(a, b, h, cb, nn + 1, wave, lr, lg, Nx);

        // ---- Y = scale (e^G Q S + P U) for token tile w (P is zero past tile w)
        f4 y = QS, y2 = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            if (jt > wave) continue;  // wave-uniform
            const int bo = lr * TP + 16 * jt + 4 * lg;
            const h4 bh = *(const h4*)(sUh + bo), bl = *(const h4*)(sUl + bo);
            y = mfma16(ph[jt], bh, y);
            y2 = mfma16(ph[jt], bl, y2);
            y2 = mfma16(pl[jt], bh, y2);
        }
        y += y2;
        if constexpr (RAW) {
            // through a buffer resource over the chunk's output rows: the
            // (head, column block) part of the offset in an SGPR, the lane's
            // token and column in one VGPR. Non-temporal when the scan runs one
            // workgroup per CU (nothing here reads the outputs again, and the
            // operands keep the L2); with two per CU (several sequences) the
            // column blocks' partial lines merge better in L2
            const __amdgpu_buffer_rsrc_t r =
                __builtin_amdgcn_make_buffer_rsrc((void*)(out + (int64_t)nn * kChunk * 4096), (short)0, 0x7fffffff, 0x00020000);
            const uint32_t so = 4u * (uint32_t)(h * 128 + kCols * cb);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int tl = 16 * wave + 4 * lg + q;  // token within the chunk
                if (nn * kChunk + tl < a.T) {
                    const uint32_t yv = __builtin_bit_cast(uint32_t, y[q] * yscale), vo = (uint32_t)tl * 16384u + 4u * (uint32_t)lr;
                    __builtin_amdgcn_raw_buffer_store_b32(yv, r, vo, so, NTY ? 2 : 0);
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int t = nn * kChunk + 16 * wave + 4 * lg + q;
                if (t < a.T) {
                    float* o = out + (int64_t)t * 4096 + h * 128 + kCols * cb + lr;
                    if constexpr (NTY)
                        __builtin_nontemporal_store(y[q] * yscale, o);
                    else
                        *o = y[q] * yscale;
                }
            }
        }

        // ---- S = e^{G_C} S + K^T (e^{G_C - G} U) for this wave's key-dim tiles
        if constexpr (RAW) {  // the three bf16 terms of (e^{G_C - G} U)^T read once for both tiles
            uint4 bw[2][3];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int bo = lr * TP + 32 * ks + 8 * lg;
                bw[ks][0] = *(const uint4*)(sWh + bo);
                bw[ks][1] = *(const uint4*)(sWm + bo);
                bw[ks][2] = *(const uint4*)(sWl + bo);
            }
#pragma unroll
            for (int a2 = 0; a2 < 2; ++a2) {
                f4 acc = S[a2] * C.eGC, acc2 = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    // K^T[16 it + lr][32 ks + 8 lg + j], j = 0..7: the 4 x 16 blocks
                    // at tokens 32 ks + 8 lg (+ 4), key dims 16 it ..
                    const _Float16* kb = kth + (32 * ks + 8 * lg + (lr >> 2)) * KRP + 16 * (2 * wave + a2) + 4 * (lr & 3);
                    const uint2 k0 = lds_read_tr16(kb), k1 = lds_read_tr16(kb + 4 * KRP);
                    const uint4 kt = make_uint4(k0.x, k0.y, k1.x, k1.y);
                    acc = mfma_bf(kt, bw[ks][0], acc);
                    acc2 = mfma_bf(kt, bw[ks][1], acc2);
                    acc2 = mfma_bf(kt, bw[ks][2], acc2);
                }
                S[a2] = acc + acc2;
            }
            return;
        }
#pragma unroll
        for (int a2 = 0; a2 < 2; ++a2) {
            f4 acc = S[a2] * C.eGC, acc2 = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int bo = lr * TP + 32 * ks + 8 * lg;
                const int ko = (16 * (2 * wave + a2) + lr) * KTP + 32 * ks + 8 * lg;
                const h8 wh = *(const h8*)(sWh + bo), kt = *(const h8*)(kth + ko);
                acc = mfma32(kt, wh, acc);
                acc2 = mfma32(kt, *(const h8*)(sWl + bo), acc2);
                if constexpr (!BF16) acc2 = mfma32(*(const h8*)(ktl + ko), wh, acc2);
            }
            S[a2] = acc + acc2;
        }
    };
    // Chunk pairs in the loop (the two operand sets stay in fixed registers)
    // and an odd last chunk after it: no path leaves the loop body midway, so
    // the compiler's wait placement sees the same outstanding loads on every
    // iteration and never waits for the next chunk's operands early.
    int n = 0;
    for (; n + 1 < a.n_chunks; n += 2) {
        chunk(n, ops[0], ops[1], sKTh[0], sKTl[0]);
        chunk(n + 1, ops[1], ops[0], sKTh[1], sKTl[1]);
    }
    if (n < a.n_chunks) chunk(n, ops[0], ops[1], sKTh[0], sKTl[0]);

    // ---- final state (transposed layout: element (i, c) of head h at h*16384 + c*128 + i)
    float* so = a.state_out + (int64_t)b * (a.so_nb3 / 4) + (int64_t)h * 16384;
#pragma unroll
    for (int a2 = 0; a2 < 2; ++a2) {
        const int it = 2 * wave + a2;
        *(float4*)(so + (int64_t)(kCols * cb + lr) * 128 + 16 * it + 4 * lg) =
            make_float4(S[a2][0] * unscale, S[a2][1] * unscale, S[a2][2] * unscale, S[a2][3] * unscale);
    }
}

// ---------------------------------------------------------------- host

static int64_t chunked_tokens(int64_t T, int32_t slots) { return slots > 1 ? T - (slots - 1) : T; }

size_t gdn_chunked_workspace_bytes(int64_t T, int64_t B, int32_t slots, bool bf16_rows) {
    const int64_t Tc = chunked_tokens(T, slots);
    if (Tc < 1) return 0;
    const int64_t nch = (Tc + kChunk - 1) / kChunk;
    (void)bf16_rows;  // the record holds f16 planes whatever the row type
    return (size_t)B * 32 * nch * kRecBytes;
}

bool gdn_chunked_available() { return true; }

template <bool BF16, bool VEC>
static void chunked_kernels(const GdnChunkArgs& a, hipStream_t stream) {
    launch("gdn_chunk_prep", gdn_chunk_prep<BF16, VEC>, dim3(16, a.n_chunks, (uint32_t)a.B), dim3(256), stream, a);
    // one sequence: one scan workgroup per CU, non-temporal output stores
    const uint32_t n_wg = (uint32_t)a.B * 32 * kColBlocks;
    if (n_wg <= 256)
        launch("gdn_chunk_scan", gdn_chunk_scan<BF16, VEC, true>, dim3(n_wg), dim3(256), stream, a);
    else
        launch("gdn_chunk_scan", gdn_chunk_scan<BF16, VEC, false>, dim3(n_wg), dim3(256), stream, a);
}

hipError_t gdn_chunked_launch(const GdnLaunch& L, hipStream_t stream) {
    const int64_t T = L.v->ne[2], B = L.v->ne[3];
    const int64_t Tc = chunked_tokens(T, L.slots);
    if (Tc < 1) return gdn_step_launch(L, stream);  // every token needs its own snapshot
    // the scan addresses a chunk's rows with 32-bit offsets from the chunk's first
    // row: row strides of 2^25 bytes or more run token by token instead
    for (const xq_tensor* t : {L.q, L.k, L.v})
        if (t->nb[2] >= ((int64_t)1 << 25)) return gdn_step_launch(L, stream);
    if (L.workspace_bytes < gdn_chunked_workspace_bytes(T, B, L.slots, L.q->type == XQ_TYPE_BF16))
        return hipErrorInvalidValue;
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
    a.B = (int32_t)B;
    a.scale = 1.0f / sqrtf(128.0f);
    const bool bf16 = L.q->type == XQ_TYPE_BF16;
    // 16-byte row loads need 16-byte aligned q/k row bases
    bool vec = true;
    for (const xq_tensor* t : {L.q, L.k}) {
        vec = vec && ((uintptr_t)t->data % 16 == 0);
        for (int i = 1; i < 4; ++i) vec = vec && (t->nb[i] % 16 == 0);
    }
    if (bf16) {
        if (vec) chunked_kernels<true, true>(a, stream);
        else chunked_kernels<true, false>(a, stream);
    } else {
        if (vec) chunked_kernels<false, true>(a, stream);
        else chunked_kernels<false, false>(a, stream);
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
