// xq_fa_mma.hip — FLASH_ATTN_EXT pass 1 on the gfx950 matrix cores.
//
// Same work decomposition and outputs as the VALU pass 1 in xq_fa.hip (one
// workgroup per (sequence, KV head, query tile, KV split), 64-row tiles,
// partial (acc, m, l) per split or the final output for one split) with both
// products on MFMA:
//   scores  q8_0 / q4_0 K: v_mfma_i32_16x16x32_i8 per 32-element block, i.e.
//           the exact integer block dot of ggml's vec_dot_q8_0_q8_0 /
//           vec_dot_q4_0_q8_0 between the q8_0-quantised Q row and the K
//           block (q4_0 nibbles enter unsigned; 8*sum(q) is subtracted in
//           integers), then scaled by d_k*d_q in f32;
//           F16 / E5M2 K: v_mfma_f32_16x16x32_f16 on the exactly-converted K
//           with Q split into f16 hi + lo parts (f32 Q to ~22 bits; the
//           NATIVE policy uses the f16-rounded Q alone);
//   values  v_mfma_f32_16x16x32_f16 with V exactly converted to f16 (int8 /
//           nibble values via the 0x6400 exponent trick, E5M2 by a byte
//           shift) and the softmax weights times the block scale rounded to
//           f16 as the other operand; f32 accumulation.
// The M dimension of both products is the (query, head) pair index (16 per
// MFMA tile, up to two tiles); N is 16 KV rows (scores, one wave per 16 rows)
// or 16 head dims (values, each wave a quarter of the head). K/V tiles move
// HBM -> LDS with global_load_lds (16-byte or 4-byte per lane), double
// buffered so the next tile streams in while the current one is computed.
// Online softmax: per-pair maxima and sums over each wave's 16 rows by DPP
// inside 16-lane rows, combined across the four waves through LDS in a fixed
// order.
#include "xq_fa_common.h"

namespace xq {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i4 __attribute__((ext_vector_type(4)));

constexpr bool is_quant(int kt) { return kt == XQ_TYPE_Q8_0 || kt == XQ_TYPE_Q4_0; }

// Bytes of one Q image row for the matrix-core engine.
//   q8_0 / q4_0 K: int8 q[D] (ggml quantize_row_q8_0 of the row), f32 d[D/32],
//                  int32 sum(q)[D/32];
//   F16 / E5M2 K:  f16 hi[D], f16 lo[D] with hi = f16(q), lo = f16(q - hi).
constexpr int mma_qrow_bytes(int kt, int d) { return is_quant(kt) ? d + 8 * (d / kQK) : 4 * d; }

template <int KT, int D>
__global__ __launch_bounds__(64) void fa_qprep_mma(const uint8_t* __restrict__ q, int64_t nb1, int64_t nb2,
                                                    int64_t nb3, int NQ, int H, int hi_only,
                                                    uint8_t* __restrict__ img_out) {
    constexpr int QRB = mma_qrow_bytes(KT, D);
    const int64_t row = blockIdx.x;
    const int h = (int)(row % H);
    const int iq = (int)((row / H) % NQ);
    const int b = (int)(row / ((int64_t)H * NQ));
    const float* src = (const float*)(q + (int64_t)b * nb3 + (int64_t)iq * nb1 + (int64_t)h * nb2);
    uint8_t* img = img_out + row * QRB;
    const int lane = threadIdx.x;
    if constexpr (is_quant(KT)) {
        constexpr int VD = D / 64;
        constexpr int LPB = kQK / VD;
        float x[VD];
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < VD; ++j) {
            x[j] = src[lane * VD + j];
            amax = fmaxf(amax, fabsf(x[j]));
        }
        amax = fmaxf(amax, dpp<0xB1>(amax));
        amax = fmaxf(amax, dpp<0x4E>(amax));
        amax = fmaxf(amax, dpp<0x141>(amax));
        if constexpr (LPB == 16) amax = fmaxf(amax, dpp<0x140>(amax));
        // ggml-cpu x86 quantize_row_q8_0: d = amax/127, id = 127/amax, round half to even
        const float dblk = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        uint32_t packed = 0;
        int qsum = 0;
#pragma unroll
        for (int j = 0; j < VD; ++j) {
            const int qv = (int)rintf(x[j] * id);
            packed |= (uint32_t)(uint8_t)(int8_t)qv << (8 * j);
            qsum += qv;
        }
        if constexpr (VD == 4)
            *(uint32_t*)(img + 4 * lane) = packed;
        else
            *(uint16_t*)(img + 2 * lane) = (uint16_t)packed;
        float qs = (float)qsum;  // exact: |sum| <= 32*127
        qs += dpp<0xB1>(qs);
        qs += dpp<0x4E>(qs);
        qs += dpp<0x141>(qs);
        if constexpr (LPB == 16) qs += dpp<0x140>(qs);
        const int blk = (lane * VD) / kQK;
        if ((lane % LPB) == 0) {
            ((float*)(img + D))[blk] = f16_bits_to_f32(f32_to_f16_bits(dblk));
            ((int*)(img + D + 4 * (D / kQK)))[blk] = (int)qs;
        }
    } else {
        uint16_t* hi = (uint16_t*)img;
        uint16_t* lo = hi + D;
        for (int e = lane; e < D; e += 64) {
            const float x = src[e];
            const uint32_t hb = f32_to_f16_bits(x);
            hi[e] = (uint16_t)hb;
            lo[e] = hi_only ? (uint16_t)0 : (uint16_t)f32_to_f16_bits(x - f16_bits_to_f32(hb));
        }
    }
}

// 8 K bytes (elements 8g..8g+7 of block b) of a q8_0 / q4_0 record in LDS as
// the int8 B operand of v_mfma_i32_16x16x32_i8. q4_0 gives unsigned nibbles.
template <int KT>
XQ_DEV int64_t k_block_bytes(const uint8_t* rec, int b, int g) {
    constexpr int BB = KT == XQ_TYPE_Q8_0 ? 34 : 18;
    const int off = KT == XQ_TYPE_Q8_0 ? BB * b + 2 + 8 * g : BB * b + 2 + 8 * (g & 1);
    const int sh = (BB * b + 2) & 3;  // 0 or 2 for every g: depends on b only
    uint32_t w0, w1;
    if (sh == 0) {
        w0 = lds_u32(rec + off);
        w1 = lds_u32(rec + off + 4);
    } else {
        const uint32_t a = lds_u32(rec + off - 2), m = lds_u32(rec + off + 2), c = lds_u32(rec + off + 6);
        w0 = __builtin_amdgcn_alignbyte(m, a, 2);
        w1 = __builtin_amdgcn_alignbyte(c, m, 2);
    }
    if constexpr (KT == XQ_TYPE_Q4_0) {
        const int ns = (g >> 1) * 4;  // lane groups 2, 3 take the high nibbles
        w0 = (w0 >> ns) & 0x0f0f0f0fu;
        w1 = (w1 >> ns) & 0x0f0f0f0fu;
    }
    return (int64_t)(((uint64_t)w1 << 32) | w0);
}

// Four f16x2 words: rows (2e, 2e+1) of one V dim column, for e = 0..3, from
// the two "dim pair" words X[e] = rowpair bytes. Exact conversions.
template <int KT>
XQ_DEV void v_pairs_to_f16(const uint32_t (&X)[4], int t, uint32_t (&out)[4]) {
    if constexpr (KT == XQ_TYPE_Q8_0 || KT == XQ_TYPE_Q4_0) {
        // q8_0: byte u = q ^ 0x80 gives f16(0x6400 | u) = 1024 + q + 128;
        // q4_0: byte u = nibble gives 1024 + nibble; subtract 1152 / 1032.
        const uint32_t sel = t == 0 ? 0x04020400u : 0x04030401u;
        const _Float16 bias = KT == XQ_TYPE_Q8_0 ? (_Float16)-1152.0f : (_Float16)-1032.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t w = __builtin_amdgcn_perm(0x64646464u, X[e], sel);
            h2 v = __builtin_bit_cast(h2, w);
            v = v + h2{bias, bias};
            out[e] = __builtin_bit_cast(uint32_t, v);
        }
    } else if constexpr (KT == XQ_TYPE_E5M2) {
        const uint32_t sel = t == 0 ? 0x020c000cu : 0x030c010cu;
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = __builtin_amdgcn_perm(X[e], X[e], sel);
    }
}

// HBM -> LDS without registers: lane l's CS bytes land at lds + l*CS
// (global_load_lds_dwordx4 / _dword). lds must be wave-uniform.
template <int CS>
XQ_DEV void lds_dma(const uint8_t* g, uint8_t* lds) {
    // the size operand must be a literal (the builtin rejects dependent values)
    if constexpr (CS == 16)
        __builtin_amdgcn_global_load_lds((const void*)g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
    else
        __builtin_amdgcn_global_load_lds((const void*)g, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}

// Each wave streams its own 16-row slices of the split (slice j of the split
// goes to wave j % 4) through a private double-buffered LDS region, with a
// private online softmax; the four wave states are merged once at the end in
// wave order. No workgroup barrier inside the row loop.
template <int KT, int D, int MT>
__global__ __launch_bounds__(kThreads) void fa_mma_pass1(FaArgs a, const uint8_t* __restrict__ qimg,
                                                          int hi_only) {
    constexpr int SUB = 16;                          // rows per wave slice
    constexpr int REC = rec_bytes(KT, D);
    constexpr int CS = REC % 16 == 0 ? 16 : 4;       // bytes per lane per global_load_lds
    constexpr int CPS = SUB * REC / CS;              // chunks per slice per tensor
    constexpr int NIS = (CPS + 63) / 64;             // wave loads per slice per tensor
    constexpr int NB = D / kQK;                      // 32-element blocks per row
    constexpr int QRB = mma_qrow_bytes(KT, D);
    constexpr int NPP = 16 * MT;
    constexpr bool QUANT = is_quant(KT);
    constexpr int SPS = SUB + 4;                     // weight transpose stride (conflict-free)
    constexpr int SLICE = SUB * REC;

    // per wave: K/V double buffers, weight transpose, V block scales. The K/V
    // region doubles as the buffer of the final wave merge (2 waves x pairs x D).
    constexpr int KV_BYTES = 4 * 2 * 2 * SLICE;
    constexpr int MERGE_BYTES = 2 * NPP * D * 4;
    __shared__ __attribute__((aligned(16))) uint8_t smem[KV_BYTES > MERGE_BYTES ? KV_BYTES : MERGE_BYTES];
    typedef uint8_t SliceBuf[2][2][SLICE];
    SliceBuf* sKV = (SliceBuf*)smem;
    __shared__ __attribute__((aligned(16))) float sPw[4][NPP * SPS];
    __shared__ __attribute__((aligned(16))) float sDv[4][QUANT ? NB * SUB : 4];
    __shared__ __attribute__((aligned(16))) float sQd[QUANT ? NB * NPP : 4];  // d_q [blk][pair]
    __shared__ __attribute__((aligned(16))) int sQs[QUANT ? NB * NPP : 4];    // sum q [blk][pair]
    __shared__ float sML[2][NPP][2];

    const uint32_t n_wg = (uint32_t)a.n_splits * a.n_qtiles * a.Hkv * a.B;
    uint32_t wg = xcd_remap(blockIdx.x, n_wg);
    const int qt = wg % a.n_qtiles;
    wg /= a.n_qtiles;
    const int split = wg % a.n_splits;
    wg /= a.n_splits;
    const int g_kv = wg % a.Hkv;
    const int b = wg / a.Hkv;
    const int iq0 = qt * a.QT;
    const int nqt = min(a.QT, a.NQ - iq0);
    const int npa = nqt * a.G;
    const int wave = wave_id();
    const int lane = lane_id();
    const int tid = threadIdx.x;
    const int lr = lane & 15;
    const int lg = lane >> 4;

    const int64_t r0 = (int64_t)split * a.split_rows;
    int64_t r_end = min(a.L, r0 + a.split_rows);
    if (a.positions) {
        int64_t lim_max = 0;
        for (int qq = 0; qq < nqt; ++qq) {
            const int32_t pos = a.positions[iq0 + qq];
            const int64_t causal = pos < a.origin ? 0 : (int64_t)pos - a.origin + 1;
            lim_max = max(lim_max, min(a.L, causal));
        }
        r_end = min(r_end, lim_max);
    }
    const uint8_t* kb = a.k + (int64_t)(b / a.rk3) * a.k_nb3 + (int64_t)g_kv * a.k_nb2;
    const uint8_t* vb = a.v + (int64_t)(b / a.rv3) * a.v_nb3 + (int64_t)g_kv * a.v_nb2;
    const int64_t rows_per_seq = (int64_t)a.NQ * a.H;

    // ---- per-pair state for this lane's MFMA rows (pairs 16m + 4lg + i)
    float m_run[MT][4], l_run[MT][4];
    int64_t lim[MT][4];
    const uint16_t* mrow[MT][4];
    float slope[MT][4];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            m_run[m][i] = -INFINITY;
            l_run[m][i] = 0.0f;
            const int p = 16 * m + 4 * lg + i;
            lim[m][i] = -1;  // padding pair: never valid
            mrow[m][i] = nullptr;
            slope[m][i] = 0.0f;
            if (p < npa) {
                const int qq = p / a.G, h = g_kv * a.G + p % a.G;
                lim[m][i] = a.L;
                if (a.positions) {
                    const int32_t pos = a.positions[iq0 + qq];
                    const int64_t causal = pos < a.origin ? 0 : (int64_t)pos - a.origin + 1;
                    lim[m][i] = min(a.L, causal);
                }
                if (a.mask) {
                    mrow[m][i] = (const uint16_t*)(a.mask + (int64_t)(iq0 + qq) * a.m_nb1 +
                                                   (int64_t)(h % a.m_ne2) * a.m_nb2 + (int64_t)(b % a.m_ne3) * a.m_nb3);
                    slope[m][i] = alibi_slope(a, h);
                }
            }
        }

    // ---- Q operands (A of the score MFMA): pair 16m + lr, elements 8lg..8lg+7 of each block
    auto img_of = [&](int p) -> const uint8_t* {
        const int qq = p / a.G, h = g_kv * a.G + p % a.G;
        return qimg + ((int64_t)(b * a.NQ + iq0 + qq) * a.H + h) * QRB;
    };
    int64_t qa[QUANT ? MT : 1][QUANT ? NB : 1];
    h8 qh[QUANT ? 1 : MT][QUANT ? 1 : NB], ql[QUANT ? 1 : MT][QUANT ? 1 : NB];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int p = 16 * m + lr;
        const bool ok = p < npa;
        const uint8_t* im = ok ? img_of(p) : qimg;
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            if constexpr (QUANT) {
                qa[m][c] = ok ? *(const int64_t*)(im + 32 * c + 8 * lg) : 0;
            } else {
                const h8 z = {0, 0, 0, 0, 0, 0, 0, 0};
                qh[m][c] = ok ? *(const h8*)(im + 2 * (32 * c + 8 * lg)) : z;
                ql[m][c] = ok ? *(const h8*)(im + 2 * D + 2 * (32 * c + 8 * lg)) : z;
            }
        }
    }
    if constexpr (QUANT) {
        for (int e = tid; e < NB * NPP; e += kThreads) {
            const int c = e / NPP, p = e % NPP;
            float dq = 0.0f;
            int sq = 0;
            if (p < npa) {
                const uint8_t* im = img_of(p);
                dq = ((const float*)(im + D))[c];
                sq = ((const int*)(im + D + 4 * NB))[c];
            }
            sQd[e] = dq;
            sQs[e] = sq;
        }
    }
    __syncthreads();

    // ---- this wave's slices: t0 = r0 + SUB*(wave + 4*j)
    // Chunk c = 64*i + lane of a slice is (row c / (REC/CS), byte (c % (REC/CS))*CS).
    int64_t koff[NIS], voff[NIS];
    int crow[NIS];
#pragma unroll
    for (int i = 0; i < NIS; ++i) {
        const int c = i * 64 + lane;
        crow[i] = c / (REC / CS);
        koff[i] = (int64_t)crow[i] * a.k_nb1 + (c % (REC / CS)) * CS;
        voff[i] = (int64_t)crow[i] * a.v_nb1 + (c % (REC / CS)) * CS;
    }
    auto stage = [&](int64_t t0, int bf) {
        const bool full = t0 + SUB <= r_end;
        const uint8_t* kt = kb + t0 * a.k_nb1;
        const uint8_t* vt = vb + t0 * a.v_nb1;
        uint8_t* lk = sKV[wave][bf][0];
        uint8_t* lv = sKV[wave][bf][1];
#pragma unroll
        for (int i = 0; i < NIS; ++i) {
            int64_t ko = koff[i], vo = voff[i];
            if (!full && t0 + crow[i] >= r_end) {  // rows past the split end reuse the last live row
                const int64_t dr = t0 + crow[i] - (r_end - 1);
                ko -= dr * a.k_nb1;
                vo -= dr * a.v_nb1;
            }
            if (CPS % 64 == 0 || i + 1 < NIS || lane < CPS % 64) {
                lds_dma<CS>(kt + ko, lk + i * 64 * CS);
                lds_dma<CS>(vt + vo, lv + i * 64 * CS);
            }
        }
    };

    f4 acc[MT][2 * NB];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < 2 * NB; ++n) acc[m][n] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    float* pw = sPw[wave];
    float* dvw = sDv[wave];
    int bf = 0;
    int64_t t0 = r0 + SUB * wave;
    if (t0 < r_end) stage(t0, 0);
    for (; t0 < r_end; t0 += 4 * SUB, bf ^= 1) {
        const int64_t tn = t0 + 4 * SUB;
        // mask values of this slice (the lane's row lr), issued before the wait
        float mv[MT][4];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                mv[m][i] = (mrow[m][i] && t0 + lr < r_end) ? slope[m][i] * f16_bits_to_f32(mrow[m][i][t0 + lr]) : 0.0f;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_wave_barrier();
        if (tn < r_end) stage(tn, bf ^ 1);
        const uint8_t* K = sKV[wave][bf][0];
        const uint8_t* V = sKV[wave][bf][1];
        const uint8_t* krec = K + lr * REC;

        // ---- scores: pairs x 16 rows
        float s[MT][4];
        if constexpr (QUANT) {
            constexpr int BB = KT == XQ_TYPE_Q8_0 ? 34 : 18;
            i4 I[MT][NB];
            float dk[NB];
#pragma unroll
            for (int c = 0; c < NB; ++c) {
                const int64_t kop = k_block_bytes<KT>(krec, c, lg);
                dk[c] = f16_bits_to_f32(lds_u16(krec + BB * c));
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const i4 z = {0, 0, 0, 0};
                    I[m][c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa[m][c], kop, z, 0, 0, 0);
                }
            }
            // V block scales of this slice (rows 0..15), written for the value step
#pragma unroll
            for (int j = 0; j < NB * SUB / 64; ++j) {
                const int e = lane + 64 * j;
                const int c = e / SUB, r = e % SUB;
                dvw[e] = f16_bits_to_f32(lds_u16(V + r * REC + BB * c));
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
#pragma unroll
                for (int i = 0; i < 4; ++i) s[m][i] = 0.0f;
#pragma unroll
                for (int c = 0; c < NB; ++c) {
                    const f4 dq = *(const f4*)(sQd + c * NPP + 16 * m + 4 * lg);
                    i4 sq4 = {0, 0, 0, 0};
                    if constexpr (KT == XQ_TYPE_Q4_0) sq4 = *(const i4*)(sQs + c * NPP + 16 * m + 4 * lg);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        int ii = I[m][c][i];
                        if constexpr (KT == XQ_TYPE_Q4_0) ii -= 8 * sq4[i];
                        s[m][i] = fmaf((float)ii, dk[c] * dq[i], s[m][i]);
                    }
                }
            }
        } else {
            f4 sc[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) sc[m] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < NB; ++c) {
                h8 kop;
                if constexpr (KT == XQ_TYPE_F16) {
                    kop = *(const h8*)(krec + 64 * c + 16 * lg);
                } else {  // E5M2: byte b -> f16 bits b << 8
                    const uint2 w = *(const uint2*)(krec + 32 * c + 8 * lg);
                    const uint4 hv = {__builtin_amdgcn_perm(w.x, w.x, 0x010c000cu), __builtin_amdgcn_perm(w.x, w.x, 0x030c020cu),
                                      __builtin_amdgcn_perm(w.y, w.y, 0x010c000cu), __builtin_amdgcn_perm(w.y, w.y, 0x030c020cu)};
                    kop = __builtin_bit_cast(h8, hv);
                }
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    sc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[m][c], kop, sc[m], 0, 0, 0);
                    if (!hi_only) sc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[m][c], kop, sc[m], 0, 0, 0);
                }
            }
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[m][i] = sc[m][i];
        }

        // ---- online softmax over this slice (rows t0 + lr), per pair
        const int64_t arow = t0 + lr;
        bool moved = false;
        float alpha[MT][4];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = 16 * m + 4 * lg + i;
                float x = s[m][i] * a.scale;
                if (a.softcap != 0.0f) x = a.softcap * tanhf(x);
                const bool valid = arow < r_end && arow < lim[m][i] && mv[m][i] != -INFINITY;
                x = valid ? x + mv[m][i] : -INFINITY;
                const float m_new = fmaxf(m_run[m][i], row16_max_ord(x));
                alpha[m][i] = m_new == -INFINITY ? 1.0f : fast_exp(m_run[m][i] - m_new);
                const float pr = x == -INFINITY ? 0.0f : fast_exp(x - m_new);
                moved |= alpha[m][i] != 1.0f;
                m_run[m][i] = m_new;
                l_run[m][i] = fmaf(l_run[m][i], alpha[m][i], row16_sum(pr));
                pw[p * SPS + lr] = pr;  // transpose through LDS: [pair][row]
            }
        if (__builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int n = 0; n < 2 * NB; ++n)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[m][n][i] *= alpha[m][i];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // ---- values: A = weights of pair 16m + lr at rows 4lg..4lg+3 (x V block scale),
        //      B = V rows 4lg..4lg+3 at dims 32*blk + 2*lr + t
        f4 pv[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) pv[m] = *(const f4*)(pw + (16 * m + lr) * SPS + 4 * lg);
#pragma unroll
        for (int blk = 0; blk < NB; ++blk) {
            f4 d4 = f4{1.0f, 1.0f, 1.0f, 1.0f};
            if constexpr (QUANT) d4 = *(const f4*)(dvw + blk * SUB + 4 * lg);
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            h4 A[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const f4 x = pv[m] * d4;
                A[m] = h4{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
            }
            uint32_t T0[2], T1[2];
            if constexpr (KT == XQ_TYPE_F16) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint32_t wa = lds_u32(V + (4 * lg + 2 * e) * REC + 64 * blk + 4 * lr);
                    const uint32_t wb2 = lds_u32(V + (4 * lg + 2 * e + 1) * REC + 64 * blk + 4 * lr);
                    T0[e] = __builtin_amdgcn_perm(wb2, wa, 0x05040100u);
                    T1[e] = __builtin_amdgcn_perm(wb2, wa, 0x07060302u);
                }
            } else {
                int off;
                if constexpr (KT == XQ_TYPE_Q8_0) off = 34 * blk + 2 + 2 * lr;
                else if constexpr (KT == XQ_TYPE_Q4_0) off = 18 * blk + 2 + 2 * (lr & 7);
                else off = 32 * blk + 2 * lr;
                uint32_t X[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint32_t ua = lds_u16(V + (4 * lg + 2 * e) * REC + off);
                    const uint32_t ub = lds_u16(V + (4 * lg + 2 * e + 1) * REC + off);
                    uint32_t x = ua | (ub << 16);
                    if constexpr (KT == XQ_TYPE_Q8_0) x ^= 0x80808080u;
                    if constexpr (KT == XQ_TYPE_Q4_0) x = (x >> ((lr >> 3) * 4)) & 0x0f0f0f0fu;
                    X[e] = x;
                }
                if constexpr (KT == XQ_TYPE_E5M2) {
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        T0[e] = __builtin_amdgcn_perm(X[e], X[e], 0x020c000cu);
                        T1[e] = __builtin_amdgcn_perm(X[e], X[e], 0x030c010cu);
                    }
                } else {
                    const _Float16 bias = KT == XQ_TYPE_Q8_0 ? (_Float16)-1152.0f : (_Float16)-1032.0f;
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        h2 v0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, X[e], 0x04020400u));
                        h2 v1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, X[e], 0x04030401u));
                        v0 = v0 + h2{bias, bias};
                        v1 = v1 + h2{bias, bias};
                        T0[e] = __builtin_bit_cast(uint32_t, v0);
                        T1[e] = __builtin_bit_cast(uint32_t, v1);
                    }
                }
            }
            typedef _Float16 h4t __attribute__((ext_vector_type(4)));
            const h4t B0 = __builtin_bit_cast(h4t, uint2{T0[0], T0[1]});
            const h4t B1 = __builtin_bit_cast(h4t, uint2{T1[0], T1[1]});
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                acc[m][2 * blk] = __builtin_amdgcn_mfma_f32_16x16x16f16(A[m], B0, acc[m][2 * blk], 0, 0, 0);
                acc[m][2 * blk + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A[m], B1, acc[m][2 * blk + 1], 0, 0, 0);
            }
        }
        __builtin_amdgcn_wave_barrier();  // pw / dvw reads done before the next slice writes them
    }

    // ---- merge the wave states: (w0 + w2) + (w1 + w3), a fixed order. Partner
    //      wave states go through LDS in the MFMA layout of the accumulators.
    float* mo = (float*)smem;  // [2][NPP][D]
    auto publish = [&](int slot) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = 16 * m + 4 * lg + i;
                if (lr == 0) {
                    sML[slot][p][0] = m_run[m][i];
                    sML[slot][p][1] = l_run[m][i];
                }
#pragma unroll
                for (int blk = 0; blk < NB; ++blk)
                    *(float2*)(mo + (slot * NPP + p) * D + 32 * blk + 2 * lr) =
                        make_float2(acc[m][2 * blk][i], acc[m][2 * blk + 1][i]);
            }
    };
    auto absorb = [&](int slot) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = 16 * m + 4 * lg + i;
                const float mp = sML[slot][p][0], lp = sML[slot][p][1];
                const float M = fmaxf(m_run[m][i], mp);
                const float fo = M == -INFINITY ? 0.0f : fast_exp(m_run[m][i] - M);
                const float fp = M == -INFINITY ? 0.0f : fast_exp(mp - M);
                l_run[m][i] = fmaf(l_run[m][i], fo, lp * fp);
                m_run[m][i] = M;
#pragma unroll
                for (int blk = 0; blk < NB; ++blk) {
                    const float2 o = *(const float2*)(mo + (slot * NPP + p) * D + 32 * blk + 2 * lr);
                    acc[m][2 * blk][i] = fmaf(acc[m][2 * blk][i], fo, o.x * fp);
                    acc[m][2 * blk + 1][i] = fmaf(acc[m][2 * blk + 1][i], fo, o.y * fp);
                }
            }
    };
    __syncthreads();  // every wave's slices done: the K/V region is free
    if (wave >= 2) publish(wave - 2);
    __syncthreads();
    if (wave < 2) absorb(wave);
    __syncthreads();
    if (wave == 1) publish(0);
    __syncthreads();
    if (wave == 0) {
        absorb(0);
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = 16 * m + 4 * lg + i;
                if (p >= npa) continue;
                const int qq = p / a.G, h = g_kv * a.G + p % a.G, iq = iq0 + qq;
                const int64_t row = (int64_t)b * rows_per_seq + (int64_t)iq * a.H + h;
                if (a.n_splits == 1) {
                    float a1, inv, l;
                    fa_finalize(m_run[m][i], l_run[m][i], a.sinks != nullptr, a.sinks ? a.sinks[h] : 0.0f, a1, inv, l);
                    float* o = (float*)(a.dst + (int64_t)b * a.d_nb3 + (int64_t)iq * a.d_nb2 + (int64_t)h * a.d_nb1);
#pragma unroll
                    for (int blk = 0; blk < NB; ++blk)
                        *(float2*)(o + 32 * blk + 2 * lr) = make_float2((acc[m][2 * blk][i] * a1) * inv,
                                                                         (acc[m][2 * blk + 1][i] * a1) * inv);
                    if (lr == 0 && a.lse) a.lse[row] = l;
                } else {
                    float* o = a.part_o + (row * a.n_splits + split) * D;
#pragma unroll
                    for (int blk = 0; blk < NB; ++blk)
                        *(float2*)(o + 32 * blk + 2 * lr) = make_float2(acc[m][2 * blk][i], acc[m][2 * blk + 1][i]);
                    if (lr == 0) a.part_ml[row * a.n_splits + split] = make_float2(m_run[m][i], l_run[m][i]);
                }
            }
    }
}

// ---------------------------------------------------------------- dispatch

using MmaPass1Fn = void (*)(FaArgs, const uint8_t*, int);
using MmaQprepFn = void (*)(const uint8_t*, int64_t, int64_t, int64_t, int, int, int, uint8_t*);

template <int KT, int D>
static MmaPass1Fn mma_for(int mt) {
    return mt == 1 ? fa_mma_pass1<KT, D, 1> : mt == 2 ? fa_mma_pass1<KT, D, 2> : nullptr;
}

static MmaPass1Fn mma_lookup(int kt, int d, int mt) {
    if (d == 128) {
        switch (kt) {
        case XQ_TYPE_Q8_0: return mma_for<XQ_TYPE_Q8_0, 128>(mt);
        case XQ_TYPE_Q4_0: return mma_for<XQ_TYPE_Q4_0, 128>(mt);
        case XQ_TYPE_F16: return mma_for<XQ_TYPE_F16, 128>(mt);
        case XQ_TYPE_E5M2: return mma_for<XQ_TYPE_E5M2, 128>(mt);
        }
    } else if (d == 256) {
        switch (kt) {
        case XQ_TYPE_Q8_0: return mma_for<XQ_TYPE_Q8_0, 256>(mt);
        case XQ_TYPE_Q4_0: return mma_for<XQ_TYPE_Q4_0, 256>(mt);
        case XQ_TYPE_F16: return mma_for<XQ_TYPE_F16, 256>(mt);
        case XQ_TYPE_E5M2: return mma_for<XQ_TYPE_E5M2, 256>(mt);
        }
    }
    return nullptr;
}

static MmaQprepFn mma_qprep_lookup(int kt, int d) {
    if (d == 128) {
        if (is_quant(kt)) return kt == XQ_TYPE_Q8_0 ? fa_qprep_mma<XQ_TYPE_Q8_0, 128> : fa_qprep_mma<XQ_TYPE_Q4_0, 128>;
        return fa_qprep_mma<XQ_TYPE_F16, 128>;
    }
    if (is_quant(kt)) return kt == XQ_TYPE_Q8_0 ? fa_qprep_mma<XQ_TYPE_Q8_0, 256> : fa_qprep_mma<XQ_TYPE_Q4_0, 256>;
    return fa_qprep_mma<XQ_TYPE_F16, 256>;
}

bool fa_mma_available(int kt, int d, int qk_mode, int n_pairs) {
    if (n_pairs < 1 || n_pairs > 32) return false;
    if (is_quant(kt) && qk_mode != kQkInt8) return false;  // f32-Q scores on quantized K stay on VALU
    return mma_lookup(kt, d, (n_pairs + 15) / 16) != nullptr;
}

size_t fa_mma_qimg_bytes(int64_t n_rows, int kt, int d) { return (size_t)n_rows * mma_qrow_bytes(kt, d); }

hipError_t fa_mma_launch(const FaArgs& a, const FaLaunch& L, uint8_t* qimg, hipStream_t stream) {
    const xq_tensor* q = L.q;
    const int D = (int)q->ne[0];
    const int kt = L.k->type;
    const int mt = (a.QT * a.G + 15) / 16;
    MmaPass1Fn p1 = mma_lookup(kt, D, mt);
    MmaQprepFn qp = mma_qprep_lookup(kt, D);
    if (!p1 || !qp) return hipErrorInvalidValue;
    const int64_t n_rows = (int64_t)a.B * a.NQ * a.H;
    const int hi_only = is_quant(kt) ? 0 : (L.q_round_f16 ? 1 : 0);
    {
        ProfScope ps("fa_qprep", stream);
        hipLaunchKernelGGL(qp, dim3((uint32_t)n_rows), dim3(64), 0, stream, (const uint8_t*)q->data,
                           (int64_t)q->nb[1], (int64_t)q->nb[2], (int64_t)q->nb[3], a.NQ, a.H, hi_only, qimg);
    }
    const uint32_t n_wg = (uint32_t)a.n_splits * a.n_qtiles * a.Hkv * a.B;
    ProfScope ps("fa_pass1", stream);
    hipLaunchKernelGGL(p1, dim3(n_wg), dim3(kThreads), 0, stream, a, (const uint8_t*)qimg, hi_only);
    return hipGetLastError();
}

}  // namespace xq
