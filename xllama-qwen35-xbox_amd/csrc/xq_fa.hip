// xq_fa.hip — GGML_OP_FLASH_ATTN_EXT decode / short multi-query verify on gfx950.
//
// Three kernels per call:
//   fa_qprep  — Q rows -> "Q image" rows in the workspace: f32 (optionally
//               rounded to f16), or ggml q8_0 (quantize_row_q8_0, x86 rules)
//               laid out to line up byte-for-byte with the K block layout so the
//               score loop can run v_dot4 on raw K dwords;
//   fa_pass1  — one workgroup per (sequence, KV head, query tile, KV split):
//               64-row K/V tiles staged HBM -> registers -> LDS with coalesced
//               chunk loads (prefetching the next tile while the current one is
//               computed); scores with one lane per KV row against the query
//               image read through scalar loads; online softmax per
//               (query, head) pair by its owning wave (DPP reductions); the
//               value phase gives each wave a quarter of the head dims and each
//               16-lane row a quarter of the tile rows; partial (acc, m, l) per
//               split, or the final output when there is a single split;
//   fa_mask_pack — only for the matrix-core engine when the mask rows are not
//               4-byte aligned (odd KV length): copies the mask rows the call
//               reads into 4-byte aligned rows in the workspace;
//   fa_reduce — merges the splits of one (sequence, query, head) in ascending
//               split order (the consistent KV-reduction order of
//               shaders/rkva/rkva_range_reduce.hlsl:12-46, with the non-finite
//               poisoning of shaders/rkva/rkva_range_reduce_opt.hlsl:39-56,126-132),
//               then applies sinks and the 1/S normalisation.
//
// Every (query, head) pair runs the same instruction sequence whatever other
// pairs share its workgroup, and the split partition never depends on the
// number of queries, so a query's result is bitwise independent of the query count of the
// call (the purpose of patches/0006-…:7-11 and patches/0008-…:40-56). The
// kernels are compiled with -ffp-contract=off and write every fused
// multiply-add explicitly.
#include <type_traits>

#include "xq_fa_common.h"

namespace xq {

// Decode VD consecutive elements starting at element e0 (multiple of VD) of a
// record in LDS. Bit-exact ggml decoders: f16 -> f32; q8_0 qs*d; q4_0
// (nibble - 8) * d with the integer converted first; E5M2 through f16.
template <int KT, int VD>
XQ_DEV void decode_v(const uint8_t* rec, int e0, float (&out)[VD]) {
    if constexpr (KT == XQ_TYPE_F16) {
        if constexpr (VD == 4) {
            const uint2 w = *(const uint2*)(rec + 2 * e0);
            out[0] = f16_bits_to_f32(w.x & 0xffffu);
            out[1] = f16_bits_to_f32(w.x >> 16);
            out[2] = f16_bits_to_f32(w.y & 0xffffu);
            out[3] = f16_bits_to_f32(w.y >> 16);
        } else {
            const uint32_t w = lds_u32(rec + 2 * e0);
            out[0] = f16_bits_to_f32(w & 0xffffu);
            out[1] = f16_bits_to_f32(w >> 16);
        }
    } else if constexpr (KT == XQ_TYPE_E5M2) {
        if constexpr (VD == 4) {
            const uint32_t w = lds_u32(rec + e0);
#pragma unroll
            for (int j = 0; j < 4; ++j) out[j] = e5m2_to_f32(w >> (8 * j));
        } else {
            const uint32_t w = lds_u16(rec + e0);
            out[0] = e5m2_to_f32(w);
            out[1] = e5m2_to_f32(w >> 8);
        }
    } else if constexpr (KT == XQ_TYPE_Q8_0) {
        const int blk = e0 >> 5, o = e0 & 31;
        const uint8_t* bp = rec + blk * 34;
        const float d = f16_bits_to_f32(lds_u16(bp));
        const uint32_t lo = lds_u16(bp + 2 + o);
        uint32_t w = lo;
        if constexpr (VD == 4) w |= lds_u16(bp + 4 + o) << 16;
#pragma unroll
        for (int j = 0; j < VD; ++j) out[j] = (float)sbyte(w, j) * d;
    } else {  // Q4_0
        const int blk = e0 >> 5, o = e0 & 31;
        const uint8_t* bp = rec + blk * 18;
        const float d = f16_bits_to_f32(lds_u16(bp));
        const int sh = o >= 16 ? 4 : 0;
        const int ob = o & 15;
        uint32_t w = lds_u16(bp + 2 + ob);
        if constexpr (VD == 4) w |= lds_u16(bp + 4 + ob) << 16;
#pragma unroll
        for (int j = 0; j < VD; ++j) out[j] = (float)((int)((w >> (8 * j + sh)) & 15u) - 8) * d;
    }
}

// Decode one 32-element block (block index c) of a record in LDS to f32.
template <int KT>
XQ_DEV void decode_block32(const uint8_t* rec, int c, float (&kf)[32]) {
    if constexpr (KT == XQ_TYPE_F16) {
        const uint4* p = (const uint4*)(rec + 64 * c);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 w = p[i];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                kf[8 * i + 2 * j] = f16_bits_to_f32(ws[j] & 0xffffu);
                kf[8 * i + 2 * j + 1] = f16_bits_to_f32(ws[j] >> 16);
            }
        }
    } else if constexpr (KT == XQ_TYPE_E5M2) {
        const uint4* p = (const uint4*)(rec + 32 * c);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint4 w = p[i];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int t = 0; t < 4; ++t) kf[16 * i + 4 * j + t] = e5m2_to_f32(ws[j] >> (8 * t));
        }
    } else {
        constexpr int BB = KT == XQ_TYPE_Q8_0 ? 34 : 18;
        const int base = BB * c;          // 2-aligned
        const int a0 = base & ~3;         // first aligned dword
        const int sh = base & 3;          // 0 or 2
        constexpr int NW = (BB + 1) / 4 + 1;  // dwords covering [base, base + BB) for sh in {0, 2}
        uint32_t w[NW];
#pragma unroll
        for (int i = 0; i < NW; ++i) w[i] = lds_u32(rec + a0 + 4 * i);
        auto byte_at = [&](int o) -> uint32_t {  // byte o of the block
            const int x = o + sh;
            return (w[x >> 2] >> (8 * (x & 3))) & 0xffu;
        };
        const float d = f16_bits_to_f32(byte_at(0) | (byte_at(1) << 8));
        if constexpr (KT == XQ_TYPE_Q8_0) {
#pragma unroll
            for (int j = 0; j < 32; ++j) kf[j] = (float)(int)(int8_t)byte_at(2 + j) * d;
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t q = byte_at(2 + j);
                kf[j] = (float)((int)(q & 15u) - 8) * d;
                kf[j + 16] = (float)((int)(q >> 4) - 8) * d;
            }
        }
    }
}

template <int KT, int D, int QKM, int NP>
__global__ __launch_bounds__(kThreads) void fa_pass1(FaArgs a, const uint32_t* __restrict__ qimg) {
    constexpr int REC = rec_bytes(KT, D);
    constexpr int RECP = pad_rec(REC);
    constexpr int CH = chunk_bytes(REC);
    constexpr int NCH = REC / CH;
    constexpr int NKC = (kTile * NCH + kThreads - 1) / kThreads;
    constexpr int UPW = NP / 4;   // pairs owned per wave
    constexpr int VD = D / 64;    // value dims per lane
    constexpr int PS = NP + 4;    // sP row stride in floats
    constexpr int IMGW = qimg_words(QKM, KT, D);
    using Ch = typename ChunkT<CH>::T;

    __shared__ __attribute__((aligned(16))) uint8_t sK[kTile * RECP];
    __shared__ __attribute__((aligned(16))) uint8_t sV[kTile * RECP];
    __shared__ __attribute__((aligned(16))) float sP[kTile * PS];
    __shared__ float sAlpha[NP];
    __shared__ float sFin[NP][2];
    __shared__ int sBad[NP];

    const uint32_t n_wg = (uint32_t)a.n_splits * a.n_qtiles * a.Hkv * a.B;
    uint32_t wg = xcd_remap(blockIdx.x, n_wg);
    const int qt = wg % a.n_qtiles;
    wg /= a.n_qtiles;
    const int split = wg % a.n_splits;
    wg /= a.n_splits;
    const int g = wg % a.Hkv;
    const int b = wg / a.Hkv;
    const int iq0 = qt * a.QT;
    const int nqt = min(a.QT, a.NQ - iq0);
    const int npa = nqt * a.G;
    const int wave = wave_id();
    const int lane = lane_id();
    const int tid = threadIdx.x;

    const int64_t r0 = (int64_t)split * a.split_rows;
    int64_t r_end = min(a.L, r0 + a.split_rows);
    if (a.positions) {  // range mode: the tile walk ends at the last visible row
        int64_t lim_max = 0;
        for (int qq = 0; qq < nqt; ++qq) {
            const int32_t pos = a.positions[iq0 + qq];
            const int64_t causal = pos < a.origin ? 0 : (int64_t)pos - a.origin + 1;
            lim_max = max(lim_max, min(a.L, causal));
        }
        r_end = min(r_end, lim_max);
    }

    const uint8_t* kb = a.k + (int64_t)(b / a.rk3) * a.k_nb3 + (int64_t)g * a.k_nb2;
    const uint8_t* vb = a.v + (int64_t)(b / a.rv3) * a.v_nb3 + (int64_t)g * a.v_nb2;

    // ---- per-pair constants (owner waves)
    float m_run[UPW], l_run[UPW], slope_u[UPW];
    int64_t lim_u[UPW];
    const uint8_t* mrow_u[UPW];
    const uint32_t* img_u[UPW];
#pragma unroll
    for (int u = 0; u < UPW; ++u) {
        m_run[u] = -INFINITY;
        l_run[u] = 0.0f;
        const int p = wave + 4 * u;
        const int pc = p < npa ? p : 0;
        const int qq = pc / a.G, h = g * a.G + pc % a.G, iq = iq0 + qq;
        slope_u[u] = alibi_slope(a, h);
        img_u[u] = qimg + ((int64_t)(b * a.NQ + iq) * a.H + h) * IMGW;
        lim_u[u] = a.L;
        if (a.positions) {
            const int32_t pos = a.positions[iq];
            const int64_t causal = pos < a.origin ? 0 : (int64_t)pos - a.origin + 1;
            lim_u[u] = min(a.L, causal);
        }
        mrow_u[u] = a.mask ? a.mask + (int64_t)iq * a.m_nb1 + (int64_t)(h % a.m_ne2) * a.m_nb2 +
                                 (int64_t)(b % a.m_ne3) * a.m_nb3
                           : nullptr;
    }

    float acc[NP][VD];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int j = 0; j < VD; ++j) acc[p][j] = 0.0f;

    const int rg = lane >> 4, li = lane & 15;
    const int d0 = wave * (D / 4) + li * VD;

    // ---- staging: global -> registers -> LDS
    Ch kr[NKC], vr[NKC];
    auto stage_load = [&](int64_t t0) {
#pragma unroll
        for (int i = 0; i < NKC; ++i) {
            const int c = tid + i * kThreads;
            kr[i] = Ch{};
            vr[i] = Ch{};
            if (c < kTile * NCH) {
                const int r = c / NCH, part = c % NCH;
                const int64_t row = t0 + r;
                if (row < r_end) {
                    kr[i] = *(const Ch*)(kb + row * a.k_nb1 + part * CH);
                    vr[i] = *(const Ch*)(vb + row * a.v_nb1 + part * CH);
                }
            }
        }
    };
    auto stage_store = [&]() {
#pragma unroll
        for (int i = 0; i < NKC; ++i) {
            const int c = tid + i * kThreads;
            if (c < kTile * NCH) {
                const int r = c / NCH, part = c % NCH;
                *(Ch*)(sK + r * RECP + part * CH) = kr[i];
                *(Ch*)(sV + r * RECP + part * CH) = vr[i];
            }
        }
    };

    for (int i = tid; i < kTile * PS; i += kThreads) sP[i] = 0.0f;
    if (tid < NP) sAlpha[tid] = 1.0f;
    if (r0 < r_end) {
        stage_load(r0);
        stage_store();
    }
    __syncthreads();

    for (int64_t t0 = r0; t0 < r_end; t0 += kTile) {
        const bool more = t0 + kTile < r_end;
        if (more) stage_load(t0 + kTile);

        // ---- scores: lane = row, wave owns pairs p = wave + 4u
        const int64_t arow = t0 + lane;
        const uint8_t* krec = sK + lane * RECP;
        float s_u[UPW];
#pragma unroll
        for (int u = 0; u < UPW; ++u) s_u[u] = 0.0f;

        if constexpr (QKM == kQkInt8 && KT == XQ_TYPE_Q8_0) {
#pragma unroll
            for (int bp = 0; bp < D / 64; ++bp) {
                uint32_t kw[17];
#pragma unroll
                for (int i = 0; i < 17; ++i) kw[i] = lds_u32(krec + bp * 68 + 4 * i);
                const float dk0 = f16_bits_to_f32(kw[0] & 0xffffu);
                const float dk1 = f16_bits_to_f32(kw[8] >> 16);
#pragma unroll
                for (int u = 0; u < UPW; ++u) {
                    const int p = wave + 4 * u;
                    if (p < npa) {
                        const uint32_t* img = img_u[u];
                        const uint32_t* qi = img + bp * 17;
                        int i0 = 0, i1 = 0;
#pragma unroll
                        for (int i = 0; i < 9; ++i) i0 = __builtin_amdgcn_sdot4((int)kw[i], (int)qi[i], i0, false);
#pragma unroll
                        for (int i = 9; i < 17; ++i) i1 = __builtin_amdgcn_sdot4((int)kw[i], (int)qi[i], i1, false);
                        const float* dq = (const float*)(img + (D / 64) * 17);
                        s_u[u] = fmaf((float)i0, dk0 * dq[2 * bp], s_u[u]);
                        s_u[u] = fmaf((float)i1, dk1 * dq[2 * bp + 1], s_u[u]);
                    }
                }
            }
        } else if constexpr (QKM == kQkInt8 && KT == XQ_TYPE_Q4_0) {
#pragma unroll
            for (int bp = 0; bp < D / 64; ++bp) {
                uint32_t kw[9];
#pragma unroll
                for (int i = 0; i < 9; ++i) kw[i] = lds_u32(krec + bp * 36 + 4 * i);
                const float dk0 = f16_bits_to_f32(kw[0] & 0xffffu);
                const float dk1 = f16_bits_to_f32(kw[4] >> 16);
                uint32_t lo[9], hi[9];
#pragma unroll
                for (int i = 0; i < 9; ++i) {
                    lo[i] = kw[i] & 0x0f0f0f0fu;
                    hi[i] = (kw[i] >> 4) & 0x0f0f0f0fu;
                }
#pragma unroll
                for (int u = 0; u < UPW; ++u) {
                    const int p = wave + 4 * u;
                    if (p < npa) {
                        const uint32_t* img = img_u[u];
                        const uint32_t* ql = img + bp * 18;
                        const uint32_t* qh = ql + 9;
                        int i0 = 0, i1 = 0;
#pragma unroll
                        for (int i = 0; i < 5; ++i) {
                            i0 = __builtin_amdgcn_sdot4((int)lo[i], (int)ql[i], i0, false);
                            i0 = __builtin_amdgcn_sdot4((int)hi[i], (int)qh[i], i0, false);
                        }
#pragma unroll
                        for (int i = 5; i < 9; ++i) {
                            i1 = __builtin_amdgcn_sdot4((int)lo[i], (int)ql[i], i1, false);
                            i1 = __builtin_amdgcn_sdot4((int)hi[i], (int)qh[i], i1, false);
                        }
                        const float* dq = (const float*)(img + (D / 64) * 18);
                        const int* sq = (const int*)(img + (D / 64) * 18 + D / kQK);
                        i0 -= 8 * sq[2 * bp];
                        i1 -= 8 * sq[2 * bp + 1];
                        s_u[u] = fmaf((float)i0, dk0 * dq[2 * bp], s_u[u]);
                        s_u[u] = fmaf((float)i1, dk1 * dq[2 * bp + 1], s_u[u]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int c = 0; c < D / kQK; ++c) {
                float kf[32];
                decode_block32<KT>(krec, c, kf);
#pragma unroll
                for (int u = 0; u < UPW; ++u) {
                    const int p = wave + 4 * u;
                    if (p < npa) {
                        const float* qf = (const float*)img_u[u] + 32 * c;
                        float s = s_u[u];
#pragma unroll
                        for (int j = 0; j < 32; ++j) s = fmaf(qf[j], kf[j], s);
                        s_u[u] = s;
                    }
                }
            }
        }

        // ---- online softmax per owned pair (ggml order: scale, softcap, + mask).
        //      A row the pair does not see (masked, past its limit or the tile)
        //      gets the weight -0, a visible row whose weight underflows +0:
        //      a tile with unseen rows is "careful", and there a non-finite V
        //      element reaches only the pairs whose weight is not -0 (ggml's
        //      loop never visits the rows it skips)
        bool unseen = false;
#pragma unroll
        for (int u = 0; u < UPW; ++u) {
            const int p = wave + 4 * u;
            if (p < npa) {
                float s = s_u[u] * a.scale;
                if (a.softcap != 0.0f) s = a.softcap * tanhf(s);
                bool valid = arow < r_end && arow < lim_u[u];
                if (valid && mrow_u[u]) {
                    const float mv = slope_u[u] * f16_bits_to_f32(((const uint16_t*)mrow_u[u])[arow]);
                    if (mv == -INFINITY) valid = false;
                    s = s + mv;
                }
                s = valid ? s : -INFINITY;
                unseen |= !valid;
                const float tmax = wave_max(s);
                const float m_new = fmaxf(m_run[u], tmax);
                const float alpha = m_new == -INFINITY ? 1.0f : fast_exp(m_run[u] - m_new);
                const float pr = s == -INFINITY ? -0.0f : fast_exp(s - m_new);
                l_run[u] = fmaf(l_run[u], alpha, wave_sum(pr));
                m_run[u] = m_new;
                sP[lane * PS + p] = pr;
                if (lane == 0) sAlpha[p] = alpha;
            }
        }
        const bool careful = __syncthreads_or(unseen);

        // ---- values: wave owns dims [wave*D/4, (wave+1)*D/4), row group rg owns rows rg + 4i
#pragma unroll
        for (int p4 = 0; p4 < NP / 4; ++p4) {
            if (4 * p4 < npa) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float al = sAlpha[4 * p4 + t];
#pragma unroll
                    for (int j = 0; j < VD; ++j) acc[4 * p4 + t][j] *= al;
                }
            }
        }
        const int nv = (int)min((int64_t)kTile, r_end - t0);
        for (int r = rg; r < nv; r += 4) {
            float vv[VD];
            decode_v<KT, VD>(sV + r * RECP, d0, vv);
            const float* pr = sP + r * PS;
            bool vbad = false;
            if (careful) {
#pragma unroll
                for (int j = 0; j < VD; ++j) vbad |= !__builtin_isfinite(vv[j]);
            }
            if (vbad) {
#pragma unroll
                for (int p4 = 0; p4 < NP / 4; ++p4) {
                    if (4 * p4 < npa) {
                        const float4 w4 = *(const float4*)(pr + 4 * p4);
                        const float ws[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            if (__float_as_uint(ws[t]) == 0x80000000u) continue;  // row unseen by the pair
#pragma unroll
                            for (int j = 0; j < VD; ++j) acc[4 * p4 + t][j] = fmaf(ws[t], vv[j], acc[4 * p4 + t][j]);
                        }
                    }
                }
            } else {
#pragma unroll
                for (int p4 = 0; p4 < NP / 4; ++p4) {
                    if (4 * p4 < npa) {
                        const float4 w4 = *(const float4*)(pr + 4 * p4);
                        const float ws[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                        for (int t = 0; t < 4; ++t)
#pragma unroll
                            for (int j = 0; j < VD; ++j) acc[4 * p4 + t][j] = fmaf(ws[t], vv[j], acc[4 * p4 + t][j]);
                    }
                }
            }
        }
        __syncthreads();
        if (more) {
            stage_store();
            __syncthreads();
        }
    }

    // ---- merge the four row groups: (g0 + g1) + (g2 + g3)
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int j = 0; j < VD; ++j) {
            float x = acc[p][j];
            x = x + __shfl_xor(x, 16);
            x = x + __shfl_xor(x, 32);
            acc[p][j] = x;
        }

    const int64_t rows_per_seq = (int64_t)a.NQ * a.H;
    if (a.n_splits == 1) {
#pragma unroll
        for (int u = 0; u < UPW; ++u) {
            const int p = wave + 4 * u;
            if (p < npa) {
                const int qq = p / a.G, h = g * a.G + p % a.G, iq = iq0 + qq;
                float a1, inv, l;
                fa_finalize(m_run[u], l_run[u], a.sinks != nullptr, a.sinks ? a.sinks[h] : 0.0f, a1, inv, l);
                if (lane == 0) {
                    sFin[p][0] = a1;
                    sFin[p][1] = inv;
                    // the split reducer's rule with one split (range calls): a
                    // non-finite or negative sum, factor or normaliser poisons the row
                    const float S = l_run[u];
                    sBad[p] = a.poison && (!__builtin_isfinite(S) || S < 0.0f || !__builtin_isfinite(inv) ||
                                           (S != 0.0f && !__builtin_isfinite(l)));
                    if (a.lse && !a.poison) a.lse[(int64_t)b * rows_per_seq + (int64_t)iq * a.H + h] = l;
                }
            }
        }
        __syncthreads();
        if (a.poison) {
            // ... and so does a non-finite output element
            if (rg == 0) {
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    if (p < npa) {
                        const float a1 = sFin[p][0], inv = sFin[p][1];
                        bool bad = false;
#pragma unroll
                        for (int j = 0; j < VD; ++j) bad |= !__builtin_isfinite((acc[p][j] * a1) * inv);
                        if (bad) sBad[p] = 1;
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int u = 0; u < UPW; ++u) {
                const int p = wave + 4 * u;
                if (p < npa && lane == 0 && a.lse) {
                    const int qq = p / a.G, h = g * a.G + p % a.G, iq = iq0 + qq;
                    float a1, inv, l;
                    fa_finalize(m_run[u], l_run[u], a.sinks != nullptr, a.sinks ? a.sinks[h] : 0.0f, a1, inv, l);
                    a.lse[(int64_t)b * rows_per_seq + (int64_t)iq * a.H + h] = sBad[p] ? NAN : l;
                }
            }
        }
        if (rg == 0) {
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                if (p < npa) {
                    const int qq = p / a.G, h = g * a.G + p % a.G, iq = iq0 + qq;
                    float* o = (float*)(a.dst + (int64_t)b * a.d_nb3 + (int64_t)iq * a.d_nb2 + (int64_t)h * a.d_nb1) + d0;
                    const float a1 = sFin[p][0], inv = sFin[p][1];
                    const bool bad = a.poison && sBad[p];
#pragma unroll
                    for (int j = 0; j < VD; ++j) o[j] = bad ? NAN : (acc[p][j] * a1) * inv;
                }
            }
        }
    } else {
        if (rg == 0) {
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                if (p < npa) {
                    const int qq = p / a.G, h = g * a.G + p % a.G, iq = iq0 + qq;
                    const int64_t row = (int64_t)b * rows_per_seq + (int64_t)iq * a.H + h;
                    float* o = a.part_o + (row * a.n_splits + split) * D + d0;
#pragma unroll
                    for (int j = 0; j < VD; ++j) o[j] = acc[p][j];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < UPW; ++u) {
            const int p = wave + 4 * u;
            if (p < npa && lane == 0) {
                const int qq = p / a.G, h = g * a.G + p % a.G, iq = iq0 + qq;
                const int64_t row = (int64_t)b * rows_per_seq + (int64_t)iq * a.H + h;
                a.part_ml[row * a.n_splits + split] = make_float2(m_run[u], l_run[u]);
            }
        }
    }
}

// One wave per (sequence, query, head) row; lane owns dims VPL*lane ..
// VPL*lane + VPL - 1 and walks the splits in ascending order with the same
// (wave-uniform) split states and weights as every other lane, so the row
// needs no barrier and no LDS. The states and the numerators of the first CH
// splits are loaded together: one memory round trip for up to CH splits (the
// automatic policy's counts), CH at a time beyond.
template <int D, int CH>
__global__ __launch_bounds__(64) void fa_reduce(FaArgs a) {
    constexpr int VPL = D / 64;
    using V = typename std::conditional<VPL == 4, float4, float2>::type;
    const int64_t row = blockIdx.x;
    const int S = a.n_splits;
    const int lane = threadIdx.x;
    const int64_t rows_per_seq = (int64_t)a.NQ * a.H;
    const int b = (int)(row / rows_per_seq);
    const int h = (int)(row % a.H);
    const float2* ml = a.part_ml + row * S;
    const float* po = a.part_o + row * S * D + VPL * lane;
    auto ldv = [&](int s) { return *(const V*)(po + (int64_t)s * D); };
    float2 st[CH];
    V v0[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        st[i] = i < S ? ml[i] : make_float2(0.0f, 0.0f);
        v0[i] = i < S ? ldv(i) : V{};
    }
    // participating splits (den != 0): the maximum; a non-finite or negative
    // den or a non-finite maximum is bad (shaders/rkva/rkva_range_reduce_opt.hlsl:39-56)
    float M = -3.402823466e38f;
    bool bad = false;
    auto visit = [&](float2 x) {
        if (x.y != 0.0f) {
            if (!__builtin_isfinite(x.y) || x.y < 0.0f || !__builtin_isfinite(x.x))
                bad = true;
            else
                M = fmaxf(M, x.x);
        }
    };
#pragma unroll
    for (int i = 0; i < CH; ++i) visit(st[i]);
    for (int s = CH; s < S; ++s) visit(ml[s]);
    float w0[CH];
    float L = 0.0f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        w0[i] = st[i].y != 0.0f ? expf(st[i].x - M) : 0.0f;
        if (st[i].y != 0.0f) L = fmaf(st[i].y, w0[i], L);
    }
    for (int s = CH; s < S; ++s) {
        const float2 x = ml[s];
        if (x.y != 0.0f) L = fmaf(x.y, expf(x.x - M), L);
    }
    float a1, inv, lse;
    fa_finalize(L == 0.0f ? -INFINITY : M, L, a.sinks != nullptr, a.sinks ? a.sinks[h] : 0.0f, a1, inv, lse);
    bad = bad || !__builtin_isfinite(L) || !__builtin_isfinite(inv) || (L != 0.0f && !__builtin_isfinite(lse));
    float acc[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) acc[j] = 0.0f;
    auto add = [&](const V& v, float w) {
        const float* e = (const float*)&v;
#pragma unroll
        for (int j = 0; j < VPL; ++j) acc[j] = fmaf(e[j], w, acc[j]);
    };
#pragma unroll
    for (int i = 0; i < CH; ++i)
        if (st[i].y != 0.0f) add(v0[i], w0[i]);
    for (int s0 = CH; s0 < S; s0 += CH) {
        V v[CH];
#pragma unroll
        for (int i = 0; i < CH; ++i) v[i] = s0 + i < S ? ldv(s0 + i) : V{};
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            if (s0 + i >= S) break;
            const float2 x = ml[s0 + i];
            if (x.y != 0.0f) add(v[i], expf(x.x - M));
        }
    }
    float out[VPL];
    bool nonfin = false;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        out[j] = (acc[j] * a1) * inv;
        nonfin |= !__builtin_isfinite(out[j]);
    }
    // range calls: any non-finite participating state, numerator or result
    // poisons the whole row (shaders/rkva/rkva_range_reduce_opt.hlsl:126-132)
    if (a.poison && (bad || __builtin_amdgcn_ballot_w64(nonfin) != 0)) {
#pragma unroll
        for (int j = 0; j < VPL; ++j) out[j] = NAN;
        lse = NAN;
    }
    if (lane == 0 && a.lse) a.lse[row] = lse;
    const int iq = (int)((row % rows_per_seq) / a.H);
    float* o = (float*)(a.dst + (int64_t)b * a.d_nb3 + (int64_t)iq * a.d_nb2 + (int64_t)h * a.d_nb1) + VPL * lane;
    V ov;
    float* oe = (float*)&ov;
#pragma unroll
    for (int j = 0; j < VPL; ++j) oe[j] = out[j];
    *(V*)o = ov;
}

// Q rows -> image rows. One wave per (sequence, query, head) row.
template <int KT, int D, int QKM>
__global__ __launch_bounds__(64) void fa_qprep(const uint8_t* __restrict__ q, int64_t nb1, int64_t nb2,
                                                int64_t nb3, int NQ, int H, int round_f16,
                                                uint32_t* __restrict__ img_out) {
    constexpr int IMGW = qimg_words(QKM, KT, D);
    const int64_t row = blockIdx.x;
    const int h = (int)(row % H);
    const int iq = (int)((row / H) % NQ);
    const int b = (int)(row / ((int64_t)H * NQ));
    const float* src = (const float*)(q + (int64_t)b * nb3 + (int64_t)iq * nb1 + (int64_t)h * nb2);
    uint32_t* img = img_out + row * IMGW;
    const int lane = threadIdx.x;
    if constexpr (QKM == kQkFloat) {
        for (int e = lane; e < D; e += 64) {
            float x = src[e];
            if (round_f16) x = f16_bits_to_f32(f32_to_f16_bits(x));
            img[e] = __float_as_uint(x);
        }
    } else {
        constexpr int VD = D / 64;          // elements per lane
        constexpr int LPB = kQK / VD;       // lanes per block: 8 (D 256) or 16 (D 128)
        __shared__ int8_t sq[D];
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
        // ggml-cpu x86 quantize_row_q8_0: d = amax/127, id = 127/amax, round half even
        const float dblk = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        int qsum = 0;
#pragma unroll
        for (int j = 0; j < VD; ++j) {
            const int qv = (int)rintf(x[j] * id);
            sq[lane * VD + j] = (int8_t)qv;
            qsum += qv;
        }
        // exact integer block sums (only q4_0 needs them)
        float qs = (float)qsum;
        qs += dpp<0xB1>(qs);
        qs += dpp<0x4E>(qs);
        qs += dpp<0x141>(qs);
        if constexpr (LPB == 16) qs += dpp<0x140>(qs);
        __syncthreads();
        const int blk = (lane * VD) / kQK;
        const bool leader = (lane % LPB) == 0;
        const float dq = f16_bits_to_f32(f32_to_f16_bits(dblk));
        if constexpr (KT == XQ_TYPE_Q8_0) {
            constexpr int PW = (D / 64) * 17;
            for (int w = lane; w < PW; w += 64) {
                const int bp = w / 17, k4 = w % 17;
                uint32_t word = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int o = 4 * k4 + j;            // byte in the 68-byte pair
                    const int bb = o < 34 ? 0 : 1;
                    const int ob = o - 34 * bb;
                    if (ob >= 2) word |= (uint32_t)(uint8_t)sq[32 * (2 * bp + bb) + ob - 2] << (8 * j);
                }
                img[w] = word;
            }
            if (leader) img[PW + blk] = __float_as_uint(dq);
        } else {
            constexpr int PW = (D / 64) * 18;
            for (int w = lane; w < PW; w += 64) {
                const int bp = w / 18, k18 = w % 18;
                const int hi = k18 >= 9, k4 = k18 % 9;
                uint32_t word = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int o = 4 * k4 + j;            // byte in the 36-byte pair
                    const int bb = o < 18 ? 0 : 1;
                    const int ob = o - 18 * bb;
                    if (ob >= 2)
                        word |= (uint32_t)(uint8_t)sq[32 * (2 * bp + bb) + (ob - 2) + (hi ? 16 : 0)] << (8 * j);
                }
                img[w] = word;
            }
            if (leader) {
                img[PW + blk] = __float_as_uint(dq);
                img[PW + D / kQK + blk] = (uint32_t)(int)qs;
            }
        }
    }
}

// ---------------------------------------------------------------- dispatch

using Pass1Fn = void (*)(FaArgs, const uint32_t*);
using ReduceFn = void (*)(FaArgs);
using QprepFn = void (*)(const uint8_t*, int64_t, int64_t, int64_t, int, int, int, uint32_t*);

template <int KT, int D, int QKM>
static Pass1Fn pass1_for(int np) {
    switch (np) {
    case 4: return fa_pass1<KT, D, QKM, 4>;
    case 8: return fa_pass1<KT, D, QKM, 8>;
    case 16: return fa_pass1<KT, D, QKM, 16>;
    case 32: return fa_pass1<KT, D, QKM, 32>;
    default: return nullptr;
    }
}

template <int D>
static Pass1Fn pass1_d(int kt, int qkm, int np) {
    if (qkm == kQkInt8) {
        if (kt == XQ_TYPE_Q8_0) return pass1_for<XQ_TYPE_Q8_0, D, kQkInt8>(np);
        if (kt == XQ_TYPE_Q4_0) return pass1_for<XQ_TYPE_Q4_0, D, kQkInt8>(np);
        return nullptr;
    }
    switch (kt) {
    case XQ_TYPE_F16: return pass1_for<XQ_TYPE_F16, D, kQkFloat>(np);
    case XQ_TYPE_Q8_0: return pass1_for<XQ_TYPE_Q8_0, D, kQkFloat>(np);
    case XQ_TYPE_Q4_0: return pass1_for<XQ_TYPE_Q4_0, D, kQkFloat>(np);
    case XQ_TYPE_E5M2: return pass1_for<XQ_TYPE_E5M2, D, kQkFloat>(np);
    default: return nullptr;
    }
}

static Pass1Fn pass1_lookup(int kt, int d, int qkm, int np) {
    if (d == 128) return pass1_d<128>(kt, qkm, np);
    if (d == 256) return pass1_d<256>(kt, qkm, np);
    return nullptr;
}

template <int D>
static QprepFn qprep_d(int kt, int qkm) {
    if (qkm == kQkFloat) return fa_qprep<XQ_TYPE_F16, D, kQkFloat>;
    if (kt == XQ_TYPE_Q8_0) return fa_qprep<XQ_TYPE_Q8_0, D, kQkInt8>;
    if (kt == XQ_TYPE_Q4_0) return fa_qprep<XQ_TYPE_Q4_0, D, kQkInt8>;
    return nullptr;
}

static int np_bin(int npairs) {
    return npairs <= 4 ? 4 : npairs <= 8 ? 8 : npairs <= 16 ? 16 : npairs <= 32 ? 32 : 0;
}

bool fa_kernel_available(int kt, int d, int qk_mode, int n_pairs) {
    const int np = np_bin(n_pairs);
    return np && pass1_lookup(kt, d, qk_mode, np) != nullptr;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Q image of the VALU engine (the matrix-core engine builds its own in LDS).
static size_t qimg_bytes(int64_t n_rows, int d, int qk_mode, int kt) {
    return (size_t)n_rows * qimg_words(qk_mode, kt, d) * 4;
}

// Mask rows re-laid with an even element count (4-byte aligned rows) for the
// matrix-core engine: one row per (query, mask head plane, mask sequence
// plane); the pad element is -inf.
__host__ __device__ static inline int64_t mask_pack_cols(int64_t L) { return (L + 1) & ~(int64_t)1; }

size_t fa_mask_pack_bytes(const xq_tensor* mask, int64_t L, int n_q) {
    if (!mask) return 0;
    return align256((size_t)mask->ne[3] * mask->ne[2] * n_q * mask_pack_cols(L) * 2);
}

__global__ __launch_bounds__(256) void fa_mask_pack(const uint8_t* __restrict__ src, int64_t nb1, int64_t nb2,
                                                    int64_t nb3, int n_q, int ne2, int64_t L,
                                                    uint32_t* __restrict__ dst) {
    const int row = blockIdx.x;  // (b * ne2 + h) * n_q + q
    const int qi = row % n_q, h = (row / n_q) % ne2, b = row / (n_q * ne2);
    const uint16_t* s = (const uint16_t*)(src + qi * nb1 + h * nb2 + b * nb3);
    const int64_t pairs = mask_pack_cols(L) / 2;
    uint32_t* d = dst + row * pairs;
    for (int64_t c = threadIdx.x; c < pairs; c += 256) {
        const uint32_t lo = s[2 * c];
        const uint32_t hi = 2 * c + 1 < L ? s[2 * c + 1] : 0xFC00u;
        d[c] = lo | (hi << 16);
    }
}

// Merge of position-split results: one wave per row, lane owns dims
// lane + 64 m. Every lane walks the parts in order (uniform loads of the LSEs).
__global__ __launch_bounds__(64) void fa_lse_merge(const float* __restrict__ po, const float* __restrict__ pl,
                                                   int n_parts, int64_t rows, int d, float* __restrict__ out,
                                                   float* __restrict__ lse) {
    constexpr int kMaxPerLane = 8;  // d <= 512
    const int64_t r = blockIdx.x;
    const int lane = threadIdx.x;
    bool bad = false, any = false;
    float M = -3.402823466e38f;
    for (int p = 0; p < n_parts; ++p) {
        const float l = pl[(int64_t)p * rows + r];
        if (l == -INFINITY) continue;
        if (!isfinite(l)) {
            bad = true;
        } else {
            any = true;
            M = fmaxf(M, l);
        }
    }
    float* o = out + r * d;
    if (!bad && !any) {  // every range empty
        for (int i = lane; i < d; i += 64) o[i] = 0.0f;
        if (lane == 0) lse[r] = -INFINITY;
        return;
    }
    float sum = 0.0f;
    if (!bad)
        for (int p = 0; p < n_parts; ++p) {
            const float l = pl[(int64_t)p * rows + r];
            if (l != -INFINITY) sum = sum + expf(l - M);
        }
    const float inv = bad ? 0.0f : 1.0f / sum;
    const float lv = bad ? NAN : M + logf(sum);
    bad = bad || !isfinite(lv) || !isfinite(inv);
    float acc[kMaxPerLane];
#pragma unroll
    for (int m = 0; m < kMaxPerLane; ++m) acc[m] = 0.0f;
    if (!bad)
        for (int p = 0; p < n_parts; ++p) {
            const float l = pl[(int64_t)p * rows + r];
            if (l == -INFINITY) continue;
            const float w = expf(l - M);
            const float* src = po + ((int64_t)p * rows + r) * d;
#pragma unroll
            for (int m = 0; m < kMaxPerLane; ++m) {
                const int i = lane + 64 * m;
                if (i < d) acc[m] = acc[m] + src[i] * w;
            }
        }
    bool lane_bad = false;
#pragma unroll
    for (int m = 0; m < kMaxPerLane; ++m) {
        acc[m] = acc[m] * inv;
        if (lane + 64 * m < d && !isfinite(acc[m])) lane_bad = true;
    }
    bad = bad || __any(lane_bad);
#pragma unroll
    for (int m = 0; m < kMaxPerLane; ++m) {
        const int i = lane + 64 * m;
        if (i < d) o[i] = bad ? NAN : acc[m];
    }
    if (lane == 0) lse[r] = bad ? NAN : lv;
}

hipError_t fa_lse_merge_launch(const float* parts_out, const float* parts_lse, int n_parts, int64_t rows, int d,
                               float* out, float* lse, hipStream_t stream) {
    launch("fa_lse_merge", fa_lse_merge, dim3((uint32_t)rows), dim3(64), stream, parts_out, parts_lse, n_parts, rows,
           d, out, lse);
    return hipGetLastError();
}

size_t fa_workspace_bytes(int64_t n_rows, int d, int qk_mode, int kt, int n_splits) {
    size_t bytes = align256(qimg_bytes(n_rows, d, qk_mode, kt));
    if (n_splits > 1) {
        bytes += align256((size_t)n_rows * n_splits * d * 4);
        bytes += align256((size_t)n_rows * n_splits * 8);
    }
    return bytes;
}

hipError_t fa_reduce_launch(const FaArgs& a, int d, hipStream_t stream) {
    const int64_t n_rows = (int64_t)a.B * a.NQ * a.H;
    const bool wide = a.n_splits > 16;
    if (d == 128)
        launch("fa_reduce", wide ? fa_reduce<128, 32> : fa_reduce<128, 16>, dim3((uint32_t)n_rows), dim3(64),
               stream, a);
    else
        launch("fa_reduce", wide ? fa_reduce<256, 32> : fa_reduce<256, 16>, dim3((uint32_t)n_rows), dim3(64),
               stream, a);
    return hipGetLastError();
}

hipError_t fa_launch(const FaLaunch& L, hipStream_t stream) {
    const xq_tensor* q = L.q;
    const xq_tensor* k = L.k;
    const xq_tensor* v = L.v;
    const int D = (int)q->ne[0];
    const int NQ = (int)q->ne[1], H = (int)q->ne[2], B = (int)q->ne[3];
    const int Hkv = (int)k->ne[2];
    const int G = H / Hkv;
    const int kt = k->type;

    FaArgs a{};
    a.k = (const uint8_t*)k->data;
    a.v = (const uint8_t*)v->data;
    a.k_nb1 = k->nb[1]; a.k_nb2 = k->nb[2]; a.k_nb3 = k->nb[3];
    a.v_nb1 = v->nb[1]; a.v_nb2 = v->nb[2]; a.v_nb3 = v->nb[3];
    if (L.mask) {
        a.mask = (const uint8_t*)L.mask->data;
        a.m_nb1 = L.mask->nb[1]; a.m_nb2 = L.mask->nb[2]; a.m_nb3 = L.mask->nb[3];
        a.m_ne2 = (int32_t)L.mask->ne[2]; a.m_ne3 = (int32_t)L.mask->ne[3];
    } else {
        a.m_ne2 = 1; a.m_ne3 = 1;
    }
    a.positions = L.positions;
    a.origin = L.origin;
    a.sinks = L.sinks ? (const float*)L.sinks->data : nullptr;
    a.dst = (uint8_t*)L.dst->data;
    a.d_nb1 = L.dst->nb[1]; a.d_nb2 = L.dst->nb[2]; a.d_nb3 = L.dst->nb[3];
    a.lse = L.lse;
    a.L = k->ne[1];
    a.split_rows = L.split_rows > 0 ? L.split_rows : 1;
    a.interleave = L.interleave && !L.positions && L.n_splits > 1 ? 1 : 0;
    a.H = H; a.Hkv = Hkv; a.G = G; a.NQ = NQ; a.B = B;
    a.rk3 = (int32_t)(B / k->ne[3]);
    a.rv3 = (int32_t)(B / v->ne[3]);
    a.n_splits = L.n_splits;
    a.softcap = L.softcap;
    a.scale = L.softcap != 0.0f ? L.scale / L.softcap : L.scale;
    a.max_bias = L.max_bias;
    {
        const uint32_t nhl2 = 1u << (uint32_t)floor(log2((double)H));
        a.n_head_log2 = (int32_t)nhl2;
        a.m0 = powf(2.0f, -(L.max_bias) / (float)nhl2);
        a.m1 = powf(2.0f, -(L.max_bias / 2.0f) / (float)nhl2);
    }
    a.poison = L.poison;

    int QT = fa_query_tile(D, G, NQ);
    if (QT < 1) QT = 1;
    a.QT = QT;
    a.n_qtiles = (NQ + QT - 1) / QT;
    const int np = np_bin(QT * G);
    const int64_t n_rows = (int64_t)B * NQ * H;
    uint8_t* ws = (uint8_t*)L.workspace;
    uint32_t* qimg = (uint32_t*)ws;
    size_t off = align256(qimg_bytes(n_rows, D, L.qk_mode, kt));
    if (L.n_splits > 1) {
        a.part_o = (float*)(ws + off);
        off += align256((size_t)n_rows * L.n_splits * D * 4);
        a.part_ml = (float2*)(ws + off);
    }

    const bool mma = L.engine != XQ_FA_ENGINE_VALU && fa_mma_available(kt, D, L.qk_mode, QT * G);
    if (L.engine == XQ_FA_ENGINE_MFMA && !mma) return hipErrorInvalidValue;
    if (mma) {
        if (!fa_mma_mask_ok(a)) {
            const size_t base = fa_workspace_bytes(n_rows, D, L.qk_mode, kt, L.n_splits);
            if (L.workspace_bytes < base + fa_mask_pack_bytes(L.mask, a.L, NQ)) return hipErrorInvalidValue;
            uint32_t* packed = (uint32_t*)(ws + base);
            const int n_pack = NQ * a.m_ne2 * a.m_ne3;
            launch("fa_mask_pack", fa_mask_pack, dim3((uint32_t)n_pack), dim3(256), stream, a.mask, a.m_nb1,
                   a.m_nb2, a.m_nb3, NQ, a.m_ne2, a.L, packed);
            a.mask = (const uint8_t*)packed;
            a.m_nb1 = mask_pack_cols(a.L) * 2;
            a.m_nb2 = (int64_t)NQ * a.m_nb1;
            a.m_nb3 = (int64_t)a.m_ne2 * a.m_nb2;
        }
        return fa_mma_launch(a, L, stream);
    }
    Pass1Fn p1 = pass1_lookup(kt, D, L.qk_mode, np);
    QprepFn qp = D == 128 ? qprep_d<128>(kt, L.qk_mode) : qprep_d<256>(kt, L.qk_mode);
    if (!p1 || !qp) return hipErrorInvalidValue;
    launch("fa_qprep", qp, dim3((uint32_t)n_rows), dim3(64), stream, (const uint8_t*)q->data,
           (int64_t)q->nb[1], (int64_t)q->nb[2], (int64_t)q->nb[3], NQ, H, L.q_round_f16, qimg);
    const uint32_t n_wg = (uint32_t)L.n_splits * a.n_qtiles * Hkv * B;
    launch("fa_pass1", p1, dim3(n_wg), dim3(kThreads), stream, a, (const uint32_t*)qimg);
    if (L.n_splits > 1) return fa_reduce_launch(a, D, stream);
    return hipGetLastError();
}

}  // namespace xq
