/*
 * xq_oracle.c — CPU oracle (TEST INFRASTRUCTURE ONLY; see xq_oracle.h).
 *
 * Plain C11 restatement of the reference's ggml CPU semantics for the
 * flash-attention and gated-delta-net path. Compiled with -ffp-contract=off so
 * every multiply and add rounds separately unless an fmaf() is written out,
 * which is how the restated orders below are expressed.
 */
#include "xq_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 32

/* ======================================================================
 * scalar codecs
 * ==================================================================== */

static inline uint32_t f32_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}
static inline float bits_f32(uint32_t u) {
    float x;
    memcpy(&x, &u, 4);
    return x;
}

/* f32 -> f16 round to nearest even, NaN -> 0x7e00|sign, overflow -> inf.
 * Same results as ggml_half_bits (shaders/rkva/rkva_store_f16.hlsl:27-61,
 * uwp/rkva/rkva-kvarn-bulk.h:21-61). Written as: build the truncated half,
 * then add the rounding increment, letting a mantissa carry roll into the
 * exponent (and on to infinity). */
uint16_t xo_f32_to_f16(float x) {
    const uint32_t u = f32_bits(x);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t ex = (u >> 23) & 0xffu;
    const uint32_t man = u & 0x7fffffu;
    if (ex == 0xffu) return (uint16_t)(sign | (man ? 0x7e00u : 0x7c00u));
    const int e = (int)ex - 112; /* rebias 127 -> 15 */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign; /* below half the smallest subnormal */
        const uint32_t m = man | 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e); /* 14..24 */
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (h & 1u))) ++h; /* may become 0x400: smallest normal */
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h; /* carry may reach 0x7c00 = inf */
    return (uint16_t)(sign | h);
}

float xo_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    if (ex == 0) {
        /* zero or subnormal: man * 2^-24 is exact in f32 */
        const float v = (float)man * 5.9604644775390625e-08f;
        return bits_f32(f32_bits(v) | sign);
    }
    if (ex == 31) return bits_f32(sign | 0x7f800000u | (man << 13));
    return bits_f32(sign | ((ex + 112u) << 23) | (man << 13));
}

/* ggml_compute_fp32_to_bf16: quiet NaNs, otherwise round to nearest even. */
uint16_t xo_f32_to_bf16(float x) {
    const uint32_t u = f32_bits(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 64u);
    return (uint16_t)((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
}

float xo_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* f16 -> FP8 E5M2: keep the upper byte with round-to-nearest-even on the
 * dropped byte and finite saturation at 0x7b (57344); inf/NaN keep their class
 * (shaders/rkva/rkva_range_bulk_f16.hlsl:156-167, uwp/rkva/rkva-kvarn-bulk.h:91-107). */
uint8_t xo_f16_to_e5m2(uint16_t h) {
    const uint8_t sign = (uint8_t)((h >> 8) & 0x80u);
    if ((h & 0x7c00u) == 0x7c00u) {
        if (!(h & 0x03ffu)) return (uint8_t)(sign | 0x7cu);
        const uint8_t top = (uint8_t)((h >> 8) & 3u);
        return (uint8_t)(sign | 0x7cu | (top ? top : 1u));
    }
    uint32_t mag = h & 0x7fffu;
    if (mag > 0x7b00u) mag = 0x7b00u;
    return (uint8_t)(sign | ((mag + 0x7fu + ((mag >> 8) & 1u)) >> 8));
}

uint16_t xo_e5m2_to_f16(uint8_t b) { return (uint16_t)((uint16_t)b << 8); }

void xo_f32_to_f16_row(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = xo_f32_to_f16(x[i]);
}
void xo_f16_to_f32_row(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = xo_f16_to_f32(x[i]);
}
void xo_f32_to_bf16_row(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = xo_f32_to_bf16(x[i]);
}
void xo_bf16_to_f32_row(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = xo_bf16_to_f32(x[i]);
}
void xo_f32_to_e5m2_row(const float* x, uint8_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = xo_f16_to_e5m2(xo_f32_to_f16(x[i]));
}

/* ======================================================================
 * block quantizers (ggml block_q8_0 / block_q4_0)
 * ==================================================================== */

/* variant 0: ggml-cpu x86 quantize_row_q8_0 — d = amax/127, id = 127/amax,
 *            q = round-half-to-even(x*id);
 * variant 1: quantize_row_q8_0_ref — d = amax/127, id = d ? 1/d : 0,
 *            q = roundf(x*id) (half away from zero).
 * Both store d as f16 (RNE). Which one filled a given cache is upstream
 * behaviour not present in the reference checkout (parity unpinned); the two
 * agree except at exact rounding ties. */
void xo_quantize_row_q8_0(const float* x, void* vy, int64_t k, int variant) {
    uint8_t* y = (uint8_t*)vy;
    for (int64_t b = 0; b < k / QK; ++b) {
        const float* xb = x + b * QK;
        uint8_t* yb = y + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < QK; ++j) {
            const float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        float id;
        if (variant == 0)
            id = amax != 0.0f ? 127.0f / amax : 0.0f;
        else
            id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = xo_f32_to_f16(d);
        memcpy(yb, &dh, 2);
        for (int j = 0; j < QK; ++j) {
            const float t = xb[j] * id;
            const float r = variant == 0 ? rintf(t) : roundf(t);
            yb[2 + j] = (uint8_t)(int8_t)(int)r;
        }
    }
}

/* quantize_row_q4_0_ref: d = max/-8 where max is the signed value of largest
 * magnitude, q = min(15, (int8)(x*id + 8.5)); element j < 16 in the low nibble
 * of qs[j], element j + 16 in its high nibble. */
void xo_quantize_row_q4_0(const float* x, void* vy, int64_t k) {
    uint8_t* y = (uint8_t*)vy;
    for (int64_t b = 0; b < k / QK; ++b) {
        const float* xb = x + b * QK;
        uint8_t* yb = y + b * 18;
        float amax = 0.0f, vmax = 0.0f;
        for (int j = 0; j < QK; ++j) {
            if (amax < fabsf(xb[j])) {
                amax = fabsf(xb[j]);
                vmax = xb[j];
            }
        }
        const float d = vmax / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = xo_f32_to_f16(d);
        memcpy(yb, &dh, 2);
        for (int j = 0; j < QK / 2; ++j) {
            int lo = (int8_t)(xb[j] * id + 8.5f);
            int hi = (int8_t)(xb[j + QK / 2] * id + 8.5f);
            if (lo > 15) lo = 15;
            if (hi > 15) hi = 15;
            yb[2 + j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

size_t xo_row_bytes(int type, int64_t k) {
    switch (type) {
    case XQ_TYPE_F32: return (size_t)k * 4;
    case XQ_TYPE_F16:
    case XQ_TYPE_BF16: return (size_t)k * 2;
    case XQ_TYPE_Q8_0: return (size_t)(k / QK) * 34;
    case XQ_TYPE_Q4_0: return (size_t)(k / QK) * 18;
    case XQ_TYPE_E5M2: return (size_t)k;
    default: return 0;
    }
}

/* Decoders: F16 f16->f32; Q8_0 qs[j]*d; Q4_0 (nibble-8)*d (int then float
 * multiply, as dequantize_row_q4_0); E5M2 via f16. Bit-exact contract of the
 * KV dequant (shaders/rkva/rkva_range_attn.hlsl:35-57). */
void xo_dequant_row(int type, const void* vx, float* y, int64_t k) {
    const uint8_t* x = (const uint8_t*)vx;
    switch (type) {
    case XQ_TYPE_F32: memcpy(y, x, (size_t)k * 4); break;
    case XQ_TYPE_F16:
        for (int64_t i = 0; i < k; ++i) {
            uint16_t h;
            memcpy(&h, x + 2 * i, 2);
            y[i] = xo_f16_to_f32(h);
        }
        break;
    case XQ_TYPE_BF16:
        for (int64_t i = 0; i < k; ++i) {
            uint16_t h;
            memcpy(&h, x + 2 * i, 2);
            y[i] = xo_bf16_to_f32(h);
        }
        break;
    case XQ_TYPE_Q8_0:
        for (int64_t b = 0; b < k / QK; ++b) {
            uint16_t dh;
            memcpy(&dh, x + b * 34, 2);
            const float d = xo_f16_to_f32(dh);
            for (int j = 0; j < QK; ++j) y[b * QK + j] = (float)(int8_t)x[b * 34 + 2 + j] * d;
        }
        break;
    case XQ_TYPE_Q4_0:
        for (int64_t b = 0; b < k / QK; ++b) {
            uint16_t dh;
            memcpy(&dh, x + b * 18, 2);
            const float d = xo_f16_to_f32(dh);
            for (int j = 0; j < QK / 2; ++j) {
                const uint8_t q = x[b * 18 + 2 + j];
                y[b * QK + j] = (float)((int)(q & 15) - 8) * d;
                y[b * QK + j + QK / 2] = (float)((int)(q >> 4) - 8) * d;
            }
        }
        break;
    case XQ_TYPE_E5M2:
        for (int64_t i = 0; i < k; ++i) y[i] = xo_f16_to_f32(xo_e5m2_to_f16(x[i]));
        break;
    default: break;
    }
}

/* ======================================================================
 * ggml CPU vec-dot orders (x86 AVX2 build; parity unpinned at bit level)
 * ==================================================================== */

/* ggml_vec_dot_f32 / ggml_vec_dot_f16 with 4 x 8-lane accumulators: lane L
 * accumulates elements i = L (mod 32) with fused multiply-add, the four
 * vectors fold 0+2, 1+3, then 0+1, the 8 lanes fold lo+hi, then two
 * horizontal adds. n is a multiple of 32 for every head size this path runs. */
static float dot32_f32(const float* a, const float* b, int64_t n) {
    float acc[32];
    for (int l = 0; l < 32; ++l) acc[l] = 0.0f;
    for (int64_t i = 0; i < n; i += 32)
        for (int l = 0; l < 32; ++l) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    float x[4][8];
    for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 8; ++l) x[j][l] = acc[j * 8 + l];
    for (int l = 0; l < 8; ++l) {
        x[0][l] = x[0][l] + x[2][l];
        x[1][l] = x[1][l] + x[3][l];
    }
    for (int l = 0; l < 8; ++l) x[0][l] = x[0][l] + x[1][l];
    float t0[4];
    for (int l = 0; l < 4; ++l) t0[l] = x[0][l] + x[0][l + 4];
    const float h0 = t0[0] + t0[1], h1 = t0[2] + t0[3];
    double s = (double)(h0 + h1);
    for (int64_t i = (n / 32) * 32; i < n; ++i) s += (double)(a[i] * b[i]);
    return (float)s;
}

/* hsum_float_8: lanes (l, l+4) then (0,2),(1,3) then (0,1). */
static float hsum8(const float a[8]) {
    float r[4];
    for (int l = 0; l < 4; ++l) r[l] = a[l + 4] + a[l];
    const float r0 = r[0] + r[2], r1 = r[1] + r[3];
    return r0 + r1;
}

/* ggml_vec_dot_q8_0_q8_0 / ggml_vec_dot_q4_0_q8_0 (AVX2): per block d = dx*dy;
 * lane L gets the exact integer sum of products of elements 4L..4L+3, converted
 * to float and fused into acc[L] = fma(d, lane, acc[L]); hsum8 at the end. */
static float dot_q_q8(int ktype, const uint8_t* kx, const uint8_t* qy, int64_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int64_t nb = n / QK;
    for (int64_t b = 0; b < nb; ++b) {
        int8_t kq[QK];
        uint16_t dkh;
        if (ktype == XQ_TYPE_Q8_0) {
            memcpy(&dkh, kx + b * 34, 2);
            for (int j = 0; j < QK; ++j) kq[j] = (int8_t)kx[b * 34 + 2 + j];
        } else {
            memcpy(&dkh, kx + b * 18, 2);
            for (int j = 0; j < QK / 2; ++j) {
                const uint8_t v = kx[b * 18 + 2 + j];
                kq[j] = (int8_t)((int)(v & 15) - 8);
                kq[j + QK / 2] = (int8_t)((int)(v >> 4) - 8);
            }
        }
        uint16_t dqh;
        memcpy(&dqh, qy + b * 34, 2);
        const float d = xo_f16_to_f32(dkh) * xo_f16_to_f32(dqh);
        for (int l = 0; l < 8; ++l) {
            int s = 0;
            for (int j = 4 * l; j < 4 * l + 4; ++j) s += (int)kq[j] * (int)(int8_t)qy[b * 34 + 2 + j];
            acc[l] = fmaf(d, (float)s, acc[l]);
        }
    }
    return hsum8(acc);
}

/* ======================================================================
 * flash attention
 * ==================================================================== */

float xo_alibi_slope(float max_bias, int n_head, int h) {
    if (!(max_bias > 0.0f)) return 1.0f;
    const uint32_t n_head_log2 = 1u << (uint32_t)floor(log2((double)n_head));
    const float m0 = powf(2.0f, -(max_bias) / (float)n_head_log2);
    const float m1 = powf(2.0f, -(max_bias / 2.0f) / (float)n_head_log2);
    return (uint32_t)h < n_head_log2 ? powf(m0, (float)(h + 1))
                                     : powf(m1, (float)(2 * (h - (int)n_head_log2) + 1));
}

static int fa_shapes_ok(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                        const xq_tensor* dst) {
    if (!q || !k || !v || !dst) return 0;
    if (q->type != XQ_TYPE_F32 || dst->type != XQ_TYPE_F32) return 0;
    if (k->ne[0] != q->ne[0] || v->ne[1] != k->ne[1]) return 0;
    if (q->ne[2] % k->ne[2] || q->ne[2] % v->ne[2] || q->ne[3] % k->ne[3] || q->ne[3] % v->ne[3])
        return 0;
    if (dst->ne[0] != v->ne[0] || dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] ||
        dst->ne[3] != q->ne[3])
        return 0;
    return 1;
}

/* Which dot the score uses (patches/0008-flash-attn-query-consistency.patch:7-9):
 * 0 = f32 Q x f32(K) (ggml_vec_dot_f32), 1 = f16(Q) x f16 K (ggml_vec_dot_f16),
 * 2 = q8_0(Q) x quantized K (vec_dot_q*_q8_0). */
static int fa_dot_kind(int ktype, int vtype, int policy) {
    if (ktype == XQ_TYPE_Q8_0 || ktype == XQ_TYPE_Q4_0) return 2;
    if (ktype == XQ_TYPE_F16) {
        if (policy == XQ_FA_QK_CONSISTENT && vtype == XQ_TYPE_F16) return 0;
        return 1;
    }
    return 0; /* F32, E5M2 */
}

/* The ggml CPU one-chunk loop for one (iq1, iq2, iq3) row, patched with the
 * consistent policies (no split-KV branch, patches/0006-…:7-11; scalar queries,
 * patches/0008-…:40-56). Loop body per KV row ic (patches/0008-…:25-38 and
 * upstream ops.cpp): skip rows whose slope*mask is -inf, s = dot*scale,
 * s = softcap*tanh(s) (scale pre-divided by softcap), s += slope*mask, then
 * the branchy online softmax: a new maximum rescales the accumulator by
 * exp(M_old - s) and adds V with weight 1, otherwise V is added with weight
 * exp(s - M). F16 V accumulates in an f16 vector when v_acc_f16 (each step
 * rounds to f16: ggml_vec_scale_f16, ggml_vec_mad_f16), otherwise in f32. */
static void fa_row(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                   const xq_tensor* mask, const xq_tensor* sinks, const xq_tensor* dst,
                   float* lse, float scale, float max_bias, float softcap, int policy,
                   int v_acc_f16, int64_t iq1, int64_t iq2, int64_t iq3, float* scratch) {
    const int64_t DK = q->ne[0], DV = v->ne[0], L = k->ne[1];
    const int64_t H = q->ne[2], NQ = q->ne[1];
    const int64_t rk2 = H / k->ne[2], rk3 = q->ne[3] / k->ne[3];
    const int64_t rv2 = H / v->ne[2], rv3 = q->ne[3] / v->ne[3];
    const int64_t ik2 = iq2 / rk2, ik3 = iq3 / rk3, iv2 = iq2 / rv2, iv3 = iq3 / rv3;
    const int kind = fa_dot_kind(k->type, v->type, policy);
    const int f16acc = v_acc_f16 && v->type == XQ_TYPE_F16;

    float* qf = scratch;              /* DK: Q as the dot consumes it */
    float* kf = qf + DK;              /* DK: expanded K row */
    float* vkq = kf + DK;             /* DV: f32 accumulator */
    float* vf = vkq + DV;             /* DV: expanded V row */
    uint16_t* vkq16 = (uint16_t*)(vf + DV); /* DV halves */
    uint8_t* qq = (uint8_t*)(vkq16 + DV + 2); /* DK/32 q8_0 blocks */

    const float* pq = (const float*)((const char*)q->data + iq1 * q->nb[1] + iq2 * q->nb[2] +
                                     iq3 * q->nb[3]);
    if (kind == 2) {
        xo_quantize_row_q8_0(pq, qq, DK, 0);
    } else if (kind == 1) {
        for (int64_t i = 0; i < DK; ++i) qf[i] = xo_f16_to_f32(xo_f32_to_f16(pq[i]));
    } else {
        memcpy(qf, pq, (size_t)DK * 4);
    }

    const float slope = xo_alibi_slope(max_bias, (int)H, (int)iq2);
    const uint16_t* mp = NULL;
    if (mask && mask->data)
        mp = (const uint16_t*)((const char*)mask->data + iq1 * mask->nb[1] +
                               (iq2 % mask->ne[2]) * mask->nb[2] + (iq3 % mask->ne[3]) * mask->nb[3]);
    const float sc = softcap != 0.0f ? scale / softcap : scale;

    float M = -INFINITY, S = 0.0f;
    for (int64_t d = 0; d < DV; ++d) {
        vkq[d] = 0.0f;
        vkq16[d] = 0;
    }
    for (int64_t ic = 0; ic < L; ++ic) {
        const float mv = mp ? slope * xo_f16_to_f32(mp[ic]) : 0.0f;
        if (mv == -INFINITY) continue;
        const uint8_t* kd = (const uint8_t*)k->data + ic * k->nb[1] + ik2 * k->nb[2] + ik3 * k->nb[3];
        float s;
        if (kind == 2) {
            s = dot_q_q8(k->type, kd, qq, DK);
        } else {
            xo_dequant_row(k->type, kd, kf, DK);
            s = dot32_f32(qf, kf, DK);
        }
        s = s * sc;
        if (softcap != 0.0f) s = softcap * tanhf(s);
        s = s + mv;

        const float Mold = M;
        float ms = 1.0f, vs = 1.0f;
        const uint8_t* vd = (const uint8_t*)v->data + ic * v->nb[1] + iv2 * v->nb[2] + iv3 * v->nb[3];
        if (f16acc) {
            if (s > M) {
                M = s;
                ms = expf(Mold - M);
                for (int64_t d = 0; d < DV; ++d)
                    vkq16[d] = xo_f32_to_f16(xo_f16_to_f32(vkq16[d]) * ms);
            } else {
                vs = expf(s - M);
            }
            for (int64_t d = 0; d < DV; ++d) {
                uint16_t vh;
                memcpy(&vh, vd + 2 * d, 2);
                vkq16[d] = xo_f32_to_f16(fmaf(xo_f16_to_f32(vh), vs, xo_f16_to_f32(vkq16[d])));
            }
        } else {
            if (s > M) {
                M = s;
                ms = expf(Mold - M);
                for (int64_t d = 0; d < DV; ++d) vkq[d] = vkq[d] * ms;
            } else {
                vs = expf(s - M);
            }
            xo_dequant_row(v->type, vd, vf, DV);
            for (int64_t d = 0; d < DV; ++d) vkq[d] = fmaf(vf[d], vs, vkq[d]);
        }
        S = fmaf(S, ms, vs);
    }
    if (f16acc)
        for (int64_t d = 0; d < DV; ++d) vkq[d] = xo_f16_to_f32(vkq16[d]);

    float Meff = M;
    if (sinks && sinks->data) {
        const float sk = ((const float*)sinks->data)[iq2];
        float ms = 1.0f, vs = 1.0f;
        if (sk > M) {
            ms = expf(M - sk);
            for (int64_t d = 0; d < DV; ++d) vkq[d] = vkq[d] * ms;
            Meff = sk;
        } else {
            vs = expf(sk - M);
        }
        S = fmaf(S, ms, vs);
    }
    const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
    float* out = (float*)((char*)dst->data + iq1 * dst->nb[2] + iq2 * dst->nb[1] + iq3 * dst->nb[3]);
    for (int64_t d = 0; d < DV; ++d) out[d] = vkq[d] * S_inv;
    if (lse) lse[(iq3 * NQ + iq1) * H + iq2] = S > 0.0f ? Meff + logf(S) : -INFINITY;
}

int xo_flash_attn_ext(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                      const xq_tensor* mask, const xq_tensor* sinks, const xq_tensor* dst,
                      float* lse, float scale, float max_bias, float softcap, int qk_policy,
                      int v_acc_f16, int n_threads) {
    if (!fa_shapes_ok(q, k, v, dst)) return 1;
    const int64_t NQ = q->ne[1], H = q->ne[2], B = q->ne[3];
    const int64_t DK = q->ne[0], DV = v->ne[0];
    const int64_t rows = NQ * H * B;
    const size_t scratch_floats = (size_t)(2 * DK + 2 * DV + DV + 8 + DK);
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads)
    {
        float* scratch = (float*)malloc(scratch_floats * sizeof(float) + 64);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            /* same (iq3, iq2, iq1) walk as ggml's ir loop: ir = iq1 + NQ*(iq2 + H*iq3) */
            const int64_t iq3 = r / (H * NQ);
            const int64_t iq2 = (r - iq3 * H * NQ) / NQ;
            const int64_t iq1 = r - iq3 * H * NQ - iq2 * NQ;
            fa_row(q, k, v, mask, sinks, dst, lse, scale, max_bias, softcap, qk_policy, v_acc_f16,
                   iq1, iq2, iq3, scratch);
        }
        free(scratch);
    }
    return 0;
}

int xo_flash_attn_f64(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                      const xq_tensor* mask, const xq_tensor* sinks, double* out, double* lse,
                      float scale, float max_bias, float softcap, int qk_policy, int q_round,
                      int n_threads) {
    if (!q || !k || !v) return 1;
    const int64_t DK = q->ne[0], DV = v->ne[0], L = k->ne[1];
    const int64_t NQ = q->ne[1], H = q->ne[2], B = q->ne[3];
    const int64_t rows = NQ * H * B;
    const int kind = fa_dot_kind(k->type, v->type, qk_policy);
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads)
    {
        float* qf = (float*)malloc((size_t)(DK + DK + DV + 64) * sizeof(float));
        float* kf = qf + DK;
        float* vf = kf + DK;
        uint8_t qq[34 * 64];
        double* sc = (double*)malloc((size_t)(L > 0 ? L : 1) * sizeof(double));
        double* acc = (double*)malloc((size_t)DV * sizeof(double));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            const int64_t iq3 = r / (H * NQ);
            const int64_t iq2 = (r - iq3 * H * NQ) / NQ;
            const int64_t iq1 = r - iq3 * H * NQ - iq2 * NQ;
            const int64_t ik2 = iq2 / (H / k->ne[2]), ik3 = iq3 / (B / k->ne[3]);
            const int64_t iv2 = iq2 / (H / v->ne[2]), iv3 = iq3 / (B / v->ne[3]);
            const float* pq = (const float*)((const char*)q->data + iq1 * q->nb[1] +
                                             iq2 * q->nb[2] + iq3 * q->nb[3]);
            if (q_round && kind == 2) {
                xo_quantize_row_q8_0(pq, qq, DK, 0);
                xo_dequant_row(XQ_TYPE_Q8_0, qq, qf, DK);
            } else if (q_round && kind == 1) {
                for (int64_t i = 0; i < DK; ++i) qf[i] = xo_f16_to_f32(xo_f32_to_f16(pq[i]));
            } else {
                memcpy(qf, pq, (size_t)DK * 4);
            }
            const double slope = (double)xo_alibi_slope(max_bias, (int)H, (int)iq2);
            const uint16_t* mp = NULL;
            if (mask && mask->data)
                mp = (const uint16_t*)((const char*)mask->data + iq1 * mask->nb[1] +
                                       (iq2 % mask->ne[2]) * mask->nb[2] +
                                       (iq3 % mask->ne[3]) * mask->nb[3]);
            double m = -INFINITY;
            for (int64_t ic = 0; ic < L; ++ic) {
                const double mv = mp ? slope * (double)xo_f16_to_f32(mp[ic]) : 0.0;
                if (mv == -INFINITY) {
                    sc[ic] = -INFINITY;
                    continue;
                }
                const uint8_t* kd = (const uint8_t*)k->data + ic * k->nb[1] + ik2 * k->nb[2] +
                                    ik3 * k->nb[3];
                xo_dequant_row(k->type, kd, kf, DK);
                double dot = 0.0;
                for (int64_t i = 0; i < DK; ++i) dot += (double)qf[i] * (double)kf[i];
                double s = dot * (double)scale;
                if (softcap != 0.0f) s = (double)softcap * tanh(s / (double)softcap);
                s += mv;
                sc[ic] = s;
                if (s > m) m = s;
            }
            if (sinks && sinks->data) {
                const double sk = (double)((const float*)sinks->data)[iq2];
                if (sk > m) m = sk;
            }
            double den = 0.0;
            for (int64_t d = 0; d < DV; ++d) acc[d] = 0.0;
            if (m != -INFINITY) {
                for (int64_t ic = 0; ic < L; ++ic) {
                    if (sc[ic] == -INFINITY) continue;
                    const double w = exp(sc[ic] - m);
                    den += w;
                    const uint8_t* vd = (const uint8_t*)v->data + ic * v->nb[1] + iv2 * v->nb[2] +
                                        iv3 * v->nb[3];
                    xo_dequant_row(v->type, vd, vf, DV);
                    for (int64_t d = 0; d < DV; ++d) acc[d] += w * (double)vf[d];
                }
                if (sinks && sinks->data)
                    den += exp((double)((const float*)sinks->data)[iq2] - m);
            }
            double* o = out + ((iq3 * NQ + iq1) * H + iq2) * DV;
            for (int64_t d = 0; d < DV; ++d) o[d] = den > 0.0 ? acc[d] / den : 0.0;
            if (lse) lse[(iq3 * NQ + iq1) * H + iq2] = den > 0.0 ? m + log(den) : -INFINITY;
        }
        free(qf);
        free(sc);
        free(acc);
    }
    return 0;
}

/* ======================================================================
 * RKVA range attention: split policy, pass 1, reducers
 * ==================================================================== */

int32_t xo_ref_split_k(uint32_t active) {
    uint32_t k = (active + 255u) / 256u;
    if (k > 32u) k = 32u;
    return (int32_t)(k < 1u ? 1u : k);
}

int32_t xo_opt_split_k(uint32_t active, uint32_t mode) {
    uint32_t target = 128u, max_splits = 128u; /* balanced (mode 1 and default) */
    if (mode == 2u) {
        target = 32u;
        max_splits = 256u;
    } else if (mode == 3u) {
        target = 512u;
        max_splits = 64u;
    }
    uint32_t want = (uint32_t)(((uint64_t)active + target - 1u) / target);
    if (want > max_splits) want = max_splits;
    if (want > 256u) want = 256u;
    return (int32_t)(want < 1u ? 1u : want);
}

uint32_t xo_split_rows(uint32_t active, uint32_t split_k) {
    return split_k ? (uint32_t)(((uint64_t)active + split_k - 1u) / split_k) : 0u;
}

void xo_q4_mq_split(uint32_t active, uint32_t mode, uint32_t* split_k, uint32_t* rows) {
    const uint32_t k0 = (uint32_t)xo_opt_split_k(active, mode);
    uint32_t r = xo_split_rows(active, k0);
    r = (r + 63u) / 64u * 64u;
    uint32_t k = r ? (uint32_t)(((uint64_t)active + r - 1u) / r) : 1u;
    *split_k = k < 1u ? 1u : k;
    *rows = r;
}

/* rkva_range_attn.hlsl:59-106, one (split, query, head) at a time: the causal
 * limit min(active, pos - origin + 1), rows [s*R, (s+1)*R) of the limit, f32 Q
 * against the decoded K row (sequential f32 dot here; the shader's lane order
 * is not bitwise), and the guarded online update
 *   next = max(M, s); old = den == 0 ? 0 : e^(M-next); w = e^(s-next);
 *   acc = acc*old + w*v; den = den*old + w. */
int xo_range_attn_partials(const float* q, const int32_t* positions, int32_t n_q, int32_t n_head,
                           const void* kp, const void* vp, int32_t n_head_kv, int32_t D,
                           int32_t kv_type, int32_t origin, int32_t active, float kq_scale,
                           int32_t split_k, float* partials) {
    if (n_head % n_head_kv || split_k < 1) return 1;
    const size_t rec = xo_row_bytes(kv_type, D);
    const uint8_t* K = (const uint8_t*)kp;
    const uint8_t* V = (const uint8_t*)vp;
    const uint32_t rows = xo_split_rows((uint32_t)active, (uint32_t)split_k);
    const int32_t total = n_q * n_head;
    float* kf = (float*)malloc((size_t)D * 2 * sizeof(float));
    float* vf = kf + D;
    for (int32_t s = 0; s < split_k; ++s) {
        for (int32_t qh = 0; qh < total; ++qh) {
            const int32_t qi = qh / n_head, head = qh % n_head;
            const int32_t kvh = head / (n_head / n_head_kv);
            const int32_t pos = positions[qi];
            const uint32_t causal = pos < origin ? 0u : (uint32_t)(pos - origin) + 1u;
            const uint32_t limit = (uint32_t)active < causal ? (uint32_t)active : causal;
            uint32_t begin = (uint32_t)s * rows, end = (uint32_t)(s + 1) * rows;
            if (begin > limit) begin = limit;
            if (end > limit) end = limit;
            float* dst = partials + ((size_t)s * total + qh) * (size_t)(D + 2);
            for (int32_t d = 0; d < D; ++d) dst[d] = 0.0f;
            float den = 0.0f, mx = -FLT_MAX;
            const float* qv = q + (size_t)qh * D;
            for (uint32_t r = begin; r < end; ++r) {
                const size_t base = ((size_t)r * n_head_kv + kvh) * rec;
                xo_dequant_row(kv_type, K + base, kf, D);
                float dot = 0.0f;
                for (int32_t d = 0; d < D; ++d) dot = dot + qv[d] * kf[d];
                const float sc = dot * kq_scale;
                const float next = mx > sc ? mx : sc;
                const float old = den == 0.0f ? 0.0f : expf(mx - next);
                const float w = expf(sc - next);
                xo_dequant_row(kv_type, V + base, vf, D);
                for (int32_t d = 0; d < D; ++d) dst[d] = dst[d] * old + w * vf[d];
                den = den * old + w;
                mx = next;
            }
            dst[D] = mx;
            dst[D + 1] = den;
        }
    }
    free(kf);
    return 0;
}

/* Ascending-split merge (the consistent KV-reduction order):
 *  M = max{m_s : den_s participates}; L = sum den_s e^(m_s - M);
 *  O = (sum acc_s e^(m_s - M)) * (L > 0 ? 1/L : 0); LSE = L > 0 ? M + ln L : -inf.
 * poison == 0: rkva_range_reduce.hlsl:12-46 (den > 0 participates).
 * poison == 1: rkva_range_reduce_opt.hlsl:25-133 (den != 0 participates; any
 * non-finite or negative participating den/max, non-finite numerator, sum,
 * 1/sum or LSE, or more than 256 splits, turns the whole row into NaN). */
int xo_range_reduce(const float* partials, int32_t n_qh, int32_t D, int32_t split_k,
                    int32_t poison, float* out, float* lse) {
    const size_t stride = (size_t)D + 2;
    for (int32_t qh = 0; qh < n_qh; ++qh) {
        float* o = out + (size_t)qh * D;
        if (!poison) {
            float M = -FLT_MAX;
            for (int32_t s = 0; s < split_k; ++s) {
                const float* p = partials + ((size_t)s * n_qh + qh) * stride;
                if (p[D + 1] > 0.0f && p[D] > M) M = p[D];
            }
            float sum = 0.0f;
            for (int32_t s = 0; s < split_k; ++s) {
                const float* p = partials + ((size_t)s * n_qh + qh) * stride;
                if (p[D + 1] > 0.0f) sum = sum + p[D + 1] * expf(p[D] - M);
            }
            const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
            lse[qh] = sum > 0.0f ? M + logf(sum) : -INFINITY;
            for (int32_t d = 0; d < D; ++d) {
                float acc = 0.0f;
                for (int32_t s = 0; s < split_k; ++s) {
                    const float* p = partials + ((size_t)s * n_qh + qh) * stride;
                    if (p[D + 1] > 0.0f) acc = acc + p[d] * expf(p[D] - M);
                }
                o[d] = acc * inv;
            }
            continue;
        }
        const int32_t splits = split_k < 256 ? split_k : 256;
        int invalid = split_k > 256;
        float M = -FLT_MAX;
        for (int32_t s = 0; s < splits; ++s) {
            const float* p = partials + ((size_t)s * n_qh + qh) * stride;
            const float den = p[D + 1];
            if (den == 0.0f) continue;
            if (!isfinite(den) || den < 0.0f || !isfinite(p[D]))
                invalid = 1;
            else if (p[D] > M)
                M = p[D];
        }
        float inv = 0.0f;
        if (!invalid) {
            float sum = 0.0f;
            for (int32_t s = 0; s < splits; ++s) {
                const float* p = partials + ((size_t)s * n_qh + qh) * stride;
                if (p[D + 1] != 0.0f) sum = sum + p[D + 1] * expf(p[D] - M);
            }
            inv = sum == 0.0f ? 0.0f : 1.0f / sum;
            if (!isfinite(sum) || sum < 0.0f || !isfinite(inv)) invalid = 1;
            const float l = sum == 0.0f ? -INFINITY : M + logf(sum);
            if (sum != 0.0f && !isfinite(l)) invalid = 1;
            lse[qh] = l;
        }
        for (int32_t d = 0; d < D && !invalid; ++d) {
            float acc = 0.0f;
            for (int32_t s = 0; s < splits; ++s) {
                const float* p = partials + ((size_t)s * n_qh + qh) * stride;
                if (p[D + 1] != 0.0f) {
                    if (!isfinite(p[d])) invalid = 1;
                    acc = acc + p[d] * expf(p[D] - M);
                }
            }
            o[d] = acc * inv;
            if (!isfinite(o[d])) invalid = 1;
        }
        if (invalid) {
            for (int32_t d = 0; d < D; ++d) o[d] = NAN;
            lse[qh] = NAN;
        }
    }
    return 0;
}

/* Merge of position-split range results: parts p = 0..n_parts-1 hold OUT
 * [rows][D] and natural-log LSE [rows] of the same (query, head) rows over
 * disjoint KV ranges (the result contract of uwp/rkva/remote-attn-protocol.h:
 * 228-231: an empty range gives O = 0, LSE = -inf). A part takes part when its
 * LSE is not -inf (the reducer's den != 0); weights e^{LSE_p - M}, M the
 * largest such LSE, accumulate in part order; a participating NaN / +inf LSE
 * or a non-finite result poisons the row with NaN, as
 * shaders/rkva/rkva_range_reduce_opt.hlsl:39-56,126-132 does for splits. */
int xo_lse_merge(const float* parts_out, const float* parts_lse, int32_t n_parts, int64_t rows,
                 int32_t D, float* out, float* lse) {
    for (int64_t r = 0; r < rows; ++r) {
        float* o = out + (size_t)r * D;
        int invalid = 0, any = 0;
        float M = -FLT_MAX;
        for (int32_t p = 0; p < n_parts; ++p) {
            const float l = parts_lse[(size_t)p * rows + r];
            if (l == -INFINITY) continue;
            if (!isfinite(l))
                invalid = 1;
            else {
                any = 1;
                if (l > M) M = l;
            }
        }
        if (!invalid && !any) {
            for (int32_t d = 0; d < D; ++d) o[d] = 0.0f;
            lse[r] = -INFINITY;
            continue;
        }
        float sum = 0.0f;
        if (!invalid)
            for (int32_t p = 0; p < n_parts; ++p) {
                const float l = parts_lse[(size_t)p * rows + r];
                if (l != -INFINITY) sum = sum + expf(l - M);
            }
        const float inv = invalid ? 0.0f : 1.0f / sum;
        const float lv = invalid ? NAN : M + logf(sum);
        if (!isfinite(lv) || !isfinite(inv)) invalid = 1;
        for (int32_t d = 0; d < D && !invalid; ++d) {
            float acc = 0.0f;
            for (int32_t p = 0; p < n_parts; ++p) {
                const float l = parts_lse[(size_t)p * rows + r];
                if (l != -INFINITY) acc = acc + parts_out[((size_t)p * rows + r) * D + d] * expf(l - M);
            }
            o[d] = acc * inv;
            if (!isfinite(o[d])) invalid = 1;
        }
        if (invalid) {
            for (int32_t d = 0; d < D; ++d) o[d] = NAN;
            lse[r] = NAN;
        } else {
            lse[r] = lv;
        }
    }
    return 0;
}

/* ======================================================================
 * gated delta net
 * ==================================================================== */

static inline float gdn_at(const xq_tensor* t, int64_t b, int64_t tok, int64_t head, int64_t i) {
    const char* p = (const char*)t->data + b * t->nb[3] + tok * t->nb[2] + head * t->nb[1];
    if (t->type == XQ_TYPE_BF16) {
        uint16_t h;
        memcpy(&h, p + 2 * i, 2);
        return xo_bf16_to_f32(h);
    }
    float f;
    memcpy(&f, p + 4 * i, 4);
    return f;
}

/* tree of d3d12_gdn_emulate's reduce lambda: strides 4, 2, 1 over 8 partials */
static inline float reduce8(float p[8]) {
    for (int stride = 4; stride > 0; stride >>= 1)
        for (int l = 0; l < stride; ++l) p[l] = p[l] + p[l + stride];
    return p[0];
}

static int gdn_shapes_ok(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                         const xq_tensor* g, const xq_tensor* beta, const xq_tensor* state,
                         int32_t slots) {
    if (!q || !k || !v || !g || !beta || !state) return 0;
    if (slots < 1 || slots > 17) return 0;
    if (q->ne[0] != 128 || q->ne[1] != 16 || k->ne[0] != 128 || k->ne[1] != 16) return 0;
    if (v->ne[0] != 128 || v->ne[1] != 32) return 0;
    if (state->ne[0] != 128 || state->ne[1] != 128 || state->ne[2] != 32) return 0;
    return 1;
}

/* src/bridge/ggml_d3d12.cpp:113-158 per sequence b: v-head h reads q/k head
 * h % 16; per token: decay = exp(g); per value column c: s *= decay,
 * kv = 8-lane partial sums of s*k (lane i % 8) folded 4-2-1,
 * delta = (v - kv) * beta, s += k*delta, y = folded 8-lane sums of s*q times
 * 1/sqrt(128); after token t the state is the snapshot of slot T-1-t when that
 * slot is kept (all slots < K for K > 1, only the final one for K == 1). */
int xo_gated_delta_net(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                       const xq_tensor* g, const xq_tensor* beta, const xq_tensor* state,
                       const xq_tensor* dst, int32_t slots, int n_threads) {
    if (!gdn_shapes_ok(q, k, v, g, beta, state, slots) || !dst) return 1;
    const int64_t T = v->ne[2], B = v->ne[3] > 0 ? v->ne[3] : 1;
    const float scale = 1.0f / sqrtf(128.0f);
    const size_t s_off = (size_t)4096 * T;
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t bh = 0; bh < B * 32; ++bh) {
        const int64_t b = bh / 32, head = bh % 32, kh = head % 16;
        float* st = (float*)malloc(128 * 128 * sizeof(float));
        float qv[128], kvv[128];
        const float* init = (const float*)((const char*)state->data + b * state->nb[3]) + head * 16384;
        memcpy(st, init, 128 * 128 * sizeof(float));
        float* out = (float*)((char*)dst->data + b * dst->nb[2]);
        for (int64_t t = 0; t < T; ++t) {
            const float decay = expf(gdn_at(g, b, t, head, 0));
            const float bt = gdn_at(beta, b, t, head, 0);
            for (int i = 0; i < 128; ++i) {
                qv[i] = gdn_at(q, b, t, kh, i);
                kvv[i] = gdn_at(k, b, t, kh, i);
            }
            for (int col = 0; col < 128; ++col) {
                float kv[8] = {0}, at[8] = {0};
                float* s = st + col * 128;
                for (int i = 0; i < 128; ++i) {
                    s[i] = s[i] * decay;
                    kv[i % 8] = kv[i % 8] + s[i] * kvv[i];
                }
                const float delta = (gdn_at(v, b, t, head, col) - reduce8(kv)) * bt;
                for (int i = 0; i < 128; ++i) {
                    s[i] = s[i] + kvv[i] * delta;
                    at[i % 8] = at[i % 8] + s[i] * qv[i];
                }
                out[(t * 32 + head) * 128 + col] = reduce8(at) * scale;
            }
            const int64_t slot = T - 1 - t;
            if ((slots > 1 && slot < slots) || (slots == 1 && t + 1 == T))
                memcpy(out + s_off + (size_t)(slots == 1 ? 0 : slot) * 524288 + head * 16384, st,
                       128 * 128 * sizeof(float));
        }
        free(st);
    }
    return 0;
}

int xo_gated_delta_net_f64(const xq_tensor* q, const xq_tensor* k, const xq_tensor* v,
                           const xq_tensor* g, const xq_tensor* beta, const xq_tensor* state,
                           double* dst, int32_t slots, int n_threads) {
    if (!gdn_shapes_ok(q, k, v, g, beta, state, slots) || !dst) return 1;
    const int64_t T = v->ne[2], B = v->ne[3] > 0 ? v->ne[3] : 1;
    const double scale = 1.0 / sqrt(128.0);
    const size_t per_seq = (size_t)4096 * (size_t)(T + (int64_t)slots * 128);
    const size_t s_off = (size_t)4096 * T;
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t bh = 0; bh < B * 32; ++bh) {
        const int64_t b = bh / 32, head = bh % 32, kh = head % 16;
        double* st = (double*)malloc(128 * 128 * sizeof(double));
        double qv[128], kvv[128];
        const float* init = (const float*)((const char*)state->data + b * state->nb[3]) + head * 16384;
        for (int i = 0; i < 128 * 128; ++i) st[i] = (double)init[i];
        double* out = dst + (size_t)b * per_seq;
        for (int64_t t = 0; t < T; ++t) {
            const double decay = exp((double)gdn_at(g, b, t, head, 0));
            const double bt = (double)gdn_at(beta, b, t, head, 0);
            for (int i = 0; i < 128; ++i) {
                qv[i] = (double)gdn_at(q, b, t, kh, i);
                kvv[i] = (double)gdn_at(k, b, t, kh, i);
            }
            for (int col = 0; col < 128; ++col) {
                double* s = st + col * 128;
                double kv = 0.0, at = 0.0;
                for (int i = 0; i < 128; ++i) {
                    s[i] *= decay;
                    kv += s[i] * kvv[i];
                }
                const double delta = ((double)gdn_at(v, b, t, head, col) - kv) * bt;
                for (int i = 0; i < 128; ++i) {
                    s[i] += kvv[i] * delta;
                    at += s[i] * qv[i];
                }
                out[(t * 32 + head) * 128 + col] = at * scale;
            }
            const int64_t slot = T - 1 - t;
            if ((slots > 1 && slot < slots) || (slots == 1 && t + 1 == T)) {
                double* snap = out + s_off + (size_t)(slots == 1 ? 0 : slot) * 524288 + head * 16384;
                memcpy(snap, st, 128 * 128 * sizeof(double));
            }
        }
        free(st);
    }
    return 0;
}

/* ======================================================================
 * KV append (shaders/rkva/rkva_store_f16.hlsl:63-85 widened to every type)
 * ==================================================================== */

int xo_kv_store(const float* src, const int32_t* positions, int32_t n_tokens, int32_t n_head_kv,
                int32_t D, int32_t kv_type, int32_t q8_variant, void* dst, int32_t capacity) {
    const size_t rec = xo_row_bytes(kv_type, D);
    if (!rec) return 1;
    uint8_t* out = (uint8_t*)dst;
    for (int32_t t = 0; t < n_tokens; ++t) {
        const int32_t pos = positions[t];
        if (pos < 0 || pos >= capacity) continue;
        for (int32_t h = 0; h < n_head_kv; ++h) {
            const float* x = src + ((size_t)t * n_head_kv + h) * D;
            uint8_t* y = out + ((size_t)pos * n_head_kv + h) * rec;
            switch (kv_type) {
            case XQ_TYPE_F32: memcpy(y, x, (size_t)D * 4); break;
            case XQ_TYPE_F16: xo_f32_to_f16_row(x, (uint16_t*)(void*)y, D); break;
            case XQ_TYPE_BF16: xo_f32_to_bf16_row(x, (uint16_t*)(void*)y, D); break;
            case XQ_TYPE_Q8_0: xo_quantize_row_q8_0(x, y, D, q8_variant); break;
            case XQ_TYPE_Q4_0: xo_quantize_row_q4_0(x, y, D); break;
            case XQ_TYPE_E5M2: xo_f32_to_e5m2_row(x, y, D); break;
            default: return 1;
            }
        }
    }
    return 0;
}
