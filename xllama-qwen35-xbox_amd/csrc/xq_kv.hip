// xq_kv.hip — KV append: F32 rows -> KV cache records at row positions.
//
// The scatter of shaders/rkva/rkva_store_f16.hlsl:63-85 (F32 -> ggml F16 RNE at
// absolute positions) widened to every KV storage type of this path, with
// ggml's block quantizers reproduced bit for bit:
//   Q8_0  quantize_row_q8_0 (x86: id = 127/amax, round half to even) or
//         quantize_row_q8_0_ref (id = 1/d, roundf);
//   Q4_0  quantize_row_q4_0_ref (d = max/-8 with max the first element of
//         largest magnitude, q = min(15, (int8)(x*id + 8.5)));
//   E5M2  f16 RNE then E5M2 RNE with finite saturation (the Q/OUT wire codec of
//         shaders/rkva/rkva_range_bulk_f16.hlsl:156-167).
// One wave per (token, KV head) record. Built with -ffp-contract=off so the
// q4_0 "x*id + 8.5" rounds twice, as the CPU reference does.
#include "xq_kernels.h"

namespace xq {

XQ_DEV uint32_t f16_to_e5m2(uint32_t h) {
    const uint32_t sign = (h >> 8) & 0x80u;
    if ((h & 0x7c00u) == 0x7c00u) {
        if (!(h & 0x03ffu)) return sign | 0x7cu;
        const uint32_t top = (h >> 8) & 3u;
        return sign | 0x7cu | (top ? top : 1u);
    }
    uint32_t mag = h & 0x7fffu;
    if (mag > 0x7b00u) mag = 0x7b00u;
    return sign | ((mag + 0x7fu + ((mag >> 8) & 1u)) >> 8);
}

XQ_DEV uint32_t f32_to_bf16_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 64u) & 0xffffu;
    return ((u + (0x7fffu + ((u >> 16) & 1u))) >> 16) & 0xffffu;
}

template <int D>
__global__ __launch_bounds__(64) void kv_store_kernel(const float* __restrict__ src,
                                                      const int32_t* __restrict__ positions,
                                                      int32_t n_head_kv, int32_t kv_type,
                                                      int32_t q8_variant, uint8_t* __restrict__ dst,
                                                      int32_t capacity) {
    constexpr int VD = D / 64;
    const int rec_id = blockIdx.x;
    const int t = rec_id / n_head_kv, h = rec_id % n_head_kv;
    const int32_t pos = positions[t];
    if (pos < 0 || pos >= capacity) return;
    const int lane = threadIdx.x;
    const float* x = src + ((int64_t)t * n_head_kv + h) * D;
    float xv[VD];
#pragma unroll
    for (int j = 0; j < VD; ++j) xv[j] = x[lane * VD + j];
    __shared__ float sx[D];

    if (kv_type == XQ_TYPE_F32) {
        float* y = (float*)(dst + ((int64_t)pos * n_head_kv + h) * (4 * D));
#pragma unroll
        for (int j = 0; j < VD; ++j) y[lane * VD + j] = xv[j];
    } else if (kv_type == XQ_TYPE_F16 || kv_type == XQ_TYPE_BF16) {
        uint16_t* y = (uint16_t*)(dst + ((int64_t)pos * n_head_kv + h) * (2 * D));
#pragma unroll
        for (int j = 0; j < VD; ++j)
            y[lane * VD + j] = (uint16_t)(kv_type == XQ_TYPE_F16 ? f32_to_f16_bits(xv[j]) : f32_to_bf16_bits(xv[j]));
    } else if (kv_type == XQ_TYPE_E5M2) {
        uint8_t* y = dst + ((int64_t)pos * n_head_kv + h) * D;
#pragma unroll
        for (int j = 0; j < VD; ++j) y[lane * VD + j] = (uint8_t)f16_to_e5m2(f32_to_f16_bits(xv[j]));
    } else if (kv_type == XQ_TYPE_Q8_0) {
        uint8_t* y = dst + ((int64_t)pos * n_head_kv + h) * (D / kQK * 34);
#pragma unroll
        for (int j = 0; j < VD; ++j) sx[lane * VD + j] = xv[j];
        __syncthreads();
        if (lane < D / kQK) {
            const float* xb = sx + lane * kQK;
            float amax = 0.0f;
            for (int j = 0; j < kQK; ++j) amax = fmaxf(amax, fabsf(xb[j]));
            const float d = amax / 127.0f;
            float id;
            if (q8_variant == 0)
                id = amax != 0.0f ? 127.0f / amax : 0.0f;
            else
                id = d != 0.0f ? 1.0f / d : 0.0f;
            uint8_t* yb = y + lane * 34;
            const uint32_t dh = f32_to_f16_bits(d);
            yb[0] = (uint8_t)(dh & 0xffu);
            yb[1] = (uint8_t)(dh >> 8);
            for (int j = 0; j < kQK; ++j) {
                const float tq = xb[j] * id;
                const float r = q8_variant == 0 ? rintf(tq) : roundf(tq);
                yb[2 + j] = (uint8_t)(int8_t)(int)r;
            }
        }
    } else if (kv_type == XQ_TYPE_Q4_0) {
        uint8_t* y = dst + ((int64_t)pos * n_head_kv + h) * (D / kQK * 18);
#pragma unroll
        for (int j = 0; j < VD; ++j) sx[lane * VD + j] = xv[j];
        __syncthreads();
        if (lane < D / kQK) {
            const float* xb = sx + lane * kQK;
            float amax = 0.0f, vmax = 0.0f;
            for (int j = 0; j < kQK; ++j) {
                if (amax < fabsf(xb[j])) {
                    amax = fabsf(xb[j]);
                    vmax = xb[j];
                }
            }
            const float d = vmax / -8.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint8_t* yb = y + lane * 18;
            const uint32_t dh = f32_to_f16_bits(d);
            yb[0] = (uint8_t)(dh & 0xffu);
            yb[1] = (uint8_t)(dh >> 8);
            for (int j = 0; j < kQK / 2; ++j) {
                const float t0 = xb[j] * id;
                const float t1 = xb[j + kQK / 2] * id;
                int lo = (int8_t)(t0 + 8.5f);
                int hi = (int8_t)(t1 + 8.5f);
                lo = lo > 15 ? 15 : lo;
                hi = hi > 15 ? 15 : hi;
                yb[2 + j] = (uint8_t)(lo | (hi << 4));
            }
        }
    }
}

hipError_t kv_store_launch(const float* src, const int32_t* positions, int32_t n_tokens,
                           int32_t n_head_kv, int32_t head_dim, int32_t kv_type,
                           int32_t q8_variant, void* dst, int32_t capacity, hipStream_t stream) {
    const dim3 grid((uint32_t)n_tokens * (uint32_t)n_head_kv);
    if (grid.x == 0) return hipSuccess;
    switch (head_dim) {
    case 64:
        launch("kv_store", kv_store_kernel<64>, grid, dim3(64), stream, src, positions, n_head_kv, kv_type, q8_variant,
               (uint8_t*)dst, capacity);
        break;
    case 128:
        launch("kv_store", kv_store_kernel<128>, grid, dim3(64), stream, src, positions, n_head_kv, kv_type, q8_variant,
               (uint8_t*)dst, capacity);
        break;
    case 256:
        launch("kv_store", kv_store_kernel<256>, grid, dim3(64), stream, src, positions, n_head_kv, kv_type, q8_variant,
               (uint8_t*)dst, capacity);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace xq
