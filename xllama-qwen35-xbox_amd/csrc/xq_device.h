// xq_device.h — device helpers shared by the gfx950 kernels: storage decoders,
// wave64 reductions (DPP inside 16-lane rows, then four readlanes), and the
// XCD-aware workgroup remap.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "xq_attn.h"

#define XQ_DEV __device__ __forceinline__

namespace xq {

constexpr int kWave = 64;

// ---------------------------------------------------------------- decoders

XQ_DEV float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
XQ_DEV float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
// E5M2 is the upper byte of an IEEE half: decode through f16 exactly.
XQ_DEV float e5m2_to_f32(uint32_t b) { return f16_bits_to_f32((b & 0xffu) << 8); }

// f32 -> f16 bits, round to nearest even (hardware v_cvt_f16_f32 in the
// default rounding mode). NaN is canonicalised to 0x7e00|sign to match ggml's
// host conversion.
XQ_DEV uint32_t f32_to_f16_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t h = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
    // a select, not a branch: callers convert whole rows with their loads in flight
    return (u & 0x7fffffffu) > 0x7f800000u ? ((u >> 16) & 0x8000u) | 0x7e00u : h;
}

// Sign-extended int8 lane k (0..3) of a dword.
XQ_DEV int sbyte(uint32_t w, int k) { return ((int)(w << (24 - 8 * k))) >> 24; }

// ---------------------------------------------------------------- reductions

template <int CTRL>
XQ_DEV float dpp(float x) {
    return __builtin_amdgcn_update_dpp(0.0f, x, CTRL, 0xf, 0xf, false);
}

// After these four steps every lane of a 16-lane row holds the row's total
// (bitwise identical in all 16 lanes: each step adds commutative pairs).
XQ_DEV float row16_sum(float x) {
    x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
    x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
    x += dpp<0x141>(x);  // row_half_mirror
    x += dpp<0x140>(x);  // row_mirror
    return x;
}
XQ_DEV float row16_max(float x) {
    x = fmaxf(x, dpp<0xB1>(x));
    x = fmaxf(x, dpp<0x4E>(x));
    x = fmaxf(x, dpp<0x141>(x));
    x = fmaxf(x, dpp<0x140>(x));
    return x;
}
template <int CTRL>
XQ_DEV int dpp_i(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, false);
}
// Order-preserving float <-> int map (valid for every non-NaN float): integer
// max then equals float max, without the IEEE canonicalisation fmaxf needs.
XQ_DEV int f2ord(float x) {
    const int i = __float_as_int(x);
    return i >= 0 ? i : i ^ 0x7fffffff;
}
XQ_DEV float ord2f(int i) { return __int_as_float(i >= 0 ? i : i ^ 0x7fffffff); }
// Row-of-16 maximum (exact) via integer DPP max.
XQ_DEV float row16_max_ord(float x) {
    int i = f2ord(x);
    i = max(i, dpp_i<0xB1>(i));
    i = max(i, dpp_i<0x4E>(i));
    i = max(i, dpp_i<0x141>(i));
    i = max(i, dpp_i<0x140>(i));
    return ord2f(i);
}

XQ_DEV float lane_read(float x, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}
// Wave-uniform totals in a fixed order: (r0 + r1) + (r2 + r3) over the rows.
XQ_DEV float wave_sum(float x) {
    x = row16_sum(x);
    return (lane_read(x, 0) + lane_read(x, 16)) + (lane_read(x, 32) + lane_read(x, 48));
}
XQ_DEV float wave_max(float x) {
    x = row16_max(x);
    return fmaxf(fmaxf(lane_read(x, 0), lane_read(x, 16)), fmaxf(lane_read(x, 32), lane_read(x, 48)));
}

XQ_DEV int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); }
XQ_DEV int lane_id() { return threadIdx.x & (kWave - 1); }

// ---------------------------------------------------------------- XCD remap

// Workgroups are dealt round-robin to the 8 XCDs (each with its own L2). Map
// the hardware id to a logical id so that consecutive logical ids run on the
// same XCD; exact bijection on [0, n).
XQ_DEV uint32_t xcd_remap(uint32_t w, uint32_t n) {
    const uint32_t q = n >> 3, r = n & 7u;
    const uint32_t xcd = w & 7u, slot = w >> 3;
    return xcd < r ? xcd * (q + 1u) + slot : r * (q + 1u) + (xcd - r) * q + slot;
}

}  // namespace xq
