// Device helpers shared by the gfx950 kernels: vector types, fp16
// rounding, uniform scalar loads and the rotate-half rotary of one 8-dim
// chunk.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace pvlc {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8_t __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4_t __attribute__((ext_vector_type(4)));


__device__ inline _Float16 to_h(float f) { return static_cast<_Float16>(f); }

// Read a wave-uniform element of a buffer the kernel never writes (block
// tables, cache lengths, positions) through the constant address space, so
// it becomes a scalar load that does not wait behind the vector loads.
__device__ inline int32_t load_const(const int32_t *base, size_t index) {
    typedef const __attribute__((address_space(4))) int32_t *constant_ptr;
    return ((constant_ptr)base)[index];
}

// Rotate-half of 8 consecutive dims [d0, d0+8) of one head row:
// x'[d] = x[d]*cos + partner*sin with partner = -x[d+64] (d < 64) or x[d-64],
// exactly the f32 expression of apply_rope_neox / apply_multimodal_rope_f32
// (cpu-ref lib.rs:459-463, :645-654); each product and the sum are rounded
// separately (this file is compiled without FP contraction), then RNE to fp16.
__device__ inline half8_t rotate_chunk(const uint16_t *row, int d0, const float *cos_row, const float *sin_row) {
    const half8_t x = *reinterpret_cast<const half8_t *>(row + d0);
    const half8_t y = *reinterpret_cast<const half8_t *>(row + (d0 < 64 ? d0 + 64 : d0 - 64));
    const float4_t c0 = *reinterpret_cast<const float4_t *>(cos_row + (d0 & 63));
    const float4_t c1 = *reinterpret_cast<const float4_t *>(cos_row + (d0 & 63) + 4);
    const float4_t s0 = *reinterpret_cast<const float4_t *>(sin_row + (d0 & 63));
    const float4_t s1 = *reinterpret_cast<const float4_t *>(sin_row + (d0 & 63) + 4);
    const float sign = d0 < 64 ? -1.0f : 1.0f;
    half8_t r;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float c = j < 4 ? c0[j] : c1[j - 4];
        const float s = j < 4 ? s0[j] : s1[j - 4];
        const float xc = static_cast<float>(x[j]) * c;
        const float ps = (sign * static_cast<float>(y[j])) * s;
        r[j] = to_h(xc + ps);
    }
    return r;
}

// The same rotation of an f32 row (the f32-operand entry points): the same
// products and sum from the f32 values, one RNE rounding to fp16.
__device__ inline half8_t rotate_chunk(const float *row, int d0, const float *cos_row, const float *sin_row) {
    const int dp = d0 < 64 ? d0 + 64 : d0 - 64;
    const float4_t x0 = *reinterpret_cast<const float4_t *>(row + d0);
    const float4_t x1 = *reinterpret_cast<const float4_t *>(row + d0 + 4);
    const float4_t y0 = *reinterpret_cast<const float4_t *>(row + dp);
    const float4_t y1 = *reinterpret_cast<const float4_t *>(row + dp + 4);
    const float4_t c0 = *reinterpret_cast<const float4_t *>(cos_row + (d0 & 63));
    const float4_t c1 = *reinterpret_cast<const float4_t *>(cos_row + (d0 & 63) + 4);
    const float4_t s0 = *reinterpret_cast<const float4_t *>(sin_row + (d0 & 63));
    const float4_t s1 = *reinterpret_cast<const float4_t *>(sin_row + (d0 & 63) + 4);
    const float sign = d0 < 64 ? -1.0f : 1.0f;
    half8_t r;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float c = j < 4 ? c0[j] : c1[j - 4];
        const float s = j < 4 ? s0[j] : s1[j - 4];
        const float xc = (j < 4 ? x0[j] : x1[j - 4]) * c;
        const float ps = (sign * (j < 4 ? y0[j] : y1[j - 4])) * s;
        r[j] = to_h(xc + ps);
    }
    return r;
}

// 8 consecutive f32 values rounded (RNE) to fp16.
__device__ inline half8_t round_chunk(const float *src) {
    const float4_t a = *reinterpret_cast<const float4_t *>(src);
    const float4_t b = *reinterpret_cast<const float4_t *>(src + 4);
    half8_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        r[j] = to_h(a[j]);
        r[j + 4] = to_h(b[j]);
    }
    return r;
}

// A DPP move of a float within the rows of 16 lanes (CTRL: the dpp_ctrl
// encoding, all rows and banks enabled).
template <int CTRL>
__device__ inline float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a wave, returned in every lane (a wave-uniform
// value).  DPP moves within each 16-lane row (xor 1 and xor 2 inside quads,
// then rotations by 4 and 8: every lane holds its row's sum), then the four
// row sums read from lanes 0, 16, 32 and 48.  A butterfly of __shfl_xor
// compiles to six dependent LDS permutes instead.
__device__ inline float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x124>(v);  // row_ror:4
    v += dpp_f32<0x128>(v);  // row_ror:8
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

}  // namespace pvlc
