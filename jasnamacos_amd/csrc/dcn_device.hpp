// Device helpers shared by the fused FP16 kernel files (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "dcn_internal.hpp"

namespace dcn {
namespace dev {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPad = DCN_CB8_PAD;         // zero border of the CB8 input planes
constexpr int kBufferFlags = 0x00020000;  // raw buffer resource, gfx9 family

// Buffer resource over [p, p + bytes): loads outside the range return zero instead of
// faulting, so every gather is bounds-checked by the hardware.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                             kBufferFlags);
}
__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                        uint32_t soff = 0) {
    return __builtin_bit_cast(u32x4,
                              __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ float load_half(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                           uint32_t soff = 0) {
    const short v = __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
    return (float)__builtin_bit_cast(_Float16, v);
}
// A BF16 value widened exactly: its 16 bits are the high half of the FP32 value.
__device__ __forceinline__ float load_bf16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                           uint32_t soff = 0) {
    const short v = __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
    return __builtin_bit_cast(float, (uint32_t)(uint16_t)v << 16);
}

// floor(x / d) for 0 <= x < 2^16 and 0 < d < 2^16, magic = ceil(2^32 / d) for d > 1
// and 0 for d == 1 (magic_for on the host).
__device__ __forceinline__ int fast_div(int x, uint32_t magic) {
    return magic ? (int)__umulhi((uint32_t)x, magic) : x;
}

// -0.0f the compiler cannot see (so that fma(x, y, -0) is not turned into a multiply).
__device__ __forceinline__ float opaque_neg_zero() {
    float z;
    asm("v_mov_b32 %0, 0x80000000" : "=v"(z));
    return z;
}

// Reference arithmetic (MetalShader.swift:369-379): FP32 bilinear in the reference's
// association, times the mask, rounded once to FP16. Eight channels of one sample.
// Each corner's first product, float(v) * (1 - ly) or float(v) * ly, is an fma with -0:
// x * y + (-0) is x * y exactly, signed zeros included, and v_fma_mix_f32 widens the FP16
// corner inside it (one instruction instead of a conversion and a multiply).
__device__ __forceinline__ h8 blend_exact(u32x4 q00, u32x4 q01, u32x4 q10, u32x4 q11, float ly,
                                          float lx, float m) {
    const h8 a = __builtin_bit_cast(h8, q00), b = __builtin_bit_cast(h8, q01);
    const h8 c = __builtin_bit_cast(h8, q10), d = __builtin_bit_cast(h8, q11);
    const float oy = 1.0f - ly, ox = 1.0f - lx, nz = opaque_neg_zero();
    h8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float s = __builtin_fmaf((float)a[e], oy, nz) * ox + __builtin_fmaf((float)b[e], oy, nz) * lx +
                        __builtin_fmaf((float)c[e], ly, nz) * ox + __builtin_fmaf((float)d[e], ly, nz) * lx;
        r[e] = round_f16(s * m);
    }
    return r;
}

// Mask folded into the four FP32 bilinear weights, each rounded once to FP16, then a
// packed-FP16 blend: 4 conversions + 16 packed FMAs per 8 channels.
__device__ __forceinline__ h8 blend_fast(u32x4 q00, u32x4 q01, u32x4 q10, u32x4 q11, float ly,
                                         float lx, float m) {
    const float t0 = m * (1.0f - ly);
    const float t1 = m * ly;
    const h8 w00 = (_Float16)(t0 * (1.0f - lx));  // scalar -> all 8 lanes
    const h8 w01 = (_Float16)(t0 * lx);
    const h8 w10 = (_Float16)(t1 * (1.0f - lx));
    const h8 w11 = (_Float16)(t1 * lx);
    h8 r = w00 * __builtin_bit_cast(h8, q00);
    r = __builtin_elementwise_fma(w01, __builtin_bit_cast(h8, q01), r);
    r = __builtin_elementwise_fma(w10, __builtin_bit_cast(h8, q10), r);
    r = __builtin_elementwise_fma(w11, __builtin_bit_cast(h8, q11), r);
    return r;
}

// blend_exact for BF16 storage: the eight BF16 channels of each corner widened exactly,
// the same FP32 arithmetic and association, each sample rounded once to BF16. Returns
// the eight BF16 values' bits in an h8 (the MFMA operand register layout is the same).
__device__ __forceinline__ h8 blend_bf16(u32x4 q00, u32x4 q01, u32x4 q10, u32x4 q11, float ly,
                                         float lx, float m) {
    u32x4 r;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t packed = 0u;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // channel 2d + h: the low (h = 0) or high (h = 1) 16 bits of dword d
            auto widen = [&](uint32_t w) {
                return __builtin_bit_cast(float, h ? (w & 0xffff0000u) : (w << 16));
            };
            const float s = widen(q00[d]) * (1.0f - ly) * (1.0f - lx) +
                            widen(q01[d]) * (1.0f - ly) * lx + widen(q10[d]) * ly * (1.0f - lx) +
                            widen(q11[d]) * ly * lx;
            packed |= (uint32_t)round_bf16_bits(s * m) << (16 * h);
        }
        r[d] = packed;
    }
    return __builtin_bit_cast(h8, r);
}

template <int SAMPLER>
__device__ __forceinline__ h8 blend(u32x4 q00, u32x4 q01, u32x4 q10, u32x4 q11, float ly, float lx,
                                    float m) {
    if constexpr (SAMPLER == kSamplerBf16) return blend_bf16(q00, q01, q10, q11, ly, lx, m);
    return SAMPLER == kSamplerExact ? blend_exact(q00, q01, q10, q11, ly, lx, m)
                                    : blend_fast(q00, q01, q10, q11, ly, lx, m);
}

}  // namespace dev
}  // namespace dcn
