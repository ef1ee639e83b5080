// Bilinear warps of FP16 planes shared by the body kernels: the temporal preparation
// (dcn_kernels_body.hip) and the conv_offset layer that computes it in its loader
// (dcn_kernels_conv.hip) must produce the same bits. Compiled with contraction off, as
// every file that includes it.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "dcn_device.hpp"
#include "dcn_internal.hpp"

namespace dcn {
namespace warp {

__device__ __forceinline__ float h2f(uint16_t v) { return (float)__builtin_bit_cast(_Float16, v); }
__device__ __forceinline__ uint16_t f2h(float v) { return __builtin_bit_cast(uint16_t, round_f16(v)); }

// sample_fp16 (MetalShader.swift:51-74): zero-padded bilinear sample of one FP16 plane,
// the reference's association.
__device__ __forceinline__ float sample_zero(const uint16_t* plane, int H, int W, float y, float x) {
    const float fy = floorf(y), fx = floorf(x);
    const int y0 = (int)fminf(fmaxf(fy, -4.0f), (float)H + 4.0f);
    const int x0 = (int)fminf(fmaxf(fx, -4.0f), (float)W + 4.0f);
    const int y1 = y0 + 1, x1 = x0 + 1;
    const float ly = y - fy, lx = x - fx;
    // Every corner is loaded from an index clamped into the plane and zeroed afterwards
    // when it lies outside: unconditional loads, all in flight together.
    const int yc0 = min(max(y0, 0), H - 1), yc1 = min(max(y1, 0), H - 1);
    const int xc0 = min(max(x0, 0), W - 1), xc1 = min(max(x1, 0), W - 1);
    const float t00 = h2f(plane[(size_t)yc0 * W + xc0]), t01 = h2f(plane[(size_t)yc0 * W + xc1]);
    const float t10 = h2f(plane[(size_t)yc1 * W + xc0]), t11 = h2f(plane[(size_t)yc1 * W + xc1]);
    const bool r0 = y0 >= 0 && y0 < H, r1 = y1 >= 0 && y1 < H;
    const bool c0 = x0 >= 0 && x0 < W, c1 = x1 >= 0 && x1 < W;
    const float v00 = (r0 && c0) ? t00 : 0.0f, v01 = (r0 && c1) ? t01 : 0.0f;
    const float v10 = (r1 && c0) ? t10 : 0.0f, v11 = (r1 && c1) ? t11 : 0.0f;
    return v00 * (1.0f - ly) * (1.0f - lx) + v01 * (1.0f - ly) * lx + v10 * ly * (1.0f - lx) + v11 * ly * lx;
}

// Bilinear sample of eight consecutive planes at one coordinate: sample_zero's arithmetic
// per plane (same association), the corner set computed once.
__device__ __forceinline__ void sample8_zero(const uint16_t* planes, size_t plane, int H, int W,
                                             float y, float x, float (&v)[8]) {
    const float fy = floorf(y), fx = floorf(x);
    const int y0 = (int)fminf(fmaxf(fy, -4.0f), (float)H + 4.0f);
    const int x0 = (int)fminf(fmaxf(fx, -4.0f), (float)W + 4.0f);
    const int y1 = y0 + 1, x1 = x0 + 1;
    const float ly = y - fy, lx = x - fx;
    const bool r0 = y0 >= 0 && y0 < H, r1 = y1 >= 0 && y1 < H;
    const bool c0 = x0 >= 0 && x0 < W, c1 = x1 >= 0 && x1 < W;
    // Unconditional loads from clamped indices (32 in flight), out-of-plane corners
    // zeroed afterwards: the same values as loading only the valid corners.
    const size_t i00 = (size_t)min(max(y0, 0), H - 1) * W + min(max(x0, 0), W - 1);
    const size_t i01 = (size_t)min(max(y0, 0), H - 1) * W + min(max(x1, 0), W - 1);
    const size_t i10 = (size_t)min(max(y1, 0), H - 1) * W + min(max(x0, 0), W - 1);
    const size_t i11 = (size_t)min(max(y1, 0), H - 1) * W + min(max(x1, 0), W - 1);
    uint16_t t[8][4];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint16_t* p = planes + (size_t)c * plane;
        t[c][0] = p[i00];
        t[c][1] = p[i01];
        t[c][2] = p[i10];
        t[c][3] = p[i11];
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const float v00 = (r0 && c0) ? h2f(t[c][0]) : 0.0f;
        const float v01 = (r0 && c1) ? h2f(t[c][1]) : 0.0f;
        const float v10 = (r1 && c0) ? h2f(t[c][2]) : 0.0f;
        const float v11 = (r1 && c1) ? h2f(t[c][3]) : 0.0f;
        v[c] = v00 * (1.0f - ly) * (1.0f - lx) + v01 * (1.0f - ly) * lx + v10 * ly * (1.0f - lx) +
               v11 * ly * lx;
    }
}


// sample8_zero over one 8-channel block of a CB8 tensor ([Hp][Wp][8] with a kPad zero
// border): the same corners, validity and per-channel arithmetic, four 16-byte gathers.
// In two halves, so that a caller can request the corners of several samples before it
// blends any of them: cb8_corner_units gives the corners' 16-byte unit indices within the
// block (clamped into the plane: corners outside it are zeroed by the blend), cb8_blend
// the eight channels from the four loaded units.
__device__ __forceinline__ void cb8_corner_units(int H, int W, float y, float x, uint32_t (&u)[4]) {
    const int Wp = W + 2 * dev::kPad;
    const float fy = floorf(y), fx = floorf(x);
    const int y0 = (int)fminf(fmaxf(fy, -4.0f), (float)H + 4.0f);
    const int x0 = (int)fminf(fmaxf(fx, -4.0f), (float)W + 4.0f);
    const int yc0 = min(max(y0, 0), H - 1) + dev::kPad, yc1 = min(max(y0 + 1, 0), H - 1) + dev::kPad;
    const int xc0 = min(max(x0, 0), W - 1) + dev::kPad, xc1 = min(max(x0 + 1, 0), W - 1) + dev::kPad;
    u[0] = (uint32_t)(yc0 * Wp + xc0);
    u[1] = (uint32_t)(yc0 * Wp + xc1);
    u[2] = (uint32_t)(yc1 * Wp + xc0);
    u[3] = (uint32_t)(yc1 * Wp + xc1);
}

__device__ __forceinline__ void cb8_blend(const dev::u32x4 (&t)[4], int H, int W, float y, float x, float (&v)[8]) {
    const float fy = floorf(y), fx = floorf(x);
    const int y0 = (int)fminf(fmaxf(fy, -4.0f), (float)H + 4.0f);
    const int x0 = (int)fminf(fmaxf(fx, -4.0f), (float)W + 4.0f);
    const int y1 = y0 + 1, x1 = x0 + 1;
    const float ly = y - fy, lx = x - fx;
    const bool r0 = y0 >= 0 && y0 < H, r1 = y1 >= 0 && y1 < H;
    const bool c0 = x0 >= 0 && x0 < W, c1 = x1 >= 0 && x1 < W;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int sh = (c & 1) * 16;
        const float v00 = (r0 && c0) ? h2f((uint16_t)(t[0][c >> 1] >> sh)) : 0.0f;
        const float v01 = (r0 && c1) ? h2f((uint16_t)(t[1][c >> 1] >> sh)) : 0.0f;
        const float v10 = (r1 && c0) ? h2f((uint16_t)(t[2][c >> 1] >> sh)) : 0.0f;
        const float v11 = (r1 && c1) ? h2f((uint16_t)(t[3][c >> 1] >> sh)) : 0.0f;
        v[c] = v00 * (1.0f - ly) * (1.0f - lx) + v01 * (1.0f - ly) * lx + v10 * ly * (1.0f - lx) +
               v11 * ly * lx;
    }
}

__device__ __forceinline__ void sample8_cb8(const uint16_t* block, int H, int W, float y, float x,
                                            float (&v)[8]) {
    uint32_t u[4];
    cb8_corner_units(H, W, y, x, u);
    const dev::u32x4* units = reinterpret_cast<const dev::u32x4*>(block);
    const dev::u32x4 t[4] = {units[u[0]], units[u[1]], units[u[2]], units[u[3]]};
    cb8_blend(t, H, W, y, x, v);
}

// The eight channels of condition block `kind` (0-24) at pixel (y, x), as CB8 halves:
// 0-7 warp(feat_prop, flow1), 8-15 feat_current, 16-23 warp(feat_n2, flow2), 24
// [flow1 (x, y), flow2 (x, y), 0, 0, 0, 0] (assemble_temporal_alignment_fp16,
// MetalShader.swift:769-813; flow2 = flow1 + warp(prev_flow, flow1) rounded to FP16,
// accumulate_second_order_flow_fp16, :738-763, or zero without second order). Features
// NCHW [64][H][W], flows [2][H][W] (x, y). flow2_bits receives the pixel's FP16 flow2.
__device__ __forceinline__ uint32_t pack_halves(uint16_t lo, uint16_t hi) { return (uint32_t)lo | ((uint32_t)hi << 16); }

__device__ __forceinline__ void temporal_flow2(const uint16_t* flow1, const uint16_t* prev_flow, int has_second_order,
                                               int H, int W, int y, int x, uint16_t (&f2)[2]) {
    const size_t pl = (size_t)H * W;
    const int p = y * W + x;
    f2[0] = 0;
    f2[1] = 0;
    if (!has_second_order) return;
    const float fx1 = h2f(flow1[p]);
    const float fy1 = h2f(flow1[pl + p]);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const float prev = sample_zero(prev_flow + (size_t)c * pl, H, W, (float)y + fy1, (float)x + fx1);
        f2[c] = f2h(h2f(flow1[(size_t)c * pl + p]) + prev);
    }
}

// Eight FP16 planes at pixel p as one CB8 unit.
template <typename V4>
__device__ __forceinline__ V4 copy8(const uint16_t* planes, size_t pl, int p) {
    uint16_t h[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) h[c] = planes[(size_t)c * pl + p];
    V4 out;
#pragma unroll
    for (int d = 0; d < 4; ++d) out[d] = pack_halves(h[2 * d], h[2 * d + 1]);
    return out;
}

// Condition block `kind` at (y, x) from the pixel's FP16 flows f1 = flow1 (x, y) and
// f2 = flow2 (x, y) (both as bits).
// With WARP_CB8, feat_prop and feat_n2 are CB8 tensors (8 blocks) and are warped through
// sample8_cb8; feat_current is NCHW either way.
template <typename V4, bool WARP_CB8 = false>
__device__ __forceinline__ V4 condition_from_flows(const uint16_t* feat_prop, const uint16_t* feat_current,
                                                   const uint16_t* feat_n2, int H, int W, int kind, int y, int x,
                                                   const uint16_t (&f1)[2], const uint16_t (&f2)[2]) {
    const size_t pl = (size_t)H * W;
    const int p = y * W + x;
    V4 out;
    if (kind >= 8 && kind < 16) return copy8<V4>(feat_current + (size_t)(kind - 8) * 8 * pl, pl, p);
    if (kind == 24) {
        out[0] = pack_halves(f1[0], f1[1]);
        out[1] = pack_halves(f2[0], f2[1]);
        out[2] = 0u;
        out[3] = 0u;
        return out;
    }
    float v[8];
    if (WARP_CB8) {
        const size_t blk = (size_t)(H + 2 * dev::kPad) * (W + 2 * dev::kPad) * 8;  // elements per block
        if (kind < 8)
            sample8_cb8(feat_prop + (size_t)kind * blk, H, W, (float)y + h2f(f1[1]), (float)x + h2f(f1[0]), v);
        else
            sample8_cb8(feat_n2 + (size_t)(kind - 16) * blk, H, W, (float)y + h2f(f2[1]), (float)x + h2f(f2[0]), v);
    } else if (kind < 8) {
        sample8_zero(feat_prop + (size_t)kind * 8 * pl, pl, H, W, (float)y + h2f(f1[1]), (float)x + h2f(f1[0]), v);
    } else {
        sample8_zero(feat_n2 + (size_t)(kind - 16) * 8 * pl, pl, H, W, (float)y + h2f(f2[1]), (float)x + h2f(f2[0]), v);
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) out[d] = pack_halves(f2h(v[2 * d]), f2h(v[2 * d + 1]));
    return out;
}

// The same from the flow planes; f2 receives the pixel's flow2 bits (zero for kinds < 16,
// which do not need it).
template <typename V4>
__device__ __forceinline__ V4 condition_block(const uint16_t* feat_prop, const uint16_t* feat_current,
                                              const uint16_t* feat_n2, const uint16_t* flow1,
                                              const uint16_t* prev_flow, int has_second_order, int H, int W,
                                              int kind, int y, int x, uint16_t (&f2)[2]) {
    const size_t pl = (size_t)H * W;
    const int p = y * W + x;
    const uint16_t f1[2] = {flow1[p], flow1[pl + p]};
    f2[0] = 0;
    f2[1] = 0;
    if (kind >= 16) temporal_flow2(flow1, prev_flow, has_second_order, H, W, y, x, f2);
    return condition_from_flows<V4>(feat_prop, feat_current, feat_n2, H, W, kind, y, x, f1, f2);
}

}  // namespace warp
}  // namespace dcn
