// Direct DCNv2 kernels: one thread per output element, summation in the CPU oracle's
// order (DeformConv.swift:98-135), no contraction. They are the FP32 entry point
// (deform_conv2d_fp32, MetalShader.swift:76-124) and the FP16 reference semantics
// (deform_conv2d_fp16, MetalShader.swift:126-174), for any valid shape.
//
// Bit-exactness rests on three facts: the file is compiled with -ffp-contract=off
// (and the pragma below), every FP16 operand widens exactly to FP32, and the
// bilinear expression keeps the reference's association
// ((v00*(1-ly))*(1-lx)) + ((v01*(1-ly))*lx) + ((v10*ly)*(1-lx)) + ((v11*ly)*lx).
#include <hip/hip_runtime.h>

#include "dcn_internal.hpp"

#pragma clang fp contract(off)

namespace dcn {
namespace {

template <typename T>
__device__ __forceinline__ float widen(T v);
template <>
__device__ __forceinline__ float widen<float>(float v) {
    return v;
}
template <>
__device__ __forceinline__ float widen<uint16_t>(uint16_t v) {
    return (float)__builtin_bit_cast(_Float16, v);
}

// DeformConvCPU.bilinear (DeformConv.swift:146-165); a corner outside the input is 0.
template <typename T>
__device__ __forceinline__ float bilinear(const T* __restrict__ input, long base, int height,
                                          int width, float y, float x) {
    // floor() of a finite float below 2^31 converts exactly; larger magnitudes are
    // clamped first so the conversion is defined (they are out of bounds either way).
    const float fy = fminf(fmaxf(floorf(y), -4.0f), (float)height + 4.0f);
    const float fx = fminf(fmaxf(floorf(x), -4.0f), (float)width + 4.0f);
    const int y0 = (int)fy;
    const int x0 = (int)fx;
    const int y1 = y0 + 1;
    const int x1 = x0 + 1;
    const float ly = y - floorf(y);
    const float lx = x - floorf(x);
    const bool ry0 = y0 >= 0 && y0 < height, ry1 = y1 >= 0 && y1 < height;
    const bool rx0 = x0 >= 0 && x0 < width, rx1 = x1 >= 0 && x1 < width;
    const float v00 = (ry0 && rx0) ? widen(input[base + (long)y0 * width + x0]) : 0.0f;
    const float v01 = (ry0 && rx1) ? widen(input[base + (long)y0 * width + x1]) : 0.0f;
    const float v10 = (ry1 && rx0) ? widen(input[base + (long)y1 * width + x0]) : 0.0f;
    const float v11 = (ry1 && rx1) ? widen(input[base + (long)y1 * width + x1]) : 0.0f;
    return v00 * (1.0f - ly) * (1.0f - lx) + v01 * (1.0f - ly) * lx +
           v10 * ly * (1.0f - lx) + v11 * ly * lx;
}

template <typename T>
__device__ __forceinline__ void store_out(T* out, long i, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* out, long i, float v) {
    out[i] = v;
}
template <>
__device__ __forceinline__ void store_out<uint16_t>(uint16_t* out, long i, float v) {
    out[i] = __builtin_bit_cast(uint16_t, round_f16(v));  // half(sum), round to nearest even
}

template <typename T>
__global__ __launch_bounds__(256) void direct_kernel(const T* __restrict__ input,
                                                     const T* __restrict__ offset,
                                                     const T* __restrict__ mask,
                                                     const T* __restrict__ weight,
                                                     const T* __restrict__ bias,
                                                     T* __restrict__ output, KShape s,
                                                     long total) {
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    const long ox = gid % s.Wo;
    long q = gid / s.Wo;
    const long oy = q % s.Ho;
    q /= s.Ho;
    const long oc = q % s.Cout;
    const long n = q / s.Cout;
    const long cpg = s.Cin / s.groups;
    const long opg = s.Cout / s.groups;
    const long cpog = s.Cin / s.og;
    const long group = oc / opg;
    const long input_plane = (long)s.H * s.W;
    const long output_plane = (long)s.Ho * s.Wo;
    const long kernel_area = (long)s.KH * s.KW;
    const long spatial = oy * s.Wo + ox;
    const long offset_base = n * 2 * s.og * kernel_area * output_plane;
    const long mask_base = n * s.og * kernel_area * output_plane;
    float sum = widen(bias[oc]);
    for (long local_ic = 0; local_ic < cpg; ++local_ic) {
        const long ic = group * cpg + local_ic;
        const long og = ic / cpog;
        const long input_base = (n * s.Cin + ic) * input_plane;
        for (long ky = 0; ky < s.KH; ++ky) {
            for (long kx = 0; kx < s.KW; ++kx) {
                const long k = ky * s.KW + kx;
                const long offset_channel = 2 * (og * kernel_area + k);
                const float off_y = widen(offset[offset_base + offset_channel * output_plane + spatial]);
                const float off_x =
                    widen(offset[offset_base + (offset_channel + 1) * output_plane + spatial]);
                const float y = (float)(oy * s.sh - s.ph + ky * s.dh) + off_y;
                const float x = (float)(ox * s.sw - s.pw + kx * s.dw) + off_x;
                const float sampled = bilinear(input, input_base, s.H, s.W, y, x);
                const float m = widen(mask[mask_base + (og * kernel_area + k) * output_plane + spatial]);
                const float w = widen(weight[((oc * cpg + local_ic) * s.KH + ky) * s.KW + kx]);
                sum += sampled * m * w;
            }
        }
    }
    store_out(output, gid, sum);
}

template <typename T>
hipError_t launch_direct(const KShape& s, const T* in, const T* off, const T* mask, const T* w,
                         const T* b, T* out, hipStream_t stream) {
    const long total = (long)s.B * s.Cout * s.Ho * s.Wo;
    const int block = 256;
    const long grid = (total + block - 1) / block;
    if (grid <= 0) return hipSuccess;
    hipLaunchKernelGGL(direct_kernel<T>, dim3((unsigned)grid), dim3(block), 0, stream, in, off,
                       mask, w, b, out, s, total);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_direct_f32(const KShape& s, const float* in, const float* off,
                             const float* mask, const float* w, const float* b, float* out,
                             hipStream_t stream) {
    return launch_direct<float>(s, in, off, mask, w, b, out, stream);
}

hipError_t launch_direct_f16(const KShape& s, const uint16_t* in, const uint16_t* off,
                             const uint16_t* mask, const uint16_t* w, const uint16_t* b,
                             uint16_t* out, hipStream_t stream) {
    return launch_direct<uint16_t>(s, in, off, mask, w, b, out, stream);
}

}  // namespace dcn
