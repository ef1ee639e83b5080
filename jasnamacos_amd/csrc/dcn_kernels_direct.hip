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

// ---- FP32 with shared samples ----------------------------------------------------------
// direct_kernel evaluates every bilinear sample once per output channel. Here a workgroup
// owns 16 output pixels x 64 output channels: each (pixel, ic, tap) sample is evaluated
// once, as sampled * mask, into LDS, and every output channel of the workgroup reads it
// there. Each output still sums bias, then ic, ky, kx in order, as
// sum + ((sampled * mask) * weight) with one rounding per operation (no contraction), so
// the result is direct_kernel's, and the oracle's, bit for bit. groups == 1 only.
//
// Lanes: pixel p = tid % 16, output-channel group q = tid / 16 of OCL channels (OCL
// independent chains per lane; 64 / OCL * 16 threads). The input channels go by in stages of 8
// (J = 8 * KA samples per pixel): stage c + 1's offsets, masks and weights are loaded
// before stage c's chains, its corner gathers issued halfway through them and its
// samples finished after them, so the loads' latency hides behind the chains.
constexpr int kSharedPix = 16;
constexpr int kSharedOc = 64;
constexpr int kSharedCh = 8;

template <int KA, int OCL>
struct SharedLayout {
    static constexpr int NT = kSharedPix * kSharedOc / OCL;      // threads
    static constexpr int J = kSharedCh * KA;  // samples per pixel and stage
    static constexpr int JP = J + 4;          // padded row (floats), rows stay 16-byte aligned
    static constexpr int PER = (kSharedPix * J + NT - 1) / NT;       // samples per thread
    static constexpr int WPER = (kSharedOc * J / 4 + NT - 1) / NT;   // weight float4s per thread
};

template <int KA, int OCL>
__global__ __launch_bounds__((SharedLayout<KA, OCL>::NT)) void direct_shared_f32_kernel(
    const float* __restrict__ input, const float* __restrict__ offset, const float* __restrict__ mask,
    const float* __restrict__ weight, const float* __restrict__ bias, float* __restrict__ output, KShape s,
    long pixels) {
    using L = SharedLayout<KA, OCL>;
    constexpr int J = L::J, JP = L::JP, NT = L::NT;
    __shared__ __attribute__((aligned(16))) float sm[2][kSharedPix][JP];  // sampled * mask
    __shared__ __attribute__((aligned(16))) float wn[2][kSharedOc][JP];   // weights [oc][j]
    const int tid = threadIdx.x;
    const int oc_base = blockIdx.y * kSharedOc;
    const long pix0 = (long)blockIdx.x * kSharedPix;

    // The pixel this thread samples (every sample of a thread has pixel tid % 16).
    const int sp = tid & 15;
    const long spix = min(pix0 + sp, pixels - 1);
    const long plane = (long)s.Ho * s.Wo;
    const long sn = spix / plane;
    const long sspatial = spix - sn * plane;
    const int soy = (int)(sspatial / s.Wo);
    const int sox = (int)(sspatial - (long)soy * s.Wo);
    const long off_base = sn * 2 * s.og * KA * plane + sspatial;
    const long mask_base = sn * s.og * KA * plane + sspatial;
    const long in_plane = (long)s.H * s.W;
    const int cpog = s.Cin / s.og;
    const int KW = s.KW;
    const long wrow = (long)s.Cin * KA;  // weights per output channel (groups == 1)

    float ofy[L::PER], ofx[L::PER], mk[L::PER];
    float4 wreg[L::WPER];
    long ibase[L::PER];
    float v[L::PER][4], ly[L::PER], lx[L::PER];

    auto sample_jj = [&](int i) { return (tid >> 4) + NT / 16 * i; };
    // Stage st's offsets, masks and weights into registers.
    auto load_stage = [&](int st) {
        const int ic0 = st * kSharedCh;
#pragma unroll
        for (int i = 0; i < L::PER; ++i) {
            const int jj = sample_jj(i);
            if (jj >= J) continue;
            const int ic = ic0 + jj / KA;
            const int k = jj % KA;
            const int og = ic / cpog;
            const long oc_ch = 2L * (og * KA + k);
            ofy[i] = offset[off_base + oc_ch * plane];
            ofx[i] = offset[off_base + (oc_ch + 1) * plane];
            mk[i] = mask[mask_base + (long)(og * KA + k) * plane];
            ibase[i] = (sn * s.Cin + ic) * in_plane;
        }
#pragma unroll
        for (int i = 0; i < L::WPER; ++i) {
            const int t = tid + NT * i;
            const int oc_l = t / (J / 4);
            const int j4 = t - oc_l * (J / 4);
            wreg[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (oc_l < kSharedOc && oc_base + oc_l < s.Cout)
                wreg[i] = *reinterpret_cast<const float4*>(weight + (long)(oc_base + oc_l) * wrow +
                                                           (long)ic0 * KA + 4 * j4);
        }
    };
    // Coordinates and the four corner loads (a corner outside the input reads 0).
    auto gather_stage = [&]() {
#pragma unroll
        for (int i = 0; i < L::PER; ++i) {
            const int jj = sample_jj(i);
            if (jj >= J) continue;
            const int k = jj % KA;
            const int ky = k / KW;
            const int kx = k - ky * KW;
            const float y = (float)(soy * s.sh - s.ph + ky * s.dh) + ofy[i];
            const float x = (float)(sox * s.sw - s.pw + kx * s.dw) + ofx[i];
            const float fy = floorf(y), fx = floorf(x);
            ly[i] = y - fy;
            lx[i] = x - fx;
            // floor() of a finite float converts exactly once clamped (clamped values are
            // out of bounds either way; NaN clamps to the lower bound).
            const int y0 = (int)fminf(fmaxf(fy, -4.0f), (float)s.H + 4.0f);
            const int x0 = (int)fminf(fmaxf(fx, -4.0f), (float)s.W + 4.0f);
            const bool ry0 = y0 >= 0 && y0 < s.H, ry1 = y0 + 1 >= 0 && y0 + 1 < s.H;
            const bool rx0 = x0 >= 0 && x0 < s.W, rx1 = x0 + 1 >= 0 && x0 + 1 < s.W;
            const long b = ibase[i] + (long)y0 * s.W + x0;
            v[i][0] = (ry0 && rx0) ? input[b] : 0.0f;
            v[i][1] = (ry0 && rx1) ? input[b + 1] : 0.0f;
            v[i][2] = (ry1 && rx0) ? input[b + s.W] : 0.0f;
            v[i][3] = (ry1 && rx1) ? input[b + s.W + 1] : 0.0f;
        }
    };
    // The samples (DeformConvCPU.bilinear's association) times the mask, and the
    // weights, into LDS buffer nb.
    auto store_stage = [&](int nb) {
#pragma unroll
        for (int i = 0; i < L::PER; ++i) {
            const int jj = sample_jj(i);
            if (jj >= J) continue;
            const float a = 1.0f - ly[i], c = 1.0f - lx[i];
            const float sampled = v[i][0] * a * c + v[i][1] * a * lx[i] + v[i][2] * ly[i] * c +
                                  v[i][3] * ly[i] * lx[i];
            sm[nb][sp][jj] = sampled * mk[i];
        }
#pragma unroll
        for (int i = 0; i < L::WPER; ++i) {
            const int t = tid + NT * i;
            const int oc_l = t / (J / 4);
            const int j4 = t - oc_l * (J / 4);
            if (oc_l < kSharedOc) *reinterpret_cast<float4*>(&wn[nb][oc_l][4 * j4]) = wreg[i];
        }
    };

    const int p = tid & 15;
    const int q = tid >> 4;
    float acc[OCL];
#pragma unroll
    for (int e = 0; e < OCL; ++e) acc[e] = oc_base + OCL * q + e < s.Cout ? bias[oc_base + OCL * q + e] : 0.0f;
    // sum + (sm * w) for samples [4 * lo, 4 * hi) of buffer nb, in order.
    auto chain = [&](int nb, int lo, int hi) {
#pragma unroll 3
        for (int j4 = lo; j4 < hi; ++j4) {
            const float4 sv = *reinterpret_cast<const float4*>(&sm[nb][p][4 * j4]);
            float4 w4[OCL];
#pragma unroll
            for (int e = 0; e < OCL; ++e) w4[e] = *reinterpret_cast<const float4*>(&wn[nb][OCL * q + e][4 * j4]);
#pragma unroll
            for (int e = 0; e < OCL; ++e) acc[e] = acc[e] + sv.x * w4[e].x;
#pragma unroll
            for (int e = 0; e < OCL; ++e) acc[e] = acc[e] + sv.y * w4[e].y;
#pragma unroll
            for (int e = 0; e < OCL; ++e) acc[e] = acc[e] + sv.z * w4[e].z;
#pragma unroll
            for (int e = 0; e < OCL; ++e) acc[e] = acc[e] + sv.w * w4[e].w;
        }
    };

    const int stages = s.Cin / kSharedCh;
    load_stage(0);
    gather_stage();
    store_stage(0);
    __syncthreads();
    for (int st = 0; st < stages; ++st) {
        const int nb = st & 1;
        const bool more = st + 1 < stages;
        if (more) load_stage(st + 1);
        chain(nb, 0, J / 8);
        if (more) gather_stage();
        chain(nb, J / 8, J / 4);
        if (more) store_stage(nb ^ 1);
        __syncthreads();
    }

    const long pix = pix0 + p;
    if (pix >= pixels) return;
    const long n = pix / plane;
    const long spatial = pix - n * plane;
#pragma unroll
    for (int e = 0; e < OCL; ++e) {
        const int oc = oc_base + OCL * q + e;
        if (oc < s.Cout) output[(n * s.Cout + oc) * plane + spatial] = acc[e];
    }
}

template <int KA>
hipError_t launch_shared_f32(const KShape& s, const float* in, const float* off, const float* mask,
                             const float* w, const float* b, float* out, hipStream_t stream) {
    // One channel per lane (1024 threads, 4 waves per SIMD) measured 38.8 us at C1
    // against 48.4 us with two and 63.3 us with four: the chains are latency-bound and
    // the extra waves hide the LDS and gather latency better than the extra ILP does.
    constexpr int OCL = 1;
    const long pixels = (long)s.B * s.Ho * s.Wo;
    const dim3 grid((unsigned)((pixels + kSharedPix - 1) / kSharedPix),
                    (unsigned)((s.Cout + kSharedOc - 1) / kSharedOc));
    hipLaunchKernelGGL((direct_shared_f32_kernel<KA, OCL>), grid, dim3(SharedLayout<KA, OCL>::NT), 0, stream, in,
                       off, mask, w, b, out, s, pixels);
    return hipGetLastError();
}

}  // namespace

// The shared-sample kernel reads weights as float4 rows (16-byte aligned when the weight
// pointer is and Cin % 8 == 0).
static bool shared_f32_supported(const KShape& s, const float* w) {
    const int ka = s.KH * s.KW;
    return s.groups == 1 && s.Cin % kSharedCh == 0 && (uintptr_t)w % 16 == 0 &&
           (ka == 1 || ka == 2 || ka == 3 || ka == 4 || ka == 6 || ka == 9) &&
           (long)s.B * s.Ho * s.Wo > 0 && (long)s.B * s.Ho * s.Wo / kSharedPix < (1L << 31);
}

hipError_t launch_direct_f32(const KShape& s, const float* in, const float* off,
                             const float* mask, const float* w, const float* b, float* out,
                             hipStream_t stream) {
    if (shared_f32_supported(s, w)) {
        switch (s.KH * s.KW) {
            case 1: return launch_shared_f32<1>(s, in, off, mask, w, b, out, stream);
            case 2: return launch_shared_f32<2>(s, in, off, mask, w, b, out, stream);
            case 3: return launch_shared_f32<3>(s, in, off, mask, w, b, out, stream);
            case 4: return launch_shared_f32<4>(s, in, off, mask, w, b, out, stream);
            case 6: return launch_shared_f32<6>(s, in, off, mask, w, b, out, stream);
            default: return launch_shared_f32<9>(s, in, off, mask, w, b, out, stream);
        }
    }
    return launch_direct<float>(s, in, off, mask, w, b, out, stream);
}

hipError_t launch_direct_f16(const KShape& s, const uint16_t* in, const uint16_t* off,
                             const uint16_t* mask, const uint16_t* w, const uint16_t* b,
                             uint16_t* out, hipStream_t stream) {
    return launch_direct<uint16_t>(s, in, off, mask, w, b, out, stream);
}

}  // namespace dcn
