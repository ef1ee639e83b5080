// SPyNet flow estimation for the propagation body's flows (gfx950): the quarter-scale
// bicubic input, the normalised image pyramid, the per-level block input (flow upsample +
// border warp + concatenation) and the basic module's 7 x 7 convolutions.
//
// The elementwise kernels evaluate the reference's FP32 expressions in the same order
// (jasna_bicubic_downsample_quarter_fp16, spynet_build_pyramid_pair_fp16,
// spynet_prepare_fp16: MetalShader.swift:473-639), so they are bit-identical to the CPU
// oracle. The convolutions are implicit GEMMs on v_mfma_f32_16x16x32_f16 like
// conv3x3_kernel, generalised to k x k taps, a batch of images and a configurable zero
// border of the CB8 activations (SPyNet's are padded by 3 for the 7 x 7 taps).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "dcn_device.hpp"
#include "dcn_internal.hpp"

#pragma clang fp contract(off)

namespace dcn {
namespace {

using namespace dev;

__device__ __forceinline__ float h2f(uint16_t v) { return (float)__builtin_bit_cast(_Float16, v); }
__device__ __forceinline__ uint16_t f2h(float v) { return __builtin_bit_cast(uint16_t, round_f16(v)); }

unsigned blocks_for(long n) { return (unsigned)((n + 255) / 256); }

// cubic_weight (MetalShader.swift:473-483), a = -0.75.
__device__ __forceinline__ float cubic_weight(float distance) {
    const float a = -0.75f;
    const float x = fabsf(distance);
    if (x <= 1.0f) return (a + 2.0f) * x * x * x - (a + 3.0f) * x * x + 1.0f;
    if (x < 2.0f) return a * x * x * x - 5.0f * a * x * x + 8.0f * a * x - 4.0f * a;
    return 0.0f;
}

// jasna_bicubic_downsample_quarter_fp16 (MetalShader.swift:488-521), any C x H x W with
// H, W multiples of 4 (every 4 x 4 footprint is then inside the image).
__global__ __launch_bounds__(256) void bicubic_quarter_kernel(const uint16_t* __restrict__ in,
                                                              uint16_t* __restrict__ out, int C, int H,
                                                              int W) {
    const int oh = H >> 2, ow = W >> 2;
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (long)C * oh * ow) return;
    const int c = (int)(gid / ((long)oh * ow));
    const int sp = (int)(gid - (long)c * oh * ow);
    const int oy = sp / ow;
    const int ox = sp - oy * ow;
    const float sy = ((float)oy + 0.5f) * 4.0f - 0.5f;
    const float sx = ((float)ox + 0.5f) * 4.0f - 0.5f;
    const int by = (int)floorf(sy);
    const int bx = (int)floorf(sx);
    float value = 0.0f;
#pragma unroll
    for (int yy = -1; yy <= 2; ++yy) {
        const float wy = cubic_weight(sy - (float)(by + yy));
        const uint16_t* row = in + ((size_t)c * H + (by + yy)) * W;
#pragma unroll
        for (int xx = -1; xx <= 2; ++xx) {
            const float wx = cubic_weight(sx - (float)(bx + xx));
            value += h2f(row[bx + xx]) * wy * wx;
        }
    }
    out[gid] = f2h(value);
}

// spynet_build_pyramid_pair_fp16 (MetalShader.swift:523-570): level l (coarsest first) of
// frame f is the direct box average over factor x factor pixels, normalised with the
// ImageNet mean/std (:560-563). One thread per output value of every level and frame.
struct PyramidArgs {
    const uint16_t* frame[2];  // frames 0 and 1; frame f >= 2 at frame[0] + f * frame_stride
    long frame_stride;
    uint16_t* level[kSpynetMaxLevels];  // level l of frame f at level[l] + f * 3 * h_l * w_l
    long offset[kSpynetMaxLevels + 1];  // first output index of each level (per frame)
    long coarse;  // outputs per frame (the first ones) summed by a whole wave
    int frames, levels, H, W;
    int aligned;  // frames 16-byte aligned and W a multiple of 8: rows of 8 pixels load as 16 bytes
};

constexpr int kPyramidWaveFactor = 16;  // levels with factor >= 16 (and <= 64): one wave per output
constexpr int kPyramidMaxFactor = 64;

// One output of the pyramid: level, channel and position of output r of a frame.
struct PyramidOut {
    int l, c, y, x, factor;
    long e;
};
__device__ __forceinline__ PyramidOut pyramid_out(const PyramidArgs& a, long r) {
    PyramidOut o;
    o.l = 0;
    while (r >= a.offset[o.l + 1]) ++o.l;
    const int shift = a.levels - 1 - o.l;
    const int lh = a.H >> shift, lw = a.W >> shift;
    o.e = r - a.offset[o.l];
    o.c = (int)(o.e / ((long)lh * lw));
    const int sp = (int)(o.e - (long)o.c * lh * lw);
    o.y = sp / lw;
    o.x = sp - o.y * lw;
    o.factor = 1 << shift;
    return o;
}

__device__ __forceinline__ const uint16_t* pyramid_frame(const PyramidArgs& a, int f) {
    return f < 2 ? a.frame[f] : a.frame[0] + (size_t)f * a.frame_stride;
}
__device__ __forceinline__ uint16_t* pyramid_dst(const PyramidArgs& a, int f, const PyramidOut& o) {
    return a.level[o.l] + (size_t)f * (a.offset[o.l + 1] - a.offset[o.l]) + o.e;
}

__device__ __forceinline__ uint16_t pyramid_value(float sum, int c, int factor) {
    const float mean = c == 0 ? 0.485f : (c == 1 ? 0.456f : 0.406f);
    const float stddev = c == 0 ? 0.229f : (c == 1 ? 0.224f : 0.225f);
    const float inverse_area = 1.0f / (float)(factor * factor);
    return f2h((sum * inverse_area - mean) / stddev);
}

// 64-thread blocks. The first coarse * frames blocks each sum one coarse output: the wave
// copies the factor x factor box into LDS with 16-byte loads, then one lane adds it in
// the reference's row-major order (a coarse level sums up to 4,096 values per output).
// The remaining blocks give one thread per output.
__global__ __launch_bounds__(64) void spynet_pyramid_kernel(PyramidArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t box[kPyramidMaxFactor * kPyramidMaxFactor];
    const long per_frame = a.offset[a.levels];
    const int lane = threadIdx.x;
    if ((long)blockIdx.x < a.coarse * a.frames) {
        const int f = (int)(blockIdx.x / a.coarse);
        const PyramidOut o = pyramid_out(a, (long)blockIdx.x - (long)f * a.coarse);
        const int F = o.factor;
        const uint16_t* src = pyramid_frame(a, f) + ((size_t)o.c * a.H + (size_t)o.y * F) * a.W + (size_t)o.x * F;
        const int row_chunks = F / 8;
        for (int ch = lane; ch < F * row_chunks; ch += 64) {
            const int yy = ch / row_chunks;
            const int xb = (ch - yy * row_chunks) * 8;
            *reinterpret_cast<u32x4*>(box + yy * F + xb) =
                *reinterpret_cast<const u32x4*>(src + (size_t)yy * a.W + xb);
        }
        __syncthreads();
        if (lane == 0) {
            float sum = 0.0f;
            for (int i = 0; i < F * F; i += 8) {
                const h8 v = __builtin_bit_cast(h8, *reinterpret_cast<const u32x4*>(box + i));
#pragma unroll
                for (int j = 0; j < 8; ++j) sum += (float)v[j];
            }
            *pyramid_dst(a, f, o) = pyramid_value(sum, o.c, F);
        }
        return;
    }
    const long fine = per_frame - a.coarse;
    const long gid = ((long)blockIdx.x - a.coarse * a.frames) * 64 + lane;
    if (gid >= fine * a.frames) return;
    const int f = (int)(gid / fine);
    const PyramidOut o = pyramid_out(a, a.coarse + (gid - (long)f * fine));
    const int factor = o.factor;
    float sum = 0.0f;
    const uint16_t* src = pyramid_frame(a, f) + ((size_t)o.c * a.H + (size_t)o.y * factor) * a.W + (size_t)o.x * factor;
    if (a.aligned && factor >= 8) {
        // Same row-major order of FP32 adds; the row segments come in 16-byte loads.
#pragma unroll 4
        for (int yy = 0; yy < factor; ++yy) {
            const uint16_t* row = src + (size_t)yy * a.W;
            for (int xb = 0; xb < factor; xb += 8) {
                const h8 v = __builtin_bit_cast(h8, *reinterpret_cast<const u32x4*>(row + xb));
#pragma unroll
                for (int j = 0; j < 8; ++j) sum += (float)v[j];
            }
        }
    } else {
        for (int yy = 0; yy < factor; ++yy)
            for (int xx = 0; xx < factor; ++xx) sum += h2f(src[(size_t)yy * a.W + xx]);
    }
    *pyramid_dst(a, f, o) = pyramid_value(sum, o.c, factor);
}

// sample_border_fp16 (MetalShader.swift:572-599).
__device__ __forceinline__ float sample_border(const uint16_t* plane, int H, int W, float y, float x) {
    y = fminf(fmaxf(y, 0.0f), (float)(H - 1));
    x = fminf(fmaxf(x, 0.0f), (float)(W - 1));
    const int y0 = (int)floorf(y);
    const int x0 = (int)floorf(x);
    const int y1 = min(y0 + 1, H - 1);
    const int x1 = min(x0 + 1, W - 1);
    const float ly = y - (float)y0;
    const float lx = x - (float)x0;
    const float v00 = h2f(plane[(size_t)y0 * W + x0]);
    const float v01 = h2f(plane[(size_t)y0 * W + x1]);
    const float v10 = h2f(plane[(size_t)y1 * W + x0]);
    const float v11 = h2f(plane[(size_t)y1 * W + x1]);
    return v00 * (1.0f - ly) * (1.0f - lx) + v01 * (1.0f - ly) * lx + v10 * ly * (1.0f - lx) +
           v11 * ly * lx;
}

// spynet_prepare_fp16 (MetalShader.swift:601-639) for a batch of (reference, support)
// pairs: base flow [b][2][H][W] = half(2 * align-corners upsample of the previous level's
// flow) (zero on the first level) and the 8-channel block input written as one 16-byte
// CB8 unit per pixel ([b][1][H + 2 pad][W + 2 pad][8]).
// Image b of a batch over P frame pairs: b < P estimates spynet(frame b, frame b + 1), b >= P
// the reverse direction spynet(frame b - P + 1, frame b - P) (the backward and forward
// flows of compute_flow; P = 1 is one pair in both directions).
__device__ __forceinline__ void pair_frames(int b, int pairs, int& ref, int& sup) {
    ref = b < pairs ? b : b - pairs + 1;
    sup = b < pairs ? b + 1 : b - pairs;
}

struct PrepareArgs {
    const uint16_t* level;  // pyramid level [frame][3][H][W]
    int pairs;
    const uint16_t* source_flow;  // [b][2][SH][SW], unused on the first level
    uint16_t* features;           // CB8, one block per image
    uint16_t* base_flow;          // [b][2][H][W]
    int batch, H, W, SH, SW, first_level, pad;
};

__global__ __launch_bounds__(256) void spynet_prepare_kernel(PrepareArgs a) {
    const int plane = a.H * a.W;
    const int gid = blockIdx.x * 256 + threadIdx.x;
    if (gid >= a.batch * plane) return;
    const int b = gid / plane;
    const int sp = gid - b * plane;
    const int y = sp / a.W;
    const int x = sp - y * a.W;
    float flow_x = 0.0f, flow_y = 0.0f;
    if (!a.first_level) {
        const float sx = a.W > 1 ? (float)x * (float)(a.SW - 1) / (float)(a.W - 1) : 0.0f;
        const float sy = a.H > 1 ? (float)y * (float)(a.SH - 1) / (float)(a.H - 1) : 0.0f;
        const uint16_t* src = a.source_flow + (size_t)b * 2 * a.SH * a.SW;
        flow_x = 2.0f * sample_border(src, a.SH, a.SW, sy, sx);
        flow_y = 2.0f * sample_border(src + (size_t)a.SH * a.SW, a.SH, a.SW, sy, sx);
    }
    uint16_t* base = a.base_flow + (size_t)b * 2 * plane;
    base[sp] = f2h(flow_x);
    base[plane + sp] = f2h(flow_y);
    int rf, sf;
    pair_frames(b, a.pairs, rf, sf);
    const uint16_t* ref = a.level + (size_t)rf * 3 * plane;
    const uint16_t* sup = a.level + (size_t)sf * 3 * plane;
    uint16_t v[8];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        v[c] = ref[(size_t)c * plane + sp];
        v[c + 3] = f2h(sample_border(sup + (size_t)c * plane, a.H, a.W, (float)y + flow_y, (float)x + flow_x));
    }
    v[6] = f2h(flow_x);
    v[7] = f2h(flow_y);
    const int Hp = a.H + 2 * a.pad, Wp = a.W + 2 * a.pad;
    u32x4 unit;
#pragma unroll
    for (int i = 0; i < 4; ++i) unit[i] = (uint32_t)v[2 * i] | ((uint32_t)v[2 * i + 1] << 16);
    *reinterpret_cast<u32x4*>(a.features + (((size_t)b * Hp + y + a.pad) * Wp + x + a.pad) * 8) = unit;
}

// k x k convolution, stride 1, pad k/2, on CB8 activations with a zero border of `pad`
// >= k/2 pixels ([B][CB][H + 2 pad][W + 2 pad][8]). conv3x3_kernel's scheme: 16-pixel
// tiles (pixels of the whole batch in order), NB 16-column blocks of output channels per
// workgroup, K-block kb = tap * CB + cb split over NW waves, cross-wave sum in LDS.
// Epilogue: + bias, ReLU (act 2), optionally out = half(base + half(acc)) (the level's
// residual flow added to its base flow, spynet_add_flow_fp16 MetalShader.swift:641-649),
// NCHW or CB8 output.
struct ConvKArgs {
    const void* xin;
    const void* wpk;      // [ksteps][NBT][64][8]
    const float* bias;
    const uint16_t* base; // optional [B][Cout][H][W]
    uint16_t* out;
    uint32_t xin_bytes, wpk_bytes;
    int B, H, W, Hp, Wp, pad, CB, KB, ksteps, NBT, Cout, tiles, act, out_cb8;
    uint32_t magic_cb;
};

template <int KS, int NW, int U, int NB>
__global__ __launch_bounds__(64 * NW) void convk_kernel(ConvKArgs a) {
    extern __shared__ float red[];  // [NW][NB][4][65]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int quarter = lane >> 4;

    const int per_xcd = (a.tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= a.tiles) return;  // whole workgroup, before any barrier
    const int chunk = blockIdx.y;

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xin, a.xin_bytes);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wpk, a.wpk_bytes);

    const int plane = a.H * a.W;
    const int M = a.B * plane;
    const int p = tile * 16 + (lane & 15);
    const int pc = p < M ? p : M - 1;
    const int b = pc / plane;
    const int sp = pc - b * plane;
    const int y = sp / a.W;
    const int x = sp - y * a.W;
    // 16-byte unit of (image b, cb 0, tap (0, 0)) in the padded planes.
    const uint32_t base = ((uint32_t)(b * a.CB * a.Hp) + y + a.pad - KS / 2) * a.Wp + x + a.pad - KS / 2;

    f32x4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{};

    const int s0 = wave * a.ksteps / NW;
    const int s1 = (wave + 1) * a.ksteps / NW;
    for (int sb = s0; sb < s1; sb += U) {
        h8 Bf[U][NB];
        u32x4 q[U];
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int s = sb + i < s1 ? sb + i : s1 - 1;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                Bf[i][nb] = __builtin_bit_cast(
                    h8, load16(wr, (uint32_t)((s * a.NBT + chunk * NB + nb) * 64 + lane) * 16u));
            const int kb = 4 * s + quarter;
            const int kbc = kb < a.KB ? kb : a.KB - 1;
            const int tap = fast_div(kbc, a.magic_cb);
            const int cb = kbc - tap * a.CB;
            const int ky = tap / KS;
            const int kx = tap - ky * KS;
            q[i] = load16(xr, (base + (uint32_t)(cb * a.Hp + ky) * a.Wp + kx) * 16u);
        }
#pragma unroll
        for (int i = 0; i < U; ++i) {
            if (sb + i < s1) {  // uniform across the wave
                const int kb = 4 * (sb + i) + quarter;
                const u32x4 z = {0u, 0u, 0u, 0u};
                const h8 A = __builtin_bit_cast(h8, kb < a.KB ? q[i] : z);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bf[i][nb], acc[nb], 0, 0, 0);
            }
        }
    }

#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[((wave * NB + nb) * 4 + v) * 65 + lane] = acc[nb][v];
    __syncthreads();

    for (int idx = tid; idx < 16 * NB * 16; idx += 64 * NW) {
        const int pl = idx & 15;
        const int ocl = idx >> 4;
        const int nb = ocl >> 4;
        const int src = ((pl >> 2) << 4) + (ocl & 15);
        const int v = pl & 3;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) sum += red[((w * NB + nb) * 4 + v) * 65 + src];
        const int oc = chunk * NB * 16 + ocl;
        const int pp = tile * 16 + pl;
        if (pp >= M || oc >= a.Cout) continue;
        const int bb = pp / plane;
        const int ss = pp - bb * plane;
        float r = sum + a.bias[oc];
        if (a.act == 2 && r < 0.0f) r = 0.0f;
        if (a.base != nullptr) r = h2f(a.base[((size_t)bb * a.Cout + oc) * plane + ss]) + (float)round_f16(r);
        size_t dst;
        if (a.out_cb8) {
            const int yy = ss / a.W;
            const int xx = ss - yy * a.W;
            dst = ((((size_t)bb * ((a.Cout + 7) >> 3) + (oc >> 3)) * a.Hp + yy + a.pad) * a.Wp + xx + a.pad) * 8 +
                  (oc & 7);
        } else {
            dst = ((size_t)bb * a.Cout + oc) * plane + ss;
        }
        a.out[dst] = f2h(r);
    }
}

// The small levels of SPyNet (at most kSmallMaxPx pixels per image) in one launch: one
// workgroup per image runs prepare + the five 7x7 convs + the flow add of every such
// level back to back, the activations held in LDS as CB8 tiles with a 3-pixel zero border
// (the per-layer launches cost 2.3-6 us each on these 4..16-pixel maps, mostly launch and
// latency). Each conv is an implicit GEMM on v_mfma_f32_16x16x32_f16: one 16-pixel row
// tile, every 16-channel column block, the K range split over the NW waves (each wave
// streams only its slice of the weights), partial sums added in wave order in LDS.
constexpr int kSmallMaxPx = 16;
constexpr int kSmallMaxNb = 4;
constexpr int kSmallLayerIn[5] = {8, 32, 64, 32, 16};
constexpr int kSmallLayerOut[5] = {32, 64, 32, 16, 2};

struct SmallLevel {
    const uint16_t* pyr;  // pyramid level [frame][3][h][w]
    const void* wpk[5];
    const float* bias[5];
    uint32_t wpk_bytes[5];
    int h, w;
};

struct SmallArgs {
    SmallLevel level[kSpynetMaxLevels];
    uint16_t* flow_out;  // [b][2][h][w] of the last fused level
    int levels, units;   // fused levels; LDS units per activation block
    int pairs;
};

template <int NW>
__global__ __launch_bounds__(64 * NW) void spynet_small_kernel(SmallArgs a) {
    constexpr int U = 8;  // K-steps of loads in flight
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int units = a.units;
    u32x4* tiles = reinterpret_cast<u32x4*>(lds);  // [2][8 blocks][units]
    f32x4* red = reinterpret_cast<f32x4*>(lds + (size_t)2 * 8 * units * 16);  // [NW][kSmallMaxNb][64]
    uint16_t* fprev = reinterpret_cast<uint16_t*>(red + NW * kSmallMaxNb * 64);  // [2][kSmallMaxPx]
    uint16_t* fbase = fprev + 2 * kSmallMaxPx;                                     // [2][kSmallMaxPx]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int quarter = lane >> 4;
    const int b = blockIdx.x;
    int rf, sf;
    pair_frames(b, a.pairs, rf, sf);

    for (int l = 0; l < a.levels; ++l) {
        const SmallLevel& L = a.level[l];
        const int h = L.h, w = L.w, npx = h * w, hp = h + 6, wp = w + 6;
        const uint16_t* ref = L.pyr + (size_t)rf * 3 * npx;
        const uint16_t* sup = L.pyr + (size_t)sf * 3 * npx;
        // This level's tile geometry: every border unit must read zero.
        for (int i = tid; i < 2 * 8 * units; i += 64 * NW) tiles[i] = u32x4{0u, 0u, 0u, 0u};
        __syncthreads();
        // spynet_prepare_fp16 (MetalShader.swift:601-639) for this image's pixels.
        if (tid < npx) {
            const int y = tid / w;
            const int x = tid - y * w;
            float flow_x = 0.0f, flow_y = 0.0f;
            if (l > 0) {
                const int sh = a.level[l - 1].h, sw = a.level[l - 1].w;
                const float sx = w > 1 ? (float)x * (float)(sw - 1) / (float)(w - 1) : 0.0f;
                const float sy = h > 1 ? (float)y * (float)(sh - 1) / (float)(h - 1) : 0.0f;
                flow_x = 2.0f * sample_border(fprev, sh, sw, sy, sx);
                flow_y = 2.0f * sample_border(fprev + kSmallMaxPx, sh, sw, sy, sx);
            }
            fbase[tid] = f2h(flow_x);
            fbase[kSmallMaxPx + tid] = f2h(flow_y);
            uint16_t v[8];
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                v[c] = ref[c * npx + tid];
                v[c + 3] = f2h(sample_border(sup + c * npx, h, w, (float)y + flow_y, (float)x + flow_x));
            }
            v[6] = f2h(flow_x);
            v[7] = f2h(flow_y);
            u32x4 unit;
#pragma unroll
            for (int i = 0; i < 4; ++i) unit[i] = (uint32_t)v[2 * i] | ((uint32_t)v[2 * i + 1] << 16);
            tiles[(y + 3) * wp + x + 3] = unit;
        }
        __syncthreads();

        // A rows: pixel lane % 16 of the single row tile (the tail repeats the last pixel).
        const int p = min(lane & 15, npx - 1);
        const int py = p / w;
        const int px = p - py * w;
        int cur = 0;
        for (int li = 0; li < 5; ++li) {
            const int CB = kSmallLayerIn[li] / 8;
            const int cout = kSmallLayerOut[li];
            const int KB = 49 * CB;
            const int ksteps = (KB + 3) / 4;
            const int nnb = (cout + 15) / 16;  // = the packed layout's column blocks
            const u32x4* in = tiles + (size_t)cur * 8 * units;
            const __amdgpu_buffer_rsrc_t wr = make_rsrc(L.wpk[li], L.wpk_bytes[li]);
            f32x4 acc[kSmallMaxNb];
#pragma unroll
            for (int nb = 0; nb < kSmallMaxNb; ++nb) acc[nb] = f32x4{};
            const int s0 = wave * ksteps / NW;
            const int s1 = (wave + 1) * ksteps / NW;
            for (int sb = s0; sb < s1; sb += U) {
                h8 Bf[U][kSmallMaxNb];
                u32x4 q[U];
#pragma unroll
                for (int i = 0; i < U; ++i) {
                    const int s = sb + i < s1 ? sb + i : s1 - 1;
#pragma unroll
                    for (int nb = 0; nb < kSmallMaxNb; ++nb)
                        if (nb < nnb)
                            Bf[i][nb] = __builtin_bit_cast(
                                h8, load16(wr, (uint32_t)((s * nnb + nb) * 64 + lane) * 16u));
                    const int kb = min(4 * s + quarter, KB - 1);
                    const int tap = kb / CB;
                    const int cb = kb - tap * CB;
                    const int ky = tap / 7;
                    const int kx = tap - ky * 7;
                    q[i] = in[(cb * hp + py + ky) * wp + px + kx];
                }
#pragma unroll
                for (int i = 0; i < U; ++i) {
                    if (sb + i < s1) {  // uniform across the wave
                        const u32x4 z = {0u, 0u, 0u, 0u};
                        const h8 A = __builtin_bit_cast(h8, 4 * (sb + i) + quarter < KB ? q[i] : z);
#pragma unroll
                        for (int nb = 0; nb < kSmallMaxNb; ++nb)
                            if (nb < nnb)
                                acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bf[i][nb], acc[nb], 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int nb = 0; nb < kSmallMaxNb; ++nb) red[(wave * kSmallMaxNb + nb) * 64 + lane] = acc[nb];
            __syncthreads();
            const float* redf = reinterpret_cast<const float*>(red);
            uint16_t* outh = reinterpret_cast<uint16_t*>(tiles + (size_t)(cur ^ 1) * 8 * units);
            for (int e = tid; e < nnb * 256; e += 64 * NW) {
                const int nb = e >> 8;
                const int r = (e >> 4) & 15;
                const int c = e & 15;
                const int oc = nb * 16 + c;
                if (r >= npx || oc >= cout) continue;
                const int src = ((r >> 2) << 4) + c;
                float sum = 0.0f;
#pragma unroll
                for (int k = 0; k < NW; ++k) sum += redf[((k * kSmallMaxNb + nb) * 64 + src) * 4 + (r & 3)];
                float v = sum + L.bias[li][oc];
                if (li < 4) {
                    if (v < 0.0f) v = 0.0f;
                    const int ry = r / w;
                    const int rx = r - ry * w;
                    outh[((size_t)((oc >> 3) * hp + ry + 3) * wp + rx + 3) * 8 + (oc & 7)] = f2h(v);
                } else {
                    // spynet_add_flow_fp16: flow = half(base + half(residual)).
                    fprev[oc * kSmallMaxPx + r] = f2h(h2f(fbase[oc * kSmallMaxPx + r]) + (float)round_f16(v));
                }
            }
            __syncthreads();
            cur ^= 1;
        }
    }
    const int npx = a.level[a.levels - 1].h * a.level[a.levels - 1].w;
    for (int t = tid; t < 2 * npx; t += 64 * NW)
        a.flow_out[(size_t)b * 2 * npx + t] = fprev[(t / npx) * kSmallMaxPx + t % npx];
}

// OIHW [Cout][Cin][KS][KS] -> [ksteps][NBT][64][8]: lane l of K-step s holds output channel
// nb * 16 + l % 16 and K-block 4 s + l / 16 = tap * CB + cb (zero past Cin, Cout, KB).
__global__ __launch_bounds__(256) void convk_prepack_kernel(const uint16_t* __restrict__ w,
                                                            const uint16_t* __restrict__ bias,
                                                            uint16_t* __restrict__ wpk,
                                                            float* __restrict__ bpk, int KS, int Cin,
                                                            int Cout, int CB, int KB, int NBT,
                                                            long total) {
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid < Cout) bpk[gid] = h2f(bias[gid]);
    if (gid >= total) return;
    const int e = (int)(gid & 7);
    const int lane = (int)((gid >> 3) & 63);
    const long q = gid >> 9;
    const int nb = (int)(q % NBT);
    const int s = (int)(q / NBT);
    const int kb = 4 * s + (lane >> 4);
    const int oc = nb * 16 + (lane & 15);
    uint16_t v = 0;
    if (kb < KB && oc < Cout) {
        const int tap = kb / CB;
        const int ic = (kb - tap * CB) * 8 + e;
        if (ic < Cin) v = w[((size_t)oc * Cin + ic) * KS * KS + tap];
    }
    wpk[gid] = v;
}

}  // namespace

ConvKGeometry convk_geometry(int ks, int cin, int cout, int height, int width) {
    ConvKGeometry g;
    g.ks = ks;
    g.cin = cin;
    g.cout = cout;
    g.h = height;
    g.w = width;
    g.cb = (cin + 7) / 8;
    g.kb = ks * ks * g.cb;
    g.ksteps = (g.kb + 3) / 4;
    g.nb = std::min(4, (cout + 15) / 16);
    g.chunks = (cout + 16 * g.nb - 1) / (16 * g.nb);
    g.nbt = g.chunks * g.nb;
    return g;
}

size_t convk_packed_bytes(const ConvKGeometry& g) { return (size_t)g.ksteps * g.nbt * 64 * 8 * 2; }

hipError_t launch_convk_prepack(const ConvKGeometry& g, const uint16_t* w, const uint16_t* bias, void* wpk,
                                float* bpk, hipStream_t stream) {
    const long total = (long)g.ksteps * g.nbt * 64 * 8;
    hipLaunchKernelGGL(convk_prepack_kernel, dim3(blocks_for(std::max<long>(total, g.cout))), dim3(256), 0,
                       stream, w, bias, (uint16_t*)wpk, bpk, g.ks, g.cin, g.cout, g.cb, g.kb, g.nbt, total);
    return hipGetLastError();
}

namespace {

template <int NB>
hipError_t launch_convk_nb(const ConvKGeometry& g, ConvKArgs& a, hipStream_t stream) {
    constexpr int NW = 8, U = 4;
    const size_t lds = (size_t)NW * NB * 4 * 65 * sizeof(float);
    const dim3 grid((unsigned)((a.tiles + 7) / 8 * 8), (unsigned)g.chunks);
    if (g.ks == 7) {
        hipLaunchKernelGGL((convk_kernel<7, NW, U, NB>), grid, dim3(64 * NW), lds, stream, a);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_convk(const ConvKGeometry& g, int batch, int pad, const void* x_cb8, const void* wpk,
                        const float* bias, int act, const uint16_t* base, uint16_t* out, int out_cb8,
                        hipStream_t stream) {
    if (pad < g.ks / 2) return hipErrorInvalidValue;
    ConvKArgs a{};
    a.xin = x_cb8;
    a.wpk = wpk;
    a.bias = bias;
    a.base = base;
    a.out = out;
    a.B = batch;
    a.H = g.h;
    a.W = g.w;
    a.pad = pad;
    a.Hp = g.h + 2 * pad;
    a.Wp = g.w + 2 * pad;
    a.CB = g.cb;
    a.KB = g.kb;
    a.ksteps = g.ksteps;
    a.NBT = g.nbt;
    a.Cout = g.cout;
    a.act = act;
    a.out_cb8 = out_cb8;
    a.xin_bytes = (uint32_t)((size_t)batch * g.cb * a.Hp * a.Wp * 16);
    a.wpk_bytes = (uint32_t)convk_packed_bytes(g);
    a.tiles = (batch * g.h * g.w + 15) / 16;
    a.magic_cb = magic_for(g.cb);
    switch (g.nb) {
        case 1: return launch_convk_nb<1>(g, a, stream);
        case 2: return launch_convk_nb<2>(g, a, stream);
        case 4: return launch_convk_nb<4>(g, a, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_bicubic_quarter(const uint16_t* in, uint16_t* out, int channels, int height, int width,
                                  hipStream_t stream) {
    const long n = (long)channels * (height / 4) * (width / 4);
    hipLaunchKernelGGL(bicubic_quarter_kernel, dim3(blocks_for(n)), dim3(256), 0, stream, in, out, channels,
                       height, width);
    return hipGetLastError();
}

hipError_t launch_spynet_pyramid(const uint16_t* frame0, const uint16_t* frame1, long frame_stride, int count,
                                 uint16_t* const* levels, int nlevels, int height, int width, hipStream_t stream) {
    if (count < 1 || nlevels < 1 || nlevels > kSpynetMaxLevels) return hipErrorInvalidValue;
    PyramidArgs a{};
    a.frames = count;
    a.levels = nlevels;
    a.H = height;
    a.W = width;
    long off = 0;
    for (int l = 0; l < nlevels; ++l) {
        a.offset[l] = off;
        const int shift = nlevels - 1 - l;
        off += 3L * (height >> shift) * (width >> shift);
        a.level[l] = levels[l];
    }
    a.offset[nlevels] = off;
    a.frame[0] = frame0;
    a.frame[1] = count > 1 ? frame1 : frame0;
    a.frame_stride = frame_stride;
    a.aligned = width % 8 == 0 && reinterpret_cast<uintptr_t>(frame0) % 16 == 0 &&
                reinterpret_cast<uintptr_t>(a.frame[1]) % 16 == 0 && (count <= 2 || frame_stride % 8 == 0);
    // Coarse levels come first; those whose factor is in [16, 64] get a wave per output.
    a.coarse = 0;
    if (a.aligned)
        for (int l = 0; l < nlevels; ++l) {
            const int factor = 1 << (nlevels - 1 - l);
            if (factor >= kPyramidWaveFactor && factor <= kPyramidMaxFactor) a.coarse = a.offset[l + 1];
        }
    for (int l = 0; l < nlevels && a.coarse > 0; ++l)  // the wave path must start at level 0
        if ((1 << (nlevels - 1 - l)) > kPyramidMaxFactor) a.coarse = 0;
    const long blocks = a.coarse * count + ((off - a.coarse) * count + 63) / 64;
    hipLaunchKernelGGL(spynet_pyramid_kernel, dim3((unsigned)blocks), dim3(64), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_spynet_prepare(int batch, int pairs, const uint16_t* pyramid_level, const uint16_t* source_flow,
                                 int source_height, int source_width, int first_level, uint16_t* features, int pad,
                                 uint16_t* base_flow, int height, int width, hipStream_t stream) {
    if (batch < 1 || pairs < 1 || batch > 2 * pairs) return hipErrorInvalidValue;
    PrepareArgs a{};
    a.level = pyramid_level;
    a.pairs = pairs;
    a.source_flow = source_flow;
    a.features = features;
    a.base_flow = base_flow;
    a.batch = batch;
    a.H = height;
    a.W = width;
    a.SH = source_height;
    a.SW = source_width;
    a.first_level = first_level;
    a.pad = pad;
    hipLaunchKernelGGL(spynet_prepare_kernel, dim3(blocks_for((long)batch * height * width)), dim3(256), 0,
                       stream, a);
    return hipGetLastError();
}

size_t spynet_small_lds_bytes(int units) {
    return (size_t)2 * 8 * units * 16 + (size_t)8 * kSmallMaxNb * 64 * 16 + (size_t)4 * kSmallMaxPx * 2;
}

hipError_t launch_spynet_small(int batch, int pairs, int levels, const int* heights, const int* widths,
                               const uint16_t* const* pyramid, const void* const (*wpk)[5],
                               const float* const (*bias)[5], const uint32_t (*wpk_bytes)[5], uint16_t* flow_out,
                               hipStream_t stream) {
    if (batch < 1 || pairs < 1 || batch > 2 * pairs || levels < 1 || levels > kSpynetMaxLevels)
        return hipErrorInvalidValue;
    constexpr int NW = 8;
    SmallArgs a{};
    a.levels = levels;
    a.pairs = pairs;
    a.flow_out = flow_out;
    int units = 0;
    for (int l = 0; l < levels; ++l) {
        if (heights[l] * widths[l] > kSmallMaxPx) return hipErrorInvalidValue;
        SmallLevel& L = a.level[l];
        L.h = heights[l];
        L.w = widths[l];
        L.pyr = pyramid[l];
        for (int i = 0; i < 5; ++i) {
            L.wpk[i] = wpk[l][i];
            L.bias[i] = bias[l][i];
            L.wpk_bytes[i] = wpk_bytes[l][i];
        }
        units = std::max(units, (L.h + 6) * (L.w + 6));
    }
    a.units = units;
    const size_t lds = spynet_small_lds_bytes(units);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    auto kernel = &spynet_small_kernel<NW>;
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), 160 * 1024);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kernel, dim3((unsigned)batch), dim3(64 * NW), lds, stream, a);
    return hipGetLastError();
}

}  // namespace dcn
