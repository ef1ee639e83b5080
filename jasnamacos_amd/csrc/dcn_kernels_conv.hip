// 3x3 convolution (stride 1, pad 1) for the propagation body's offset branch and
// backbone: FP16 storage, FP32 accumulation on v_mfma_f32_16x16x32_f16.
//
// Implicit GEMM over the CB8 input ([Cin/8][H+4][W+4][8], 2-pixel zero border): out
// [pixel][oc] = sum over K-blocks kb = tap * CB + cb of x[cb][y + ky - 1][x + kx - 1][0..7]
// . W[oc][8 cb .. 8 cb + 7][ky][kx]. A K-block of one pixel is one 16-byte load and the
// border supplies the zero padding, so the A fragment needs no arithmetic at all (the
// deformable kernels' sampler with integer offsets and no blend). Lane layout, tiling,
// K split over waves and the LDS reduction follow dcn_kernels_narrow.hip: 16-pixel tiles,
// lane l takes pixel l%16 and K-block 4s + l/16 of K-step s.
//
// Workgroup (tile, chunk) computes 64 output channels (4 column blocks of 16) of 16
// pixels; chunks split Cout (432 -> 7 chunks, the last one partly padded with zero
// weights). Epilogue: + bias, activation (none / LeakyReLU(slope) / ReLU), optional
// residual r1 and second residual r2, each add rounded to FP16 as a separate FP16 op:
// out = half(r2 + half(r1 + act(acc))). Output NCHW or CB8. conv_offsets_kernel (the
// body's last conv_offset layer) turns the FP16 conv output into DCN offsets and masks.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "dcn_device.hpp"
#include "dcn_warp.hpp"
#include "dcn_internal.hpp"

#pragma clang fp contract(off)

namespace dcn {
namespace {

using namespace dev;

constexpr int kConvChunk = 64;  // output channels per workgroup
constexpr int kConvNbc = kConvChunk / 16;
constexpr int kConvRedStride = 68;  // conv3x3_kernel's partial-sum row (64 lanes + padding)
static_assert(kConvChunk == 64, "the conv epilogues map 64 channels to a wave");

struct ConvArgs {
    const void* xin;        // CB8 input
    const void* wpk;        // [ksteps][NBT][64][8] FP16
    const float* bias;      // [Cout] FP32
    const uint16_t* res1;   // optional residual (layout res1_layout)
    const uint16_t* res2;   // optional second residual (layout res2_layout)
    uint16_t* out;
    uint32_t xin_bytes, wpk_bytes;
    int res1_layout, res2_layout, out_layout;
    int res2_coff;          // channel offset of the second residual inside its tensor
    // conv_offsets_kernel (cout 432): offsets and masks from half(conv + bias).
    int offsets;
    const uint16_t* flow1;  // [2][H][W] (x, y)
    const uint16_t* flow2;
    uint16_t* offset;       // [288][H][W]
    uint16_t* mask;         // [144][H][W]
    int H, W, Hp, Wp, CB, KB, ksteps, NBT, Cout, tiles, act;
    float slope;
    uint32_t magic_cb;
    // Image blockIdx.z of a batch: every tensor advances by its per-image stride (elements).
    long xin_ts, res1_ts, res2_ts, out_ts, flow_ts, offset_ts, mask_ts;
};

// The arguments of image z of a batch of images.
__device__ __forceinline__ ConvArgs conv_image_at(const ConvArgs& a0, long z) {
    ConvArgs a = a0;
    a.xin = static_cast<const uint16_t*>(a0.xin) + z * a0.xin_ts;
    if (a.res1) a.res1 += z * a0.res1_ts;
    if (a.res2) a.res2 += z * a0.res2_ts;
    if (a.out) a.out += z * a0.out_ts;
    if (a.flow1) a.flow1 += z * a0.flow_ts;
    if (a.flow2) a.flow2 += z * a0.flow_ts;
    if (a.offset) a.offset += z * a0.offset_ts;
    if (a.mask) a.mask += z * a0.mask_ts;
    return a;
}
__device__ __forceinline__ ConvArgs conv_image(const ConvArgs& a0) { return conv_image_at(a0, blockIdx.z); }

__device__ __forceinline__ size_t conv_index(int layout, int c, int y, int x, int H, int W, int Hp,
                                             int Wp) {
    if (layout == kLayoutCB8) return ((size_t)((c >> 3) * Hp + y + kPad) * Wp + x + kPad) * 8 + (c & 7);
    return ((size_t)c * H + y) * W + x;
}

template <int NW, int U>
__global__ __launch_bounds__(64 * NW) void conv3x3_kernel(ConvArgs a0) {
    const ConvArgs a = conv_image(a0);
    constexpr int NB = kConvNbc;
    // Partial sums [NW][NB][4][kConvRedStride]: rows of 64 lanes padded to 68 floats, so that
    // the epilogue's channel-fastest reads (bank 16 nb + oc % 16) are conflict-free.
    extern __shared__ float red[];
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

    const int M = a.H * a.W;
    const int p = tile * 16 + (lane & 15);
    const bool pvalid = p < M;
    const int pc = pvalid ? p : M - 1;
    const int y = pc / a.W;
    const int x = pc - y * a.W;
    // 16-byte unit of (cb 0, y - 1, x - 1) in the padded plane.
    const uint32_t base = (uint32_t)(y + kPad - 1) * a.Wp + x + kPad - 1;

    // The epilogue's biases, requested first (clamped index, no branch): loaded in the
    // epilogue they cost a round trip after the reduction.
    constexpr int kItems = 16 * kConvChunk;
    constexpr int kIters = (kItems + 64 * NW - 1) / (64 * NW);
    float biasv[kIters];
#pragma unroll
    for (int j = 0; j < kIters; ++j)
        biasv[j] = a.bias[min(chunk * kConvChunk + ((tid + j * 64 * NW) & (kConvChunk - 1)), a.Cout - 1)];

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
            if (sb + i >= s1) continue;  // uniform across the wave; the slot stays unused
            const int s = sb + i;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                Bf[i][nb] = __builtin_bit_cast(
                    h8, load16(wr, (uint32_t)((s * a.NBT + chunk * NB + nb) * 64 + lane) * 16u));
            const int kb = 4 * s + quarter;
            const int kbc = kb < a.KB ? kb : a.KB - 1;
            const int tap = fast_div(kbc, a.magic_cb);
            const int cb = kbc - tap * a.CB;
            const int ky = (tap * 11) >> 5;  // tap / 3 for tap < 9
            const int kx = tap - ky * 3;
            q[i] = load16(xr, (base + (uint32_t)(cb * a.Hp + ky) * a.Wp + kx) * 16u);
        }
#pragma unroll
        for (int i = 0; i < U; ++i) {
            if (sb + i < s1) {  // uniform across the wave
                const int kb = 4 * (sb + i) + quarter;
                const u32x4 z = {0u, 0u, 0u, 0u};
                // Padding K-blocks multiply zero weights; zero A keeps a non-finite
                // input from turning 0 * inf into NaN there.
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
        for (int v = 0; v < 4; ++v) red[((wave * NB + nb) * 4 + v) * kConvRedStride + lane] = acc[nb][v];
    __syncthreads();

    // Item idx: channel idx % 64 of pixel idx / 64, so that a wave's stores fill whole CB8
    // units (eight consecutive channels of a pixel).
#pragma unroll
    for (int j = 0; j < kIters; ++j) {
        const int idx = tid + j * 64 * NW;
        if (idx >= kItems) break;
        const int ocl = idx & (kConvChunk - 1);
        const int pl = idx >> 6;
        const int nb = ocl >> 4;
        const int src = ((pl >> 2) << 4) + (ocl & 15);
        const int v = pl & 3;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) sum += red[((w * NB + nb) * 4 + v) * kConvRedStride + src];
        const int oc = chunk * kConvChunk + ocl;
        const int pp = tile * 16 + pl;
        if (pp >= M || oc >= a.Cout) continue;
        const int yy = pp / a.W;
        const int xx = pp - yy * a.W;
        float r = sum + biasv[j];
        if (a.act == 1 && r < 0.0f) r = r * a.slope;
        if (a.act == 2 && r < 0.0f) r = 0.0f;
        if (a.res1 != nullptr) {
            const float id = (float)__builtin_bit_cast(
                _Float16, a.res1[conv_index(a.res1_layout, oc, yy, xx, a.H, a.W, a.Hp, a.Wp)]);
            r = id + r;
        }
        if (a.res2 != nullptr) {
            const float r1 = (float)round_f16(r);
            const float id = (float)__builtin_bit_cast(
                _Float16, a.res2[conv_index(a.res2_layout, a.res2_coff + oc, yy, xx, a.H, a.W, a.Hp, a.Wp)]);
            r = id + r1;
        }
        a.out[conv_index(a.out_layout, oc, yy, xx, a.H, a.W, a.Hp, a.Wp)] =
            __builtin_bit_cast(uint16_t, round_f16(r));
    }
}

// conv3x3_kernel<NW, U> for a batch of images (the body over many tiles): workgroup
// (tile, chunk, z) runs images z * zpw .. z * zpw + zpw - 1 one after another. Each wave
// keeps the weight fragments of its K range (at most KMAX K-steps) in registers for all of
// them and requests the next image's rows before the current one is reduced. Same K split
// and summation order as conv3x3_kernel: every image's results are the same bits.
template <int NW, int KMAX>
__global__ __launch_bounds__(64 * NW) void conv3x3_images_kernel(ConvArgs a0, int images, int zpw) {
    constexpr int NB = kConvNbc;
    constexpr int kItems = 16 * kConvChunk;
    constexpr int kIters = (kItems + 64 * NW - 1) / (64 * NW);
    extern __shared__ float red[];  // [NW][NB][4][kConvRedStride], as conv3x3_kernel
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int quarter = lane >> 4;

    const int per_xcd = (a0.tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= a0.tiles) return;  // whole workgroup, before any barrier
    const int chunk = blockIdx.y;
    const int z0 = blockIdx.z * zpw;
    const int z1 = min(z0 + zpw, images);

    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a0.wpk, a0.wpk_bytes);
    const int M = a0.H * a0.W;
    const int pc = min(tile * 16 + (lane & 15), M - 1);
    const int y = pc / a0.W;
    const uint32_t base = (uint32_t)(y + kPad - 1) * a0.Wp + (pc - y * a0.W) + kPad - 1;

    const int s0 = wave * a0.ksteps / NW;
    const int s1 = (wave + 1) * a0.ksteps / NW;
    h8 Bf[KMAX][NB];
    uint32_t koff[KMAX];
    bool kin[KMAX];
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
        const int s = s0 + i < s1 ? s0 + i : s1 - 1;
        if (s0 + i < s1)  // uniform across the wave; slots past the range stay unused
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                Bf[i][nb] = __builtin_bit_cast(
                    h8, load16(wr, (uint32_t)((s * a0.NBT + chunk * NB + nb) * 64 + lane) * 16u));
        const int kb = 4 * s + quarter;
        kin[i] = kb < a0.KB;
        const int kbc = kin[i] ? kb : a0.KB - 1;
        const int tap = fast_div(kbc, a0.magic_cb);
        const int cb = kbc - tap * a0.CB;
        const int ky = (tap * 11) >> 5;  // tap / 3 for tap < 9
        const int kx = tap - ky * 3;
        koff[i] = (uint32_t)(cb * a0.Hp + ky) * a0.Wp + kx;
    }
    u32x4 q[KMAX];
    auto load_rows = [&](int z) {
        const __amdgpu_buffer_rsrc_t xr =
            make_rsrc(static_cast<const uint16_t*>(a0.xin) + (long)z * a0.xin_ts, a0.xin_bytes);
#pragma unroll
        for (int i = 0; i < KMAX; ++i)
            if (s0 + i < s1) q[i] = load16(xr, (base + koff[i]) * 16u);
    };
    load_rows(z0);
    float biasv[kIters];
#pragma unroll
    for (int j = 0; j < kIters; ++j) {
        const int oc = chunk * kConvChunk + ((tid + j * 64 * NW) & (kConvChunk - 1));
        biasv[j] = oc < a0.Cout ? a0.bias[oc] : 0.0f;
    }

    for (int z = z0; z < z1; ++z) {
        const ConvArgs a = conv_image_at(a0, z);
        f32x4 acc[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{};
#pragma unroll
        for (int i = 0; i < KMAX; ++i) {
            if (s0 + i < s1) {  // uniform across the wave
                const u32x4 zero = {0u, 0u, 0u, 0u};
                // Padding K-blocks multiply zero weights; zero A keeps a non-finite
                // input from turning 0 * inf into NaN there.
                const h8 A = __builtin_bit_cast(h8, kin[i] ? q[i] : zero);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bf[i][nb], acc[nb], 0, 0, 0);
            }
        }
        if (z + 1 < z1) load_rows(z + 1);  // in flight through the reduction and epilogue
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int v = 0; v < 4; ++v) red[((wave * NB + nb) * 4 + v) * kConvRedStride + lane] = acc[nb][v];
        __syncthreads();

#pragma unroll
        for (int j = 0; j < kIters; ++j) {  // channel-fastest items, as conv3x3_kernel
            const int idx = tid + j * 64 * NW;
            const int ocl = idx & (kConvChunk - 1);
            const int pl = idx >> 6;
            const int nb = ocl >> 4;
            const int src = ((pl >> 2) << 4) + (ocl & 15);
            const int v = pl & 3;
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) sum += red[((w * NB + nb) * 4 + v) * kConvRedStride + src];
            const int oc = chunk * kConvChunk + ocl;
            const int pp = tile * 16 + pl;
            if (pp >= M || oc >= a.Cout) continue;
            const int yy = pp / a.W;
            const int xx = pp - yy * a.W;
            float r = sum + biasv[j];
            if (a.act == 1 && r < 0.0f) r = r * a.slope;
            if (a.act == 2 && r < 0.0f) r = 0.0f;
            if (a.res1 != nullptr) {
                const float id = (float)__builtin_bit_cast(
                    _Float16, a.res1[conv_index(a.res1_layout, oc, yy, xx, a.H, a.W, a.Hp, a.Wp)]);
                r = id + r;
            }
            if (a.res2 != nullptr) {
                const float r1 = (float)round_f16(r);
                const float id = (float)__builtin_bit_cast(
                    _Float16, a.res2[conv_index(a.res2_layout, a.res2_coff + oc, yy, xx, a.H, a.W, a.Hp, a.Wp)]);
                r = id + r1;
            }
            a.out[conv_index(a.out_layout, oc, yy, xx, a.H, a.W, a.Hp, a.Wp)] =
                __builtin_bit_cast(uint16_t, round_f16(r));
        }
        if (z + 1 < z1) __syncthreads();  // sums read before the next image's partials
    }
}

// The last conv_offset layer (64 -> 432) with prepare_dcn_offsets_fp16 in its epilogue.
// Its 1,792 workgroups (256 tiles x 7 chunks of 64 channels) queue on the CUs, so
// occupancy sets its time: conv3x3_kernel<8, 4> holds four K-steps of weight fragments
// (108 VGPRs, two workgroups per CU, four rounds). This kernel keeps U K-steps in flight
// under a MINW waves-per-SIMD bound; the launcher uses U = 2, MINW = 6 (65 VGPRs, three
// workgroups per CU). Measured per body frame against conv3x3_kernel: 95.3 -> 91.5 us.
// Wider tiles (RT row tiles x 16 NB channels: 2 x 144 and 1 x 144) cut the weight
// traffic but measured slower (96.0 and 96.5 us: fewer, longer workgroups per CU).
// Same K split and summation order as conv3x3_kernel<NW, U>: the results are the same
// bits.
template <int NW, int U, int NB, int RT, int MINW>
__global__ __launch_bounds__(64 * NW, MINW) void conv_offsets_kernel(ConvArgs a0) {
    const ConvArgs a = conv_image(a0);
    extern __shared__ __attribute__((aligned(16))) f32x4 red4[];  // [NW][RT][NB][64] partial sums
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

    const int M = a.H * a.W;
    uint32_t base[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int pc = min((tile * RT + rt) * 16 + (lane & 15), M - 1);
        const int y = pc / a.W;
        const int x = pc - y * a.W;
        base[rt] = (uint32_t)(y + kPad - 1) * a.Wp + x + kPad - 1;
    }

    f32x4 acc[RT][NB];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[rt][nb] = f32x4{};

    const int s0 = wave * a.ksteps / NW;
    const int s1 = (wave + 1) * a.ksteps / NW;
    for (int sb = s0; sb < s1; sb += U) {
        h8 Bf[U][NB];
        u32x4 q[U][RT];
#pragma unroll
        for (int i = 0; i < U; ++i) {
            if (sb + i >= s1) continue;  // uniform across the wave; the slot stays unused
            const int s = sb + i;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                Bf[i][nb] = __builtin_bit_cast(
                    h8, load16(wr, (uint32_t)((s * a.NBT + chunk * NB + nb) * 64 + lane) * 16u));
            const int kb = 4 * s + quarter;
            const int kbc = kb < a.KB ? kb : a.KB - 1;
            const int tap = fast_div(kbc, a.magic_cb);
            const int cb = kbc - tap * a.CB;
            const int ky = (tap * 11) >> 5;  // tap / 3 for tap < 9
            const int kx = tap - ky * 3;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                q[i][rt] = load16(xr, (base[rt] + (uint32_t)(cb * a.Hp + ky) * a.Wp + kx) * 16u);
        }
#pragma unroll
        for (int i = 0; i < U; ++i) {
            if (sb + i < s1) {  // uniform across the wave
                const int kb = 4 * (sb + i) + quarter;
                const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const h8 A = __builtin_bit_cast(h8, kb < a.KB ? q[i][rt] : z);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        acc[rt][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bf[i][nb], acc[rt][nb], 0, 0, 0);
                }
            }
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) red4[((wave * RT + rt) * NB + nb) * 64 + lane] = acc[rt][nb];
    __syncthreads();

    // Thread (rt, nb, l, h) sums the 8-byte half h of rows (w, rt, nb, l) over the waves in
    // wave order (consecutive threads read consecutive 8 bytes: no bank conflicts), giving
    // pixels (tile * RT + rt) * 16 + 4 (l / 16) + 2 h + j (j = 0, 1) of channel
    // chunk * 16 NB + 16 nb + l % 16. Two outputs per thread keep every wave busy in the
    // transcendental epilogue.
    const size_t plane = (size_t)M;
    const float2* red2 = reinterpret_cast<const float2*>(red4);
    for (int g = tid; g < RT * NB * 128; g += 64 * NW) {
        const int h = g & 1;
        const int row = g >> 1;  // (rt, nb, l)
        const int l = row & 63;
        const int nb = (row >> 6) % NB;
        const int rt = row / (NB * 64);
        float2 sum = {0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float2 t = red2[(((w * RT + rt) * NB + nb) * 64 + l) * 2 + h];
            sum.x += t.x;
            sum.y += t.y;
        }
        const int oc = chunk * 16 * NB + nb * 16 + (l & 15);
        if (oc >= a.Cout) continue;
        const float bias = a.bias[oc];
        const int p0 = (tile * RT + rt) * 16 + 4 * (l >> 4) + 2 * h;
        // prepare_dcn_offsets_fp16 (MetalShader.swift:815-839) on the FP16 conv output.
        const uint16_t* flow = oc < 144 ? a.flow1 : a.flow2;
        const int flow_channel = ((oc % 144) & 1) == 0 ? 1 : 0;  // even = dy = flow y
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int px = p0 + j;
            if (px >= M) continue;
            const float raw = (float)round_f16((j ? sum.y : sum.x) + bias);
            if (oc < 288) {
                const float residue = 10.0f * tanhf(raw);
                const float f = (float)__builtin_bit_cast(_Float16, flow[flow_channel * plane + px]);
                a.offset[(size_t)oc * plane + px] = __builtin_bit_cast(uint16_t, round_f16(residue + f));
            } else {
                a.mask[(size_t)(oc - 288) * plane + px] =
                    __builtin_bit_cast(uint16_t, round_f16(1.0f / (1.0f + expf(-raw))));
            }
        }
    }
}

// Conv weights OIHW FP16 [Cout][Cin][3][3] -> B fragments [ksteps][NBT][64][8]:
// lane l of K-step s holds output channel nb*16 + l%16 and K-block 4s + l/16 =
// tap * CB + cb, channels 8 cb .. 8 cb + 7 (zero past Cin, past Cout and past KB).
__global__ __launch_bounds__(256) void conv_prepack_kernel(const uint16_t* __restrict__ w,
                                                           const uint16_t* __restrict__ bias,
                                                           uint16_t* __restrict__ wpk,
                                                           float* __restrict__ bpk, int Cin,
                                                           int Cout, int CB, int KB, int NBT,
                                                           long total) {
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid < Cout) bpk[gid] = (float)__builtin_bit_cast(_Float16, bias[gid]);
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
        if (ic < Cin) v = w[((size_t)oc * Cin + ic) * 9 + tap];
    }
    wpk[gid] = v;
}

// Two chained 64 -> 64 convolutions in one launch (a residual block, or two conv_offset
// layers): t = half(act1(conv1(x) + b1)), out = epilogue(conv2(t) + b2) with the
// epilogue of conv3x3_kernel. A workgroup owns a 2 x 8 output tile (256 workgroups on a
// 64 x 64 map, one per CU). It computes t on the 4 x 10 halo of that tile (t is zero
// outside the image: conv2's zero padding) and keeps it in LDS, so the intermediate
// tensor never reaches HBM and the pair costs one launch. Measured on a 64 x 64 body:
// 2 x 8 tiles beat 4 x 8 ones (half the workgroups, each with the whole weight traffic
// of both convs) by about 1 us per pair.
//
// Both convs split K over the NW waves exactly as conv3x3_kernel<NW, U> does (wave w owns
// K-steps [w * 18 / NW, (w + 1) * 18 / NW), MFMA chains in K-step order, partial sums added
// in wave order from 0), so every value equals the two-launch result bit for bit.
//
// Batches: workgroup (tile, z) runs the same tile of images z * zpw .. z * zpw + zpw - 1 one
// after another. Each wave keeps its weight fragments of both convs in registers for all of
// them (the 144 KB of B fragments are fetched once per workgroup instead of once per image)
// and requests the next image's conv1 rows while the current one is reduced and runs conv2.
// The arithmetic of every image is the single-image arithmetic.
constexpr int kPairTH = 2, kPairTW = 8;                 // output tile
constexpr int kPairHH = kPairTH + 2, kPairHW = kPairTW + 2;
constexpr int kPairHalo = kPairHH * kPairHW;            // halo pixels
constexpr int kPairRT1 = (kPairHalo + 15) / 16;         // 16-pixel row tiles of the halo
constexpr int kPairRT2 = kPairTH * kPairTW / 16;        // of the output tile
constexpr int kPairKsteps = 18;                         // 64 channels: 72 K-blocks / 4
constexpr int kPairTStride = kPairRT1 * 16;             // t tile: [8 cb][RT1 * 16 px] 16-byte units

struct PairArgs {
    const void* xin;   // CB8 input, 64 channels
    const void* wpk1;  // [18][4][64][8] FP16
    const void* wpk2;
    const float* bias1;
    const float* bias2;
    const uint16_t* res1;
    const uint16_t* res2;
    uint16_t* out;
    uint16_t* out2;    // optional second copy of the output, CB8 (64 channels)
    uint32_t xin_bytes, wpk_bytes;
    int act1, act2;
    float slope;
    int res1_layout, res2_layout, out_layout, res2_coff;
    int H, W, Hp, Wp, tiles_x, tiles;
    int images, zpw;                        // batch size, images per workgroup
    long xin_ts, res1_ts, res2_ts, out_ts, out2_ts;  // per-image strides of a batch
};

__host__ __device__ constexpr size_t pair_lds_bytes(int nw) {
    return (size_t)nw * kPairRT1 * kConvNbc * 64 * 16 + (size_t)8 * kPairTStride * 16;
}

template <int NW>
__global__ __launch_bounds__(64 * NW) void conv_pair_kernel(PairArgs a) {
    constexpr int NB = kConvNbc;
    constexpr int KMAX = (kPairKsteps + NW - 1) / NW;  // K-steps of the busiest wave
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    f32x4* red4 = reinterpret_cast<f32x4*>(lds);  // [NW][RT][NB][64] partial sums
    u32x4* tt = reinterpret_cast<u32x4*>(lds + (size_t)NW * kPairRT1 * NB * 64 * 16);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int quarter = lane >> 4;

    const int per_xcd = (a.tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= a.tiles) return;  // whole workgroup, before any barrier
    const int ty = tile / a.tiles_x;
    const int oy0 = ty * kPairTH;
    const int ox0 = (tile - ty * a.tiles_x) * kPairTW;

    const int z0 = blockIdx.z * a.zpw;
    const int z1 = min(z0 + a.zpw, a.images);
    const __amdgpu_buffer_rsrc_t w1 = make_rsrc(a.wpk1, a.wpk_bytes);
    const __amdgpu_buffer_rsrc_t w2 = make_rsrc(a.wpk2, a.wpk_bytes);

    // conv1 rows: halo pixel rt * 16 + lane % 16 at image (oy0 - 1 + hy, ox0 - 1 + hx),
    // clamped into [-1, H] x [-1, W] so that every tap stays inside the padded plane
    // (the clamped rows are zeroed below).
    uint32_t base1[kPairRT1];
#pragma unroll
    for (int rt = 0; rt < kPairRT1; ++rt) {
        const int hp = min(rt * 16 + (lane & 15), kPairHalo - 1);
        const int hy = hp / kPairHW;
        const int iy = min(max(oy0 - 1 + hy, -1), a.H);
        const int ix = min(max(ox0 - 1 + hp - hy * kPairHW, -1), a.W);
        base1[rt] = (uint32_t)(iy + kPad - 1) * a.Wp + ix + kPad - 1;
    }

    const int s0 = wave * kPairKsteps / NW;
    const int s1 = (wave + 1) * kPairKsteps / NW;
    // Offset of K-step slot i's K-block (tap, channel block) in the padded CB8 input.
    uint32_t koff[KMAX];
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
        const int s = s0 + i < s1 ? s0 + i : s1 - 1;
        const int kb = 4 * s + quarter;
        const int tap = kb >> 3;
        const int cb = kb & 7;
        const int ky = (tap * 11) >> 5;  // tap / 3 for tap < 9
        const int kx = tap - ky * 3;
        koff[i] = (uint32_t)(cb * a.Hp + ky) * a.Wp + kx;
    }
    h8 B1[KMAX][NB], B2[KMAX][NB];
    u32x4 q[KMAX][kPairRT1];
    auto load_rows = [&](int z) {
        const __amdgpu_buffer_rsrc_t xr =
            make_rsrc(static_cast<const uint16_t*>(a.xin) + (long)z * a.xin_ts, a.xin_bytes);
#pragma unroll
        for (int i = 0; i < KMAX; ++i)
            if (s0 + i < s1)  // uniform across the wave; slots past the range stay unused
#pragma unroll
                for (int rt = 0; rt < kPairRT1; ++rt) q[i][rt] = load16(xr, (base1[rt] + koff[i]) * 16u);
    };
#pragma unroll
    for (int i = 0; i < KMAX; ++i)
        if (s0 + i < s1)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                B1[i][nb] = __builtin_bit_cast(h8, load16(w1, (uint32_t)(((s0 + i) * NB + nb) * 64 + lane) * 16u));
    load_rows(z0);
    // conv2's fragments are requested once conv1's products are issued (first image): in
    // flight behind conv1's operands they only delayed conv1's first wait; they arrive
    // during the two reductions before conv2.
    auto load_b2 = [&]() {
#pragma unroll
        for (int i = 0; i < KMAX; ++i)
            if (s0 + i < s1)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    B2[i][nb] = __builtin_bit_cast(h8, load16(w2, (uint32_t)(((s0 + i) * NB + nb) * 64 + lane) * 16u));
    };

    // Per-thread constants of the two reductions, the same for every image: the biases,
    // and the epilogue's output positions (thread tid < 256 owns output pixels
    // 4 (l / 16) + v of channel 16 nb + l % 16, l = tid % 64, nb = tid / 64).
    constexpr int kSums1 = kPairRT1 * NB * 64;
    constexpr int kIters1 = (kSums1 + 64 * NW - 1) / (64 * NW);
    constexpr int kSums2 = kPairRT2 * NB * 64;
    static_assert(kPairRT2 == 1 && kSums2 <= 64 * NW, "one epilogue item per thread");
    float bias1v[kIters1];
#pragma unroll
    for (int j = 0; j < kIters1; ++j) {
        const int g = tid + j * 64 * NW;
        bias1v[j] = g < kSums1 ? a.bias1[((g >> 6) % NB) * 16 + (g & 15)] : 0.0f;
    }
    const bool epi = tid < kSums2;
    const int epi_oc = ((tid >> 6) % NB) * 16 + (tid & 15);
    const float bias2v = epi ? a.bias2[epi_oc] : 0.0f;
    bool epi_in[4];
    uint32_t epi_out[4], epi_out2[4], epi_r1[4], epi_r2[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int op = 4 * ((tid & 63) >> 4) + v;
        const int yy = oy0 + (op >> 3);
        const int xx = ox0 + (op & 7);
        epi_in[v] = epi && yy < a.H && xx < a.W;
        epi_out[v] = (uint32_t)conv_index(a.out_layout, epi_oc, yy, xx, a.H, a.W, a.Hp, a.Wp);
        epi_out2[v] = (uint32_t)conv_index(kLayoutCB8, epi_oc, yy, xx, a.H, a.W, a.Hp, a.Wp);
        epi_r1[v] = (uint32_t)conv_index(a.res1_layout, epi_oc, yy, xx, a.H, a.W, a.Hp, a.Wp);
        epi_r2[v] = (uint32_t)conv_index(a.res2_layout, a.res2_coff + epi_oc, yy, xx, a.H, a.W, a.Hp, a.Wp);
    }

    // One image; the first (peeled, `first_c`) also requests conv2's fragments.
    auto image = [&](int z, auto first_c) {
        const uint16_t* res1 = a.res1 ? a.res1 + (long)z * a.res1_ts : nullptr;
        const uint16_t* res2 = a.res2 ? a.res2 + (long)z * a.res2_ts : nullptr;
        uint16_t* out = a.out + (long)z * a.out_ts;
        uint16_t* out2 = a.out2 ? a.out2 + (long)z * a.out2_ts : nullptr;
        // The epilogue's residual inputs, requested now so that they arrive during the convs.
        // Every lane issues the same loads on every path (clamped index; an absent tensor is
        // a buffer of 0 bytes, whose loads return 0 without touching memory) into 32-bit
        // registers: a per-lane branch around a 16-bit load, or registers zeroed on one
        // path, make the compiler wait for that load, and so for every load issued before
        // it (conv2's weights included), before conv1 can start.
        const __amdgpu_buffer_rsrc_t r1r = make_rsrc(res1 ? (const void*)res1 : (const void*)a.out,
                                                     res1 ? 0x7ffffffeu : 0u);
        const __amdgpu_buffer_rsrc_t r2r = make_rsrc(res2 ? (const void*)res2 : (const void*)a.out,
                                                     res2 ? 0x7ffffffeu : 0u);
        uint32_t r1v[4], r2v[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            r1v[v] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r1r, (int)((epi_in[v] ? epi_r1[v] : 0u) * 2u), 0, 0);
            r2v[v] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r2r, (int)((epi_in[v] ? epi_r2[v] : 0u) * 2u), 0, 0);
        }
        f32x4 acc1[kPairRT1][NB];
#pragma unroll
        for (int rt = 0; rt < kPairRT1; ++rt)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) acc1[rt][nb] = f32x4{};
#pragma unroll
        for (int i = 0; i < KMAX; ++i) {
            if (s0 + i < s1) {  // uniform across the wave
#pragma unroll
                for (int rt = 0; rt < kPairRT1; ++rt) {
                    const h8 A = __builtin_bit_cast(h8, q[i][rt]);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        acc1[rt][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B1[i][nb], acc1[rt][nb], 0, 0, 0);
                }
            }
        }
        if constexpr (decltype(first_c)::value) load_b2();
        if (z + 1 < z1) load_rows(z + 1);  // in flight through the reductions and conv2
#pragma unroll
        for (int rt = 0; rt < kPairRT1; ++rt)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) red4[((wave * kPairRT1 + rt) * NB + nb) * 64 + lane] = acc1[rt][nb];
        __syncthreads();

        // t tile: thread (rt, nb, l) sums the 16-byte partial rows (w, rt, nb, l) over the
        // waves (consecutive lanes read consecutive rows: no bank conflicts), giving the four
        // halo pixels rt * 16 + 4 (l / 16) + v of channel 16 nb + l % 16.
#pragma unroll
        for (int j = 0; j < kIters1; ++j) {
            const int g = tid + j * 64 * NW;
            if (g >= kSums1) break;
            const int l = g & 63;
            const int nb = (g >> 6) % NB;
            const int rt = g / (NB * 64);
            f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const f32x4 t = red4[((w * kPairRT1 + rt) * NB + nb) * 64 + l];
#pragma unroll
                for (int v = 0; v < 4; ++v) sum[v] += t[v];
            }
            const int oc = nb * 16 + (l & 15);
            const float bias = bias1v[j];
            _Float16* th = reinterpret_cast<_Float16*>(tt + (oc >> 3) * kPairTStride);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int px = rt * 16 + 4 * (l >> 4) + v;
                const int hy = min(px, kPairHalo - 1) / kPairHW;
                const int iy = oy0 - 1 + hy;
                const int ix = ox0 - 1 + px - hy * kPairHW;
                const bool inside = px < kPairHalo && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
                float val = sum[v] + bias;
                if (a.act1 == 1 && val < 0.0f) val = val * a.slope;
                if (a.act1 == 2 && val < 0.0f) val = 0.0f;
                th[px * 8 + (oc & 7)] = inside ? round_f16(val) : (_Float16)0.0f;
            }
        }
        __syncthreads();

        // conv2 on the output tile, A fragments from the t tile.
        f32x4 acc2[kPairRT2][NB];
#pragma unroll
        for (int rt = 0; rt < kPairRT2; ++rt)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) acc2[rt][nb] = f32x4{};
#pragma unroll
        for (int i = 0; i < KMAX; ++i) {
            if (s0 + i < s1) {
                const int kb = 4 * (s0 + i) + quarter;
                const int tap = kb >> 3;
                const int cb = kb & 7;
                const int ky = (tap * 11) >> 5;
                const int kx = tap - ky * 3;
#pragma unroll
                for (int rt = 0; rt < kPairRT2; ++rt) {
                    const int op = rt * 16 + (lane & 15);
                    const int hpx = ((op >> 3) + ky) * kPairHW + (op & 7) + kx;
                    const h8 A = __builtin_bit_cast(h8, tt[cb * kPairTStride + hpx]);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        acc2[rt][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B2[i][nb], acc2[rt][nb], 0, 0, 0);
                }
            }
        }
        // conv1's partial sums were all read before the last barrier: reuse their LDS.
#pragma unroll
        for (int rt = 0; rt < kPairRT2; ++rt)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) red4[((wave * kPairRT2 + rt) * NB + nb) * 64 + lane] = acc2[rt][nb];
        __syncthreads();

        // Thread (nb, l) sums rows (w, nb, l) as for the t tile: output pixels
        // 4 (l / 16) + v of channel 16 nb + l % 16.
        if (epi) {
            const int l = tid & 63;
            const int nb = (tid >> 6) % NB;
            f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const f32x4 t = red4[(w * NB + nb) * 64 + l];
#pragma unroll
                for (int v = 0; v < 4; ++v) sum[v] += t[v];
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if (!epi_in[v]) continue;
                float val = sum[v] + bias2v;
                if (a.act2 == 1 && val < 0.0f) val = val * a.slope;
                if (a.act2 == 2 && val < 0.0f) val = 0.0f;
                if (res1 != nullptr) val = (float)__builtin_bit_cast(_Float16, (uint16_t)r1v[v]) + val;
                if (res2 != nullptr) {
                    const float r1 = (float)round_f16(val);
                    val = (float)__builtin_bit_cast(_Float16, (uint16_t)r2v[v]) + r1;
                }
                const uint16_t h = __builtin_bit_cast(uint16_t, round_f16(val));
                out[epi_out[v]] = h;
                if (out2 != nullptr) out2[epi_out2[v]] = h;
            }
        }
    };
    image(z0, std::true_type{});
    for (int z = z0 + 1; z < z1; ++z) {
        __syncthreads();  // sums read before the next image's partials
        image(z, std::false_type{});
    }
}

// The temporal preparation and the first conv_offset layer (196 -> 64, LeakyReLU) in one
// launch, for one image per workgroup. A workgroup owns a 2 x 8 output tile: it computes
// the 25 condition blocks [warp(feat_prop, flow1), feat_current, warp(feat_n2, flow2),
// flow1, flow2] on the tile's 4 x 10 halo straight into LDS (zero outside the image: the
// conv's padding), writes the pointwise outputs of its own 16 pixels (flow2, the DCN
// input [feat_prop, feat_n2] and the backbone input's [feat_current, prefix...] in CB8),
// then runs the conv with A fragments from LDS. The conditions are condition_block's bits
// (the separate body_temporal_kernel's), and the conv keeps conv3x3_kernel's K split over 8 waves
// (wave w owns K-steps [w * 57 / 8, (w + 1) * 57 / 8), K-block 4 s + lane / 16 = tap * 25
// + block) and its wave-ordered sum, so the output is the two-launch result bit for bit.
// The halo is 2.5 times the tile, so each workgroup samples 2.5 times the pixels it
// outputs; in exchange the 200-channel condition tensor never reaches HBM and the step
// loses a launch.
constexpr int kTcTH = 2, kTcTW = 8;
constexpr int kTcHW = kTcTW + 2;
constexpr int kTcHalo = (kTcTH + 2) * kTcHW;
constexpr int kTcBlocks = 25;  // 196 condition channels + 4 zero ones

struct TemporalConvArgs {
    const uint16_t *feat_prop, *feat_current, *feat_n2, *flow1, *prev_flow, *p0, *p1, *p2;
    uint16_t *flow2, *deform, *bb, *out;
    const void* wpk;     // conv_offset 1 B fragments [57][4][64][8]
    const float* bias;   // [64]
    uint32_t wpk_bytes, magic_cb;
    int nprefix, has_second_order, H, W, tiles_x, tiles, KB, ksteps;
    float slope;
};

// WARP_CB8: feat_prop and feat_n2 are CB8 tensors (the clip's mirrors of its propagated
// features): each warped block is four 16-byte gathers instead of 32 two-byte ones, and
// the DCN input blocks are 16-byte copies. Same bits either way.
template <int NW, int KMAX, bool WARP_CB8>
__global__ __launch_bounds__(64 * NW) void temporal_conv_kernel(TemporalConvArgs a) {
    constexpr int NB = kConvNbc;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    float* red = reinterpret_cast<float*>(lds);  // [NW][NB][4][kConvRedStride]
    u32x4* cond = reinterpret_cast<u32x4*>(lds + (size_t)NW * NB * 4 * kConvRedStride * sizeof(float));  // [25][halo]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int quarter = lane >> 4;

    const int per_xcd = (a.tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= a.tiles) return;  // whole workgroup, before any barrier
    const int ty = tile / a.tiles_x;
    const int oy0 = ty * kTcTH;
    const int ox0 = (tile - ty * a.tiles_x) * kTcTW;
    const int H = a.H, W = a.W;
    const size_t pl = (size_t)H * W;
    const int Hp = H + 2 * kPad, Wp = W + 2 * kPad;

    // This wave's weight fragments are requested after the conditions' loads: issued
    // first, their 32 KB per wave queued ahead of every flow and corner load, and each wait
    // of the sampling (which waits for everything issued before the loads it needs) also
    // waited for them.
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wpk, a.wpk_bytes);
    // 196 channels: 25 blocks x 9 taps = 225 K-blocks, 57 K-steps; a wave owns at least
    // kMinSteps of them, a count the compiler can use for its waits.
    constexpr int kSteps = (9 * kTcBlocks + 3) / 4;
    constexpr int kMinSteps = kSteps / NW;
    const int s0 = wave * kSteps / NW;
    const int s1 = (wave + 1) * kSteps / NW;
    h8 Bf[KMAX][NB];
    auto load_bf = [&]() {
#pragma unroll
        for (int i = 0; i < KMAX; ++i)
            if (i < kMinSteps || s0 + i < s1)  // uniform across the wave
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    Bf[i][nb] = __builtin_bit_cast(h8, load16(wr, (uint32_t)(((s0 + i) * NB + nb) * 64 + lane) * 16u));
    };

    uint16_t* hflow = reinterpret_cast<uint16_t*>(cond + kTcBlocks * kTcHalo);  // [halo][f1x, f1y, f2x, f2y]
    auto halo_xy = [&](int hp, int& y, int& x) {
        const int hy = hp / kTcHW;
        y = oy0 - 1 + hy;
        x = ox0 - 1 + hp - hy * kTcHW;
    };
    constexpr int kCondItems = kTcBlocks * kTcHalo;
    // The flows of the halo pixels: f1 = flow1 and f2 = flow1 + warp(prev_flow, flow1), so
    // that every condition below is one round of corner loads. Wave `fw` computes them.
    auto halo_flows = [&](int hp) {
        int y, x;
        halo_xy(hp, y, x);
        uint16_t f1[2] = {0, 0}, f2[2] = {0, 0};
        if (y >= 0 && y < H && x >= 0 && x < W) {
            const int p = y * W + x;
            f1[0] = a.flow1[p];
            f1[1] = a.flow1[pl + p];
            warp::temporal_flow2(a.flow1, a.prev_flow, a.has_second_order, H, W, y, x, f2);
        }
        hflow[hp * 4 + 0] = f1[0];
        hflow[hp * 4 + 1] = f1[1];
        hflow[hp * 4 + 2] = f2[0];
        hflow[hp * 4 + 3] = f2[1];
    };
    if constexpr (WARP_CB8) {
        // Items by load pattern, one loop per pattern with item counts that are multiples of
        // 64, so that a wave's loads follow one pattern (loads in divergent branches made
        // the compiler wait for every load in flight wherever the branches' registers
        // met). Every pattern's loads are requested before any item is finished: a loop that
        // finished each item before starting the next waited for each round's loads in
        // turn. W: the 16 warped condition blocks (four corner units each); N: the 8
        // feat_current condition blocks, then the backbone input's NCHW blocks (eight halves
        // in 32-bit registers; 128 items per source tensor, so that a wave's source pointer
        // is uniform); U: the DCN input's 16 CB8 blocks (one unit each). A pixel outside
        // the image loads a clamped pixel, and its item writes zero or nothing. N and U are
        // requested before the flows, which the last wave computes (N and U items leave it
        // idle at nprefix 0).
        constexpr int kPx = kTcTH * kTcTW;
        constexpr int kT = 64 * NW;
        constexpr int kW = 16 * kTcHalo;
        constexpr int kNc = 8 * kTcHalo;
        constexpr int kU = 16 * kPx;
        constexpr int kRW = (kW + kT - 1) / kT;
        constexpr int kRN = (kNc + 8 * 4 * kPx + kT - 1) / kT;  // nprefix <= 3
        constexpr int kRU = (kU + kT - 1) / kT;
        static_assert(kW % 64 == 0 && kNc % 64 == 0 && kU % 64 == 0 && (8 * kPx) % 64 == 0,
                      "wave-uniform item classes");
        const int nN = kNc + 8 * (1 + a.nprefix) * kPx;
        const size_t blk_units = (size_t)Hp * Wp;
        const u32x4* prop_u = reinterpret_cast<const u32x4*>(a.feat_prop);
        const u32x4* n2_u = reinterpret_cast<const u32x4*>(a.feat_n2);
        auto clamp_yx = [&](int& y, int& x) {
            y = min(max(y, 0), H - 1);
            x = min(max(x, 0), W - 1);
        };
        // N item i: condition block 8 + i / 40 at halo pixel i % 40, or, from kNc, the
        // backbone input's block (i - kNc) / 16 at tile pixel (i - kNc) % 16.
        auto n_item = [&](int i, int& y, int& x) {
            if (i < kNc) {
                halo_xy(i % kTcHalo, y, x);
            } else {
                const int op = (i - kNc) & 15;
                y = oy0 + (op >> 3);
                x = ox0 + (op & 7);
            }
        };
        uint32_t hv[kRN][8];
        u32x4 tu[kRU];
#pragma unroll
        for (int r = 0; r < kRN; ++r) {
            const int i = tid + r * kT;
            if (i < nN) {
                int y, x;
                n_item(i, y, x);
                clamp_yx(y, x);
                const uint16_t* src;
                if (i < kNc) {
                    src = a.feat_current + (size_t)(i / kTcHalo) * 8 * pl;
                } else {
                    const int which = __builtin_amdgcn_readfirstlane(i - kNc) >> 7;
                    const uint16_t* base = which == 0 ? a.feat_current : (which == 1 ? a.p0 : (which == 2 ? a.p1 : a.p2));
                    src = base + (size_t)(((i - kNc) >> 4) & 7) * 8 * pl;
                }
                src += y * W + x;
#pragma unroll
                for (int c = 0; c < 8; ++c) hv[r][c] = src[(size_t)c * pl];
            }
        }
#pragma unroll
        for (int r = 0; r < kRU; ++r) {
            const int i = tid + r * kT;
            if (i < kU) {
                const int dblock = i >> 4;
                const int op = i & 15;
                int y = oy0 + (op >> 3), x = ox0 + (op & 7);
                clamp_yx(y, x);
                tu[r] = (dblock < 8 ? prop_u : n2_u)[(size_t)(dblock & 7) * blk_units + (size_t)(y + kPad) * Wp + x + kPad];
            }
        }
        const int fw = NW - 1;
        if (tid >= fw * 64 && tid - fw * 64 < kTcHalo) halo_flows(tid - fw * 64);
        __syncthreads();

        // W item i: warped condition block (i / 40 < 8 ? i / 40 : i / 40 + 8) at halo pixel
        // i % 40, flow1 for feat_prop, flow2 for feat_n2.
        auto w_coord = [&](int i, int& blk, int& hp, int& y, int& x, float& yf, float& xf) {
            const int b16 = i / kTcHalo;
            hp = i - b16 * kTcHalo;
            blk = b16 < 8 ? b16 : b16 + 8;
            halo_xy(hp, y, x);
            const int f = b16 < 8 ? 0 : 2;
            yf = (float)y + warp::h2f(hflow[hp * 4 + f + 1]);
            xf = (float)x + warp::h2f(hflow[hp * 4 + f]);
        };
        u32x4 tw[kRW][4];
#pragma unroll
        for (int r = 0; r < kRW; ++r) {
            const int i = tid + r * kT;
            if (i < kW) {
                int blk, hp, y, x;
                float yf, xf;
                w_coord(i, blk, hp, y, x, yf, xf);
                uint32_t u[4];
                warp::cb8_corner_units(H, W, yf, xf, u);
                const u32x4* units = (blk < 8 ? prop_u : n2_u) + (size_t)(blk & 7) * blk_units;
#pragma unroll
                for (int k = 0; k < 4; ++k) tw[r][k] = units[u[k]];
            }
        }

        load_bf();  // in flight behind the corners, through the finishing of the items

        // Finish: the N and U items (their loads were issued first), then W, then the items
        // without loads (condition block 24 and flow2).
#pragma unroll
        for (int r = 0; r < kRN; ++r) {
            const int i = tid + r * kT;
            if (i < nN) {
                int y, x;
                n_item(i, y, x);
                u32x4 v;
#pragma unroll
                for (int d = 0; d < 4; ++d) v[d] = __builtin_amdgcn_perm(hv[r][2 * d + 1], hv[r][2 * d], 0x05040100u);
                if (i < kNc) {
                    const bool inside = y >= 0 && y < H && x >= 0 && x < W;
                    cond[(8 + i / kTcHalo) * kTcHalo + i % kTcHalo] = inside ? v : u32x4{0u, 0u, 0u, 0u};
                } else if (y < H && x < W) {
                    const int dblock = (i - kNc) >> 4;
                    reinterpret_cast<u32x4*>(a.bb)[((size_t)dblock * Hp + y + kPad) * Wp + x + kPad] = v;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < kRU; ++r) {
            const int i = tid + r * kT;
            if (i < kU) {
                const int dblock = i >> 4;
                const int op = i & 15;
                const int y = oy0 + (op >> 3), x = ox0 + (op & 7);
                if (y < H && x < W)
                    reinterpret_cast<u32x4*>(a.deform)[((size_t)dblock * Hp + y + kPad) * Wp + x + kPad] = tu[r];
            }
        }
#pragma unroll
        for (int r = 0; r < kRW; ++r) {
            const int i = tid + r * kT;
            if (i < kW) {
                int blk, hp, y, x;
                float yf, xf;
                w_coord(i, blk, hp, y, x, yf, xf);
                u32x4 v = {0u, 0u, 0u, 0u};
                if (y >= 0 && y < H && x >= 0 && x < W) {
                    float c8[8];
                    warp::cb8_blend(tw[r], H, W, yf, xf, c8);
#pragma unroll
                    for (int d = 0; d < 4; ++d) v[d] = warp::pack_halves(warp::f2h(c8[2 * d]), warp::f2h(c8[2 * d + 1]));
                }
                cond[blk * kTcHalo + hp] = v;
            }
        }
        if (tid < kTcHalo) {  // condition block 24: flow1 (x, y), flow2 (x, y), zero outside
            int y, x;
            halo_xy(tid, y, x);
            u32x4 v = {0u, 0u, 0u, 0u};
            if (y >= 0 && y < H && x >= 0 && x < W) {
                v[0] = warp::pack_halves(hflow[tid * 4 + 0], hflow[tid * 4 + 1]);
                v[1] = warp::pack_halves(hflow[tid * 4 + 2], hflow[tid * 4 + 3]);
            }
            cond[24 * kTcHalo + tid] = v;
        } else if (tid >= 64 && tid < 64 + kPx) {  // flow2 of the tile's pixels
            const int op = tid - 64;
            const int y = oy0 + (op >> 3), x = ox0 + (op & 7);
            if (y < H && x < W) {
                const int hp = ((op >> 3) + 1) * kTcHW + (op & 7) + 1;  // the pixel's halo slot
                a.flow2[y * W + x] = hflow[hp * 4 + 2];
                a.flow2[pl + y * W + x] = hflow[hp * 4 + 3];
            }
        }
    } else {
        if (tid < kTcHalo) halo_flows(tid);
        __syncthreads();

        // Conditions of the halo, block-major: item (block, halo pixel); then the pointwise
        // outputs of the tile's pixels: item (kind, pixel), kind 0 flow2, 1-16 the DCN input
        // blocks, then the backbone input's leading blocks. One loop, so that the loads of
        // both kinds of item are in flight together.
        const int items = kCondItems + (17 + 8 * (1 + a.nprefix)) * kTcTH * kTcTW;
        for (int it = tid; it < items; it += 64 * NW) {
            if (it < kCondItems) {
                const int blk = it / kTcHalo;
                const int hp = it - blk * kTcHalo;
                int y, x;
                halo_xy(hp, y, x);
                u32x4 v = {0u, 0u, 0u, 0u};
                if (y >= 0 && y < H && x >= 0 && x < W) {
                    const uint16_t f1[2] = {hflow[hp * 4 + 0], hflow[hp * 4 + 1]};
                    const uint16_t f2[2] = {hflow[hp * 4 + 2], hflow[hp * 4 + 3]};
                    v = warp::condition_from_flows<u32x4, WARP_CB8>(a.feat_prop, a.feat_current, a.feat_n2, H, W, blk, y, x,
                                                                     f1, f2);
                }
                cond[blk * kTcHalo + hp] = v;
                continue;
            }
            const int pt = it - kCondItems;
            const int kind = pt >> 4;
            const int op = pt & 15;
            const int y = oy0 + (op >> 3);
            const int x = ox0 + (op & 7);
            if (y >= H || x >= W) continue;
            const int p = y * W + x;
            if (kind == 0) {
                const int hp = ((op >> 3) + 1) * kTcHW + (op & 7) + 1;  // the pixel's halo slot
                a.flow2[p] = hflow[hp * 4 + 2];
                a.flow2[pl + p] = hflow[hp * 4 + 3];
                continue;
            }
            uint16_t* dst;
            int dblock;
            const uint16_t* src;
            if (kind <= 16) {
                dst = a.deform;
                dblock = kind - 1;
                src = dblock < 8 ? a.feat_prop + (size_t)dblock * 8 * pl : a.feat_n2 + (size_t)(dblock - 8) * 8 * pl;
            } else {
                dst = a.bb;
                dblock = kind - 17;
                const int which = dblock >> 3;
                const uint16_t* base = which == 0 ? a.feat_current : (which == 1 ? a.p0 : (which == 2 ? a.p1 : a.p2));
                src = base + (size_t)(dblock & 7) * 8 * pl;
            }
            reinterpret_cast<u32x4*>(dst)[((size_t)dblock * Hp + y + kPad) * Wp + x + kPad] = warp::copy8<u32x4>(src, pl, p);
        }
    }
    if constexpr (!WARP_CB8) load_bf();
    __syncthreads();

    // The conv: lane l supplies tile pixel l % 16 (row (l % 16) / 8, column l % 8).
    f32x4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{};
    const int r = lane & 15;
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
        if (i < kMinSteps || s0 + i < s1) {  // uniform across the wave
            const int kb = 4 * (s0 + i) + quarter;
            const int kbc = kb < a.KB ? kb : a.KB - 1;
            const int tap = fast_div(kbc, a.magic_cb);
            const int blk = kbc - tap * kTcBlocks;
            const int ky = (tap * 11) >> 5;  // tap / 3 for tap < 9
            const int kx = tap - ky * 3;
            const u32x4 z = {0u, 0u, 0u, 0u};
            const u32x4 q = cond[blk * kTcHalo + ((r >> 3) + ky) * kTcHW + (r & 7) + kx];
            // Padding K-blocks multiply zero weights; zero A keeps a non-finite condition
            // from turning 0 * inf into NaN there (as conv3x3_kernel).
            const h8 A = __builtin_bit_cast(h8, kb < a.KB ? q : z);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bf[i][nb], acc[nb], 0, 0, 0);
        }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[((wave * NB + nb) * 4 + v) * kConvRedStride + lane] = acc[nb][v];
    __syncthreads();

    // Channel-fastest items, as conv3x3_kernel's epilogue: conflict-free reads, whole CB8
    // units per store.
    for (int idx = tid; idx < 16 * kConvChunk; idx += 64 * NW) {
        const int ocl = idx & (kConvChunk - 1);
        const int px = idx >> 6;
        const int nb = ocl >> 4;
        const int src = ((px >> 2) << 4) + (ocl & 15);
        const int v = px & 3;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) sum += red[((w * NB + nb) * 4 + v) * kConvRedStride + src];
        const int yy = oy0 + (px >> 3);
        const int xx = ox0 + (px & 7);
        if (yy >= H || xx >= W) continue;
        float val = sum + a.bias[ocl];
        if (val < 0.0f) val = val * a.slope;  // LeakyReLU
        a.out[conv_index(kLayoutCB8, ocl, yy, xx, H, W, Hp, Wp)] = __builtin_bit_cast(uint16_t, round_f16(val));
    }
}

}  // namespace

ConvGeometry conv_geometry(int cin, int cout, int height, int width) {
    ConvGeometry g;
    g.cin = cin;
    g.cout = cout;
    g.h = height;
    g.w = width;
    g.cb = (cin + 7) / 8;
    g.kb = 9 * g.cb;
    g.ksteps = (g.kb + 3) / 4;
    g.chunks = (cout + kConvChunk - 1) / kConvChunk;
    g.nbt = g.chunks * kConvNbc;
    return g;
}

size_t conv_packed_bytes(const ConvGeometry& g) { return (size_t)g.ksteps * g.nbt * 64 * 8 * 2; }

hipError_t launch_conv_prepack(const ConvGeometry& g, const uint16_t* w, const uint16_t* bias,
                               void* wpk, float* bpk, hipStream_t stream) {
    const long total = (long)g.ksteps * g.nbt * 64 * 8;
    const long grid = (std::max<long>(total, g.cout) + 255) / 256;
    hipLaunchKernelGGL(conv_prepack_kernel, dim3((unsigned)grid), dim3(256), 0, stream, w, bias,
                       (uint16_t*)wpk, bpk, g.cin, g.cout, g.cb, g.kb, g.nbt, total);
    return hipGetLastError();
}

namespace {

// Images per workgroup of a batched conv pair or conv3x3: up to kMax, balanced over the
// workgroups of a tile. Measured for a body step over 16 tiles (images per workgroup ->
// us per step), each kernel tuned in turn: conv pair 1 -> 955, 2 -> 828, 4 -> 768,
// 8 -> 738, 16 -> 723 (over 64 tiles 16 beat 8 by 2 %); conv3x3 2 -> 685, 4 -> 667,
// 8 -> 658, 16 -> 654.
template <int kMax>
static int images_per_group(int images) {
    const int groups = (images + kMax - 1) / kMax;
    return (images + groups - 1) / groups;
}

hipError_t run_conv(const ConvGeometry& g, ConvArgs& a, const ConvBatch& batch, hipStream_t stream) {
    constexpr int NW = 8, U = 4;
    if (batch.images < 1) return hipErrorInvalidValue;
    a.xin_ts = batch.x;
    a.res1_ts = batch.res1;
    a.res2_ts = batch.res2;
    a.out_ts = batch.out;
    a.H = g.h;
    a.W = g.w;
    a.Hp = g.h + 2 * kPad;
    a.Wp = g.w + 2 * kPad;
    a.xin_bytes = (uint32_t)((size_t)g.cb * a.Hp * a.Wp * 16);
    a.wpk_bytes = (uint32_t)conv_packed_bytes(g);
    a.CB = g.cb;
    a.KB = g.kb;
    a.ksteps = g.ksteps;
    a.NBT = g.nbt;
    a.Cout = g.cout;
    a.tiles = (g.h * g.w + 15) / 16;
    a.magic_cb = magic_for(g.cb);
    const size_t lds = (size_t)NW * kConvNbc * 4 * kConvRedStride * sizeof(float);  // >= the images kernel's 65
    const int kmax = (g.ksteps + NW - 1) / NW;  // K-steps of the busiest wave
    if (batch.images > 1 && kmax <= 8) {
        const int zpw = images_per_group<16>(batch.images);
        const dim3 grid((unsigned)((a.tiles + 7) / 8 * 8), (unsigned)g.chunks,
                        (unsigned)((batch.images + zpw - 1) / zpw));
        if (kmax <= 3)
            hipLaunchKernelGGL((conv3x3_images_kernel<NW, 3>), grid, dim3(64 * NW), lds, stream, a, batch.images, zpw);
        else if (kmax <= 5)
            hipLaunchKernelGGL((conv3x3_images_kernel<NW, 5>), grid, dim3(64 * NW), lds, stream, a, batch.images, zpw);
        else
            hipLaunchKernelGGL((conv3x3_images_kernel<NW, 8>), grid, dim3(64 * NW), lds, stream, a, batch.images, zpw);
        return hipGetLastError();
    }
    // One image: a wave requests all its K-steps at once where they fit (kmax up to 8), so
    // that no wave waits for a second round of loads (128 -> 64: 4 or 5 K-steps per wave).
    const dim3 grid((unsigned)((a.tiles + 7) / 8 * 8), (unsigned)g.chunks, (unsigned)batch.images);
    if (kmax == 5)
        hipLaunchKernelGGL((conv3x3_kernel<NW, 5>), grid, dim3(64 * NW), lds, stream, a);
    else if (kmax > U && kmax <= 8)
        hipLaunchKernelGGL((conv3x3_kernel<NW, 8>), grid, dim3(64 * NW), lds, stream, a);
    else
        hipLaunchKernelGGL((conv3x3_kernel<NW, U>), grid, dim3(64 * NW), lds, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_conv3x3_offsets(const ConvGeometry& g, const void* x_cb8, const void* wpk,
                                  const float* bias, const uint16_t* flow1, const uint16_t* flow2,
                                  uint16_t* offset, uint16_t* mask, hipStream_t stream, int images) {
    if (g.cout != 432 || images < 1) return hipErrorInvalidValue;
    constexpr int NW = 8, U = 2, NB = 4, RT = 1, MINW = 6;
    ConvArgs a{};
    a.xin = x_cb8;
    a.wpk = wpk;
    a.bias = bias;
    a.offsets = 1;
    a.flow1 = flow1;
    a.flow2 = flow2;
    a.offset = offset;
    a.mask = mask;
    a.H = g.h;
    a.W = g.w;
    a.Hp = g.h + 2 * kPad;
    a.Wp = g.w + 2 * kPad;
    a.xin_bytes = (uint32_t)((size_t)g.cb * a.Hp * a.Wp * 16);
    a.wpk_bytes = (uint32_t)conv_packed_bytes(g);
    a.CB = g.cb;
    a.KB = g.kb;
    a.ksteps = g.ksteps;
    a.NBT = g.nbt;
    a.Cout = g.cout;
    a.tiles = (g.h * g.w + 16 * RT - 1) / (16 * RT);
    a.magic_cb = magic_for(g.cb);
    const long plane = (long)g.h * g.w;
    a.xin_ts = (long)g.cb * a.Hp * a.Wp * 8;
    a.flow_ts = 2 * plane;
    a.offset_ts = 288 * plane;
    a.mask_ts = 144 * plane;
    constexpr size_t lds = (size_t)NW * RT * NB * 64 * sizeof(f32x4);
    auto kernel = &conv_offsets_kernel<NW, U, NB, RT, MINW>;
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), (int)lds);
    if (attr != hipSuccess) return attr;
    const dim3 grid((unsigned)((a.tiles + 7) / 8 * 8), (unsigned)((g.cout + 16 * NB - 1) / (16 * NB)),
                    (unsigned)images);
    hipLaunchKernelGGL(kernel, grid, dim3(64 * NW), lds, stream, a);
    return hipGetLastError();
}

hipError_t launch_temporal_conv(const ConvGeometry& g, const uint16_t* feat_prop, const uint16_t* feat_current,
                                const uint16_t* feat_n2, const uint16_t* flow1, const uint16_t* prev_flow,
                                int has_second_order, const uint16_t* const* prefix, int nprefix,
                                uint16_t* flow2, uint16_t* deform_cb8, uint16_t* bb_cb8, const void* wpk,
                                const float* bias, float slope, uint16_t* out_cb8, hipStream_t stream,
                                bool warp_cb8) {
    constexpr int NW = 8, KMAX = 8;
    if (g.cin != 196 || g.cout != 64 || g.ksteps != (9 * kTcBlocks + 3) / 4 || g.ksteps > NW * KMAX || nprefix < 0 ||
        nprefix > 3)
        return hipErrorInvalidValue;
    TemporalConvArgs a{};
    a.feat_prop = feat_prop;
    a.feat_current = feat_current;
    a.feat_n2 = feat_n2;
    a.flow1 = flow1;
    a.prev_flow = prev_flow;
    const uint16_t* pre[3];
    for (int i = 0; i < 3; ++i) pre[i] = i < nprefix ? prefix[i] : feat_current;
    a.p0 = pre[0];
    a.p1 = pre[1];
    a.p2 = pre[2];
    a.flow2 = flow2;
    a.deform = deform_cb8;
    a.bb = bb_cb8;
    a.out = out_cb8;
    a.wpk = wpk;
    a.bias = bias;
    a.wpk_bytes = (uint32_t)conv_packed_bytes(g);
    a.magic_cb = magic_for(g.cb);
    a.nprefix = nprefix;
    a.has_second_order = has_second_order;
    a.H = g.h;
    a.W = g.w;
    a.tiles_x = (g.w + kTcTW - 1) / kTcTW;
    a.tiles = (g.h + kTcTH - 1) / kTcTH * a.tiles_x;
    a.KB = g.kb;
    a.ksteps = g.ksteps;
    a.slope = slope;
    const size_t lds = (size_t)NW * kConvNbc * 4 * kConvRedStride * sizeof(float) + (size_t)kTcBlocks * kTcHalo * 16 +
                       (size_t)kTcHalo * 4 * sizeof(uint16_t);
    auto kernel = warp_cb8 ? &temporal_conv_kernel<NW, KMAX, true> : &temporal_conv_kernel<NW, KMAX, false>;
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), (int)lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kernel, dim3((unsigned)((a.tiles + 7) / 8 * 8)), dim3(64 * NW), lds, stream, a);
    return hipGetLastError();
}

hipError_t launch_conv3x3(const ConvGeometry& g, const void* x_cb8, const void* wpk,
                          const float* bias, int act, float slope, const uint16_t* res1,
                          int res1_layout, const uint16_t* res2, int res2_layout, uint16_t* out,
                          int out_layout, hipStream_t stream, int res2_coff, const ConvBatch& batch) {
    ConvArgs a{};
    a.res2_coff = res2_coff;
    a.xin = x_cb8;
    a.wpk = wpk;
    a.bias = bias;
    a.res1 = res1;
    a.res2 = res2;
    a.out = out;
    a.res1_layout = res1_layout;
    a.res2_layout = res2_layout;
    a.out_layout = out_layout;
    a.act = act;
    a.slope = slope;
    return run_conv(g, a, batch, stream);
}

hipError_t launch_conv3x3_pair(const ConvGeometry& g1, const ConvGeometry& g2, const void* x_cb8,
                               const void* wpk1, const float* bias1, int act1, const void* wpk2,
                               const float* bias2, int act2, float slope, const uint16_t* res1,
                               int res1_layout, const uint16_t* res2, int res2_layout,
                               uint16_t* out, int out_layout, hipStream_t stream, int res2_coff,
                               const ConvBatch& batch, uint16_t* out2_cb8) {
    if (g1.cin != 64 || g1.cout != 64 || g2.cin != 64 || g2.cout != 64 || g1.h != g2.h ||
        g1.w != g2.w || g1.ksteps != kPairKsteps || g1.nbt != kConvNbc || batch.images < 1)
        return hipErrorInvalidValue;
    constexpr int NW = 8;
    PairArgs a{};
    a.xin = x_cb8;
    a.wpk1 = wpk1;
    a.wpk2 = wpk2;
    a.bias1 = bias1;
    a.bias2 = bias2;
    a.res1 = res1;
    a.res2 = res2;
    a.out = out;
    a.act1 = act1;
    a.act2 = act2;
    a.slope = slope;
    a.res1_layout = res1_layout;
    a.res2_layout = res2_layout;
    a.out_layout = out_layout;
    a.res2_coff = res2_coff;
    a.xin_ts = batch.x;
    a.res1_ts = batch.res1;
    a.res2_ts = batch.res2;
    a.out_ts = batch.out;
    a.out2 = out2_cb8;
    a.out2_ts = batch.out2;
    a.images = batch.images;
    a.zpw = images_per_group<16>(batch.images);
    a.H = g1.h;
    a.W = g1.w;
    a.Hp = g1.h + 2 * kPad;
    a.Wp = g1.w + 2 * kPad;
    a.xin_bytes = (uint32_t)((size_t)g1.cb * a.Hp * a.Wp * 16);
    a.wpk_bytes = (uint32_t)conv_packed_bytes(g1);
    a.tiles_x = (g1.w + kPairTW - 1) / kPairTW;
    a.tiles = (g1.h + kPairTH - 1) / kPairTH * a.tiles_x;
    constexpr size_t lds = pair_lds_bytes(NW);
    auto kernel = &conv_pair_kernel<NW>;
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), (int)lds);
    if (attr != hipSuccess) return attr;
    const unsigned groups_z = (unsigned)((batch.images + a.zpw - 1) / a.zpw);
    hipLaunchKernelGGL(kernel, dim3((unsigned)((a.tiles + 7) / 8 * 8), 1, groups_z), dim3(64 * NW), lds,
                       stream, a);
    return hipGetLastError();
}

}  // namespace dcn
