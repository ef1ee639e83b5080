// The propagation body's last conv_offset layer (64 -> 432, offsets and masks) and its
// DCNv2 (128 -> 64, 3x3, 16 deformable groups) in one launch.
//
// Why: the two run back to back on the same 16-pixel tile, and the offsets of a tile are
// only ever read by the DCN of that tile. Fused, the 432 offset/mask channels stay in LDS
// (no HBM round trip, SURVEY's "directly in the DCN sampler from raw conv output"), and a
// frame saves one launch and one kernel's load/reduce latency chain.
//
// Workgroup: 12 waves on one 16-pixel tile of one image (grid z = image).
//  * Phase A, the offsets conv: the tile's A fragments (18 K-steps of 64 lanes) are staged
//    in LDS once; wave w owns 16-channel column blocks w, w + 12 (and w + 24 for w < 3) of
//    the 27 and runs every K-step for them, streaming its weight fragments. The K range is
//    summed in conv_offsets_kernel's order: chains over the eight ranges
//    [r * 18 / 8, (r + 1) * 18 / 8) from zero, added to a zero sum in range order, so each
//    raw value, and each offset and mask after prepare_dcn_offsets_fp16
//    (MetalShader.swift:815-839), is the same bits as conv_offsets_kernel's.
//  * Phase B, the DCN: narrow_kernel<4, 12, 3> with the offsets and masks read from LDS
//    (same K split, blend and summation order): the aligned feature is the same bits as
//    the two-kernel path.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "dcn_device.hpp"
#include "dcn_internal.hpp"

#pragma clang fp contract(off)

namespace dcn {
namespace {

using namespace dev;

constexpr int kOdWaves = 12;
constexpr int kOdThreads = 64 * kOdWaves;
constexpr int kOffChannels = 432;
constexpr int kOffBlocks = kOffChannels / 16;  // 27 column blocks of the offsets conv
constexpr int kOffKsteps = 18;                 // 64 channels x 9 taps / 32
constexpr int kOffSplit = 8;                   // conv_offsets_kernel's K split (sum order)
constexpr int kOffRing = 3;                    // weight K-steps in flight per wave
constexpr int kDcnKsteps = 36;                 // 128 channels x 9 taps / 32
constexpr int kDcnNb = 4;                      // 64 output channels
constexpr int kDcnPerWave = kDcnKsteps / kOdWaves;

constexpr size_t kStageBytes = (size_t)kOffKsteps * 64 * 16;       // A fragments
constexpr size_t kOffsBytes = (size_t)kOffChannels * 16 * 2;        // [432][16] FP16
constexpr size_t kRedBytes = (size_t)kOdWaves * kDcnNb * 4 * 65 * 4;  // narrow_kernel's sums
constexpr size_t kOdLds = kStageBytes + kOffsBytes + kRedBytes;

// True when K-step s ends one of the eight K ranges of conv_offsets_kernel.
__host__ __device__ constexpr bool range_end(int s) {
    for (int r = 0; r < kOffSplit; ++r)
        if ((r + 1) * kOffKsteps / kOffSplit - 1 == s) return true;
    return false;
}

struct OffsetsDcnArgs {
    const void* xoff;       // CB8 offset-branch features (64 channels), per image xoff_ts
    const void* woff;       // conv_prepack_kernel layout [18][nbt][64][8]
    const float* boff;      // [432]
    const uint16_t* flow1;  // [2][H][W] (x, y), per image flow_ts
    const uint16_t* flow2;
    const void* xin;        // CB8 DCN input (128 channels), per image xin_ts
    const void* wdcn;       // prepack_kernel layout [36][4][64][8] (16-wide column groups)
    const float* bdcn;      // [64]
    uint16_t* out;          // CB8 backbone input, per image out_ts
    uint32_t xoff_bytes, woff_bytes, xin_bytes, wdcn_bytes;
    int H, W, Hp, Wp, nbt, tiles, out_coff, out_cblk;
    long xoff_ts, flow_ts, xin_ts, out_ts;
};

template <int SAMPLER>
__global__ __launch_bounds__(kOdThreads) void offsets_dcn_kernel(OffsetsDcnArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    u32x4* stage = reinterpret_cast<u32x4*>(lds);                          // [18][64]
    uint16_t* offs = reinterpret_cast<uint16_t*>(lds + kStageBytes);      // [432][16]
    float* red = reinterpret_cast<float*>(lds + kStageBytes + kOffsBytes);  // [12][4][4][65]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int quarter = lane >> 4;

    const int per_xcd = (a.tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= a.tiles) return;  // whole workgroup, before any barrier
    const long z = blockIdx.z;
    const int M = a.H * a.W;

    const __amdgpu_buffer_rsrc_t xor_ =
        make_rsrc(static_cast<const uint16_t*>(a.xoff) + z * a.xoff_ts, a.xoff_bytes);
    const __amdgpu_buffer_rsrc_t wor = make_rsrc(a.woff, a.woff_bytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(static_cast<const uint16_t*>(a.xin) + z * a.xin_ts, a.xin_bytes);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wdcn, a.wdcn_bytes);
    const uint16_t* flow1 = a.flow1 + z * a.flow_ts;
    const uint16_t* flow2 = a.flow2 + z * a.flow_ts;

    // ---- phase A: the offsets conv on this tile ----------------------------------------
    // A fragment of K-step s, lane l: pixel l % 16 (clamped into the image), K-block
    // 4 s + l / 16 = tap * 8 + cb, as conv_offsets_kernel loads it.
    for (int u = tid; u < kOffKsteps * 64; u += kOdThreads) {
        const int s = u >> 6;
        const int l = u & 63;
        const int pc = min(tile * 16 + (l & 15), M - 1);
        const int y = pc / a.W;
        const uint32_t base = (uint32_t)(y + kPad - 1) * a.Wp + (pc - y * a.W) + kPad - 1;
        const int kb = 4 * s + (l >> 4);
        const int tap = kb >> 3;
        const int cb = kb & 7;
        const int ky = (tap * 11) >> 5;  // tap / 3 for tap < 9
        const int kx = tap - ky * 3;
        stage[u] = load16(xor_, (base + (uint32_t)(cb * a.Hp + ky) * a.Wp + kx) * 16u);
    }

    // Column blocks of this wave, and the flow under each of its outputs (pixel
    // 4 (l / 16) + v of the tile, channel 16 nb + l % 16), requested up front.
    const int nblocks = wave < kOffBlocks - 2 * kOdWaves ? 3 : 2;
    uint16_t fl[3][4];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int oc = (wave + kOdWaves * j) * 16 + (lane & 15);
        const uint16_t* flow = oc < 144 ? flow1 : flow2;
        const int channel = ((oc % 144) & 1) == 0 ? 1 : 0;  // even = dy = flow y
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int px = tile * 16 + 4 * quarter + v;
            fl[j][v] = (j < nblocks && oc < 288 && px < M) ? flow[channel * (size_t)M + px] : (uint16_t)0;
        }
    }

    h8 Bq[kOffRing][3];
    auto load_b = [&](int slot, int s) {
#pragma unroll
        for (int j = 0; j < 3; ++j)
            if (j < nblocks)
                Bq[slot][j] = __builtin_bit_cast(
                    h8, load16(wor, (uint32_t)((s * a.nbt + wave + kOdWaves * j) * 64 + lane) * 16u));
    };
#pragma unroll
    for (int s = 0; s < kOffRing; ++s) load_b(s, s);
    __syncthreads();  // A fragments staged

    f32x4 acc[3], sum[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        acc[j] = f32x4{};
        sum[j] = f32x4{};
    }
#pragma unroll
    for (int s = 0; s < kOffKsteps; ++s) {
        const h8 A = __builtin_bit_cast(h8, stage[s * 64 + lane]);
        const int slot = s % kOffRing;
#pragma unroll
        for (int j = 0; j < 3; ++j)
            if (j < nblocks) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bq[slot][j], acc[j], 0, 0, 0);
        if (s + kOffRing < kOffKsteps) load_b(slot, s + kOffRing);
        if (range_end(s)) {
#pragma unroll
            for (int j = 0; j < 3; ++j) {
#pragma unroll
                for (int v = 0; v < 4; ++v) sum[j][v] += acc[j][v];
                acc[j] = f32x4{};
            }
        }
    }
    // prepare_dcn_offsets_fp16 (MetalShader.swift:815-839) on the FP16 conv output, into
    // the LDS offsets [channel][pixel].
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        if (j >= nblocks) continue;
        const int oc = (wave + kOdWaves * j) * 16 + (lane & 15);
        const float bias = a.boff[oc];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int px = 4 * quarter + v;
            const float raw = (float)round_f16(sum[j][v] + bias);
            _Float16 r;
            if (oc < 288) {
                const float residue = 10.0f * tanhf(raw);
                r = round_f16(residue + (float)__builtin_bit_cast(_Float16, fl[j][v]));
            } else {
                r = round_f16(1.0f / (1.0f + expf(-raw)));
            }
            offs[oc * 16 + px] = __builtin_bit_cast(uint16_t, r);
        }
    }
    __syncthreads();  // offsets and masks of the tile complete

    // ---- phase B: the DCN (narrow_kernel<4, 12, 3> with offsets from LDS) ---------------
    const int p = tile * 16 + (lane & 15);
    const bool pvalid = p < M;
    const int sp = pvalid ? p : M - 1;
    const int oy = sp / a.W;
    const int ox = sp - oy * a.W;
    const int base_y = oy - 1;  // stride 1, pad 1
    const int base_x = ox - 1;
    const uint32_t xinb = (uint32_t)kPad * a.Wp + kPad;  // 16-byte units, border shift

    const int s0 = wave * kDcnPerWave;
    h8 Bf[kDcnPerWave][kDcnNb];
#pragma unroll
    for (int i = 0; i < kDcnPerWave; ++i)
#pragma unroll
        for (int nb = 0; nb < kDcnNb; ++nb)
            Bf[i][nb] = __builtin_bit_cast(h8, load16(wr, (uint32_t)(((s0 + i) * kDcnNb + nb) * 64 + lane) * 16u));
    u32x4 q[kDcnPerWave][4];
    float ly[kDcnPerWave], lx[kDcnPerWave], m[kDcnPerWave];
#pragma unroll
    for (int i = 0; i < kDcnPerWave; ++i) {
        const int gt = 4 * (s0 + i) + quarter;  // K-block = g * 9 + tap (8 channels per group)
        const int g = (gt * 57) >> 9;           // gt / 9 for gt < 144
        const int tap = gt - g * 9;
        const int ky = (tap * 11) >> 5;
        const int kx = tap - ky * 3;
        const int pl = lane & 15;
        const float dy = (float)__builtin_bit_cast(_Float16, offs[(2 * gt) * 16 + pl]);
        const float dx = (float)__builtin_bit_cast(_Float16, offs[(2 * gt + 1) * 16 + pl]);
        const float mk = (float)__builtin_bit_cast(_Float16, offs[(288 + gt) * 16 + pl]);
        // y = float(oy*sh - ph + ky*dh) + dy, as MetalShader.swift:327-332. Dead lanes
        // (tile tail) sample the zero border with weight 0.
        const float y = pvalid ? (float)(base_y + ky) + dy : -16.0f;
        const float x = pvalid ? (float)(base_x + kx) + dx : -16.0f;
        m[i] = pvalid ? mk : 0.0f;
        const float fy = floorf(y);
        const float fx = floorf(x);
        ly[i] = y - fy;
        lx[i] = x - fx;
        const int iy = (int)fminf(fmaxf(fy, (float)-kPad), (float)a.H);
        const int ix = (int)fminf(fmaxf(fx, (float)-kPad), (float)a.W);
        const uint32_t uu = xinb + (uint32_t)(g * a.Hp + iy) * a.Wp + ix;
        q[i][0] = load16(xr, uu * 16u);
        q[i][1] = load16(xr, uu * 16u + 16u);
        q[i][2] = load16(xr, (uu + a.Wp) * 16u);
        q[i][3] = load16(xr, (uu + a.Wp) * 16u + 16u);
    }
    f32x4 dacc[kDcnNb];
#pragma unroll
    for (int nb = 0; nb < kDcnNb; ++nb) dacc[nb] = f32x4{};
#pragma unroll
    for (int i = 0; i < kDcnPerWave; ++i) {
        const h8 A = blend<SAMPLER>(q[i][0], q[i][1], q[i][2], q[i][3], ly[i], lx[i], m[i]);
#pragma unroll
        for (int nb = 0; nb < kDcnNb; ++nb)
            dacc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bf[i][nb], dacc[nb], 0, 0, 0);
    }
#pragma unroll
    for (int nb = 0; nb < kDcnNb; ++nb)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[((wave * kDcnNb + nb) * 4 + v) * 65 + lane] = dacc[nb][v];
    __syncthreads();

    uint16_t* out = a.out + z * a.out_ts;
    for (int idx = tid; idx < 16 * kDcnNb * 16; idx += kOdThreads) {
        const int pl = idx & 15;
        const int oc = idx >> 4;
        const int nb = oc >> 4;
        const int src = ((pl >> 2) << 4) + (oc & 15);
        const int v = pl & 3;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kOdWaves; ++w) s += red[((w * kDcnNb + nb) * 4 + v) * 65 + src];
        if (pvalid) {  // pl == lane % 16: this lane's pixel
            const int c = a.out_coff + oc;
            const size_t dst = ((size_t)((c >> 3) * (a.H + 2 * kPad) + oy + kPad) * (a.W + 2 * kPad) + ox + kPad) * 8 +
                               (c & 7);
            out[dst] = __builtin_bit_cast(uint16_t, round_f16(s + a.bdcn[oc]));
        }
    }
}

}  // namespace

size_t offsets_dcn_lds_bytes() { return kOdLds; }

hipError_t launch_offsets_dcn(const ConvGeometry& goff, const void* xoff_cb8, const void* woff,
                              const float* boff, const uint16_t* flow1, const uint16_t* flow2,
                              const void* xin_cb8, const void* wdcn, size_t wdcn_bytes,
                              const float* bdcn, uint16_t* out_cb8, int out_coff, int out_cblk,
                              int images, hipStream_t stream) {
    if (goff.cin != 64 || goff.cout != kOffChannels || goff.ksteps != kOffKsteps || images < 1 ||
        wdcn_bytes != (size_t)kDcnKsteps * kDcnNb * 64 * 16)
        return hipErrorInvalidValue;
    OffsetsDcnArgs a{};
    a.xoff = xoff_cb8;
    a.woff = woff;
    a.boff = boff;
    a.flow1 = flow1;
    a.flow2 = flow2;
    a.xin = xin_cb8;
    a.wdcn = wdcn;
    a.bdcn = bdcn;
    a.out = out_cb8;
    a.H = goff.h;
    a.W = goff.w;
    a.Hp = goff.h + 2 * kPad;
    a.Wp = goff.w + 2 * kPad;
    a.nbt = goff.nbt;
    a.tiles = (goff.h * goff.w + 15) / 16;
    a.out_coff = out_coff;
    a.out_cblk = out_cblk;
    const long unit = (long)a.Hp * a.Wp * 8;  // elements of one 8-channel CB8 block
    a.xoff_ts = 8 * unit;
    a.xin_ts = 16 * unit;
    a.out_ts = (long)out_cblk * unit;
    a.flow_ts = 2L * goff.h * goff.w;
    a.xoff_bytes = (uint32_t)(a.xoff_ts * 2);
    a.xin_bytes = (uint32_t)(a.xin_ts * 2);
    a.woff_bytes = (uint32_t)conv_packed_bytes(goff);
    a.wdcn_bytes = (uint32_t)wdcn_bytes;
    auto kernel = &offsets_dcn_kernel<kSamplerFast>;
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), (int)kOdLds);
    if (attr != hipSuccess) return attr;
    const dim3 grid((unsigned)((a.tiles + 7) / 8 * 8), 1, (unsigned)images);
    hipLaunchKernelGGL(kernel, grid, dim3(kOdThreads), kOdLds, stream, a);
    return hipGetLastError();
}

}  // namespace dcn
