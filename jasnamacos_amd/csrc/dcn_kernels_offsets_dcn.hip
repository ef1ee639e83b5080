// The propagation body's last conv_offset layer (64 -> 432, offsets and masks) and its
// DCNv2 (128 -> 64, 3x3, 16 deformable groups) in one launch.
//
// Why: the two run back to back on the same 16-pixel tile, and the offsets of a tile are
// only ever read by the DCN of that tile. Fused, the 432 offset/mask channels stay in LDS
// (the DCN samples straight from the conv's output, with no HBM round trip), and a frame
// saves one launch and one kernel's load/reduce latency chain.
//
// Workgroup: 12 waves on one 16-pixel tile of up to four images (grid z = image group).
//  * Phase A, the offsets conv: the tile's A fragments (18 K-steps of 64 lanes per image)
//    are staged in LDS once; wave w owns 16-channel column blocks w, w + 12 (and w + 24 for
//    w < 3) of the 27 and runs every K-step for them, streaming its weight fragments and
//    applying each to every image of the group. The K range is
//    summed in conv_offsets_kernel's order: chains over the eight ranges
//    [r * 18 / 8, (r + 1) * 18 / 8) from zero, added to a zero sum in range order, so each
//    raw value, and each offset and mask after prepare_dcn_offsets_fp16
//    (MetalShader.swift:815-839), is the same bits as conv_offsets_kernel's.
//  * Phase B, the DCN, image by image with the weight fragments held in registers:
//    narrow_kernel<4, 12, 3> with the offsets and masks read from LDS (same K split, blend
//    and summation order): the aligned feature is the same bits as the two-kernel path.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

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

constexpr size_t kStageBytes = (size_t)kOffKsteps * 64 * 16;       // A fragments of an image
constexpr size_t kOffsBytes = (size_t)kOffChannels * 16 * 2;        // [432][16] FP16 per image
constexpr int kOdRedStride = 68;  // partial-sum rows of 64 lanes, padded: conflict-free channel-fastest reads
constexpr size_t kRedBytes = (size_t)kOdWaves * kDcnNb * 4 * kOdRedStride * 4;
constexpr size_t kFlowBytes = 2 * 2 * 16 * 2;                      // [flow][channel][16] FP16 per image
// From three images on, the DCN's partial sums reuse the A-fragment stage (dead by then).
__host__ __device__ constexpr bool od_red_in_stage(int images) { return images * kStageBytes >= kRedBytes; }
__host__ __device__ constexpr size_t od_lds_bytes(int images) {
    return (size_t)images * (kStageBytes + kOffsBytes + kFlowBytes) + (od_red_in_stage(images) ? 0 : kRedBytes);
}

// Bit s set when K-step s ends one of the eight K ranges of conv_offsets_kernel.
__host__ __device__ constexpr uint32_t range_ends() {
    uint32_t m = 0;
    for (int r = 0; r < kOffSplit; ++r) m |= 1u << ((r + 1) * kOffKsteps / kOffSplit - 1);
    return m;
}
constexpr uint32_t kRangeEnds = range_ends();

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
    int H, W, Hp, Wp, nbt, tiles, out_coff, out_cblk, images;
    long xoff_ts, flow_ts, xin_ts, out_ts;
};

// Workgroup (tile, zg) runs images zg * Z .. zg * Z + Z - 1 (fewer in the last group):
// phase A for all of them at once (each weight fragment applied to every image's A
// fragment), then phase B image by image with the DCN weights held in registers.
template <int SAMPLER, int Z>
__global__ __launch_bounds__(kOdThreads) void offsets_dcn_kernel(OffsetsDcnArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    u32x4* stage = reinterpret_cast<u32x4*>(lds);                                 // [Z][18][64]
    uint16_t* offs = reinterpret_cast<uint16_t*>(lds + Z * kStageBytes);         // [Z][432][16]
    constexpr bool kRedInStage = od_red_in_stage(Z);
    float* red = reinterpret_cast<float*>(kRedInStage ? lds : lds + Z * (kStageBytes + kOffsBytes));  // [12][4][4][kOdRedStride]
    uint16_t* flows = reinterpret_cast<uint16_t*>(lds + Z * (kStageBytes + kOffsBytes) +
                                                  (kRedInStage ? 0 : kRedBytes));  // [Z][2][2][16]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int quarter = lane >> 4;

    const int per_xcd = (a.tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= a.tiles) return;  // whole workgroup, before any barrier
    const long z0 = (long)blockIdx.z * Z;
    const int nimg = (int)min((long)Z, (long)a.images - z0);  // uniform, >= 1
    const int M = a.H * a.W;
    const __amdgpu_buffer_rsrc_t wor = make_rsrc(a.woff, a.woff_bytes);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wdcn, a.wdcn_bytes);

    // ---- phase A: the offsets conv on this tile ----------------------------------------
    // Column blocks of this wave.
    const int nblocks = wave < kOffBlocks - 2 * kOdWaves ? 3 : 2;
    // The DCN epilogue's biases (output channel idx / 16 of items idx = tid, tid + 768) and
    // the transform's, requested first: loads complete in order, and a bias requested late
    // costs a round trip (or waits for everything requested before it).
    constexpr int kDcnItems = 16 * kDcnNb * 16;
    constexpr int kDcnIters = (kDcnItems + kOdThreads - 1) / kOdThreads;
    float bdcnv[kDcnIters];
#pragma unroll
    for (int k = 0; k < kDcnIters; ++k) bdcnv[k] = a.bdcn[min(tid + k * kOdThreads, kDcnItems - 1) & (16 * kDcnNb - 1)];
    float boffv[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) boffv[j] = a.boff[(wave + kOdWaves * min(j, nblocks - 1)) * 16 + (lane & 15)];

    // Waves own 3 or 2 column blocks; the ring's loads and MFMAs are instantiated for each
    // count (a uniform branch picks one), so that the compiler's waits count the loads in
    // flight exactly (with a per-block condition it waited for all but one).
    h8 Bq[kOffRing][3];
    auto load_b = [&](int slot, int s, auto nbl_c) {
        constexpr int NBL = decltype(nbl_c)::value;
#pragma unroll
        for (int j = 0; j < NBL; ++j)
            Bq[slot][j] = __builtin_bit_cast(h8, load16(wor, (uint32_t)((s * a.nbt + wave + kOdWaves * j) * 64 + lane) * 16u));
    };
    typedef std::integral_constant<int, 3> Three;
    typedef std::integral_constant<int, 2> Two;
    if (nblocks == 3) {
#pragma unroll
        for (int s = 0; s < kOffRing; ++s) load_b(s, s, Three{});
    } else {
#pragma unroll
        for (int s = 0; s < kOffRing; ++s) load_b(s, s, Two{});
    }

    // The tile's flows (both flows, both channels, 16 pixels per image; a clamped pixel,
    // zeroed when written), requested before the A fragments.
    const int px_flow = tile * 16 + (tid & 15);
    uint16_t flow_v = 0;
    if (tid < nimg * 64) {  // whole waves
        const int img = tid >> 6;
        const int f = (tid >> 5) & 1;
        const int c = (tid >> 4) & 1;
        const uint16_t* flow = (f == 0 ? a.flow1 : a.flow2) + (z0 + img) * a.flow_ts;
        flow_v = flow[c * (size_t)M + min(px_flow, M - 1)];
    }
    // A fragment of K-step s, lane l: pixel l % 16 (clamped into the image), K-block
    // 4 s + l / 16 = tap * 8 + cb, as conv_offsets_kernel loads it; copied straight into
    // LDS (buffer_load ... lds: lane l's 16 bytes land at the wave's base + 16 l), so no
    // load waits for the one before it.
    for (int u0 = __builtin_amdgcn_readfirstlane(wave) * 64; u0 < nimg * kOffKsteps * 64; u0 += kOdThreads) {
        const int u = u0 + lane;
        const int img = u0 / (kOffKsteps * 64);  // wave-uniform: 64 divides an image's units
        const int r = u - img * (kOffKsteps * 64);
        const int s = r >> 6;
        const int l = r & 63;
        const __amdgpu_buffer_rsrc_t xor_ =
            make_rsrc(static_cast<const uint16_t*>(a.xoff) + (z0 + img) * a.xoff_ts, a.xoff_bytes);
        const int pc = min(tile * 16 + (l & 15), M - 1);
        const int y = pc / a.W;
        const uint32_t base = (uint32_t)(y + kPad - 1) * a.Wp + (pc - y * a.W) + kPad - 1;
        const int kb = 4 * s + (l >> 4);
        const int tap = kb >> 3;
        const int cb = kb & 7;
        const int ky = (tap * 11) >> 5;  // tap / 3 for tap < 9
        const int kx = tap - ky * 3;
        if (u < nimg * kOffKsteps * 64)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xor_, (__attribute__((address_space(3))) void*)(stage + u0),
                16, (int)((base + (uint32_t)(cb * a.Hp + ky) * a.Wp + kx) * 16u), 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies (the compiler does not track them)
    if (tid < nimg * 64) flows[tid] = px_flow < M ? flow_v : (uint16_t)0;
    __syncthreads();  // A fragments staged, flows in LDS

    f32x4 acc[Z][3], sum[Z][3];
#pragma unroll
    for (int i = 0; i < Z; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            acc[i][j] = f32x4{};
            sum[i][j] = f32x4{};
        }
    // Groups of kOffRing K-steps, one ring slot each.
    static_assert(kOffKsteps % kOffRing == 0, "whole ring groups");
    auto conv_loop = [&](auto nbl_c) {
        constexpr int NBL = decltype(nbl_c)::value;
        auto group = [&](int sg) {
#pragma unroll
            for (int slot = 0; slot < kOffRing; ++slot) {
                const int s = sg + slot;
#pragma unroll
                for (int i = 0; i < Z; ++i) {
                    if (i >= nimg) continue;
                    const h8 A = __builtin_bit_cast(h8, stage[(i * kOffKsteps + s) * 64 + lane]);
#pragma unroll
                    for (int j = 0; j < NBL; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bq[slot][j], acc[i][j], 0, 0, 0);
                }
                if (s + kOffRing < kOffKsteps) load_b(slot, s + kOffRing, nbl_c);
                if constexpr (Z == 1) __builtin_amdgcn_sched_barrier(0);
                if ((kRangeEnds >> s) & 1) {
#pragma unroll
                    for (int i = 0; i < Z; ++i)
#pragma unroll
                        for (int j = 0; j < 3; ++j) {
#pragma unroll
                            for (int v = 0; v < 4; ++v) sum[i][j][v] += acc[i][j][v];
                            acc[i][j] = f32x4{};
                        }
                }
            }
        };
        // One image: unrolled (a rolled loop's header merges the wait state of its back
        // edge and waits for every slot), a scheduling barrier per K-step keeping later
        // loads where they are. Batches stay rolled (unrolled, their accumulators spill).
        if constexpr (Z == 1) {
#pragma unroll
            for (int sg = 0; sg < kOffKsteps; sg += kOffRing) group(sg);
        } else {
#pragma unroll 1
            for (int sg = 0; sg < kOffKsteps; sg += kOffRing) group(sg);
        }
    };
    if (nblocks == 3)
        conv_loop(Three{});
    else
        conv_loop(Two{});
    // The DCN's weight fragments, requested now: they pass the texture addresser during
    // the offset transform and its barrier instead of ahead of the DCN's corner gathers.
    const int s0 = wave * kDcnPerWave;
    h8 Bf[kDcnPerWave][kDcnNb];
#pragma unroll
    for (int i = 0; i < kDcnPerWave; ++i)
#pragma unroll
        for (int nb = 0; nb < kDcnNb; ++nb)
            Bf[i][nb] = __builtin_bit_cast(h8, load16(wr, (uint32_t)(((s0 + i) * kDcnNb + nb) * 64 + lane) * 16u));

    // prepare_dcn_offsets_fp16 (MetalShader.swift:815-839) on the FP16 conv output, into
    // the LDS offsets [image][channel][pixel].
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        if (j >= nblocks) continue;
        const int oc = (wave + kOdWaves * j) * 16 + (lane & 15);
        const float bias = boffv[j];
#pragma unroll
        for (int i = 0; i < Z; ++i) {
            if (i >= nimg) continue;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int px = 4 * quarter + v;
                const float raw = (float)round_f16(sum[i][j][v] + bias);
                _Float16 r;
                if (oc < 288) {
                    // flow1 under channels < 144, flow2 above; even channels (dy) take
                    // the flow's y component (channel 1).
                    const float residue = 10.0f * tanhf(raw);
                    const int fc = ((oc % 144) & 1) == 0 ? 1 : 0;
                    const uint16_t f = flows[((i * 2 + (oc < 144 ? 0 : 1)) * 2 + fc) * 16 + px];
                    r = round_f16(residue + (float)__builtin_bit_cast(_Float16, f));
                } else {
                    r = round_f16(1.0f / (1.0f + expf(-raw)));
                }
                offs[(i * kOffChannels + oc) * 16 + px] = __builtin_bit_cast(uint16_t, r);
            }
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

    for (int img = 0; img < nimg; ++img) {
        const long z = z0 + img;
        const __amdgpu_buffer_rsrc_t xr =
            make_rsrc(static_cast<const uint16_t*>(a.xin) + z * a.xin_ts, a.xin_bytes);
        const uint16_t* io = offs + img * kOffChannels * 16;
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
            const float dy = (float)__builtin_bit_cast(_Float16, io[(2 * gt) * 16 + pl]);
            const float dx = (float)__builtin_bit_cast(_Float16, io[(2 * gt + 1) * 16 + pl]);
            const float mk = (float)__builtin_bit_cast(_Float16, io[(288 + gt) * 16 + pl]);
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
        if (img > 0) __syncthreads();  // the previous image's sums were read
#pragma unroll
        for (int nb = 0; nb < kDcnNb; ++nb)
#pragma unroll
            for (int v = 0; v < 4; ++v) red[((wave * kDcnNb + nb) * 4 + v) * kOdRedStride + lane] = dacc[nb][v];
        __syncthreads();

        uint16_t* out = a.out + z * a.out_ts;
#pragma unroll
        for (int k = 0; k < kDcnIters; ++k) {
            const int idx = tid + k * kOdThreads;
            if (idx >= kDcnItems) break;
            // Channel-fastest items (a wave's stores fill whole CB8 units): pixel pl is the
            // same for the wave, its position that of lane pl.
            const int oc = idx & (16 * kDcnNb - 1);
            const int pl = idx / (16 * kDcnNb);
            const int nb = oc >> 4;
            const int src = ((pl >> 2) << 4) + (oc & 15);
            const int v = pl & 3;
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < kOdWaves; ++w) s += red[((w * kDcnNb + nb) * 4 + v) * kOdRedStride + src];
            const int py = __shfl(oy, pl), px = __shfl(ox, pl);
            if (__shfl((int)pvalid, pl)) {
                const int c = a.out_coff + oc;
                const size_t dst =
                    ((size_t)((c >> 3) * (a.H + 2 * kPad) + py + kPad) * (a.W + 2 * kPad) + px + kPad) * 8 + (c & 7);
                out[dst] = __builtin_bit_cast(uint16_t, round_f16(s + bdcnv[k]));
            }
        }
    }
}

template <int Z>
hipError_t launch_od_t(const OffsetsDcnArgs& a, hipStream_t stream) {
    auto kernel = &offsets_dcn_kernel<kSamplerFast, Z>;
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), od_lds_bytes(Z));
    if (attr != hipSuccess) return attr;
    const dim3 grid((unsigned)((a.tiles + 7) / 8 * 8), 1, (unsigned)((a.images + Z - 1) / Z));
    hipLaunchKernelGGL(kernel, grid, dim3(kOdThreads), od_lds_bytes(Z), stream, a);
    return hipGetLastError();
}

}  // namespace

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
    a.images = images;
    // Images per workgroup: up to four (LDS 130 KB, the DCN's sums in the dead stage),
    // measured for a body step over 16 tiles: 621 us (one), 580 (two), 574 (three), 565
    // (four); over 64 tiles 2478, 2294, 2258, 2230 us.
    if (images >= 4) return launch_od_t<4>(a, stream);
    if (images >= 3) return launch_od_t<3>(a, stream);
    if (images == 2) return launch_od_t<2>(a, stream);
    return launch_od_t<1>(a, stream);
}

}  // namespace dcn
