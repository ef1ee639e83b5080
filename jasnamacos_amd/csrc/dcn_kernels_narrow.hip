// Narrow-tile fused FP16 DCNv2 for gfx950: small problems (one 64x64 map is 4096
// output pixels).
//
// Why: every gather corner and every weight fragment of the fused kernels passes
// through the vector L1 of the CU that runs the workgroup. Per workgroup that is
// (tile pixels x K-blocks x 64 B) of corners plus the whole packed weight matrix
// (147 KB at 128 -> 64, 3x3). With 32-pixel tiles a 64x64 map has 128 workgroups:
// half the CUs idle and 442 KB through each busy L1. 16-pixel tiles put one
// workgroup on each of the 256 CUs with 295 KB each.
//
// MFMA: v_mfma_f32_16x16x32_f16. Lane l supplies A row l%16 with K elements
// 8*(l/16) .. +7, and B column l%16 with the same K elements; output element v of
// lane l is row 4*(l/16) + v, column l%16. K-step s covers K-blocks 4s .. 4s+3 (a
// K-block is 8 channels of one offset group and tap, as in the other fused kernels),
// so lane l samples K-block 4s + l/16 for pixel l%16: one bilinear coordinate, four
// 16-byte corners of the CB8 input. prepack_kernel with 16-wide column groups writes
// the weights in the same order.
//
// Workgroup: NW waves split the K-steps; every wave covers all 16 pixels and all Cout
// columns. A wave issues all loads of U K-steps (weight fragments, offsets and mask,
// then corners) before the first blend, so its critical path is two dependent memory
// round trips rather than one per K-step. Partial sums meet in LDS; the epilogue adds
// the bias, rounds to FP16 and stores 16 consecutive pixels per output channel.
// Tiles are ordered so that the workgroups of one XCD cover consecutive pixels.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "dcn_device.hpp"
#include "dcn_internal.hpp"

#pragma clang fp contract(off)

namespace dcn {
namespace {

using namespace dev;

struct NarrowArgs {
    const void* xin;       // CB8 input [B][CBLK][Hp][Wp][8]
    const uint16_t* off;   // [B][2*G*KA][HWo]
    const uint16_t* msk;   // [B][G*KA][HWo]
    const void* wpk;       // [ksteps][NB][64][8] FP16, 16-wide column groups
    const float* bias;     // [Cout]
    uint16_t* out;         // [B][Cout][HWo]
    uint32_t xin_bytes, off_bytes, msk_bytes, wpk_bytes;
    int H, W, Ho, Wo, HWo, KW, KA, ph, pw, sh, sw, dh, dw;
    int GKA, CB, CBLK, Hp, Wp, KB, ksteps, M, Cout, tiles;  // GKA = G * KA
    uint32_t magic_cb, magic_ka, magic_kw;  // fast_div constants for CB, KA, KW
    // Output placement: NCHW [B][Cout][HWo], or channels out_coff.. of a CB8 tensor with
    // out_cblk 8-channel blocks per image ([B][out_cblk][Ho+4][Wo+4][8]).
    int out_cb8, out_coff, out_cblk;
    // Rows above and below the sampled band that the L2 warm-up loads (0: no warm-up).
    int pf_halo;
};

// L2 warm-up of narrow_kernel. The CB8 input is usually fresh (written by the repack or by
// its producer just before this launch) and in no XCD's L2, so each XCD fetches the lines
// its corner gathers touch over the fabric (measured: 1.4 us of the 10.5 us C2 call). The
// workgroups of one XCD hold consecutive tiles, i.e. a band of output rows of one image;
// their waves together copy the input rows that band samples (receptive field plus
// pf_halo rows each side, every channel block) to a 1 KB slot of LDS that nothing reads:
// exactly two LDS-DMA instructions of 1 KB per wave (chunks past the band, and units
// past the buffer, read nothing: buffer bounds). A fixed count keeps the compiler's wait
// counts exact. Issued after the wave's offset loads and before its corner gathers:
// loads complete in issue order, so earlier they would delay the offsets.
constexpr int kNarrowWarmLoads = 2;  // LDS-DMA instructions per wave

template <int NW, int LOADS>
__device__ __forceinline__ void warm_band(const NarrowArgs& a, __amdgpu_buffer_rsrc_t xr, int per_xcd,
                                          int wave, int lane, uint8_t* slot) {
    const int t_lo = (blockIdx.x & 7) * per_xcd;
    const int t_hi = min(t_lo + per_xcd, a.tiles) - 1;
    const int p_lo = t_lo * 16;
    const int p_hi = min(t_hi * 16 + 15, a.M - 1);
    const int img = p_lo / a.HWo;
    if (img != p_hi / a.HWo) return;  // a band across two images: no warm-up
    const int kh = a.KA / a.KW;
    const int r0 = max((p_lo - img * a.HWo) / a.Wo * a.sh - a.ph - a.pf_halo + kPad, 0);
    const int r1 = min((p_hi - img * a.HWo) / a.Wo * a.sh - a.ph + (kh - 1) * a.dh + a.pf_halo + kPad + 1,
                       a.Hp - 1);
    const uint32_t run = (uint32_t)max(r1 - r0 + 1, 0) * a.Wp;  // 16-byte units per channel block
    const uint32_t per_block = (run + 63) / 64;                 // 1 KB chunks per channel block
    const uint32_t chunks = per_block * a.CBLK;
    const uint32_t j0 = (uint32_t)(blockIdx.x >> 3) * NW + (uint32_t)__builtin_amdgcn_readfirstlane(wave);
    const uint32_t step = (uint32_t)(t_hi - t_lo + 1) * NW;  // waves on this XCD
#pragma unroll
    for (int t = 0; t < LOADS; ++t) {
        const uint32_t j = j0 + t * step;
        const uint32_t jc = j < chunks ? j : 0;
        const uint32_t c = jc / per_block;
        const uint32_t unit = ((uint32_t)(img * a.CBLK + c) * a.Hp + r0) * a.Wp + (jc - c * per_block) * 64 + lane;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*)slot, 16,
                                                 (int)(j < chunks ? unit * 16u : 0xFFFFFFF0u), 0, 0, 0);
    }
}

template <int NB, int NW, int U, int SAMPLER>
__global__ __launch_bounds__(64 * NW) void narrow_kernel(NarrowArgs a) {
    // BF16 storage (kSamplerBf16): offsets, masks, input and weights are BF16 bits, the
    // samples are the exact sampler's FP32 bilinear rounded once to BF16, the products
    // run on the BF16 MFMA, the output is bf16(sum + bias).
    constexpr bool kBf16 = SAMPLER == kSamplerBf16;
    extern __shared__ __attribute__((aligned(16))) float red[];  // [NW][NB][64] f32x4, 1 KB slot
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int quarter = lane >> 4;

    const int per_xcd = (a.tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= a.tiles) return;  // whole workgroup, before any barrier

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xin, a.xin_bytes);
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.off, a.off_bytes);
    const __amdgpu_buffer_rsrc_t mr = make_rsrc(a.msk, a.msk_bytes);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wpk, a.wpk_bytes);

    // Pixel of this lane (and of every epilogue element it stores: the epilogue stride is
    // a multiple of 16). The tile's first pixel is split on the scalar unit; the lane's
    // 0..15 step is carried across rows and images without a per-lane division. Lanes
    // past the last pixel take the last pixel (their results are never stored).
    const int p0 = tile * 16;
    const bool pvalid = p0 + (lane & 15) < a.M;
    const int step = pvalid ? (lane & 15) : (a.M - 1 - p0);
    int b = p0 / a.HWo;
    const int sp0 = p0 - b * a.HWo;
    int oy = sp0 / a.Wo;
    int ox = sp0 - oy * a.Wo + step;
    while (ox >= a.Wo) {  // at most 15 / Wo + 1 steps
        ox -= a.Wo;
        if (++oy == a.Ho) {
            oy = 0;
            ++b;
        }
    }
    const int sp = oy * a.Wo + ox;
    const int base_y = oy * a.sh - a.ph;
    const int base_x = ox * a.sw - a.pw;
    const uint32_t offb = (uint32_t)(b * 2 * a.GKA) * a.HWo + sp;
    const uint32_t mskb = (uint32_t)(b * a.GKA) * a.HWo + sp;
    // 16-byte units; includes the border shift so (iy, ix) may be negative down to -2.
    const uint32_t xinb = (uint32_t)(b * a.CBLK * a.Hp + kPad) * a.Wp + kPad;
    // This pixel's place in an output plane (NCHW) or CB8 channel block.
    const uint32_t pix_out = a.out_cb8 ? (uint32_t)(((oy + kPad) * (a.Wo + 2 * kPad) + ox + kPad) * 8)
                                       : (uint32_t)sp;

    f32x4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{};

    const int s0 = wave * a.ksteps / NW;
    const int s1 = (wave + 1) * a.ksteps / NW;
    for (int sb = s0; sb < s1; sb += U) {
        h8 Bf[U][NB];
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int s = sb + i < s1 ? sb + i : s1 - 1;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                Bf[i][nb] = __builtin_bit_cast(h8, load16(wr, (uint32_t)((s * NB + nb) * 64 + lane) * 16u));
        }
        float dy[U], dx[U], m[U];
        int plane[U], yb[U], xb[U];
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int kb = 4 * (sb + i) + quarter;
            const int kbc = kb < a.KB ? kb : a.KB - 1;
            const int gt = fast_div(kbc, a.magic_cb);  // g * KA + tap
            const int cb = kbc - gt * a.CB;
            const int g = fast_div(gt, a.magic_ka);
            const int tap = gt - g * a.KA;
            const int ky = fast_div(tap, a.magic_kw);
            const int kx = tap - ky * a.KW;
            plane[i] = g * a.CB + cb;
            yb[i] = base_y + ky * a.dh;
            xb[i] = base_x + kx * a.dw;
            const uint32_t dyo = (offb + (uint32_t)(2 * gt) * a.HWo) * 2u;
            const uint32_t dxo = (offb + (uint32_t)(2 * gt + 1) * a.HWo) * 2u;
            const uint32_t mo = (mskb + (uint32_t)gt * a.HWo) * 2u;
            dy[i] = kBf16 ? load_bf16(orr, dyo) : load_half(orr, dyo);
            dx[i] = kBf16 ? load_bf16(orr, dxo) : load_half(orr, dxo);
            m[i] = kBf16 ? load_bf16(mr, mo) : load_half(mr, mo);
        }
        if constexpr (SAMPLER == kSamplerFast) {
            // (C2 call 10.3 -> 10.1 us with halo 16 and two loads per wave; halo 12 or 20
            // and three loads per wave measured slower. The exact sampler loses 0.6 us
            // with it.)
            if (sb == s0 && a.pf_halo > 0)
                warm_band<NW, kNarrowWarmLoads>(a, xr, per_xcd, wave, lane,
                                                reinterpret_cast<uint8_t*>(red) + NW * NB * 64 * 16);
        }
        u32x4 q[U][4];
        float ly[U], lx[U];
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int kb = 4 * (sb + i) + quarter;
            const bool live = pvalid && sb + i < s1 && kb < a.KB;
            // y = float(oy*sh - ph + ky*dh) + dy, as MetalShader.swift:327-332. Dead
            // units (tile tail, K padding) sample the zero border with weight 0.
            const float y = live ? (float)yb[i] + dy[i] : -16.0f;
            const float x = live ? (float)xb[i] + dx[i] : -16.0f;
            m[i] = live ? m[i] : 0.0f;
            const float fy = floorf(y);
            const float fx = floorf(x);
            ly[i] = y - fy;
            lx[i] = x - fx;
            const int iy = (int)fminf(fmaxf(fy, (float)-kPad), (float)a.H);
            const int ix = (int)fminf(fmaxf(fx, (float)-kPad), (float)a.W);
            const uint32_t u = xinb + (uint32_t)(plane[i] * a.Hp + iy) * a.Wp + ix;
            q[i][0] = load16(xr, u * 16u);
            q[i][1] = load16(xr, u * 16u + 16u);
            q[i][2] = load16(xr, (u + a.Wp) * 16u);
            q[i][3] = load16(xr, (u + a.Wp) * 16u + 16u);
        }
        // Every corner of the U K-steps is requested before the first blend: left alone,
        // the scheduler issues the first K-step's corners, waits for them and multiplies
        // before it requests the rest, a second gather round trip per wave.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < U; ++i) {
            if (sb + i < s1) {  // uniform across the wave
                const h8 A = blend<SAMPLER>(q[i][0], q[i][1], q[i][2], q[i][3], ly[i], lx[i], m[i]);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    if constexpr (kBf16)
                        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf8, A), __builtin_bit_cast(bf8, Bf[i][nb]), acc[nb], 0, 0, 0);
                    else
                        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bf[i][nb], acc[nb], 0, 0, 0);
                }
            }
        }
    }

    // Cross-wave sum: each wave's MFMA rows go to LDS as f32x4 rows [NW][NB][64]; lane l of
    // wave nb (mod NW) adds rows (w, nb, l) over the waves in wave order (consecutive
    // lanes read consecutive 16-byte rows: no bank conflicts), giving pixels 4 (l / 16) + v
    // of channel 16 nb + l % 16, whose output positions come from the lanes owning them.
    f32x4* red4 = reinterpret_cast<f32x4*>(red);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) red4[(wave * NB + nb) * 64 + lane] = acc[nb];
    __syncthreads();
    for (int nb = wave; nb < NB; nb += NW) {  // uniform per wave
        const int oc = nb * 16 + (lane & 15);
        f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const f32x4 t = red4[(w * NB + nb) * 64 + lane];
#pragma unroll
            for (int v = 0; v < 4; ++v) sum[v] += t[v];
        }
        const float bias = a.bias[oc];
        const int c = a.out_coff + oc;
        const size_t plane_cb8 = (size_t)(a.Ho + 2 * kPad) * (a.Wo + 2 * kPad) * 8;
        auto bits = [&](float x) -> uint32_t {
            return kBf16 ? round_bf16_bits(x) : __builtin_bit_cast(uint16_t, round_f16(x));
        };
        if (!a.out_cb8 && a.HWo % 16 == 0 && ((uintptr_t)a.out & 7) == 0) {
            // NCHW planes of a multiple of 16 pixels: every tile is whole and inside one
            // image, so the lane's four pixels are consecutive in the plane (8-byte aligned
            // on an 8-byte aligned output): one 8-byte store. Pixel pe of the tile is pixel
            // sp0 + pe of image p0 / HWo.
            const int pe = 4 * (lane >> 4);
            const uint32_t pix = (uint32_t)(sp0 + pe);
            const int pb = p0 / a.HWo;
            uint2 w;
            w.x = bits(sum[0] + bias) | (bits(sum[1] + bias) << 16);
            w.y = bits(sum[2] + bias) | (bits(sum[3] + bias) << 16);
            *reinterpret_cast<uint2*>(a.out + ((size_t)pb * a.Cout + oc) * a.HWo + pix) = w;
            continue;
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int pe = 4 * (lane >> 4) + v;  // owned by lane pe
            const uint32_t pix = (uint32_t)__shfl((int)pix_out, pe);
            const int pb = __shfl(b, pe);
            if (p0 + pe < a.M) {
                const size_t dst = a.out_cb8 ? ((size_t)pb * a.out_cblk + (c >> 3)) * plane_cb8 + pix + (c & 7)
                                             : ((size_t)pb * a.Cout + oc) * a.HWo + pix;
                a.out[dst] = kBf16 ? round_bf16_bits(sum[v] + bias)
                                   : __builtin_bit_cast(uint16_t, round_f16(sum[v] + bias));
            }
        }
    }
}

// narrow_kernel for a batch of images (the propagation body over many tiles): workgroup
// (tile, z) runs the same 16 pixels of images z * zpw .. z * zpw + zpw - 1 one after
// another (tiles never span images here). Each wave keeps the weight fragments of its K
// range (at most KMAX K-steps) in registers for all of them, and while image z is
// reduced the corners of image z + 1 and the offsets of image z + 2 are in flight. Same
// K split, blend and summation order as narrow_kernel: every image's results are the
// same bits.
template <int NB, int NW, int KMAX, int SAMPLER>
__global__ __launch_bounds__(64 * NW) void narrow_images_kernel(NarrowArgs a, int images, int zpw) {
    extern __shared__ float red[];  // [NW][NB][4][65]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int quarter = lane >> 4;

    const int per_xcd = (a.tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= a.tiles) return;  // whole workgroup, before any barrier
    const int z0 = blockIdx.z * zpw;
    const int z1 = min(z0 + zpw, images);

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xin, a.xin_bytes);
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.off, a.off_bytes);
    const __amdgpu_buffer_rsrc_t mr = make_rsrc(a.msk, a.msk_bytes);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wpk, a.wpk_bytes);

    // Pixel of this lane within its image; lanes past the last pixel take the last one
    // (their results are never stored).
    const int p = tile * 16 + (lane & 15);
    const bool pvalid = p < a.HWo;
    const int sp = pvalid ? p : a.HWo - 1;
    const int oy = sp / a.Wo;
    const int ox = sp - oy * a.Wo;
    const int base_y = oy * a.sh - a.ph;
    const int base_x = ox * a.sw - a.pw;

    const int s0 = wave * a.ksteps / NW;
    const int s1 = (wave + 1) * a.ksteps / NW;
    h8 Bf[KMAX][NB];
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
        const int s = s0 + i < s1 ? s0 + i : s1 - 1;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            Bf[i][nb] = __builtin_bit_cast(h8, load16(wr, (uint32_t)((s * NB + nb) * 64 + lane) * 16u));
    }
    // K-block of slot i -> (g * KA + tap, input plane, ky, kx); recomputed per use rather
    // than kept live across the image loop (the weight fragments take the registers).
    auto kblock = [&](int i, int& gt, int& plane, int& ky, int& kx) {
        const int kb = 4 * (s0 + i) + quarter;
        const int kbc = kb < a.KB ? kb : a.KB - 1;
        gt = fast_div(kbc, a.magic_cb);
        const int cb = kbc - gt * a.CB;
        const int g = fast_div(gt, a.magic_ka);
        const int tap = gt - g * a.KA;
        ky = fast_div(tap, a.magic_kw);
        kx = tap - ky * a.KW;
        plane = g * a.CB + cb;
    };

    float dy[KMAX], dx[KMAX], m[KMAX];
    auto load_raw = [&](int b) {
        const uint32_t offb = (uint32_t)(b * 2 * a.GKA) * a.HWo + sp;
        const uint32_t mskb = (uint32_t)(b * a.GKA) * a.HWo + sp;
#pragma unroll
        for (int i = 0; i < KMAX; ++i) {
            int gt, plane, ky, kx;
            kblock(i, gt, plane, ky, kx);
            dy[i] = load_half(orr, (offb + (uint32_t)(2 * gt) * a.HWo) * 2u);
            dx[i] = load_half(orr, (offb + (uint32_t)(2 * gt + 1) * a.HWo) * 2u);
            m[i] = load_half(mr, (mskb + (uint32_t)gt * a.HWo) * 2u);
        }
    };
    u32x4 q[KMAX][4];
    float ly[KMAX], lx[KMAX], mm[KMAX];
    auto load_corners = [&](int b) {
        // 16-byte units; includes the border shift so (iy, ix) may be negative down to -2.
        const uint32_t xinb = (uint32_t)(b * a.CBLK * a.Hp + kPad) * a.Wp + kPad;
#pragma unroll
        for (int i = 0; i < KMAX; ++i) {
            int gt, plane, ky, kx;
            kblock(i, gt, plane, ky, kx);
            const bool live = pvalid && s0 + i < s1 && 4 * (s0 + i) + quarter < a.KB;
            // y = float(oy*sh - ph + ky*dh) + dy, as MetalShader.swift:327-332. Dead
            // units (tile tail, K padding) sample the zero border with weight 0.
            const float y = live ? (float)(base_y + ky * a.dh) + dy[i] : -16.0f;
            const float x = live ? (float)(base_x + kx * a.dw) + dx[i] : -16.0f;
            mm[i] = live ? m[i] : 0.0f;
            const float fy = floorf(y);
            const float fx = floorf(x);
            ly[i] = y - fy;
            lx[i] = x - fx;
            const int iy = (int)fminf(fmaxf(fy, (float)-kPad), (float)a.H);
            const int ix = (int)fminf(fmaxf(fx, (float)-kPad), (float)a.W);
            const uint32_t u = xinb + (uint32_t)(plane * a.Hp + iy) * a.Wp + ix;
            q[i][0] = load16(xr, u * 16u);
            q[i][1] = load16(xr, u * 16u + 16u);
            q[i][2] = load16(xr, (u + a.Wp) * 16u);
            q[i][3] = load16(xr, (u + a.Wp) * 16u + 16u);
        }
    };
    load_raw(z0);
    load_corners(z0);
    if (z0 + 1 < z1) load_raw(z0 + 1);

    for (int z = z0; z < z1; ++z) {
        f32x4 acc[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{};
#pragma unroll
        for (int i = 0; i < KMAX; ++i) {
            if (s0 + i < s1) {  // uniform across the wave
                const h8 A = blend<SAMPLER>(q[i][0], q[i][1], q[i][2], q[i][3], ly[i], lx[i], mm[i]);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bf[i][nb], acc[nb], 0, 0, 0);
            }
        }
        if (z + 1 < z1) {
            load_corners(z + 1);
            if (z + 2 < z1) load_raw(z + 2);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int v = 0; v < 4; ++v) red[((wave * NB + nb) * 4 + v) * 65 + lane] = acc[nb][v];
        __syncthreads();

        for (int idx = tid; idx < 16 * NB * 16; idx += 64 * NW) {
            const int pl = idx & 15;
            const int oc = idx >> 4;
            const int nb = oc >> 4;
            const int src = ((pl >> 2) << 4) + (oc & 15);
            const int v = pl & 3;
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) sum += red[((w * NB + nb) * 4 + v) * 65 + src];
            if (pvalid) {  // pl == lane % 16: this lane's pixel
                size_t dst;
                if (a.out_cb8) {
                    const int c = a.out_coff + oc;
                    dst = (((size_t)z * a.out_cblk + (c >> 3)) * (a.Ho + 2 * kPad) + oy + kPad) *
                              (size_t)(a.Wo + 2 * kPad) * 8 + (size_t)(ox + kPad) * 8 + (c & 7);
                } else {
                    dst = ((size_t)z * a.Cout + oc) * a.HWo + sp;
                }
                a.out[dst] = __builtin_bit_cast(uint16_t, round_f16(sum + a.bias[oc]));
            }
        }
        if (z + 1 < z1) __syncthreads();  // sums read before the next image's partials
    }
}

// Images per workgroup of the batched narrow kernel: up to 16, balanced over the
// workgroups of a tile. Measured for a body step over 16 tiles (images per workgroup ->
// us per step): 2 -> 642, 4 -> 632, 8 -> 628, 16 -> 627 (654 with one image per
// workgroup of narrow_kernel).
static int narrow_images_per_group(int images) {
    constexpr int kMax = 16;
    const int groups = (images + kMax - 1) / kMax;
    return (images + groups - 1) / groups;
}

template <int NB, int NW, int SAMPLER>
hipError_t launch_narrow_images_t(NarrowArgs a, int images, hipStream_t stream) {
    constexpr int KMAX = 3;
    const size_t lds = (size_t)NW * NB * 4 * 65 * sizeof(float);
    auto kernel = &narrow_images_kernel<NB, NW, KMAX, SAMPLER>;
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), (int)lds);
    if (attr != hipSuccess) return attr;
    a.tiles = (a.HWo + 15) / 16;  // per image
    const int zpw = narrow_images_per_group(images);
    const dim3 grid((unsigned)((a.tiles + 7) / 8 * 8), 1, (unsigned)((images + zpw - 1) / zpw));
    hipLaunchKernelGGL(kernel, grid, dim3(64 * NW), lds, stream, a, images, zpw);
    return hipGetLastError();
}

template <int NB, int NW, int SAMPLER>
hipError_t launch_narrow_t(const NarrowArgs& a, hipStream_t stream) {
    // K-steps whose loads are in flight at once, sized to the register budget of
    // NW / 4 waves per SIMD (more output columns hold more weight fragments).
    constexpr int U = NB >= 6 ? (NW == 12 ? 2 : 3) : (NW == 12 ? 3 : 5);
    const size_t lds = (size_t)NW * NB * 64 * 4 * sizeof(float) + 1024;  // + the warm-up slot
    auto kernel = &narrow_kernel<NB, NW, U, SAMPLER>;
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), (int)lds);
    if (attr != hipSuccess) return attr;
    const int grid = (a.tiles + 7) / 8 * 8;
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(64 * NW), lds, stream, a);
    return hipGetLastError();
}

template <int SAMPLER>
hipError_t launch_narrow_s(const NarrowArgs& a, int nb, int nw, hipStream_t stream) {
    if (nw == 8) {
        switch (nb) {
            case 2: return launch_narrow_t<2, 8, SAMPLER>(a, stream);
            case 4: return launch_narrow_t<4, 8, SAMPLER>(a, stream);
            case 6: return launch_narrow_t<6, 8, SAMPLER>(a, stream);
            case 8: return launch_narrow_t<8, 8, SAMPLER>(a, stream);
        }
    } else if (nw == 12) {
        switch (nb) {
            case 2: return launch_narrow_t<2, 12, SAMPLER>(a, stream);
            case 4: return launch_narrow_t<4, 12, SAMPLER>(a, stream);
            case 6: return launch_narrow_t<6, 12, SAMPLER>(a, stream);
            case 8: return launch_narrow_t<8, 12, SAMPLER>(a, stream);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace

// Rows each side of a band's receptive field that narrow_kernel's L2 warm-up loads.
constexpr int kNarrowWarmHalo = 16;

int narrow_ksteps(const FusedGeometry& g) { return (g.kb + 3) / 4; }

size_t narrow_packed_bytes(const FusedGeometry& g) {
    return (size_t)narrow_ksteps(g) * (g.nb * 2) * 64 * 8 * sizeof(uint16_t);
}

hipError_t launch_narrow_f16(const KShape& s, const FusedGeometry& g, const FusedConfig& cfg,
                             const void* cb8, const uint16_t* off, const uint16_t* mask,
                             const void* packed_w, const float* packed_b, uint16_t* out,
                             hipStream_t stream, OutPlacement place) {
    NarrowArgs a;
    a.out_cb8 = place.cb8;
    a.out_coff = place.coff;
    a.out_cblk = place.cblk;
    a.xin = cb8;
    a.off = off;
    a.msk = mask;
    a.wpk = packed_w;
    a.bias = packed_b;
    a.out = out;
    const size_t hwo = (size_t)s.Ho * s.Wo;
    a.xin_bytes = (uint32_t)((size_t)s.B * g.cblk * g.hp * g.wp * 16);
    a.off_bytes = (uint32_t)((size_t)s.B * 2 * s.og * g.ka * hwo * 2);
    a.msk_bytes = (uint32_t)((size_t)s.B * s.og * g.ka * hwo * 2);
    a.wpk_bytes = (uint32_t)narrow_packed_bytes(g);
    a.H = s.H;
    a.W = s.W;
    a.Ho = s.Ho;
    a.Wo = s.Wo;
    a.HWo = (int)hwo;
    a.KW = s.KW;
    a.KA = g.ka;
    a.ph = s.ph;
    a.pw = s.pw;
    a.sh = s.sh;
    a.sw = s.sw;
    a.dh = s.dh;
    a.dw = s.dw;
    a.GKA = s.og * g.ka;
    a.CB = g.cb;
    a.CBLK = g.cblk;
    a.Hp = g.hp;
    a.Wp = g.wp;
    a.KB = g.kb;
    a.ksteps = narrow_ksteps(g);
    a.M = (int)g.m;
    a.Cout = s.Cout;
    a.tiles = (int)((g.m + 15) / 16);
    a.magic_cb = magic_for(g.cb);
    a.magic_ka = magic_for(g.ka);
    a.magic_kw = magic_for(s.KW);
    a.pf_halo = kNarrowWarmHalo;
    // Batches of images whose K range fits three K-steps per wave (the body's 128 -> 64
    // DCN over many tiles): weights stay in registers across the images of a workgroup.
    // From four images on (C3's tiles at batch 2: 19.5 us against 18.6 us for
    // narrow_kernel; at batch 4: 33.0 against 33.7 us).
    if (cfg.sampler == kSamplerBf16) return launch_narrow_s<kSamplerBf16>(a, g.nb * 2, cfg.ks, stream);
    if (s.B >= 4 && g.nb * 2 == 4 && cfg.ks == 12 && (a.ksteps + 11) / 12 <= 3)
        return cfg.sampler == kSamplerExact ? launch_narrow_images_t<4, 12, kSamplerExact>(a, s.B, stream)
                                            : launch_narrow_images_t<4, 12, kSamplerFast>(a, s.B, stream);
    if (cfg.sampler == kSamplerExact) return launch_narrow_s<kSamplerExact>(a, g.nb * 2, cfg.ks, stream);
    return launch_narrow_s<kSamplerFast>(a, g.nb * 2, cfg.ks, stream);
}

}  // namespace dcn
