// Fused FP16 DCNv2 for gfx950: bilinear sampler -> MFMA GEMM in one kernel.
//
// GEMM view (executeJasnaSIMDGroupGEMM, MetalRunner.swift:696-761):
//   out[pixel][oc] = sum_k A[pixel][k] * Bw[k][oc] + bias[oc],
//   A[pixel][k] = half(bilinear(x[ic], p + k-tap + offset) * mask),  K = Cin * Kh * Kw.
// The reference writes A to HBM (deform_conv2d_fp16_jasna_gather, 9.4 MB at 64x64)
// and reads it back in a second kernel. Here each wave computes A directly in the
// register layout of v_mfma_f32_32x32x16_f16 and never stores it.
//
// K order. K is split into "K-blocks" of 8 consecutive input channels that share
// one offset group and one kernel tap: kb = (g * KA + tap) * CB + cb, channels
// ic = g*Cg + cb*8 + 0..7. One MFMA K-step (16) is two K-blocks. In the MFMA operand
// layout lane l supplies row l%32 and K elements 8*(l/32) .. +7, so lane l of step s
// samples exactly one K-block (2s + l/32) for one pixel: one bilinear coordinate,
// four 16-byte corner loads, eight channels. Weights are prepacked in the same K
// order (prepack_kernel), so A and B agree by construction.
//
// Input layout ("CB8"): [B][Cin/8][H+4][W+4][8] FP16 with a 2-pixel zero border.
// A corner load is one 16-byte vector. Clamping the top-left corner into
// [-2, H] x [-2, W] keeps both rows/columns inside the padded plane; any sample whose
// true corner lies outside that range touches only border zeros, so the reference's
// per-corner zero padding holds exactly without per-corner tests.
//
// Workgroup = KS waves on one tile of 32*MT output pixels; wave w owns a contiguous
// slice of the K-steps and all Cout columns. Partial sums meet in LDS; the epilogue
// adds the bias, rounds to FP16 and stores NCHW rows of consecutive pixels.
//
// All gathers use buffer loads with the exact buffer size as the range, so an
// access outside a tensor returns zero instead of faulting.
#include <algorithm>

#include <hip/hip_runtime.h>

#include "dcn_device.hpp"
#include "dcn_internal.hpp"

#pragma clang fp contract(off)

namespace dcn {
namespace {

using namespace dev;

constexpr size_t kMaxLds = 160 * 1024;  // LDS per workgroup on gfx950

struct FusedArgs {
    const void* xin;       // CB8 input
    const uint16_t* off;   // [B][2*G*KA][HWo]
    const uint16_t* msk;   // [B][G*KA][HWo]
    const void* wpk;       // [ksteps][NB][64][8] FP16
    const float* bias;     // [Cout]
    uint16_t* out;         // [B][Cout][HWo]
    uint32_t xin_bytes, off_bytes, msk_bytes, wpk_bytes;
    int H, W, Wo, HWo, KW, KA, ph, pw, sh, sw, dh, dw;
    int G, CB, CBLK, Hp, Wp, KB, ksteps, M, Cout;
};

template <int NB, int MT, int KS, int SAMPLER>
__global__ __launch_bounds__(64 * KS) void fused_kernel(FusedArgs a) {
    extern __shared__ float red[];  // [KS][MT][NB][16][65]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row = lane & 31;
    const int kb_half = lane >> 5;
    const int p0 = blockIdx.x * 32 * MT;

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xin, a.xin_bytes);
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.off, a.off_bytes);
    const __amdgpu_buffer_rsrc_t mr = make_rsrc(a.msk, a.msk_bytes);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wpk, a.wpk_bytes);

    int base_y[MT], base_x[MT];
    uint32_t offb[MT], mskb[MT], xinb[MT];
    bool pvalid[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int p = p0 + mt * 32 + row;
        pvalid[mt] = p < a.M;
        const int pc = pvalid[mt] ? p : a.M - 1;
        const int b = pc / a.HWo;
        const int sp = pc - b * a.HWo;
        const int oy = sp / a.Wo;
        const int ox = sp - oy * a.Wo;
        base_y[mt] = oy * a.sh - a.ph;
        base_x[mt] = ox * a.sw - a.pw;
        offb[mt] = (uint32_t)(b * 2 * a.G * a.KA) * a.HWo + sp;
        mskb[mt] = (uint32_t)(b * a.G * a.KA) * a.HWo + sp;
        // 16-byte units; includes the border shift so (iy, ix) may be negative down to -2.
        xinb[mt] = (uint32_t)(b * a.CBLK * a.Hp + kPad) * a.Wp + kPad;
    }

    f32x16 acc[MT][NB];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mt][nb] = f32x16{};

    const int s0 = wave * a.ksteps / KS;
    const int s1 = (wave + 1) * a.ksteps / KS;
    for (int s = s0; s < s1; ++s) {
        const int kb = 2 * s + kb_half;
        const bool kvalid = kb < a.KB;
        const int kbc = kvalid ? kb : a.KB - 1;
        const int gt = (a.CB == 1) ? kbc : kbc / a.CB;  // g * KA + tap
        const int cb = kbc - gt * a.CB;
        const int g = gt / a.KA;
        const int tap = gt - g * a.KA;
        const int ky = tap / a.KW;
        const int kx = tap - ky * a.KW;
        const int plane = g * a.CB + cb;

        h8 A[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const bool live = pvalid[mt] && kvalid;
            constexpr bool kBf16 = SAMPLER == kSamplerBf16;
            const uint32_t dyo = (offb[mt] + (uint32_t)(2 * gt) * a.HWo) * 2u;
            const uint32_t dxo = (offb[mt] + (uint32_t)(2 * gt + 1) * a.HWo) * 2u;
            const uint32_t mo = (mskb[mt] + (uint32_t)gt * a.HWo) * 2u;
            const float dy = kBf16 ? load_bf16(orr, dyo) : load_half(orr, dyo);
            const float dx = kBf16 ? load_bf16(orr, dxo) : load_half(orr, dxo);
            float m = kBf16 ? load_bf16(mr, mo) : load_half(mr, mo);
            // y = float(oy*sh - ph + ky*dh) + dy, as MetalShader.swift:327-332.
            float y = (float)(base_y[mt] + ky * a.dh) + dy;
            float x = (float)(base_x[mt] + kx * a.dw) + dx;
            // Dead lanes (tile tail, odd K-block pad) sample the zero border with weight 0.
            y = live ? y : -16.0f;
            x = live ? x : -16.0f;
            m = live ? m : 0.0f;
            const float fy = floorf(y);
            const float fx = floorf(x);
            const float ly = y - fy;
            const float lx = x - fx;
            const int iy = (int)fminf(fmaxf(fy, (float)-kPad), (float)a.H);
            const int ix = (int)fminf(fmaxf(fx, (float)-kPad), (float)a.W);
            const uint32_t u = xinb[mt] + (uint32_t)(plane * a.Hp + iy) * a.Wp + ix;
            const uint32_t byte0 = u * 16u;
            const uint32_t byte1 = (u + a.Wp) * 16u;
            const u32x4 q00 = load16(xr, byte0);
            const u32x4 q01 = load16(xr, byte0 + 16u);
            const u32x4 q10 = load16(xr, byte1);
            const u32x4 q11 = load16(xr, byte1 + 16u);
            A[mt] = blend<SAMPLER>(q00, q01, q10, q11, ly, lx, m);
        }
        h8 Bf[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            Bf[nb] = __builtin_bit_cast(h8, load16(wr, (uint32_t)((s * NB + nb) * 64 + lane) * 16u));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                if constexpr (SAMPLER == kSamplerBf16)
                    acc[mt][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf8, A[mt]), __builtin_bit_cast(bf8, Bf[nb]), acc[mt][nb], 0, 0, 0);
                else
                    acc[mt][nb] =
                        __builtin_amdgcn_mfma_f32_32x32x16_f16(A[mt], Bf[nb], acc[mt][nb], 0, 0, 0);
            }
    }

    // Accumulator layout of a 32x32 MFMA: lane l holds column j = l%32 and rows
    // i = 8*(v/4) + 4*(l/32) + v%4 in element v. Row stride 65 floats avoids bank conflicts.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int v = 0; v < 16; ++v)
                red[(((wave * MT + mt) * NB + nb) * 16 + v) * 65 + lane] = acc[mt][nb][v];
    __syncthreads();

    constexpr int kTilePixels = 32 * MT;
    for (int idx = threadIdx.x; idx < kTilePixels * NB * 32; idx += 64 * KS) {
        const int pl = idx % kTilePixels;
        const int oc = idx / kTilePixels;
        const int mt = pl >> 5;
        const int i = pl & 31;
        const int nb = oc >> 5;
        const int j = oc & 31;
        const int v = 4 * (i >> 3) + (i & 3);
        const int src = j + 32 * ((i >> 2) & 1);
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < KS; ++w) sum += red[(((w * MT + mt) * NB + nb) * 16 + v) * 65 + src];
        const int p = p0 + pl;
        if (p < a.M) {
            const int b = p / a.HWo;
            const int sp = p - b * a.HWo;
            a.out[((size_t)b * a.Cout + oc) * a.HWo + sp] =
                SAMPLER == kSamplerBf16 ? round_bf16_bits(sum + a.bias[oc])
                                        : __builtin_bit_cast(uint16_t, round_f16(sum + a.bias[oc]));
        }
    }
}

// ---- LDS-staged variant -----------------------------------------------------------
// Phase 1 (sampler): thread t owns pixel t % TP of the tile and K-blocks
// t / TP + i * (T / TP). It gathers UB units at a time with every load in flight
// (offsets and mask, then the four 16-byte corners of each unit), blends them and
// writes 16 bytes into the LDS A tile laid out [K-block][pixel][8 channels]: the
// modulated im2col tile of the reference's gather kernel, kept on chip.
// Phase 2 (GEMM): wave w takes K-steps [w*ksteps/NW, (w+1)*ksteps/NW) for all TP/32
// pixel blocks and all Cout columns. A fragments are 16-byte LDS reads of 32
// consecutive pixels (conflict-free), B fragments come from the prepacked buffer.
// Phase 3: partial sums of the NW waves meet in LDS (reusing the A tile), then bias,
// FP16 rounding and NCHW stores of consecutive pixels.
struct StagedArgs {
    FusedArgs f;
    uint32_t magic_cb, magic_ka, magic_kw;  // ceil(2^32 / d) for d = CB, KA, KW
};


template <int NB, int MT, int NW, int UB, int SPW, int SAMPLER>
__global__ __launch_bounds__(64 * NW) void staged_kernel(StagedArgs sa) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const FusedArgs& a = sa.f;
    constexpr int TP = 32 * MT;
    constexpr int T = 64 * NW;
    constexpr int KSTRIDE = T / TP;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int p0 = blockIdx.x * TP;
    const int kbp = 2 * a.ksteps;

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xin, a.xin_bytes);
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.off, a.off_bytes);
    const __amdgpu_buffer_rsrc_t mr = make_rsrc(a.msk, a.msk_bytes);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wpk, a.wpk_bytes);

    // ---- phase 1: sampler -> LDS ---------------------------------------------------
    {
        const int pl = tid % TP;
        const int p = p0 + pl;
        const bool pvalid = p < a.M;
        const int pc = pvalid ? p : a.M - 1;
        const int b = pc / a.HWo;
        const int sp = pc - b * a.HWo;
        const int oy = sp / a.Wo;
        const int ox = sp - oy * a.Wo;
        const int base_y = oy * a.sh - a.ph;
        const int base_x = ox * a.sw - a.pw;
        const uint32_t offb = (uint32_t)(b * 2 * a.G * a.KA) * a.HWo + sp;
        const uint32_t mskb = (uint32_t)(b * a.G * a.KA) * a.HWo + sp;
        const uint32_t xinb = (uint32_t)(b * a.CBLK * a.Hp + kPad) * a.Wp + kPad;
        const int kb0 = tid / TP;
        const int units = (kbp - kb0 + KSTRIDE - 1) / KSTRIDE;
        for (int base = 0; base < units; base += UB) {
            float dy[UB], dx[UB], m[UB];
            int plane[UB], yb[UB], xb[UB];
#pragma unroll
            for (int i = 0; i < UB; ++i) {
                const int kb = kb0 + (base + i) * KSTRIDE;
                const int kbc = kb < a.KB ? kb : a.KB - 1;
                const int gt = a.CB == 1 ? kbc : fast_div(kbc, sa.magic_cb);
                const int cb = kbc - gt * a.CB;
                const int g = fast_div(gt, sa.magic_ka);
                const int tap = gt - g * a.KA;
                const int ky = fast_div(tap, sa.magic_kw);
                const int kx = tap - ky * a.KW;
                plane[i] = g * a.CB + cb;
                yb[i] = base_y + ky * a.dh;
                xb[i] = base_x + kx * a.dw;
                dy[i] = load_half(orr, (offb + (uint32_t)(2 * gt) * a.HWo) * 2u);
                dx[i] = load_half(orr, (offb + (uint32_t)(2 * gt + 1) * a.HWo) * 2u);
                m[i] = load_half(mr, (mskb + (uint32_t)gt * a.HWo) * 2u);
            }
            u32x4 q[UB][4];
            float ly[UB], lx[UB];
#pragma unroll
            for (int i = 0; i < UB; ++i) {
                const int kb = kb0 + (base + i) * KSTRIDE;
                const bool live = pvalid && kb < a.KB;
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
#pragma unroll
            for (int i = 0; i < UB; ++i) {
                const int kb = kb0 + (base + i) * KSTRIDE;
                if (kb < kbp) {
                    const h8 v = blend<SAMPLER>(q[i][0], q[i][1], q[i][2], q[i][3], ly[i], lx[i], m[i]);
                    *reinterpret_cast<h8*>(lds + ((size_t)kb * TP + pl) * 16) = v;
                }
            }
        }
    }
    __syncthreads();

    // ---- phase 2: MFMA over this wave's K-steps --------------------------------------
    const int s0 = wave * a.ksteps / NW;
    const int s1 = (wave + 1) * a.ksteps / NW;
    f32x16 acc[MT][NB];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mt][nb] = f32x16{};
    for (int sb = s0; sb < s1; sb += SPW) {
        h8 Bf[SPW][NB];
#pragma unroll
        for (int j = 0; j < SPW; ++j)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int s = sb + j < s1 ? sb + j : s1 - 1;
                Bf[j][nb] = __builtin_bit_cast(h8, load16(wr, (uint32_t)((s * NB + nb) * 64 + lane) * 16u));
            }
#pragma unroll
        for (int j = 0; j < SPW; ++j) {
            if (sb + j < s1) {
                const int kb = 2 * (sb + j) + (lane >> 5);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const h8 A = *reinterpret_cast<const h8*>(lds + ((size_t)kb * TP + mt * 32 + (lane & 31)) * 16);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        acc[mt][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A, Bf[j][nb], acc[mt][nb], 0, 0, 0);
                }
            }
        }
    }
    __syncthreads();  // the A tile is dead from here on

    // ---- phase 3: cross-wave reduction, bias, FP16, NCHW store -----------------------
    float* red = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int v = 0; v < 16; ++v)
                red[(((wave * MT + mt) * NB + nb) * 16 + v) * 65 + lane] = acc[mt][nb][v];
    __syncthreads();
    for (int idx = tid; idx < TP * NB * 32; idx += T) {
        const int pl = idx % TP;
        const int oc = idx / TP;
        const int mt = pl >> 5;
        const int i = pl & 31;
        const int nb = oc >> 5;
        const int j = oc & 31;
        const int v = 4 * (i >> 3) + (i & 3);
        const int src = j + 32 * ((i >> 2) & 1);
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) sum += red[(((w * MT + mt) * NB + nb) * 16 + v) * 65 + src];
        const int p = p0 + pl;
        if (p < a.M) {
            const int b = p / a.HWo;
            const int sp = p - b * a.HWo;
            a.out[((size_t)b * a.Cout + oc) * a.HWo + sp] =
                __builtin_bit_cast(uint16_t, round_f16(sum + a.bias[oc]));
        }
    }
}

// An empty kernel: what any kernel of its launch shape (workgroups, threads, dynamic LDS)
// pays for dispatch, wave launch and completion. Nothing is read or written.
__global__ void launch_floor_kernel() {}

// NCHW FP16 -> padded CB8. Grid (ceil(Hp*Wp / 256), B * Cin/8): one thread per padded
// position of one channel block, eight 2-byte loads (coalesced along x) and one 16-byte
// store; border positions get zeros. 32-bit index math only.
__global__ __launch_bounds__(256) void pack_cb8_kernel(const uint16_t* __restrict__ in,
                                                       u32x4* __restrict__ out, int H, int W,
                                                       int Hp, int Wp) {
    const int pos = blockIdx.x * 256 + threadIdx.x;
    const int plane_p = Hp * Wp;
    if (pos >= plane_p) return;
    const int yp = pos / Wp;
    const int y = yp - kPad;
    const int x = pos - yp * Wp - kPad;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (y >= 0 && y < H && x >= 0 && x < W) {
        const size_t plane = (size_t)H * W;
        // blockIdx.y = b * Cin/8 + cblk: the first of its 8 NCHW planes is 8 * blockIdx.y.
        const uint16_t* src = in + (size_t)blockIdx.y * 8 * plane + (size_t)y * W + x;
#pragma unroll
        for (int d = 0; d < 4; ++d)
            v[d] = (uint32_t)src[(2 * d) * plane] | ((uint32_t)src[(2 * d + 1) * plane] << 16);
    }
    out[(size_t)blockIdx.y * plane_p + pos] = v;
}

// Weights -> MFMA B fragments [ksteps][NB][64 lanes][8] for column groups of MW
// output channels (32: v_mfma_f32_32x32x16_f16, 16: v_mfma_f32_16x16x32_f16). Lane l
// of K-step s holds output channel nb*MW + l%MW and K-block (64/MW)*s + l/MW, the
// order in which the fused kernels sample A. layout 0 = OIHW, 1 = [ic][k][oc]
// (.dcnfp16). Bias widened to FP32 (when bpk is non-null).
__global__ __launch_bounds__(256) void prepack_kernel(const uint16_t* __restrict__ w, int layout,
                                                      const uint16_t* __restrict__ bias,
                                                      uint16_t* __restrict__ wpk,
                                                      float* __restrict__ bpk, int Cin, int Cout,
                                                      int KA, int CB, int KB, int NB, int MW,
                                                      long total, int bias_bf16) {
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (bpk != nullptr && gid < Cout)
        bpk[gid] = bias_bf16 ? __builtin_bit_cast(float, (uint32_t)bias[gid] << 16)
                             : (float)__builtin_bit_cast(_Float16, bias[gid]);
    if (gid >= total) return;
    const int e = (int)(gid & 7);
    const int lane = (int)((gid >> 3) & 63);
    const long q = gid >> 9;
    const int nb = (int)(q % NB);
    const int s = (int)(q / NB);
    const int kb = (64 / MW) * s + lane / MW;
    const int oc = nb * MW + lane % MW;
    uint16_t v = 0;
    if (kb < KB && oc < Cout) {
        const int gt = kb / CB;
        const int cb = kb - gt * CB;
        const int g = gt / KA;
        const int tap = gt - g * KA;
        const int ic = (g * CB + cb) * 8 + e;
        v = layout == DCN_LAYOUT_OIHW ? w[((size_t)oc * Cin + ic) * KA + tap]
                                      : w[((size_t)ic * KA + tap) * Cout + oc];
    }
    wpk[gid] = v;
}

// deform_conv2d_fp16_jasna_gather (MetalShader.swift:299-381) for any offset-group
// count: one thread per im2col element, reference arithmetic.
__global__ __launch_bounds__(256) void im2col_kernel(const uint16_t* __restrict__ input,
                                                     const uint16_t* __restrict__ offset,
                                                     const uint16_t* __restrict__ mask,
                                                     uint16_t* __restrict__ columns, KShape s,
                                                     long total) {
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    const long ka = (long)s.KH * s.KW;
    const long ncol = (long)s.Cin * ka;
    const long row = gid / ncol;
    const long col = gid - row * ncol;
    const long ic = col / ka;
    const long k = col - ic * ka;
    const long plane = (long)s.Ho * s.Wo;
    const long n = row / plane;
    const long sp = row - n * plane;
    const long oy = sp / s.Wo;
    const long ox = sp - oy * s.Wo;
    const long og = ic / (s.Cin / s.og);
    const long ky = k / s.KW;
    const long kx = k - ky * s.KW;
    const long sample = og * ka + k;
    const long obase = n * 2 * s.og * ka * plane;
    const float y = (float)(oy * s.sh + ky * s.dh - s.ph) +
                    (float)__builtin_bit_cast(_Float16, offset[obase + 2 * sample * plane + sp]);
    const float x = (float)(ox * s.sw + kx * s.dw - s.pw) +
                    (float)__builtin_bit_cast(_Float16, offset[obase + (2 * sample + 1) * plane + sp]);
    const float fy = fminf(fmaxf(floorf(y), -4.0f), (float)s.H + 4.0f);
    const float fx = fminf(fmaxf(floorf(x), -4.0f), (float)s.W + 4.0f);
    const int y0 = (int)fy, x0 = (int)fx, y1 = y0 + 1, x1 = x0 + 1;
    const float ly = y - floorf(y);
    const float lx = x - floorf(x);
    const uint16_t* src = input + (n * s.Cin + ic) * (long)s.H * s.W;
    auto value = [&](int yy, int xx) -> float {
        return (yy >= 0 && yy < s.H && xx >= 0 && xx < s.W)
                   ? (float)__builtin_bit_cast(_Float16, src[(long)yy * s.W + xx])
                   : 0.0f;
    };
    const float sampled = value(y0, x0) * (1.0f - ly) * (1.0f - lx) +
                          value(y0, x1) * (1.0f - ly) * lx + value(y1, x0) * ly * (1.0f - lx) +
                          value(y1, x1) * ly * lx;
    const float m = (float)__builtin_bit_cast(_Float16, mask[n * s.og * ka * plane + sample * plane + sp]);
    columns[gid] = __builtin_bit_cast(uint16_t, round_f16(sampled * m));
}

// flag_non_finite_fp16 (MetalShader.swift:454-463): exponent all ones -> NaN or Inf.
__global__ __launch_bounds__(256) void nonfinite_kernel(const uint16_t* __restrict__ values,
                                                        size_t count, uint32_t* flag) {
    bool bad = false;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x)
        bad |= (values[i] & 0x7c00u) == 0x7c00u;
    if (__builtin_amdgcn_ballot_w64(bad) != 0 && (threadIdx.x & 63) == 0) atomicOr(flag, 1u);
}

template <int NB, int MT, int KS, int SAMPLER>
hipError_t launch_fused_t(const FusedArgs& a, long tiles, hipStream_t stream) {
    const size_t lds = (size_t)KS * MT * NB * 16 * 65 * sizeof(float);
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(&fused_kernel<NB, MT, KS, SAMPLER>), lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((fused_kernel<NB, MT, KS, SAMPLER>), dim3((unsigned)tiles), dim3(64 * KS),
                       lds, stream, a);
    return hipGetLastError();
}

template <int NB, int SAMPLER>
hipError_t launch_fused_nb(const FusedArgs& a, const FusedConfig& cfg, hipStream_t stream) {
    const long tiles = ((long)a.M + 32 * cfg.mt - 1) / (32 * cfg.mt);
    if (cfg.mt == 1 && cfg.ks == 8) return launch_fused_t<NB, 1, 8, SAMPLER>(a, tiles, stream);
    if (cfg.mt == 1 && cfg.ks == 4) return launch_fused_t<NB, 1, 4, SAMPLER>(a, tiles, stream);
    if (cfg.mt == 2 && cfg.ks == 4) return launch_fused_t<NB, 2, 4, SAMPLER>(a, tiles, stream);
    if (cfg.mt == 2 && cfg.ks == 2) return launch_fused_t<NB, 2, 2, SAMPLER>(a, tiles, stream);
    return hipErrorInvalidValue;
}

template <int NB, int MT, int NW, int SAMPLER>
hipError_t launch_staged_t(const StagedArgs& sa, long tiles, size_t lds, hipStream_t stream) {
    // Units gathered per batch and K-steps whose B fragments are held at once, sized so
    // the batch fits the register budget of the occupancy (2 or 4 waves per SIMD).
    constexpr int UB = NW == 8 ? 9 : 5;
    constexpr int kRegs = NW == 8 ? 200 : 96;
    constexpr int kSpw = (kRegs - MT * NB * 16) / (NB * 4);
    constexpr int SPW = kSpw < 1 ? 1 : (kSpw > (NW == 8 ? 9 : 5) ? (NW == 8 ? 9 : 5) : kSpw);
    auto kernel = &staged_kernel<NB, MT, NW, UB, SPW, SAMPLER>;
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), kMaxLds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kernel, dim3((unsigned)tiles), dim3(64 * NW), lds, stream, sa);
    return hipGetLastError();
}

template <int NB, int SAMPLER>
hipError_t launch_staged_nb(const StagedArgs& sa, const FusedConfig& cfg, size_t lds, hipStream_t stream) {
    const long tiles = ((long)sa.f.M + 32 * cfg.mt - 1) / (32 * cfg.mt);
    if (cfg.mt == 1 && cfg.ks == 8) return launch_staged_t<NB, 1, 8, SAMPLER>(sa, tiles, lds, stream);
    if (cfg.mt == 1 && cfg.ks == 16) return launch_staged_t<NB, 1, 16, SAMPLER>(sa, tiles, lds, stream);
    if (cfg.mt == 2 && cfg.ks == 8) return launch_staged_t<NB, 2, 8, SAMPLER>(sa, tiles, lds, stream);
    if (cfg.mt == 2 && cfg.ks == 16) return launch_staged_t<NB, 2, 16, SAMPLER>(sa, tiles, lds, stream);
    return hipErrorInvalidValue;
}

template <int SAMPLER>
hipError_t launch_staged_s(const StagedArgs& sa, int nb, const FusedConfig& cfg, size_t lds,
                           hipStream_t stream) {
    switch (nb) {
        case 1: return launch_staged_nb<1, SAMPLER>(sa, cfg, lds, stream);
        case 2: return launch_staged_nb<2, SAMPLER>(sa, cfg, lds, stream);
        case 3: return launch_staged_nb<3, SAMPLER>(sa, cfg, lds, stream);
        case 4: return launch_staged_nb<4, SAMPLER>(sa, cfg, lds, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int SAMPLER>
hipError_t launch_fused_s(const FusedArgs& a, int nb, const FusedConfig& cfg, hipStream_t stream) {
    switch (nb) {
        case 1: return launch_fused_nb<1, SAMPLER>(a, cfg, stream);
        case 2: return launch_fused_nb<2, SAMPLER>(a, cfg, stream);
        case 3: return launch_fused_nb<3, SAMPLER>(a, cfg, stream);
        case 4: return launch_fused_nb<4, SAMPLER>(a, cfg, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool fused_geometry(const dcn_shape& s, FusedGeometry* g) {
    if (s.groups != 1 || s.input_channels % s.offset_groups != 0) return false;
    const int cg = s.input_channels / s.offset_groups;
    if (cg % 8 != 0 || s.output_channels % 32 != 0 || s.output_channels > 128) return false;
    g->cblk = s.input_channels / 8;
    g->cb = cg / 8;
    g->ka = s.kernel_height * s.kernel_width;
    g->kb = s.offset_groups * g->ka * g->cb;
    g->ksteps = (g->kb + 1) / 2;
    g->nb = s.output_channels / 32;
    g->hp = s.input_height + 2 * kPad;
    g->wp = s.input_width + 2 * kPad;
    g->m = (long long)s.batch * s.output_height * s.output_width;
    return true;
}

hipError_t launch_floor(int workgroups, int threads, int lds_bytes, hipStream_t stream) {
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(&launch_floor_kernel), lds_bytes);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(launch_floor_kernel, dim3((unsigned)workgroups), dim3((unsigned)threads),
                       (size_t)lds_bytes, stream);
    return hipGetLastError();
}

hipError_t launch_pack_cb8(const KShape& s, const FusedGeometry& g, const uint16_t* in_nchw,
                           void* cb8, hipStream_t stream) {
    const long planes = (long)s.B * g.cblk;
    if (planes > 65535) return hipErrorInvalidValue;  // grid.y limit
    const unsigned gx = (unsigned)(((long)g.hp * g.wp + 255) / 256);
    hipLaunchKernelGGL(pack_cb8_kernel, dim3(gx, (unsigned)planes), dim3(256), 0, stream, in_nchw,
                       (u32x4*)cb8, s.H, s.W, g.hp, g.wp);
    return hipGetLastError();
}

hipError_t launch_prepack_weights(const KShape& s, const FusedGeometry& g, const uint16_t* w,
                                  int layout, const uint16_t* bias, void* packed_w,
                                  float* packed_b, hipStream_t stream, bool bias_bf16) {
    const long total = (long)g.ksteps * g.nb * 64 * 8;
    const long grid = (std::max<long>(total, s.Cout) + 255) / 256;
    hipLaunchKernelGGL(prepack_kernel, dim3((unsigned)grid), dim3(256), 0, stream, w, layout, bias,
                       (uint16_t*)packed_w, packed_b, s.Cin, s.Cout, g.ka, g.cb, g.kb, g.nb, 32,
                       total, bias_bf16 ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_prepack_narrow(const KShape& s, const FusedGeometry& g, const uint16_t* w,
                                 int layout, void* packed_w, hipStream_t stream) {
    const long total = (long)narrow_ksteps(g) * (2 * g.nb) * 64 * 8;
    const long grid = (total + 255) / 256;
    hipLaunchKernelGGL(prepack_kernel, dim3((unsigned)grid), dim3(256), 0, stream, w, layout,
                       (const uint16_t*)nullptr, (uint16_t*)packed_w, (float*)nullptr, s.Cin,
                       s.Cout, g.ka, g.cb, g.kb, 2 * g.nb, 16, total, 0);
    return hipGetLastError();
}

hipError_t launch_fused_f16(const KShape& s, const FusedGeometry& g, const FusedConfig& cfg,
                            const void* cb8, const uint16_t* off, const uint16_t* mask,
                            const void* packed_w, const float* packed_b, uint16_t* out,
                            hipStream_t stream) {
    FusedArgs a;
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
    a.wpk_bytes = (uint32_t)packed_weight_bytes(g);
    a.H = s.H;
    a.W = s.W;
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
    a.G = s.og;
    a.CB = g.cb;
    a.CBLK = g.cblk;
    a.Hp = g.hp;
    a.Wp = g.wp;
    a.KB = g.kb;
    a.ksteps = g.ksteps;
    a.M = (int)g.m;
    a.Cout = s.Cout;
    if (cfg.variant == kVariantStaged) {
        StagedArgs sa{a, magic_for(g.cb), magic_for(g.ka), magic_for(s.KW)};
        const size_t lds = staged_lds_bytes(g, cfg);
        if (lds > kMaxLds) return hipErrorInvalidValue;
        if (cfg.sampler == kSamplerExact) return launch_staged_s<kSamplerExact>(sa, g.nb, cfg, lds, stream);
        return launch_staged_s<kSamplerFast>(sa, g.nb, cfg, lds, stream);
    }
    if (cfg.sampler == kSamplerBf16) {
        if (cfg.variant != kVariantRegister) return hipErrorInvalidValue;
        return launch_fused_s<kSamplerBf16>(a, g.nb, cfg, stream);
    }
    if (cfg.sampler == kSamplerExact) return launch_fused_s<kSamplerExact>(a, g.nb, cfg, stream);
    return launch_fused_s<kSamplerFast>(a, g.nb, cfg, stream);
}

size_t staged_lds_bytes(const FusedGeometry& g, const FusedConfig& cfg) {
    const size_t tile = (size_t)2 * g.ksteps * 32 * cfg.mt * 16;
    const size_t red = (size_t)cfg.ks * cfg.mt * g.nb * 16 * 65 * sizeof(float);
    return std::max(tile, red);
}

hipError_t launch_im2col_f16(const KShape& s, const uint16_t* in, const uint16_t* off,
                             const uint16_t* mask, uint16_t* columns, hipStream_t stream) {
    const long total = (long)s.B * s.Ho * s.Wo * s.Cin * s.KH * s.KW;
    const long grid = (total + 255) / 256;
    hipLaunchKernelGGL(im2col_kernel, dim3((unsigned)grid), dim3(256), 0, stream, in, off, mask,
                       columns, s, total);
    return hipGetLastError();
}

hipError_t launch_flag_nonfinite_f16(const uint16_t* values, size_t count, uint32_t* flag,
                                     hipStream_t stream) {
    if (count == 0) return hipSuccess;
    const size_t grid = std::min<size_t>((count + 255) / 256, 4096);
    hipLaunchKernelGGL(nonfinite_kernel, dim3((unsigned)grid), dim3(256), 0, stream, values, count,
                       flag);
    return hipGetLastError();
}

}  // namespace dcn
