// Window-staged fused FP16 DCNv2 for gfx950 (3x3 kernels, 8 channels per offset group).
//
// Why: a deformable gather reads four random 16-byte corners per (pixel, group, tap).
// Served from the vector L1 these reads miss about half the time and keep the texture
// addresser stalled on the cache, and when tiles of many images share an XCD the 4 MB
// L2 thrashes (measured 3.5x the compulsory HBM bytes). Here each workgroup owns a 2D
// tile of output pixels and walks the offset groups in stages of GPS groups. For each
// group it computes the exact bounding box of all its sample corners over the tile,
// copies that window of the padded input plane into LDS with coalesced 16-byte loads,
// and gathers from LDS (optionally the lower corner row from the L1, which then holds
// the same window, to split the gather load between the two paths).
//
// Work split: NW waves, wave w owns one row block of 32 consecutive output pixels of the
// tile (TR rows x NW/TR row blocks) and all Cout columns over the whole K range, so no
// cross-wave reduction is needed. Within a stage, K-step k of v_mfma_f32_32x32x16_f16
// takes unit u = 2k + l/32 (lane l): group u/9 of the stage, tap u%9 — one bilinear
// coordinate and four 16-byte corners per lane. GPS = 2 pairs two groups into 9 K-steps
// with no padding; GPS = 1 uses 5 K-steps with a zero tenth unit. The weights are
// prepacked in the same order (prepack_group_kernel).
//
// Pipeline per stage (windows double-buffered): the next stage's offsets are loaded
// before this stage is multiplied; its windows are computed and copied after.
// A window larger than its LDS buffer makes that group gather from global memory
// (same arithmetic), so any offset field is handled. Lanes past the image edge sample
// a clamped in-image pixel: their accumulator rows are never stored.
//
// Tiles are ordered so that workgroup blockIdx lands on XCD blockIdx % 8 with a
// contiguous eighth of the pixels: each XCD's L2 holds the inputs of its own images
// (or image band) instead of all of them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>

#include "dcn_device.hpp"
#include "dcn_internal.hpp"

#pragma clang fp contract(off)

namespace dcn {
namespace {

using namespace dev;

// LDS for the windows of a workgroup: double-buffered (one workgroup per CU) or single
// (two workgroups share a CU and overlap each other's copy and compute phases).
__host__ __device__ constexpr int window_lds(int nbuf) { return nbuf == 2 ? 144 * 1024 : 72 * 1024; }

struct WindowArgs {
    const void* xin;      // CB8 input [B][CBLK][Hp][Wp][8]
    const uint16_t* off;  // [B][2*G*9][HWo]
    const uint16_t* msk;  // [B][G*9][HWo]
    const void* wpk;      // [stages][KS][NB][64][8] FP16 (prepack_group_kernel)
    const float* bias;    // [Cout]
    uint16_t* out;        // [B][Cout][HWo]
    uint32_t xin_bytes, off_bytes, msk_bytes, wpk_bytes;
    int B, H, W, Ho, Wo, HWo, ph, pw, sh, sw, dh, dw;
    int G, CBLK, Hp, Wp, Cout;
    int tiles_y, tiles_x, tiles;  // tile grid per image, total
};

// Unit u of a stage (0 .. 2*KS-1): group offset within the stage and tap.
template <int GPS>
__host__ __device__ constexpr int unit_group(int u) {
    return GPS == 2 ? (u >= 9 ? 1 : 0) : 0;
}
template <int GPS>
__host__ __device__ constexpr int unit_tap(int u) {
    return GPS == 2 ? u - 9 * (u >= 9 ? 1 : 0) : (u < 9 ? u : 8);
}

template <int NB, int NW, int TR, int GPS, int SAMPLER, int SPLIT, int NBUF, int UNI>
__global__ __launch_bounds__(64 * NW, UNI ? 2 : 1) void window_kernel(WindowArgs a) {
    // BF16 storage (kSamplerBf16): BF16 offsets, masks, windows and weights; the exact
    // sampler's FP32 bilinear rounded once to BF16, the BF16 MFMA, bf16(sum + bias).
    constexpr bool kBf16 = SAMPLER == kSamplerBf16;
    auto mfma32 = [](const h8& A, const h8& B, const f32x16& c) {
        if constexpr (kBf16)
            return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8, A), __builtin_bit_cast(bf8, B),
                                                           c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(A, B, c, 0, 0, 0);
    };
    constexpr int kWindowLds = window_lds(NBUF);
    constexpr int TCB = NW / TR;              // row blocks across the tile
    constexpr int T = 64 * NW;
    constexpr int KS = GPS == 2 ? 9 : 5;      // K-steps per stage
    constexpr int WIN = kWindowLds / (NBUF * GPS);  // bytes per window buffer
    constexpr int CPT = (WIN / 16 + T - 1) / T;  // chunks per thread for a full window
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int* box = reinterpret_cast<int*>(lds + kWindowLds);  // [2][GPS][NW][4]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;

    // XCD-aware tile order: blockIdx lands on XCD blockIdx % 8.
    const int per_xcd = (a.tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= a.tiles) return;  // whole workgroup, before any barrier
    const int tiles_img = a.tiles_y * a.tiles_x;
    const int b = tile / tiles_img;
    const int trem = tile - b * tiles_img;
    const int ty = trem / a.tiles_x;
    const int tx = trem - ty * a.tiles_x;
    const int oy_row = ty * TR + wave / TCB;
    const int ox0 = (tx * TCB + wave % TCB) * 32;
    // Lanes past the edge use a clamped pixel; their accumulator rows are not stored.
    const int oyc = min(oy_row, a.Ho - 1);
    const int oxc = min(ox0 + (lane & 31), a.Wo - 1);
    const int sp = oyc * a.Wo + oxc;

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xin, a.xin_bytes);
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.off, a.off_bytes);
    const __amdgpu_buffer_rsrc_t mr = make_rsrc(a.msk, a.msk_bytes);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wpk, a.wpk_bytes);

    // Per-lane constants: base coordinates float(oy*sh - ph + ky*dh),
    // float(ox*sw - pw + kx*dw) (MetalShader.swift:327-332) come from the pixel base
    // plus the tap; offset/mask byte offsets from a per-lane base plus the channel.
    const uint32_t hwo2 = (uint32_t)a.HWo * 2u;
    const int by = oyc * a.sh - a.ph;
    const int bx = oxc * a.sw - a.pw;
    const uint32_t off_lane = ((uint32_t)b * 2 * a.G * 9 * a.HWo + sp) * 2u;
    const uint32_t msk_lane = ((uint32_t)b * a.G * 9 * a.HWo + sp) * 2u;
    const int stages = a.G / GPS;
    // Tap and group offset of this lane's unit in K-step k (two compile-time choices).
    auto unit_of = [&](int k, int& tap, int& go) {
        tap = half ? unit_tap<GPS>(2 * k + 1) : unit_tap<GPS>(2 * k);
        go = half ? unit_group<GPS>(2 * k + 1) : unit_group<GPS>(2 * k);
    };

    // Raw offsets/mask of a stage, then sample state.
    float rdy[KS], rdx[KS], rm[KS];
    auto load_raw = [&](int st) {
        const uint32_t so = 2u * (uint32_t)(st * GPS * 9) * hwo2;  // dy of group st*GPS, tap 0
        const uint32_t sm = (uint32_t)(st * GPS * 9) * hwo2;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            int tap, go;
            unit_of(k, tap, go);
            const uint32_t ch = (uint32_t)(go * 9 + tap);
            if constexpr (kBf16) {
                rdy[k] = load_bf16(orr, off_lane + 2u * ch * hwo2, so);
                rdx[k] = load_bf16(orr, off_lane + (2u * ch + 1u) * hwo2, so);
                rm[k] = load_bf16(mr, msk_lane + ch * hwo2, sm);
            } else {
                rdy[k] = load_half(orr, off_lane + 2u * ch * hwo2, so);
                rdx[k] = load_half(orr, off_lane + (2u * ch + 1u) * hwo2, so);
                rm[k] = load_half(mr, msk_lane + ch * hwo2, sm);
            }
        }
    };
    int iy[KS], ix[KS];
    float ly[KS], lx[KS], mm[KS];
    int bmin_y[GPS], bmax_y[GPS], bmin_x[GPS], bmax_x[GPS];
    auto make_state = [&]() {
#pragma unroll
        for (int g = 0; g < GPS; ++g) {
            bmin_y[g] = INT_MAX;
            bmax_y[g] = INT_MIN;
            bmin_x[g] = INT_MAX;
            bmax_x[g] = INT_MIN;
        }
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            int tap, go;
            unit_of(k, tap, go);
            const int ky = tap / 3, kx = tap - 3 * (tap / 3);
            const float y = (float)(by + ky * a.dh) + rdy[k];
            const float x = (float)(bx + kx * a.dw) + rdx[k];
            const float fy = floorf(y), fx = floorf(x);
            ly[k] = y - fy;
            lx[k] = x - fx;
            mm[k] = rm[k];
            // Clamped so both rows/columns of the corner pair stay in the padded plane.
            iy[k] = (int)__builtin_amdgcn_fmed3f(fy, (float)-kPad, (float)a.H);
            ix[k] = (int)__builtin_amdgcn_fmed3f(fx, (float)-kPad, (float)a.W);
            const int g0 = unit_group<GPS>(2 * k), g1 = unit_group<GPS>(2 * k + 1);
            if (g0 == g1) {
                bmin_y[g0] = min(bmin_y[g0], iy[k]);
                bmax_y[g0] = max(bmax_y[g0], iy[k]);
                bmin_x[g0] = min(bmin_x[g0], ix[k]);
                bmax_x[g0] = max(bmax_x[g0], ix[k]);
            } else {  // the K-step straddles the two groups of the stage
                bmin_y[g0] = min(bmin_y[g0], half ? INT_MAX : iy[k]);
                bmax_y[g0] = max(bmax_y[g0], half ? INT_MIN : iy[k]);
                bmin_x[g0] = min(bmin_x[g0], half ? INT_MAX : ix[k]);
                bmax_x[g0] = max(bmax_x[g0], half ? INT_MIN : ix[k]);
                bmin_y[g1] = min(bmin_y[g1], half ? iy[k] : INT_MAX);
                bmax_y[g1] = max(bmax_y[g1], half ? iy[k] : INT_MIN);
                bmin_x[g1] = min(bmin_x[g1], half ? ix[k] : INT_MAX);
                bmax_x[g1] = max(bmax_x[g1], half ? ix[k] : INT_MIN);
            }
        }
    };
    auto publish_box = [&](int slot) {
#pragma unroll
        for (int g = 0; g < GPS; ++g) {
            const int v0 = __ockl_wfred_min_i32(bmin_y[g]);
            const int v1 = __ockl_wfred_max_i32(bmax_y[g]);
            const int v2 = __ockl_wfred_min_i32(bmin_x[g]);
            const int v3 = __ockl_wfred_max_i32(bmax_x[g]);
            if (lane == 0) {
                int* sb = box + ((slot * GPS + g) * NW + wave) * 4;
                sb[0] = v0;
                sb[1] = v1;
                sb[2] = v2;
                sb[3] = v3;
            }
        }
    };

    struct Win {
        int y0, x0, ww, hh;
        bool in_lds;
    };
    auto read_box = [&](int slot, int g) {
        int ymin = INT_MAX, ymax = INT_MIN, xmin = INT_MAX, xmax = INT_MIN;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int4 v = *reinterpret_cast<const int4*>(box + ((slot * GPS + g) * NW + w) * 4);
            ymin = min(ymin, v.x);
            ymax = max(ymax, v.y);
            xmin = min(xmin, v.z);
            xmax = max(xmax, v.w);
        }
        Win win;
        win.y0 = ymin;
        win.x0 = xmin;
        win.ww = xmax - xmin + 2;
        win.hh = ymax - ymin + 2;
        win.in_lds = win.hh * win.ww * 16 <= WIN;
        return win;
    };

    // Copy a window of group `grp` into buffer slot/g. Branch-free: the tail lanes
    // recopy the last position into itself.
    auto copy_window = [&](int grp, const Win& w, uint8_t* dst) {
        if (!w.in_lds) return;
        const int count = w.hh * w.ww;
        const uint32_t plane_row0 = (uint32_t)(b * a.CBLK + grp) * a.Hp + (uint32_t)(w.y0 + kPad);
        const float inv_ww = 1.0f / (float)w.ww;
        for (int c0 = 0; c0 < count; c0 += T * CPT) {
            u32x4 v[CPT];
            int cc[CPT];
#pragma unroll
            for (int i = 0; i < CPT; ++i) {
                const int c = min(c0 + i * T + tid, count - 1);
                int r = (int)((float)c * inv_ww);
                r -= (r * w.ww > c) ? 1 : 0;
                r += ((r + 1) * w.ww <= c) ? 1 : 0;
                const int col = c - r * w.ww;
                const uint32_t gpos = (plane_row0 + (uint32_t)r) * a.Wp + (uint32_t)(w.x0 + col + kPad);
                cc[i] = c;
                v[i] = load16(xr, gpos * 16u, 0);
            }
#pragma unroll
            for (int i = 0; i < CPT; ++i) *reinterpret_cast<u32x4*>(dst + (size_t)cc[i] * 16) = v[i];
        }
    };

    f32x16 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x16{};

    // B fragments in a ring of kBDepth K-steps: step k's fragment is requested kBDepth
    // steps before it is used, across the stage boundary (the window copy hides it).
    // A slot must hold the same K-step of every stage, so the depth divides KS: 3 of the 9
    // K-steps of two groups per stage, all 5 of one group per stage.
    constexpr int kBDepth = KS % 3 == 0 ? 3 : KS;
    h8 Bq[kBDepth][NB];
    auto load_b = [&](int slot, int st, int k) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            Bq[slot][nb] = __builtin_bit_cast(
                h8, load16(wr, (uint32_t)(((st * KS + k) * NB + nb) * 64 + lane) * 16u, 0));
    };

    // ---- prologue: stage 0 ----
    load_raw(0);
    make_state();
    publish_box(0);
#pragma unroll
    for (int j = 0; j < kBDepth; ++j) load_b(j, 0, j);
    __syncthreads();
    Win win[GPS];
#pragma unroll
    for (int g = 0; g < GPS; ++g) {
        win[g] = read_box(0, g);
        copy_window(g, win[g], lds + (size_t)g * WIN);
    }
    __syncthreads();

    for (int st = 0; st < stages; ++st) {
        const int buf = st & 1;
        const bool more = st + 1 < stages;
        // Prefetch the next stage's offsets; this stage's sample state stays in iy..mm
        // until make_state() rebuilds it after the multiply.
        if (more) load_raw(st + 1);

        // UNI: when every window of the stage is in LDS, a K-loop with no global fallback,
        // so no wait on outstanding vector loads before the corner reads. Its registers
        // need the two-waves-per-SIMD bound above (otherwise one wave per SIMD).
        bool all_lds = UNI != 0;
#pragma unroll
        for (int g = 0; g < GPS; ++g) all_lds = all_lds && win[g].in_lds;
        if (all_lds && !SPLIT) {
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                const int g0 = unit_group<GPS>(2 * k), g1 = unit_group<GPS>(2 * k + 1);
                const int gi = (g0 == g1) ? g0 : half;
                const Win& w = (g0 == g1) ? win[g0] : (half ? win[g1] : win[g0]);
                const uint8_t* base = lds + (size_t)((NBUF == 2 ? buf : 0) * GPS + gi) * WIN;
                const int idx = (iy[k] - w.y0) * w.ww + (ix[k] - w.x0);
                const uint8_t* p = base + (size_t)idx * 16;
                const u32x4 q00 = *reinterpret_cast<const u32x4*>(p);
                const u32x4 q01 = *reinterpret_cast<const u32x4*>(p + 16);
                const u32x4 q10 = *reinterpret_cast<const u32x4*>(p + (size_t)w.ww * 16);
                const u32x4 q11 = *reinterpret_cast<const u32x4*>(p + (size_t)w.ww * 16 + 16);
                h8 A = blend<SAMPLER>(q00, q01, q10, q11, ly[k], lx[k], mm[k]);
                if (GPS == 1 && k == KS - 1 && half) A = h8{};  // the zero tenth unit
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    acc[nb] = mfma32(A, Bq[k % kBDepth][nb], acc[nb]);
                if (k + kBDepth < KS) load_b(k % kBDepth, st, k + kBDepth);
                else if (more) load_b(k % kBDepth, st + 1, k + kBDepth - KS);
                __builtin_amdgcn_sched_barrier(0);  // keep K-steps apart (register pressure)
            }
        } else
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const int g0 = unit_group<GPS>(2 * k), g1 = unit_group<GPS>(2 * k + 1);
            const int gi = (g0 == g1) ? g0 : half;  // group of this lane's unit within the stage
            const Win& w = (g0 == g1) ? win[g0] : (half ? win[g1] : win[g0]);
            const int grp = st * GPS + gi;
            u32x4 q00, q01, q10, q11;
            const uint32_t gbase =
                ((uint32_t)(b * a.CBLK + grp) * a.Hp + (uint32_t)(iy[k] + kPad)) * a.Wp +
                (uint32_t)(ix[k] + kPad);
            if (w.in_lds) {
                const uint8_t* base = lds + (size_t)((NBUF == 2 ? buf : 0) * GPS + gi) * WIN;
                const int idx = (iy[k] - w.y0) * w.ww + (ix[k] - w.x0);
                const uint8_t* p = base + (size_t)idx * 16;
                q00 = *reinterpret_cast<const u32x4*>(p);
                q01 = *reinterpret_cast<const u32x4*>(p + 16);
                if (SPLIT) {
                    q10 = load16(xr, (gbase + a.Wp) * 16u, 0);
                    q11 = load16(xr, (gbase + a.Wp) * 16u + 16u, 0);
                } else {
                    q10 = *reinterpret_cast<const u32x4*>(p + (size_t)w.ww * 16);
                    q11 = *reinterpret_cast<const u32x4*>(p + (size_t)w.ww * 16 + 16);
                }
            } else {
                q00 = load16(xr, gbase * 16u, 0);
                q01 = load16(xr, gbase * 16u + 16u, 0);
                q10 = load16(xr, (gbase + a.Wp) * 16u, 0);
                q11 = load16(xr, (gbase + a.Wp) * 16u + 16u, 0);
            }
            h8 A = blend<SAMPLER>(q00, q01, q10, q11, ly[k], lx[k], mm[k]);
            if (GPS == 1 && k == KS - 1 && half) A = h8{};  // the zero tenth unit
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                acc[nb] = mfma32(A, Bq[k % kBDepth][nb], acc[nb]);
            if (k + kBDepth < KS) load_b(k % kBDepth, st, k + kBDepth);
            else if (more) load_b(k % kBDepth, st + 1, k + kBDepth - KS);
        }

        if (more) {
            make_state();
            publish_box(buf ^ 1);
            __syncthreads();  // boxes of stage st+1 visible; every wave is past its multiply
#pragma unroll
            for (int g = 0; g < GPS; ++g) {
                win[g] = read_box(buf ^ 1, g);
                copy_window((st + 1) * GPS + g, win[g],
                            lds + (size_t)((NBUF == 2 ? (buf ^ 1) : 0) * GPS + g) * WIN);
            }
            __syncthreads();  // windows of stage st+1 complete
        }
    }

    // ---- epilogue: bias, FP16, coalesced NCHW stores through LDS ----
    __syncthreads();
    uint16_t* stage = reinterpret_cast<uint16_t*>(lds) + (size_t)wave * 32 * NB * 32;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int oc = nb * 32 + (lane & 31);
        const float bias = a.bias[oc];
#pragma unroll
        for (int k = 0; k < 4; ++k) {  // row-block pixels 8 k + 4 half .. + 3: one 8-byte write
            uint32_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                h[e] = kBf16 ? round_bf16_bits(acc[nb][4 * k + e] + bias)
                             : __builtin_bit_cast(uint16_t, round_f16(acc[nb][4 * k + e] + bias));
            *reinterpret_cast<uint2*>(stage + oc * 32 + 8 * k + 4 * half) =
                make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
        }
    }
    __syncthreads();
    if (oy_row < a.Ho) {
        for (int idx = lane; idx < NB * 32 * 8; idx += 64) {
            const int oc = idx >> 3;
            const int q = (idx & 7) * 4;
            const uint16_t* src = stage + oc * 32 + q;
            uint16_t* dst = a.out + ((size_t)b * a.Cout + oc) * a.HWo + (size_t)oy_row * a.Wo + ox0 + q;
            if (ox0 + q + 3 < a.Wo && ((((uintptr_t)dst) & 7u) == 0)) {
                *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(src);
            } else if (ox0 + q + 3 < a.Wo && ((((uintptr_t)dst) & 3u) == 0)) {
                reinterpret_cast<uint32_t*>(dst)[0] = (uint32_t)src[0] | ((uint32_t)src[1] << 16);
                reinterpret_cast<uint32_t*>(dst)[1] = (uint32_t)src[2] | ((uint32_t)src[3] << 16);
            } else {
                for (int e = 0; e < 4; ++e)
                    if (ox0 + q + e < a.Wo) dst[e] = src[e];
            }
        }
    }
}

// ---- asynchronous window pipeline (LDS DMA) ------------------------------------------
// Same K order, tiles and weights as window_kernel with GPS = 2, one workgroup of eight
// waves per CU on an 8 x 32 tile, but the copies run in the background: while stage s is
// multiplied from LDS, global_load_lds_dwordx4 streams stage s+1's two input windows and
// its 18 KB of B fragments straight into the other half of a double buffer (no VGPRs, no
// LDS store instructions), and the offsets of stage s+2 are loaded. The stage loop then
// reads only LDS, so the copy latency that bounds window_kernel is hidden behind the
// multiply. B fragments come from LDS once per workgroup instead of once per wave.

// 64 lanes x 16 bytes from `g` (one per lane) into LDS [dst, dst + 1 KB) at dst + lane * 16,
// as one global_load_lds_dwordx4. dst is wave-uniform; the compiler sets M0 from it. The
// caller keeps every g inside its buffer and waits with wait_dma() before reading.
__device__ __forceinline__ void dma16(const void* g, uint8_t* dst) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}
__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0); }

constexpr int kAsyncNw = 8;     // waves per workgroup = tile rows
constexpr int kAsyncLds = 160 * 1024;
template <int NB>
struct AsyncLayout {
    static constexpr int kStageB = 9 * NB * 1024;  // B fragments of one stage
    static constexpr int kBox = 2 * 2 * kAsyncNw * 4 * (int)sizeof(int);
    static constexpr int kWin = ((kAsyncLds - 2 * kStageB - kBox) / 4) & ~1023;  // bytes per window
    static constexpr int kBufB = 4 * kWin;           // offset of the B double buffer
    static constexpr int kBoxes = kBufB + 2 * kStageB;
    static constexpr int kBytes = kBoxes + kBox;
};

template <int NB, int SAMPLER>
__global__ __launch_bounds__(64 * kAsyncNw) void window_async_kernel(WindowArgs a) {
    using L = AsyncLayout<NB>;
    constexpr int NW = kAsyncNw, GPS = 2, KS = 9;
    static_assert(L::kBytes <= kAsyncLds && L::kWin >= 8 * 1024, "LDS plan");
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    int* box = reinterpret_cast<int*>(lds + L::kBoxes);  // [2][GPS][NW][4]
    auto win_buf = [&](int buf, int g) { return lds + (buf * GPS + g) * L::kWin; };
    auto b_buf = [&](int buf) { return lds + L::kBufB + buf * L::kStageB; };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;

    const int per_xcd = (a.tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= a.tiles) return;  // whole workgroup, before any barrier
    const int tiles_img = a.tiles_y * a.tiles_x;
    const int b = tile / tiles_img;
    const int trem = tile - b * tiles_img;
    const int ty = trem / a.tiles_x;
    const int tx = trem - ty * a.tiles_x;
    const int oy_row = ty * NW + wave;
    const int ox0 = tx * 32;
    const int oyc = min(oy_row, a.Ho - 1);
    const int oxc = min(ox0 + (lane & 31), a.Wo - 1);
    const int sp = oyc * a.Wo + oxc;

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xin, a.xin_bytes);
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.off, a.off_bytes);
    const __amdgpu_buffer_rsrc_t mr = make_rsrc(a.msk, a.msk_bytes);
    const uint8_t* xin = static_cast<const uint8_t*>(a.xin);
    const uint8_t* wpk = static_cast<const uint8_t*>(a.wpk);

    const uint32_t hwo2 = (uint32_t)a.HWo * 2u;
    const int by = oyc * a.sh - a.ph;
    const int bx = oxc * a.sw - a.pw;
    const uint32_t off_lane = ((uint32_t)b * 2 * a.G * 9 * a.HWo + sp) * 2u;
    const uint32_t msk_lane = ((uint32_t)b * a.G * 9 * a.HWo + sp) * 2u;
    const int stages = a.G / GPS;

    auto unit_of = [&](int k, int& tap, int& go) {
        tap = half ? unit_tap<GPS>(2 * k + 1) : unit_tap<GPS>(2 * k);
        go = half ? unit_group<GPS>(2 * k + 1) : unit_group<GPS>(2 * k);
    };
    float rdy[KS], rdx[KS], rm[KS];
    auto load_raw = [&](int st) {
        const uint32_t so = 2u * (uint32_t)(st * GPS * 9) * hwo2;
        const uint32_t sm = (uint32_t)(st * GPS * 9) * hwo2;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            int tap, go;
            unit_of(k, tap, go);
            const uint32_t ch = (uint32_t)(go * 9 + tap);
            rdy[k] = load_half(orr, off_lane + 2u * ch * hwo2, so);
            rdx[k] = load_half(orr, off_lane + (2u * ch + 1u) * hwo2, so);
            rm[k] = load_half(mr, msk_lane + ch * hwo2, sm);
        }
    };
    // Sample state of a stage (from rdy/rdx/rm) and the bounding box of its corners.
    int iy[KS], ix[KS], niy[KS], nix[KS];
    float ly[KS], lx[KS], mm[KS], nly[KS], nlx[KS], nmm[KS];
    int bmin_y[GPS], bmax_y[GPS], bmin_x[GPS], bmax_x[GPS];
    auto make_next_state = [&]() {
#pragma unroll
        for (int g = 0; g < GPS; ++g) {
            bmin_y[g] = INT_MAX;
            bmax_y[g] = INT_MIN;
            bmin_x[g] = INT_MAX;
            bmax_x[g] = INT_MIN;
        }
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            int tap, go;
            unit_of(k, tap, go);
            const int ky = tap / 3, kx = tap - 3 * (tap / 3);
            const float y = (float)(by + ky * a.dh) + rdy[k];
            const float x = (float)(bx + kx * a.dw) + rdx[k];
            const float fy = floorf(y), fx = floorf(x);
            nly[k] = y - fy;
            nlx[k] = x - fx;
            nmm[k] = rm[k];
            niy[k] = (int)__builtin_amdgcn_fmed3f(fy, (float)-kPad, (float)a.H);
            nix[k] = (int)__builtin_amdgcn_fmed3f(fx, (float)-kPad, (float)a.W);
            const int g0 = unit_group<GPS>(2 * k), g1 = unit_group<GPS>(2 * k + 1);
            if (g0 == g1) {
                bmin_y[g0] = min(bmin_y[g0], niy[k]);
                bmax_y[g0] = max(bmax_y[g0], niy[k]);
                bmin_x[g0] = min(bmin_x[g0], nix[k]);
                bmax_x[g0] = max(bmax_x[g0], nix[k]);
            } else {
                bmin_y[g0] = min(bmin_y[g0], half ? INT_MAX : niy[k]);
                bmax_y[g0] = max(bmax_y[g0], half ? INT_MIN : niy[k]);
                bmin_x[g0] = min(bmin_x[g0], half ? INT_MAX : nix[k]);
                bmax_x[g0] = max(bmax_x[g0], half ? INT_MIN : nix[k]);
                bmin_y[g1] = min(bmin_y[g1], half ? niy[k] : INT_MAX);
                bmax_y[g1] = max(bmax_y[g1], half ? niy[k] : INT_MIN);
                bmin_x[g1] = min(bmin_x[g1], half ? nix[k] : INT_MAX);
                bmax_x[g1] = max(bmax_x[g1], half ? nix[k] : INT_MIN);
            }
        }
    };
    auto take_next_state = [&]() {
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            iy[k] = niy[k];
            ix[k] = nix[k];
            ly[k] = nly[k];
            lx[k] = nlx[k];
            mm[k] = nmm[k];
        }
    };
    auto publish_box = [&](int slot) {
#pragma unroll
        for (int g = 0; g < GPS; ++g) {
            const int v0 = __ockl_wfred_min_i32(bmin_y[g]);
            const int v1 = __ockl_wfred_max_i32(bmax_y[g]);
            const int v2 = __ockl_wfred_min_i32(bmin_x[g]);
            const int v3 = __ockl_wfred_max_i32(bmax_x[g]);
            if (lane == 0) {
                int* sb = box + ((slot * GPS + g) * NW + wave) * 4;
                sb[0] = v0;
                sb[1] = v1;
                sb[2] = v2;
                sb[3] = v3;
            }
        }
    };
    struct Win {
        int y0, x0, ww, hh;
        bool in_lds;
    };
    auto read_box = [&](int slot, int g) {
        int ymin = INT_MAX, ymax = INT_MIN, xmin = INT_MAX, xmax = INT_MIN;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int4 v = *reinterpret_cast<const int4*>(box + ((slot * GPS + g) * NW + w) * 4);
            ymin = min(ymin, v.x);
            ymax = max(ymax, v.y);
            xmin = min(xmin, v.z);
            xmax = max(xmax, v.w);
        }
        Win w;
        w.y0 = ymin;
        w.x0 = xmin;
        w.ww = xmax - xmin + 2;
        w.hh = ymax - ymin + 2;
        // whole 64-chunk blocks: the last block's tail lanes land in the window's slack
        w.in_lds = ((w.hh * w.ww + 63) / 64) * 1024 <= L::kWin;
        return w;
    };
    // Background copies of a stage: its two windows (if they fit) and its B fragments.
    // Block j of 64 chunks goes to wave j % NW. Every source address lies inside the
    // CB8 input (the box is clamped into the padded plane) or the packed weights.
    auto dma_stage = [&](int st, int buf, const Win (&w)[GPS]) {
#pragma unroll
        for (int g = 0; g < GPS; ++g) {
            if (!w[g].in_lds) continue;
            const int count = w[g].hh * w[g].ww;
            const int blocks = (count + 63) / 64;
            const uint32_t row0 = (uint32_t)(b * a.CBLK + st * GPS + g) * a.Hp + (uint32_t)(w[g].y0 + kPad);
            const float inv_ww = 1.0f / (float)w[g].ww;
            uint8_t* dst = win_buf(buf, g);
            for (int j = wave; j < blocks; j += NW) {
                const int c = min(j * 64 + lane, count - 1);
                int r = (int)((float)c * inv_ww);
                r -= (r * w[g].ww > c) ? 1 : 0;
                r += ((r + 1) * w[g].ww <= c) ? 1 : 0;
                const int col = c - r * w[g].ww;
                const uint32_t unit = (row0 + (uint32_t)r) * a.Wp + (uint32_t)(w[g].x0 + col + kPad);
                dma16(xin + (size_t)unit * 16, dst + j * 1024);
            }
        }
        const uint8_t* src = wpk + (size_t)st * L::kStageB;
        uint8_t* dst = b_buf(buf);
        for (int j = wave; j < 9 * NB; j += NW)
            dma16(src + (size_t)j * 1024 + (size_t)lane * 16, dst + j * 1024);
    };

    f32x16 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x16{};

    // ---- prologue: stage 0 state and copies, stage 1 offsets ----
    load_raw(0);
    make_next_state();
    take_next_state();
    publish_box(0);
    __syncthreads();
    Win win[GPS];
#pragma unroll
    for (int g = 0; g < GPS; ++g) win[g] = read_box(0, g);
    dma_stage(0, 0, win);
    if (stages > 1) load_raw(1);

    for (int st = 0; st < stages; ++st) {
        const int buf = st & 1;
        const bool more = st + 1 < stages;
        // Stage st's copies and stage st+1's offsets have landed.
        wait_dma();
        Win cur[GPS];
#pragma unroll
        for (int g = 0; g < GPS; ++g) cur[g] = win[g];
        if (more) {
            make_next_state();
            publish_box(buf ^ 1);
        }
        // Copies of stage st visible to all waves; every wave is done with stage st-1,
        // whose buffers the next copies overwrite.
        __syncthreads();
        if (more) {
#pragma unroll
            for (int g = 0; g < GPS; ++g) win[g] = read_box(buf ^ 1, g);
            dma_stage(st + 1, buf ^ 1, win);
            if (st + 2 < stages) load_raw(st + 2);
        }

        const uint8_t* bsrc = b_buf(buf);
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const int g0 = unit_group<GPS>(2 * k), g1 = unit_group<GPS>(2 * k + 1);
            const int gi = (g0 == g1) ? g0 : half;
            const Win& w = (g0 == g1) ? cur[g0] : (half ? cur[g1] : cur[g0]);
            u32x4 q0, q1, q2, q3;
            if (w.in_lds) {
                // 0 <= iy - y0 < hh and 0 <= ix - x0 < ww by construction of the box.
                const uint8_t* p = win_buf(buf, gi) +
                                   (size_t)((iy[k] - w.y0) * w.ww + (ix[k] - w.x0)) * 16;
                q0 = *reinterpret_cast<const u32x4*>(p);
                q1 = *reinterpret_cast<const u32x4*>(p + 16);
                q2 = *reinterpret_cast<const u32x4*>(p + (size_t)w.ww * 16);
                q3 = *reinterpret_cast<const u32x4*>(p + (size_t)w.ww * 16 + 16);
            } else {
                const uint32_t g = ((uint32_t)(b * a.CBLK + st * GPS + gi) * a.Hp + (uint32_t)(iy[k] + kPad)) *
                                       a.Wp + (uint32_t)(ix[k] + kPad);
                q0 = load16(xr, g * 16u, 0);
                q1 = load16(xr, g * 16u + 16u, 0);
                q2 = load16(xr, (g + a.Wp) * 16u, 0);
                q3 = load16(xr, (g + a.Wp) * 16u + 16u, 0);
            }
            const h8 A = blend<SAMPLER>(q0, q1, q2, q3, ly[k], lx[k], mm[k]);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const h8 B = *reinterpret_cast<const h8*>(bsrc + ((k * NB + nb) * 64 + lane) * 16);
                acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A, B, acc[nb], 0, 0, 0);
            }
        }
        if (more) take_next_state();
    }

    // ---- epilogue: bias, FP16, coalesced NCHW stores through LDS ----
    __syncthreads();
    uint16_t* stage = reinterpret_cast<uint16_t*>(lds) + (size_t)wave * 32 * NB * 32;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int oc = nb * 32 + (lane & 31);
        const float bias = a.bias[oc];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int i = 8 * (v >> 2) + 4 * half + (v & 3);
            stage[oc * 32 + i] = __builtin_bit_cast(uint16_t, round_f16(acc[nb][v] + bias));
        }
    }
    __syncthreads();
    if (oy_row < a.Ho) {
        for (int idx = lane; idx < NB * 32 * 8; idx += 64) {
            const int oc = idx >> 3;
            const int q = (idx & 7) * 4;
            const uint16_t* src = stage + oc * 32 + q;
            uint16_t* dst = a.out + ((size_t)b * a.Cout + oc) * a.HWo + (size_t)oy_row * a.Wo + ox0 + q;
            if (ox0 + q + 3 < a.Wo && ((((uintptr_t)dst) & 3u) == 0)) {
                reinterpret_cast<uint32_t*>(dst)[0] = (uint32_t)src[0] | ((uint32_t)src[1] << 16);
                reinterpret_cast<uint32_t*>(dst)[1] = (uint32_t)src[2] | ((uint32_t)src[3] << 16);
            } else {
                for (int e = 0; e < 4; ++e)
                    if (ox0 + q + e < a.Wo) dst[e] = src[e];
            }
        }
    }
}

template <int NB, int SAMPLER>
hipError_t launch_window_async_t(const WindowArgs& a, hipStream_t stream) {
    auto kernel = &window_async_kernel<NB, SAMPLER>;
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), AsyncLayout<NB>::kBytes);
    if (attr != hipSuccess) return attr;
    const unsigned grid = (unsigned)(((a.tiles + 7) / 8) * 8);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kAsyncNw), AsyncLayout<NB>::kBytes, stream, a);
    return hipGetLastError();
}

// Weights -> B fragments [stages][KS][NB][64][8] for window_kernel: lane l of K-step k
// of stage st holds unit u = 2k + l/32 (group st*GPS + u/9 (GPS 2) or st (GPS 1), tap
// u%9; zero for the padding unit 9 of GPS 1) of output channel nb*32 + l%32, channels
// group*8 .. group*8+7.
__global__ __launch_bounds__(256) void prepack_group_kernel(const uint16_t* __restrict__ w, int layout,
                                                            uint16_t* __restrict__ wpk, int Cin,
                                                            int Cout, int NB, int gps, long total) {
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    const int ks = gps == 2 ? 9 : 5;
    const int e = (int)(gid & 7);
    const int lane = (int)((gid >> 3) & 63);
    long q = gid >> 9;
    const int nb = (int)(q % NB);
    q /= NB;
    const int k = (int)(q % ks);
    const int st = (int)(q / ks);
    const int u = 2 * k + (lane >> 5);
    const int grp = gps == 2 ? st * 2 + (u >= 9 ? 1 : 0) : st;
    const int tap = gps == 2 ? (u >= 9 ? u - 9 : u) : u;
    const int oc = nb * 32 + (lane & 31);
    const int ic = grp * 8 + e;
    uint16_t v = 0;
    if (tap < 9 && oc < Cout && ic < Cin)
        v = layout == DCN_LAYOUT_OIHW ? w[((size_t)oc * Cin + ic) * 9 + tap]
                                      : w[((size_t)ic * 9 + tap) * Cout + oc];
    wpk[gid] = v;
}

template <int NB, int NW, int TR, int GPS, int SAMPLER, int SPLIT>
hipError_t launch_window_t(const WindowArgs& a, hipStream_t stream) {
    constexpr int NBUF = NW == 8 ? 2 : 1;
    const size_t lds = (size_t)window_lds(NBUF) + 2 * GPS * NW * 4 * sizeof(int);
    // The uniform LDS K-loop for batches of small maps (C3's 16 tiles: 58.0 -> 55.1 us),
    // where the windows of a stage almost always fit; large maps with large flows (C5:
    // windows over its LDS budget in many stages) keep the single loop (71.1 us there,
    // 74.1 us with the uniform loop's code beside it).
    constexpr bool kUniOk = NW == 4 && GPS == 2 && SPLIT == 0;
    auto kernel = &window_kernel<NB, NW, TR, GPS, SAMPLER, SPLIT, NBUF, 0>;
    if constexpr (kUniOk) {
        if (a.B > 1 && a.H * a.W <= 64 * 64) kernel = &window_kernel<NB, NW, TR, GPS, SAMPLER, SPLIT, NBUF, 1>;
    }
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), (int)lds);
    if (attr != hipSuccess) return attr;
    const unsigned grid = (unsigned)(((a.tiles + 7) / 8) * 8);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * NW), lds, stream, a);
    return hipGetLastError();
}

template <int NW, int TR, int GPS, int SAMPLER, int SPLIT>
hipError_t launch_window_nb(const WindowArgs& a, int nb, hipStream_t stream) {
    switch (nb) {
        case 1: return launch_window_t<1, NW, TR, GPS, SAMPLER, SPLIT>(a, stream);
        case 2: return launch_window_t<2, NW, TR, GPS, SAMPLER, SPLIT>(a, stream);
        case 3: return launch_window_t<3, NW, TR, GPS, SAMPLER, SPLIT>(a, stream);
        case 4: return launch_window_t<4, NW, TR, GPS, SAMPLER, SPLIT>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int GPS, int SAMPLER, int SPLIT>
hipError_t launch_window_g(const WindowArgs& a, int nb, int nw, int tr, hipStream_t stream) {
    if (nw == 8 && tr == 8) return launch_window_nb<8, 8, GPS, SAMPLER, SPLIT>(a, nb, stream);
    if (nw == 8 && tr == 4) return launch_window_nb<8, 4, GPS, SAMPLER, SPLIT>(a, nb, stream);
    if (nw == 4 && tr == 4) return launch_window_nb<4, 4, GPS, SAMPLER, SPLIT>(a, nb, stream);
    if (nw == 4 && tr == 2) return launch_window_nb<4, 2, GPS, SAMPLER, SPLIT>(a, nb, stream);
    return hipErrorInvalidValue;
}

}  // namespace

bool window_supported(const dcn_shape& s) {
    return s.groups == 1 && s.kernel_height == 3 && s.kernel_width == 3 &&
           s.input_channels == 8 * s.offset_groups && s.output_channels % 32 == 0 &&
           s.output_channels <= 128;
}

int window_gps(const dcn_shape& s) { return s.offset_groups % 2 == 0 ? 2 : 1; }

size_t window_packed_bytes(const dcn_shape& s) {
    const int gps = window_gps(s);
    const int ks = gps == 2 ? 9 : 5;
    return (size_t)(s.offset_groups / gps) * ks * (s.output_channels / 32) * 64 * 8 * sizeof(uint16_t);
}

hipError_t launch_prepack_group(const KShape& s, const uint16_t* w, int layout, void* wpk,
                                hipStream_t stream) {
    dcn_shape shape{s.B, s.Cin, s.H, s.W, s.Cout, s.Ho, s.Wo, s.KH, s.KW, s.ph, s.pw,
                    s.sh, s.sw, s.dh, s.dw, s.groups, s.og};
    const int gps = window_gps(shape);
    const int nb = s.Cout / 32;
    const long total = (long)(window_packed_bytes(shape) / sizeof(uint16_t));
    const long grid = (total + 255) / 256;
    hipLaunchKernelGGL(prepack_group_kernel, dim3((unsigned)grid), dim3(256), 0, stream, w, layout,
                       (uint16_t*)wpk, s.Cin, s.Cout, nb, gps, total);
    return hipGetLastError();
}

hipError_t launch_window_f16(const KShape& s, const FusedGeometry& g, const FusedConfig& cfg,
                             const void* cb8, const uint16_t* off, const uint16_t* mask,
                             const void* packed_w, const float* packed_b, uint16_t* out,
                             hipStream_t stream) {
    WindowArgs a;
    a.xin = cb8;
    a.off = off;
    a.msk = mask;
    a.wpk = packed_w;
    a.bias = packed_b;
    a.out = out;
    const size_t hwo = (size_t)s.Ho * s.Wo;
    dcn_shape shape{s.B, s.Cin, s.H, s.W, s.Cout, s.Ho, s.Wo, s.KH, s.KW, s.ph, s.pw,
                    s.sh, s.sw, s.dh, s.dw, s.groups, s.og};
    a.xin_bytes = (uint32_t)((size_t)s.B * g.cblk * g.hp * g.wp * 16);
    a.off_bytes = (uint32_t)((size_t)s.B * 2 * s.og * 9 * hwo * 2);
    a.msk_bytes = (uint32_t)((size_t)s.B * s.og * 9 * hwo * 2);
    a.wpk_bytes = (uint32_t)window_packed_bytes(shape);
    a.B = s.B;
    a.H = s.H;
    a.W = s.W;
    a.Ho = s.Ho;
    a.Wo = s.Wo;
    a.HWo = (int)hwo;
    a.ph = s.ph;
    a.pw = s.pw;
    a.sh = s.sh;
    a.sw = s.sw;
    a.dh = s.dh;
    a.dw = s.dw;
    a.G = s.og;
    a.CBLK = g.cblk;
    a.Hp = g.hp;
    a.Wp = g.wp;
    a.Cout = s.Cout;
    if (cfg.variant == kVariantWindowAsync) {
        if (window_gps(shape) != 2) return hipErrorInvalidValue;
        a.tiles_y = (s.Ho + kAsyncNw - 1) / kAsyncNw;
        a.tiles_x = (s.Wo + 31) / 32;
        a.tiles = a.tiles_y * a.tiles_x * s.B;
        const bool exact = cfg.sampler == kSamplerExact;
        switch (g.nb) {
            case 1: return exact ? launch_window_async_t<1, kSamplerExact>(a, stream)
                                 : launch_window_async_t<1, kSamplerFast>(a, stream);
            case 2: return exact ? launch_window_async_t<2, kSamplerExact>(a, stream)
                                 : launch_window_async_t<2, kSamplerFast>(a, stream);
            case 3: return exact ? launch_window_async_t<3, kSamplerExact>(a, stream)
                                 : launch_window_async_t<3, kSamplerFast>(a, stream);
            case 4: return exact ? launch_window_async_t<4, kSamplerExact>(a, stream)
                                 : launch_window_async_t<4, kSamplerFast>(a, stream);
            default: return hipErrorInvalidValue;
        }
    }
    const int nw = cfg.ks;
    const int tr = cfg.mt;  // for the window variant, mt carries the tile rows
    const int tcb = nw / tr;
    a.tiles_y = (s.Ho + tr - 1) / tr;
    a.tiles_x = (s.Wo + 32 * tcb - 1) / (32 * tcb);
    a.tiles = a.tiles_y * a.tiles_x * s.B;
    const int gps = window_gps(shape);
    const bool split = cfg.split != 0;
    if (cfg.sampler == kSamplerBf16) {  // BF16: 4 x 32 tiles on 4 waves, one window per group
        if (nw != 4 || tr != 4 || split) return hipErrorInvalidValue;
        return gps == 2 ? launch_window_nb<4, 4, 2, kSamplerBf16, 0>(a, g.nb, stream)
                        : launch_window_nb<4, 4, 1, kSamplerBf16, 0>(a, g.nb, stream);
    }
    if (cfg.sampler == kSamplerExact) {
        if (gps == 2) return split ? launch_window_g<2, kSamplerExact, 1>(a, g.nb, nw, tr, stream)
                                   : launch_window_g<2, kSamplerExact, 0>(a, g.nb, nw, tr, stream);
        return split ? launch_window_g<1, kSamplerExact, 1>(a, g.nb, nw, tr, stream)
                     : launch_window_g<1, kSamplerExact, 0>(a, g.nb, nw, tr, stream);
    }
    if (gps == 2) return split ? launch_window_g<2, kSamplerFast, 1>(a, g.nb, nw, tr, stream)
                               : launch_window_g<2, kSamplerFast, 0>(a, g.nb, nw, tr, stream);
    return split ? launch_window_g<1, kSamplerFast, 1>(a, g.nb, nw, tr, stream)
                 : launch_window_g<1, kSamplerFast, 0>(a, g.nb, nw, tr, stream);
}

}  // namespace dcn
