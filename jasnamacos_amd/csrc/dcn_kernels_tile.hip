// Tile-window fused FP16 DCNv2 for gfx950 (3x3 kernels, 8 channels per offset group,
// an even number of offset groups, Cout 32 or 64): batches of maps and large maps.
//
// Why this shape. Measured on MI355X, per CU, with L2-resident data:
//   - random 16-byte gathers through the vector L1: 6.8 B/clk (every lane's corner is
//     its own L2 request, ~2.2 cycles each);
//   - random 16-byte LDS reads: 70 B/clk;
//   - coalesced loads, or LDS DMA into LDS: 35-53 B/clk for the whole CU.
// So the corners are gathered from LDS. The input reaches LDS as a window per offset
// group: the exact bounding box of every corner the tile's samples touch, copied by LDS
// DMA (buffer_load ... lds: no VGPRs, no LDS store instructions).
//
// The L2 -> CU path is then the scarce resource, and it is counted in instructions as
// much as in bytes: 64 addresses take the texture addresser many cycles whatever their
// size. Reading each sample's offsets and mask with 2-byte loads (27 per pixel and stage)
// saturated it and doubled the kernel's time. So a stage's 54 offset and mask channels
// for the tile's 128 pixels (13.5 KB) are copied to LDS by LDS DMA and every lane reads
// its values from there. The path also carries the windows and the weight fragments.
// With one 32-pixel segment per wave, every wave would stream the whole weight set;
// here each wave holds two 32-pixel segments (the MFMA B fragment is used for both) and
// about half the taps of a stage, so each weight fragment crosses the path once per two
// segments, and the two halves of each pixel's sum meet in LDS at the end, in a fixed
// order (the half of waves 0-1 + the half of waves 2-3).
//
// The sampler's VALU is the other limit. One sample (8 channels) feeds 64 output
// channels, i.e. two v_mfma_f32_32x32x16_f16, while its bilinear blend alone is 16 packed
// FP16 instructions. So each sample's coordinates and FP16 corner weights are computed
// once, off the K-loop (inside the previous stage's first K-steps), and the K-loop does
// an address select and the blend.
//
// Layout. Workgroup = 4 waves (kTileWaves) on a 128-pixel tile (kTilePix): 8 x 16 pixels
// (TW = 16) or 4 x 32 (TW = 32). Wave w owns pixel block w & 1 (64 pixels = two segments
// of 32, each 32 / TW tile rows); waves 0-1 take taps 0-3 of both segments and the
// centre tap 4 of the first, waves 2-3 taps 5-8 of both and tap 4 of the second: 9
// samples per lane and stage in every wave. A stage is two offset groups; K-step k of
// stage s is tap k of both: lanes 0-31 give group 2s, lanes 32-63 group 2s+1 (the A
// operand of v_mfma_f32_32x32x16_f16 is 32 pixels x 16 K, 8 per lane), and the weights
// are prepacked in that order (tile_prepack_kernel).
//
// Pipeline (two workgroups per CU, each with one 64 KB window buffer, kTileBuf), stage s:
//   - the K-loop of stage s, whose first two K-steps also compute stage s+1's corner
//     coordinates and bounding box (from s+1's offsets, already in LDS), and which
//     requests stage s+1's weight fragment of each tap as soon as tap k of s is done;
//   - a barrier; the box reduced; stage s+1's windows and stage s+2's offsets requested
//     by LDS DMA (the window buffer is free: every wave is past s's corner reads);
//     s+1's coordinates turned into LDS addresses;
//   - a wait for the DMA and a barrier.
// One workgroup's copies overlap the other workgroup's K-loop on the same CU.
// Vector-memory results return in issue order (one vmcnt counter), so a wait for a
// weight fragment also waits for every older load: each stage's fragments are all in
// registers before the stage starts, so the K-loop never waits on memory.
// A stage whose two windows do not fit the buffer together but each fits alone runs one
// pass per group (the other group's lanes read zeros); a stage with a window larger than
// the buffer gathers from the global CB8 input instead (same arithmetic, no copy), so any
// offset field is handled.
#include <hip/hip_runtime.h>

#include <climits>
#include <type_traits>

#include "dcn_device.hpp"
#include "dcn_internal.hpp"

#pragma clang fp contract(off)

namespace dcn {
namespace {

using namespace dev;

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int kTileWaves = 4;                         // waves per workgroup (2 per CU)
constexpr int kTilePix = 128;                         // pixels per tile
constexpr int kTileBuf = 64 * 1024;                   // the window buffer (a stage)
constexpr int kTileOffCh = 54;                        // offset + mask channels of a stage
constexpr int kTileOff = kTileOffCh * kTilePix * 2;   // [36 dy/dx + 18 mask][128 px] FP16
constexpr int kTileBox = 2 * kTileWaves * 2 * 4;      // [group][wave][min, max]
constexpr int kTileZero = kTileBuf + kTileOff + kTileBox;  // 32 zero bytes (masked lanes' corners)
constexpr int kTileLds = kTileZero + 32;               // 79,456 B: two workgroups per CU
constexpr int kTileMaxSide = 32000;                    // input height / width (16-bit corners)
constexpr int kTileSlots = 5;                          // weight slots per wave and stage
// Pair placement: where every wave's stage-0 weight fragments wait in the window buffer
// (free until stage 0's windows; its first 4 KB hold the waves' estimate channels).
constexpr int kTilePairB = 14 * 1024;
static_assert(kTilePairB >= kTileWaves * 1024 && kTilePairB + kTileWaves * kTileSlots * 2 * 1024 <= kTileBuf,
              "the pair placement's copies fit the window buffer");

struct TileArgs {
    const void* xin;      // CB8 input [B][CBLK][Hp][Wp][8]
    const uint16_t* off;  // [B][2*G*9][HWo]
    const uint16_t* msk;  // [B][G*9][HWo]
    const void* wpk;      // [G/2][9][NB][64][8] FP16 (tile_prepack_kernel)
    const float* bias;    // [Cout]
    uint16_t* out;        // [B][Cout][HWo]
    uint32_t xin_bytes, off_bytes, msk_bytes, wpk_bytes;
    int H, W, Ho, Wo, HWo, ph, pw, sh, sw, dh, dw;
    int G, CBLK, Hp, Wp, Cout;
    float one;  // 1.0f, opaque to the compiler (see coords)
    int tiles_y, tiles_x, tiles;
    int plan;   // 1: planned placement of a band's tiles where it applies: cost-ordered
                // (tile_band_slot, 33-63 tiles) or heavier-of-two first (tile_pair_slot, 64)
    // Per-workgroup clock stamps (diagnostics) or null: workgroup b writes
    // clock[4b .. 4b+3] = {start, end of wave 0, end of wave 1, HW_ID << 32 | XCC_ID << 28 |
    // tile} on the 100 MHz constant clock (s_memrealtime); workgroups without a tile write
    // nothing. (Tiles stay below 2^28: a tensor holds fewer than 2^29 elements.)
    unsigned long long* clock;
};

// 16-byte LDS DMA: unit `voff` of the buffer to LDS lds_base + 16 * lane (lds_base uniform).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint8_t* lds_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)lds_base, 16, (int)voff, 0, 0, 0);
}

// Lane exchange within 32 lanes (ds_swizzle xor patterns stay inside each half-wave).
template <int XOR>
__device__ __forceinline__ uint32_t swz(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x1F | (XOR << 10));
}
__device__ __forceinline__ s16x2 as_s16x2(uint32_t v) { return __builtin_bit_cast(s16x2, v); }
__device__ __forceinline__ uint32_t as_u32(s16x2 v) { return __builtin_bit_cast(uint32_t, v); }
template <int XOR>
__device__ __forceinline__ void box_step(uint32_t& mn, uint32_t& mx) {
    mn = as_u32(__builtin_elementwise_min(as_s16x2(mn), as_s16x2(swz<XOR>(mn))));
    mx = as_u32(__builtin_elementwise_max(as_s16x2(mx), as_s16x2(swz<XOR>(mx))));
}

// Eight channels of one sample: the four FP16 corner weights w00, w01 (in w0) and w10,
// w11 (in w1) applied as packed FP16 FMAs, the fast sampler of the other fused kernels.
__device__ __forceinline__ h8 blend_w(const u32x4 (&q)[4], uint32_t w0, uint32_t w1) {
    const h2 a = __builtin_bit_cast(h2, w0), c = __builtin_bit_cast(h2, w1);
    const h8 w00 = a.x, w01 = a.y, w10 = c.x, w11 = c.y;
    h8 r = w00 * __builtin_bit_cast(h8, q[0]);
    r = __builtin_elementwise_fma(w01, __builtin_bit_cast(h8, q[1]), r);
    r = __builtin_elementwise_fma(w10, __builtin_bit_cast(h8, q[2]), r);
    r = __builtin_elementwise_fma(w11, __builtin_bit_cast(h8, q[3]), r);
    return r;
}

// Placement of a band's tiles on its XCD's CUs. Workgroups are dispatched to an XCD in
// blockIdx order (blockIdx % 8), and within an XCD local index l goes to CU l % 32: with
// n tiles per band, 32 < n < 64, locals l and l + 32 (l < n - 32) share a CU and locals
// n - 32 .. 31 run alone (measured on MI355X with per-workgroup hardware ids). A tile
// whose stages split (windows that do not fit the buffer together) takes 1.2-1.4x the time
// of the others and, when two such tiles share a CU, sets the kernel's time. So the
// band's tiles are ranked by an estimate of their window area, the heaviest take the
// alone slots, and the rest are paired heaviest with lightest.
// The estimate of a tile: the extent of the clamped sample positions of one offset
// channel pair (group 0, centre tap; the offset field's flow part is common to all
// groups and taps, its residue spans the same range in each) over half of the tile's rows
// (the first, the last and evenly spaced ones between): (rows + 3) x (columns + 3). On C5
// it ranks the tiles with a rank correlation of 0.98 to their window bytes (0.99 with
// every row, at twice the loads). Every workgroup of the band reads the same offsets and runs
// the same arithmetic, so all of them compute the same ranking without communicating.
// Returns the band-local index of the tile that local slot `loc` runs. All threads of the
// workgroup call it (it has a barrier); `sh` is 2.5 KB of LDS that nothing else writes
// before the workgroup's next barrier.
template <int TW>
__device__ int tile_band_slot(const TileArgs& a, __amdgpu_buffer_rsrc_t orr, int band0, int n, int loc,
                              float* sh) {
    constexpr int TH = 128 / TW;
    constexpr int kPieces = TW / 8;           // 16-byte pieces of a tile row
    constexpr int kRows = TW == 16 ? 4 : 2;      // rows sampled: 4 of 8 (TW 16), 2 of 4 (TW 32)
    constexpr int kHalf = kRows * kPieces;       // 8: pieces of one channel (dy or dx) of a tile
    constexpr int kUnits = 2 * kHalf;            // 16: dy and dx pieces of a tile
    static_assert((kHalf == 4 || kHalf == 8) && TH >= kRows && kRows >= 2,
                  "a tile's estimate is 8 or 16 units of 8 pixels");
    const int tid = threadIdx.x;
    const int u = tid % kUnits;
    const int ch = u / kHalf;                    // 0: dy, 1: dx
    const int w = u % kHalf;
    // Sampled row r of kRows: tile row round(r (TH - 1) / (kRows - 1)), so the first and
    // last rows and evenly spaced ones between (0, 2, 5, 7 of 8; 0, 3 of 4).
    const int row = ((w / kPieces) * (TH - 1) * 2 + (kRows - 1)) / (2 * (kRows - 1));
    const int piece = w % kPieces;
    constexpr int kPass = 64 * kTileWaves / kUnits;  // tiles per pass (16)
    constexpr int kPasses = 64 / kPass;              // 4: a band has at most 63 tiles
    static_assert(kPass * kPasses == 64, "the passes cover 64 tiles");
    const int tiles_img = a.tiles_y * a.tiles_x;
    // Centre tap (ky = kx = 1 of the 3x3 kernel) of group 0: offset channels 8 (dy), 9 (dx).
    // Every pass loads (tiles past the band read its last tile again and are masked), so
    // the loads are in flight together: one memory round trip for the whole plan.
    float mn[kPasses], mx[kPasses];
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
        const int i = pass * kPass + tid / kUnits;
        mn[pass] = 3.0e38f;
        mx[pass] = -3.0e38f;
        const int t = band0 + min(i, n - 1);
        const int b = t / tiles_img, r = t - b * tiles_img;
        const int ty = r / a.tiles_x, tx = r - ty * a.tiles_x;
        const int oy = min(ty * TH + row, a.Ho - 1);
        const int ox0 = tx * TW + piece * 8;
        const bool valid = i < n && ox0 < a.Wo;  // output rows are whole 8-pixel pieces
        const uint32_t at = ((uint32_t)(b * 2 * a.G * 9 + 8 + ch) * (uint32_t)a.HWo +
                             (uint32_t)(oy * a.Wo + min(ox0, a.Wo - 8))) * 2u;
        const u32x4 q = load16(orr, at, 0);
        const h8 v = __builtin_bit_cast(h8, q);
        const float base = ch ? (float)(ox0 * a.sw - a.pw + a.dw) : (float)(oy * a.sh - a.ph + a.dh);
        const float step = ch ? (float)a.sw : 0.0f;
        const float hi = ch ? (float)a.W : (float)a.H;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float c = __builtin_amdgcn_fmed3f(base + (float)j * step + (float)v[j], -2.0f, hi);
            mn[pass] = fminf(mn[pass], c);
            mx[pass] = fmaxf(mx[pass], c);
        }
        if (!valid) {
            mn[pass] = 3.0e38f;
            mx[pass] = -3.0e38f;
        }
    }
    // Extent per (tile, channel): a min / max over the kHalf lanes of its pieces by DPP
    // (quad_perm [1,0,3,2], [2,3,0,1], then row_half_mirror for 8: lane i meets lanes
    // i ^ 1, i ^ 2, then the other quad of its 8).
    auto lanes = [](float v, bool take_min) {
        auto step = [&](float x, auto ctrl_c) {
            const float y = __builtin_bit_cast(
                float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(ctrl_c)::value, 0xF, 0xF, false));
            return take_min ? fminf(x, y) : fmaxf(x, y);
        };
        v = step(v, std::integral_constant<int, 0xB1>{});
        v = step(v, std::integral_constant<int, 0x4E>{});
        if constexpr (kHalf == 8) v = step(v, std::integral_constant<int, 0x141>{});
        return v;
    };
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
        if (pass * kPass >= n) continue;
        mn[pass] = lanes(mn[pass], true);
        mx[pass] = lanes(mx[pass], false);
        const int i = pass * kPass + tid / kUnits;
        if (w == 0 && i < n) sh[2 * i + ch] = mx[pass] - mn[pass];
    }
    __syncthreads();  // every tile's extents in sh[0 .. 2n) (the plan's only barrier)
    // Each wave ranks the band's tiles itself (the same arithmetic in every wave, so the
    // same ranks): lane l < n holds tile l's key and writes it to the wave's own row of
    // LDS, which the wave then reads back in order (LDS operations of one wave complete
    // in issue order; no other wave touches the row). Key = cost bits << 32 | ~l: the costs
    // are positive, so their bit patterns order like their values, and a larger key is a
    // larger cost or the same cost at a smaller index.
    const int l = tid & 63;
    unsigned long long* keys = reinterpret_cast<unsigned long long*>(sh + 128) + 64 * (tid >> 6);
    unsigned long long key = 0;
    if (l < n) {
        float c = (sh[2 * l] + 3.0f) * (sh[2 * l + 1] + 3.0f);
        c = c == c ? c : 0.0f;
        key = ((unsigned long long)__builtin_bit_cast(uint32_t, c) << 32) | (uint32_t)~l;
        keys[l] = key;
    }
    __builtin_amdgcn_wave_barrier();
    // Rank = place in descending cost order (ties by index); the slot's rank: alone slots
    // n-32 .. 31 the heaviest, then CU c < n - 32 pairs rank (64 - n) + c with n - 1 - c.
    const int pairs = n - 32;
    const int want = loc >= 32 ? n - 1 - (loc - 32) : loc >= pairs ? loc - pairs : (32 - pairs) + loc;
    int rank = 0;
    for (int j = 0; j < n; ++j) rank += keys[j] > key ? 1 : 0;
    const unsigned long long hit = __builtin_amdgcn_ballot_w64(l < n && rank == want);
    // (The ranks are a permutation of 0 .. n-1, so exactly one lane hits.)
    const int pick = hit ? (int)__builtin_ctzll(hit) : loc;
    return min(max(pick, 0), n - 1);
}

// LDS DMA of stage st's offsets (channels 36st .. 36st+35) and masks (18st .. 18st+17) of
// tile (b, ty, tx): 864 chunks of 8 pixels, chunk c -> dst + 16c ([channel][128 px], a
// channel's pixels row by row). Rows past the map repeat its last row (the clamped pixels
// read those).
template <int TW>
__device__ __forceinline__ void tile_copy_offsets(const TileArgs& a, __amdgpu_buffer_rsrc_t orr,
                                                  __amdgpu_buffer_rsrc_t mr, int b, int ty, int tx, int st,
                                                  uint8_t* dst, int wave, int lane) {
    constexpr int NW = kTileWaves;
    constexpr int TH = kTilePix / TW;
    constexpr int kChunksPerCh = kTilePix / 8;  // 16
    constexpr int kRowChunks = TW / 8;
    constexpr int kChunks = kTileOffCh * kChunksPerCh;  // 864
    constexpr int kOffInstr = 36 * kChunksPerCh / 64;   // instructions of the 36 offset channels
    // Chunk c = 64 i + lane is channel c / 16 = 4 i + lane / 16 at tile position c % 16 =
    // lane % 16 for every i, so a lane's source only steps by 4 NW channels per
    // instruction: the address is set up once and then advanced by one add.
    const int rem = lane % kChunksPerCh;
    const int y = min(ty * TH + rem / kRowChunks, a.Ho - 1);
    const int x = tx * TW + (rem % kRowChunks) * 8;
    const uint32_t pix = (uint32_t)(y * a.Wo + x);
    const int ch0 = wave * 4 + lane / kChunksPerCh;  // channel of instruction i = wave
    const uint32_t step = (uint32_t)(4 * NW) * (uint32_t)a.HWo * 2u;
    // (Modular arithmetic: the mask address is only used once it is past channel 36.)
    uint32_t off_src = ((uint32_t)(b * 2 * a.G * 9 + 36 * st + ch0) * (uint32_t)a.HWo + pix) * 2u;
    uint32_t msk_src = ((uint32_t)(b * a.G * 9 + 18 * st + ch0 - 36) * (uint32_t)a.HWo + pix) * 2u;
    for (int i = wave; i * 64 < kChunks; i += NW) {
        const bool is_off = i < kOffInstr;  // uniform per instruction
        if (i * 64 + lane < kChunks) dma16(is_off ? orr : mr, is_off ? off_src : msk_src, dst + i * 64 * 16);
        off_src += step;
        msk_src += step;
    }
}

// A tile's estimate for the pair placement: the extent of its clamped corner positions
// (floor of the sample position, clamped like the stage loop's corners) for group 0's
// centre tap over every pixel, (rows + 3) x (columns + 3). It is the window box of one
// offset channel pair (the flow part of the offset field is common to all groups and taps,
// and its residue spans the same range in each). `src` holds stage 0's offset channels 8
// (dy) and 9 (dx) of the tile, 128 FP16 each in tile_copy_offsets' pixel order; lane l
// takes pixels l and l + 64, and (row, column) pairs are reduced as 16-bit pairs.
template <int TW>
__device__ __forceinline__ int tile_pair_cost(const TileArgs& a, const uint8_t* src_bytes, int ty, int tx,
                                              int lane) {
    constexpr int TH = kTilePix / TW;
    const _Float16* src = reinterpret_cast<const _Float16*>(src_bytes);
    s16x2 mn = s16x2{SHRT_MAX, SHRT_MAX}, mx = s16x2{SHRT_MIN, SHRT_MIN};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int px = lane + 64 * h;
        const int oy = min(ty * TH + px / TW, a.Ho - 1);
        const int ox = min(tx * TW + px % TW, a.Wo - 1);
        const float y = (float)(oy * a.sh - a.ph + a.dh) + (float)src[px];
        const float x = (float)(ox * a.sw - a.pw + a.dw) + (float)src[kTilePix + px];
        const int iy = (int)__builtin_amdgcn_fmed3f(floorf(y), (float)-kPad, (float)a.H);
        const int ix = (int)__builtin_amdgcn_fmed3f(floorf(x), (float)-kPad, (float)a.W);
        const s16x2 v = as_s16x2(__builtin_amdgcn_perm((uint32_t)ix, (uint32_t)iy, 0x05040100u));
        mn = __builtin_elementwise_min(mn, v);
        mx = __builtin_elementwise_max(mx, v);
    }
    // Over the 64 lanes: DPP within each row of 16 (quad_perm [1,0,3,2], [2,3,0,1],
    // row_half_mirror, row_mirror), then the four rows.
    auto step = [&](auto ctrl_c) {
        constexpr int kCtrl = decltype(ctrl_c)::value;
        mn = __builtin_elementwise_min(mn, as_s16x2(__builtin_amdgcn_update_dpp(0, (int)as_u32(mn), kCtrl, 0xF, 0xF, false)));
        mx = __builtin_elementwise_max(mx, as_s16x2(__builtin_amdgcn_update_dpp(0, (int)as_u32(mx), kCtrl, 0xF, 0xF, false)));
    };
    step(std::integral_constant<int, 0xB1>{});
    step(std::integral_constant<int, 0x4E>{});
    step(std::integral_constant<int, 0x141>{});
    step(std::integral_constant<int, 0x140>{});
    s16x2 lo = as_s16x2(__builtin_amdgcn_readlane((int)as_u32(mn), 0));
    s16x2 hi = as_s16x2(__builtin_amdgcn_readlane((int)as_u32(mx), 0));
#pragma unroll
    for (int row = 1; row < 4; ++row) {
        lo = __builtin_elementwise_min(lo, as_s16x2(__builtin_amdgcn_readlane((int)as_u32(mn), 16 * row)));
        hi = __builtin_elementwise_max(hi, as_s16x2(__builtin_amdgcn_readlane((int)as_u32(mx), 16 * row)));
    }
    return ((int)hi.x - (int)lo.x + 3) * ((int)hi.y - (int)lo.y + 3);
}

// A tile whose estimate exceeds this is likely to have split stages: three quarters of a
// group's share of the window buffer in 16-byte units (kTileBuf / 2 / 16 = 2048). On C3's
// inputs (8 seeds, 4096 tiles) every tile with 4 or more split stages estimates 1560 or
// more, and 95 % of all tiles less than 1520.
constexpr int kTilePairHeavy = 3 * kTileBuf / 128;

// Placement in a band of exactly 64 tiles: every CU of the XCD runs two workgroups, locals
// c and c + 32 (c < 32), and the one with the lower blockIdx is dispatched first. The
// kernel ends with a heavy tile dispatched second; dispatched first, the same tile ends
// 5-7 us earlier. So locals c and c + 32 run tiles c and c + 32 of the band, swapped when
// tile c + 32 is heavy (estimate above kTilePairHeavy) and heavier than tile c. Each
// workgroup copies its own tile's stage-0 offsets to dst0 (the offsets area), and each
// wave the two tiles' estimate channels to its own 1 KB of the window buffer at dst1 (free
// until stage 0's windows), so that its own wait suffices, and its stage-0 weight
// fragments to dst1 + kTilePairB: one wait for all of it, the memory round trip every
// workgroup makes for stage 0 anyway. Both workgroups estimate both tiles from the same
// values with the same arithmetic, so they agree. A swapped pair (a few per launch) then
// fetches the other tile's stage-0 offsets, which its partner has brought into L2.
// Returns the tile; all threads call it.
template <int NB, int TW>
__device__ __forceinline__ int tile_pair_slot(const TileArgs& a, __amdgpu_buffer_rsrc_t orr,
                                              __amdgpu_buffer_rsrc_t mr, __amdgpu_buffer_rsrc_t wr, int band0,
                                              int loc, uint8_t* dst0, uint8_t* dst1) {
    constexpr int TH = kTilePix / TW;
    constexpr int kRowChunks = TW / 8;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tiles_img = a.tiles_y * a.tiles_x;
    int b[2], ty[2], tx[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // k = 0: tile c, 1: tile c + 32
        const int t = band0 + (loc & 31) + 32 * k;
        b[k] = t / tiles_img;
        const int r = t - b[k] * tiles_img;
        ty[k] = r / a.tiles_x;
        tx[k] = r - ty[k] * a.tiles_x;
    }
    const int mine = loc < 32 ? 0 : 1;
    tile_copy_offsets<TW>(a, orr, mr, b[mine], ty[mine], tx[mine], 0, dst0, wave, lane);
    // Estimate channels: lane l copies 8 pixels (chunk l % 16) of channel 8 + (l / 16) % 2 of
    // tile l / 32 to slot + 16 l, i.e. [tile][channel][128 px].
    uint8_t* slot = dst1 + wave * 1024;
    {
        const int k = lane / 32, rem = lane % 16, ch = 8 + (lane / 16) % 2;
        const int bk = k ? b[1] : b[0], tyk = k ? ty[1] : ty[0], txk = k ? tx[1] : tx[0];
        const int y = min(tyk * TH + rem / kRowChunks, a.Ho - 1);
        const int x = txk * TW + (rem % kRowChunks) * 8;
        dma16(orr, ((uint32_t)(bk * 2 * a.G * 9 + ch) * (uint32_t)a.HWo + (uint32_t)(y * a.Wo + x)) * 2u, slot);
    }
    // The wave's stage-0 weight slots as the stage loop numbers them (taps 0-3 and the
    // centre tap for waves 0-1, taps 5-8 and the centre tap for waves 2-3), to dst1 +
    // kTilePairB, where the stage loop's prologue reads them.
#pragma unroll
    for (int s = 0; s < kTileSlots; ++s) {
        const int tap = s == 4 ? 4 : (wave < 2 ? 0 : 5) + s;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            dma16(wr, (uint32_t)((tap * NB + nb) * 64 + lane) * 16u,
                  dst1 + kTilePairB + ((wave * kTileSlots + s) * NB + nb) * 1024);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies
    const int c0 = tile_pair_cost<TW>(a, slot, ty[0], tx[0], lane);
    const int c1 = tile_pair_cost<TW>(a, slot + 2 * kTilePix * 2, ty[1], tx[1], lane);
    const int own = band0 + loc;
    if (!(c1 > kTilePairHeavy && c1 > c0)) return own;
    __syncthreads();  // (uniform) every wave's copy of its own tile's offsets is done
    const int other = 1 - mine;
    tile_copy_offsets<TW>(a, orr, mr, b[other], ty[other], tx[other], 0, dst0, wave, lane);
    __builtin_amdgcn_s_waitcnt(0);
    return band0 + (loc ^ 32);
}

template <int NB, int TW, bool EXACT, bool PAIR>
__global__ __launch_bounds__(64 * kTileWaves, 2) void tile_kernel(TileArgs a) {
    constexpr int NW = kTileWaves;
    constexpr int RPW = 32 / TW;  // tile rows per 32-pixel segment
    constexpr int TH = 4 * RPW;   // 2 pixel blocks x 2 segments
    constexpr int NS = 2;         // segments (32-pixel A operands) per wave
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    uint8_t* offs = lds + kTileBuf;  // a stage's offsets and masks [54][128] FP16
    uint32_t* boxes = reinterpret_cast<uint32_t*>(offs + kTileOff);  // [2][NW][2]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = lane >> 5;  // the offset group of this lane within a stage
    const int p = lane & 31;
    const int pblk = wave & 1;   // pixel block (64 pixels)

    // XCD-aware tile order: blockIdx lands on XCD blockIdx % 8, which runs a band of
    // consecutive tiles; within the band a cost-ordered placement where some of the XCD's
    // CUs run one tile and others two.
    const int per_xcd = (a.tiles + 7) / 8;
    const int band0 = (blockIdx.x & 7) * per_xcd;
    const int band_n = min(per_xcd, a.tiles - band0);
    const int loc = blockIdx.x >> 3;
    if (loc >= band_n) return;  // whole workgroup, before any barrier
    unsigned long long* const clock = a.clock ? a.clock + 4 * (size_t)blockIdx.x : nullptr;
    if (clock && tid == 0) clock[0] = __builtin_amdgcn_s_memrealtime();
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.off, a.off_bytes);
    const __amdgpu_buffer_rsrc_t mr = make_rsrc(a.msk, a.msk_bytes);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wpk, a.wpk_bytes);
    // Bands of exactly 64 tiles (the PAIR instantiation): the pair placement, which also
    // leaves stage 0's offsets in the offsets area and this wave's stage-0 weight fragments
    // in the window buffer.
    const bool pair_plan = PAIR && a.plan && band_n == 64;
    const int tile = pair_plan ? tile_pair_slot<NB, TW>(a, orr, mr, wr, band0, loc, offs, lds)
                               : band0 + (a.plan && band_n > 32 && band_n < 64
                                              ? tile_band_slot<TW>(a, orr, band0, band_n, loc,
                                                                   reinterpret_cast<float*>(lds))
                                              : loc);
    if (clock && tid == 0) {  // HW_ID: wave, SIMD, CU, shader array and engine; XCC_ID: the XCD
        const uint32_t hw = (uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 4);
        const uint32_t xcc = (uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 20) & 15u;
        clock[3] = ((unsigned long long)hw << 32) | (xcc << 28) | (uint32_t)tile;
    }
    const int tiles_img = a.tiles_y * a.tiles_x;
    const int b = tile / tiles_img;
    const int trem = tile - b * tiles_img;
    const int ty = trem / a.tiles_x;
    const int tx = trem - ty * a.tiles_x;

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xin, a.xin_bytes);
    const int stages = a.G / 2;

    // Pixel of this lane in segment s (tile rows (2 * pblk + s) * RPW ..): lanes past the
    // edge sample a clamped in-image pixel; their results are not stored. Per segment:
    // integer sample base (oy*sh - ph, ox*sw - pw) and the byte offsets of the pixel's
    // first dy (channel 18 * half) and first mask (channel 36 + 9 * half) of group
    // 2s + half in the LDS copy of the stage's offsets.
    int ybi[NS], xbi[NS];
    uint32_t offs_lane[NS], mask_lane[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int oy = ty * TH + (2 * pblk + s) * RPW + p / TW;
        const int ox = tx * TW + p % TW;
        const int oyc = min(oy, a.Ho - 1), oxc = min(ox, a.Wo - 1);
        ybi[s] = oyc * a.sh - a.ph;
        xbi[s] = oxc * a.sw - a.pw;
        const int lp = (oyc - ty * TH) * TW + (oxc - tx * TW);
        offs_lane[s] = (uint32_t)((18 * half * kTilePix + lp) * 2);
        mask_lane[s] = (uint32_t)(((36 + 9 * half) * kTilePix + lp) * 2);
    }
    // The same bases per kernel row / column, as floats (exact: small integers).
    float ybf[NS][3], xbf[NS][3];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int t = 0; t < 3; ++t) {
            ybf[s][t] = (float)(ybi[s] + t * a.dh);
            xbf[s][t] = (float)(xbi[s] + t * a.dw);
        }
    auto copy_offsets = [&](int st) { tile_copy_offsets<TW>(a, orr, mr, b, ty, tx, st, offs, wave, lane); };

    // Window geometry of a stage (wave-uniform): origin, size in units, LDS placement.
    struct Win {
        int y0[2], x0[2], ww[2], hh[2], off[2];
        bool lds;    // both windows are in LDS
        bool split;  // else each fits alone: one pass per group, its window at 0
                     // (neither: the stage gathers from global memory)
    };
    auto read_windows = [&]() {
        // Lanes 0-7 read one wave's box of group lane / 4; reduce over the 4 waves.
        uint32_t mn = as_u32(s16x2{SHRT_MAX, SHRT_MAX}), mx = as_u32(s16x2{SHRT_MIN, SHRT_MIN});
        if (lane < 2 * NW) {
            const uint32_t* s = boxes + lane * 2;  // [group][wave]
            mn = s[0];
            mx = s[1];
        }
        box_step<1>(mn, mx);
        box_step<2>(mn, mx);
        Win w;
        int size[2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const uint32_t lo = __builtin_amdgcn_readlane(mn, NW * g);
            const uint32_t hi = __builtin_amdgcn_readlane(mx, NW * g);
            w.y0[g] = (int)(short)(lo & 0xffffu);
            w.x0[g] = (int)(short)(lo >> 16);
            w.hh[g] = (int)(short)(hi & 0xffffu) - w.y0[g] + 2;
            w.ww[g] = (int)(short)(hi >> 16) - w.x0[g] + 2;
            size[g] = w.hh[g] * w.ww[g] * 16;
        }
        w.lds = size[0] + size[1] <= kTileBuf;
        w.split = !w.lds && size[0] <= kTileBuf && size[1] <= kTileBuf;
        w.off[0] = 0;
        w.off[1] = w.split ? 0 : size[0];
        return w;
    };
    // LDS DMA of the windows of stage st (both, or only window `only` of a split stage) as
    // chunks of 64 consecutive window units (one instruction each), window g's chunks at
    // LDS offset off[g] + 1024 c.
    auto copy_windows = [&](int st, const Win& w, int only) {
        if (!w.lds && !w.split) return;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            if (only >= 0 && g != only) continue;
            const int ww = g ? w.ww[1] : w.ww[0];
            const int units = ww * (g ? w.hh[1] : w.hh[0]);
            const int chunks = (units + 63) >> 6;
            // Wave `wave` issues chunks wave, wave + NW, ... A lane's unit f = 64 c + lane is
            // row f / ww, column f % ww: found once (the FP32 reciprocal, then corrected by
            // one either way), then stepped by NW * 64 units = dq rows + dr columns.
            int f = wave * 64 + lane;
            int r = (int)(((float)f + 0.5f) * __builtin_amdgcn_rcpf((float)ww));
            r -= r * ww > f ? 1 : 0;
            r += (r + 1) * ww <= f ? 1 : 0;
            int col = f - r * ww;
            const int dq = (NW * 64) / ww, dr = NW * 64 - dq * ww;  // wave-uniform
            const uint32_t row0 = (uint32_t)(b * a.CBLK + 2 * st + g) * a.Hp + (uint32_t)((g ? w.y0[1] : w.y0[0]) + kPad);
            uint32_t unit = (row0 + (uint32_t)r) * a.Wp + (uint32_t)((g ? w.x0[1] : w.x0[0]) + kPad + col);
            const uint32_t unit_step = (uint32_t)dq * a.Wp + (uint32_t)dr;
            const uint32_t wrap = (uint32_t)(a.Wp - ww);  // next row's first column
            uint8_t* dst = lds + (g ? w.off[1] : w.off[0]) + wave * 1024;
            for (int c = wave; c < chunks; c += NW) {
                if (f < units) dma16(xr, unit * 16u, dst);
                f += NW * 64;
                col += dr;
                unit += unit_step;
                if (col >= ww) {
                    col -= ww;
                    unit += wrap;
                }
                dst += NW * 1024;
            }
        }
    };

    f32x16 acc[NS][NB];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[s][nb] = f32x16{};

    // The stage loop of a wave pair (compile-time): taps TF .. TF + 3 for both segments
    // and the centre tap 4 for segment SODD only (waves 0-1: taps 0-3 + tap 4 of segment
    // 0; waves 2-3: taps 5-8 + tap 4 of segment 1), 9 samples per lane and stage for
    // every wave. Sample j = 2 k + s (j < 8) is tap TF + k, segment s; j = 8 is the
    // centre tap. Weight slot k (0-3) holds tap TF + k, slot 4 the centre tap.
    auto run = [&](auto tf_c, auto sodd_c) {
        constexpr int TF = decltype(tf_c)::value;
        constexpr int SODD = decltype(sodd_c)::value;
        constexpr int NSMP = 9;   // samples per lane and stage
        constexpr int NSLOT = kTileSlots;  // weight slots
        auto tap_of = [](int j) { return j == 8 ? 4 : TF + j / 2; };
        auto seg_of = [](int j) { return j == 8 ? SODD : j % 2; };
        auto slot_of = [](int j) { return j == 8 ? 4 : j / 2; };
        auto slot_done = [](int j) { return j == 8 || j % 2 == 1; };  // the slot's last sample

        // A sample's dy, dx and mask from the LDS copy of the stage's offsets (an LDS
        // pointer, so each read is one ds_read_u16 with an immediate offset from the lane's
        // base).
        typedef const __attribute__((address_space(3))) _Float16* lds_h;
        const lds_h offs_h = (lds_h)(const __attribute__((address_space(3))) uint8_t*)(lds + kTileBuf);
        auto offset_of = [&](int j, int which) {  // which: 0 = dy, 1 = dx, 2 = mask
            const int s = seg_of(j), k = tap_of(j);
            const uint32_t at = which == 2 ? mask_lane[s] + (uint32_t)(k * kTilePix * 2)
                                           : offs_lane[s] + (uint32_t)((2 * k + which) * kTilePix * 2);
            return offs_h[at / 2];
        };
        // Sample state of a stage: a[] = clamped corner (iy, ix) as a 16-bit pair, then
        // the sample's address; w0/w1 = the FP16 corner weights.
        // a = the clamped corner (iy, ix) as a 16-bit pair, then the sample's address.
        // Fast sampler: w0 / w1 = the four mask-folded FP16 corner weights. Exact sampler
        // (EXACT): w0 / w1 = the FP32 fractions ly / lx, m = the FP16 masks of samples 2i
        // and 2i + 1, for the reference's FP32 blend.
        struct Samples {
            uint32_t a[NSMP], w0[NSMP], w1[NSMP];
            uint32_t m[EXACT ? (NSMP + 1) / 2 : 1];
        };
        s16x2 bmin, bmax;
        auto box_reset = [&]() {
            bmin = s16x2{SHRT_MAX, SHRT_MAX};
            bmax = s16x2{SHRT_MIN, SHRT_MIN};
        };
        auto coords = [&](int j, Samples& C) {
            const int s = seg_of(j), k = tap_of(j);
            // float(oy*sh - ph + ky*dh) + dy (MetalShader.swift:327-332), one rounding: an
            // fma with 1 is the same single rounding and takes the FP16 offset as it is
            // (v_fma_mix_f32; with a literal 1 the compiler folds it back into convert + add).
            const float y = __builtin_fmaf((float)offset_of(j, 0), a.one, ybf[s][k / 3]);
            const float x = __builtin_fmaf((float)offset_of(j, 1), a.one, xbf[s][k % 3]);
            const float fy = floorf(y), fx = floorf(x);
            const float ly = y - fy, lx = x - fx;
            // Clamped so both rows/columns of the corner pair stay in the padded plane.
            const int iy = (int)__builtin_amdgcn_fmed3f(fy, (float)-kPad, (float)a.H);
            const int ix = (int)__builtin_amdgcn_fmed3f(fx, (float)-kPad, (float)a.W);
            C.a[j] = __builtin_amdgcn_perm((uint32_t)ix, (uint32_t)iy, 0x05040100u);
            bmin = __builtin_elementwise_min(bmin, as_s16x2(C.a[j]));
            bmax = __builtin_elementwise_max(bmax, as_s16x2(C.a[j]));
            if constexpr (EXACT) {
                C.w0[j] = __builtin_bit_cast(uint32_t, ly);
                C.w1[j] = __builtin_bit_cast(uint32_t, lx);
                const uint32_t mb = __builtin_bit_cast(uint16_t, offset_of(j, 2));
                C.m[j / 2] = (j & 1) ? (C.m[j / 2] & 0xffffu) | (mb << 16) : mb;
                return;
            }
            const float m = (float)offset_of(j, 2);
            // Mask folded into the four bilinear weights, each rounded once to FP16 (the
            // mask products as fmas with +0: the products are not negative, so the same
            // single rounding, with the FP16 mask taken as it is).
            const float t0 = __builtin_fmaf(m, 1.0f - ly, 0.0f);
            const float t1 = __builtin_fmaf(m, ly, 0.0f);
            C.w0[j] = __builtin_bit_cast(uint32_t, h2{(_Float16)(t0 * (1.0f - lx)), (_Float16)(t0 * lx)});
            C.w1[j] = __builtin_bit_cast(uint32_t, h2{(_Float16)(t1 * (1.0f - lx)), (_Float16)(t1 * lx)});
        };
        // This wave's box (per half = per group) to LDS.
        auto publish_box = [&]() {
            uint32_t mn = as_u32(bmin), mx = as_u32(bmax);
            box_step<1>(mn, mx);
            box_step<2>(mn, mx);
            box_step<4>(mn, mx);
            box_step<8>(mn, mx);
            box_step<16>(mn, mx);
            if (p == 0) {
                uint32_t* d = boxes + (half * NW + wave) * 2;
                d[0] = mn;
                d[1] = mx;
            }
        };
        // Addresses of a stage: LDS byte addresses when its windows are in LDS, else the
        // byte offset of the corner in the CB8 input; `pitch` steps to the lower row.
        struct Addressing {
            int rs, c;  // address = iy * rs + ix * 16 + c
            uint32_t pitch;
        };
        auto addressing = [&](int st, const Win& w) {
            const int g = half;
            const int y0 = g ? w.y0[1] : w.y0[0];
            const int x0 = g ? w.x0[1] : w.x0[0];
            const int ww = g ? w.ww[1] : w.ww[0];
            const int off = g ? w.off[1] : w.off[0];
            const bool in_lds = w.lds || w.split;
            Addressing r;
            r.rs = in_lds ? ww * 16 : a.Wp * 16;
            r.pitch = (uint32_t)r.rs;
            r.c = in_lds ? off - y0 * ww * 16 - x0 * 16
                         : ((((b * a.CBLK + 2 * st + g) * a.Hp + kPad) * a.Wp) + kPad) * 16;
            return r;
        };
        auto make_address = [&](int j, Samples& C, const Addressing& r) {
            const int iy = (int)(short)(C.a[j] & 0xffffu);
            const int ix = (int)(short)(C.a[j] >> 16);
            // iy in [-2, H] and rs (<= 16 Wp) fit 24 bits signed (input sides below 32000):
            // the full-rate 24-bit multiply gives the same low 32 bits.
            C.a[j] = (uint32_t)(__mul24(iy, r.rs) + ix * 16 + r.c);
        };
        // Weight fragments of this wave's taps of one stage, one slot per tap: a slot of
        // stage st+1 is requested as soon as its tap's last sample of stage st has used it.
        h8 Bq[NSLOT][NB];
        auto load_b = [&](int st, int slot) {
            const int tap = slot == 4 ? 4 : TF + slot;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                Bq[slot][nb] = __builtin_bit_cast(
                    h8, load16(wr, (uint32_t)(((st * 9 + tap) * NB + nb) * 64 + lane) * 16u, 0));
        };
        // The LDS reads are issued in both modes: lanes that are not `active` (all of them
        // when the stage gathers from global memory, the other group's in a pass of a
        // split stage) read the 32 zero bytes, so their blend is 0 (their global loads then
        // replace them, and this branch waits for those at once). The compiler's waits are
        // placed for every path of the control flow and count memory operations in issue
        // order: with the LDS reads inside the branch (or global loads left in flight), the
        // blend of each sample waited for the next sample's corner reads, or for the weight
        // fragments requested after them, and the prefetch hid nothing. Only stages whose
        // windows do not fit the buffer one at a time take the global branch.
        auto corners = [&](int j, const Samples& C, const Addressing& r, bool from_lds, bool active,
                           uint32_t lds_pitch, u32x4 (&q)[4]) {
            const uint32_t a0 = C.a[j];
            const uint32_t l0 = active ? a0 : (uint32_t)kTileZero, l1 = l0 + lds_pitch;
            typedef const __attribute__((address_space(3))) u32x4* lds_u32x4;
            q[0] = *(lds_u32x4)(uintptr_t)l0;
            q[1] = *(lds_u32x4)(uintptr_t)(l0 + 16);
            q[2] = *(lds_u32x4)(uintptr_t)l1;
            q[3] = *(lds_u32x4)(uintptr_t)(l1 + 16);
            if (!from_lds) {
                const uint32_t a1 = a0 + r.pitch;
                q[0] = load16(xr, a0, 0);
                q[1] = load16(xr, a0 + 16u, 0);
                q[2] = load16(xr, a1, 0);
                q[3] = load16(xr, a1 + 16u, 0);
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            }
        };
        // K-loop of one stage (or one pass of a split stage): per sample j the next
        // sample's corners are requested before this one is blended and multiplied; after a
        // tap's last sample its weight slot is refilled (in the stage's last pass), and
        // side(j) runs after every sample (the next stage's work, in the first pass).
        auto kloop = [&](int st, const Samples& C, const Addressing& r, bool from_lds, bool active,
                         bool last_pass, bool first_pass, auto&& side) {
            const uint32_t lds_pitch = active ? r.pitch : 0u;
            u32x4 qa[4], qb[4];
            corners(0, C, r, from_lds, active, lds_pitch, qa);
#pragma unroll
            for (int j = 0; j < NSMP; ++j) {
                u32x4(&cur)[4] = (j & 1) ? qb : qa;
                u32x4(&nxt)[4] = (j & 1) ? qa : qb;
                // The next sample's corners are requested before this one's blend; with the
                // exact sampler (a blend long enough to cover the LDS round trip) after it,
                // so the two samples' corners need not be live together.
                if (!EXACT && j + 1 < NSMP) corners(j + 1, C, r, from_lds, active, lds_pitch, nxt);
                const int kk = slot_of(j), s = seg_of(j);
                h8 A;
                if constexpr (EXACT) {
                    const float m = (float)__builtin_bit_cast(_Float16, (uint16_t)(C.m[j / 2] >> (16 * (j & 1))));
                    A = blend_exact(cur[0], cur[1], cur[2], cur[3], __builtin_bit_cast(float, C.w0[j]),
                                    __builtin_bit_cast(float, C.w1[j]), m);
                } else {
                    A = blend_w(cur, C.w0[j], C.w1[j]);
                }
                if (EXACT && j + 1 < NSMP) corners(j + 1, C, r, from_lds, active, lds_pitch, nxt);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    acc[s][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A, Bq[kk][nb], acc[s][nb], 0, 0, 0);
                if (slot_done(j) && last_pass && st + 1 < stages) load_b(st + 1, kk);
                if (first_pass) side(j);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        // After the K-loop of stage st (or the prologue): stage st+1's box reduced, its
        // windows and stage st+2's offsets requested, its addresses made, every DMA done.
        Win win;
        Addressing ad;
        auto next_stage = [&](int st1, Samples& C) {
            publish_box();
            __syncthreads();  // every box; every wave past its corner and offset reads
            win = read_windows();
            copy_windows(st1, win, win.split ? 0 : -1);
            if (st1 + 1 < stages) copy_offsets(st1 + 1);
            ad = addressing(st1, win);
#pragma unroll
            for (int j = 0; j < NSMP; ++j) make_address(j, C, ad);
            __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA
            __syncthreads();                // every wave's DMA
        };

        // ---- prologue: stage 0's offsets, coordinates, windows and addresses ----
        Samples ca, cb;
#pragma unroll
        for (int slot = 0; slot < NSLOT; ++slot) {
            if (pair_plan) {  // the pair placement's copy (its wait is done)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    Bq[slot][nb] = __builtin_bit_cast(
                        h8, *reinterpret_cast<const u32x4*>(lds + kTilePairB + ((wave * NSLOT + slot) * NB + nb) * 1024 +
                                                            lane * 16));
            } else {
                load_b(0, slot);
            }
        }
        if (!pair_plan) copy_offsets(0);
        if (tid < 8) reinterpret_cast<uint32_t*>(lds + kTileZero)[tid] = 0u;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // stage 0's offsets in LDS; the zero bytes
        box_reset();
#pragma unroll
        for (int j = 0; j < NSMP; ++j) coords(j, ca);
        next_stage(0, ca);

        // Stage st: `cur` holds its addresses; after its samples 1 and 3 the K-loop also
        // computes stage st+1's coordinates into `nxt` (from the offsets copied with st's
        // windows), which then serve stage st+1. A split stage has a second pass: group 0's window is in LDS
        // (next_stage), then group 1's.
        // With the fast sampler, stages run in pairs with the two sample states swapping
        // roles, so that no state is copied (27 register moves per stage: C5 1.2 us, C3
        // 0.35 us). The exact sampler's larger state then spills twice as many registers
        // (C3 +3 us), so it copies.
        auto stage = [&](int st, Samples& cur, Samples& nxt) {
            const bool more = st + 1 < stages;
            if (more) box_reset();
            constexpr int kPerCoord = (NSMP + 1) / 2;
            auto side = [&](int j) {
                if (!more || (j != 1 && j != 3)) return;
                const int h = j == 1 ? 0 : 1;
#pragma unroll
                for (int i = 0; i < kPerCoord; ++i)
                    if (h * kPerCoord + i < NSMP) coords(h * kPerCoord + i, nxt);
            };
            const bool in_lds = win.lds || win.split;
            kloop(st, cur, ad, in_lds, win.lds || (win.split && half == 0), !win.split, true, side);
            if (win.split) {
                __syncthreads();  // every wave is done with group 0's window
                copy_windows(st, win, 1);
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();  // group 1's window in LDS
                kloop(st, cur, ad, true, half == 1, true, false, side);
            }
            if (more) next_stage(st + 1, nxt);
        };
        if constexpr (EXACT) {
            for (int st = 0; st < stages; ++st) {
                stage(st, ca, cb);
                ca = cb;
            }
        } else {
            int st = 0;
            for (; st + 1 < stages; st += 2) {
                stage(st, ca, cb);
                stage(st + 1, cb, ca);
            }
            if (st < stages) stage(st, ca, cb);
        }
    };
    if (wave < 2) run(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    else run(std::integral_constant<int, 5>{}, std::integral_constant<int, 1>{});

    // ---- epilogue: the two tap halves summed (waves 0-1's + waves 2-3's), bias, FP16, NCHW
    // stores through LDS ----
    __syncthreads();  // every wave is done with the windows
    float* red = reinterpret_cast<float*>(lds);  // [2 pixel blocks][NS][NB][16][64]
    if (wave >= 2) {
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int v = 0; v < 16; ++v) red[(((pblk * NS + s) * NB + nb) * 16 + v) * 64 + lane] = acc[s][nb][v];
    }
    __syncthreads();
    if (wave >= 2) return;  // no barrier follows
    uint16_t* stage = reinterpret_cast<uint16_t*>(lds + 2 * NS * NB * 16 * 64 * 4) + (size_t)wave * NS * 32 * NB * 32;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int oc = nb * 32 + p;
            const float bias = a.bias[oc];
#pragma unroll
            for (int k = 0; k < 4; ++k) {  // segment pixels 8 k + 4 half .. + 3: one 8-byte write
                uint32_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int v = 4 * k + e;
                    const float sum = acc[s][nb][v] + red[(((pblk * NS + s) * NB + nb) * 16 + v) * 64 + lane];
                    h[e] = __builtin_bit_cast(uint16_t, round_f16(sum + bias));
                }
                *reinterpret_cast<uint2*>(stage + (s * NB * 32 + oc) * 32 + 8 * k + 4 * half) =
                    make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
            }
        }
    // Each item: 4 consecutive pixels of one output channel and tile row. No barrier is
    // needed: each wave stores only what it staged.
    constexpr int kQ = TW / 4;
    const int ox0 = tx * TW;
    for (int it = lane; it < NS * NB * 32 * RPW * kQ; it += 64) {
        const int q = it % kQ;
        const int rr = (it / kQ) % RPW;
        const int oc = (it / (kQ * RPW)) % (NB * 32);
        const int s = it / (kQ * RPW * NB * 32);
        const int y = ty * TH + (2 * pblk + s) * RPW + rr;
        const int x = ox0 + 4 * q;
        if (y >= a.Ho) continue;
        const uint16_t* src = stage + (s * NB * 32 + oc) * 32 + rr * TW + 4 * q;
        uint16_t* dst = a.out + ((size_t)b * a.Cout + oc) * a.HWo + (size_t)y * a.Wo + x;
        if (x + 3 < a.Wo && (((uintptr_t)dst) & 7u) == 0) {
            *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(src);
        } else {
            for (int e = 0; e < 4; ++e)
                if (x + e < a.Wo) dst[e] = src[e];
        }
    }
    if (clock && lane == 0) clock[1 + wave] = __builtin_amdgcn_s_memrealtime();  // stores issued
}

// Weights -> the tile kernel's B fragments [G/2][9][NB][64][8]: lane l of K-step k, stage
// s holds output channel nb*32 + l%32 and the 8 channels of group 2s + l/32, tap k.
// layout 0 = OIHW, 1 = [ic][k][oc] (.dcnfp16).
__global__ __launch_bounds__(256) void tile_prepack_kernel(const uint16_t* __restrict__ w, int layout,
                                                           uint16_t* __restrict__ wpk, int Cin,
                                                           int Cout, int NB, long total) {
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    const int e = (int)(gid & 7);
    const int lane = (int)((gid >> 3) & 63);
    long q = gid >> 9;
    const int nb = (int)(q % NB);
    q /= NB;
    const int k = (int)(q % 9);
    const int st = (int)(q / 9);
    const int grp = 2 * st + (lane >> 5);
    const int oc = nb * 32 + (lane & 31);
    const int ic = grp * 8 + e;
    uint16_t v = 0;
    if (oc < Cout && ic < Cin)
        v = layout == DCN_LAYOUT_OIHW ? w[((size_t)oc * Cin + ic) * 9 + k]
                                      : w[((size_t)ic * 9 + k) * Cout + oc];
    wpk[gid] = v;
}

template <int NB, int TW, bool EXACT, bool PAIR>
hipError_t launch_tile_p(const TileArgs& a, hipStream_t stream) {
    auto kernel = &tile_kernel<NB, TW, EXACT, PAIR>;
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(kernel), kTileLds);
    if (attr != hipSuccess) return attr;
    const unsigned grid = (unsigned)(((a.tiles + 7) / 8) * 8);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kTileWaves), kTileLds, stream, a);
    return hipGetLastError();
}

// The pair placement's instantiation where the planned placement has bands of exactly 64
// tiles (every CU of an XCD runs two); every other shape runs the kernel without it.
template <int NB, int TW, bool EXACT>
hipError_t launch_tile_t(const TileArgs& a, hipStream_t stream) {
    return a.plan && (a.tiles + 7) / 8 == 64 ? launch_tile_p<NB, TW, EXACT, true>(a, stream)
                                             : launch_tile_p<NB, TW, EXACT, false>(a, stream);
}

template <int TW>
hipError_t launch_tile_nb(const TileArgs& a, int nb, bool exact, hipStream_t stream) {
    switch (nb * 2 + (exact ? 1 : 0)) {
        case 2: return launch_tile_t<1, TW, false>(a, stream);
        case 3: return launch_tile_t<1, TW, true>(a, stream);
        case 4: return launch_tile_t<2, TW, false>(a, stream);
        case 5: return launch_tile_t<2, TW, true>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool tile_supported(const dcn_shape& s) {
    // Output rows of 8-pixel multiples: the offsets are copied as 16-byte chunks of rows.
    // Clamped corner coordinates (-2 .. H, -2 .. W) travel as signed 16-bit pairs through
    // the box reduction and the address set-up, so both input sides stay below 2^15 with
    // room for the clamp.
    return s.groups == 1 && s.kernel_height == 3 && s.kernel_width == 3 &&
           s.input_channels == 8 * s.offset_groups && s.offset_groups % 2 == 0 &&
           s.output_channels % 32 == 0 && s.output_channels <= 64 && s.output_width % 8 == 0 &&
           s.input_height <= kTileMaxSide && s.input_width <= kTileMaxSide;
}

size_t tile_packed_bytes(const dcn_shape& s) {
    return (size_t)(s.offset_groups / 2) * 9 * (s.output_channels / 32) * 64 * 8 * sizeof(uint16_t);
}

hipError_t launch_tile_prepack(const KShape& s, const uint16_t* w, int layout, void* wpk,
                               hipStream_t stream) {
    const int nb = s.Cout / 32;
    const long total = (long)(s.og / 2) * 9 * nb * 64 * 8;
    const long grid = (total + 255) / 256;
    hipLaunchKernelGGL(tile_prepack_kernel, dim3((unsigned)grid), dim3(256), 0, stream, w, layout,
                       (uint16_t*)wpk, s.Cin, s.Cout, nb, total);
    return hipGetLastError();
}

hipError_t launch_tile_f16(const KShape& s, const FusedGeometry& g, const FusedConfig& cfg,
                           const void* cb8, const uint16_t* off, const uint16_t* mask,
                           const void* packed_w, const float* packed_b, uint16_t* out,
                           hipStream_t stream, unsigned long long* clock) {
    TileArgs a;
    a.clock = clock;
    a.xin = cb8;
    a.off = off;
    a.msk = mask;
    a.wpk = packed_w;
    a.bias = packed_b;
    a.out = out;
    const size_t hwo = (size_t)s.Ho * s.Wo;
    a.xin_bytes = (uint32_t)((size_t)s.B * g.cblk * g.hp * g.wp * 16);
    a.off_bytes = (uint32_t)((size_t)s.B * 2 * s.og * 9 * hwo * 2);
    a.msk_bytes = (uint32_t)((size_t)s.B * s.og * 9 * hwo * 2);
    a.wpk_bytes = (uint32_t)((size_t)(s.og / 2) * 9 * (s.Cout / 32) * 64 * 8 * 2);
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
    a.one = 1.0f;
    a.plan = cfg.ks == 8 ? 1 : 0;  // for this variant, ks 8 = planned placement, 1 = fixed
    const int tw = cfg.mt == 32 ? 32 : 16;  // for this variant, mt carries the tile width
    const int th = 4 * 32 / tw;  // 2 pixel blocks x 2 segments of 32 pixels
    a.tiles_y = (s.Ho + th - 1) / th;
    a.tiles_x = (s.Wo + tw - 1) / tw;
    a.tiles = a.tiles_y * a.tiles_x * s.B;
    const bool exact = cfg.sampler == kSamplerExact;
    return tw == 32 ? launch_tile_nb<32>(a, g.nb, exact, stream) : launch_tile_nb<16>(a, g.nb, exact, stream);
}

size_t tile_grid(const KShape& s, const FusedConfig& cfg) {
    const int tw = cfg.mt == 32 ? 32 : 16;
    const int th = 4 * 32 / tw;
    const size_t tiles = (size_t)((s.Ho + th - 1) / th) * ((s.Wo + tw - 1) / tw) * s.B;
    return (tiles + 7) / 8 * 8;
}

}  // namespace dcn
