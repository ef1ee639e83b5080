// Internal declarations shared by the C-ABI host layer and the HIP kernel files.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <set>
#include <string>
#include <tuple>

#include "dcn/dcn.h"

namespace dcn {

// hipFuncSetAttribute(MaxDynamicSharedMemorySize) on the current device, once per
// (kernel, device, size): a launch above 64 KB of dynamic LDS needs it, and a process may
// drive more than one device.
inline hipError_t allow_dynamic_lds(const void* kernel, size_t bytes) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    static std::mutex mu;
    static std::set<std::tuple<const void*, int, size_t>> done;
    std::lock_guard<std::mutex> lock(mu);
    if (done.count(std::make_tuple(kernel, device, bytes))) return hipSuccess;
    e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess) done.insert(std::make_tuple(kernel, device, bytes));
    return e;
}

// Shape as seen by device code: the 17 reference fields, by value.
struct KShape {
    int32_t B, Cin, H, W, Cout, Ho, Wo, KH, KW, ph, pw, sh, sw, dh, dw, groups, og;
};

inline KShape to_kshape(const dcn_shape& s) {
    return KShape{s.batch,         s.input_channels,  s.input_height,    s.input_width,
                  s.output_channels, s.output_height, s.output_width,    s.kernel_height,
                  s.kernel_width,  s.pad_height,      s.pad_width,       s.stride_height,
                  s.stride_width,  s.dilation_height, s.dilation_width,  s.groups,
                  s.offset_groups};
}

// Geometry of the fused FP16 path for one shape (see dcn_kernels_fused.hip).
struct FusedGeometry {
    int cblk;     // Cin / 8: number of 8-channel blocks (padded planes)
    int cb;       // 8-channel blocks per offset group
    int ka;       // Kh * Kw
    int kb;       // K-blocks of 8 = G * KA * CB
    int ksteps;   // MFMA K-steps of 16 = ceil(kb / 2)
    int nb;       // N-blocks of 32 output channels
    int hp, wp;   // padded input height / width
    long long m;  // output pixels B * Ho * Wo
};
bool fused_geometry(const dcn_shape& s, FusedGeometry* g);

// Sampler arithmetic of the fused kernel.
enum SamplerMode : int {
    // The reference's gather arithmetic, FP32, same association, then half(s * mask):
    // bit-identical im2col values to deform_conv2d_fp16_jasna_gather.
    kSamplerExact = 0,
    // Mask folded into the four bilinear weights, packed-FP16 blend. Faster; within
    // the FP16 tolerance against the FP32 oracle.
    kSamplerFast = 1,
    // BF16 storage (input, offsets, mask, weights, output): the exact sampler's FP32
    // arithmetic on the widened BF16 corners, each sample rounded once to BF16, and the
    // BF16 MFMA. The BF16 forwards run the narrow variant up to 1024 tiles of 32 pixels,
    // above that the window variant (4 x 32 tiles, 4 waves) where the shape allows it,
    // else the register variant.
    kSamplerBf16 = 2,
};

enum FusedVariant : int {
    kVariantAuto = 0,
    // Each wave samples its A fragments straight into registers (one K-block per lane
    // per MFMA step); no LDS tile. Handles any K.
    kVariantRegister = 1,
    // A sampler phase fills an LDS im2col tile for the whole K range, then an MFMA
    // phase consumes it. Needs the tile to fit in LDS.
    kVariantStaged = 2,
    // Per-group LDS windows of the input (3x3 kernels, 8 channels per offset group): a
    // 2D pixel tile per workgroup, gathers served from LDS. Config: mt = tile rows,
    // ks = waves (row blocks of 32 pixels).
    kVariantWindow = 3,
    // kVariantWindow with the lower corner row of each sample read through the L1
    // (the window is there too after its copy), splitting gathers between LDS and L1.
    kVariantWindowSplit = 4,
    // 16-pixel tiles on v_mfma_f32_16x16x32_f16 with every load of a wave's K-steps in
    // flight at once: one workgroup per CU on small problems. Config: ks = waves (8, 12).
    kVariantNarrow = 5,
    // kVariantWindow (8 x 32 tiles, 8 waves, two groups per stage) with the next stage's
    // windows and B fragments streamed into a double buffer by LDS DMA while the current
    // stage is multiplied. Needs an even group count.
    kVariantWindowAsync = 6,
    // Tile windows (dcn_kernels_tile.hip): 4 waves on a 128-pixel tile, 8 x 16 (mt 16) or
    // 4 x 32 (mt 32); two offset groups per stage, waves 0-1 taking taps 0-4 and waves 2-3
    // taps 5-8 of both. Each stage's offsets and masks and the two groups' sample windows
    // are copied into LDS by DMA (one 64 KB window buffer, two workgroups per CU); a stage
    // whose windows do not fit gathers from global memory. 3x3 kernels, 8 channels per
    // group, an even group count, Cout 32 or 64; fast sampler only. mt = tile width, ks = 8.
    kVariantTile = 7,
};

struct FusedConfig {
    int variant;  // FusedVariant
    int mt;       // 32-pixel row blocks per tile (1 or 2)
    int ks;       // waves per workgroup splitting the K range
    int sampler;  // SamplerMode
    int split = 0;  // window variant: lower corner row from the L1
};
size_t staged_lds_bytes(const FusedGeometry& g, const FusedConfig& cfg);
bool window_supported(const dcn_shape& s);
int window_gps(const dcn_shape& s);
size_t window_packed_bytes(const dcn_shape& s);
hipError_t launch_prepack_group(const KShape& s, const uint16_t* w, int layout, void* wpk,
                                hipStream_t stream);
hipError_t launch_window_f16(const KShape& s, const FusedGeometry& g, const FusedConfig& cfg,
                             const void* cb8, const uint16_t* off, const uint16_t* mask,
                             const void* packed_w, const float* packed_b, uint16_t* out,
                             hipStream_t stream);
bool tile_supported(const dcn_shape& s);
size_t tile_packed_bytes(const dcn_shape& s);
hipError_t launch_tile_prepack(const KShape& s, const uint16_t* w, int layout, void* wpk,
                               hipStream_t stream);
// clock: per-workgroup clock stamps [tile_grid(s, cfg)][4] (TileArgs::clock) or null.
hipError_t launch_tile_f16(const KShape& s, const FusedGeometry& g, const FusedConfig& cfg,
                           const void* cb8, const uint16_t* off, const uint16_t* mask,
                           const void* packed_w, const float* packed_b, uint16_t* out,
                           hipStream_t stream, unsigned long long* clock = nullptr);
size_t tile_grid(const KShape& s, const FusedConfig& cfg);  // workgroups of a tile launch

// ---- launchers (return hipSuccess or the launch error) ---------------------------
hipError_t launch_direct_f32(const KShape& s, const float* in, const float* off,
                             const float* mask, const float* w, const float* b, float* out,
                             hipStream_t stream);
hipError_t launch_direct_f16(const KShape& s, const uint16_t* in, const uint16_t* off,
                             const uint16_t* mask, const uint16_t* w, const uint16_t* b,
                             uint16_t* out, hipStream_t stream);
hipError_t launch_floor(int workgroups, int threads, int lds_bytes, hipStream_t stream);
hipError_t launch_pack_cb8(const KShape& s, const FusedGeometry& g, const uint16_t* in_nchw,
                           void* cb8, hipStream_t stream);
// Allocation-free entry point (dcn_scratch.hip): resolve the device address of the
// file-scope scratch array for `device` (which must be current; once per device), and
// look it up afterwards (null when it was never resolved).
hipError_t noalloc_scratch_init(int device);
// One call's use of the device's allocation-free scratch (dcn_scratch.hip): while it
// lives, the library's lock is held; on construction the stream waits for the previous
// call if that ran on another stream, on destruction the call's completion is recorded.
class NoallocScratchUse {
public:
    NoallocScratchUse(int device, hipStream_t stream);
    ~NoallocScratchUse();
    NoallocScratchUse(const NoallocScratchUse&) = delete;
    NoallocScratchUse& operator=(const NoallocScratchUse&) = delete;
    void* ptr() const { return ptr_; }        // null: not resolved on this device
    hipError_t error() const { return error_; }
private:
    std::unique_lock<std::mutex> lock_;
    int device_;
    hipStream_t stream_;
    void* ptr_ = nullptr;
    bool ordered_ = false;
    hipError_t error_ = hipSuccess;
};
hipError_t launch_prepack_weights(const KShape& s, const FusedGeometry& g, const uint16_t* w,
                                  int layout, const uint16_t* bias, void* packed_w,
                                  float* packed_b, hipStream_t stream, bool bias_bf16 = false);
hipError_t launch_fused_f16(const KShape& s, const FusedGeometry& g, const FusedConfig& cfg,
                            const void* cb8, const uint16_t* off, const uint16_t* mask,
                            const void* packed_w, const float* packed_b, uint16_t* out,
                            hipStream_t stream);
hipError_t launch_im2col_f16(const KShape& s, const uint16_t* in, const uint16_t* off,
                             const uint16_t* mask, uint16_t* columns, hipStream_t stream);
hipError_t launch_flag_nonfinite_f16(const uint16_t* values, size_t count, uint32_t* flag,
                                     hipStream_t stream);

// Narrow variant (16-pixel tiles, v_mfma_f32_16x16x32_f16; dcn_kernels_narrow.hip).
int narrow_ksteps(const FusedGeometry& g);
size_t narrow_packed_bytes(const FusedGeometry& g);
hipError_t launch_prepack_narrow(const KShape& s, const FusedGeometry& g, const uint16_t* w,
                                 int layout, void* packed_w, hipStream_t stream);
// Where a kernel writes its output: NCHW, or channels coff.. of a CB8 tensor with cblk
// 8-channel blocks per image.
struct OutPlacement {
    int cb8 = 0;
    int coff = 0;
    int cblk = 0;
};
hipError_t launch_narrow_f16(const KShape& s, const FusedGeometry& g, const FusedConfig& cfg,
                             const void* cb8, const uint16_t* off, const uint16_t* mask,
                             const void* packed_w, const float* packed_b, uint16_t* out,
                             hipStream_t stream, OutPlacement place = OutPlacement{});

// Propagation-body kernels (dcn_kernels_body.hip, dcn_kernels_conv.hip).
constexpr int kLayoutNCHW = DCN_TENSOR_NCHW;
constexpr int kLayoutCB8 = DCN_TENSOR_CB8;

struct ConvGeometry {
    int cin, cout, h, w;
    int cb;      // ceil(cin / 8) input channel blocks
    int kb;      // K-blocks = 9 * cb
    int ksteps;  // K-steps of 4 K-blocks
    int chunks;  // 64-channel output chunks
    int nbt;     // 16-column blocks over all chunks
};
ConvGeometry conv_geometry(int cin, int cout, int height, int width);
size_t conv_packed_bytes(const ConvGeometry& g);
hipError_t launch_conv_prepack(const ConvGeometry& g, const uint16_t* w, const uint16_t* bias,
                               void* wpk, float* bpk, hipStream_t stream);
// A batch of `images` independent images in one launch (grid z): each tensor argument
// advances by its per-image stride in elements (zero for a tensor shared by the batch).
struct ConvBatch {
    int images = 1;
    long x = 0, res1 = 0, res2 = 0, out = 0;
    long out2 = 0;  // per-image stride of a conv pair's second (CB8) output
};
// The temporal preparation and the first conv_offset layer (196 -> 64, LeakyReLU) in one
// launch (one image): writes flow2, the DCN input and the backbone input's leading blocks
// as launch_body_temporal does, and the conv's output in CB8, without the conditions.
// warp_cb8: feat_prop and feat_n2 are CB8 tensors (8 blocks) instead of NCHW.
hipError_t launch_temporal_conv(const ConvGeometry& g, const uint16_t* feat_prop, const uint16_t* feat_current,
                                const uint16_t* feat_n2, const uint16_t* flow1, const uint16_t* prev_flow,
                                int has_second_order, const uint16_t* const* prefix, int nprefix,
                                uint16_t* flow2, uint16_t* deform_cb8, uint16_t* bb_cb8, const void* wpk,
                                const float* bias, float slope, uint16_t* out_cb8, hipStream_t stream,
                                bool warp_cb8 = false);
hipError_t launch_conv3x3(const ConvGeometry& g, const void* x_cb8, const void* wpk,
                          const float* bias, int act, float slope, const uint16_t* res1,
                          int res1_layout, const uint16_t* res2, int res2_layout, uint16_t* out,
                          int out_layout, hipStream_t stream, int res2_coff = 0,
                          const ConvBatch& batch = ConvBatch{});
// Two chained 64 -> 64 convs in one launch: t = half(act1(conv1(x) + b1)) held in LDS,
// then conv2 over t with launch_conv3x3's epilogue; bit-identical to two launches.
hipError_t launch_conv3x3_pair(const ConvGeometry& g1, const ConvGeometry& g2, const void* x_cb8,
                               const void* wpk1, const float* bias1, int act1, const void* wpk2,
                               const float* bias2, int act2, float slope, const uint16_t* res1,
                               int res1_layout, const uint16_t* res2, int res2_layout,
                               uint16_t* out, int out_layout, hipStream_t stream, int res2_coff = 0,
                               const ConvBatch& batch = ConvBatch{}, uint16_t* out2_cb8 = nullptr);
// SPyNet (dcn_kernels_spynet.hip).
constexpr int kSpynetMaxLevels = DCN_SPYNET_LEVELS;
struct ConvKGeometry {
    int ks, cin, cout, h, w;
    int cb;      // ceil(cin / 8)
    int kb;      // K-blocks = ks * ks * cb
    int ksteps;  // K-steps of 4 K-blocks
    int nb;      // 16-column blocks per workgroup (1, 2 or 4)
    int chunks;  // workgroup columns
    int nbt;     // 16-column blocks over all chunks
};
ConvKGeometry convk_geometry(int ks, int cin, int cout, int height, int width);
size_t convk_packed_bytes(const ConvKGeometry& g);
hipError_t launch_convk_prepack(const ConvKGeometry& g, const uint16_t* w, const uint16_t* bias, void* wpk,
                                float* bpk, hipStream_t stream);
// k x k conv over `batch` CB8 images with a `pad`-pixel zero border (pad >= ks / 2);
// act 2 = ReLU; base (optional, NCHW) makes out = half(base + half(acc)); out NCHW or CB8
// with the same border.
hipError_t launch_convk(const ConvKGeometry& g, int batch, int pad, const void* x_cb8, const void* wpk,
                        const float* bias, int act, const uint16_t* base, uint16_t* out, int out_cb8,
                        hipStream_t stream);
hipError_t launch_bicubic_quarter(const uint16_t* in, uint16_t* out, int channels, int height, int width,
                                  hipStream_t stream);
// Pyramids of `count` RGB frames (frame 0, frame 1, frame f >= 2 at frame0 + f * stride):
// level l of frame f at levels[l] + f * 3 * h_l * w_l, h_l = h >> (n - 1 - l).
hipError_t launch_spynet_pyramid(const uint16_t* frame0, const uint16_t* frame1, long frame_stride, int count,
                                 uint16_t* const* levels, int nlevels, int height, int width, hipStream_t stream);
// Images b < batch over `pairs` frame pairs: b < pairs is spynet(frame b, frame b + 1), the
// rest the reverse direction of pair b - pairs.
hipError_t launch_spynet_prepare(int batch, int pairs, const uint16_t* pyramid_level, const uint16_t* source_flow,
                                 int source_height, int source_width, int first_level, uint16_t* features, int pad,
                                 uint16_t* base_flow, int height, int width, hipStream_t stream);
// The leading levels with at most 16 pixels per image in one launch (one workgroup per
// image, activations in LDS); writes the last fused level's flow [b][2][h][w].
size_t spynet_small_lds_bytes(int units);
hipError_t launch_spynet_small(int batch, int pairs, int levels, const int* heights, const int* widths,
                               const uint16_t* const* pyramid, const void* const (*wpk)[5],
                               const float* const (*bias)[5], const uint32_t (*wpk_bytes)[5], uint16_t* flow_out,
                               hipStream_t stream);

// The last conv_offset layer (cout 432) with prepare_dcn_offsets_fp16 in its epilogue:
// raw = half(conv + bias), offsets = half(10 tanh(raw) + flow), masks = half(sigmoid(raw)).
// `images` images: CB8 inputs, flows [2][plane], offsets and masks at their own strides.
// The body's last conv_offset layer (64 -> 432 with the offset/mask transform) and its
// DCN (128 -> 64, narrow_kernel arithmetic) in one launch, the offsets kept in LDS; the
// aligned feature goes to channels out_coff.. of the CB8 backbone input (out_cblk blocks).
hipError_t launch_offsets_dcn(const ConvGeometry& goff, const void* xoff_cb8, const void* woff,
                              const float* boff, const uint16_t* flow1, const uint16_t* flow2,
                              const void* xin_cb8, const void* wdcn, size_t wdcn_bytes,
                              const float* bdcn, uint16_t* out_cb8, int out_coff, int out_cblk,
                              int images, hipStream_t stream);
hipError_t launch_conv3x3_offsets(const ConvGeometry& g, const void* x_cb8, const void* wpk,
                                  const float* bias, const uint16_t* flow1, const uint16_t* flow2,
                                  uint16_t* offset, uint16_t* mask, hipStream_t stream, int images = 1);
// One kernel for the body's temporal inputs: second-order flow (NCHW), conditions and
// the DCN input in CB8, and the backbone input's leading [feat_current, prefix...] in CB8.
// Backbone input of a branch's first step: [feat_current, prefix...] and a zero aligned
// slot, CB8 with 64 * (nprefix + 2) channels.
hipError_t launch_body_initial(const uint16_t* feat_current, const uint16_t* const* prefix, int nprefix,
                               uint16_t* bb_cb8, int H, int W, hipStream_t stream, int images = 1);
hipError_t launch_body_temporal(const uint16_t* feat_prop, const uint16_t* feat_current,
                                const uint16_t* feat_n2, const uint16_t* flow1,
                                const uint16_t* prev_flow, int has_second_order,
                                const uint16_t* const* prefix, int nprefix, uint16_t* flow2,
                                uint16_t* cond_cb8, uint16_t* deform_cb8, uint16_t* bb_cb8, int H,
                                int W, hipStream_t stream, int images = 1);
hipError_t launch_second_order_flow(const uint16_t* flow1, const uint16_t* prev, uint16_t* flow2,
                                    int H, int W, int has_second_order, hipStream_t stream);
hipError_t launch_temporal_assemble(const uint16_t* feat_prop, const uint16_t* feat_current,
                                    const uint16_t* feat_n2, const uint16_t* flow1,
                                    const uint16_t* flow2, uint16_t* conditions, int cond_layout,
                                    uint16_t* deform_input, int deform_layout, int H, int W,
                                    hipStream_t stream);
hipError_t launch_offset_transform(const uint16_t* raw, const uint16_t* flow1, const uint16_t* flow2,
                                   uint16_t* offset, uint16_t* mask, int plane, hipStream_t stream);
hipError_t launch_assemble(const uint16_t* const* sources, int count, uint16_t* out, int out_layout,
                           int H, int W, hipStream_t stream);
hipError_t launch_add_residual(const uint16_t* aligned, const uint16_t* backbone, uint16_t* out,
                               long count, hipStream_t stream);
hipError_t launch_cb8_to_nchw(const uint16_t* cb8, uint16_t* out, int C, int H, int W,
                              hipStream_t stream);
inline size_t cb8_tensor_elems(int channels, int h, int w) {
    return (size_t)((channels + 7) / 8) * 8 * (h + 2 * DCN_CB8_PAD) * (w + 2 * DCN_CB8_PAD);
}

// Constant of dev::fast_div: ceil(2^32 / d) for d > 1, 0 for d == 1.
inline uint32_t magic_for(int d) {
    return d <= 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + (uint64_t)d - 1) / (uint64_t)d);
}

// Bytes of the prepacked B-fragment buffer for a geometry.
inline size_t packed_weight_bytes(const FusedGeometry& g) {
    return (size_t)g.ksteps * g.nb * 64 * 8 * sizeof(uint16_t);
}
inline size_t cb8_bytes(const dcn_shape& s, const FusedGeometry& g) {
    return (size_t)s.batch * g.cblk * g.hp * g.wp * 16;
}

#if defined(__HIPCC__)
// Round an FP32 value to FP16 (nearest even) *as an FP32 register value*. The empty
// asm makes the value opaque, so the conversion cannot be folded into the operation
// that produced it (v_fma_mixlo_f16 would round an exact product or sum once, where
// the reference rounds to FP32 first and then to FP16).
__device__ __forceinline__ _Float16 round_f16(float v) {
    __asm__ volatile("" : "+v"(v));
    return (_Float16)v;
}
// The same for BF16 (nearest even, v_cvt_pk_bf16_f32), returned as its 16 bits.
__device__ __forceinline__ uint16_t round_bf16_bits(float v) {
    __asm__ volatile("" : "+v"(v));
    return __builtin_bit_cast(uint16_t, (__bf16)v);
}
#endif

// Host utilities (dcn_host_util.cpp).
uint16_t f32_to_f16_bits(float value);
float f16_bits_to_f32(uint16_t bits);

}  // namespace dcn

// Opaque handle types of the C ABI.
struct dcn_context {
    int device = 0;
    std::string last_error;
    void* workspace = nullptr;  // padded channel-block input copy
    size_t workspace_bytes = 0;
    uint32_t* flag = nullptr;   // device flag for the non-finite check
    dcn::FusedConfig fused_override{0, 0, 0, -1};
    unsigned long long* tile_clock = nullptr;  // dcn_set_tile_clock_dev (diagnostics)
    size_t tile_clock_count = 0;
};

struct dcn_packed {
    dcn_shape shape{};          // the layer shape the weights were packed for
    dcn::FusedGeometry geometry{};
    void* weights = nullptr;    // B fragments, packed_weight_bytes(geometry)
    void* weights_group = nullptr;  // per-group B fragments of the window variant (or null)
    void* weights_narrow = nullptr; // 16-wide B fragments of the narrow variant
    void* weights_tile = nullptr;   // tap-major B fragments of the tile variant (or null)
    float* bias = nullptr;      // Cout floats
    int device = 0;
    bool bf16 = false;          // BF16 weights (dcn_prepack_bf16*): narrow, window or register
                                // variant, no tile fragments
};
