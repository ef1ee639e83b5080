// Propagation-body glue kernels (BasicVSR++ second-order propagation, one branch):
// second-order flow, temporal alignment inputs, DCN offset/mask transform, backbone
// input assembly and the alignment residual. FP16 storage, FP32 arithmetic, each
// rounding where the reference's Metal kernels round.
//
// Tensor layouts: `NCHW` is the reference's planar [C][H][W] for one image; `CB8` is the
// padded channel-block layout of the fused kernels, [C/8][H+4][W+4][8] with a 2-pixel
// zero border (the conv3x3 and DCN kernels read it without bounds tests). Writers of a
// CB8 tensor touch only interior positions of real channels: the border and the
// channels past C stay as the owner cleared them.
#include <hip/hip_runtime.h>

#include "dcn_device.hpp"
#include "dcn_internal.hpp"
#include "dcn_warp.hpp"

#pragma clang fp contract(off)

namespace dcn {
namespace {

using namespace dev;
using namespace warp;

// Index of (channel c, pixel y, x) in a tensor of the given layout.
__device__ __forceinline__ size_t tensor_index(int layout, int c, int y, int x, int H, int W) {
    if (layout == kLayoutCB8) {
        const int Hp = H + 2 * kPad, Wp = W + 2 * kPad;
        return ((size_t)((c >> 3) * Hp + y + kPad) * Wp + x + kPad) * 8 + (c & 7);
    }
    return ((size_t)c * H + y) * W + x;
}

// accumulate_second_order_flow_fp16 (MetalShader.swift:738-763):
// flow2 = flow1 + warp(previous_flow, flow1), or zero without second order. Flows are
// [x, y] planes.
__global__ __launch_bounds__(256) void second_order_flow_kernel(const uint16_t* __restrict__ flow1,
                                                                const uint16_t* __restrict__ prev,
                                                                uint16_t* __restrict__ flow2, int H,
                                                                int W, int has_second_order) {
    const int plane = H * W;
    const int gid = blockIdx.x * 256 + threadIdx.x;
    if (gid >= 2 * plane) return;
    if (!has_second_order) {
        flow2[gid] = 0;
        return;
    }
    const int channel = gid / plane;
    const int spatial = gid - channel * plane;
    const int y = spatial / W;
    const int x = spatial - y * W;
    const float fx = h2f(flow1[spatial]);
    const float fy = h2f(flow1[plane + spatial]);
    const float previous = sample_zero(prev + (size_t)channel * plane, H, W, (float)y + fy, (float)x + fx);
    flow2[gid] = f2h(h2f(flow1[gid]) + previous);
}

// assemble_temporal_alignment_fp16 (MetalShader.swift:766-813):
// conditions[196] = [warp(featProp, flow1), featCurrent, warp(featN2, flow2), flow1, flow2],
// deformInput[128] = [featProp, featN2]; either output NCHW or CB8.
__global__ __launch_bounds__(256) void temporal_assemble_kernel(
    const uint16_t* __restrict__ feat_prop, const uint16_t* __restrict__ feat_current,
    const uint16_t* __restrict__ feat_n2, const uint16_t* __restrict__ flow1,
    const uint16_t* __restrict__ flow2, uint16_t* __restrict__ conditions, int cond_layout,
    uint16_t* __restrict__ deform_input, int deform_layout, int H, int W) {
    const int plane = H * W;
    const int gid = blockIdx.x * 256 + threadIdx.x;
    if (gid >= 196 * plane) return;
    const int channel = gid / plane;
    const int spatial = gid - channel * plane;
    const int y = spatial / W;
    const int x = spatial - y * W;
    if (channel < 128) {
        const uint16_t v = channel < 64 ? feat_prop[gid] : feat_n2[(size_t)(channel - 64) * plane + spatial];
        deform_input[tensor_index(deform_layout, channel, y, x, H, W)] = v;
    }
    uint16_t c;
    if (channel < 64) {
        const float fx = h2f(flow1[spatial]);
        const float fy = h2f(flow1[plane + spatial]);
        c = f2h(sample_zero(feat_prop + (size_t)channel * plane, H, W, (float)y + fy, (float)x + fx));
    } else if (channel < 128) {
        c = feat_current[(size_t)(channel - 64) * plane + spatial];
    } else if (channel < 192) {
        const float fx = h2f(flow2[spatial]);
        const float fy = h2f(flow2[plane + spatial]);
        c = f2h(sample_zero(feat_n2 + (size_t)(channel - 128) * plane, H, W, (float)y + fy, (float)x + fx));
    } else if (channel < 194) {
        c = flow1[(size_t)(channel - 192) * plane + spatial];
    } else {
        c = flow2[(size_t)(channel - 194) * plane + spatial];
    }
    conditions[tensor_index(cond_layout, channel, y, x, H, W)] = c;
}

// prepare_dcn_offsets_fp16 (MetalShader.swift:815-839): raw conv_offset output
// [o1 (144), o2 (144), mask (144)] -> offsets 10*tanh(raw) + flow (interleaved dy, dx;
// first 144 channels with flow1, next 144 with flow2) and sigmoid masks.
__global__ __launch_bounds__(256) void offset_transform_kernel(const uint16_t* __restrict__ raw,
                                                               const uint16_t* __restrict__ flow1,
                                                               const uint16_t* __restrict__ flow2,
                                                               uint16_t* __restrict__ offset,
                                                               uint16_t* __restrict__ mask,
                                                               int plane) {
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;
    if (gid >= 432L * plane) return;
    const int channel = (int)(gid / plane);
    const int spatial = (int)(gid - (long)channel * plane);
    if (channel < 288) {
        const int local = channel % 144;
        const uint16_t* flow = channel < 144 ? flow1 : flow2;
        const int flow_channel = (local & 1) == 0 ? 1 : 0;  // flow is [x, y]; even = dy
        const float residue = 10.0f * tanhf(h2f(raw[gid]));
        offset[gid] = f2h(residue + h2f(flow[(size_t)flow_channel * plane + spatial]));
    } else {
        const float value = h2f(raw[gid]);
        mask[(size_t)(channel - 288) * plane + spatial] = f2h(1.0f / (1.0f + expf(-value)));
    }
}

struct AssembleArgs {
    const uint16_t* src[5];  // 64-channel NCHW sources, in channel order
    int sources;
    uint16_t* out;
    int out_layout;
    int H, W;
};

// assemble_propagation_backbone_fp16 / assemble_temporal_backbone_fp16
// (MetalShader.swift:841-855, 899-929): concatenate 64-channel planar sources.
__global__ __launch_bounds__(256) void assemble_kernel(AssembleArgs a) {
    const int plane = a.H * a.W;
    const int gid = blockIdx.x * 256 + threadIdx.x;
    if (gid >= 64 * a.sources * plane) return;
    const int channel = gid / plane;
    const int spatial = gid - channel * plane;
    const int source = channel >> 6;
    const int y = spatial / a.W;
    const int x = spatial - y * a.W;
    const uint16_t* s = a.src[0];
#pragma unroll
    for (int i = 1; i < 5; ++i)
        if (source == i) s = a.src[i];
    a.out[tensor_index(a.out_layout, channel, y, x, a.H, a.W)] = s[(size_t)(channel & 63) * plane + spatial];
}

// add_propagation_residual_fp16 (MetalShader.swift:857-867): out = half(aligned + backbone).
__global__ __launch_bounds__(256) void add_residual_kernel(const uint16_t* __restrict__ aligned,
                                                           const uint16_t* __restrict__ backbone,
                                                           uint16_t* __restrict__ out, long count) {
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;
    if (gid < count) out[gid] = f2h(h2f(aligned[gid]) + h2f(backbone[gid]));
}

// CB8 <-> NCHW for one image of C channels (C % 8 == 0 not required: channels past C
// are neither read nor written).
__global__ __launch_bounds__(256) void cb8_to_nchw_kernel(const uint16_t* __restrict__ cb8,
                                                          uint16_t* __restrict__ out, int C, int H,
                                                          int W) {
    const int plane = H * W;
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (long)C * plane) return;
    const int channel = (int)(gid / plane);
    const int spatial = (int)(gid - (long)channel * plane);
    const int y = spatial / W;
    const int x = spatial - y * W;
    out[gid] = cb8[tensor_index(kLayoutCB8, channel, y, x, H, W)];
}

struct BodyTemporalArgs {
    const uint16_t *feat_prop, *feat_current, *feat_n2, *flow1, *prev_flow;
    const uint16_t* prefix[3];
    int nprefix, has_second_order, H, W;
    uint16_t *flow2, *cond, *deform, *bb;
};

// The arguments of image blockIdx.z of a batch of tiles: features [64][H][W] and flows
// [2][H][W] per image; CB8 conditions (25 blocks), DCN input (16) and backbone input
// (8 (nprefix + 2)) per image. Plain fields, no array and no member function: either
// would keep the local struct in scratch memory (measured: 7.4 -> 18 us).
struct BodyImage {
    const uint16_t *feat_prop, *feat_current, *feat_n2, *flow1, *prev_flow, *p0, *p1, *p2;
    uint16_t *flow2, *cond, *deform, *bb;
    int nprefix, has_second_order, H, W;
};

__device__ __forceinline__ BodyImage temporal_image(const BodyTemporalArgs& a0) {
    BodyImage a;
    const long z = blockIdx.z;
    const long fs = z * 64 * a0.H * a0.W;  // per-image offset of a feature, then of a flow
    const long ls = z * 2 * a0.H * a0.W;
    const long unit = (long)(a0.H + 2 * kPad) * (a0.W + 2 * kPad) * 8;
    a.feat_prop = a0.feat_prop + fs;
    a.feat_current = a0.feat_current + fs;
    a.feat_n2 = a0.feat_n2 + fs;
    a.flow1 = a0.flow1 + ls;
    a.prev_flow = a0.prev_flow + ls;
    a.p0 = a0.prefix[0] + fs;
    a.p1 = a0.prefix[1] + fs;
    a.p2 = a0.prefix[2] + fs;
    a.flow2 = a0.flow2 + ls;
    a.cond = a0.cond + z * 25 * unit;
    a.deform = a0.deform + z * 16 * unit;
    a.bb = a0.bb + z * 8 * (a0.nprefix + 2) * unit;
    a.nprefix = a0.nprefix;
    a.has_second_order = a0.has_second_order;
    a.H = a0.H;
    a.W = a0.W;
    return a;
}

// The body's temporal inputs in one pass. Workgroup row blockIdx.y selects an 8-channel
// output block: 0-24 the conditions [warp(feat_prop, flow1), feat_current,
// warp(feat_n2, flow2), flow1, flow2, 4 zero channels], 25-40 the DCN input
// [feat_prop, feat_n2], then the backbone input's [feat_current, prefix...]; one thread
// per pixel writes the block's 16 bytes of CB8. The second-order flow of a pixel is
// recomputed by each thread that needs it (same arithmetic, same bits) and stored by
// the flow block's thread.
__global__ __launch_bounds__(256) void body_temporal_kernel(BodyTemporalArgs a0) {
    const BodyImage a = temporal_image(a0);
    const int plane = a.H * a.W;
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= plane) return;
    const int kind = blockIdx.y;
    const int y = p / a.W;
    const int x = p - y * a.W;
    const size_t pl = (size_t)plane;
    uint16_t* dst;
    int dblock;
    u32x4 out;
    if (kind < 25) {
        dst = a.cond;
        dblock = kind;
        uint16_t f2[2];
        out = condition_block<u32x4>(a.feat_prop, a.feat_current, a.feat_n2, a.flow1, a.prev_flow,
                                     a.has_second_order, a.H, a.W, kind, y, x, f2);
        if (kind == 24) {
            a.flow2[p] = f2[0];
            a.flow2[pl + p] = f2[1];
        }
    } else if (kind < 41) {
        dst = a.deform;
        dblock = kind - 25;
        out = copy8<u32x4>(dblock < 8 ? a.feat_prop + (size_t)dblock * 8 * pl : a.feat_n2 + (size_t)(dblock - 8) * 8 * pl,
                           pl, p);
    } else {
        dst = a.bb;
        dblock = kind - 41;
        const int src = dblock >> 3;
        const uint16_t* base = src == 0 ? a.feat_current : (src == 1 ? a.p0 : (src == 2 ? a.p1 : a.p2));
        out = copy8<u32x4>(base + (size_t)(dblock & 7) * 8 * pl, pl, p);
    }
    const int Hp = a.H + 2 * kPad, Wp = a.W + 2 * kPad;
    reinterpret_cast<u32x4*>(dst)[((size_t)dblock * Hp + y + kPad) * Wp + x + kPad] = out;
}

// The backbone input of a branch's first step: [feat_current, prefix...] copied into CB8
// and the aligned slot (the last 64 channels) written as zeros. Workgroup row blockIdx.y
// is the 8-channel output block.
__global__ __launch_bounds__(256) void body_initial_kernel(BodyTemporalArgs a0) {
    const BodyImage a = temporal_image(a0);
    const int plane = a.H * a.W;
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= plane) return;
    const int dblock = blockIdx.y;
    const int y = p / a.W;
    const int x = p - y * a.W;
    const size_t pl = (size_t)plane;
    const int src = dblock >> 3;
    u32x4 out = {0u, 0u, 0u, 0u};
    if (src <= a.nprefix) {
        const uint16_t* base = src == 0 ? a.feat_current : (src == 1 ? a.p0 : (src == 2 ? a.p1 : a.p2));
        const uint16_t* copy_src = base + (size_t)(dblock & 7) * 8 * pl;
        uint16_t h[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) h[c] = copy_src[(size_t)c * pl + p];
#pragma unroll
        for (int d = 0; d < 4; ++d) out[d] = (uint32_t)h[2 * d] | ((uint32_t)h[2 * d + 1] << 16);
    }
    const int Hp = a.H + 2 * kPad, Wp = a.W + 2 * kPad;
    reinterpret_cast<u32x4*>(a.bb)[((size_t)dblock * Hp + y + kPad) * Wp + x + kPad] = out;
}

unsigned blocks_for(long n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t launch_second_order_flow(const uint16_t* flow1, const uint16_t* prev, uint16_t* flow2,
                                    int H, int W, int has_second_order, hipStream_t stream) {
    hipLaunchKernelGGL(second_order_flow_kernel, dim3(blocks_for(2L * H * W)), dim3(256), 0, stream,
                       flow1, prev, flow2, H, W, has_second_order);
    return hipGetLastError();
}

hipError_t launch_temporal_assemble(const uint16_t* feat_prop, const uint16_t* feat_current,
                                    const uint16_t* feat_n2, const uint16_t* flow1,
                                    const uint16_t* flow2, uint16_t* conditions, int cond_layout,
                                    uint16_t* deform_input, int deform_layout, int H, int W,
                                    hipStream_t stream) {
    hipLaunchKernelGGL(temporal_assemble_kernel, dim3(blocks_for(196L * H * W)), dim3(256), 0, stream,
                       feat_prop, feat_current, feat_n2, flow1, flow2, conditions, cond_layout,
                       deform_input, deform_layout, H, W);
    return hipGetLastError();
}

hipError_t launch_body_temporal(const uint16_t* feat_prop, const uint16_t* feat_current,
                                const uint16_t* feat_n2, const uint16_t* flow1,
                                const uint16_t* prev_flow, int has_second_order,
                                const uint16_t* const* prefix, int nprefix, uint16_t* flow2,
                                uint16_t* cond_cb8, uint16_t* deform_cb8, uint16_t* bb_cb8, int H,
                                int W, hipStream_t stream, int images) {
    if (nprefix < 0 || nprefix > 3 || images < 1) return hipErrorInvalidValue;
    BodyTemporalArgs a{};
    a.feat_prop = feat_prop;
    a.feat_current = feat_current;
    a.feat_n2 = feat_n2;
    a.flow1 = flow1;
    a.prev_flow = prev_flow;
    for (int i = 0; i < 3; ++i) a.prefix[i] = i < nprefix ? prefix[i] : feat_current;
    a.nprefix = nprefix;
    a.has_second_order = has_second_order;
    a.H = H;
    a.W = W;
    a.flow2 = flow2;
    a.cond = cond_cb8;
    a.deform = deform_cb8;
    a.bb = bb_cb8;
    const dim3 grid(blocks_for((long)H * W), (unsigned)(41 + 8 * (1 + nprefix)), (unsigned)images);
    hipLaunchKernelGGL(body_temporal_kernel, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_body_initial(const uint16_t* feat_current, const uint16_t* const* prefix, int nprefix,
                               uint16_t* bb_cb8, int H, int W, hipStream_t stream, int images) {
    if (nprefix < 0 || nprefix > 3 || images < 1) return hipErrorInvalidValue;
    BodyTemporalArgs a{};
    a.feat_current = feat_current;
    for (int i = 0; i < 3; ++i) a.prefix[i] = i < nprefix ? prefix[i] : feat_current;
    a.nprefix = nprefix;
    a.H = H;
    a.W = W;
    a.bb = bb_cb8;
    const dim3 grid(blocks_for((long)H * W), (unsigned)(8 * (2 + nprefix)), (unsigned)images);
    hipLaunchKernelGGL(body_initial_kernel, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_offset_transform(const uint16_t* raw, const uint16_t* flow1, const uint16_t* flow2,
                                   uint16_t* offset, uint16_t* mask, int plane, hipStream_t stream) {
    hipLaunchKernelGGL(offset_transform_kernel, dim3(blocks_for(432L * plane)), dim3(256), 0, stream,
                       raw, flow1, flow2, offset, mask, plane);
    return hipGetLastError();
}

hipError_t launch_assemble(const uint16_t* const* sources, int count, uint16_t* out, int out_layout,
                           int H, int W, hipStream_t stream) {
    if (count < 1 || count > 5) return hipErrorInvalidValue;
    AssembleArgs a{};
    for (int i = 0; i < count; ++i) a.src[i] = sources[i];
    for (int i = count; i < 5; ++i) a.src[i] = sources[0];
    a.sources = count;
    a.out = out;
    a.out_layout = out_layout;
    a.H = H;
    a.W = W;
    hipLaunchKernelGGL(assemble_kernel, dim3(blocks_for(64L * count * H * W)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_add_residual(const uint16_t* aligned, const uint16_t* backbone, uint16_t* out,
                               long count, hipStream_t stream) {
    hipLaunchKernelGGL(add_residual_kernel, dim3(blocks_for(count)), dim3(256), 0, stream, aligned,
                       backbone, out, count);
    return hipGetLastError();
}

hipError_t launch_cb8_to_nchw(const uint16_t* cb8, uint16_t* out, int C, int H, int W,
                              hipStream_t stream) {
    hipLaunchKernelGGL(cb8_to_nchw_kernel, dim3(blocks_for((long)C * H * W)), dim3(256), 0, stream,
                       cb8, out, C, H, W);
    return hipGetLastError();
}

}  // namespace dcn
