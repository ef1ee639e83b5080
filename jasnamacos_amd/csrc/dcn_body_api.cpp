// C-ABI host layer of the propagation body: glue entry points, conv3x3 layers and the
// per-step body with hipGraph capture. Reference: runDCNOffsetTransform and
// runTemporalPreparation (MetalRunner.swift:469-582), the body glue kernels
// (MetalShader.swift:738-929) and the per-step body of verifyFusedFourPassRecurrence
// (FusedFourPassRecurrenceProbe.swift:570-664, retained graph :904-937).
#include <cstring>
#include <string>
#include <vector>

#include "dcn_host.hpp"
#include "dcn_internal.hpp"

using namespace dcn::host;

struct dcn_conv {
    dcn::ConvGeometry g{};
    void* wpk = nullptr;
    float* bias = nullptr;
    int device = 0;
};

struct dcn_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int device = 0;
};

struct dcn_clip {
    dcn_context* ctx = nullptr;
    int h = 0, w = 0, frames = 0, blocks = 0, tiles = 1;
    dcn_body* body[4] = {};
    uint16_t* zero_feat = nullptr;  // 64 x plane zeros: the feat_n2 of positions 0 and 1
    uint16_t* flow2 = nullptr;      // 2 x plane second-order flow scratch
    uint16_t* triplet_prop = nullptr;  // [4][3][64] x plane: the zero-motion triplet rung's output
    // Single-tile clips: a CB8 copy of every propagated feature ([4][T] tensors of 8
    // blocks), written by each step's last conv pair and warped by the next steps, a CB8
    // zero feature, and the triplet rung's mirrors ([4][3]).
    uint16_t* mirror = nullptr;
    uint16_t* zero_cb8 = nullptr;
    uint16_t* triplet_mirror = nullptr;
    std::vector<void*> buffers;
    hipStream_t capture_stream = nullptr;
};

struct dcn_body {
    dcn_context* ctx = nullptr;
    int h = 0, w = 0, branch = 0, blocks = 0, tiles = 1;  // tiles: images per step
    dcn_conv* offset_conv[4] = {};
    dcn_conv* backbone[1 + 2 * DCN_BODY_MAX_BLOCKS] = {};
    dcn_packed* dcn = nullptr;
    std::vector<void*> buffers;  // every device intermediate, freed with the body
    uint16_t* cond_cb8 = nullptr;    // conditions, 196 channels
    uint16_t* deform_cb8 = nullptr;  // DCN input [feat_prop, feat_n2], 128 channels
    uint16_t* off_a = nullptr;       // conv_offset intermediates, 64 channels CB8
    uint16_t* off_b = nullptr;
    uint16_t* bb_in = nullptr;       // backbone input [feat_current, prefix..., aligned] CB8
    uint16_t* feat[2] = {};          // backbone features, 64 channels CB8
    hipStream_t capture_stream = nullptr;
};

namespace {

dcn_status check_plane(dcn_context* ctx, int width, int height) {
    if (width <= 0 || height <= 0 || (long long)width * height * 432 >= (1LL << 30))
        return fail(ctx, DCN_INVALID_SHAPE, "invalid body plane size");
    return DCN_OK;
}

dcn_status require_count(dcn_context* ctx, size_t actual, size_t expected) {
    // The reference's guards throw invalidShape on any count mismatch
    // (MetalRunner.swift:475-477, :520-526).
    if (actual != expected) return fail(ctx, DCN_INVALID_SHAPE, "array count does not match the plane");
    return DCN_OK;
}

template <typename T>
dcn_status alloc(dcn_context* ctx, std::vector<void*>& owned, T** p, size_t elems) {
    void* raw = nullptr;
    DCN_HIP(ctx, hipMalloc(&raw, std::max<size_t>(elems, 1) * sizeof(uint16_t)));
    owned.push_back(raw);
    *p = static_cast<T*>(raw);
    return DCN_OK;
}

dcn_status run_conv(dcn_context* ctx, const dcn_conv* c, const void* x, int act, const void* r1,
                    int r1_layout, const void* r2, int r2_layout, void* out, int out_layout,
                    hipStream_t stream, const dcn::ConvBatch& batch = dcn::ConvBatch{}) {
    DCN_HIP(ctx, dcn::launch_conv3x3(c->g, x, c->wpk, c->bias, act, 0.1f, (const uint16_t*)r1,
                                     r1_layout, (const uint16_t*)r2, r2_layout, (uint16_t*)out,
                                     out_layout, stream, 0, batch));
    return DCN_OK;
}

// Elements per image of a CB8 tensor of `blocks` 8-channel blocks.
long cb8_image(const dcn_body* b, int blocks) {
    return (long)blocks * (b->h + 2 * DCN_CB8_PAD) * (b->w + 2 * DCN_CB8_PAD) * 8;
}

dcn_shape body_dcn_shape(int h, int w) {
    return dcn_shape{1, 128, h, w, 64, h, w, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16};
}

}  // namespace

extern "C" {

size_t dcn_cb8_tensor_count(int channels, int height, int width) {
    if (channels <= 0 || height <= 0 || width <= 0) return 0;
    return dcn::cb8_tensor_elems(channels, height, width);
}

dcn_status dcn_offset_transform_f16_dev(dcn_context* ctx, size_t plane, const void* d_raw,
                                        const void* d_flow1, const void* d_flow2, void* d_offset,
                                        void* d_mask, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    if (plane == 0 || plane * 432 >= ((size_t)1 << 30))
        return fail(ctx, DCN_INVALID_SHAPE, "invalid plane size");
    if (!d_raw || !d_flow1 || !d_flow2 || !d_offset || !d_mask)
        return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DeviceGuard guard(ctx->device);
    DCN_HIP(ctx, dcn::launch_offset_transform((const uint16_t*)d_raw, (const uint16_t*)d_flow1,
                                              (const uint16_t*)d_flow2, (uint16_t*)d_offset,
                                              (uint16_t*)d_mask, (int)plane, (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_offset_transform_f16(dcn_context* ctx, size_t plane, const uint16_t* raw,
                                    size_t raw_count, const uint16_t* flow1, size_t flow1_count,
                                    const uint16_t* flow2, size_t flow2_count, uint16_t* offset,
                                    size_t offset_count, uint16_t* mask, size_t mask_count) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    if (plane == 0) return fail(ctx, DCN_INVALID_SHAPE, "plane is 0");
    DCN_TRY(require_count(ctx, raw_count, 432 * plane));
    DCN_TRY(require_count(ctx, flow1_count, 2 * plane));
    DCN_TRY(require_count(ctx, flow2_count, 2 * plane));
    DCN_TRY(require_count(ctx, offset_count, 288 * plane));
    DCN_TRY(require_count(ctx, mask_count, 144 * plane));
    if (!raw || !flow1 || !flow2 || !offset || !mask)
        return fail(ctx, DCN_INVALID_ARGUMENT, "host pointer is null");
    DeviceGuard guard(ctx->device);
    DevBuf r, f1, f2, o, m;
    DCN_TRY(upload(ctx, r, raw, raw_count));
    DCN_TRY(upload(ctx, f1, flow1, flow1_count));
    DCN_TRY(upload(ctx, f2, flow2, flow2_count));
    DCN_HIP(ctx, hipMalloc(&o.p, offset_count * 2));
    DCN_HIP(ctx, hipMalloc(&m.p, mask_count * 2));
    DCN_TRY(dcn_offset_transform_f16_dev(ctx, plane, r.p, f1.p, f2.p, o.p, m.p, nullptr));
    DCN_HIP(ctx, hipMemcpy(offset, o.p, offset_count * 2, hipMemcpyDeviceToHost));
    DCN_HIP(ctx, hipMemcpy(mask, m.p, mask_count * 2, hipMemcpyDeviceToHost));
    return DCN_OK;
}

dcn_status dcn_temporal_prepare_f16_dev(dcn_context* ctx, int width, int height,
                                        const void* d_feat_prop, const void* d_feat_current,
                                        const void* d_feat_n2, const void* d_flow1,
                                        const void* d_prev_flow, int has_second_order,
                                        void* d_flow2, void* d_conditions,
                                        dcn_tensor_layout conditions_layout, void* d_deform_input,
                                        dcn_tensor_layout deform_input_layout, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DCN_TRY(check_plane(ctx, width, height));
    if (!d_feat_prop || !d_feat_current || !d_feat_n2 || !d_flow1 || !d_prev_flow || !d_flow2 ||
        !d_conditions || !d_deform_input)
        return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    if ((conditions_layout != DCN_TENSOR_NCHW && conditions_layout != DCN_TENSOR_CB8) ||
        (deform_input_layout != DCN_TENSOR_NCHW && deform_input_layout != DCN_TENSOR_CB8))
        return fail(ctx, DCN_INVALID_ARGUMENT, "unknown tensor layout");
    DeviceGuard guard(ctx->device);
    const hipStream_t s = (hipStream_t)stream;
    DCN_HIP(ctx, dcn::launch_second_order_flow((const uint16_t*)d_flow1, (const uint16_t*)d_prev_flow,
                                               (uint16_t*)d_flow2, height, width,
                                               has_second_order ? 1 : 0, s));
    DCN_HIP(ctx, dcn::launch_temporal_assemble(
                     (const uint16_t*)d_feat_prop, (const uint16_t*)d_feat_current,
                     (const uint16_t*)d_feat_n2, (const uint16_t*)d_flow1, (const uint16_t*)d_flow2,
                     (uint16_t*)d_conditions, conditions_layout, (uint16_t*)d_deform_input,
                     deform_input_layout, height, width, s));
    return DCN_OK;
}

dcn_status dcn_temporal_prepare_f16(dcn_context* ctx, int width, int height,
                                    const uint16_t* feat_prop, size_t feat_prop_count,
                                    const uint16_t* feat_current, size_t feat_current_count,
                                    const uint16_t* feat_n2, size_t feat_n2_count,
                                    const uint16_t* flow1, size_t flow1_count,
                                    const uint16_t* prev_flow, size_t prev_flow_count,
                                    int has_second_order, uint16_t* conditions,
                                    size_t conditions_count, uint16_t* deform_input,
                                    size_t deform_input_count, uint16_t* flow2, size_t flow2_count) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DCN_TRY(check_plane(ctx, width, height));
    const size_t plane = (size_t)width * height;
    DCN_TRY(require_count(ctx, feat_prop_count, 64 * plane));
    DCN_TRY(require_count(ctx, feat_current_count, 64 * plane));
    DCN_TRY(require_count(ctx, feat_n2_count, 64 * plane));
    DCN_TRY(require_count(ctx, flow1_count, 2 * plane));
    DCN_TRY(require_count(ctx, prev_flow_count, 2 * plane));
    DCN_TRY(require_count(ctx, conditions_count, 196 * plane));
    DCN_TRY(require_count(ctx, deform_input_count, 128 * plane));
    DCN_TRY(require_count(ctx, flow2_count, 2 * plane));
    if (!feat_prop || !feat_current || !feat_n2 || !flow1 || !prev_flow || !conditions ||
        !deform_input || !flow2)
        return fail(ctx, DCN_INVALID_ARGUMENT, "host pointer is null");
    DeviceGuard guard(ctx->device);
    DevBuf fp, fc, fn, f1, pf, f2, c, d;
    DCN_TRY(upload(ctx, fp, feat_prop, feat_prop_count));
    DCN_TRY(upload(ctx, fc, feat_current, feat_current_count));
    DCN_TRY(upload(ctx, fn, feat_n2, feat_n2_count));
    DCN_TRY(upload(ctx, f1, flow1, flow1_count));
    DCN_TRY(upload(ctx, pf, prev_flow, prev_flow_count));
    DCN_HIP(ctx, hipMalloc(&f2.p, flow2_count * 2));
    DCN_HIP(ctx, hipMalloc(&c.p, conditions_count * 2));
    DCN_HIP(ctx, hipMalloc(&d.p, deform_input_count * 2));
    DCN_TRY(dcn_temporal_prepare_f16_dev(ctx, width, height, fp.p, fc.p, fn.p, f1.p, pf.p,
                                         has_second_order, f2.p, c.p, DCN_TENSOR_NCHW, d.p,
                                         DCN_TENSOR_NCHW, nullptr));
    DCN_HIP(ctx, hipMemcpy(conditions, c.p, conditions_count * 2, hipMemcpyDeviceToHost));
    DCN_HIP(ctx, hipMemcpy(deform_input, d.p, deform_input_count * 2, hipMemcpyDeviceToHost));
    DCN_HIP(ctx, hipMemcpy(flow2, f2.p, flow2_count * 2, hipMemcpyDeviceToHost));
    return DCN_OK;
}

dcn_status dcn_assemble_backbone_f16_dev(dcn_context* ctx, int width, int height,
                                         const void* const* d_sources, int count, void* d_out,
                                         dcn_tensor_layout layout, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DCN_TRY(check_plane(ctx, width, height));
    if (!d_sources || count < 1 || count > 5 || !d_out)
        return fail(ctx, DCN_INVALID_ARGUMENT, "assemble needs 1..5 sources and an output");
    if (layout != DCN_TENSOR_NCHW && layout != DCN_TENSOR_CB8)
        return fail(ctx, DCN_INVALID_ARGUMENT, "unknown tensor layout");
    const uint16_t* src[5];
    for (int i = 0; i < count; ++i) {
        if (!d_sources[i]) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
        src[i] = (const uint16_t*)d_sources[i];
    }
    DeviceGuard guard(ctx->device);
    DCN_HIP(ctx, dcn::launch_assemble(src, count, (uint16_t*)d_out, layout, height, width,
                                      (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_add_residual_f16_dev(dcn_context* ctx, size_t count, const void* d_aligned,
                                    const void* d_backbone, void* d_out, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    if (!d_aligned || !d_backbone || !d_out) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    if (count == 0) return DCN_OK;
    DeviceGuard guard(ctx->device);
    DCN_HIP(ctx, dcn::launch_add_residual((const uint16_t*)d_aligned, (const uint16_t*)d_backbone,
                                          (uint16_t*)d_out, (long)count, (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_cb8_to_nchw_f16_dev(dcn_context* ctx, int channels, int height, int width,
                                   const void* d_cb8, void* d_out, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DCN_TRY(check_plane(ctx, width, height));
    if (channels <= 0 || (long long)channels * width * height >= (1LL << 30))
        return fail(ctx, DCN_INVALID_SHAPE, "invalid channel count");
    if (!d_cb8 || !d_out) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DeviceGuard guard(ctx->device);
    DCN_HIP(ctx, dcn::launch_cb8_to_nchw((const uint16_t*)d_cb8, (uint16_t*)d_out, channels, height,
                                         width, (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_conv3x3_create_dev(dcn_context* ctx, int cin, int cout, int height, int width,
                                  const void* d_weight, const void* d_bias, void* stream,
                                  dcn_conv** out) {
    if (!ctx || !out) return DCN_INVALID_ARGUMENT;
    *out = nullptr;
    DCN_TRY(check_plane(ctx, width, height));
    if (cin <= 0 || cout <= 0 || cin > 4096 || cout > 4096)
        return fail(ctx, DCN_INVALID_SHAPE, "invalid conv channel counts");
    if (!d_weight || !d_bias) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DeviceGuard guard(ctx->device);
    auto* c = new dcn_conv();
    c->g = dcn::conv_geometry(cin, cout, height, width);
    c->device = ctx->device;
    if (hipMalloc(&c->wpk, dcn::conv_packed_bytes(c->g)) != hipSuccess ||
        hipMalloc((void**)&c->bias, (size_t)cout * sizeof(float)) != hipSuccess) {
        dcn_conv3x3_free(c);
        return fail(ctx, DCN_COMMAND_FAILED, "hipMalloc of packed conv weights failed");
    }
    const hipError_t e = dcn::launch_conv_prepack(c->g, (const uint16_t*)d_weight,
                                                  (const uint16_t*)d_bias, c->wpk, c->bias,
                                                  (hipStream_t)stream);
    if (e != hipSuccess) {
        dcn_conv3x3_free(c);
        return hip_fail(ctx, e, "conv prepack launch");
    }
    *out = c;
    return DCN_OK;
}

void dcn_conv3x3_free(dcn_conv* conv) {
    if (!conv) return;
    DeviceGuard guard(conv->device);
    if (conv->wpk) (void)hipFree(conv->wpk);
    if (conv->bias) (void)hipFree(conv->bias);
    delete conv;
}

dcn_status dcn_conv3x3_f16_dev(dcn_context* ctx, const dcn_conv* conv, const void* d_x_cb8,
                               int activation, float slope, const void* d_res1,
                               dcn_tensor_layout res1_layout, const void* d_res2,
                               dcn_tensor_layout res2_layout, void* d_out,
                               dcn_tensor_layout out_layout, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    if (!conv || !d_x_cb8 || !d_out) return fail(ctx, DCN_INVALID_ARGUMENT, "null conv or pointer");
    if (activation < 0 || activation > 2) return fail(ctx, DCN_INVALID_ARGUMENT, "unknown activation");
    for (int l : {(int)res1_layout, (int)res2_layout, (int)out_layout})
        if (l != DCN_TENSOR_NCHW && l != DCN_TENSOR_CB8)
            return fail(ctx, DCN_INVALID_ARGUMENT, "unknown tensor layout");
    DeviceGuard guard(ctx->device);
    DCN_HIP(ctx, dcn::launch_conv3x3(conv->g, d_x_cb8, conv->wpk, conv->bias, activation, slope,
                                     (const uint16_t*)d_res1, res1_layout, (const uint16_t*)d_res2,
                                     res2_layout, (uint16_t*)d_out, out_layout, (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_conv3x3_offsets_f16_dev(dcn_context* ctx, const dcn_conv* conv, const void* d_x_cb8,
                                       const void* d_flow1, const void* d_flow2, void* d_offset,
                                       void* d_mask, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    if (!conv || !d_x_cb8 || !d_flow1 || !d_flow2 || !d_offset || !d_mask)
        return fail(ctx, DCN_INVALID_ARGUMENT, "null conv or pointer");
    if (conv->g.cout != 432) return fail(ctx, DCN_INVALID_SHAPE, "the offset conv has 432 output channels");
    DeviceGuard guard(ctx->device);
    DCN_HIP(ctx, dcn::launch_conv3x3_offsets(conv->g, d_x_cb8, conv->wpk, conv->bias, (const uint16_t*)d_flow1,
                                             (const uint16_t*)d_flow2, (uint16_t*)d_offset, (uint16_t*)d_mask,
                                             (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_conv3x3_pair_f16_dev(dcn_context* ctx, const dcn_conv* conv1, const dcn_conv* conv2,
                                    const void* d_x_cb8, int activation1, int activation2, float slope,
                                    const void* d_res1, dcn_tensor_layout res1_layout, const void* d_res2,
                                    dcn_tensor_layout res2_layout, void* d_out, dcn_tensor_layout out_layout,
                                    void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    if (!conv1 || !conv2 || !d_x_cb8 || !d_out) return fail(ctx, DCN_INVALID_ARGUMENT, "null conv or pointer");
    for (int act : {activation1, activation2})
        if (act < 0 || act > 2) return fail(ctx, DCN_INVALID_ARGUMENT, "unknown activation");
    for (int l : {(int)res1_layout, (int)res2_layout, (int)out_layout})
        if (l != DCN_TENSOR_NCHW && l != DCN_TENSOR_CB8)
            return fail(ctx, DCN_INVALID_ARGUMENT, "unknown tensor layout");
    if (conv1->g.cin != 64 || conv1->g.cout != 64 || conv2->g.cin != 64 || conv2->g.cout != 64 ||
        conv1->g.h != conv2->g.h || conv1->g.w != conv2->g.w)
        return fail(ctx, DCN_INVALID_SHAPE, "a conv pair needs two 64 -> 64 convs of one plane");
    DeviceGuard guard(ctx->device);
    DCN_HIP(ctx, dcn::launch_conv3x3_pair(conv1->g, conv2->g, d_x_cb8, conv1->wpk, conv1->bias, activation1,
                                          conv2->wpk, conv2->bias, activation2, slope,
                                          (const uint16_t*)d_res1, res1_layout, (const uint16_t*)d_res2,
                                          res2_layout, (uint16_t*)d_out, out_layout, (hipStream_t)stream));
    return DCN_OK;
}

void dcn_body_destroy(dcn_body* body) {
    if (!body) return;
    DeviceGuard guard(body->ctx ? body->ctx->device : 0);
    for (auto* c : body->offset_conv) dcn_conv3x3_free(c);
    for (auto* c : body->backbone) dcn_conv3x3_free(c);
    dcn_packed_free(body->dcn);
    for (void* p : body->buffers) (void)hipFree(p);
    if (body->capture_stream) (void)hipStreamDestroy(body->capture_stream);
    delete body;
}

dcn_status dcn_body_create(dcn_context* ctx, int height, int width, int branch, int blocks,
                           const dcn_body_weights* weights, void* stream, dcn_body** out) {
    return dcn_body_create_tiles(ctx, height, width, branch, blocks, 1, weights, stream, out);
}

dcn_status dcn_body_create_tiles(dcn_context* ctx, int height, int width, int branch, int blocks, int tiles,
                                 const dcn_body_weights* weights, void* stream, dcn_body** out) {
    if (!ctx || !out) return DCN_INVALID_ARGUMENT;
    *out = nullptr;
    DCN_TRY(check_plane(ctx, width, height));
    if (branch < 0 || branch > 3 || blocks < 1 || blocks > DCN_BODY_MAX_BLOCKS || !weights)
        return fail(ctx, DCN_INVALID_ARGUMENT, "body needs branch 0..3, 1..8 blocks and weights");
    if (tiles < 1 || tiles > 1024 || (long long)tiles * width * height * 432 >= (1LL << 30))
        return fail(ctx, DCN_INVALID_SHAPE, "a body batches 1..1024 tiles");
    DeviceGuard guard(ctx->device);
    auto* b = new dcn_body();
    b->ctx = ctx;
    b->h = height;
    b->w = width;
    b->branch = branch;
    b->blocks = blocks;
    b->tiles = tiles;
    const hipStream_t s = (hipStream_t)stream;
    auto bail = [&](dcn_status st) {
        dcn_body_destroy(b);
        return st;
    };
    static const int kOffsetIn[4] = {196, 64, 64, 64};
    static const int kOffsetOut[4] = {64, 64, 64, 432};
    for (int i = 0; i < 4; ++i) {
        const dcn_status st = dcn_conv3x3_create_dev(ctx, kOffsetIn[i], kOffsetOut[i], height, width,
                                                     weights->offset_weight[i], weights->offset_bias[i],
                                                     stream, &b->offset_conv[i]);
        if (st != DCN_OK) return bail(st);
    }
    const int bb_in = 64 * (branch + 2);
    for (int i = 0; i < 1 + 2 * blocks; ++i) {
        const dcn_status st = dcn_conv3x3_create_dev(ctx, i == 0 ? bb_in : 64, 64, height, width,
                                                     weights->backbone_weight[i],
                                                     weights->backbone_bias[i], stream, &b->backbone[i]);
        if (st != DCN_OK) return bail(st);
    }
    const dcn_shape ds = body_dcn_shape(height, width);
    {
        const dcn_status st = dcn_prepack_f16_dev(ctx, &ds, weights->dcn_weight, DCN_LAYOUT_OIHW,
                                                  weights->dcn_bias, stream, &b->dcn);
        if (st != DCN_OK) return bail(st);
    }
    const size_t T = (size_t)tiles;
    dcn_status st = DCN_OK;
    auto a16 = [&](uint16_t** p, size_t elems) {
        if (st == DCN_OK) st = alloc(ctx, b->buffers, p, elems);
    };
    a16(&b->cond_cb8, T * dcn::cb8_tensor_elems(196, height, width));
    a16(&b->deform_cb8, T * dcn::cb8_tensor_elems(128, height, width));
    a16(&b->off_a, T * dcn::cb8_tensor_elems(64, height, width));
    a16(&b->off_b, T * dcn::cb8_tensor_elems(64, height, width));
    a16(&b->bb_in, T * dcn::cb8_tensor_elems(bb_in, height, width));
    for (auto& f : b->feat) a16(&f, T * dcn::cb8_tensor_elems(64, height, width));
    if (st != DCN_OK) return bail(st);
    // CB8 borders and padding channels are zero once and never written again, so a
    // step (and its captured graph) holds no memset.
    for (uint16_t* p : {b->cond_cb8, b->deform_cb8, b->off_a, b->off_b, b->bb_in, b->feat[0],
                        b->feat[1]}) {
        size_t elems = 0;
        if (p == b->cond_cb8) elems = T * dcn::cb8_tensor_elems(196, height, width);
        else if (p == b->deform_cb8) elems = T * dcn::cb8_tensor_elems(128, height, width);
        else if (p == b->bb_in) elems = T * dcn::cb8_tensor_elems(bb_in, height, width);
        else elems = T * dcn::cb8_tensor_elems(64, height, width);
        if (hipMemsetAsync(p, 0, elems * 2, s) != hipSuccess)
            return bail(fail(ctx, DCN_COMMAND_FAILED, "clearing body buffers failed"));
    }
    if (hipStreamCreateWithFlags(&b->capture_stream, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(ctx, DCN_COMMAND_FAILED, "hipStreamCreate failed"));
    if (hipStreamSynchronize(s) != hipSuccess)
        return bail(fail(ctx, DCN_COMMAND_FAILED, "body set-up failed"));
    *out = b;
    return DCN_OK;
}

}  // extern "C"

namespace {

// Backbone of a step from the body's backbone input (aligned slot filled): conv 128+ -> 64
// with LeakyReLU 0.1, then residual blocks t = ReLU(conv(x)); x = x + conv(t). The last
// one also adds the aligned feature: feat_prop = aligned + backbone
// (add_propagation_residual_fp16).
dcn_status run_backbone(dcn_body* body, void* d_feat_prop_out, hipStream_t s, void* d_out_cb8 = nullptr) {
    dcn_context* ctx = body->ctx;
    const int NCHW = DCN_TENSOR_NCHW, CB8 = DCN_TENSOR_CB8;
    const int aligned_c = 64 * (body->branch + 1);
    const long feat_ts = cb8_image(body, 8), bb_ts = cb8_image(body, 8 * (body->branch + 2));
    const long out_ts = 64L * body->h * body->w;
    dcn::ConvBatch in_conv;
    in_conv.images = body->tiles;
    in_conv.x = bb_ts;
    in_conv.out = feat_ts;
    DCN_TRY(run_conv(ctx, body->backbone[0], body->bb_in, 1, nullptr, NCHW, nullptr, NCHW,
                     body->feat[0], CB8, s, in_conv));
    // Each block's two convs run as one launch (t = ReLU(conv(x)) stays in LDS).
    int x = 0;
    for (int i = 0; i < body->blocks; ++i) {
        const int y = x ^ 1;
        const bool last = i + 1 == body->blocks;
        const dcn_conv* c1 = body->backbone[1 + 2 * i];
        const dcn_conv* c2 = body->backbone[2 + 2 * i];
        dcn::ConvBatch pb;
        pb.images = body->tiles;
        pb.x = feat_ts;
        pb.res1 = feat_ts;
        pb.res2 = last ? bb_ts : 0;
        pb.out = last ? out_ts : feat_ts;
        pb.out2 = feat_ts;
        DCN_HIP(ctx, dcn::launch_conv3x3_pair(c1->g, c2->g, body->feat[x], c1->wpk, c1->bias, 2, c2->wpk,
                                              c2->bias, 0, 0.1f, body->feat[x], CB8,
                                              last ? body->bb_in : nullptr, CB8,
                                              last ? (uint16_t*)d_feat_prop_out : body->feat[y],
                                              last ? NCHW : CB8, s, aligned_c, pb,
                                              last ? (uint16_t*)d_out_cb8 : nullptr));
        x = y;
    }
    return DCN_OK;
}

// One step. With m.warp (single-tile bodies only) feat_prop and feat_n2 are CB8 tensors
// (warped with 16-byte gathers) and m.out receives a CB8 copy of the output.
struct Cb8Step {
    bool warp = false;
    void* out = nullptr;
};

dcn_status body_step(dcn_body* body, const void* d_feat_current, const void* d_flow1, const void* d_prev_flow,
                     const void* d_feat_prop, const void* d_feat_n2, const void* const* d_prefix,
                     int has_second_order, void* d_flow2_out, void* d_feat_prop_out, const Cb8Step& m,
                     void* stream) {
    if (!body) return DCN_INVALID_ARGUMENT;
    dcn_context* ctx = body->ctx;
    if (!d_feat_current || !d_flow1 || !d_prev_flow || !d_feat_prop || !d_feat_n2 || !d_flow2_out ||
        !d_feat_prop_out || (body->branch > 0 && !d_prefix) || (m.warp && !m.out))
        return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    if (m.warp && body->tiles != 1)
        return fail(ctx, DCN_INVALID_SHAPE, "CB8 feature steps take single-tile bodies");
    DeviceGuard guard(ctx->device);
    const hipStream_t s = (hipStream_t)stream;
    const int H = body->h, W = body->w;
    const int NCHW = DCN_TENSOR_NCHW, CB8 = DCN_TENSOR_CB8;
    const uint16_t* prefix[3] = {};
    for (int i = 0; i < body->branch; ++i) {
        if (!d_prefix[i]) return fail(ctx, DCN_INVALID_ARGUMENT, "prefix pointer is null");
        prefix[i] = (const uint16_t*)d_prefix[i];
    }
    const long off_ts = cb8_image(body, 8);
    const dcn_conv* c0 = body->offset_conv[0];
    if (body->tiles == 1) {
        // Second-order flow, the conditions (in LDS only), DCN input, the backbone input's
        // leading [feat_current, prefix...] and the first conv_offset layer in one launch.
        DCN_HIP(ctx, dcn::launch_temporal_conv(c0->g, (const uint16_t*)d_feat_prop, (const uint16_t*)d_feat_current,
                                               (const uint16_t*)d_feat_n2, (const uint16_t*)d_flow1,
                                               (const uint16_t*)d_prev_flow, has_second_order ? 1 : 0, prefix,
                                               body->branch, (uint16_t*)d_flow2_out, body->deform_cb8, body->bb_in,
                                               c0->wpk, c0->bias, 0.1f, body->off_a, s, m.warp));
    } else {
        // Many tiles: the batched conv shares each workgroup's weight fragments over up to
        // 16 images, which the per-image fused kernel cannot; the temporal preparation
        // runs as its own kernel into the CB8 conditions.
        DCN_HIP(ctx, dcn::launch_body_temporal((const uint16_t*)d_feat_prop, (const uint16_t*)d_feat_current,
                                               (const uint16_t*)d_feat_n2, (const uint16_t*)d_flow1,
                                               (const uint16_t*)d_prev_flow, has_second_order ? 1 : 0,
                                               prefix, body->branch, (uint16_t*)d_flow2_out, body->cond_cb8,
                                               body->deform_cb8, body->bb_in, H, W, s, body->tiles));
        dcn::ConvBatch cond_conv;
        cond_conv.images = body->tiles;
        cond_conv.x = cb8_image(body, 25);
        cond_conv.out = off_ts;
        DCN_TRY(run_conv(ctx, c0, body->cond_cb8, 1, nullptr, NCHW, nullptr, NCHW, body->off_a, CB8, s, cond_conv));
    }
    // conv_offset: 196 -> 64 -> 64 -> 64 (LeakyReLU 0.1) -> 432, the last one turning its
    // output into offsets and masks for the DCN of the same launch.
    const dcn_conv* c1 = body->offset_conv[1];
    const dcn_conv* c2 = body->offset_conv[2];
    dcn::ConvBatch off_pair;
    off_pair.images = body->tiles;
    off_pair.x = off_ts;
    off_pair.out = off_ts;
    DCN_HIP(ctx, dcn::launch_conv3x3_pair(c1->g, c2->g, body->off_a, c1->wpk, c1->bias, 1, c2->wpk, c2->bias,
                                          1, 0.1f, nullptr, NCHW, nullptr, NCHW, body->off_b, CB8, s, 0, off_pair));
    // The last conv_offset layer (offsets and masks kept in LDS) and the DCN in one
    // launch; the DCN writes the aligned feature into the backbone input (CB8, after the
    // prefix).
    const dcn_conv* c3 = body->offset_conv[3];
    DCN_HIP(ctx, dcn::launch_offsets_dcn(c3->g, body->off_b, c3->wpk, c3->bias, (const uint16_t*)d_flow1,
                                         (const uint16_t*)d_flow2_out, body->deform_cb8, body->dcn->weights_narrow,
                                         dcn::narrow_packed_bytes(body->dcn->geometry), body->dcn->bias,
                                         body->bb_in, 64 * (body->branch + 1), 8 * (body->branch + 2),
                                         body->tiles, s));
    return run_backbone(body, d_feat_prop_out, s, m.out);
}

dcn_status body_initial(dcn_body* body, const void* d_feat_current, const void* const* d_prefix,
                        void* d_feat_prop_out, void* d_out_cb8, void* stream) {
    if (!body) return DCN_INVALID_ARGUMENT;
    dcn_context* ctx = body->ctx;
    if (!d_feat_current || !d_feat_prop_out || (body->branch > 0 && !d_prefix))
        return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DeviceGuard guard(ctx->device);
    const hipStream_t s = (hipStream_t)stream;
    const uint16_t* prefix[3] = {};
    for (int i = 0; i < body->branch; ++i) {
        if (!d_prefix[i]) return fail(ctx, DCN_INVALID_ARGUMENT, "prefix pointer is null");
        prefix[i] = (const uint16_t*)d_prefix[i];
    }
    DCN_HIP(ctx, dcn::launch_body_initial((const uint16_t*)d_feat_current, prefix, body->branch, body->bb_in,
                                          body->h, body->w, s, body->tiles));
    return run_backbone(body, d_feat_prop_out, s, d_out_cb8);
}

}  // namespace

extern "C" {

dcn_status dcn_body_step_dev(dcn_body* body, const void* d_feat_current, const void* d_flow1,
                             const void* d_prev_flow, const void* d_feat_prop,
                             const void* d_feat_n2, const void* const* d_prefix,
                             int has_second_order, void* d_flow2_out, void* d_feat_prop_out,
                             void* stream) {
    return body_step(body, d_feat_current, d_flow1, d_prev_flow, d_feat_prop, d_feat_n2, d_prefix, has_second_order,
                     d_flow2_out, d_feat_prop_out, Cb8Step{}, stream);
}

dcn_status dcn_body_step_cb8_dev(dcn_body* body, const void* d_feat_current, const void* d_flow1,
                                 const void* d_prev_flow, const void* d_feat_prop_cb8,
                                 const void* d_feat_n2_cb8, const void* const* d_prefix,
                                 int has_second_order, void* d_flow2_out, void* d_feat_prop_out,
                                 void* d_feat_prop_out_cb8, void* stream) {
    Cb8Step m;
    m.warp = true;
    m.out = d_feat_prop_out_cb8;
    return body_step(body, d_feat_current, d_flow1, d_prev_flow, d_feat_prop_cb8, d_feat_n2_cb8, d_prefix,
                     has_second_order, d_flow2_out, d_feat_prop_out, m, stream);
}

dcn_status dcn_body_initial_step_dev(dcn_body* body, const void* d_feat_current,
                                     const void* const* d_prefix, void* d_feat_prop_out,
                                     void* stream) {
    return body_initial(body, d_feat_current, d_prefix, d_feat_prop_out, nullptr, stream);
}

dcn_status dcn_body_initial_step_cb8_dev(dcn_body* body, const void* d_feat_current,
                                         const void* const* d_prefix, void* d_feat_prop_out,
                                         void* d_feat_prop_out_cb8, void* stream) {
    if (!body) return DCN_INVALID_ARGUMENT;
    if (!d_feat_prop_out_cb8) return fail(body->ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    return body_initial(body, d_feat_current, d_prefix, d_feat_prop_out, d_feat_prop_out_cb8, stream);
}

}  // extern "C"

namespace {

// `enqueue` (a step on the given stream) captured into one executable graph.
template <class F>
dcn_status capture_graph(dcn_body* body, dcn_graph** out, F&& enqueue) {
    if (!body || !out) return DCN_INVALID_ARGUMENT;
    *out = nullptr;
    dcn_context* ctx = body->ctx;
    DeviceGuard guard(ctx->device);
    const hipStream_t s = body->capture_stream;
    DCN_HIP(ctx, hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    const dcn_status st = enqueue(s);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(s, &graph);
    if (st != DCN_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return st;
    }
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamEndCapture");
    auto* g = new dcn_graph();
    g->graph = graph;
    g->device = ctx->device;
    const hipError_t ie = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    if (ie != hipSuccess) {
        dcn_graph_destroy(g);
        return hip_fail(ctx, ie, "hipGraphInstantiate");
    }
    *out = g;
    return DCN_OK;
}

}  // namespace

extern "C" {

dcn_status dcn_body_capture(dcn_body* body, const void* d_feat_current, const void* d_flow1,
                            const void* d_prev_flow, const void* d_feat_prop,
                            const void* d_feat_n2, const void* const* d_prefix,
                            int has_second_order, void* d_flow2_out, void* d_feat_prop_out,
                            dcn_graph** out) {
    return capture_graph(body, out, [&](hipStream_t s) {
        return dcn_body_step_dev(body, d_feat_current, d_flow1, d_prev_flow, d_feat_prop, d_feat_n2, d_prefix,
                                 has_second_order, d_flow2_out, d_feat_prop_out, s);
    });
}

dcn_status dcn_body_capture_cb8(dcn_body* body, const void* d_feat_current, const void* d_flow1,
                                const void* d_prev_flow, const void* d_feat_prop_cb8,
                                const void* d_feat_n2_cb8, const void* const* d_prefix,
                                int has_second_order, void* d_flow2_out, void* d_feat_prop_out,
                                void* d_feat_prop_out_cb8, dcn_graph** out) {
    return capture_graph(body, out, [&](hipStream_t s) {
        return dcn_body_step_cb8_dev(body, d_feat_current, d_flow1, d_prev_flow, d_feat_prop_cb8, d_feat_n2_cb8,
                                     d_prefix, has_second_order, d_flow2_out, d_feat_prop_out,
                                     d_feat_prop_out_cb8, s);
    });
}

dcn_status dcn_graph_launch(dcn_graph* graph, void* stream) {
    if (!graph || !graph->exec) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(graph->device);
    return hipGraphLaunch(graph->exec, (hipStream_t)stream) == hipSuccess ? DCN_OK
                                                                          : DCN_COMMAND_FAILED;
}

void dcn_graph_destroy(dcn_graph* graph) {
    if (!graph) return;
    DeviceGuard guard(graph->device);
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
}


void dcn_clip_destroy(dcn_clip* clip) {
    if (!clip) return;
    DeviceGuard guard(clip->ctx ? clip->ctx->device : 0);
    for (auto* b : clip->body) dcn_body_destroy(b);
    for (void* p : clip->buffers) (void)hipFree(p);
    if (clip->capture_stream) (void)hipStreamDestroy(clip->capture_stream);
    delete clip;
}

dcn_status dcn_clip_create(dcn_context* ctx, int height, int width, int frames, int blocks,
                           const dcn_body_weights* weights, void* stream, dcn_clip** out) {
    return dcn_clip_create_tiles(ctx, height, width, frames, blocks, 1, weights, stream, out);
}

dcn_status dcn_clip_create_tiles(dcn_context* ctx, int height, int width, int frames, int blocks, int tiles,
                                 const dcn_body_weights* weights, void* stream, dcn_clip** out) {
    if (!ctx || !out) return DCN_INVALID_ARGUMENT;
    *out = nullptr;
    if (frames <= 0) return fail(ctx, DCN_INVALID_SHAPE, "a clip needs at least one frame");
    if (!weights) return fail(ctx, DCN_INVALID_ARGUMENT, "clip weights are null");
    DCN_TRY(check_plane(ctx, width, height));
    DeviceGuard guard(ctx->device);
    auto* c = new dcn_clip();
    c->ctx = ctx;
    c->h = height;
    c->w = width;
    c->frames = frames;
    c->blocks = blocks;
    c->tiles = tiles;
    auto bail = [&](dcn_status st) {
        dcn_clip_destroy(c);
        return st;
    };
    for (int b = 0; b < 4; ++b) {
        const dcn_status st =
            dcn_body_create_tiles(ctx, height, width, b, blocks, tiles, &weights[b], stream, &c->body[b]);
        if (st != DCN_OK) return bail(st);
    }
    const size_t plane = (size_t)width * height * tiles;
    const size_t cb8 = (size_t)dcn::cb8_tensor_elems(64, height, width);  // one 64-channel CB8 feature
    dcn_status st = alloc(ctx, c->buffers, &c->zero_feat, 64 * plane);
    if (st == DCN_OK) st = alloc(ctx, c->buffers, &c->flow2, 2 * plane);
    if (st == DCN_OK && tiles == 1) st = alloc(ctx, c->buffers, &c->mirror, 4 * (size_t)frames * cb8);
    if (st == DCN_OK && tiles == 1) st = alloc(ctx, c->buffers, &c->zero_cb8, cb8);
    if (st != DCN_OK) return bail(st);
    const hipStream_t s = (hipStream_t)stream;
    if (hipMemsetAsync(c->zero_feat, 0, 64 * plane * 2, s) != hipSuccess ||
        hipMemsetAsync(c->flow2, 0, 2 * plane * 2, s) != hipSuccess ||
        (c->mirror && hipMemsetAsync(c->mirror, 0, 4 * (size_t)frames * cb8 * 2, s) != hipSuccess) ||
        (c->zero_cb8 && hipMemsetAsync(c->zero_cb8, 0, cb8 * 2, s) != hipSuccess))
        return bail(fail(ctx, DCN_COMMAND_FAILED, "clearing clip buffers failed"));
    if (hipStreamCreateWithFlags(&c->capture_stream, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(ctx, DCN_COMMAND_FAILED, "hipStreamCreate failed"));
    if (hipStreamSynchronize(s) != hipSuccess) return bail(fail(ctx, DCN_COMMAND_FAILED, "clip set-up failed"));
    *out = c;
    return DCN_OK;
}

}  // extern "C"

namespace {

// Elements of one 64-channel CB8 feature of a clip.
long cb8_feat(const dcn_clip* clip) { return dcn::cb8_tensor_elems(64, clip->h, clip->w); }

// One recurrence of all four branches over n frames (frame indices 0 .. n-1 of the
// accessors), in schedule order. feat(i) is frame i's spatial feature, flow(backward, i)
// the flow that frame i's step reads (backward flows are indexed by the frame, forward
// flows by the frame before it), prop(b, i) branch b's feat_prop of frame i, and mir(b, i)
// its CB8 copy (null for clips over several tiles, whose steps warp the NCHW features).
template <class Feat, class Flow, class Prop, class Mir>
dcn_status run_recurrence(dcn_clip* clip, int n, Feat feat, Flow flow, Prop prop, Mir mir, void* stream) {
    for (int b = 0; b < 4; ++b) {
        const bool backward = b % 2 == 0;
        auto frame_at = [&](int position) { return backward ? n - 1 - position : position; };
        for (int p = 0; p < n; ++p) {
            const int frame = frame_at(p);
            const void* prefix[3] = {};
            for (int i = 0; i < b; ++i) prefix[i] = prop(i, frame);
            uint16_t* m = mir(b, frame);
            if (p == 0) {
                if (m)
                    DCN_TRY(dcn_body_initial_step_cb8_dev(clip->body[b], feat(frame), prefix, prop(b, frame), m, stream));
                else
                    DCN_TRY(dcn_body_initial_step_dev(clip->body[b], feat(frame), prefix, prop(b, frame), stream));
                continue;
            }
            const int prev = frame_at(p - 1);
            const uint16_t* flow1 = flow(backward, frame);
            const uint16_t* prev_flow = p >= 2 ? flow(backward, prev) : flow1;
            if (m) {
                const uint16_t* n2 = p >= 2 ? mir(b, frame_at(p - 2)) : clip->zero_cb8;
                DCN_TRY(dcn_body_step_cb8_dev(clip->body[b], feat(frame), flow1, prev_flow, mir(b, prev), n2, prefix,
                                              p >= 2 ? 1 : 0, clip->flow2, prop(b, frame), m, stream));
            } else {
                const uint16_t* feat_n2 = p >= 2 ? prop(b, frame_at(p - 2)) : clip->zero_feat;
                DCN_TRY(dcn_body_step_dev(clip->body[b], feat(frame), flow1, prev_flow, prop(b, prev), feat_n2,
                                          prefix, p >= 2 ? 1 : 0, clip->flow2, prop(b, frame), stream));
            }
        }
    }
    return DCN_OK;
}

}  // namespace

extern "C" {

dcn_status dcn_clip_run_dev(dcn_clip* clip, const void* d_spatial, const void* d_backward_flows,
                            const void* d_forward_flows, void* d_propagated,
                            int max_frames_per_chunk, void* stream) {
    if (!clip) return DCN_INVALID_ARGUMENT;
    dcn_context* ctx = clip->ctx;
    const int T = clip->frames;
    if (!d_spatial || !d_propagated || (T > 1 && (!d_backward_flows || !d_forward_flows)))
        return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    std::vector<int> starts(1, 0), sizes(1, T);
    if (max_frames_per_chunk != 0) {
        size_t n = 0;
        starts.assign((size_t)T, 0);
        sizes.assign((size_t)T, 0);
        DCN_TRY(dcn_temporal_chunk_ranges(T, max_frames_per_chunk, starts.data(), sizes.data(),
                                          starts.size(), &n));
        starts.resize(n);
        sizes.resize(n);
    }
    DeviceGuard guard(ctx->device);
    // Every per-frame tensor holds all tiles: [tiles][C][H][W].
    const size_t plane = (size_t)clip->w * clip->h * clip->tiles;
    const uint16_t* spatial = (const uint16_t*)d_spatial;
    const uint16_t* bflows = (const uint16_t*)d_backward_flows;
    const uint16_t* fflows = (const uint16_t*)d_forward_flows;
    uint16_t* propagated = (uint16_t*)d_propagated;
    for (size_t r = 0; r < starts.size(); ++r) {
        const int c0 = starts[r];
        auto feat = [&](int i) { return spatial + (size_t)(c0 + i) * 64 * plane; };
        auto flow = [&](bool backward, int i) {
            const int frame = c0 + i;
            return backward ? bflows + (size_t)frame * 2 * plane : fflows + (size_t)(frame - 1) * 2 * plane;
        };
        auto prop = [&](int b, int i) { return propagated + ((size_t)b * T + c0 + i) * 64 * plane; };
        auto mir = [&](int b, int i) {
            return clip->mirror ? clip->mirror + ((size_t)b * T + c0 + i) * (size_t)cb8_feat(clip) : nullptr;
        };
        DCN_TRY(run_recurrence(clip, sizes[r], feat, flow, prop, mir, stream));
    }
    return DCN_OK;
}

dcn_status dcn_clip_run_with_fallback_dev(dcn_clip* clip, const void* d_spatial, const void* d_backward_flows,
                                          const void* d_forward_flows, void* d_propagated, void* stream,
                                          dcn_report_fn report, void* report_user, int* recovered_with) {
    if (!clip || !recovered_with) return DCN_INVALID_ARGUMENT;
    *recovered_with = 0;
    dcn_context* ctx = clip->ctx;
    const int T = clip->frames;
    if (!d_spatial || !d_propagated || (T > 1 && (!d_backward_flows || !d_forward_flows)))
        return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DeviceGuard guard(ctx->device);
    const hipStream_t s = (hipStream_t)stream;
    const size_t plane = (size_t)clip->w * clip->h * clip->tiles;
    const size_t feat_bytes = 64 * plane * sizeof(uint16_t);
    const uint16_t* spatial = (const uint16_t*)d_spatial;
    uint16_t* propagated = (uint16_t*)d_propagated;
    auto say = [&](const std::string& msg) {
        if (report) report(msg.c_str(), report_user);
    };
    // A rung fails recoverably when its output holds a NaN or Inf (the reference's
    // recurrence throws nonFiniteOutput then); any other error ends the ladder.
    auto attempt = [&](int chunk) -> dcn_status {
        DCN_TRY(dcn_clip_run_dev(clip, d_spatial, d_backward_flows, d_forward_flows, d_propagated, chunk, stream));
        return dcn_check_nonfinite_f16_dev(ctx, d_propagated, 4 * (size_t)T * 64 * plane, stream);
    };
    dcn_status st = attempt(0);
    if (st == DCN_OK) return DCN_OK;
    if (!dcn_status_is_recoverable(st)) return st;
    std::string last = ctx->last_error;
    say("clip failed its full temporal window (" + last + "); retrying shorter recurrence chunks");
    for (int chunk : {10, 5, 3}) {
        if (chunk >= T) continue;
        st = attempt(chunk);
        if (st == DCN_OK) {
            say("clip recovered with at most " + std::to_string(chunk) + " frames per recurrence chunk");
            *recovered_with = chunk;
            return DCN_OK;
        }
        if (!dcn_status_is_recoverable(st)) return st;
        last = ctx->last_error;
        say("clip also failed with " + std::to_string(chunk) + "-frame chunks (" + last + ")");
    }
    // Independent zero-motion triplets: frame t alone as the clip [t, t, t] with zero
    // flows; every branch keeps the middle frame's feat_prop.
    if (!clip->triplet_prop) DCN_TRY(alloc(ctx, clip->buffers, &clip->triplet_prop, 12 * 64 * plane));
    if (clip->mirror && !clip->triplet_mirror) {
        DCN_TRY(alloc(ctx, clip->buffers, &clip->triplet_mirror, 12 * (size_t)cb8_feat(clip)));
        DCN_HIP(ctx, hipMemsetAsync(clip->triplet_mirror, 0, 12 * (size_t)cb8_feat(clip) * 2, s));
    }
    st = DCN_OK;
    for (int t = 0; t < T && st == DCN_OK; ++t) {
        const uint16_t* frame = spatial + (size_t)t * 64 * plane;
        auto feat = [&](int) { return frame; };
        auto flow = [&](bool, int) { return (const uint16_t*)clip->zero_feat; };  // >= 2 x plane zeros
        auto prop = [&](int b, int i) { return clip->triplet_prop + (size_t)(b * 3 + i) * 64 * plane; };
        auto mir = [&](int b, int i) {
            return clip->triplet_mirror ? clip->triplet_mirror + (size_t)(b * 3 + i) * (size_t)cb8_feat(clip) : nullptr;
        };
        DCN_TRY(run_recurrence(clip, 3, feat, flow, prop, mir, stream));
        st = dcn_check_nonfinite_f16_dev(ctx, clip->triplet_prop, 12 * 64 * plane, stream);
        if (st != DCN_OK) break;
        for (int b = 0; b < 4; ++b)
            DCN_HIP(ctx, hipMemcpyAsync(propagated + ((size_t)b * T + t) * 64 * plane, prop(b, 1), feat_bytes,
                                        hipMemcpyDeviceToDevice, s));
    }
    if (st == DCN_OK) {
        DCN_HIP(ctx, hipStreamSynchronize(s));
        say("clip recovered with independent zero-motion frame triplets");
        *recovered_with = DCN_CLIP_RECOVERED_TRIPLETS;
        return DCN_OK;
    }
    if (!dcn_status_is_recoverable(st)) return st;
    last = ctx->last_error;
    say("clip also failed independent frame recovery (" + last + ")");
    // Passthrough of finite input: every branch's feat_prop of frame t is frame t's
    // spatial feature, unchanged.
    st = dcn_check_nonfinite_f16_dev(ctx, d_spatial, (size_t)T * 64 * plane, stream);
    if (st == DCN_NONFINITE_OUTPUT)
        return fail(ctx, DCN_COMMAND_FAILED, "clip has non-finite input features after model failure: " + last);
    if (st != DCN_OK) return st;
    for (int b = 0; b < 4; ++b)
        DCN_HIP(ctx, hipMemcpyAsync(propagated + (size_t)b * T * 64 * plane, spatial, (size_t)T * feat_bytes,
                                    hipMemcpyDeviceToDevice, s));
    DCN_HIP(ctx, hipStreamSynchronize(s));
    say("WARNING: clip is using finite input passthrough because all recurrence recovery modes failed (" +
        last + ")");
    *recovered_with = DCN_CLIP_RECOVERED_PASSTHROUGH;
    return DCN_OK;
}

dcn_status dcn_clip_capture(dcn_clip* clip, const void* d_spatial, const void* d_backward_flows,
                            const void* d_forward_flows, void* d_propagated,
                            int max_frames_per_chunk, dcn_graph** out) {
    if (!clip || !out) return DCN_INVALID_ARGUMENT;
    *out = nullptr;
    dcn_context* ctx = clip->ctx;
    DeviceGuard guard(ctx->device);
    const hipStream_t s = clip->capture_stream;
    DCN_HIP(ctx, hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    const dcn_status st = dcn_clip_run_dev(clip, d_spatial, d_backward_flows, d_forward_flows,
                                           d_propagated, max_frames_per_chunk, s);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(s, &graph);
    if (st != DCN_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return st;
    }
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamEndCapture");
    auto* g = new dcn_graph();
    g->graph = graph;
    g->device = ctx->device;
    const hipError_t ie = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    if (ie != hipSuccess) {
        dcn_graph_destroy(g);
        return hip_fail(ctx, ie, "hipGraphInstantiate");
    }
    *out = g;
    return DCN_OK;
}

}  // extern "C"
