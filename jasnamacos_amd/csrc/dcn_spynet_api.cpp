// C-ABI host layer of SPyNet flow estimation: the quarter-scale bicubic input and the
// six-level pyramid network that produces the first-order flows of the propagation body.
// Reference: jasna_bicubic_downsample_quarter_fp16 and the SPyNet kernels
// (MetalShader.swift:473-649), the bidirectional pair of verifySPyNetPair
// (SPyNetPairProbe.swift:47-449) and the trace-friendly SPyNet forward whose level order
// it follows (tools/convert_basicvsrpp.py:40-100).
#include <string>
#include <vector>

#include "dcn_host.hpp"
#include "dcn_internal.hpp"

using namespace dcn::host;

namespace {

// Basic-module layers of every level: 8 -> 32 -> 64 -> 32 -> 16 -> 2, 7 x 7, ReLU between
// (the SPyNet basic module of the external BasicVSR++ checkpoint; the reference exports it
// as one package per level, tools/convert_basicvsrpp.py:168-180).
constexpr int kLayerIn[DCN_SPYNET_LAYERS] = {8, 32, 64, 32, 16};
constexpr int kLayerOut[DCN_SPYNET_LAYERS] = {32, 64, 32, 16, 2};
constexpr int kKernel = 7;
constexpr int kPadSpy = 3;  // zero border of SPyNet's CB8 activations

struct SpyLayer {
    dcn::ConvKGeometry g{};
    void* wpk = nullptr;
    float* bias = nullptr;
};

}  // namespace

struct dcn_spynet {
    dcn_context* ctx = nullptr;
    int h = 0, w = 0, max_frames = 0, max_images = 0;
    SpyLayer layer[DCN_SPYNET_LEVELS][DCN_SPYNET_LAYERS];
    uint16_t* pyramid[DCN_SPYNET_LEVELS] = {};   // [frame][3][h_l][w_l]
    uint16_t* features[DCN_SPYNET_LEVELS] = {};  // CB8, images x 1 block, border 3
    uint16_t* act_a[DCN_SPYNET_LEVELS] = {};     // CB8, images x up to 64 channels
    uint16_t* act_b[DCN_SPYNET_LEVELS] = {};
    uint16_t* base[DCN_SPYNET_LEVELS] = {};      // [image][2][h_l][w_l]
    uint16_t* flow[DCN_SPYNET_LEVELS] = {};      // [image][2][h_l][w_l] (the last level: caller's)
    std::vector<void*> buffers;
};

namespace {

int level_h(const dcn_spynet* s, int l) { return s->h >> (DCN_SPYNET_LEVELS - 1 - l); }
int level_w(const dcn_spynet* s, int l) { return s->w >> (DCN_SPYNET_LEVELS - 1 - l); }

size_t cb8_spy_elems(int images, int channels, int h, int w) {
    return (size_t)images * ((channels + 7) / 8) * (h + 2 * kPadSpy) * (w + 2 * kPadSpy) * 8;
}

}  // namespace

extern "C" {

void dcn_spynet_destroy(dcn_spynet* s) {
    if (!s) return;
    DeviceGuard guard(s->ctx ? s->ctx->device : 0);
    for (auto& level : s->layer)
        for (auto& l : level) {
            if (l.wpk) (void)hipFree(l.wpk);
            if (l.bias) (void)hipFree(l.bias);
        }
    for (void* p : s->buffers) (void)hipFree(p);
    delete s;
}

dcn_status dcn_spynet_create(dcn_context* ctx, int height, int width, int max_frames,
                             const dcn_spynet_weights* weights, void* stream, dcn_spynet** out) {
    if (!ctx || !out) return DCN_INVALID_ARGUMENT;
    *out = nullptr;
    constexpr int kCoarsest = 1 << (DCN_SPYNET_LEVELS - 1);
    if (height < kCoarsest || width < kCoarsest || height % kCoarsest || width % kCoarsest ||
        height > 4096 || width > 4096)
        return fail(ctx, DCN_INVALID_SHAPE, "SPyNet needs a plane whose sides are multiples of 32");
    if (max_frames < 2 || max_frames > 1024)
        return fail(ctx, DCN_INVALID_SHAPE, "SPyNet needs 2..1024 frames per call");
    if (!weights) return fail(ctx, DCN_INVALID_ARGUMENT, "null SPyNet weights");
    for (int l = 0; l < DCN_SPYNET_LEVELS; ++l)
        for (int i = 0; i < DCN_SPYNET_LAYERS; ++i)
            if (!weights->weight[l][i] || !weights->bias[l][i])
                return fail(ctx, DCN_INVALID_ARGUMENT, "SPyNet weight pointer is null");
    DeviceGuard guard(ctx->device);
    auto* s = new dcn_spynet();
    s->ctx = ctx;
    s->h = height;
    s->w = width;
    s->max_frames = max_frames;
    s->max_images = 2 * (max_frames - 1);
    const int images = s->max_images;
    const hipStream_t st = (hipStream_t)stream;
    auto bail = [&](dcn_status status, const std::string& message) {
        dcn_spynet_destroy(s);
        return fail(ctx, status, message);
    };
    auto alloc = [&](uint16_t** p, size_t elems) {
        void* raw = nullptr;
        if (hipMalloc(&raw, std::max<size_t>(elems, 1) * sizeof(uint16_t)) != hipSuccess) return false;
        s->buffers.push_back(raw);
        *p = static_cast<uint16_t*>(raw);
        return true;
    };
    for (int l = 0; l < DCN_SPYNET_LEVELS; ++l) {
        const int lh = level_h(s, l), lw = level_w(s, l);
        for (int i = 0; i < DCN_SPYNET_LAYERS; ++i) {
            SpyLayer& L = s->layer[l][i];
            L.g = dcn::convk_geometry(kKernel, kLayerIn[i], kLayerOut[i], lh, lw);
            if (hipMalloc(&L.wpk, dcn::convk_packed_bytes(L.g)) != hipSuccess ||
                hipMalloc((void**)&L.bias, (size_t)kLayerOut[i] * sizeof(float)) != hipSuccess)
                return bail(DCN_COMMAND_FAILED, "hipMalloc of packed SPyNet weights failed");
            const hipError_t e = dcn::launch_convk_prepack(L.g, (const uint16_t*)weights->weight[l][i],
                                                           (const uint16_t*)weights->bias[l][i], L.wpk,
                                                           L.bias, st);
            if (e != hipSuccess) return bail(DCN_COMMAND_FAILED, "SPyNet prepack launch failed");
        }
        const size_t plane = (size_t)lh * lw;
        bool ok = alloc(&s->pyramid[l], (size_t)max_frames * 3 * plane) &&
                  alloc(&s->features[l], cb8_spy_elems(images, 8, lh, lw)) &&
                  alloc(&s->act_a[l], cb8_spy_elems(images, 64, lh, lw)) &&
                  alloc(&s->act_b[l], cb8_spy_elems(images, 64, lh, lw)) &&
                  alloc(&s->base[l], (size_t)images * 2 * plane);
        if (ok && l + 1 < DCN_SPYNET_LEVELS) ok = alloc(&s->flow[l], (size_t)images * 2 * plane);
        if (!ok) return bail(DCN_COMMAND_FAILED, "hipMalloc of SPyNet buffers failed");
        // The CB8 borders are zero once and never written, so a call holds no memset.
        for (uint16_t* p : {s->features[l], s->act_a[l], s->act_b[l]}) {
            const size_t elems = p == s->features[l] ? cb8_spy_elems(images, 8, lh, lw)
                                                     : cb8_spy_elems(images, 64, lh, lw);
            if (hipMemsetAsync(p, 0, elems * sizeof(uint16_t), st) != hipSuccess)
                return bail(DCN_COMMAND_FAILED, "clearing SPyNet buffers failed");
        }
    }
    if (hipStreamSynchronize(st) != hipSuccess) return bail(DCN_COMMAND_FAILED, "SPyNet set-up failed");
    *out = s;
    return DCN_OK;
}

}  // extern "C"

namespace {

// Pyramids of `frames` frames, then every level for the batch of images over `pairs`
// frame pairs (image b < pairs: spynet(frame b, frame b + 1); the rest the reverse
// direction), the last level's flow [batch][2][h][w] into d_flow.
dcn_status run_spynet(dcn_spynet* s, const uint16_t* frame0, const uint16_t* frame1, long frame_stride,
                      int frames, int pairs, int batch, void* d_flow, hipStream_t st) {
    dcn_context* ctx = s->ctx;
    DCN_HIP(ctx, dcn::launch_spynet_pyramid(frame0, frame1, frame_stride, frames, s->pyramid, DCN_SPYNET_LEVELS,
                                            s->h, s->w, st));
    // The leading levels of at most 16 pixels run in one launch, their activations in LDS.
    int fused = 0, units = 0;
    while (fused < DCN_SPYNET_LEVELS - 1 && level_h(s, fused) * level_w(s, fused) <= 16) {
        const int u = std::max(units, (level_h(s, fused) + 6) * (level_w(s, fused) + 6));
        if (dcn::spynet_small_lds_bytes(u) > 160 * 1024) break;
        units = u;
        ++fused;
    }
    if (fused > 0) {
        int hs[DCN_SPYNET_LEVELS], ws[DCN_SPYNET_LEVELS];
        const uint16_t* pyr[DCN_SPYNET_LEVELS];
        const void* wpk[DCN_SPYNET_LEVELS][DCN_SPYNET_LAYERS];
        const float* bias[DCN_SPYNET_LEVELS][DCN_SPYNET_LAYERS];
        uint32_t wbytes[DCN_SPYNET_LEVELS][DCN_SPYNET_LAYERS];
        for (int l = 0; l < fused; ++l) {
            hs[l] = level_h(s, l);
            ws[l] = level_w(s, l);
            pyr[l] = s->pyramid[l];
            for (int i = 0; i < DCN_SPYNET_LAYERS; ++i) {
                wpk[l][i] = s->layer[l][i].wpk;
                bias[l][i] = s->layer[l][i].bias;
                wbytes[l][i] = (uint32_t)dcn::convk_packed_bytes(s->layer[l][i].g);
            }
        }
        DCN_HIP(ctx, dcn::launch_spynet_small(batch, pairs, fused, hs, ws, pyr, wpk, bias, wbytes,
                                              s->flow[fused - 1], st));
    }
    for (int l = fused; l < DCN_SPYNET_LEVELS; ++l) {
        const int lh = level_h(s, l), lw = level_w(s, l);
        const bool first = l == 0;
        DCN_HIP(ctx, dcn::launch_spynet_prepare(batch, pairs, s->pyramid[l], first ? nullptr : s->flow[l - 1],
                                                first ? 1 : level_h(s, l - 1), first ? 1 : level_w(s, l - 1),
                                                first ? 1 : 0, s->features[l], kPadSpy, s->base[l], lh, lw, st));
        const uint16_t* in = s->features[l];
        uint16_t* bufs[2] = {s->act_a[l], s->act_b[l]};
        for (int i = 0; i < DCN_SPYNET_LAYERS; ++i) {
            const SpyLayer& L = s->layer[l][i];
            const bool last = i + 1 == DCN_SPYNET_LAYERS;
            uint16_t* out = last ? (l + 1 == DCN_SPYNET_LEVELS ? (uint16_t*)d_flow : s->flow[l]) : bufs[i & 1];
            DCN_HIP(ctx, dcn::launch_convk(L.g, batch, kPadSpy, in, L.wpk, L.bias, last ? 0 : 2,
                                           last ? s->base[l] : nullptr, out, last ? 0 : 1, st));
            in = out;
        }
    }
    return DCN_OK;
}

}  // namespace

extern "C" {

dcn_status dcn_spynet_flow_dev(dcn_spynet* s, const void* d_reference, const void* d_support,
                               int both_directions, void* d_flow, void* stream) {
    if (!s) return DCN_INVALID_ARGUMENT;
    dcn_context* ctx = s->ctx;
    if (!d_reference || !d_support || !d_flow) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DeviceGuard guard(ctx->device);
    return run_spynet(s, (const uint16_t*)d_reference, (const uint16_t*)d_support, 0, 2, 1,
                      both_directions ? 2 : 1, d_flow, (hipStream_t)stream);
}

dcn_status dcn_spynet_clip_flows_dev(dcn_spynet* s, const void* d_frames, int frames, void* d_flows,
                                     void* stream) {
    if (!s) return DCN_INVALID_ARGUMENT;
    dcn_context* ctx = s->ctx;
    if (!d_frames || !d_flows) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    if (frames < 2 || frames > s->max_frames)
        return fail(ctx, DCN_INVALID_SHAPE, "clip frame count outside 2..max_frames of this SPyNet");
    DeviceGuard guard(ctx->device);
    const long stride = 3L * s->h * s->w;
    const uint16_t* f0 = (const uint16_t*)d_frames;
    return run_spynet(s, f0, f0 + stride, stride, frames, frames - 1, 2 * (frames - 1), d_flows,
                      (hipStream_t)stream);
}

dcn_status dcn_spynet_pyramid_f16_dev(dcn_context* ctx, int height, int width, const void* d_frame, void* d_out,
                                      void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    constexpr int kCoarsest = 1 << (DCN_SPYNET_LEVELS - 1);
    if (height < kCoarsest || width < kCoarsest || height % kCoarsest || width % kCoarsest || height > 4096 ||
        width > 4096)
        return fail(ctx, DCN_INVALID_SHAPE, "SPyNet needs a plane whose sides are multiples of 32");
    if (!d_frame || !d_out) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DeviceGuard guard(ctx->device);
    uint16_t* levels[dcn::kSpynetMaxLevels] = {};
    size_t off = 0;
    for (int l = 0; l < DCN_SPYNET_LEVELS; ++l) {
        levels[l] = (uint16_t*)d_out + off;
        off += (size_t)3 * (height >> (DCN_SPYNET_LEVELS - 1 - l)) * (width >> (DCN_SPYNET_LEVELS - 1 - l));
    }
    DCN_HIP(ctx, dcn::launch_spynet_pyramid((const uint16_t*)d_frame, nullptr, 0, 1, levels, DCN_SPYNET_LEVELS,
                                            height, width, (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_bicubic_quarter_f16_dev(dcn_context* ctx, int channels, int height, int width,
                                       const void* d_in, void* d_out, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    if (channels <= 0 || height < 4 || width < 4 || height % 4 || width % 4 || height > 65536 ||
        width > 65536 || (long long)channels * height * width > (1LL << 31))
        return fail(ctx, DCN_INVALID_SHAPE, "bicubic quarter downsample needs sides that are multiples of 4");
    if (!d_in || !d_out) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DeviceGuard guard(ctx->device);
    DCN_HIP(ctx, dcn::launch_bicubic_quarter((const uint16_t*)d_in, (uint16_t*)d_out, channels, height, width,
                                             (hipStream_t)stream));
    return DCN_OK;
}

}  // extern "C"
