// C-ABI host layer of libdcn: validation, context/workspace management, host<->device
// staging and kernel dispatch. Reference: MetalDeformConv (MetalRunner.swift:92-842),
// DeformConvShape/DeformConvError (DeformConv.swift:3-73),
// DeformConvWeightSet (DeformConvWeights.swift:4-46).
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "dcn_host.hpp"
#include "dcn_internal.hpp"

namespace {

using namespace dcn::host;

dcn_status validated_counts(dcn_context* ctx, const dcn_shape* shape, dcn_counts* c) {
    if (!shape) return fail(ctx, DCN_INVALID_ARGUMENT, "shape is null");
    if (dcn_shape_validate(shape) != DCN_OK)
        return fail(ctx, DCN_INVALID_SHAPE, "Invalid deformable-convolution shape");
    dcn_shape_counts(shape, c);
    // Device code indexes with 32-bit offsets: every tensor (FP32 at most) must stay
    // below 2^31 bytes, i.e. 2^29 elements.
    const size_t limit = (size_t)1 << 29;
    if (c->input >= limit || c->offset >= limit || c->mask >= limit || c->output >= limit ||
        c->weight >= limit)
        return fail(ctx, DCN_INVALID_SHAPE, "tensor too large for 32-bit device indexing");
    return DCN_OK;
}

bool packed_matches(const dcn_packed* p, const dcn_shape* s) {
    return p->shape.input_channels == s->input_channels &&
           p->shape.output_channels == s->output_channels &&
           p->shape.kernel_height == s->kernel_height &&
           p->shape.kernel_width == s->kernel_width && p->shape.groups == s->groups &&
           p->shape.offset_groups == s->offset_groups;
}

// `o`: the caller's dcn_set_fused_config override ({0, 0, 0, -1}: none).
dcn::FusedConfig choose_config(dcn::FusedConfig o, const dcn::FusedGeometry& g, const dcn_shape& shape,
                               bool window_ok, bool tile_ok) {
    // Problems of more than 32K output pixels run fastest on the tile kernel: batches of
    // small maps (C3: 16 x 64 x 64, 47.2 us against 55.2 us for the window kernel) and
    // single large maps (C5: 1 x 180 x 320, 51.2 us with the cost-ordered tile placement,
    // against 70.9 us; its wide-flow stages whose two windows do not fit LDS together run
    // one pass per window).
    // The same holds for the exact sampler (the reference's FP32 blend, about 104 VALU per
    // sample): C3 67.4 against 67.6 us for the window kernel, C5 71.9 against 73.2.
    if (o.variant == 0 && tile_ok && (g.m + 31) / 32 > 1024) o.variant = dcn::kVariantTile;
    // A shape the tile variant does not cover gets the automatic choice below, with only
    // the sampler pinned.
    if (o.variant == dcn::kVariantTile) {
        if (tile_ok)
            return dcn::FusedConfig{dcn::kVariantTile, o.mt > 0 ? o.mt : 16, o.ks > 0 ? o.ks : 8,
                                    o.sampler == dcn::kSamplerExact ? dcn::kSamplerExact : dcn::kSamplerFast};
        o = dcn::FusedConfig{0, 0, 0, o.sampler};
    }
    const long long tiles32 = (g.m + 31) / 32;
    // Variant: small problems (one 64x64 map is 128 row blocks of 32 pixels) need every
    // CU busy and use 16-pixel tiles; large ones use LDS windows over 2D tiles.
    int variant = o.variant > 0 && o.variant != dcn::kVariantTile
                      ? o.variant
                      : (window_ok && tiles32 > 1024 ? dcn::kVariantWindow : dcn::kVariantNarrow);
    const bool window = variant == dcn::kVariantWindow || variant == dcn::kVariantWindowSplit ||
                        variant == dcn::kVariantWindowAsync;
    if (window && !window_ok) variant = dcn::kVariantNarrow;
    dcn::FusedConfig cfg{variant, 1, 8, dcn::kSamplerFast};
    if (variant == dcn::kVariantNarrow) {
        cfg.mt = 1;
        cfg.ks = 12;  // waves: 36 K-steps of the reference layer in 3 per wave
    } else if (variant == dcn::kVariantWindowAsync) {
        cfg.mt = 8;  // tile rows = waves
        cfg.ks = 8;
        if (g.kb % 18 != 0) cfg.variant = dcn::kVariantWindow;  // needs two groups per stage
    } else if (variant == dcn::kVariantWindow || variant == dcn::kVariantWindowSplit) {
        // A 4 x 32 tile on 4 waves with single-buffered windows: two workgroups share a
        // CU, so one copies its windows while the other multiplies.
        cfg.mt = 4;  // tile rows
        cfg.ks = 4;  // waves = 32-pixel row blocks
        cfg.split = variant == dcn::kVariantWindowSplit ? 1 : 0;
    } else if (variant == dcn::kVariantStaged) {
        cfg.mt = tiles32 > 1024 ? 2 : 1;
        cfg.ks = 8;
    } else {
        cfg.mt = tiles32 > 1024 ? 2 : 1;
        cfg.ks = cfg.mt == 1 ? 8 : 4;
    }
    if (o.mt > 0) cfg.mt = o.mt;
    if (o.ks > 0) cfg.ks = o.ks;
    if (o.sampler >= 0) cfg.sampler = o.sampler;
    if (cfg.variant == dcn::kVariantStaged && dcn::staged_lds_bytes(g, cfg) > 160 * 1024 &&
        o.variant != dcn::kVariantStaged) {
        // The im2col tile does not fit: register sampling handles any K.
        cfg.variant = dcn::kVariantRegister;
        if (o.ks <= 0) cfg.ks = cfg.mt == 1 ? 8 : 4;
    }
    return cfg;
}

bool config_supported(const dcn::FusedConfig& c, const dcn::FusedGeometry& g) {
    if (c.variant == dcn::kVariantTile)  // ks: 8 = cost-ordered tile placement, 1 = fixed
        return (c.mt == 16 || c.mt == 32) && (c.ks == 8 || c.ks == 1) &&
               (c.sampler == dcn::kSamplerFast || c.sampler == dcn::kSamplerExact);
    if (c.variant == dcn::kVariantWindowAsync) return c.mt == 8 && c.ks == 8;
    if (c.variant == dcn::kVariantNarrow) return c.mt == 1 && (c.ks == 8 || c.ks == 12);
    if (c.variant == dcn::kVariantWindow || c.variant == dcn::kVariantWindowSplit)
        return (c.ks == 8 && (c.mt == 8 || c.mt == 4)) || (c.ks == 4 && (c.mt == 4 || c.mt == 2));
    if (c.variant == dcn::kVariantStaged)
        return (c.mt == 1 || c.mt == 2) && (c.ks == 8 || c.ks == 16) &&
               dcn::staged_lds_bytes(g, c) <= 160 * 1024;
    return (c.mt == 1 && (c.ks == 8 || c.ks == 4)) || (c.mt == 2 && (c.ks == 4 || c.ks == 2));
}

dcn_status ensure_workspace(dcn_context* ctx, size_t bytes, hipStream_t stream) {
    if (ctx->workspace_bytes >= bytes) return DCN_OK;
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &status) == hipSuccess &&
        status != hipStreamCaptureStatusNone)
        return fail(ctx, DCN_COMMAND_FAILED,
                    "workspace too small inside stream capture; call dcn_reserve first");
    if (ctx->workspace) {
        DCN_HIP(ctx, hipDeviceSynchronize());
        DCN_HIP(ctx, hipFree(ctx->workspace));
        ctx->workspace = nullptr;
        ctx->workspace_bytes = 0;
    }
    DCN_HIP(ctx, hipMalloc(&ctx->workspace, bytes));
    ctx->workspace_bytes = bytes;
    return DCN_OK;
}

// `repack`: where an NCHW input's padded channel-block copy goes (null: the context's
// workspace, grown on demand; else a buffer of `repack_bytes` that is never grown).
dcn_status fused_prepacked_dev(dcn_context* ctx, const dcn_shape* shape, const void* d_input,
                               bool input_is_cb8, const void* d_offset, const void* d_mask,
                               const dcn_packed* packed, void* d_output, hipStream_t stream,
                               void* repack = nullptr, size_t repack_bytes = 0, bool bf16 = false) {
    dcn_counts c;
    DCN_TRY(validated_counts(ctx, shape, &c));
    if (!packed) return fail(ctx, DCN_INVALID_ARGUMENT, "packed weights are null");
    if (!d_input || !d_offset || !d_mask || !d_output)
        return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    dcn::FusedGeometry g;
    if (!dcn::fused_geometry(*shape, &g))
        return fail(ctx, DCN_INVALID_SHAPE,
                    "fused FP16 path needs groups 1, (Cin/offsetGroups) % 8 == 0, Cout % 32 == 0, Cout <= 128");
    if (!packed_matches(packed, shape))
        return fail(ctx, DCN_INVALID_SHAPE, "packed weights were prepared for another layer shape");
    if (packed->device != ctx->device)
        return fail(ctx, DCN_INVALID_ARGUMENT, "packed weights live on another device");
    if (packed->bf16 != bf16)
        return fail(ctx, DCN_INVALID_ARGUMENT,
                    packed->bf16 ? "packed weights are BF16: use dcn_forward_bf16_prepacked*"
                                 : "packed weights are FP16: use dcn_forward_f16_prepacked*");
    if (dcn::cb8_bytes(*shape, g) >= ((size_t)1 << 31))
        return fail(ctx, DCN_INVALID_SHAPE, "padded input too large for 32-bit device indexing");
    // The packed weights carry the window / tile fragments only when the layer's shape at
    // prepack allowed those kernels; this call's shape must allow them too.
    // BF16: 16-pixel tiles on 12 waves (the narrow kernel) up to 1024 tiles of 32 pixels,
    // as FP16 does; above, LDS windows over 4 x 32 tiles where the shape allows them, else
    // the register variant with 64-pixel tiles over 4 K-waves.
    const long long tiles32 = (g.m + 31) / 32;
    const bool bf16_window = packed->weights_group != nullptr && dcn::window_supported(*shape);
    const dcn::FusedConfig cfg =
        bf16 ? (tiles32 <= 1024 ? dcn::FusedConfig{dcn::kVariantNarrow, 1, 12, dcn::kSamplerBf16}
                : bf16_window   ? dcn::FusedConfig{dcn::kVariantWindow, 4, 4, dcn::kSamplerBf16}
                                : dcn::FusedConfig{dcn::kVariantRegister, 2, 4, dcn::kSamplerBf16})
             : choose_config(ctx->fused_override, g, *shape, packed->weights_group != nullptr && dcn::window_supported(*shape),
                             packed->weights_tile != nullptr && dcn::tile_supported(*shape));
    if (!config_supported(cfg, g))
        return fail(ctx, DCN_INVALID_ARGUMENT,
                    "unsupported fused config (variant " + std::to_string(cfg.variant) + ", mt " +
                        std::to_string(cfg.mt) + ", ks " + std::to_string(cfg.ks) + ")");
    if (g.kb >= (1 << 16)) return fail(ctx, DCN_INVALID_SHAPE, "K too large for the fused path");
    const dcn::KShape ks = dcn::to_kshape(*shape);
    if (cfg.variant == dcn::kVariantTile && ctx->tile_clock &&
        ctx->tile_clock_count < 4 * dcn::tile_grid(ks, cfg))
        return fail(ctx, DCN_INVALID_ARGUMENT,
                    "tile clock buffer holds " + std::to_string(ctx->tile_clock_count) +
                        " stamps; this launch needs " + std::to_string(4 * dcn::tile_grid(ks, cfg)));
    const void* cb8 = d_input;
    if (!input_is_cb8) {
        void* dst = repack;
        if (dst) {
            const size_t need = dcn::cb8_bytes(*shape, g);
            if (need > repack_bytes)
                return fail(ctx, DCN_INVALID_SHAPE,
                            "padded input needs " + std::to_string(need) + " bytes; the allocation-free "
                            "entry point holds at most " + std::to_string(repack_bytes));
        } else {
            DCN_TRY(ensure_workspace(ctx, dcn::cb8_bytes(*shape, g), stream));
            dst = ctx->workspace;
        }
        DCN_HIP(ctx, dcn::launch_pack_cb8(ks, g, (const uint16_t*)d_input, dst, stream));
        cb8 = dst;
    }
    if (cfg.variant == dcn::kVariantTile) {
        if (!packed->weights_tile)
            return fail(ctx, DCN_INVALID_ARGUMENT, "the tile variant does not support this shape");
        DCN_HIP(ctx, dcn::launch_tile_f16(ks, g, cfg, cb8, (const uint16_t*)d_offset,
                                          (const uint16_t*)d_mask, packed->weights_tile,
                                          packed->bias, (uint16_t*)d_output, stream, ctx->tile_clock));
        return DCN_OK;
    }
    if (cfg.variant == dcn::kVariantNarrow) {
        DCN_HIP(ctx, dcn::launch_narrow_f16(ks, g, cfg, cb8, (const uint16_t*)d_offset,
                                            (const uint16_t*)d_mask, packed->weights_narrow,
                                            packed->bias, (uint16_t*)d_output, stream));
        return DCN_OK;
    }
    if (cfg.variant == dcn::kVariantWindow || cfg.variant == dcn::kVariantWindowSplit ||
        cfg.variant == dcn::kVariantWindowAsync) {
        DCN_HIP(ctx, dcn::launch_window_f16(ks, g, cfg, cb8, (const uint16_t*)d_offset,
                                            (const uint16_t*)d_mask, packed->weights_group,
                                            packed->bias, (uint16_t*)d_output, stream));
        return DCN_OK;
    }
    DCN_HIP(ctx, dcn::launch_fused_f16(ks, g, cfg, cb8, (const uint16_t*)d_offset,
                                       (const uint16_t*)d_mask, packed->weights, packed->bias,
                                       (uint16_t*)d_output, stream));
    return DCN_OK;
}

template <typename T>
dcn_status forward_direct_host(dcn_context* ctx, const dcn_shape* shape, const T* input,
                                      size_t input_count, const T* offset, size_t offset_count,
                                      const T* mask, size_t mask_count, const T* weight,
                                      size_t weight_count, const T* bias, size_t bias_count,
                                      T* output, size_t output_count, bool f32) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    dcn_counts c;
    DCN_TRY(validated_counts(ctx, shape, &c));
    DCN_TRY(check_count(ctx, "input", input_count, c.input));
    DCN_TRY(check_count(ctx, "offset", offset_count, c.offset));
    DCN_TRY(check_count(ctx, "mask", mask_count, c.mask));
    DCN_TRY(check_count(ctx, "weight", weight_count, c.weight));
    DCN_TRY(check_count(ctx, "bias", bias_count, c.bias));
    DCN_TRY(check_count(ctx, "output", output_count, c.output));
    if (!input || !offset || !mask || !weight || !bias || !output)
        return fail(ctx, DCN_INVALID_ARGUMENT, "host pointer is null");
    DevBuf di, doff, dm, dw, db, dout;
    DCN_TRY(upload(ctx, di, input, c.input));
    DCN_TRY(upload(ctx, doff, offset, c.offset));
    DCN_TRY(upload(ctx, dm, mask, c.mask));
    DCN_TRY(upload(ctx, dw, weight, c.weight));
    DCN_TRY(upload(ctx, db, bias, c.bias));
    DCN_HIP(ctx, hipMalloc(&dout.p, c.output * sizeof(T)));
    dcn_status st = f32 ? dcn_forward_f32_dev(ctx, shape, di.p, doff.p, dm.p, dw.p, db.p, dout.p, nullptr)
                        : dcn_forward_f16_dev(ctx, shape, di.p, doff.p, dm.p, dw.p, db.p, dout.p, nullptr);
    if (st != DCN_OK) return st;
    DCN_HIP(ctx, hipMemcpy(output, dout.p, c.output * sizeof(T), hipMemcpyDeviceToHost));
    DCN_HIP(ctx, hipDeviceSynchronize());
    return DCN_OK;
}

}  // namespace

extern "C" {

int dcn_abi_version(void) { return DCN_ABI_VERSION; }

int dcn_status_is_recoverable(dcn_status status) { return status == DCN_NONFINITE_OUTPUT; }

const char* dcn_status_string(dcn_status status) {
    // DeformConvError.description (DeformConv.swift:57-72)
    switch (status) {
        case DCN_OK: return "OK";
        case DCN_INVALID_SHAPE: return "Invalid deformable-convolution shape";
        case DCN_INVALID_ARRAY_COUNT: return "Array has the wrong number of elements";
        case DCN_DEVICE_UNAVAILABLE: return "No HIP device is available";
        case DCN_KERNEL_MISSING: return "The DCN kernels are missing for this device";
        case DCN_NONFINITE_OUTPUT: return "Model produced non-finite output";
        case DCN_COMMAND_FAILED: return "HIP command failed";
        case DCN_INVALID_ARGUMENT: return "Invalid argument";
    }
    return "Unknown status";
}

dcn_status dcn_shape_validate(const dcn_shape* s) {
    // DeformConvShape.validate (DeformConv.swift:29-41)
    if (!s) return DCN_INVALID_ARGUMENT;
    if (!(s->batch > 0 && s->input_channels > 0 && s->output_channels > 0 &&
          s->input_height > 0 && s->input_width > 0 && s->output_height > 0 &&
          s->output_width > 0 && s->kernel_height > 0 && s->kernel_width > 0 && s->groups > 0 &&
          s->offset_groups > 0 && s->input_channels % s->groups == 0 &&
          s->output_channels % s->groups == 0 && s->input_channels % s->offset_groups == 0))
        return DCN_INVALID_SHAPE;
    return DCN_OK;
}

dcn_status dcn_shape_counts(const dcn_shape* s, dcn_counts* c) {
    if (!s || !c) return DCN_INVALID_ARGUMENT;
    if (dcn_shape_validate(s) != DCN_OK) return DCN_INVALID_SHAPE;
    // DeformConv.swift:22-27
    c->kernel_area = (size_t)s->kernel_height * s->kernel_width;
    c->input = (size_t)s->batch * s->input_channels * s->input_height * s->input_width;
    c->output = (size_t)s->batch * s->output_channels * s->output_height * s->output_width;
    c->offset = (size_t)s->batch * 2 * s->offset_groups * c->kernel_area * s->output_height *
                s->output_width;
    c->mask = c->offset / 2;
    c->weight = (size_t)s->output_channels * (s->input_channels / s->groups) * c->kernel_area;
    c->bias = (size_t)s->output_channels;
    return DCN_OK;
}

int dcn_shape_fused_supported(const dcn_shape* shape) {
    if (!shape || dcn_shape_validate(shape) != DCN_OK) return 0;
    dcn::FusedGeometry g;
    return dcn::fused_geometry(*shape, &g) ? 1 : 0;
}

dcn_status dcn_create(dcn_context** out, int device) {
    if (!out) return DCN_INVALID_ARGUMENT;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return DCN_DEVICE_UNAVAILABLE;
    if (device < 0 || device >= count) return DCN_DEVICE_UNAVAILABLE;
    auto* ctx = new dcn_context();
    ctx->device = device;
    DeviceGuard guard(device);
    if (hipMalloc((void**)&ctx->flag, sizeof(uint32_t)) != hipSuccess) {
        delete ctx;
        return DCN_DEVICE_UNAVAILABLE;
    }
    // Set-up of the allocation-free entry point: the scratch array's device address on
    // this device (once per device; the device is current here).
    if (dcn::noalloc_scratch_init(device) != hipSuccess) {
        (void)hipFree(ctx->flag);
        delete ctx;
        return DCN_KERNEL_MISSING;
    }
    *out = ctx;
    return DCN_OK;
}

void dcn_destroy(dcn_context* ctx) {
    if (!ctx) return;
    DeviceGuard guard(ctx->device);
    (void)hipDeviceSynchronize();
    if (ctx->workspace) (void)hipFree(ctx->workspace);
    if (ctx->flag) (void)hipFree(ctx->flag);
    delete ctx;
}

const char* dcn_last_error(const dcn_context* ctx) {
    return ctx ? ctx->last_error.c_str() : "null context";
}

dcn_status dcn_reserve(dcn_context* ctx, const dcn_shape* shape) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    dcn_counts c;
    DCN_TRY(validated_counts(ctx, shape, &c));
    dcn::FusedGeometry g;
    if (!dcn::fused_geometry(*shape, &g)) return DCN_OK;  // nothing to reserve
    return ensure_workspace(ctx, dcn::cb8_bytes(*shape, g), nullptr);
}

dcn_status dcn_set_fused_config(dcn_context* ctx, int variant, int mt, int ks, int sampler) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    if (variant < 0 || variant > 7 || mt < 0 || mt > 32 || ks < 0 || sampler < -1 || sampler > 1)
        return fail(ctx, DCN_INVALID_ARGUMENT, "invalid fused config");
    ctx->fused_override = dcn::FusedConfig{variant, mt, ks, sampler};
    return DCN_OK;
}

dcn_status dcn_set_tile_clock_dev(dcn_context* ctx, void* d_clock, size_t count) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    if (d_clock && count == 0) return fail(ctx, DCN_INVALID_ARGUMENT, "tile clock buffer is empty");
    ctx->tile_clock = static_cast<unsigned long long*>(d_clock);
    ctx->tile_clock_count = d_clock ? count : 0;
    return DCN_OK;
}

dcn_status dcn_get_fused_config(dcn_context* ctx, const dcn_shape* shape, int* variant, int* mt,
                                int* ks, int* sampler) {
    if (!variant || !mt || !ks || !sampler) return DCN_INVALID_ARGUMENT;
    dcn_counts c;
    DCN_TRY(validated_counts(ctx, shape, &c));
    dcn::FusedGeometry g;
    if (!dcn::fused_geometry(*shape, &g)) return fail(ctx, DCN_INVALID_SHAPE, "not a fused shape");
    // A null context asks for the automatic choice (no override); it touches no device.
    const dcn::FusedConfig none{0, 0, 0, -1};
    const dcn::FusedConfig cfg = choose_config(ctx ? ctx->fused_override : none, g, *shape,
                                               dcn::window_supported(*shape), dcn::tile_supported(*shape));
    *variant = cfg.variant;
    *mt = cfg.mt;
    *ks = cfg.ks;
    *sampler = cfg.sampler;
    return DCN_OK;
}

// ---- direct paths --------------------------------------------------------------

dcn_status dcn_forward_f32_dev(dcn_context* ctx, const dcn_shape* shape, const void* d_input,
                               const void* d_offset, const void* d_mask, const void* d_weight,
                               const void* d_bias, void* d_output, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    dcn_counts c;
    DCN_TRY(validated_counts(ctx, shape, &c));
    if (!d_input || !d_offset || !d_mask || !d_weight || !d_bias || !d_output)
        return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DCN_HIP(ctx, dcn::launch_direct_f32(dcn::to_kshape(*shape), (const float*)d_input,
                                        (const float*)d_offset, (const float*)d_mask,
                                        (const float*)d_weight, (const float*)d_bias,
                                        (float*)d_output, (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_forward_f16_dev(dcn_context* ctx, const dcn_shape* shape, const void* d_input,
                               const void* d_offset, const void* d_mask, const void* d_weight,
                               const void* d_bias, void* d_output, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    dcn_counts c;
    DCN_TRY(validated_counts(ctx, shape, &c));
    if (!d_input || !d_offset || !d_mask || !d_weight || !d_bias || !d_output)
        return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DCN_HIP(ctx, dcn::launch_direct_f16(dcn::to_kshape(*shape), (const uint16_t*)d_input,
                                        (const uint16_t*)d_offset, (const uint16_t*)d_mask,
                                        (const uint16_t*)d_weight, (const uint16_t*)d_bias,
                                        (uint16_t*)d_output, (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_forward_f32(dcn_context* ctx, const dcn_shape* shape, const float* input,
                           size_t input_count, const float* offset, size_t offset_count,
                           const float* mask, size_t mask_count, const float* weight,
                           size_t weight_count, const float* bias, size_t bias_count,
                           float* output, size_t output_count) {
    return forward_direct_host<float>(ctx, shape, input, input_count, offset, offset_count, mask,
                                      mask_count, weight, weight_count, bias, bias_count, output,
                                      output_count, true);
}

dcn_status dcn_forward_f16(dcn_context* ctx, const dcn_shape* shape, const uint16_t* input,
                           size_t input_count, const uint16_t* offset, size_t offset_count,
                           const uint16_t* mask, size_t mask_count, const uint16_t* weight,
                           size_t weight_count, const uint16_t* bias, size_t bias_count,
                           uint16_t* output, size_t output_count) {
    return forward_direct_host<uint16_t>(ctx, shape, input, input_count, offset, offset_count,
                                         mask, mask_count, weight, weight_count, bias, bias_count,
                                         output, output_count, false);
}

// ---- prepack -------------------------------------------------------------------

static dcn_status make_packed(dcn_context* ctx, const dcn_shape* shape, dcn_packed** created,
                              bool bf16) {
    dcn::FusedGeometry g;
    if (!dcn::fused_geometry(*shape, &g))
        return fail(ctx, DCN_INVALID_SHAPE,
                    "fused FP16 path needs groups 1, (Cin/offsetGroups) % 8 == 0, Cout % 32 == 0, Cout <= 128");
    auto* p = new dcn_packed();
    p->shape = *shape;
    p->geometry = g;
    p->device = ctx->device;
    p->bf16 = bf16;
    // BF16 runs the register, narrow and window variants: no tile fragments.
    if (hipMalloc(&p->weights, dcn::packed_weight_bytes(g)) != hipSuccess ||
        hipMalloc((void**)&p->bias, (size_t)shape->output_channels * sizeof(float)) != hipSuccess ||
        hipMalloc(&p->weights_narrow, dcn::narrow_packed_bytes(g)) != hipSuccess ||
        (dcn::window_supported(*shape) &&
         hipMalloc(&p->weights_group, dcn::window_packed_bytes(*shape)) != hipSuccess) ||
        (!bf16 && dcn::tile_supported(*shape) &&
         hipMalloc(&p->weights_tile, dcn::tile_packed_bytes(*shape)) != hipSuccess)) {
        dcn_packed_free(p);
        return fail(ctx, DCN_COMMAND_FAILED, "hipMalloc of packed weights failed");
    }
    *created = p;
    return DCN_OK;
}

static dcn_status prepack_dev(dcn_context* ctx, const dcn_shape* shape, const void* d_weight,
                              dcn_weight_layout layout, const void* d_bias, void* stream,
                              dcn_packed** out, bool bf16) {
    if (!ctx || !out) return DCN_INVALID_ARGUMENT;
    *out = nullptr;
    DeviceGuard guard(ctx->device);
    dcn_counts c;
    DCN_TRY(validated_counts(ctx, shape, &c));
    if (!d_weight || !d_bias) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    if (layout != DCN_LAYOUT_OIHW && layout != DCN_LAYOUT_IC_K_OC)
        return fail(ctx, DCN_INVALID_ARGUMENT, "unknown weight layout");
    dcn_packed* p = nullptr;
    DCN_TRY(make_packed(ctx, shape, &p, bf16));
    hipError_t e = dcn::launch_prepack_weights(dcn::to_kshape(*shape), p->geometry,
                                               (const uint16_t*)d_weight, (int)layout,
                                               (const uint16_t*)d_bias, p->weights, p->bias,
                                               (hipStream_t)stream, bf16);
    if (e == hipSuccess && p->weights_narrow)
        e = dcn::launch_prepack_narrow(dcn::to_kshape(*shape), p->geometry, (const uint16_t*)d_weight,
                                       (int)layout, p->weights_narrow, (hipStream_t)stream);
    if (e == hipSuccess && p->weights_group)
        e = dcn::launch_prepack_group(dcn::to_kshape(*shape), (const uint16_t*)d_weight, (int)layout,
                                      p->weights_group, (hipStream_t)stream);
    if (e == hipSuccess && p->weights_tile)
        e = dcn::launch_tile_prepack(dcn::to_kshape(*shape), (const uint16_t*)d_weight, (int)layout,
                                     p->weights_tile, (hipStream_t)stream);
    if (e != hipSuccess) {
        dcn_packed_free(p);
        return hip_fail(ctx, e, "prepack launch");
    }
    *out = p;
    return DCN_OK;
}

dcn_status dcn_prepack_f16_dev(dcn_context* ctx, const dcn_shape* shape, const void* d_weight,
                               dcn_weight_layout layout, const void* d_bias, void* stream,
                               dcn_packed** out) {
    return prepack_dev(ctx, shape, d_weight, layout, d_bias, stream, out, false);
}

dcn_status dcn_prepack_bf16_dev(dcn_context* ctx, const dcn_shape* shape, const void* d_weight,
                                dcn_weight_layout layout, const void* d_bias, void* stream,
                                dcn_packed** out) {
    return prepack_dev(ctx, shape, d_weight, layout, d_bias, stream, out, true);
}

static dcn_status prepack_host(dcn_context* ctx, const dcn_shape* shape, const uint16_t* weight,
                               size_t weight_count, dcn_weight_layout layout, const uint16_t* bias,
                               size_t bias_count, dcn_packed** out, bool bf16) {
    if (!ctx || !out) return DCN_INVALID_ARGUMENT;
    *out = nullptr;
    DeviceGuard guard(ctx->device);
    dcn_counts c;
    DCN_TRY(validated_counts(ctx, shape, &c));
    DCN_TRY(check_count(ctx, "weight", weight_count, c.weight));
    DCN_TRY(check_count(ctx, "bias", bias_count, c.bias));
    if (!weight || !bias) return fail(ctx, DCN_INVALID_ARGUMENT, "host pointer is null");
    DevBuf dw, db;
    DCN_TRY(upload(ctx, dw, weight, c.weight));
    DCN_TRY(upload(ctx, db, bias, c.bias));
    dcn_packed* p = nullptr;
    DCN_TRY(prepack_dev(ctx, shape, dw.p, layout, db.p, nullptr, &p, bf16));
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        dcn_packed_free(p);
        return hip_fail(ctx, e, "prepack");
    }
    *out = p;
    return DCN_OK;
}

dcn_status dcn_prepack_f16(dcn_context* ctx, const dcn_shape* shape, const uint16_t* weight,
                           size_t weight_count, dcn_weight_layout layout, const uint16_t* bias,
                           size_t bias_count, dcn_packed** out) {
    return prepack_host(ctx, shape, weight, weight_count, layout, bias, bias_count, out, false);
}

dcn_status dcn_prepack_bf16(dcn_context* ctx, const dcn_shape* shape, const uint16_t* weight,
                            size_t weight_count, dcn_weight_layout layout, const uint16_t* bias,
                            size_t bias_count, dcn_packed** out) {
    return prepack_host(ctx, shape, weight, weight_count, layout, bias, bias_count, out, true);
}

void dcn_packed_free(dcn_packed* p) {
    if (!p) return;
    DeviceGuard guard(p->device);
    if (p->weights) (void)hipFree(p->weights);
    if (p->bias) (void)hipFree(p->bias);
    if (p->weights_group) (void)hipFree(p->weights_group);
    if (p->weights_narrow) (void)hipFree(p->weights_narrow);
    if (p->weights_tile) (void)hipFree(p->weights_tile);
    delete p;
}

size_t dcn_dcnfp16_bytes(void) { return (size_t)(128 * 9 * 64 + 64) * 2; }

dcn_status dcn_load_dcnfp16(dcn_context* ctx, const char* path, dcn_packed** out) {
    // DeformConvWeightSet.init (DeformConvWeights.swift:11-21): the file must hold
    // exactly 73,728 FP16 weights [ic=128][k=9][oc=64] followed by 64 FP16 biases.
    if (!ctx || !path || !out) return DCN_INVALID_ARGUMENT;
    *out = nullptr;
    FILE* f = std::fopen(path, "rb");
    if (!f) return fail(ctx, DCN_COMMAND_FAILED, std::string("cannot open ") + path);
    std::vector<uint8_t> data;
    uint8_t chunk[65536];
    size_t n;
    while ((n = std::fread(chunk, 1, sizeof chunk, f)) > 0) data.insert(data.end(), chunk, chunk + n);
    std::fclose(f);
    const size_t expected = dcn_dcnfp16_bytes();
    if (data.size() != expected) {
        std::string name(path);
        const size_t slash = name.find_last_of('/');
        if (slash != std::string::npos) name = name.substr(slash + 1);
        return fail(ctx, DCN_COMMAND_FAILED,
                    name + " has " + std::to_string(data.size()) + " bytes; expected " +
                        std::to_string(expected));
    }
    std::vector<uint16_t> words(expected / 2);
    std::memcpy(words.data(), data.data(), expected);  // little-endian host, as the file
    const dcn_shape shape{1, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16};
    return dcn_prepack_f16(ctx, &shape, words.data(), 128 * 9 * 64, DCN_LAYOUT_IC_K_OC,
                           words.data() + 128 * 9 * 64, 64, out);
}

// ---- fused FP16 ------------------------------------------------------------------

size_t dcn_cb8_count(const dcn_shape* shape) {
    dcn::FusedGeometry g;
    if (!shape || dcn_shape_validate(shape) != DCN_OK || shape->input_channels % 8 != 0) return 0;
    g.cblk = shape->input_channels / 8;
    g.hp = shape->input_height + 2 * DCN_CB8_PAD;
    g.wp = shape->input_width + 2 * DCN_CB8_PAD;
    return (size_t)shape->batch * g.cblk * g.hp * g.wp * 8;
}

dcn_status dcn_pack_input_cb8_dev(dcn_context* ctx, const dcn_shape* shape,
                                  const void* d_input_nchw, void* d_cb8, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    dcn_counts c;
    DCN_TRY(validated_counts(ctx, shape, &c));
    if (!d_input_nchw || !d_cb8) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    dcn::FusedGeometry g;
    if (!dcn::fused_geometry(*shape, &g)) return fail(ctx, DCN_INVALID_SHAPE, "not a fused shape");
    DCN_HIP(ctx, dcn::launch_pack_cb8(dcn::to_kshape(*shape), g, (const uint16_t*)d_input_nchw,
                                      d_cb8, (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_forward_f16_prepacked_dev(dcn_context* ctx, const dcn_shape* shape,
                                         const void* d_input, const void* d_offset,
                                         const void* d_mask, const dcn_packed* packed,
                                         void* d_output, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    return fused_prepacked_dev(ctx, shape, d_input, false, d_offset, d_mask, packed, d_output,
                               (hipStream_t)stream);
}

dcn_status dcn_forward_f16_prepacked_cb8_dev(dcn_context* ctx, const dcn_shape* shape,
                                             const void* d_cb8, const void* d_offset,
                                             const void* d_mask, const dcn_packed* packed,
                                             void* d_output, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    return fused_prepacked_dev(ctx, shape, d_cb8, true, d_offset, d_mask, packed, d_output,
                               (hipStream_t)stream);
}

dcn_status dcn_forward_f16_prepacked_noalloc_dev(dcn_context* ctx, const dcn_shape* shape,
                                                 const void* d_input, const void* d_offset,
                                                 const void* d_mask, const dcn_packed* packed,
                                                 void* d_output, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    // The device address of the scratch array, resolved by dcn_create on this device; the
    // call's use of it is ordered after the previous call's (another stream's included).
    dcn::NoallocScratchUse use(ctx->device, (hipStream_t)stream);
    if (!use.ptr())
        return fail(ctx, DCN_COMMAND_FAILED, "allocation-free scratch is not resolved on this device");
    if (use.error() != hipSuccess)
        return fail(ctx, DCN_COMMAND_FAILED,
                    std::string("ordering after the previous allocation-free call: ") + hipGetErrorString(use.error()));
    return fused_prepacked_dev(ctx, shape, d_input, false, d_offset, d_mask, packed, d_output,
                               (hipStream_t)stream, use.ptr(), DCN_NOALLOC_SCRATCH_BYTES);
}

dcn_status dcn_forward_bf16_prepacked_dev(dcn_context* ctx, const dcn_shape* shape,
                                          const void* d_input, const void* d_offset,
                                          const void* d_mask, const dcn_packed* packed,
                                          void* d_output, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    return fused_prepacked_dev(ctx, shape, d_input, false, d_offset, d_mask, packed, d_output,
                               (hipStream_t)stream, nullptr, 0, true);
}

dcn_status dcn_forward_bf16_prepacked_cb8_dev(dcn_context* ctx, const dcn_shape* shape,
                                              const void* d_cb8, const void* d_offset,
                                              const void* d_mask, const dcn_packed* packed,
                                              void* d_output, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    return fused_prepacked_dev(ctx, shape, d_cb8, true, d_offset, d_mask, packed, d_output,
                               (hipStream_t)stream, nullptr, 0, true);
}

static dcn_status forward_prepacked_host(dcn_context* ctx, const dcn_shape* shape,
                                         const uint16_t* input, size_t input_count,
                                         const uint16_t* offset, size_t offset_count,
                                         const uint16_t* mask, size_t mask_count,
                                         const dcn_packed* packed, uint16_t* output,
                                         size_t output_count, bool bf16) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    dcn_counts c;
    DCN_TRY(validated_counts(ctx, shape, &c));
    DCN_TRY(check_count(ctx, "input", input_count, c.input));
    DCN_TRY(check_count(ctx, "offset", offset_count, c.offset));
    DCN_TRY(check_count(ctx, "mask", mask_count, c.mask));
    DCN_TRY(check_count(ctx, "output", output_count, c.output));
    if (!input || !offset || !mask || !output)
        return fail(ctx, DCN_INVALID_ARGUMENT, "host pointer is null");
    DevBuf di, doff, dm, dout;
    DCN_TRY(upload(ctx, di, input, c.input));
    DCN_TRY(upload(ctx, doff, offset, c.offset));
    DCN_TRY(upload(ctx, dm, mask, c.mask));
    DCN_HIP(ctx, hipMalloc(&dout.p, c.output * sizeof(uint16_t)));
    DCN_TRY(fused_prepacked_dev(ctx, shape, di.p, false, doff.p, dm.p, packed, dout.p, nullptr,
                                nullptr, 0, bf16));
    DCN_HIP(ctx, hipMemcpy(output, dout.p, c.output * sizeof(uint16_t), hipMemcpyDeviceToHost));
    DCN_HIP(ctx, hipDeviceSynchronize());
    return DCN_OK;
}

dcn_status dcn_forward_f16_prepacked(dcn_context* ctx, const dcn_shape* shape,
                                     const uint16_t* input, size_t input_count,
                                     const uint16_t* offset, size_t offset_count,
                                     const uint16_t* mask, size_t mask_count,
                                     const dcn_packed* packed, uint16_t* output,
                                     size_t output_count) {
    return forward_prepacked_host(ctx, shape, input, input_count, offset, offset_count, mask,
                                  mask_count, packed, output, output_count, false);
}

dcn_status dcn_forward_bf16_prepacked(dcn_context* ctx, const dcn_shape* shape,
                                      const uint16_t* input, size_t input_count,
                                      const uint16_t* offset, size_t offset_count,
                                      const uint16_t* mask, size_t mask_count,
                                      const dcn_packed* packed, uint16_t* output,
                                      size_t output_count) {
    return forward_prepacked_host(ctx, shape, input, input_count, offset, offset_count, mask,
                                  mask_count, packed, output, output_count, true);
}

dcn_status dcn_im2col_f16_dev(dcn_context* ctx, const dcn_shape* shape, const void* d_input,
                              const void* d_offset, const void* d_mask, void* d_columns,
                              void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    dcn_counts c;
    DCN_TRY(validated_counts(ctx, shape, &c));
    if (!d_input || !d_offset || !d_mask || !d_columns)
        return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    if ((size_t)shape->batch * shape->output_height * shape->output_width *
            shape->input_channels * c.kernel_area >= ((size_t)1 << 31))
        return fail(ctx, DCN_INVALID_SHAPE, "im2col matrix too large");
    DCN_HIP(ctx, dcn::launch_im2col_f16(dcn::to_kshape(*shape), (const uint16_t*)d_input,
                                        (const uint16_t*)d_offset, (const uint16_t*)d_mask,
                                        (uint16_t*)d_columns, (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_launch_floor_dev(dcn_context* ctx, int workgroups, int threads, int lds_bytes,
                                void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    if (workgroups < 1 || workgroups > (1 << 20) || threads < 1 || threads > 1024 || lds_bytes < 0 ||
        lds_bytes > 160 * 1024)
        return fail(ctx, DCN_INVALID_ARGUMENT, "launch shape out of range");
    DCN_HIP(ctx, dcn::launch_floor(workgroups, threads, lds_bytes, (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_flag_nonfinite_f16_dev(dcn_context* ctx, const void* d_values, size_t count,
                                      void* d_flag, void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    if (!d_values || !d_flag) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DCN_HIP(ctx, dcn::launch_flag_nonfinite_f16((const uint16_t*)d_values, count,
                                                (uint32_t*)d_flag, (hipStream_t)stream));
    return DCN_OK;
}

dcn_status dcn_check_nonfinite_f16_dev(dcn_context* ctx, const void* d_values, size_t count,
                                       void* stream) {
    if (!ctx) return DCN_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    if (!d_values) return fail(ctx, DCN_INVALID_ARGUMENT, "device pointer is null");
    DCN_HIP(ctx, hipMemsetAsync(ctx->flag, 0, sizeof(uint32_t), (hipStream_t)stream));
    DCN_HIP(ctx, dcn::launch_flag_nonfinite_f16((const uint16_t*)d_values, count, ctx->flag,
                                                (hipStream_t)stream));
    uint32_t flag = 0;
    DCN_HIP(ctx, hipMemcpyAsync(&flag, ctx->flag, sizeof flag, hipMemcpyDeviceToHost,
                                (hipStream_t)stream));
    DCN_HIP(ctx, hipStreamSynchronize((hipStream_t)stream));
    if (flag)
        return fail(ctx, DCN_NONFINITE_OUTPUT,
                    "Model produced non-finite output: " + std::to_string(count) + " values checked");
    return DCN_OK;
}

}  // extern "C"
