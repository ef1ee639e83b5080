/*
 * CPU oracle for the DCNv2 hot path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU deformable convolution and of the
 * FP16 rounding points of its Metal kernels, used as the checker in tests/, in
 * __graft_entry__.smoke() and as bench.py's CPU baseline. Nothing in the product
 * (libdcn, the jasnamacos_amd package) links, loads or calls it.
 *
 * Every function names the reference file:line it follows (paths relative to
 * Sources/JasnaMetalPoC/ in ken8303/jasnaMacOS). Build: oracle/Makefile
 * (gcc -O2 -ffp-contract=off, no fast-math) so that float expressions evaluate
 * exactly in source order, as the Swift original does.
 */
#ifndef DCN_ORACLE_H
#define DCN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same 17 fields, same order as DeformConvShape (DeformConv.swift:3-20). */
typedef struct oracle_shape {
    int32_t batch, input_channels, input_height, input_width;
    int32_t output_channels, output_height, output_width;
    int32_t kernel_height, kernel_width, pad_height, pad_width;
    int32_t stride_height, stride_width, dilation_height, dilation_width;
    int32_t groups, offset_groups;
} oracle_shape;

/* DeformConvShape.validate (DeformConv.swift:29-41): 0 if valid, 1 = invalidShape. */
int oracle_shape_validate(const oracle_shape* s);

/* DeformConvCPU.run (DeformConv.swift:76-138) with bilinear (:146-165).
 * Loop order n, oc, oy, ox, localIC, ky, kx; sum starts at bias[oc];
 * sum += (sampled * mask) * weight. Returns 0, or 1 for an invalid shape.
 * Coordinates must be finite (the Swift original traps on Int(floor(nan))). */
int oracle_dcn_forward_f32(const oracle_shape* s, const float* input, const float* offset,
                           const float* mask, const float* weight, const float* bias,
                           float* output);

/* Output-channel slice [oc_begin, oc_end) of oracle_dcn_forward_f32, for bounded
 * CPU-baseline samples; same arithmetic. */
int oracle_dcn_forward_f32_oc_range(const oracle_shape* s, const float* input,
                                    const float* offset, const float* mask,
                                    const float* weight, const float* bias, float* output,
                                    int oc_begin, int oc_end);

/* oracle_dcn_forward_f32 with output channels spread over `threads` OpenMP threads;
 * every element is computed by the same serial code, so results are identical. */
int oracle_dcn_forward_f32_threads(const oracle_shape* s, const float* input,
                                   const float* offset, const float* mask, const float* weight,
                                   const float* bias, float* output, int threads);

/* deform_conv2d_fp16 (MetalShader.swift:126-174): FP16 storage widened exactly to
 * FP32, the oracle's summation order, output rounded once to FP16 (RNE). */
int oracle_dcn_forward_f16_direct(const oracle_shape* s, const uint16_t* input,
                                  const uint16_t* offset, const uint16_t* mask,
                                  const uint16_t* weight, const uint16_t* bias,
                                  uint16_t* output);

/* deform_conv2d_fp16_jasna_gather (MetalShader.swift:299-381), any offset-group
 * count: columns[row][ic*KA + k] = half(bilinear(ic, k) * mask), row = n*Ho*Wo + sp. */
int oracle_dcn_im2col_f16(const oracle_shape* s, const uint16_t* input,
                          const uint16_t* offset, const uint16_t* mask, uint16_t* columns);

/* BF16 storage (no counterpart in the reference, which has FP16 and FP32 only): the
 * same gather as oracle_dcn_im2col_f16 over BF16 input, offsets and mask, each sample
 * rounded once to BF16. The library's BF16 fused path computes these columns. */
int oracle_dcn_im2col_bf16(const oracle_shape* s, const uint16_t* input,
                           const uint16_t* offset, const uint16_t* mask, uint16_t* columns);
/* IEEE binary32 -> bfloat16, round to nearest even (NaN -> quiet NaN); bfloat16 ->
 * binary32 exactly (the 16 bits are the high half). */
uint16_t oracle_f32_to_bf16(float value);
float oracle_bf16_to_f32(uint16_t bits);

/* deform_conv2d_fp16_jasna_simdgroup_gemm_fused (MetalShader.swift:387-452), groups 1:
 * out[n][oc][sp] = half(sum_k col[row][k] * w[oc][k] + bias[oc]), FP32 sum in k order.
 * Weight OIHW FP16. */
int oracle_dcn_gemm_f16(const oracle_shape* s, const uint16_t* columns,
                        const uint16_t* weight, const uint16_t* bias, uint16_t* output);

/* IEEE binary16 <-> binary32, round to nearest even (Swift Float16(Float)). */
uint16_t oracle_f32_to_f16(float value);
float oracle_f16_to_f32(uint16_t bits);

/* flag_non_finite_fp16 (MetalShader.swift:454-463): 1 if any value is NaN/Inf. */
uint32_t oracle_flag_nonfinite_f16(const uint16_t* values, size_t count);

/* prepare_dcn_offsets_fp16 (MetalShader.swift:817-839) over FP16 planes:
 * raw [432][plane] + flow1/flow2 [2][plane] (x, y) -> offset [288][plane], mask [144][plane].
 * offset[c] = half(10*tanh(raw[c]) + flow_{c<144?1:2}[(c%144 even) ? y : x]),
 * mask[c] = half(1/(1+exp(-raw[288+c]))). FP32 math (tanhf, expf). */
void oracle_offset_transform_f16(size_t plane, const uint16_t* raw, const uint16_t* flow1,
                                 const uint16_t* flow2, uint16_t* offset, uint16_t* mask);

/* Zero-padded bilinear sample of an FP16 plane (sample_fp16, MetalShader.swift:51-74). */
float oracle_sample_zero_f16(const uint16_t* values, size_t base, int height, int width,
                             float y, float x);

/* accumulate_second_order_flow_fp16 + assemble_temporal_alignment_fp16
 * (MetalShader.swift:739-813) for a 64-channel feature of width x height:
 * flow2 = has_second_order ? half(flow1 + warp(prev, flow1)) : 0;
 * conditions [196][plane] = [warp(featProp, flow1), featCurrent, warp(featN2, flow2),
 * flow1, flow2]; deform_input [128][plane] = [featProp, featN2]. */
void oracle_temporal_prepare_f16(int width, int height, int has_second_order,
                                 const uint16_t* feat_prop, const uint16_t* feat_current,
                                 const uint16_t* feat_n2, const uint16_t* flow1,
                                 const uint16_t* prev_flow, uint16_t* flow2,
                                 uint16_t* conditions, uint16_t* deform_input);

/* 3x3 convolution, stride 1, pad 1, FP16 storage, FP32 accumulation in (ic, ky, kx)
 * order starting from the bias, optional LeakyReLU(slope) and optional residual:
 * out = half(residual + act(acc)), the residual added in FP32 to the unrounded activation
 * and the sum rounded once (the GPU conv epilogue's first residual; a second residual is
 * a separate FP16 add on that rounded output, oracle_add_f16). The body's offset branch and backbone
 * layers (conv_offset / backbone modules exported by tools/convert_basicvsrpp.py:181-197). */
void oracle_conv3x3_f16(int cin, int cout, int height, int width, const uint16_t* input,
                        const uint16_t* weight, const uint16_t* bias, int activation,
                        float slope, const uint16_t* residual, uint16_t* output);

/* ---- SPyNet flow estimation (the producer of the flows that feed the offsets) ---- */

/* jasna_bicubic_downsample_quarter_fp16 (MetalShader.swift:488-521) with cubic_weight
 * (:473-483, a = -0.75): out [c][h/4][w/4] = half(sum_{yy,xx in -1..2} in * wy * wx) at
 * the half-pixel source position 4 o + 1.5; every 4x4 footprint is inside the image when
 * h and w are multiples of 4 (torch interpolate(scale_factor=0.25, mode="bicubic")). */
void oracle_bicubic_quarter_f16(int channels, int height, int width, const uint16_t* input,
                                uint16_t* output);

/* spynet_build_pyramid_pair_fp16 (MetalShader.swift:523-570) for one frame: level l of
 * `levels` has size (h >> (levels - 1 - l)) x (w >> ...); each value is the direct box
 * average of the RGB frame over the level's factor x factor footprint, normalised by the
 * ImageNet mean/std and rounded once to FP16. out[l] = [3][h_l][w_l]. */
void oracle_spynet_pyramid_f16(int height, int width, int levels, const uint16_t* frame,
                               uint16_t* const* out);

/* sample_border_fp16 (MetalShader.swift:572-599): bilinear sample of plane `base` with
 * coordinates clamped into the image (grid_sample border padding, align_corners). */
float oracle_sample_border_f16(const uint16_t* values, size_t base, int height, int width,
                               float y, float x);

/* spynet_prepare_fp16 (MetalShader.swift:601-639): base flow [2][h][w] = half(2 *
 * align-corners upsample of source_flow [2][sh][sw]) (zero on the first level), and the
 * 8-channel block input [reference (3), support warped by the FP32 base flow with border
 * padding (3), base flow (2)]. */
void oracle_spynet_prepare_f16(int width, int height, int first_level, const uint16_t* reference,
                               const uint16_t* support, const uint16_t* source_flow,
                               int source_width, int source_height, uint16_t* features,
                               uint16_t* base_flow);

/* spynet_add_flow_fp16 (MetalShader.swift:641-649): out = half(base + residual), FP16 add. */
void oracle_add_f16(size_t count, const uint16_t* base, const uint16_t* residual, uint16_t* out);

/* k x k convolution (odd k), stride 1, pad k/2, otherwise as oracle_conv3x3_f16: FP32
 * accumulation in (ic, ky, kx) order from the bias, activation, output rounded to FP16.
 * SPyNet's basic-module layers are 7 x 7. */
void oracle_convk_f16(int k, int cin, int cout, int height, int width, const uint16_t* input,
                      const uint16_t* weight, const uint16_t* bias, int activation, float slope,
                      uint16_t* output);

#ifdef __cplusplus
}
#endif

#endif /* DCN_ORACLE_H */
