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
 * order starting from the bias, optional LeakyReLU(slope) and optional residual add
 * (res + half(conv)), output rounded to FP16. The body's offset branch and backbone
 * layers (conv_offset / backbone modules exported by tools/convert_basicvsrpp.py:181-197). */
void oracle_conv3x3_f16(int cin, int cout, int height, int width, const uint16_t* input,
                        const uint16_t* weight, const uint16_t* bias, int activation,
                        float slope, const uint16_t* residual, uint16_t* output);

#ifdef __cplusplus
}
#endif

#endif /* DCN_ORACLE_H */
