/*
 * CPU oracle for the DCNv2 hot path — TEST INFRASTRUCTURE ONLY (see dcn_oracle.h).
 *
 * Compiled with -O2 -ffp-contract=off and no fast-math: every float expression below
 * is evaluated in source order with one IEEE rounding per operation, like the Swift
 * original (Swift does not contract a*b+c into a fused multiply-add).
 */
#include "dcn_oracle.h"

#include <math.h>
#include <string.h>

int oracle_shape_validate(const oracle_shape* s) {
    /* DeformConv.swift:29-41 */
    if (!(s->batch > 0 && s->input_channels > 0 && s->output_channels > 0 &&
          s->input_height > 0 && s->input_width > 0 && s->output_height > 0 &&
          s->output_width > 0 && s->kernel_height > 0 && s->kernel_width > 0 &&
          s->groups > 0 && s->offset_groups > 0 &&
          s->input_channels % s->groups == 0 && s->output_channels % s->groups == 0 &&
          s->input_channels % s->offset_groups == 0))
        return 1;
    return 0;
}

/* DeformConvCPU.bilinear (DeformConv.swift:146-165). `long` stands in for Swift's Int. */
static float bilinear_f32(const float* input, size_t base, int height, int width, float y,
                          float x) {
    long y0 = (long)floorf(y);
    long x0 = (long)floorf(x);
    long y1 = y0 + 1;
    long x1 = x0 + 1;
    float ly = y - (float)y0;
    float lx = x - (float)x0;
#define ORACLE_VALUE(yy, xx)                                                          \
    (((yy) >= 0 && (yy) < height && (xx) >= 0 && (xx) < width)                         \
         ? input[base + (size_t)(yy) * (size_t)width + (size_t)(xx)]                   \
         : 0.0f)
    float v00 = ORACLE_VALUE(y0, x0);
    float v01 = ORACLE_VALUE(y0, x1);
    float v10 = ORACLE_VALUE(y1, x0);
    float v11 = ORACLE_VALUE(y1, x1);
#undef ORACLE_VALUE
    /* value(y0,x0)*(1-ly)*(1-lx) + value(y0,x1)*(1-ly)*lx + value(y1,x0)*ly*(1-lx)
     * + value(y1,x1)*ly*lx, left to right (DeformConv.swift:161-164). */
    return v00 * (1 - ly) * (1 - lx) + v01 * (1 - ly) * lx + v10 * ly * (1 - lx) +
           v11 * ly * lx;
}

/* The same bilinear over FP16 storage, widened exactly (sample_fp16, MetalShader.swift:51-74). */
float oracle_sample_zero_f16(const uint16_t* values, size_t base, int height, int width,
                             float y, float x) {
    long y0 = (long)floorf(y);
    long x0 = (long)floorf(x);
    long y1 = y0 + 1;
    long x1 = x0 + 1;
    float ly = y - (float)y0;
    float lx = x - (float)x0;
#define ORACLE_VALUE16(yy, xx)                                                        \
    (((yy) >= 0 && (yy) < height && (xx) >= 0 && (xx) < width)                         \
         ? oracle_f16_to_f32(values[base + (size_t)(yy) * (size_t)width + (size_t)(xx)]) \
         : 0.0f)
    float v00 = ORACLE_VALUE16(y0, x0);
    float v01 = ORACLE_VALUE16(y0, x1);
    float v10 = ORACLE_VALUE16(y1, x0);
    float v11 = ORACLE_VALUE16(y1, x1);
#undef ORACLE_VALUE16
    return v00 * (1.0f - ly) * (1.0f - lx) + v01 * (1.0f - ly) * lx +
           v10 * ly * (1.0f - lx) + v11 * ly * lx;
}

int oracle_dcn_forward_f32_oc_range(const oracle_shape* s, const float* input,
                                    const float* offset, const float* mask,
                                    const float* weight, const float* bias, float* output,
                                    int oc_begin, int oc_end) {
    if (oracle_shape_validate(s)) return 1;
    /* DeformConv.swift:91-95 */
    const long channels_per_group = s->input_channels / s->groups;
    const long outputs_per_group = s->output_channels / s->groups;
    const long channels_per_offset_group = s->input_channels / s->offset_groups;
    const long output_plane = (long)s->output_height * s->output_width;
    const long input_plane = (long)s->input_height * s->input_width;
    const long kernel_area = (long)s->kernel_height * s->kernel_width;

    /* DeformConv.swift:98-135 */
    for (long n = 0; n < s->batch; ++n) {
        for (long oc = oc_begin; oc < oc_end; ++oc) {
            const long group = oc / outputs_per_group;
            for (long oy = 0; oy < s->output_height; ++oy) {
                for (long ox = 0; ox < s->output_width; ++ox) {
                    float sum = bias[oc];
                    for (long local_ic = 0; local_ic < channels_per_group; ++local_ic) {
                        const long ic = group * channels_per_group + local_ic;
                        const long offset_group = ic / channels_per_offset_group;
                        for (long ky = 0; ky < s->kernel_height; ++ky) {
                            for (long kx = 0; kx < s->kernel_width; ++kx) {
                                const long kernel_index = ky * s->kernel_width + kx;
                                const long offset_channel =
                                    2 * (offset_group * kernel_area + kernel_index);
                                const long spatial = oy * s->output_width + ox;
                                const long offset_base =
                                    n * 2 * s->offset_groups * kernel_area * output_plane;
                                const float offset_y =
                                    offset[offset_base + offset_channel * output_plane + spatial];
                                const float offset_x =
                                    offset[offset_base + (offset_channel + 1) * output_plane +
                                           spatial];
                                const float y = (float)(oy * s->stride_height - s->pad_height +
                                                        ky * s->dilation_height) +
                                                offset_y;
                                const float x = (float)(ox * s->stride_width - s->pad_width +
                                                        kx * s->dilation_width) +
                                                offset_x;
                                const float sampled = bilinear_f32(
                                    input, (size_t)((n * s->input_channels + ic) * input_plane),
                                    s->input_height, s->input_width, y, x);
                                const long mask_base =
                                    n * s->offset_groups * kernel_area * output_plane;
                                const long mask_index =
                                    mask_base +
                                    (offset_group * kernel_area + kernel_index) * output_plane +
                                    spatial;
                                const long weight_index =
                                    ((oc * channels_per_group + local_ic) * s->kernel_height +
                                     ky) * s->kernel_width + kx;
                                /* sum += sampled * mask * weight  ==  sum + ((sampled*mask)*weight) */
                                sum += sampled * mask[mask_index] * weight[weight_index];
                            }
                        }
                    }
                    output[((n * s->output_channels + oc) * s->output_height + oy) *
                               s->output_width + ox] = sum;
                }
            }
        }
    }
    return 0;
}

int oracle_dcn_forward_f32(const oracle_shape* s, const float* input, const float* offset,
                           const float* mask, const float* weight, const float* bias,
                           float* output) {
    if (oracle_shape_validate(s)) return 1;
    return oracle_dcn_forward_f32_oc_range(s, input, offset, mask, weight, bias, output, 0,
                                           s->output_channels);
}

int oracle_dcn_forward_f32_threads(const oracle_shape* s, const float* input,
                                   const float* offset, const float* mask, const float* weight,
                                   const float* bias, float* output, int threads) {
    if (oracle_shape_validate(s)) return 1;
    /* Output channels are independent; each is computed exactly as in the serial loop. */
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
    for (int oc = 0; oc < s->output_channels; ++oc)
        oracle_dcn_forward_f32_oc_range(s, input, offset, mask, weight, bias, output, oc, oc + 1);
    return 0;
}

uint16_t oracle_f32_to_f16(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exponent = (x >> 23) & 0xffu;
    uint32_t mantissa = x & 0x7fffffu;
    if (exponent == 0xffu) return (uint16_t)(sign | (mantissa ? 0x7e00u : 0x7c00u));
    const int e = (int)exponent - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mantissa |= 0x800000u;
        const int shift = 14 - e;
        uint32_t h = mantissa >> shift;
        const uint32_t rest = mantissa & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1);
        if (rest > halfway || (rest == halfway && (h & 1u))) ++h;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (mantissa >> 13);
    const uint32_t rest = mantissa & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h; /* carry may reach Inf: correct */
    return (uint16_t)h;
}

float oracle_f16_to_f32(uint16_t bits) {
    const uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    const uint32_t exponent = ((uint32_t)bits >> 10) & 0x1fu;
    uint32_t mantissa = (uint32_t)bits & 0x3ffu;
    uint32_t x;
    if (exponent == 0) {
        if (mantissa == 0) {
            x = sign;
        } else {
            int e = -1;
            do {
                ++e;
                mantissa <<= 1;
            } while (!(mantissa & 0x400u));
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mantissa & 0x3ffu) << 13);
        }
    } else if (exponent == 31) {
        x = sign | 0x7f800000u | (mantissa << 13);
    } else {
        x = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float f;
    memcpy(&f, &x, sizeof f);
    return f;
}

static size_t shape_input_count(const oracle_shape* s) {
    return (size_t)s->batch * s->input_channels * s->input_height * s->input_width;
}
static size_t shape_output_count(const oracle_shape* s) {
    return (size_t)s->batch * s->output_channels * s->output_height * s->output_width;
}
static size_t shape_offset_count(const oracle_shape* s) {
    return (size_t)s->batch * 2 * s->offset_groups * s->kernel_height * s->kernel_width *
           s->output_height * s->output_width;
}
static size_t shape_mask_count(const oracle_shape* s) {
    return shape_offset_count(s) / 2;
}
static size_t shape_weight_count(const oracle_shape* s) {
    return (size_t)s->output_channels * (s->input_channels / s->groups) * s->kernel_height *
           s->kernel_width;
}

static void widen(const uint16_t* in, float* out, size_t count) {
    for (size_t i = 0; i < count; ++i) out[i] = oracle_f16_to_f32(in[i]);
}

#include <stdlib.h>

int oracle_dcn_forward_f16_direct(const oracle_shape* s, const uint16_t* input,
                                  const uint16_t* offset, const uint16_t* mask,
                                  const uint16_t* weight, const uint16_t* bias,
                                  uint16_t* output) {
    if (oracle_shape_validate(s)) return 1;
    /* deform_conv2d_fp16 widens every FP16 operand exactly and keeps the oracle's
     * FP32 expression, so it equals the FP32 oracle on widened inputs, rounded once
     * (MetalShader.swift:157-173). */
    const size_t ni = shape_input_count(s), no = shape_offset_count(s),
                 nm = shape_mask_count(s), nw = shape_weight_count(s),
                 nb = (size_t)s->output_channels, nout = shape_output_count(s);
    float* fi = (float*)malloc(ni * sizeof(float));
    float* fo = (float*)malloc(no * sizeof(float));
    float* fm = (float*)malloc(nm * sizeof(float));
    float* fw = (float*)malloc(nw * sizeof(float));
    float* fb = (float*)malloc(nb * sizeof(float));
    float* out = (float*)malloc(nout * sizeof(float));
    int rc = 2;
    if (fi && fo && fm && fw && fb && out) {
        widen(input, fi, ni);
        widen(offset, fo, no);
        widen(mask, fm, nm);
        widen(weight, fw, nw);
        widen(bias, fb, nb);
        rc = oracle_dcn_forward_f32(s, fi, fo, fm, fw, fb, out);
        if (rc == 0)
            for (size_t i = 0; i < nout; ++i) output[i] = oracle_f32_to_f16(out[i]);
    }
    free(fi);
    free(fo);
    free(fm);
    free(fw);
    free(fb);
    free(out);
    return rc;
}

int oracle_dcn_im2col_f16(const oracle_shape* s, const uint16_t* input,
                          const uint16_t* offset, const uint16_t* mask, uint16_t* columns) {
    if (oracle_shape_validate(s)) return 1;
    const long plane = (long)s->output_height * s->output_width;
    const long input_plane = (long)s->input_height * s->input_width;
    const long kernel_area = (long)s->kernel_height * s->kernel_width;
    const long cpog = s->input_channels / s->offset_groups;
    const long columns_per_row = (long)s->input_channels * kernel_area;
    const long rows = (long)s->batch * plane;
    for (long row = 0; row < rows; ++row) {
        const long n = row / plane;
        const long spatial = row % plane;
        const long oy = spatial / s->output_width;
        const long ox = spatial % s->output_width;
        const long offset_base = n * 2 * s->offset_groups * kernel_area * plane;
        const long mask_base = n * s->offset_groups * kernel_area * plane;
        for (long ic = 0; ic < s->input_channels; ++ic) {
            const long og = ic / cpog;
            for (long k = 0; k < kernel_area; ++k) {
                const long ky = k / s->kernel_width;
                const long kx = k % s->kernel_width;
                const long sample = og * kernel_area + k;
                /* MetalShader.swift:327-332: float(int(oy*sh + ky*dh) - int(ph)) + offset */
                const float y = (float)(oy * s->stride_height + ky * s->dilation_height -
                                        s->pad_height) +
                                oracle_f16_to_f32(offset[offset_base + 2 * sample * plane + spatial]);
                const float x =
                    (float)(ox * s->stride_width + kx * s->dilation_width - s->pad_width) +
                    oracle_f16_to_f32(offset[offset_base + (2 * sample + 1) * plane + spatial]);
                const float sampled = oracle_sample_zero_f16(
                    input, (size_t)((n * s->input_channels + ic) * input_plane),
                    s->input_height, s->input_width, y, x);
                const float m = oracle_f16_to_f32(mask[mask_base + sample * plane + spatial]);
                /* MetalShader.swift:377-379: gathered = half(sampled * mask) */
                columns[row * columns_per_row + ic * kernel_area + k] =
                    oracle_f32_to_f16(sampled * m);
            }
        }
    }
    return 0;
}

uint16_t oracle_f32_to_bf16(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof x);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u); /* NaN */
    x += 0x7fffu + ((x >> 16) & 1u); /* nearest, ties to even; a carry may reach Inf */
    return (uint16_t)(x >> 16);
}

float oracle_bf16_to_f32(uint16_t bits) {
    const uint32_t x = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &x, sizeof f);
    return f;
}

/* oracle_sample_zero_f16 over BF16 storage: the same corners, zero padding and
 * association, values widened from BF16. */
static float sample_zero_bf16(const uint16_t* values, size_t base, int height, int width,
                              float y, float x) {
    long y0 = (long)floorf(y);
    long x0 = (long)floorf(x);
    long y1 = y0 + 1;
    long x1 = x0 + 1;
    float ly = y - (float)y0;
    float lx = x - (float)x0;
#define ORACLE_VALUE_BF16(yy, xx)                                                       \
    (((yy) >= 0 && (yy) < height && (xx) >= 0 && (xx) < width)                           \
         ? oracle_bf16_to_f32(values[base + (size_t)(yy) * (size_t)width + (size_t)(xx)]) \
         : 0.0f)
    float v00 = ORACLE_VALUE_BF16(y0, x0);
    float v01 = ORACLE_VALUE_BF16(y0, x1);
    float v10 = ORACLE_VALUE_BF16(y1, x0);
    float v11 = ORACLE_VALUE_BF16(y1, x1);
#undef ORACLE_VALUE_BF16
    return v00 * (1.0f - ly) * (1.0f - lx) + v01 * (1.0f - ly) * lx +
           v10 * ly * (1.0f - lx) + v11 * ly * lx;
}

int oracle_dcn_im2col_bf16(const oracle_shape* s, const uint16_t* input,
                           const uint16_t* offset, const uint16_t* mask, uint16_t* columns) {
    if (oracle_shape_validate(s)) return 1;
    const long plane = (long)s->output_height * s->output_width;
    const long input_plane = (long)s->input_height * s->input_width;
    const long kernel_area = (long)s->kernel_height * s->kernel_width;
    const long cpog = s->input_channels / s->offset_groups;
    const long columns_per_row = (long)s->input_channels * kernel_area;
    const long rows = (long)s->batch * plane;
    for (long row = 0; row < rows; ++row) {
        const long n = row / plane;
        const long spatial = row % plane;
        const long oy = spatial / s->output_width;
        const long ox = spatial % s->output_width;
        const long offset_base = n * 2 * s->offset_groups * kernel_area * plane;
        const long mask_base = n * s->offset_groups * kernel_area * plane;
        for (long ic = 0; ic < s->input_channels; ++ic) {
            const long og = ic / cpog;
            for (long k = 0; k < kernel_area; ++k) {
                const long ky = k / s->kernel_width;
                const long kx = k % s->kernel_width;
                const long sample = og * kernel_area + k;
                /* the coordinate arithmetic of oracle_dcn_im2col_f16 */
                const float y = (float)(oy * s->stride_height + ky * s->dilation_height -
                                        s->pad_height) +
                                oracle_bf16_to_f32(offset[offset_base + 2 * sample * plane + spatial]);
                const float x =
                    (float)(ox * s->stride_width + kx * s->dilation_width - s->pad_width) +
                    oracle_bf16_to_f32(offset[offset_base + (2 * sample + 1) * plane + spatial]);
                const float sampled = sample_zero_bf16(
                    input, (size_t)((n * s->input_channels + ic) * input_plane),
                    s->input_height, s->input_width, y, x);
                const float m = oracle_bf16_to_f32(mask[mask_base + sample * plane + spatial]);
                columns[row * columns_per_row + ic * kernel_area + k] =
                    oracle_f32_to_bf16(sampled * m);
            }
        }
    }
    return 0;
}

int oracle_dcn_gemm_f16(const oracle_shape* s, const uint16_t* columns,
                        const uint16_t* weight, const uint16_t* bias, uint16_t* output) {
    if (oracle_shape_validate(s) || s->groups != 1) return 1;
    const long plane = (long)s->output_height * s->output_width;
    const long kdim = (long)s->input_channels * s->kernel_height * s->kernel_width;
    const long rows = (long)s->batch * plane;
    float* wf = (float*)malloc((size_t)kdim * s->output_channels * sizeof(float));
    float* cf = (float*)malloc((size_t)kdim * sizeof(float));
    if (!wf || !cf) {
        free(wf);
        free(cf);
        return 2;
    }
    widen(weight, wf, (size_t)kdim * s->output_channels);
    for (long row = 0; row < rows; ++row) {
        const long n = row / plane;
        const long spatial = row % plane;
        widen(columns + row * kdim, cf, (size_t)kdim);
        for (long oc = 0; oc < s->output_channels; ++oc) {
            const float* w = wf + oc * kdim;
            float acc = 0.0f;
            for (long k = 0; k < kdim; ++k) acc += cf[k] * w[k];
            /* MetalShader.swift:447-449: half(acc + bias) */
            output[(n * s->output_channels + oc) * plane + spatial] =
                oracle_f32_to_f16(acc + oracle_f16_to_f32(bias[oc]));
        }
    }
    free(wf);
    free(cf);
    return 0;
}

uint32_t oracle_flag_nonfinite_f16(const uint16_t* values, size_t count) {
    /* !isfinite(float(v)) <=> exponent bits all ones (MetalShader.swift:454-463) */
    for (size_t i = 0; i < count; ++i)
        if ((values[i] & 0x7c00u) == 0x7c00u) return 1u;
    return 0u;
}

void oracle_offset_transform_f16(size_t plane, const uint16_t* raw, const uint16_t* flow1,
                                 const uint16_t* flow2, uint16_t* offset, uint16_t* mask) {
    /* MetalShader.swift:824-838 */
    for (size_t channel = 0; channel < 432; ++channel) {
        for (size_t spatial = 0; spatial < plane; ++spatial) {
            const size_t gid = channel * plane + spatial;
            if (channel < 288) {
                const size_t local = channel % 144;
                const uint16_t* flow = channel < 144 ? flow1 : flow2;
                /* flow is [x, y]; even local channels are dy, odd are dx */
                const size_t flow_channel = (local & 1u) == 0 ? 1 : 0;
                const float residue = 10.0f * tanhf(oracle_f16_to_f32(raw[gid]));
                offset[gid] = oracle_f32_to_f16(
                    residue + oracle_f16_to_f32(flow[flow_channel * plane + spatial]));
            } else {
                const float value = oracle_f16_to_f32(raw[gid]);
                mask[(channel - 288) * plane + spatial] =
                    oracle_f32_to_f16(1.0f / (1.0f + expf(-value)));
            }
        }
    }
}

void oracle_temporal_prepare_f16(int width, int height, int has_second_order,
                                 const uint16_t* feat_prop, const uint16_t* feat_current,
                                 const uint16_t* feat_n2, const uint16_t* flow1,
                                 const uint16_t* prev_flow, uint16_t* flow2,
                                 uint16_t* conditions, uint16_t* deform_input) {
    const size_t plane = (size_t)width * height;
    /* accumulate_second_order_flow_fp16 (MetalShader.swift:742-763) */
    for (size_t gid = 0; gid < 2 * plane; ++gid) {
        if (!has_second_order) {
            flow2[gid] = 0;
            continue;
        }
        const size_t channel = gid / plane, spatial = gid % plane;
        const int y = (int)(spatial / (size_t)width), x = (int)(spatial % (size_t)width);
        const float fx = oracle_f16_to_f32(flow1[spatial]);
        const float fy = oracle_f16_to_f32(flow1[plane + spatial]);
        const float previous = oracle_sample_zero_f16(prev_flow, channel * plane, height, width,
                                                      (float)y + fy, (float)x + fx);
        flow2[gid] = oracle_f32_to_f16(oracle_f16_to_f32(flow1[gid]) + previous);
    }
    /* assemble_temporal_alignment_fp16 (MetalShader.swift:769-813) */
    for (size_t gid = 0; gid < 196 * plane; ++gid) {
        const size_t channel = gid / plane, spatial = gid % plane;
        const int y = (int)(spatial / (size_t)width), x = (int)(spatial % (size_t)width);
        if (gid < 128 * plane)
            deform_input[gid] =
                channel < 64 ? feat_prop[gid] : feat_n2[(channel - 64) * plane + spatial];
        uint16_t value;
        if (channel < 64) {
            const float fx = oracle_f16_to_f32(flow1[spatial]);
            const float fy = oracle_f16_to_f32(flow1[plane + spatial]);
            value = oracle_f32_to_f16(oracle_sample_zero_f16(feat_prop, channel * plane, height,
                                                             width, (float)y + fy, (float)x + fx));
        } else if (channel < 128) {
            value = feat_current[(channel - 64) * plane + spatial];
        } else if (channel < 192) {
            const float fx = oracle_f16_to_f32(flow2[spatial]);
            const float fy = oracle_f16_to_f32(flow2[plane + spatial]);
            value = oracle_f32_to_f16(oracle_sample_zero_f16(feat_n2, (channel - 128) * plane,
                                                             height, width, (float)y + fy,
                                                             (float)x + fx));
        } else if (channel < 194) {
            value = flow1[(channel - 192) * plane + spatial];
        } else {
            value = flow2[(channel - 194) * plane + spatial];
        }
        conditions[gid] = value;
    }
}

void oracle_conv3x3_f16(int cin, int cout, int height, int width, const uint16_t* input,
                        const uint16_t* weight, const uint16_t* bias, int activation,
                        float slope, const uint16_t* residual, uint16_t* output) {
    /* activation: 0 none, 1 LeakyReLU(slope), 2 ReLU. out = half(residual + act(acc)):
     * one rounding after the FP32 residual add, not half(residual + half(act(acc))).
     * FP16 -> FP32 is exact, so the operands are widened once up front; every product and
     * sum is then the same FP32 operation, in the same order, as widening in the loop. */
    const size_t plane = (size_t)width * height;
    const size_t in_count = (size_t)cin * plane, w_count = (size_t)cout * cin * 9;
    float* in32 = (float*)malloc(in_count * sizeof(float));
    float* w32 = (float*)malloc(w_count * sizeof(float));
    if (!in32 || !w32) abort(); /* test infrastructure: fail loudly rather than leave output unset */
    for (size_t i = 0; i < in_count; ++i) in32[i] = oracle_f16_to_f32(input[i]);
    for (size_t i = 0; i < w_count; ++i) w32[i] = oracle_f16_to_f32(weight[i]);
    /* Output channels are independent; each element is computed by the same serial code. */
#pragma omp parallel for schedule(static)
    for (int oc = 0; oc < cout; ++oc) {
        for (int oy = 0; oy < height; ++oy) {
            for (int ox = 0; ox < width; ++ox) {
                float acc = oracle_f16_to_f32(bias[oc]);
                for (int ic = 0; ic < cin; ++ic) {
                    const float* src = in32 + (size_t)ic * plane;
                    const float* wk = w32 + ((size_t)oc * cin + ic) * 9;
                    for (int ky = 0; ky < 3; ++ky) {
                        const int iy = oy + ky - 1;
                        if (iy < 0 || iy >= height) continue;
                        for (int kx = 0; kx < 3; ++kx) {
                            const int ix = ox + kx - 1;
                            if (ix < 0 || ix >= width) continue;
                            acc += src[(size_t)iy * width + ix] * wk[ky * 3 + kx];
                        }
                    }
                }
                if (activation == 1 && acc < 0.0f) acc = acc * slope;
                if (activation == 2 && acc < 0.0f) acc = 0.0f;
                const size_t index = (size_t)oc * plane + (size_t)oy * width + ox;
                if (residual) acc = oracle_f16_to_f32(residual[index]) + acc;
                output[index] = oracle_f32_to_f16(acc);
            }
        }
    }
    free(in32);
    free(w32);
}

/* ---- SPyNet flow estimation ---- */

/* cubic_weight (MetalShader.swift:473-483), a = -0.75. */
static float cubic_weight(float distance) {
    const float a = -0.75f;
    const float x = fabsf(distance);
    if (x <= 1.0f) return (a + 2.0f) * x * x * x - (a + 3.0f) * x * x + 1.0f;
    if (x < 2.0f) return a * x * x * x - 5.0f * a * x * x + 8.0f * a * x - 4.0f * a;
    return 0.0f;
}

void oracle_bicubic_quarter_f16(int channels, int height, int width, const uint16_t* input,
                                uint16_t* output) {
    /* jasna_bicubic_downsample_quarter_fp16 (MetalShader.swift:488-521). */
    const int oh = height / 4, ow = width / 4;
    for (int c = 0; c < channels; ++c) {
        for (int oy = 0; oy < oh; ++oy) {
            for (int ox = 0; ox < ow; ++ox) {
                const float sy = ((float)oy + 0.5f) * 4.0f - 0.5f;
                const float sx = ((float)ox + 0.5f) * 4.0f - 0.5f;
                const int by = (int)floorf(sy);
                const int bx = (int)floorf(sx);
                float value = 0.0f;
                for (int yy = -1; yy <= 2; ++yy) {
                    const float wy = cubic_weight(sy - (float)(by + yy));
                    for (int xx = -1; xx <= 2; ++xx) {
                        const float wx = cubic_weight(sx - (float)(bx + xx));
                        const size_t src = ((size_t)c * height + (size_t)(by + yy)) * width + (size_t)(bx + xx);
                        value += oracle_f16_to_f32(input[src]) * wy * wx;
                    }
                }
                output[((size_t)c * oh + oy) * ow + ox] = oracle_f32_to_f16(value);
            }
        }
    }
}

void oracle_spynet_pyramid_f16(int height, int width, int levels, const uint16_t* frame,
                               uint16_t* const* out) {
    /* spynet_build_pyramid_pair_fp16 (MetalShader.swift:523-570): direct box averages,
     * ImageNet normalisation (:560-563). */
    static const float mean[3] = {0.485f, 0.456f, 0.406f};
    static const float stddev[3] = {0.229f, 0.224f, 0.225f};
    for (int l = 0; l < levels; ++l) {
        const int shift = levels - 1 - l;
        const int lh = height >> shift, lw = width >> shift;
        const int factor = 1 << shift;
        const float inverse_area = 1.0f / (float)(factor * factor);
        for (int c = 0; c < 3; ++c) {
            for (int y = 0; y < lh; ++y) {
                for (int x = 0; x < lw; ++x) {
                    float sum = 0.0f;
                    for (int yy = 0; yy < factor; ++yy)
                        for (int xx = 0; xx < factor; ++xx)
                            sum += oracle_f16_to_f32(
                                frame[((size_t)c * height + (size_t)(y * factor + yy)) * width + x * factor + xx]);
                    out[l][((size_t)c * lh + y) * lw + x] =
                        oracle_f32_to_f16((sum * inverse_area - mean[c]) / stddev[c]);
                }
            }
        }
    }
}

float oracle_sample_border_f16(const uint16_t* values, size_t base, int height, int width,
                               float y, float x) {
    /* sample_border_fp16 (MetalShader.swift:572-599). */
    y = fminf(fmaxf(y, 0.0f), (float)(height - 1));
    x = fminf(fmaxf(x, 0.0f), (float)(width - 1));
    const int y0 = (int)floorf(y);
    const int x0 = (int)floorf(x);
    const int y1 = y0 + 1 < height - 1 ? y0 + 1 : height - 1;
    const int x1 = x0 + 1 < width - 1 ? x0 + 1 : width - 1;
    const float ly = y - (float)y0;
    const float lx = x - (float)x0;
    const float v00 = oracle_f16_to_f32(values[base + (size_t)y0 * width + x0]);
    const float v01 = oracle_f16_to_f32(values[base + (size_t)y0 * width + x1]);
    const float v10 = oracle_f16_to_f32(values[base + (size_t)y1 * width + x0]);
    const float v11 = oracle_f16_to_f32(values[base + (size_t)y1 * width + x1]);
    return v00 * (1.0f - ly) * (1.0f - lx) + v01 * (1.0f - ly) * lx + v10 * ly * (1.0f - lx) +
           v11 * ly * lx;
}

void oracle_spynet_prepare_f16(int width, int height, int first_level, const uint16_t* reference,
                               const uint16_t* support, const uint16_t* source_flow,
                               int source_width, int source_height, uint16_t* features,
                               uint16_t* base_flow) {
    /* spynet_prepare_fp16 (MetalShader.swift:601-639). */
    const size_t plane = (size_t)width * height;
    const size_t source_plane = (size_t)source_width * source_height;
    for (int y = 0; y < height; ++y) {
        for (int x = 0; x < width; ++x) {
            const size_t gid = (size_t)y * width + x;
            float flow_x = 0.0f, flow_y = 0.0f;
            if (!first_level) {
                const float sx = width > 1 ? (float)x * (float)(source_width - 1) / (float)(width - 1) : 0.0f;
                const float sy = height > 1 ? (float)y * (float)(source_height - 1) / (float)(height - 1) : 0.0f;
                flow_x = 2.0f * oracle_sample_border_f16(source_flow, 0, source_height, source_width, sy, sx);
                flow_y = 2.0f * oracle_sample_border_f16(source_flow, source_plane, source_height, source_width,
                                                         sy, sx);
            }
            base_flow[gid] = oracle_f32_to_f16(flow_x);
            base_flow[plane + gid] = oracle_f32_to_f16(flow_y);
            for (int c = 0; c < 3; ++c) {
                features[(size_t)c * plane + gid] = reference[(size_t)c * plane + gid];
                const float warped = oracle_sample_border_f16(support, (size_t)c * plane, height, width,
                                                              (float)y + flow_y, (float)x + flow_x);
                features[(size_t)(c + 3) * plane + gid] = oracle_f32_to_f16(warped);
            }
            features[6 * plane + gid] = oracle_f32_to_f16(flow_x);
            features[7 * plane + gid] = oracle_f32_to_f16(flow_y);
        }
    }
}

void oracle_add_f16(size_t count, const uint16_t* base, const uint16_t* residual, uint16_t* out) {
    /* spynet_add_flow_fp16 (MetalShader.swift:641-649): a half + half add is the exact
     * sum rounded once. */
    for (size_t i = 0; i < count; ++i)
        out[i] = oracle_f32_to_f16(oracle_f16_to_f32(base[i]) + oracle_f16_to_f32(residual[i]));
}

void oracle_convk_f16(int k, int cin, int cout, int height, int width, const uint16_t* input,
                      const uint16_t* weight, const uint16_t* bias, int activation, float slope,
                      uint16_t* output) {
    const size_t plane = (size_t)width * height;
    const int pad = k / 2;
#pragma omp parallel for schedule(static)
    for (int oc = 0; oc < cout; ++oc) {
        for (int oy = 0; oy < height; ++oy) {
            for (int ox = 0; ox < width; ++ox) {
                float acc = oracle_f16_to_f32(bias[oc]);
                for (int ic = 0; ic < cin; ++ic) {
                    for (int ky = 0; ky < k; ++ky) {
                        const int iy = oy + ky - pad;
                        if (iy < 0 || iy >= height) continue;
                        for (int kx = 0; kx < k; ++kx) {
                            const int ix = ox + kx - pad;
                            if (ix < 0 || ix >= width) continue;
                            acc += oracle_f16_to_f32(input[(size_t)ic * plane + (size_t)iy * width + ix]) *
                                   oracle_f16_to_f32(weight[(((size_t)oc * cin + ic) * k + ky) * k + kx]);
                        }
                    }
                }
                if (activation == 1 && acc < 0.0f) acc = acc * slope;
                if (activation == 2 && acc < 0.0f) acc = 0.0f;
                output[(size_t)oc * plane + (size_t)oy * width + ox] = oracle_f32_to_f16(acc);
            }
        }
    }
}
