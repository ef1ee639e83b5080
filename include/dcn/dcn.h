/*
 * libdcn — MI355X (gfx950) modulated deformable convolution (DCNv2) behind a C ABI.
 *
 * This header is the drop-in boundary for the deformable-convolution operator of
 * ken8303/jasnaMacOS. The reference's surface is Swift-internal; each declaration
 * below names the reference item (file:line under Sources/JasnaMetalPoC/ unless
 * stated) that it replaces. A SwiftPM C module target wraps this header as is
 * (jasnamacos_amd/swift: module CDCN, link "dcn").
 *
 * Conventions
 *  - Plain pointers and element counts. Host-pointer entry points validate every
 *    count against the shape and report name/expected/actual through
 *    dcn_last_error(), as DeformConvCPU.require does (DeformConv.swift:140-144).
 *  - FP16 data is passed as IEEE binary16 bit patterns (uint16_t).
 *  - Tensors are NCHW, as in the reference: input [B][Cin][H][W],
 *    offset [B][2*G*Kh*Kw][Ho][Wo] with channel 2*(g*Kh*Kw+k) = dy and +1 = dx,
 *    mask [B][G*Kh*Kw][Ho][Wo], weight OIHW [Cout][Cin/groups][Kh][Kw],
 *    output [B][Cout][Ho][Wo] (DeformConv.swift:110-132).
 *  - One context per host thread; a context is not internally locked. Host-pointer
 *    calls synchronise before returning. *_dev calls are asynchronous on the stream
 *    given and never allocate once dcn_reserve() has sized the context's workspace,
 *    so they can be captured into a hipGraph.
 *  - The caller owns every buffer it passes. Packed weights are owned by their
 *    handle (dcn_packed_free).
 */
#ifndef DCN_DCN_H
#define DCN_DCN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DCN_ABI_VERSION 1

/* Error taxonomy. Replaces DeformConvError (DeformConv.swift:44-73):
 * invalidShape, invalidArrayCount, metalUnavailable, shaderResourceMissing,
 * nonFiniteOutput, commandFailed. DCN_INVALID_ARGUMENT has no Swift counterpart:
 * it reports a null pointer or a null context, which Swift arrays cannot be. */
typedef enum dcn_status {
    DCN_OK = 0,
    DCN_INVALID_SHAPE = 1,
    DCN_INVALID_ARRAY_COUNT = 2,
    DCN_DEVICE_UNAVAILABLE = 3,
    DCN_KERNEL_MISSING = 4,
    DCN_NONFINITE_OUTPUT = 5,
    DCN_COMMAND_FAILED = 6,
    DCN_INVALID_ARGUMENT = 7
} dcn_status;

/* 1 only for DCN_NONFINITE_OUTPUT (isRecoverableNumericalFailure, DeformConv.swift:52-55). */
int dcn_status_is_recoverable(dcn_status status);
/* Static description of a status (DeformConvError.description, DeformConv.swift:57-72). */
const char* dcn_status_string(dcn_status status);
int dcn_abi_version(void);

/* DeformConvShape (DeformConv.swift:3-20), same field order. Output H/W are given,
 * not derived, as in the reference. */
typedef struct dcn_shape {
    int32_t batch;
    int32_t input_channels;
    int32_t input_height;
    int32_t input_width;
    int32_t output_channels;
    int32_t output_height;
    int32_t output_width;
    int32_t kernel_height;
    int32_t kernel_width;
    int32_t pad_height;
    int32_t pad_width;
    int32_t stride_height;
    int32_t stride_width;
    int32_t dilation_height;
    int32_t dilation_width;
    int32_t groups;
    int32_t offset_groups;
} dcn_shape;

/* Derived element counts (DeformConv.swift:22-27). */
typedef struct dcn_counts {
    size_t input;
    size_t output;
    size_t kernel_area;
    size_t offset;
    size_t mask;
    size_t weight;
    size_t bias;
} dcn_counts;

/* DeformConvShape.validate (DeformConv.swift:29-41): positive sizes, groups and
 * offset groups; Cin % groups == 0, Cout % groups == 0, Cin % offsetGroups == 0.
 * Returns DCN_INVALID_SHAPE otherwise. */
dcn_status dcn_shape_validate(const dcn_shape* shape);
dcn_status dcn_shape_counts(const dcn_shape* shape, dcn_counts* counts);
/* 1 if the fused FP16 sampler+MFMA path serves this shape: groups == 1,
 * (Cin/offsetGroups) % 8 == 0, Cout % 32 == 0 and Cout <= 128. The prepacked
 * entry points return DCN_INVALID_SHAPE otherwise, as executeJasnaSIMDGroupGEMM
 * does for shapes its kernels do not cover (MetalRunner.swift:696-710). */
int dcn_shape_fused_supported(const dcn_shape* shape);

/* ---- context: MetalDeformConv.init (MetalRunner.swift:107-144) ---------------- */
typedef struct dcn_context dcn_context;
dcn_status dcn_create(dcn_context** out, int device);
void dcn_destroy(dcn_context* ctx);
/* Detail of the last failure on this context ("offset has 3 elements; expected 4"). */
const char* dcn_last_error(const dcn_context* ctx);
/* Size the context's device workspace for `shape` so later *_dev calls do not
 * allocate (call before hipGraph capture). */
dcn_status dcn_reserve(dcn_context* ctx, const dcn_shape* shape);

/* ---- host-pointer entry points (copy in, run, copy out, synchronise) ------------ */

/* FP32 DCNv2. MetalDeformConv.runFloat32 (MetalRunner.swift:159-185) over
 * deform_conv2d_fp32 (MetalShader.swift:76-124). Same summation order as
 * DeformConvCPU.run (DeformConv.swift:98-135) with contraction off, so results
 * are bit-identical to that oracle. Any valid shape. */
dcn_status dcn_forward_f32(dcn_context* ctx, const dcn_shape* shape,
                           const float* input, size_t input_count,
                           const float* offset, size_t offset_count,
                           const float* mask, size_t mask_count,
                           const float* weight, size_t weight_count,
                           const float* bias, size_t bias_count,
                           float* output, size_t output_count);

/* FP16 storage, FP32 accumulation in the oracle's order, half(sum) output:
 * deform_conv2d_fp16 (MetalShader.swift:126-174) as dispatched by
 * benchmarkJasnaShape's baseline (MetalRunner.swift:277-283). OIHW weights. */
dcn_status dcn_forward_f16(dcn_context* ctx, const dcn_shape* shape,
                           const uint16_t* input, size_t input_count,
                           const uint16_t* offset, size_t offset_count,
                           const uint16_t* mask, size_t mask_count,
                           const uint16_t* weight, size_t weight_count,
                           const uint16_t* bias, size_t bias_count,
                           uint16_t* output, size_t output_count);

/* ---- one-time weight prepack ---------------------------------------------------- */
typedef enum dcn_weight_layout {
    /* [Cout][Cin][Kh][Kw], PyTorch / DeformConvCPU order. */
    DCN_LAYOUT_OIHW = 0,
    /* [Cin][Kh*Kw][Cout], the .dcnfp16 / Metal packed order
     * (tools/export_deform_weights.py:47, MetalRunner.swift:235-243). */
    DCN_LAYOUT_IC_K_OC = 1
} dcn_weight_layout;

typedef struct dcn_packed dcn_packed;

/* Pack FP16 weights + bias once into the MFMA B-fragment layout held on the
 * context's device. Replaces the OIHW -> [ic][k][oc] packing of
 * benchmarkJasnaShape (MetalRunner.swift:214-243) and the weight-buffer cache
 * MetalResourceCache.deformConvWeightBuffers (MetalResourceCache.swift:86-106). */
dcn_status dcn_prepack_f16(dcn_context* ctx, const dcn_shape* shape,
                           const uint16_t* weight, size_t weight_count,
                           dcn_weight_layout layout,
                           const uint16_t* bias, size_t bias_count,
                           dcn_packed** out);
/* Same, from device buffers (stream-ordered; the handle is valid once the
 * stream reaches this point). */
dcn_status dcn_prepack_f16_dev(dcn_context* ctx, const dcn_shape* shape,
                               const void* d_weight, dcn_weight_layout layout,
                               const void* d_bias, void* stream, dcn_packed** out);
void dcn_packed_free(dcn_packed* packed);
/* Load a 147,584-byte .dcnfp16 file (FP16 weight [128][9][64] then bias [64])
 * and prepack it for the 1x128xHxW -> 64, 3x3, 16-group shape.
 * DeformConvWeightSet.init + makeBuffers (DeformConvWeights.swift:4-36). A file
 * of another size fails with DCN_COMMAND_FAILED and the byte counts in
 * dcn_last_error, as the reference does. */
dcn_status dcn_load_dcnfp16(dcn_context* ctx, const char* path, dcn_packed** out);
/* Expected .dcnfp16 size in bytes (DeformConvWeightSet.expectedBytes). */
size_t dcn_dcnfp16_bytes(void);

/* FP16 DCNv2 with prepacked weights: fused bilinear sampler + MFMA GEMM, FP32
 * accumulation, half(acc + bias) output. Replaces the gather + SIMD-group GEMM pair
 * executeJasnaSIMDGroupGEMM (MetalRunner.swift:696-761) over
 * deform_conv2d_fp16_jasna_gather / _simdgroup_gemm_fused (MetalShader.swift:299-452).
 * The im2col tile never reaches HBM. */
dcn_status dcn_forward_f16_prepacked(dcn_context* ctx, const dcn_shape* shape,
                                     const uint16_t* input, size_t input_count,
                                     const uint16_t* offset, size_t offset_count,
                                     const uint16_t* mask, size_t mask_count,
                                     const dcn_packed* packed,
                                     uint16_t* output, size_t output_count);

/* ---- device-pointer, stream-ordered entry points (hipGraph capturable) -------- */
/* `stream` is a hipStream_t (NULL = the default stream). Device pointers must
 * hold the element counts dcn_shape_counts reports. */
dcn_status dcn_forward_f32_dev(dcn_context* ctx, const dcn_shape* shape,
                               const void* d_input, const void* d_offset, const void* d_mask,
                               const void* d_weight, const void* d_bias, void* d_output,
                               void* stream);
dcn_status dcn_forward_f16_dev(dcn_context* ctx, const dcn_shape* shape,
                               const void* d_input, const void* d_offset, const void* d_mask,
                               const void* d_weight, const void* d_bias, void* d_output,
                               void* stream);
/* NCHW FP16 input; the context's workspace receives the padded channel-block copy. */
dcn_status dcn_forward_f16_prepacked_dev(dcn_context* ctx, const dcn_shape* shape,
                                         const void* d_input, const void* d_offset,
                                         const void* d_mask, const dcn_packed* packed,
                                         void* d_output, void* stream);

/* The padded channel-block input layout the fused sampler reads:
 * [B][Cin/8][H+2*DCN_CB8_PAD][W+2*DCN_CB8_PAD][8] FP16 with a zero border.
 * Producers that can write it directly (the propagation body does) skip the
 * NCHW repack. dcn_cb8_count gives its element count. */
#define DCN_CB8_PAD 2
size_t dcn_cb8_count(const dcn_shape* shape);
/* Repack NCHW FP16 -> padded channel-block layout; writes interior and border. */
dcn_status dcn_pack_input_cb8_dev(dcn_context* ctx, const dcn_shape* shape,
                                  const void* d_input_nchw, void* d_cb8, void* stream);
dcn_status dcn_forward_f16_prepacked_cb8_dev(dcn_context* ctx, const dcn_shape* shape,
                                             const void* d_cb8, const void* d_offset,
                                             const void* d_mask, const dcn_packed* packed,
                                             void* d_output, void* stream);

/* ---- BF16 storage ------------------------------------------------------------- */
/* The fused sampler + MFMA GEMM over BF16 tensors (input, offsets, mask, weight, bias,
 * output as 16-bit BF16 bit patterns; FP32 accumulation). No counterpart in the
 * reference, which computes in FP16 and FP32 only: this is the BF16 form of the fused
 * FP16 GEMM that DCN's hot path asks for. The arithmetic is the FP16 exact sampler's
 * (the reference gather of MetalShader.swift:299-381 in FP32, each sample rounded once,
 * here to BF16), then bf16(acc + bias). Packed weights from dcn_prepack_bf16* only work
 * with these entry points, and FP16 ones only with the FP16 entry points (a mismatch
 * fails with DCN_INVALID_ARGUMENT). */
dcn_status dcn_prepack_bf16(dcn_context* ctx, const dcn_shape* shape,
                            const uint16_t* weight, size_t weight_count,
                            dcn_weight_layout layout,
                            const uint16_t* bias, size_t bias_count,
                            dcn_packed** out);
dcn_status dcn_prepack_bf16_dev(dcn_context* ctx, const dcn_shape* shape,
                                const void* d_weight, dcn_weight_layout layout,
                                const void* d_bias, void* stream, dcn_packed** out);
dcn_status dcn_forward_bf16_prepacked(dcn_context* ctx, const dcn_shape* shape,
                                      const uint16_t* input, size_t input_count,
                                      const uint16_t* offset, size_t offset_count,
                                      const uint16_t* mask, size_t mask_count,
                                      const dcn_packed* packed,
                                      uint16_t* output, size_t output_count);
dcn_status dcn_forward_bf16_prepacked_dev(dcn_context* ctx, const dcn_shape* shape,
                                          const void* d_input, const void* d_offset,
                                          const void* d_mask, const dcn_packed* packed,
                                          void* d_output, void* stream);
/* The same from an input already in the padded channel-block layout (BF16 bits in the
 * FP16 layout's places; dcn_pack_input_cb8_dev copies 16-bit words, so it makes it). */
dcn_status dcn_forward_bf16_prepacked_cb8_dev(dcn_context* ctx, const dcn_shape* shape,
                                              const void* d_cb8, const void* d_offset,
                                              const void* d_mask, const dcn_packed* packed,
                                              void* d_output, void* stream);

/* Allocation-free variant of dcn_forward_f16_prepacked_dev. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under hipGraph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The padded
 * channel-block copy of the input goes to a device array of DCN_NOALLOC_SCRATCH_BYTES
 * that the library holds on every device it runs on (resolved by dcn_create) instead
 * of the context's workspace; the call allocates nothing (no hipMalloc / hipFree).
 * A shape whose padded input (dcn_cb8_count * 2 bytes) exceeds the array fails with
 * DCN_INVALID_SHAPE. All calls on one device share that device's array, so the library
 * orders them: a call on another stream than the previous call's (any context, any host
 * thread) makes its stream wait, on the device, for the previous call's work
 * (hipStreamWaitEvent on an event created with the context; nothing is allocated), and
 * calls from several threads enqueue one at a time. Under hipGraph capture a call neither
 * waits nor records: captured calls that could overlap in time on one device race unless
 * the caller orders them. Each call writes every element it reads, so the array needs no
 * clearing between calls. */
#define DCN_NOALLOC_SCRATCH_BYTES (24u << 20)
dcn_status dcn_forward_f16_prepacked_noalloc_dev(dcn_context* ctx, const dcn_shape* shape,
                                                 const void* d_input, const void* d_offset,
                                                 const void* d_mask, const dcn_packed* packed,
                                                 void* d_output, void* stream);

/* Fused-kernel tuning. variant: 1 = register sampling (each lane gathers its MFMA A
 * fragment directly), 2 = LDS-staged im2col tile (a sampler phase fills the tile for
 * the whole K range, an MFMA phase consumes it), 3 = LDS input windows (3x3 kernels:
 * per offset group, the bounding box of a 2D pixel tile's samples is copied to LDS and
 * gathered from there; mt = tile rows, ks = waves = 32-pixel row blocks), 4 = variant 3
 * with the lower corner row of each sample read through the L1 cache instead of LDS,
 * 5 = narrow 16-pixel tiles on 16x16x32 MFMA, one workgroup per CU on small maps
 * (mt = 1, ks = waves splitting K: 8 or 12), 6 = variant 3 on 8 x 32 tiles whose next
 * stage's windows and weights stream into LDS by DMA during the current stage (mt = ks
 * = 8; an even offset-group count), 7 = tile windows: 4 waves on a 128-pixel tile, 8 x 16
 * (mt = 16) or 4 x 32 (mt = 32), two offset groups per stage split by tap across the
 * waves, each stage's offsets, masks and sample windows copied into LDS by DMA, global
 * gathers for a stage whose windows do not fit (3x3 kernels, 8 channels per group, an
 * even group count, Cout 32 or 64, input sides up to 32000; ks = 8: the tiles of an
 * XCD's band are placed on its CUs by estimated cost where some CUs run one tile and
 * others two (33-63 tiles per band), and where every CU runs two (64 tiles per band) a
 * heavy tile goes to the slot dispatched first; ks = 1: fixed placement; the outputs are
 * the same bits either way; the automatic choice for problems of more than 1024 tiles of 32
 * pixels, with either sampler). sampler: 0 = reference arithmetic
 * (FP32 bilinear in the reference's association, half(sampled*mask): the im2col
 * values of deform_conv2d_fp16_jasna_gather bit for bit), 1 = fast (mask folded into
 * the bilinear weights, packed-FP16 blend). mt = 32-pixel row blocks per tile (1, 2),
 * ks = waves per workgroup (register: 2, 4, 8; staged: 8, 16). 0 / -1 = automatic.
 * The setting applies to the FP16 prepacked forwards; the BF16 forwards choose their
 * kernel themselves (narrow up to 1024 tiles of 32 pixels, then windows where the shape
 * allows them, else register sampling).
 * No counterpart in the reference (its tile size is the compile-time
 * fusedGEMMRowsPerTile, MetalShader.swift:2). */
dcn_status dcn_set_fused_config(dcn_context* ctx, int variant, int mt, int ks, int sampler);
/* The configuration the next FP16 fused call on `shape` would use. ctx may be null: the
 * automatic choice without an override (no device is touched). */
dcn_status dcn_get_fused_config(dcn_context* ctx, const dcn_shape* shape, int* variant, int* mt,
                                int* ks, int* sampler);

/* Diagnostics: an empty kernel of the given launch shape (workgroups of `threads`
 * threads, `lds_bytes` of dynamic LDS each), enqueued on `stream`. Its duration is the
 * dispatch, wave-launch and completion floor that every kernel of that shape pays (the
 * fused kernels' times are read against it). No counterpart in the reference. */
dcn_status dcn_launch_floor_dev(dcn_context* ctx, int workgroups, int threads, int lds_bytes,
                                void* stream);
/* Diagnostics: per-workgroup clock stamps of the tile kernel (variant 7). While set, every
 * tile launch of this context writes, for workgroup b, d_clock[4b .. 4b+3] = {start, end
 * of wave 0, end of wave 1, HW_ID << 32 | (XCC_ID & 15) << 28 | tile} as uint64, start
 * and ends on the 100 MHz constant clock (s_memrealtime), the ends when the wave has
 * issued its output stores; HW_ID and XCC_ID are the hardware registers of that name
 * (bits 15:8 of HW_ID and XCC_ID together name the CU). Workgroups without a tile write nothing, so the caller clears the buffer.
 * `count` is in uint64 elements; a tile launch needs 4 x its workgroup count
 * (8 x ceil(tiles / 8)) and fails with DCN_INVALID_ARGUMENT when the buffer is smaller.
 * A null d_clock turns the stamps off. No counterpart in the reference. */
dcn_status dcn_set_tile_clock_dev(dcn_context* ctx, void* d_clock, size_t count);

/* Sampler alone: the modulated FP16 im2col matrix [B*Ho*Wo][Cin*Kh*Kw] with
 * column ic*Kh*Kw + k and value half(bilinear * mask), exactly
 * deform_conv2d_fp16_jasna_gather (MetalShader.swift:299-381) generalised to any
 * offset-group count. Used for sampler parity and phase timing; the fused path
 * never materialises it. */
dcn_status dcn_im2col_f16_dev(dcn_context* ctx, const dcn_shape* shape,
                              const void* d_input, const void* d_offset, const void* d_mask,
                              void* d_columns, void* stream);

/* Non-finite flag: *d_flag (uint32) is set to 1 if any of `count` FP16 values is
 * NaN or Inf; it is never cleared here (flag_non_finite_fp16,
 * MetalShader.swift:454-463). */
dcn_status dcn_flag_nonfinite_f16_dev(dcn_context* ctx, const void* d_values, size_t count,
                                      void* d_flag, void* stream);
/* Host wrapper: clears a flag, runs the check, synchronises; DCN_NONFINITE_OUTPUT if
 * set (FusedFourPassRecurrenceProbe.swift:714-743). */
dcn_status dcn_check_nonfinite_f16_dev(dcn_context* ctx, const void* d_values, size_t count,
                                       void* stream);

/* ---- deterministic inputs, checksum, statistics (host only) -------------------- */

/* SeededGenerator (DeformConv.swift:168-181): SplitMix64, seed 0 -> 0x9E3779B97F4A7C15. */
uint64_t dcn_splitmix64_seed(uint64_t seed);
uint64_t dcn_splitmix64_next(uint64_t* state);
/* SeededGenerator.floats(count:range:) (DeformConv.swift:183-185): Swift's
 * Float.random(in: lo...hi, using:) per element, in order. */
void dcn_seeded_floats(uint64_t* state, size_t count, float lo, float hi, float* out);

/* Benchmark configurations: 1 = FP32 1x128x64x64->64, 2 = same in FP16,
 * 3 = 16 tiles batched FP16, 5 = 1x128x180x320 FP16. (4, the propagation body,
 * has its own entry points.) */
dcn_status dcn_config_shape(int config, dcn_shape* out);
/* Fill FP32 arrays for `config` from `seed` (x ~ N(0,1); weight He-uniform bound
 * sqrt(6/fan_in); bias U(-0.1,0.1); offsets 10*tanh(N(0,s)) + smooth flow; mask
 * sigmoid(N(0,1)), with exact 0/1 sites for config 5). */
dcn_status dcn_generate_config_inputs(int config, uint64_t seed,
                                      float* input, size_t input_count,
                                      float* offset, size_t offset_count,
                                      float* mask, size_t mask_count,
                                      float* weight, size_t weight_count,
                                      float* bias, size_t bias_count);

/* IEEE binary16 round-to-nearest-even conversions (Swift Float16(Float)). */
uint16_t dcn_f32_to_f16(float value);
float dcn_f16_to_f32(uint16_t bits);
void dcn_f32_to_f16_array(const float* in, uint16_t* out, size_t count);
void dcn_f16_to_f32_array(const uint16_t* in, float* out, size_t count);

/* Benchmark checksum: sum in double of values at indices 0, 257, 514, ...
 * (MetalRunner.swift:332-337; JasnaCLI.swift:1413-1420 for raw .dcnfp16 bytes). */
double dcn_checksum_f32(const float* values, size_t count);
double dcn_checksum_f16(const uint16_t* values, size_t count);

/* BenchmarkStatistics (BenchmarkStatistics.swift:3-44): min, max, median, mean,
 * population stddev, P10, P90 by linear interpolation. Empty or non-finite
 * input -> DCN_INVALID_ARGUMENT (the Swift init returns nil). */
typedef struct dcn_statistics {
    double minimum;
    double maximum;
    double median;
    double mean;
    double standard_deviation;
    double percentile10;
    double percentile90;
    size_t count;
} dcn_statistics;
dcn_status dcn_compute_statistics(const double* samples, size_t count, dcn_statistics* out);

/* ---- propagation body (BasicVSR++ second-order propagation, one branch) ----------
 * The layers around the deformable convolution in one propagation step, FP16 storage:
 * temporal alignment inputs, the conv_offset branch, the offset/mask transform, the
 * DCN, the residual backbone and the alignment residual. Feature maps are one image,
 * 64 channels; flows are [2][H][W] planes ordered (x, y). */

/* Layout of a body tensor. NCHW: planar [C][H][W]. CB8: [ceil(C/8)][H+4][W+4][8], a
 * 2-pixel zero border and 8 channels per 16-byte vector (the layout the fused kernels
 * gather from). A CB8 buffer must be zero-filled once by its owner; writers only
 * touch interior positions of real channels. */
typedef enum dcn_tensor_layout {
    DCN_TENSOR_NCHW = 0,
    DCN_TENSOR_CB8 = 1
} dcn_tensor_layout;

/* Elements of a CB8 tensor of `channels` x height x width (uint16_t units). */
size_t dcn_cb8_tensor_count(int channels, int height, int width);

/* runDCNOffsetTransform (MetalRunner.swift:469-508), prepare_dcn_offsets_fp16
 * (MetalShader.swift:815-839): raw [432][plane] = [o1, o2, mask logits] and flows
 * flow1/flow2 [2][plane] -> offset [288][plane] = half(10*tanh(raw) + flow) with even
 * channels dy (flow y) and odd dx (flow x), flow1 for the first 144 channels and
 * flow2 for the rest; mask [144][plane] = half(sigmoid(raw[288 + c])). Count
 * mismatches give DCN_INVALID_SHAPE, as the reference's guard. */
dcn_status dcn_offset_transform_f16(dcn_context* ctx, size_t plane, const uint16_t* raw,
                                    size_t raw_count, const uint16_t* flow1, size_t flow1_count,
                                    const uint16_t* flow2, size_t flow2_count, uint16_t* offset,
                                    size_t offset_count, uint16_t* mask, size_t mask_count);
dcn_status dcn_offset_transform_f16_dev(dcn_context* ctx, size_t plane, const void* d_raw,
                                        const void* d_flow1, const void* d_flow2, void* d_offset,
                                        void* d_mask, void* stream);

/* runTemporalPreparation (MetalRunner.swift:510-582): accumulate_second_order_flow_fp16
 * + assemble_temporal_alignment_fp16 (MetalShader.swift:738-813).
 * flow2 [2][plane] = has_second_order ? half(flow1 + warp(prev_flow, flow1)) : 0;
 * conditions [196] = [warp(feat_prop, flow1), feat_current, warp(feat_n2, flow2), flow1,
 * flow2]; deform_input [128] = [feat_prop, feat_n2]. Inputs are NCHW: features 64
 * channels, flows 2. The host call returns NCHW outputs and checks counts like the
 * reference (DCN_INVALID_SHAPE). */
dcn_status dcn_temporal_prepare_f16(dcn_context* ctx, int width, int height,
                                    const uint16_t* feat_prop, size_t feat_prop_count,
                                    const uint16_t* feat_current, size_t feat_current_count,
                                    const uint16_t* feat_n2, size_t feat_n2_count,
                                    const uint16_t* flow1, size_t flow1_count,
                                    const uint16_t* prev_flow, size_t prev_flow_count,
                                    int has_second_order, uint16_t* conditions,
                                    size_t conditions_count, uint16_t* deform_input,
                                    size_t deform_input_count, uint16_t* flow2, size_t flow2_count);
dcn_status dcn_temporal_prepare_f16_dev(dcn_context* ctx, int width, int height,
                                        const void* d_feat_prop, const void* d_feat_current,
                                        const void* d_feat_n2, const void* d_flow1,
                                        const void* d_prev_flow, int has_second_order,
                                        void* d_flow2, void* d_conditions,
                                        dcn_tensor_layout conditions_layout, void* d_deform_input,
                                        dcn_tensor_layout deform_input_layout, void* stream);

/* assemble_temporal_backbone_fp16 / assemble_propagation_backbone_fp16
 * (MetalShader.swift:841-855, 899-929): concatenate `count` (1..5) 64-channel NCHW
 * sources into out (64 * count channels) in the given layout. */
dcn_status dcn_assemble_backbone_f16_dev(dcn_context* ctx, int width, int height,
                                         const void* const* d_sources, int count, void* d_out,
                                         dcn_tensor_layout layout, void* stream);

/* add_propagation_residual_fp16 (MetalShader.swift:857-867): out = half(aligned + backbone). */
dcn_status dcn_add_residual_f16_dev(dcn_context* ctx, size_t count, const void* d_aligned,
                                    const void* d_backbone, void* d_out, void* stream);

/* CB8 -> NCHW copy of one image of `channels` channels. */
dcn_status dcn_cb8_to_nchw_f16_dev(dcn_context* ctx, int channels, int height, int width,
                                   const void* d_cb8, void* d_out, void* stream);

/* 3x3 convolution, stride 1, pad 1, of the body's conv_offset branch and backbone
 * (the conv modules exported by tools/convert_basicvsrpp.py:181-197): weights OIHW
 * FP16 [cout][cin][3][3], packed once into MFMA fragments. */
typedef struct dcn_conv dcn_conv;
dcn_status dcn_conv3x3_create_dev(dcn_context* ctx, int cin, int cout, int height, int width,
                                  const void* d_weight, const void* d_bias, void* stream,
                                  dcn_conv** out);
void dcn_conv3x3_free(dcn_conv* conv);
/* out = half(r2 + half(r1 + act(conv(x) + bias))), each residual optional (null).
 * activation: 0 none, 1 LeakyReLU(slope), 2 ReLU. x is CB8 (cin channels); out and the
 * residuals (cout channels) in the layouts given. */
dcn_status dcn_conv3x3_f16_dev(dcn_context* ctx, const dcn_conv* conv, const void* d_x_cb8,
                               int activation, float slope, const void* d_res1,
                               dcn_tensor_layout res1_layout, const void* d_res2,
                               dcn_tensor_layout res2_layout, void* d_out,
                               dcn_tensor_layout out_layout, void* stream);

/* The last conv_offset layer (cin -> 432) fused with prepare_dcn_offsets_fp16
 * (MetalShader.swift:815-839; runDCNOffsetTransform, MetalRunner.swift:469-508): raw =
 * half(conv(x) + b), offset [288][plane] = half(10 tanh(raw) + flow), mask [144][plane] =
 * half(sigmoid(raw)); flows [2][plane] (x, y), flow1 for the first 144 offset channels and
 * flow2 for the rest. Equals dcn_conv3x3_f16_dev (NCHW) followed by
 * dcn_offset_transform_f16_dev bit for bit. DCN_INVALID_SHAPE unless cout is 432. */
dcn_status dcn_conv3x3_offsets_f16_dev(dcn_context* ctx, const dcn_conv* conv, const void* d_x_cb8,
                                       const void* d_flow1, const void* d_flow2, void* d_offset,
                                       void* d_mask, void* stream);

/* Two chained 64 -> 64 convs of one plane in one launch: t = half(act1(conv1(x) + b1)),
 * out = half(r2 + half(r1 + act2(conv2(t) + b2))). The residual block of the backbone
 * (conv-ReLU-conv + skip) and two LeakyReLU layers of conv_offset
 * (tools/convert_basicvsrpp.py:181-197); t never leaves the chip, and the result equals
 * two dcn_conv3x3_f16_dev calls bit for bit. DCN_INVALID_SHAPE unless both convs are
 * 64 -> 64 over the same plane. */
dcn_status dcn_conv3x3_pair_f16_dev(dcn_context* ctx, const dcn_conv* conv1, const dcn_conv* conv2,
                                    const void* d_x_cb8, int activation1, int activation2, float slope,
                                    const void* d_res1, dcn_tensor_layout res1_layout,
                                    const void* d_res2, dcn_tensor_layout res2_layout, void* d_out,
                                    dcn_tensor_layout out_layout, void* stream);

/* ---- SPyNet flow estimation: the producer of the first-order flows ---- */

/* jasna_bicubic_downsample_quarter_fp16 (MetalShader.swift:488-521): out [c][h/4][w/4] =
 * torch interpolate(scale_factor=0.25, mode="bicubic", a = -0.75) of in [c][h][w], FP32
 * sums in the reference's order, one FP16 rounding. h and w multiples of 4 (the 256 x 256
 * LQ tile -> the 64 x 64 SPyNet input). */
dcn_status dcn_bicubic_quarter_f16_dev(dcn_context* ctx, int channels, int height, int width,
                                       const void* d_in, void* d_out, void* stream);

/* SPyNet: six levels (h/32 .. h), each [reference, support warped by the upsampled flow
 * (border padding), flow] -> 7x7 convs 8->32->64->32->16->2 (ReLU between) -> flow +=
 * residual (spynet_build_pyramid_pair_fp16, spynet_prepare_fp16, spynet_add_flow_fp16,
 * MetalShader.swift:523-649; level order of tools/convert_basicvsrpp.py:82-100; the
 * bidirectional pair of verifySPyNetPair, SPyNetPairProbe.swift:47-449). Weights OIHW
 * FP16 device pointers, level 0 = the coarsest; packed at creation. */
#define DCN_SPYNET_LEVELS 6
#define DCN_SPYNET_LAYERS 5
typedef struct dcn_spynet_weights {
    const void* weight[DCN_SPYNET_LEVELS][DCN_SPYNET_LAYERS];
    const void* bias[DCN_SPYNET_LEVELS][DCN_SPYNET_LAYERS];
} dcn_spynet_weights;
typedef struct dcn_spynet dcn_spynet;
/* height and width multiples of 32 (the reference's 64 x 64); max_frames (>= 2) sizes the
 * clip entry point (2 for pairs only). */
dcn_status dcn_spynet_create(dcn_context* ctx, int height, int width, int max_frames,
                             const dcn_spynet_weights* weights, void* stream, dcn_spynet** out);
void dcn_spynet_destroy(dcn_spynet* spynet);
/* spynet_build_pyramid_pair_fp16 (MetalShader.swift:523-570) for one RGB frame [3][h][w]:
 * out = the DCN_SPYNET_LEVELS normalised levels [3][h >> (5 - l)][w >> (5 - l)],
 * coarsest first, one after the other (the pyramid dcn_spynet_flow_dev builds inside). */
dcn_status dcn_spynet_pyramid_f16_dev(dcn_context* ctx, int height, int width, const void* d_frame,
                                      void* d_out, void* stream);
/* reference, support: RGB [3][h][w] FP16 in [0, 1]. d_flow [1 + both][2][h][w] (x, y):
 * image 0 = spynet(reference, support), image 1 (both_directions) = spynet(support,
 * reference). Stream-ordered, no allocation, no memset: graph-capturable. */
dcn_status dcn_spynet_flow_dev(dcn_spynet* spynet, const void* d_reference, const void* d_support,
                               int both_directions, void* d_flow, void* stream);
/* All flows of a clip in one pass (FusedSPyNetClipGraph.swift:29-315, compute_flow):
 * d_frames [frames][3][h][w] (the 64 x 64 copies), d_flows [2][frames - 1][2][h][w]:
 * [0][t] = spynet(frame t, frame t + 1) (the backward flows), [1][t] = spynet(frame t + 1,
 * frame t) (the forward flows), as dcn_clip_run_dev takes them. Every level runs once over
 * the batch of 2 (frames - 1) images. frames <= max_frames. */
dcn_status dcn_spynet_clip_flows_dev(dcn_spynet* spynet, const void* d_frames, int frames, void* d_flows,
                                     void* stream);

/* One propagation body: conv_offset (196->64->64->64->432, LeakyReLU 0.1 between), the
 * offset transform, the 128->64 DCN (16 deformable groups, 3x3), the backbone
 * ([feat_current, extra prefix features..., aligned] -> 64 conv + LeakyReLU 0.1, then
 * `blocks` residual blocks conv-ReLU-conv + skip) and feat_prop = aligned + backbone.
 * Replaces the per-step body of verifyFusedFourPassRecurrence
 * (FusedFourPassRecurrenceProbe.swift:570-664) for one branch; prefix features = branch
 * index (0: [spatial], 3: [spatial, b1, f1, b2], MetalShader.swift:899-929). All weights
 * OIHW FP16 device pointers; the body packs them at creation and owns its
 * intermediates, so a step allocates nothing. */
#define DCN_BODY_MAX_BLOCKS 8
typedef struct dcn_body_weights {
    const void* offset_weight[4];
    const void* offset_bias[4];
    const void* dcn_weight;
    const void* dcn_bias;
    const void* backbone_weight[1 + 2 * DCN_BODY_MAX_BLOCKS];
    const void* backbone_bias[1 + 2 * DCN_BODY_MAX_BLOCKS];
} dcn_body_weights;
typedef struct dcn_body dcn_body;
dcn_status dcn_body_create(dcn_context* ctx, int height, int width, int branch, int blocks,
                           const dcn_body_weights* weights, void* stream, dcn_body** out);
/* dcn_body_create for `tiles` independent tiles per step (1..1024; the production
 * pipeline runs many tiles of a frame, README.md:589-591): every tensor of a step then
 * holds all tiles, [tiles][C][H][W], and each kernel runs once over the batch. */
dcn_status dcn_body_create_tiles(dcn_context* ctx, int height, int width, int branch, int blocks, int tiles,
                                 const dcn_body_weights* weights, void* stream, dcn_body** out);
void dcn_body_destroy(dcn_body* body);
/* One step, stream-ordered. feat_current, feat_prop, feat_n2, feat_prop_out: NCHW
 * [64][H][W]; flow1, prev_flow, flow2_out: [2][H][W]; d_prefix: `branch` further
 * 64-channel NCHW backbone inputs (null when branch is 0). */
dcn_status dcn_body_step_dev(dcn_body* body, const void* d_feat_current, const void* d_flow1,
                             const void* d_prev_flow, const void* d_feat_prop,
                             const void* d_feat_n2, const void* const* d_prefix,
                             int has_second_order, void* d_flow2_out, void* d_feat_prop_out,
                             void* stream);
/* The same step captured into an executable hipGraph (the retained per-step graph of
 * FusedFourPassRecurrenceProbe.swift:904-937); replay with dcn_graph_launch. */
typedef struct dcn_graph dcn_graph;
dcn_status dcn_body_capture(dcn_body* body, const void* d_feat_current, const void* d_flow1,
                            const void* d_prev_flow, const void* d_feat_prop,
                            const void* d_feat_n2, const void* const* d_prefix,
                            int has_second_order, void* d_flow2_out, void* d_feat_prop_out,
                            dcn_graph** out);
dcn_status dcn_graph_launch(dcn_graph* graph, void* stream);
void dcn_graph_destroy(dcn_graph* graph);

/* The first step of a branch (position 0 of its traversal): no alignment, so the
 * backbone input is [feat_current, prefix..., 0] and feat_prop_out = half(0 + backbone)
 * (initialAssemblyArguments / initialResidualArguments,
 * FusedFourPassRecurrenceProbe.swift:300-318, encoded at :528-566). */
dcn_status dcn_body_initial_step_dev(dcn_body* body, const void* d_feat_current,
                                     const void* const* d_prefix, void* d_feat_prop_out,
                                     void* stream);

/* The same step and first step with the warped features in CB8, for a recurrence that
 * keeps its propagated features in both layouts (the clip does): feat_prop and feat_n2
 * are 64-channel CB8 tensors ([8][H+4][W+4][8], zero border) and feat_prop_out_cb8
 * receives a CB8 copy of the output beside the NCHW feat_prop_out. The warps then gather
 * 8 channels per 16-byte load. Same bits as the NCHW entry points; single-tile bodies
 * only (DCN_INVALID_SHAPE otherwise). No counterpart in the reference (its Metal buffers
 * have one layout). */
dcn_status dcn_body_step_cb8_dev(dcn_body* body, const void* d_feat_current, const void* d_flow1,
                                 const void* d_prev_flow, const void* d_feat_prop_cb8,
                                 const void* d_feat_n2_cb8, const void* const* d_prefix,
                                 int has_second_order, void* d_flow2_out, void* d_feat_prop_out,
                                 void* d_feat_prop_out_cb8, void* stream);
dcn_status dcn_body_initial_step_cb8_dev(dcn_body* body, const void* d_feat_current,
                                         const void* const* d_prefix, void* d_feat_prop_out,
                                         void* d_feat_prop_out_cb8, void* stream);
dcn_status dcn_body_capture_cb8(dcn_body* body, const void* d_feat_current, const void* d_flow1,
                                const void* d_prev_flow, const void* d_feat_prop_cb8,
                                const void* d_feat_n2_cb8, const void* const* d_prefix,
                                int has_second_order, void* d_flow2_out, void* d_feat_prop_out,
                                void* d_feat_prop_out_cb8, dcn_graph** out);

/* ---- temporal schedule and the four-branch clip ------------------------------------
 * TemporalSchedule (TemporalSchedule.swift:27-68): branches backward_1, forward_1,
 * backward_2, forward_2 (branch index 0..3, backbone inputs (2 + index) * 64 channels)
 * each walk the frames backward (T-1 .. 0) or forward (0 .. T-1). -1 stands for the
 * reference's nil. */
typedef struct dcn_schedule_step {
    int branch;              /* 0..3 */
    int position;            /* index within the branch's traversal */
    int frame;
    int flow_index;          /* backward: frame, forward: frame - 1; -1 at position 0 */
    int second_order_frame;  /* traversal[position - 2]; -1 below position 2 */
} dcn_schedule_step;
/* The 4 * frame_count steps, branch-major, into steps[0 .. capacity); *count receives
 * 4 * frame_count. DCN_INVALID_SHAPE for frame_count <= 0, DCN_INVALID_ARGUMENT when
 * capacity is too small. */
dcn_status dcn_temporal_schedule(int frame_count, dcn_schedule_step* steps, size_t capacity,
                                 size_t* count);
/* TemporalSchedule.persistentTensorBytes: FP16 LQ frames 3x256x256, five 64x64x64
 * feature sets per frame and both directions' flows 2x64x64. */
size_t dcn_schedule_persistent_bytes(int frame_count);
/* SideBySideRestoration.temporalChunkRanges (SideBySideRestoration.swift:1213-1230):
 * frame_count frames cut into max(1, min(ceil(T / n), T / 3)) balanced chunks, the
 * first T % chunks one frame longer. starts/sizes receive *count ranges.
 * DCN_INVALID_SHAPE unless frame_count >= 3 and max_frames_per_chunk >= 3. */
dcn_status dcn_temporal_chunk_ranges(int frame_count, int max_frames_per_chunk, int* starts,
                                     int* sizes, size_t capacity, size_t* count);

/* A four-branch propagation clip: one body per branch (weights[0..3] = backward_1,
 * forward_1, backward_2, forward_2), frames x height x width, owning its scratch
 * (second-order flow, a zero feature). */
typedef struct dcn_clip dcn_clip;
dcn_status dcn_clip_create(dcn_context* ctx, int height, int width, int frames, int blocks,
                           const dcn_body_weights* weights, void* stream, dcn_clip** out);
/* dcn_clip_create for `tiles` tiles: spatial [T][tiles][64][H][W], flows
 * [T-1][tiles][2][H][W], propagated [4][T][tiles][64][H][W]. */
dcn_status dcn_clip_create_tiles(dcn_context* ctx, int height, int width, int frames, int blocks, int tiles,
                                 const dcn_body_weights* weights, void* stream, dcn_clip** out);
void dcn_clip_destroy(dcn_clip* clip);
/* The whole clip in schedule order, stream-ordered: spatial [frames][64][H][W];
 * backward_flows / forward_flows [frames-1][2][H][W] indexed by the schedule's
 * flow_index; propagated [4][frames][64][H][W] receives every branch's feat_prop (the
 * propagationBuffers of FusedFourPassRecurrenceProbe.swift:221-225), which later
 * branches read as their prefix features. max_frames_per_chunk = 0 runs one
 * recurrence over the clip; n >= 3 runs each range of dcn_temporal_chunk_ranges as an
 * independent clip (restoreTileFrames, SideBySideRestoration.swift:1174-1211). */
dcn_status dcn_clip_run_dev(dcn_clip* clip, const void* d_spatial, const void* d_backward_flows,
                            const void* d_forward_flows, void* d_propagated,
                            int max_frames_per_chunk, void* stream);
/* The same clip captured into one executable hipGraph (the retained whole-clip command
 * buffer of FusedFourPassRecurrenceProbe.swift:904-937). */
dcn_status dcn_clip_capture(dcn_clip* clip, const void* d_spatial, const void* d_backward_flows,
                            const void* d_forward_flows, void* d_propagated,
                            int max_frames_per_chunk, dcn_graph** out);

/* The recoverable-error ladder of restoreTileWithFallback
 * (SideBySideRestoration.swift:1065-1136, restoreTileFramesIndependently :1140-1172) over
 * dcn_clip_run_dev. A rung fails recoverably when its output holds a NaN or Inf
 * (DCN_NONFINITE_OUTPUT); any other error is returned at once. The rungs:
 *   1. the whole clip (*recovered_with = 0);
 *   2. recurrence chunks of at most 10, 5, 3 frames, those shorter than the clip
 *      (*recovered_with = the chunk size);
 *   3. independent zero-motion triplets: each frame t runs alone as the clip [t, t, t]
 *      with zero flows and every branch keeps the middle frame's feat_prop
 *      (*recovered_with = DCN_CLIP_RECOVERED_TRIPLETS);
 *   4. if every spatial feature is finite, passthrough: every branch's feat_prop of
 *      frame t is frame t's spatial feature, unchanged
 *      (*recovered_with = DCN_CLIP_RECOVERED_PASSTHROUGH); otherwise DCN_COMMAND_FAILED.
 * Host-synchronous (each rung's check waits for the stream). report, when not null,
 * receives the reference's progress messages. */
#define DCN_CLIP_RECOVERED_TRIPLETS (-1)
#define DCN_CLIP_RECOVERED_PASSTHROUGH (-2)
typedef void (*dcn_report_fn)(const char* message, void* user);
dcn_status dcn_clip_run_with_fallback_dev(dcn_clip* clip, const void* d_spatial, const void* d_backward_flows,
                                          const void* d_forward_flows, void* d_propagated, void* stream,
                                          dcn_report_fn report, void* report_user, int* recovered_with);

#ifdef __cplusplus
}
#endif

#endif /* DCN_DCN_H */
