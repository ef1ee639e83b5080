// HIPDeformConv: MetalDeformConv's host surface (MetalRunner.swift:92-185) over the libdcn
// C ABI (include/dcn/dcn.h), throwing the reference's DeformConvError
// (DeformConv.swift:44-73). Value-semantics arrays in and out on the host-pointer calls;
// raw device pointers and a hipStream_t (as UnsafeMutableRawPointer) on the stream-ordered
// ones. One thread at a time per instance, as MetalDeformConv.
import CDCN

/// Prepacked FP16 weights (dcn_packed), freed with the handle.
public final class PackedWeights {
    let handle: OpaquePointer
    init(_ handle: OpaquePointer) { self.handle = handle }
    deinit { dcn_packed_free(handle) }
}

public final class HIPDeformConv {
    private var ctx: OpaquePointer?

    /// MetalDeformConv.init (MetalRunner.swift:107): fails with metalUnavailable when no
    /// device exists, shaderResourceMissing when the kernels do not load.
    public init(device: Int32 = 0) throws {
        var c: OpaquePointer?
        let status = dcn_create(&c, device)
        ctx = c
        try check(status)
    }

    deinit { dcn_destroy(ctx) }

    func check(_ status: dcn_status) throws {
        let detail = ctx.map { String(cString: dcn_last_error($0)) } ?? ""
        switch status {
        case DCN_OK: return
        case DCN_INVALID_SHAPE: throw DeformConvError.invalidShape
        case DCN_INVALID_ARRAY_COUNT:
            // "<name> has <actual> elements; expected <expected>"
            let parts = detail.split(separator: " ")
            guard parts.count == 6, let actual = Int(parts[2]), let expected = Int(parts[5]) else {
                throw DeformConvError.commandFailed(detail)
            }
            throw DeformConvError.invalidArrayCount(name: String(parts[0]), expected: expected, actual: actual)
        case DCN_DEVICE_UNAVAILABLE: throw DeformConvError.metalUnavailable
        case DCN_KERNEL_MISSING: throw DeformConvError.shaderResourceMissing
        case DCN_NONFINITE_OUTPUT: throw DeformConvError.nonFiniteOutput(detail)
        default: throw DeformConvError.commandFailed(detail)
        }
    }

    static func cShape(_ s: DeformConvShape) -> dcn_shape {
        dcn_shape(batch: Int32(s.batch), input_channels: Int32(s.inputChannels),
                  input_height: Int32(s.inputHeight), input_width: Int32(s.inputWidth),
                  output_channels: Int32(s.outputChannels), output_height: Int32(s.outputHeight),
                  output_width: Int32(s.outputWidth), kernel_height: Int32(s.kernelHeight),
                  kernel_width: Int32(s.kernelWidth), pad_height: Int32(s.padHeight),
                  pad_width: Int32(s.padWidth), stride_height: Int32(s.strideHeight),
                  stride_width: Int32(s.strideWidth), dilation_height: Int32(s.dilationHeight),
                  dilation_width: Int32(s.dilationWidth), groups: Int32(s.groups),
                  offset_groups: Int32(s.offsetGroups))
    }

    static func bits(_ values: [Float16]) -> [UInt16] { values.map { $0.bitPattern } }
    static func halves(_ values: [UInt16]) -> [Float16] { values.map { Float16(bitPattern: $0) } }

    /// runFloat32 (MetalRunner.swift:159-185): bit-identical to DeformConvCPU.run.
    public func runFloat32(shape: DeformConvShape, input: [Float], offset: [Float], mask: [Float],
                           weight: [Float], bias: [Float]) throws -> [Float] {
        var s = Self.cShape(shape)
        var out = [Float](repeating: 0, count: shape.outputCount)
        try check(dcn_forward_f32(ctx, &s, input, input.count, offset, offset.count, mask, mask.count,
                                  weight, weight.count, bias, bias.count, &out, out.count))
        return out
    }

    /// FP16 storage, FP32 accumulation in the oracle's order (deform_conv2d_fp16,
    /// MetalShader.swift:126-174).
    public func runFloat16(shape: DeformConvShape, input: [Float16], offset: [Float16], mask: [Float16],
                           weight: [Float16], bias: [Float16]) throws -> [Float16] {
        var s = Self.cShape(shape)
        let i = Self.bits(input), o = Self.bits(offset), m = Self.bits(mask)
        let w = Self.bits(weight), b = Self.bits(bias)
        var out = [UInt16](repeating: 0, count: shape.outputCount)
        try check(dcn_forward_f16(ctx, &s, i, i.count, o, o.count, m, m.count, w, w.count, b, b.count,
                                  &out, out.count))
        return Self.halves(out)
    }

    /// One-time weight prepack (OIHW or the .dcnfp16 [ic][k][oc] order).
    public func prepack(shape: DeformConvShape, weight: [Float16], bias: [Float16],
                        icKOc: Bool = false) throws -> PackedWeights {
        var s = Self.cShape(shape)
        let w = Self.bits(weight), b = Self.bits(bias)
        var packed: OpaquePointer?
        try check(dcn_prepack_f16(ctx, &s, w, w.count, icKOc ? DCN_LAYOUT_IC_K_OC : DCN_LAYOUT_OIHW,
                                  b, b.count, &packed))
        guard let handle = packed else { throw DeformConvError.commandFailed("prepack returned no handle") }
        return PackedWeights(handle)
    }

    /// DeformConvWeightSet (DeformConvWeights.swift:4-36): a 147,584-byte .dcnfp16 file.
    public func loadWeightSet(path: String) throws -> PackedWeights {
        var packed: OpaquePointer?
        try check(dcn_load_dcnfp16(ctx, path, &packed))
        guard let handle = packed else { throw DeformConvError.commandFailed("load returned no handle") }
        return PackedWeights(handle)
    }

    /// The fused sampler + MFMA path (executeJasnaSIMDGroupGEMM, MetalRunner.swift:696-761).
    public func runFloat16Prepacked(shape: DeformConvShape, input: [Float16], offset: [Float16],
                                    mask: [Float16], packed: PackedWeights) throws -> [Float16] {
        var s = Self.cShape(shape)
        let i = Self.bits(input), o = Self.bits(offset), m = Self.bits(mask)
        var out = [UInt16](repeating: 0, count: shape.outputCount)
        try check(dcn_forward_f16_prepacked(ctx, &s, i, i.count, o, o.count, m, m.count, packed.handle,
                                            &out, out.count))
        return Self.halves(out)
    }

    /// Stream-ordered, device-resident form (hipGraph capturable): FP16 NCHW buffers.
    public func forwardFloat16Prepacked(shape: DeformConvShape, input: UnsafeRawPointer,
                                        offset: UnsafeRawPointer, mask: UnsafeRawPointer,
                                        packed: PackedWeights, output: UnsafeMutableRawPointer,
                                        stream: UnsafeMutableRawPointer? = nil) throws {
        var s = Self.cShape(shape)
        try check(dcn_forward_f16_prepacked_dev(ctx, &s, input, offset, mask, packed.handle, output, stream))
    }

    /// restoreTileWithFallback's ladder (SideBySideRestoration.swift:1065-1172) over a
    /// four-branch clip (a dcn_clip*): returns 0 (whole clip), the chunk size,
    /// DCN_CLIP_RECOVERED_TRIPLETS or DCN_CLIP_RECOVERED_PASSTHROUGH.
    public func runClipWithFallback(clip: OpaquePointer, spatial: UnsafeRawPointer,
                                    backwardFlows: UnsafeRawPointer?, forwardFlows: UnsafeRawPointer?,
                                    propagated: UnsafeMutableRawPointer, stream: UnsafeMutableRawPointer? = nil,
                                    report: @escaping (String) -> Void) throws -> Int32 {
        final class Reporter {
            let send: (String) -> Void
            init(_ send: @escaping (String) -> Void) { self.send = send }
        }
        let box = Unmanaged.passRetained(Reporter(report))
        defer { box.release() }
        var recovered: Int32 = 0
        let status = dcn_clip_run_with_fallback_dev(
            clip, spatial, backwardFlows, forwardFlows, propagated, stream,
            { message, user in
                guard let message = message, let user = user else { return }
                Unmanaged<Reporter>.fromOpaque(user).takeUnretainedValue().send(String(cString: message))
            },
            box.toOpaque(), &recovered)
        try check(status)
        return recovered
    }
}

/// SeededGenerator (DeformConv.swift:168-181) over libdcn's SplitMix64, so
/// Float.random(in:using:) draws the reference's benchmark and test inputs.
public struct SplitMix64Generator: RandomNumberGenerator {
    var state: UInt64
    public init(seed: UInt64) { state = dcn_splitmix64_seed(seed) }
    public mutating func next() -> UInt64 { dcn_splitmix64_next(&state) }
}
