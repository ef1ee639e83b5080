// Self-test of the Swift binding: the reference's FP32 correctness case
// (correctnessTest, JasnaCLI.swift:68-110: SeededGenerator(0xC0FFEE), 1x2x5x5 -> 3) through
// HIPDeformConv, then benchmarkJasnaShape's inputs (seed 0x4A41534E41) at the C2 shape
// through the FP16 prepacked path against the FP16 direct baseline (the benchmark's 2e-3
// gate on the SIMD-group GEMM, MetalRunner.swift:338-354).
// Prints one line per check; exits 1 on a failed check.
import Foundation
import HIPDeformConv

func floats(_ count: Int, _ lo: Float, _ hi: Float, _ gen: inout SplitMix64Generator) -> [Float] {
    (0..<count).map { _ in Float.random(in: lo...hi, using: &gen) }
}

func shape(_ b: Int, _ cin: Int, _ h: Int, _ w: Int, _ cout: Int, _ og: Int) -> DeformConvShape {
    DeformConvShape(batch: b, inputChannels: cin, inputHeight: h, inputWidth: w, outputChannels: cout,
                    outputHeight: h, outputWidth: w, kernelHeight: 3, kernelWidth: 3, padHeight: 1, padWidth: 1,
                    strideHeight: 1, strideWidth: 1, dilationHeight: 1, dilationWidth: 1, groups: 1,
                    offsetGroups: og)
}

var failed = false
do {
    let dcn = try HIPDeformConv()
    var gen = SplitMix64Generator(seed: 0xC0FFEE)
    let s = shape(1, 2, 5, 5, 3, 1)
    let input = floats(s.inputCount, -1, 1, &gen), offset = floats(s.offsetCount, -0.4, 0.4, &gen)
    let mask = floats(s.maskCount, 0.1, 0.9, &gen), weight = floats(s.weightCount, -0.2, 0.2, &gen)
    let bias = floats(s.outputChannels, -0.1, 0.1, &gen)
    let out = try dcn.runFloat32(shape: s, input: input, offset: offset, mask: mask, weight: weight, bias: bias)
    let finite = out.allSatisfy { $0.isFinite }
    print("fp32 self-test: first inputs \(input.prefix(3)), output[0...2] \(out.prefix(3)), finite \(finite)")
    failed = failed || !finite

    var g2 = SplitMix64Generator(seed: 0x4A41534E41)
    let c2 = shape(1, 128, 64, 64, 64, 16)
    let h = { (n: Int, lo: Float, hi: Float) in floats(n, lo, hi, &g2).map { Float16($0) } }
    let i16 = h(c2.inputCount, -1, 1), o16 = h(c2.offsetCount, -0.25, 0.25), m16 = h(c2.maskCount, 0.25, 0.75)
    let w16 = h(c2.weightCount, -0.02, 0.02), b16 = h(c2.outputChannels, -0.02, 0.02)
    let packed = try dcn.prepack(shape: c2, weight: w16, bias: b16)
    let fused = try dcn.runFloat16Prepacked(shape: c2, input: i16, offset: o16, mask: m16, packed: packed)
    let baseline = try dcn.runFloat16(shape: c2, input: i16, offset: o16, mask: m16, weight: w16, bias: b16)
    let maxErr = zip(fused, baseline).map { abs(Float($0) - Float($1)) }.max() ?? .infinity
    print("fp16 prepacked vs fp16 direct at 1x128x64x64 -> 64: max abs difference \(maxErr) (gate 2e-3)")
    failed = failed || !(maxErr <= 2e-3)
} catch {
    print("error: \(error)")
    failed = true
}
if failed { exit(1) }
