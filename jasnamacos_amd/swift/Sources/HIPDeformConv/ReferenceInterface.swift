// The reference's shape and error types (DeformConv.swift:3-73), restated with the same
// member names so HIPDeformConv.swift builds on its own in this package. Inside the
// reference package its own definitions are used and this file is left out.

public struct DeformConvShape: Sendable {
    public let batch, inputChannels, inputHeight, inputWidth: Int
    public let outputChannels, outputHeight, outputWidth: Int
    public let kernelHeight, kernelWidth, padHeight, padWidth: Int
    public let strideHeight, strideWidth, dilationHeight, dilationWidth: Int
    public let groups, offsetGroups: Int

    public init(batch: Int, inputChannels: Int, inputHeight: Int, inputWidth: Int, outputChannels: Int,
                outputHeight: Int, outputWidth: Int, kernelHeight: Int, kernelWidth: Int, padHeight: Int,
                padWidth: Int, strideHeight: Int, strideWidth: Int, dilationHeight: Int, dilationWidth: Int,
                groups: Int, offsetGroups: Int) {
        self.batch = batch; self.inputChannels = inputChannels
        self.inputHeight = inputHeight; self.inputWidth = inputWidth
        self.outputChannels = outputChannels; self.outputHeight = outputHeight; self.outputWidth = outputWidth
        self.kernelHeight = kernelHeight; self.kernelWidth = kernelWidth
        self.padHeight = padHeight; self.padWidth = padWidth
        self.strideHeight = strideHeight; self.strideWidth = strideWidth
        self.dilationHeight = dilationHeight; self.dilationWidth = dilationWidth
        self.groups = groups; self.offsetGroups = offsetGroups
    }

    public var kernelArea: Int { kernelHeight * kernelWidth }
    public var inputCount: Int { batch * inputChannels * inputHeight * inputWidth }
    public var outputCount: Int { batch * outputChannels * outputHeight * outputWidth }
    public var offsetCount: Int { batch * 2 * offsetGroups * kernelArea * outputHeight * outputWidth }
    public var maskCount: Int { batch * offsetGroups * kernelArea * outputHeight * outputWidth }
    public var weightCount: Int { outputChannels * (inputChannels / groups) * kernelArea }
}

public enum DeformConvError: Error, CustomStringConvertible {
    case invalidShape
    case invalidArrayCount(name: String, expected: Int, actual: Int)
    case metalUnavailable         // no HIP device
    case shaderResourceMissing    // no kernels for the device
    case nonFiniteOutput(String)
    case commandFailed(String)

    /// Only a non-finite output is retried by the recovery ladder.
    public var isRecoverableNumericalFailure: Bool {
        if case .nonFiniteOutput = self { return true }
        return false
    }

    public var description: String {
        switch self {
        case .invalidShape: return "Invalid deformable-convolution shape"
        case let .invalidArrayCount(name, expected, actual): return "\(name) has \(actual) elements; expected \(expected)"
        case .metalUnavailable: return "No HIP device is available"
        case .shaderResourceMissing: return "The DCN kernels are missing for this device"
        case let .nonFiniteOutput(message): return "Model produced non-finite output: \(message)"
        case let .commandFailed(message): return "HIP command failed: \(message)"
        }
    }
}
