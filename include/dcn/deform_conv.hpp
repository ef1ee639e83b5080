// C++ host layer over libdcn (dcn.h): the reference's Swift operator surface for the
// deformable convolution, restated in C++17 — the same type and method names, argument
// meaning and error behaviour, so a C++ host (or tests) reads like the Swift original.
//
//   DeformConvShape        DeformConv.swift:3-42
//   DeformConvError        DeformConv.swift:44-73
//   SeededGenerator        DeformConv.swift:168-186
//   HipDeformConv          MetalDeformConv (MetalRunner.swift:92-388): runFloat32,
//                          runFloat16, prepacked weights, benchmarkJasnaShape
//   DeformConvWeightSet    DeformConvWeights.swift:4-46
//   BenchmarkStatistics    BenchmarkStatistics.swift:3-44
//   TemporalSchedule       TemporalSchedule.swift:3-101
//   temporalChunkRanges    SideBySideRestoration.swift:1213-1230
//   SPyNetPairResult,      SPyNetPairProbe.swift:4-18, :47-449
//   verifySPyNetPair       (the deterministic inputs of tools/export_spynet_oracle.py:14-19)
//
// Link with -ldcn (and the HIP runtime for benchmarkJasnaShape's device buffers).
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "dcn/dcn.h"

namespace jasna {

class DeformConvError : public std::exception {
public:
    // DeformConvError's cases; `metalUnavailable` is the "no device" case.
    enum class Kind { invalidShape, invalidArrayCount, metalUnavailable, shaderResourceMissing,
                      nonFiniteOutput, commandFailed };

    static DeformConvError invalidShape() { return DeformConvError(Kind::invalidShape, "Invalid deformable-convolution shape"); }
    static DeformConvError invalidArrayCount(const std::string& name, long expected, long actual) {
        DeformConvError e(Kind::invalidArrayCount,
                          name + " has " + std::to_string(actual) + " elements; expected " + std::to_string(expected));
        e.name_ = name;
        e.expected_ = expected;
        e.actual_ = actual;
        return e;
    }
    static DeformConvError metalUnavailable() { return DeformConvError(Kind::metalUnavailable, "No HIP device is available"); }
    static DeformConvError shaderResourceMissing() { return DeformConvError(Kind::shaderResourceMissing, "A device kernel is missing"); }
    static DeformConvError nonFiniteOutput(const std::string& m) { return DeformConvError(Kind::nonFiniteOutput, m); }
    static DeformConvError commandFailed(const std::string& m) { return DeformConvError(Kind::commandFailed, m); }

    Kind kind() const { return kind_; }
    // Only a non-finite model output is recoverable (DeformConv.swift:52-55).
    bool isRecoverableNumericalFailure() const { return kind_ == Kind::nonFiniteOutput; }
    const char* what() const noexcept override { return message_.c_str(); }
    const std::string& name() const { return name_; }
    long expected() const { return expected_; }
    long actual() const { return actual_; }

private:
    DeformConvError(Kind k, std::string m) : kind_(k), message_(std::move(m)) {}
    Kind kind_;
    std::string message_, name_;
    long expected_ = 0, actual_ = 0;
};

struct DeformConvShape {
    int batch, inputChannels, inputHeight, inputWidth;
    int outputChannels, outputHeight, outputWidth;
    int kernelHeight, kernelWidth, padHeight, padWidth;
    int strideHeight, strideWidth, dilationHeight, dilationWidth;
    int groups, offsetGroups;

    long inputCount() const { return (long)batch * inputChannels * inputHeight * inputWidth; }
    long outputCount() const { return (long)batch * outputChannels * outputHeight * outputWidth; }
    long kernelArea() const { return (long)kernelHeight * kernelWidth; }
    long offsetCount() const { return (long)batch * 2 * offsetGroups * kernelArea() * outputHeight * outputWidth; }
    long maskCount() const { return (long)batch * offsetGroups * kernelArea() * outputHeight * outputWidth; }
    long weightCount() const { return groups > 0 ? (long)outputChannels * (inputChannels / groups) * kernelArea() : 0; }

    dcn_shape toC() const {
        return dcn_shape{batch, inputChannels, inputHeight, inputWidth, outputChannels, outputHeight,
                         outputWidth, kernelHeight, kernelWidth, padHeight, padWidth, strideHeight,
                         strideWidth, dilationHeight, dilationWidth, groups, offsetGroups};
    }
    void validate() const {
        const dcn_shape s = toC();
        if (dcn_shape_validate(&s) != DCN_OK) throw DeformConvError::invalidShape();
    }
};

// The BenchmarkJasnaShape layer shape (MetalRunner.swift:191-208).
inline DeformConvShape jasnaShape() { return DeformConvShape{1, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16}; }

struct SeededGenerator {
    uint64_t state;
    explicit SeededGenerator(uint64_t seed) : state(dcn_splitmix64_seed(seed)) {}
    uint64_t next() { return dcn_splitmix64_next(&state); }
    // floats(count:range:) — uniform in [lo, hi].
    std::vector<float> floats(size_t count, float lo, float hi) {
        std::vector<float> out(count);
        dcn_seeded_floats(&state, count, lo, hi, out.data());
        return out;
    }
};

struct BenchmarkStatistics {
    std::vector<double> samples;  // sorted
    double minimum = 0, maximum = 0, median = 0, mean = 0, standardDeviation = 0;
    double percentile10 = 0, percentile90 = 0;

    // nil for empty or non-finite samples, as the Swift initializer.
    static std::optional<BenchmarkStatistics> make(std::vector<double> values) {
        dcn_statistics s{};
        if (dcn_compute_statistics(values.data(), values.size(), &s) != DCN_OK) return std::nullopt;
        BenchmarkStatistics b;
        std::sort(values.begin(), values.end());
        b.samples = std::move(values);
        b.minimum = s.minimum;
        b.maximum = s.maximum;
        b.median = s.median;
        b.mean = s.mean;
        b.standardDeviation = s.standard_deviation;
        b.percentile10 = s.percentile10;
        b.percentile90 = s.percentile90;
        return b;
    }
};

struct DeformConvWeightSet {
    static constexpr long weightElements = 128 * 9 * 64;
    static constexpr long biasElements = 64;
    static constexpr long expectedBytes = (weightElements + biasElements) * 2;

    std::string direction;
    std::string path;
    std::vector<uint8_t> data;

    // DeformConvWeightSet.init (DeformConvWeights.swift:11-21): the size check.
    DeformConvWeightSet(std::string dir, const std::string& file) : direction(std::move(dir)), path(file) {
        std::ifstream in(file, std::ios::binary);
        if (!in) throw DeformConvError::commandFailed("cannot open " + file);
        data.assign(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
        if ((long)data.size() != expectedBytes) {
            const std::string name = file.substr(file.find_last_of('/') + 1);
            throw DeformConvError::commandFailed(name + " has " + std::to_string(data.size()) +
                                                 " bytes; expected " + std::to_string(expectedBytes));
        }
    }
    // The --validate-deform-weights checksum (JasnaCLI.swift:1415-1421).
    double checksum() const {
        return dcn_checksum_f16(reinterpret_cast<const uint16_t*>(data.data()), data.size() / 2);
    }
};

inline std::vector<DeformConvWeightSet> loadDeformConvWeightSets(const std::string& directory) {
    std::vector<DeformConvWeightSet> sets;
    for (const char* d : {"backward_1", "forward_1", "backward_2", "forward_2"})
        sets.emplace_back(d, directory + "/" + d + ".dcnfp16");
    return sets;
}

// PropagationBranch / PropagationStep / TemporalSchedule (TemporalSchedule.swift:3-101).
struct PropagationBranch {
    std::string name;
    bool backward;
    int pass;
    int branchIndex;
    int backboneInputChannels() const { return (2 + branchIndex) * 64; }
};

struct PropagationStep {
    int branch;                                // index into TemporalSchedule::branches
    int position;
    int frameIndex;
    std::optional<int> flowIndex;              // nil at position 0
    std::optional<int> secondOrderFrameIndex;  // nil below position 2
};

struct TemporalSchedule {
    int frameCount;
    std::vector<PropagationBranch> branches;
    std::vector<PropagationStep> steps;

    explicit TemporalSchedule(int frames) : frameCount(frames) {
        if (frames <= 0) throw DeformConvError::invalidShape();
        branches = {{"backward_1", true, 1, 0}, {"forward_1", false, 1, 1},
                    {"backward_2", true, 2, 2}, {"forward_2", false, 2, 3}};
        std::vector<dcn_schedule_step> raw(4 * (size_t)frames);
        size_t n = 0;
        if (dcn_temporal_schedule(frames, raw.data(), raw.size(), &n) != DCN_OK)
            throw DeformConvError::commandFailed("invalid propagation schedule size");
        for (size_t i = 0; i < n; ++i) {
            const dcn_schedule_step& r = raw[i];
            PropagationStep st{r.branch, r.position, r.frame, std::nullopt, std::nullopt};
            if (r.flow_index >= 0) st.flowIndex = r.flow_index;
            if (r.second_order_frame >= 0) st.secondOrderFrameIndex = r.second_order_frame;
            steps.push_back(st);
        }
    }
    int flowCountPerDirection() const { return std::max(frameCount - 1, 0); }
    size_t persistentTensorBytes() const { return dcn_schedule_persistent_bytes(frameCount); }
    std::vector<PropagationStep> stepsOf(const std::string& name) const {
        std::vector<PropagationStep> out;
        for (const auto& st : steps)
            if (branches[(size_t)st.branch].name == name) out.push_back(st);
        return out;
    }
};

// Half-open frame ranges [first, second).
inline std::vector<std::pair<int, int>> temporalChunkRanges(int frameCount, int maximumFramesPerChunk) {
    std::vector<int> starts((size_t)std::max(frameCount, 1)), sizes(starts.size());
    size_t n = 0;
    if (dcn_temporal_chunk_ranges(frameCount, maximumFramesPerChunk, starts.data(), sizes.data(), starts.size(),
                                  &n) != DCN_OK)
        throw DeformConvError::invalidShape();
    std::vector<std::pair<int, int>> out;
    for (size_t i = 0; i < n; ++i) out.emplace_back(starts[i], starts[i] + sizes[i]);
    return out;
}

class PackedWeights {
public:
    PackedWeights() = default;
    explicit PackedWeights(dcn_packed* p) : p_(p) {}
    PackedWeights(PackedWeights&& o) noexcept : p_(std::exchange(o.p_, nullptr)) {}
    PackedWeights& operator=(PackedWeights&& o) noexcept {
        if (this != &o) {
            dcn_packed_free(p_);
            p_ = std::exchange(o.p_, nullptr);
        }
        return *this;
    }
    PackedWeights(const PackedWeights&) = delete;
    PackedWeights& operator=(const PackedWeights&) = delete;
    ~PackedWeights() { dcn_packed_free(p_); }
    const dcn_packed* get() const { return p_; }

private:
    dcn_packed* p_ = nullptr;
};

struct BenchmarkResult {  // BenchmarkResult (MetalRunner.swift:67-90), this build's variants
    BenchmarkStatistics baseline, gather, fused;  // milliseconds
    double checksum = 0;
    float maxDifferenceFromBaseline = 0;
    int iterations = 0;
};

// MetalDeformConv's role on a HIP device.
// SPyNetPairResult (SPyNetPairProbe.swift:4-18): timing of the bidirectional pair over 7
// samples, per-direction maxima and stride-257 checksums, repeat and oracle errors, flows.
struct SPyNetPairResult {
    double medianMilliseconds = 0, minimumMilliseconds = 0, maximumMilliseconds = 0;
    int iterations = 0;
    int elementCount = 0;
    float backwardMaximum = 0, forwardMaximum = 0, repeatMaximumError = 0, oracleMaximumError = 0;
    double backwardChecksum = 0, forwardChecksum = 0;
    std::vector<uint16_t> backwardFlow, forwardFlow;
};

// The six basic modules of SPyNet, OIHW FP16 bit patterns, level 0 the coarsest; layer i
// of every level is kSPyNetLayers[i] = {cin, cout}, 7 x 7.
struct SPyNetWeights {
    static constexpr int layers[DCN_SPYNET_LAYERS][2] = {{8, 32}, {32, 64}, {64, 32}, {32, 16}, {16, 2}};
    std::vector<uint16_t> weight[DCN_SPYNET_LEVELS][DCN_SPYNET_LAYERS];
    std::vector<uint16_t> bias[DCN_SPYNET_LEVELS][DCN_SPYNET_LAYERS];
    void validate() const {
        for (int l = 0; l < DCN_SPYNET_LEVELS; ++l)
            for (int i = 0; i < DCN_SPYNET_LAYERS; ++i) {
                const size_t expected = (size_t)layers[i][0] * layers[i][1] * 49;
                if (weight[l][i].size() != expected)
                    throw DeformConvError::invalidArrayCount("spynet.weight", (long)expected, (long)weight[l][i].size());
                if (bias[l][i].size() != (size_t)layers[i][1])
                    throw DeformConvError::invalidArrayCount("spynet.bias", layers[i][1], (long)bias[l][i].size());
            }
    }
};

// deterministic_frame of tools/export_spynet_oracle.py:14-19: RGB 3 x 64 x 64 values
// ((i * multiplier + addend) % modulus) / divisor rounded to FP16.
inline std::vector<uint16_t> deterministicSPyNetFrame(long multiplier, long addend, long modulus, long divisor,
                                                     int size = 64) {
    std::vector<float> v((size_t)3 * size * size);
    for (size_t i = 0; i < v.size(); ++i) v[i] = (float)(((long)i * multiplier + addend) % modulus) / (float)divisor;
    std::vector<uint16_t> h(v.size());
    dcn_f32_to_f16_array(v.data(), h.data(), v.size());
    return h;
}

class HipDeformConv {
public:
    explicit HipDeformConv(int device = 0) {
        if (dcn_create(&ctx_, device) != DCN_OK) throw DeformConvError::metalUnavailable();
    }
    ~HipDeformConv() { dcn_destroy(ctx_); }
    HipDeformConv(const HipDeformConv&) = delete;
    HipDeformConv& operator=(const HipDeformConv&) = delete;
    dcn_context* context() const { return ctx_; }

    // runFloat32 (MetalRunner.swift:159-185).
    std::vector<float> runFloat32(const DeformConvShape& shape, const std::vector<float>& input,
                                  const std::vector<float>& offset, const std::vector<float>& mask,
                                  const std::vector<float>& weight, const std::vector<float>& bias) {
        shape.validate();
        std::vector<float> out((size_t)shape.outputCount());
        const dcn_shape s = shape.toC();
        check(dcn_forward_f32(ctx_, &s, input.data(), input.size(), offset.data(), offset.size(),
                              mask.data(), mask.size(), weight.data(), weight.size(), bias.data(),
                              bias.size(), out.data(), out.size()));
        return out;
    }
    // FP16 storage, FP32 arithmetic (deform_conv2d_fp16, MetalShader.swift:126-174);
    // binary16 bit patterns.
    std::vector<uint16_t> runFloat16(const DeformConvShape& shape, const std::vector<uint16_t>& input,
                                     const std::vector<uint16_t>& offset, const std::vector<uint16_t>& mask,
                                     const std::vector<uint16_t>& weight, const std::vector<uint16_t>& bias) {
        shape.validate();
        std::vector<uint16_t> out((size_t)shape.outputCount());
        const dcn_shape s = shape.toC();
        check(dcn_forward_f16(ctx_, &s, input.data(), input.size(), offset.data(), offset.size(),
                              mask.data(), mask.size(), weight.data(), weight.size(), bias.data(),
                              bias.size(), out.data(), out.size()));
        return out;
    }
    PackedWeights prepack(const DeformConvShape& shape, const std::vector<uint16_t>& weight,
                          const std::vector<uint16_t>& bias, dcn_weight_layout layout = DCN_LAYOUT_OIHW) {
        const dcn_shape s = shape.toC();
        dcn_packed* p = nullptr;
        check(dcn_prepack_f16(ctx_, &s, weight.data(), weight.size(), layout, bias.data(), bias.size(), &p));
        return PackedWeights(p);
    }
    PackedWeights loadWeightSet(const DeformConvWeightSet& set) {
        dcn_packed* p = nullptr;
        check(dcn_load_dcnfp16(ctx_, set.path.c_str(), &p));
        return PackedWeights(p);
    }
    // The fused sampler + MFMA GEMM (the role of executeJasnaSIMDGroupGEMM).
    std::vector<uint16_t> runFloat16Prepacked(const DeformConvShape& shape, const std::vector<uint16_t>& input,
                                              const std::vector<uint16_t>& offset,
                                              const std::vector<uint16_t>& mask, const PackedWeights& packed) {
        shape.validate();
        std::vector<uint16_t> out((size_t)shape.outputCount());
        const dcn_shape s = shape.toC();
        check(dcn_forward_f16_prepacked(ctx_, &s, input.data(), input.size(), offset.data(), offset.size(),
                                        mask.data(), mask.size(), packed.get(), out.data(), out.size()));
        return out;
    }

    // flag_non_finite_fp16 (MetalShader.swift:454-463) as MetalNonFiniteFlagTests drives
    // it: a zeroed flag, one check over `values`, the flag read back (0 or 1).
    uint32_t flagNonFinite(const std::vector<uint16_t>& values) {
        if (values.empty()) throw DeformConvError::invalidShape();
        DeviceBuffer dv(values), flag(2);
        if (hipMemset(flag.p, 0, 4) != hipSuccess) throw DeformConvError::commandFailed("flag clear failed");
        check(dcn_flag_nonfinite_f16_dev(ctx_, dv.p, values.size(), flag.p, nullptr));
        uint32_t result = 0;
        if (hipMemcpy(&result, flag.p, 4, hipMemcpyDeviceToHost) != hipSuccess)
            throw DeformConvError::commandFailed("flag read failed");
        return result;
    }

    // benchmarkJasnaShape (MetalRunner.swift:187-388): the reference's seeded inputs (or a
    // weight set), 2 warm-ups and `iterations` timed calls per variant on device buffers
    // (direct FP16 baseline, gather alone, fused path), checksum over the fused output,
    // and the 2e-3 gate against the baseline.
    BenchmarkResult benchmarkJasnaShape(int iterations = 20, const DeformConvWeightSet* weightSet = nullptr) {
        const DeformConvShape shape = jasnaShape();
        SeededGenerator rng(0x4A41534E41ull);
        auto half = [](const std::vector<float>& v) {
            std::vector<uint16_t> h(v.size());
            dcn_f32_to_f16_array(v.data(), h.data(), v.size());
            return h;
        };
        const auto input = half(rng.floats((size_t)shape.inputCount(), -1.0f, 1.0f));
        const auto offset = half(rng.floats((size_t)shape.offsetCount(), -0.25f, 0.25f));
        const auto mask = half(rng.floats((size_t)shape.maskCount(), 0.25f, 0.75f));
        std::vector<uint16_t> weight((size_t)shape.weightCount()), bias(64);
        if (weightSet) {
            const uint16_t* v = reinterpret_cast<const uint16_t*>(weightSet->data.data());
            for (int ic = 0; ic < 128; ++ic)
                for (int k = 0; k < 9; ++k)
                    for (int oc = 0; oc < 64; ++oc) weight[((size_t)oc * 128 + ic) * 9 + k] = v[((size_t)ic * 9 + k) * 64 + oc];
            for (int oc = 0; oc < 64; ++oc) bias[oc] = v[DeformConvWeightSet::weightElements + oc];
        } else {
            weight = half(rng.floats(weight.size(), -0.02f, 0.02f));
            bias = half(rng.floats(64, -0.02f, 0.02f));
        }
        DeviceBuffer dx(input), doff(offset), dm(mask), dw(weight), db(bias);
        DeviceBuffer base((size_t)shape.outputCount()), fused((size_t)shape.outputCount());
        DeviceBuffer cols((size_t)shape.outputHeight * shape.outputWidth * shape.inputChannels * shape.kernelArea());
        const dcn_shape s = shape.toC();
        dcn_packed* pp = nullptr;
        check(dcn_prepack_f16_dev(ctx_, &s, dw.p, DCN_LAYOUT_OIHW, db.p, nullptr, &pp));
        PackedWeights packed(pp);
        check(dcn_reserve(ctx_, &s));
        Event e0, e1;
        auto time = [&](auto&& call) {
            for (int i = 0; i < 2; ++i) call();
            std::vector<double> ms;
            for (int i = 0; i < std::max(iterations, 1); ++i) {
                hip(hipEventRecord(e0.e, nullptr));
                call();
                hip(hipEventRecord(e1.e, nullptr));
                hip(hipEventSynchronize(e1.e));
                float t = 0;
                hip(hipEventElapsedTime(&t, e0.e, e1.e));
                ms.push_back(t);
            }
            auto st = BenchmarkStatistics::make(ms);
            if (!st) throw DeformConvError::commandFailed("invalid DCNv2 benchmark samples");
            return *st;
        };
        BenchmarkResult r;
        r.baseline = time([&] { check(dcn_forward_f16_dev(ctx_, &s, dx.p, doff.p, dm.p, dw.p, db.p, base.p, nullptr)); });
        r.gather = time([&] { check(dcn_im2col_f16_dev(ctx_, &s, dx.p, doff.p, dm.p, cols.p, nullptr)); });
        r.fused = time([&] {
            check(dcn_forward_f16_prepacked_dev(ctx_, &s, dx.p, doff.p, dm.p, packed.get(), fused.p, nullptr));
        });
        const std::vector<uint16_t> b = base.download(), f = fused.download();
        for (size_t i = 0; i < f.size(); ++i)
            r.maxDifferenceFromBaseline = std::max(r.maxDifferenceFromBaseline,
                                                   std::fabs(dcn_f16_to_f32(f[i]) - dcn_f16_to_f32(b[i])));
        if (r.maxDifferenceFromBaseline > 0.002f)
            throw DeformConvError::commandFailed("fused FP16 result differs from baseline by " +
                                                 std::to_string(r.maxDifferenceFromBaseline));
        r.checksum = dcn_checksum_f16(f.data(), f.size());
        r.iterations = std::max(iterations, 1);
        return r;
    }

    // jasna_bicubic_downsample_quarter_fp16 (MetalShader.swift:488-521) on host arrays.
    std::vector<uint16_t> bicubicQuarter(int channels, int height, int width, const std::vector<uint16_t>& input) {
        if (input.size() != (size_t)channels * height * width)
            throw DeformConvError::invalidArrayCount("input", (long)channels * height * width, (long)input.size());
        DeviceBuffer in(input), out((size_t)channels * (height / 4) * (width / 4));
        check(dcn_bicubic_quarter_f16_dev(ctx_, channels, height, width, in.p, out.p, nullptr));
        return out.download();
    }

    // verifySPyNetPair (SPyNetPairProbe.swift:47-449): the bidirectional pair on 64 x 64
    // frames (default: the deterministic frames of tools/export_spynet_oracle.py), 2 warm-ups
    // and 7 timed runs, then the reference's gates: both maxima > 0.001, repeat error <=
    // 0.001 and, when an oracle directory with backward.f16 / forward.f16 is given, oracle
    // error <= 0.05. Throws commandFailed when a gate fails or a flow is non-finite.
    SPyNetPairResult verifySPyNetPair(const SPyNetWeights& weights, const std::vector<uint16_t>* reference = nullptr,
                                      const std::vector<uint16_t>* support = nullptr,
                                      const std::string& oracleDirectory = "") {
        constexpr int size = 64, plane = size * size;
        weights.validate();
        const std::vector<uint16_t> ref = reference ? *reference : deterministicSPyNetFrame(29, 17, 1021, 1020);
        const std::vector<uint16_t> sup = support ? *support : deterministicSPyNetFrame(43, 31, 1019, 1018);
        if (ref.size() != (size_t)3 * plane) throw DeformConvError::invalidArrayCount("reference", 3 * plane, (long)ref.size());
        if (sup.size() != (size_t)3 * plane) throw DeformConvError::invalidArrayCount("support", 3 * plane, (long)sup.size());
        std::vector<std::unique_ptr<DeviceBuffer>> wbuf;
        dcn_spynet_weights w{};
        for (int l = 0; l < DCN_SPYNET_LEVELS; ++l)
            for (int i = 0; i < DCN_SPYNET_LAYERS; ++i) {
                wbuf.emplace_back(new DeviceBuffer(weights.weight[l][i]));
                w.weight[l][i] = wbuf.back()->p;
                wbuf.emplace_back(new DeviceBuffer(weights.bias[l][i]));
                w.bias[l][i] = wbuf.back()->p;
            }
        dcn_spynet* raw = nullptr;
        check(dcn_spynet_create(ctx_, size, size, 2, &w, nullptr, &raw));
        std::unique_ptr<dcn_spynet, void (*)(dcn_spynet*)> net(raw, dcn_spynet_destroy);
        DeviceBuffer dref(ref), dsup(sup), flow((size_t)4 * plane);
        Event e0, e1;
        auto execute = [&](std::vector<uint16_t>* out) {
            hip(hipEventRecord(e0.e, nullptr));
            check(dcn_spynet_flow_dev(net.get(), dref.p, dsup.p, 1, flow.p, nullptr));
            hip(hipEventRecord(e1.e, nullptr));
            hip(hipEventSynchronize(e1.e));
            float t = 0;
            hip(hipEventElapsedTime(&t, e0.e, e1.e));
            if (out) *out = flow.download();
            return (double)t;
        };
        execute(nullptr);
        execute(nullptr);
        std::vector<uint16_t> first, last;
        std::vector<double> samples{execute(&first)};
        for (int i = 1; i < 7; ++i) samples.push_back(execute(&last));
        std::sort(samples.begin(), samples.end());
        std::vector<uint16_t> oracle[2];
        if (!oracleDirectory.empty()) {
            const char* names[2] = {"backward.f16", "forward.f16"};
            for (int d = 0; d < 2; ++d) {
                std::ifstream f(oracleDirectory + "/" + names[d], std::ios::binary);
                std::vector<char> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
                if (!f.good() && !f.eof()) throw DeformConvError::commandFailed("cannot read the SPyNet oracle");
                if (bytes.size() != (size_t)2 * plane * 2) throw DeformConvError::commandFailed("invalid SPyNet oracle size");
                oracle[d].resize((size_t)2 * plane);
                std::memcpy(oracle[d].data(), bytes.data(), bytes.size());
            }
        }
        SPyNetPairResult r;
        float maxima[2] = {0, 0};
        double checksums[2] = {0, 0};
        for (int d = 0; d < 2; ++d)
            for (size_t i = 0; i < (size_t)2 * plane; ++i) {
                const size_t k = (size_t)d * 2 * plane + i;
                const float v = dcn_f16_to_f32(last[k]);
                if (!std::isfinite(v)) throw DeformConvError::commandFailed("SPyNet produced a non-finite flow");
                maxima[d] = std::max(maxima[d], std::fabs(v));
                r.repeatMaximumError = std::max(r.repeatMaximumError, std::fabs(dcn_f16_to_f32(first[k]) - v));
                if (!oracle[d].empty())
                    r.oracleMaximumError = std::max(r.oracleMaximumError, std::fabs(dcn_f16_to_f32(oracle[d][i]) - v));
                if (i % 257 == 0) checksums[d] += (double)v;
            }
        if (!(maxima[0] > 0.001f && maxima[1] > 0.001f) || r.repeatMaximumError > 0.001f || r.oracleMaximumError > 0.05f)
            throw DeformConvError::commandFailed("SPyNet validation failed (maxima=[" + std::to_string(maxima[0]) + ", " +
                                                 std::to_string(maxima[1]) + "], repeat=" +
                                                 std::to_string(r.repeatMaximumError) + ", oracle=" +
                                                 std::to_string(r.oracleMaximumError) + ")");
        r.medianMilliseconds = samples[samples.size() / 2];
        r.minimumMilliseconds = samples.front();
        r.maximumMilliseconds = samples.back();
        r.iterations = (int)samples.size();
        r.elementCount = 2 * 2 * plane;
        r.backwardMaximum = maxima[0];
        r.forwardMaximum = maxima[1];
        r.backwardChecksum = checksums[0];
        r.forwardChecksum = checksums[1];
        r.backwardFlow.assign(last.begin(), last.begin() + 2 * plane);
        r.forwardFlow.assign(last.begin() + 2 * plane, last.end());
        return r;
    }

private:
    void check(dcn_status st) const {
        switch (st) {
            case DCN_OK: return;
            case DCN_INVALID_SHAPE: throw DeformConvError::invalidShape();
            case DCN_INVALID_ARRAY_COUNT: {
                // "<name> has <actual> elements; expected <expected>"
                const std::string m = dcn_last_error(ctx_);
                char name[64] = {0};
                long actual = 0, expected = 0;
                if (std::sscanf(m.c_str(), "%63s has %ld elements; expected %ld", name, &actual, &expected) == 3)
                    throw DeformConvError::invalidArrayCount(name, expected, actual);
                throw DeformConvError::commandFailed(m);
            }
            case DCN_DEVICE_UNAVAILABLE: throw DeformConvError::metalUnavailable();
            case DCN_KERNEL_MISSING: throw DeformConvError::shaderResourceMissing();
            case DCN_NONFINITE_OUTPUT: throw DeformConvError::nonFiniteOutput(dcn_last_error(ctx_));
            default: throw DeformConvError::commandFailed(dcn_last_error(ctx_));
        }
    }
    static void hip(hipError_t e) {
        if (e != hipSuccess) throw DeformConvError::commandFailed(hipGetErrorString(e));
    }
    struct DeviceBuffer {
        void* p = nullptr;
        size_t n = 0;
        explicit DeviceBuffer(size_t count) : n(count) {
            if (hipMalloc(&p, std::max<size_t>(n, 1) * 2) != hipSuccess) throw DeformConvError::metalUnavailable();
        }
        explicit DeviceBuffer(const std::vector<uint16_t>& h) : DeviceBuffer(h.size()) {
            if (hipMemcpy(p, h.data(), n * 2, hipMemcpyHostToDevice) != hipSuccess)
                throw DeformConvError::commandFailed("upload failed");
        }
        std::vector<uint16_t> download() const {
            std::vector<uint16_t> h(n);
            if (hipMemcpy(h.data(), p, n * 2, hipMemcpyDeviceToHost) != hipSuccess)
                throw DeformConvError::commandFailed("download failed");
            return h;
        }
        ~DeviceBuffer() { (void)hipFree(p); }
        DeviceBuffer(const DeviceBuffer&) = delete;
        DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    };
    struct Event {
        hipEvent_t e = nullptr;
        Event() { hip(hipEventCreate(&e)); }
        ~Event() { (void)hipEventDestroy(e); }
    };
    dcn_context* ctx_ = nullptr;
};

}  // namespace jasna
