// C++ tests of the host layer in include/dcn/deform_conv.hpp, written after the reference's
// Swift tests so each reads like its original:
//   DeformConvCPUTests.swift:4-33, 35-41     (1x1 known answer, recoverability)
//   BenchmarkStatisticsTests.swift:5-20      (summary of [4,1,3,2]; nil for [] and [1, inf])
//   MetalNonFiniteFlagTests.swift:5-53       (flag_non_finite_fp16 on finite / inf / nan)
//   JasnaCLI.swift:68-110                    (correctnessTest: seeded 1x2x5x5 -> 3, 2e-5 gate)
//   TemporalScheduleTests.swift:4-40         (traversal, widths, second order, 30 frames)
//   RestorationResumeTests.swift:51-72       (temporalChunkRanges)
//   SPyNetPairProbe.swift:47-449             (verifySPyNetPair: gates, oracle files)
// plus the weight-set loader and benchmarkJasnaShape. The CPU oracle (oracle/liboracle.so)
// stands in for DeformConvCPU as the checker; the library under test never calls it.
//
// Usage: host_tests cpu | gpu   (exit status 0 when every test of the group passes)
#include "dcn/deform_conv.hpp"

#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

extern "C" {
#include "dcn_oracle.h"
}

namespace {

struct TestCase {
    const char* group;
    const char* name;
    std::function<void()> body;
};
std::vector<TestCase>& registry() {
    static std::vector<TestCase> r;
    return r;
}
struct Register {
    Register(const char* g, const char* n, std::function<void()> f) { registry().push_back({g, n, std::move(f)}); }
};
#define TEST(group, name)                                       \
    static void name();                                         \
    static Register reg_##name(#group, #name, name);            \
    static void name()

struct Failure {
    std::string what;
};
#define EXPECT(cond)                                                                        \
    do {                                                                                    \
        if (!(cond)) throw Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) +  \
                                   ": expected " #cond};                                    \
    } while (0)

template <class F>
jasna::DeformConvError expectThrows(F&& f) {
    try {
        f();
    } catch (const jasna::DeformConvError& e) {
        return e;
    }
    throw Failure{"expected a DeformConvError"};
}

using jasna::DeformConvError;
using jasna::DeformConvShape;

// DeformConvCPU.run's role: the CPU oracle.
std::vector<float> cpuRun(const DeformConvShape& s, const std::vector<float>& input, const std::vector<float>& offset,
                          const std::vector<float>& mask, const std::vector<float>& weight,
                          const std::vector<float>& bias) {
    oracle_shape o;
    static_assert(sizeof(o) == sizeof(DeformConvShape), "17 int fields");
    std::memcpy(&o, &s, sizeof(o));
    std::vector<float> out((size_t)s.outputCount());
    if (oracle_dcn_forward_f32(&o, input.data(), offset.data(), mask.data(), weight.data(), bias.data(),
                               out.data()) != 0)
        throw DeformConvError::invalidShape();
    return out;
}

std::vector<uint16_t> toHalf(const std::vector<float>& v) {
    std::vector<uint16_t> h(v.size());
    dcn_f32_to_f16_array(v.data(), h.data(), v.size());
    return h;
}
std::vector<float> toFloat(const std::vector<uint16_t>& h) {
    std::vector<float> v(h.size());
    dcn_f16_to_f32_array(h.data(), v.data(), h.size());
    return v;
}

const DeformConvShape kOneByOne{1, 1, 2, 2, 1, 2, 2, 1, 1, 0, 0, 1, 1, 1, 1, 1, 1};

std::string tempFile(const std::vector<uint8_t>& bytes, const char* suffix) {
    char dir[] = "/tmp/dcn_host_tests_XXXXXX";
    if (!mkdtemp(dir)) throw Failure{"mkdtemp failed"};
    const std::string path = std::string(dir) + "/" + suffix;
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) throw Failure{"cannot write " + path};
    std::fwrite(bytes.data(), 1, bytes.size(), f);
    std::fclose(f);
    return path;
}

// ---- CPU group ---------------------------------------------------------------------

TEST(cpu, oneByOneConvolutionMatchesExpectedValues) {
    const auto output = cpuRun(kOneByOne, {1, 2, 3, 4}, std::vector<float>((size_t)kOneByOne.offsetCount(), 0.0f),
                               std::vector<float>((size_t)kOneByOne.maskCount(), 0.5f), {2}, {1});
    EXPECT((output == std::vector<float>{2, 3, 4, 5}));
}

TEST(cpu, onlyNonFiniteModelOutputIsRecoverable) {
    EXPECT(DeformConvError::nonFiniteOutput("overflow").isRecoverableNumericalFailure());
    EXPECT(!DeformConvError::invalidShape().isRecoverableNumericalFailure());
    EXPECT(!DeformConvError::metalUnavailable().isRecoverableNumericalFailure());
    EXPECT(!DeformConvError::shaderResourceMissing().isRecoverableNumericalFailure());
    EXPECT(!DeformConvError::commandFailed("device lost").isRecoverableNumericalFailure());
    EXPECT(!DeformConvError::invalidArrayCount("offset", 4, 3).isRecoverableNumericalFailure());
}

TEST(cpu, benchmarkStatisticsSummarizeEvenSampleSet) {
    const auto st = jasna::BenchmarkStatistics::make({4, 1, 3, 2});
    EXPECT(st.has_value());
    EXPECT((st->samples == std::vector<double>{1, 2, 3, 4}));
    EXPECT(st->minimum == 1);
    EXPECT(st->maximum == 4);
    EXPECT(st->median == 2.5);
    EXPECT(st->mean == 2.5);
    EXPECT(std::fabs(st->standardDeviation - std::sqrt(1.25)) < 1e-12);
    EXPECT(std::fabs(st->percentile10 - 1.3) < 1e-12);
    EXPECT(std::fabs(st->percentile90 - 3.7) < 1e-12);
}

TEST(cpu, benchmarkStatisticsRejectEmptyAndNonfiniteSamples) {
    EXPECT(!jasna::BenchmarkStatistics::make({}).has_value());
    EXPECT(!jasna::BenchmarkStatistics::make({1, INFINITY}).has_value());
}

TEST(cpu, shapeValidationRejectsWhatTheReferenceRejects) {
    jasna::jasnaShape().validate();
    kOneByOne.validate();
    auto bad = [](auto edit) {
        DeformConvShape s = jasna::jasnaShape();
        edit(s);
        EXPECT(expectThrows([&] { s.validate(); }).kind() == DeformConvError::Kind::invalidShape);
    };
    bad([](DeformConvShape& s) { s.batch = 0; });
    bad([](DeformConvShape& s) { s.inputChannels = 0; });
    bad([](DeformConvShape& s) { s.outputHeight = 0; });
    bad([](DeformConvShape& s) { s.kernelWidth = 0; });
    bad([](DeformConvShape& s) { s.groups = 3; });        // 128 % 3 != 0
    bad([](DeformConvShape& s) { s.offsetGroups = 3; });  // 128 % 3 != 0
}

TEST(cpu, shapeCountsFollowTheReference) {
    const DeformConvShape s = jasna::jasnaShape();
    EXPECT(s.inputCount() == 128L * 64 * 64);
    EXPECT(s.offsetCount() == 2L * 16 * 9 * 64 * 64);
    EXPECT(s.maskCount() == 16L * 9 * 64 * 64);
    EXPECT(s.weightCount() == 64L * 128 * 9);
    EXPECT(s.outputCount() == 64L * 64 * 64);
    const dcn_shape c = s.toC();
    dcn_counts n{};
    EXPECT(dcn_shape_counts(&c, &n) == DCN_OK);
    EXPECT((long)n.input == s.inputCount() && (long)n.offset == s.offsetCount() && (long)n.mask == s.maskCount() &&
           (long)n.weight == s.weightCount() && (long)n.output == s.outputCount());
}

TEST(cpu, seededGeneratorIsDeterministicAndInRange) {
    jasna::SeededGenerator a(0xC0FFEE), b(0xC0FFEE), c(0xC0FFEF);
    const auto x = a.floats(1000, -0.4f, 0.4f), y = b.floats(1000, -0.4f, 0.4f), z = c.floats(1000, -0.4f, 0.4f);
    EXPECT(x == y);
    EXPECT(x != z);
    for (float v : x) EXPECT(v >= -0.4f && v <= 0.4f);
    EXPECT(a.next() == b.next());
}

TEST(cpu, weightSetRejectsWrongSize) {
    const std::string path = tempFile(std::vector<uint8_t>(1000, 0), "forward_1.dcnfp16");
    const auto e = expectThrows([&] { jasna::DeformConvWeightSet("forward_1", path); });
    EXPECT(e.kind() == DeformConvError::Kind::commandFailed);
    EXPECT(std::string(e.what()) == "forward_1.dcnfp16 has 1000 bytes; expected 147584");
}

TEST(cpu, weightSetChecksumIsTheStride257Sum) {
    // Every value 1.0 (0x3C00): the checksum counts the sampled indices 0, 257, ..., the
    // 288 multiples of 257 below 73,792 values.
    std::vector<uint8_t> bytes((size_t)jasna::DeformConvWeightSet::expectedBytes);
    for (size_t i = 0; i < bytes.size(); i += 2) {
        bytes[i] = 0x00;
        bytes[i + 1] = 0x3C;
    }
    const jasna::DeformConvWeightSet set("backward_1", tempFile(bytes, "backward_1.dcnfp16"));
    EXPECT(set.checksum() == 288.0);
    EXPECT(dcn_dcnfp16_bytes() == (size_t)jasna::DeformConvWeightSet::expectedBytes);
}

std::vector<int> frames(const std::vector<jasna::PropagationStep>& v) {
    std::vector<int> out;
    for (const auto& s : v) out.push_back(s.frameIndex);
    return out;
}
std::vector<int> flows(const std::vector<jasna::PropagationStep>& v) {  // -1 for nil
    std::vector<int> out;
    for (const auto& s : v) out.push_back(s.flowIndex.value_or(-1));
    return out;
}
std::vector<int> secondOrder(const std::vector<jasna::PropagationStep>& v) {
    std::vector<int> out;
    for (const auto& s : v) out.push_back(s.secondOrderFrameIndex.value_or(-1));
    return out;
}

TEST(cpu, temporalScheduleMatchesBasicVSRTraversal) {
    const jasna::TemporalSchedule schedule(4);
    const auto backward = schedule.stepsOf("backward_1"), forward = schedule.stepsOf("forward_1");
    EXPECT((frames(backward) == std::vector<int>{3, 2, 1, 0}));
    EXPECT((flows(backward) == std::vector<int>{-1, 2, 1, 0}));
    EXPECT((frames(forward) == std::vector<int>{0, 1, 2, 3}));
    EXPECT((flows(forward) == std::vector<int>{-1, 0, 1, 2}));
    EXPECT(backward[2].secondOrderFrameIndex == 3);
    EXPECT(forward[2].secondOrderFrameIndex == 0);
}

TEST(cpu, temporalScheduleUsesExpectedBackboneWidths) {
    const jasna::TemporalSchedule schedule(3);
    std::vector<int> widths;
    for (const auto& b : schedule.branches) widths.push_back(b.backboneInputChannels());
    EXPECT((widths == std::vector<int>{128, 192, 256, 320}));
    EXPECT(schedule.steps.size() == 12);
    EXPECT(schedule.flowCountPerDirection() == 2);
}

TEST(cpu, fiveFrameScheduleCarriesRollingSecondOrderHistory) {
    const jasna::TemporalSchedule schedule(5);
    const auto backward = schedule.stepsOf("backward_1"), forward = schedule.stepsOf("forward_1");
    EXPECT((frames(backward) == std::vector<int>{4, 3, 2, 1, 0}));
    EXPECT((flows(backward) == std::vector<int>{-1, 3, 2, 1, 0}));
    EXPECT((secondOrder(backward) == std::vector<int>{-1, -1, 4, 3, 2}));
    EXPECT((frames(forward) == std::vector<int>{0, 1, 2, 3, 4}));
    EXPECT((flows(forward) == std::vector<int>{-1, 0, 1, 2, 3}));
    EXPECT((secondOrder(forward) == std::vector<int>{-1, -1, 0, 1, 2}));
}

TEST(cpu, thirtyFrameScheduleHasProductionLengthResources) {
    const jasna::TemporalSchedule schedule(30);
    EXPECT(schedule.flowCountPerDirection() == 29);
    EXPECT(schedule.steps.size() == 120);
    EXPECT(schedule.persistentTensorBytes() == 91389952u);
    EXPECT(expectThrows([] { jasna::TemporalSchedule(0); }).kind() == DeformConvError::Kind::invalidShape);
}

TEST(cpu, temporalChunkRangesMatchTheReference) {
    using R = std::vector<std::pair<int, int>>;
    EXPECT((jasna::temporalChunkRanges(30, 10) == R{{0, 10}, {10, 20}, {20, 30}}));
    EXPECT((jasna::temporalChunkRanges(29, 10) == R{{0, 10}, {10, 20}, {20, 29}}));
    EXPECT((jasna::temporalChunkRanges(11, 5) == R{{0, 4}, {4, 8}, {8, 11}}));
    EXPECT((jasna::temporalChunkRanges(5, 3) == R{{0, 5}}));
    EXPECT(expectThrows([] { jasna::temporalChunkRanges(2, 10); }).kind() == DeformConvError::Kind::invalidShape);
}

// ---- GPU group ---------------------------------------------------------------------

TEST(gpu, hipOneByOneConvolutionMatchesExpectedValues) {
    jasna::HipDeformConv runner;
    const std::vector<float> zeros((size_t)kOneByOne.offsetCount(), 0.0f), halfs((size_t)kOneByOne.maskCount(), 0.5f);
    EXPECT((runner.runFloat32(kOneByOne, {1, 2, 3, 4}, zeros, halfs, {2}, {1}) == std::vector<float>{2, 3, 4, 5}));
    const auto out16 = runner.runFloat16(kOneByOne, toHalf({1, 2, 3, 4}), toHalf(zeros), toHalf(halfs), toHalf({2}),
                                         toHalf({1}));
    EXPECT((toFloat(out16) == std::vector<float>{2, 3, 4, 5}));
}

TEST(gpu, correctnessTest) {
    // JasnaCLI.swift:68-110, seed 0xC0FFEE; the reference gates at 2e-5, this build is
    // bit-identical to the oracle.
    const DeformConvShape shape{1, 2, 5, 5, 3, 5, 5, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1};
    jasna::SeededGenerator rng(0xC0FFEE);
    const auto input = rng.floats((size_t)shape.inputCount(), -1, 1);
    const auto offset = rng.floats((size_t)shape.offsetCount(), -0.4f, 0.4f);
    const auto mask = rng.floats((size_t)shape.maskCount(), 0.1f, 0.9f);
    const auto weight = rng.floats((size_t)shape.weightCount(), -0.2f, 0.2f);
    const auto bias = rng.floats((size_t)shape.outputChannels, -0.1f, 0.1f);
    const auto expected = cpuRun(shape, input, offset, mask, weight, bias);
    jasna::HipDeformConv runner;
    const auto actual = runner.runFloat32(shape, input, offset, mask, weight, bias);
    float maxAbs = 0;
    for (size_t i = 0; i < expected.size(); ++i) maxAbs = std::max(maxAbs, std::fabs(expected[i] - actual[i]));
    EXPECT(maxAbs < 2e-5f);
    EXPECT(std::memcmp(expected.data(), actual.data(), expected.size() * 4) == 0);
    std::printf("  correctness: max abs %.3g over %zu outputs\n", maxAbs, expected.size());
}

TEST(gpu, invalidArrayCountNamesTheArray) {
    jasna::HipDeformConv runner;
    const std::vector<float> zeros3(3, 0.0f), halfs((size_t)kOneByOne.maskCount(), 0.5f);
    const auto e = expectThrows([&] { runner.runFloat32(kOneByOne, {1, 2, 3, 4}, zeros3, halfs, {2}, {1}); });
    EXPECT(e.kind() == DeformConvError::Kind::invalidArrayCount);
    EXPECT(e.name() == "offset");
    EXPECT(e.expected() == kOneByOne.offsetCount());
    EXPECT(e.actual() == 3);
    DeformConvShape bad = kOneByOne;
    bad.groups = 0;
    EXPECT(expectThrows([&] { runner.runFloat32(bad, {1, 2, 3, 4}, zeros3, halfs, {2}, {1}); }).kind() ==
           DeformConvError::Kind::invalidShape);
}

TEST(gpu, metalNonFiniteFlagDetectsInfinity) {
    jasna::HipDeformConv runner;
    EXPECT(runner.flagNonFinite(toHalf({0, 1, -2, 0.5f})) == 0);
    EXPECT(runner.flagNonFinite(toHalf({0, INFINITY, 1})) == 1);
    EXPECT(runner.flagNonFinite(toHalf({0, NAN, 1})) == 1);
    EXPECT(expectThrows([&] { runner.flagNonFinite({}); }).kind() == DeformConvError::Kind::invalidShape);
}

TEST(gpu, jasnaShapeFloat16MatchesTheDirectOracleAndThePrepackedPath) {
    const DeformConvShape shape = jasna::jasnaShape();
    jasna::SeededGenerator rng(0x4A41534E41ull);
    const auto input = toHalf(rng.floats((size_t)shape.inputCount(), -1, 1));
    const auto offset = toHalf(rng.floats((size_t)shape.offsetCount(), -0.25f, 0.25f));
    const auto mask = toHalf(rng.floats((size_t)shape.maskCount(), 0.25f, 0.75f));
    const auto weight = toHalf(rng.floats((size_t)shape.weightCount(), -0.02f, 0.02f));
    const auto bias = toHalf(rng.floats(64, -0.02f, 0.02f));
    jasna::HipDeformConv runner;
    const auto direct = runner.runFloat16(shape, input, offset, mask, weight, bias);
    oracle_shape o;
    std::memcpy(&o, &shape, sizeof(o));
    std::vector<uint16_t> expected(direct.size());
    EXPECT(oracle_dcn_forward_f16_direct(&o, input.data(), offset.data(), mask.data(), weight.data(), bias.data(),
                                         expected.data()) == 0);
    EXPECT(direct == expected);
    const auto packed = runner.prepack(shape, weight, bias);
    const auto fused = toFloat(runner.runFloat16Prepacked(shape, input, offset, mask, packed));
    const auto base = toFloat(direct);
    float maxDiff = 0;
    for (size_t i = 0; i < fused.size(); ++i) maxDiff = std::max(maxDiff, std::fabs(fused[i] - base[i]));
    EXPECT(maxDiff <= 2e-3f);
}

TEST(gpu, weightSetLoadsAndRunsLikeItsUnpackedWeights) {
    const DeformConvShape shape = jasna::jasnaShape();
    jasna::SeededGenerator rng(7);
    const auto payload = toHalf(rng.floats(jasna::DeformConvWeightSet::weightElements + 64, -0.05f, 0.05f));
    std::vector<uint8_t> bytes(payload.size() * 2);
    std::memcpy(bytes.data(), payload.data(), bytes.size());
    const std::string dir = tempFile(bytes, "backward_1.dcnfp16");
    const jasna::DeformConvWeightSet set("backward_1", dir);
    // [ic][k][oc] -> OIHW
    std::vector<uint16_t> weight((size_t)shape.weightCount()), bias(payload.end() - 64, payload.end());
    for (int ic = 0; ic < 128; ++ic)
        for (int k = 0; k < 9; ++k)
            for (int oc = 0; oc < 64; ++oc) weight[((size_t)oc * 128 + ic) * 9 + k] = payload[((size_t)ic * 9 + k) * 64 + oc];
    const auto input = toHalf(rng.floats((size_t)shape.inputCount(), -1, 1));
    const auto offset = toHalf(rng.floats((size_t)shape.offsetCount(), -3, 3));
    const auto mask = toHalf(rng.floats((size_t)shape.maskCount(), 0, 1));
    jasna::HipDeformConv runner;
    const auto fromFile = runner.runFloat16Prepacked(shape, input, offset, mask, runner.loadWeightSet(set));
    const auto fromArrays = runner.runFloat16Prepacked(shape, input, offset, mask, runner.prepack(shape, weight, bias));
    EXPECT(fromFile == fromArrays);
    const auto direct = toFloat(runner.runFloat16(shape, input, offset, mask, weight, bias));
    const auto fused = toFloat(fromFile);
    float maxDiff = 0;
    for (size_t i = 0; i < fused.size(); ++i) maxDiff = std::max(maxDiff, std::fabs(fused[i] - direct[i]));
    EXPECT(maxDiff <= 2e-3f);
}

TEST(gpu, benchmarkJasnaShapeReportsGatedStatistics) {
    jasna::HipDeformConv runner;
    const auto r = runner.benchmarkJasnaShape(3);
    EXPECT(r.iterations == 3);
    EXPECT(r.fused.samples.size() == 3 && r.baseline.samples.size() == 3 && r.gather.samples.size() == 3);
    EXPECT(r.fused.minimum > 0 && std::isfinite(r.checksum));
    EXPECT(r.maxDifferenceFromBaseline <= 2e-3f);
    std::printf("  jasna shape: baseline median %.4f ms, gather %.4f ms, fused %.4f ms, checksum %.6f\n",
                r.baseline.median, r.gather.median, r.fused.median, r.checksum);
}

// Random SPyNet basic modules: He-uniform 7x7 weights for the ReLU layers, small ones for
// the flow layer (no checkpoint in this tree).
jasna::SPyNetWeights randomSPyNetWeights(uint64_t seed) {
    jasna::SeededGenerator rng(seed);
    jasna::SPyNetWeights w;
    auto half = [](const std::vector<float>& v) {
        std::vector<uint16_t> h(v.size());
        dcn_f32_to_f16_array(v.data(), h.data(), v.size());
        return h;
    };
    for (int l = 0; l < DCN_SPYNET_LEVELS; ++l)
        for (int i = 0; i < DCN_SPYNET_LAYERS; ++i) {
            const int cin = jasna::SPyNetWeights::layers[i][0], cout = jasna::SPyNetWeights::layers[i][1];
            const float bound = i + 1 < DCN_SPYNET_LAYERS ? std::sqrt(6.0f / (cin * 49.0f)) : 0.07f;
            w.weight[l][i] = half(rng.floats((size_t)cout * cin * 49, -bound, bound));
            w.bias[l][i] = half(rng.floats((size_t)cout, -0.01f, 0.01f));
        }
    return w;
}

TEST(gpu, verifySPyNetPairPassesItsGatesAndChecksAnOracle) {
    jasna::HipDeformConv runner;
    const auto weights = randomSPyNetWeights(0x5350594E4554ull);
    const auto r = runner.verifySPyNetPair(weights);
    EXPECT(r.iterations == 7 && r.elementCount == 2 * 2 * 4096);
    EXPECT(r.backwardMaximum > 0.001f && r.forwardMaximum > 0.001f);
    EXPECT(r.repeatMaximumError == 0.0f && r.oracleMaximumError == 0.0f);
    EXPECT(r.minimumMilliseconds <= r.medianMilliseconds && r.medianMilliseconds <= r.maximumMilliseconds);
    EXPECT(r.backwardFlow.size() == 2 * 4096 && r.forwardFlow.size() == 2 * 4096);
    EXPECT(std::isfinite(r.backwardChecksum) && std::isfinite(r.forwardChecksum));
    std::printf("  spynet pair: median %.4f ms, maxima %.3f / %.3f, checksums %.6f / %.6f\n", r.medianMilliseconds,
                r.backwardMaximum, r.forwardMaximum, r.backwardChecksum, r.forwardChecksum);
    // Oracle files in the reference's format (raw FP16 [2][64][64] per direction): this run's
    // own flows pass with error 0; one value moved by 0.25 px fails the 0.05 gate.
    char dir[] = "/tmp/spynet_oracle_XXXXXX";
    EXPECT(mkdtemp(dir) != nullptr);
    auto write = [&](const char* name, const std::vector<uint16_t>& v) {
        std::FILE* f = std::fopen((std::string(dir) + "/" + name).c_str(), "wb");
        EXPECT(f != nullptr);
        std::fwrite(v.data(), 2, v.size(), f);
        std::fclose(f);
    };
    write("backward.f16", r.backwardFlow);
    write("forward.f16", r.forwardFlow);
    const auto again = runner.verifySPyNetPair(weights, nullptr, nullptr, dir);
    EXPECT(again.oracleMaximumError == 0.0f && again.backwardChecksum == r.backwardChecksum);
    auto moved = r.forwardFlow;
    moved[100] = dcn_f32_to_f16(dcn_f16_to_f32(moved[100]) + 0.25f);
    write("forward.f16", moved);
    bool threw = false;
    try {
        runner.verifySPyNetPair(weights, nullptr, nullptr, dir);
    } catch (const jasna::DeformConvError& e) {
        threw = e.kind() == jasna::DeformConvError::Kind::commandFailed;
    }
    EXPECT(threw);
    std::remove((std::string(dir) + "/backward.f16").c_str());
    std::remove((std::string(dir) + "/forward.f16").c_str());
    rmdir(dir);
}

TEST(gpu, bicubicQuarterKeepsAConstantImageConstant) {
    jasna::HipDeformConv runner;
    const std::vector<uint16_t> in((size_t)3 * 256 * 256, dcn_f32_to_f16(0.375f));
    const auto out = runner.bicubicQuarter(3, 256, 256, in);
    EXPECT(out.size() == (size_t)3 * 64 * 64);
    for (uint16_t v : out) EXPECT(v == dcn_f32_to_f16(0.375f));
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 2 || (std::strcmp(argv[1], "cpu") != 0 && std::strcmp(argv[1], "gpu") != 0)) {
        std::fprintf(stderr, "usage: %s cpu|gpu\n", argv[0]);
        return 2;
    }
    int run = 0, failed = 0;
    for (const auto& t : registry()) {
        if (std::strcmp(t.group, argv[1]) != 0) continue;
        ++run;
        std::printf("[ RUN  ] %s\n", t.name);
        std::fflush(stdout);
        try {
            t.body();
            std::printf("[  OK  ] %s\n", t.name);
        } catch (const Failure& f) {
            ++failed;
            std::printf("[ FAIL ] %s: %s\n", t.name, f.what.c_str());
        } catch (const std::exception& e) {
            ++failed;
            std::printf("[ FAIL ] %s: unexpected exception: %s\n", t.name, e.what());
        }
        std::fflush(stdout);
    }
    std::printf("%d run, %d failed\n", run, failed);
    return failed ? 1 : 0;
}
