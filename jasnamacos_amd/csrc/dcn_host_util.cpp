// Host-side utilities of the C ABI: FP16 conversion, the seeded generator, the
// benchmark-configuration input generators, the benchmark checksum and statistics.
#include <cmath>
#include <cstring>
#include <vector>
#include <algorithm>

#include "dcn_internal.hpp"

namespace dcn {

// Round-to-nearest-even binary32 -> binary16 by integer arithmetic on the bit pattern.
uint16_t f32_to_f16_bits(float value) {
    uint32_t x;
    std::memcpy(&x, &value, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t abs = x & 0x7fffffffu;
    if (abs >= 0x7f800000u) return sign | (abs > 0x7f800000u ? 0x7e00u : 0x7c00u);
    if (abs >= 0x477ff000u) return sign | 0x7c00u;  // >= 65520 rounds to Inf
    if (abs < 0x38800000u) {                        // below 2^-14: subnormal half or zero
        if (abs < 0x33000000u) return sign;         // < 2^-25 -> 0 (2^-25 itself ties to 0)
        const uint32_t e = abs >> 23;
        const uint32_t m = (abs & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;            // 14..24 for e in 102..112
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        h += (rem > half) || (rem == half && (h & 1u));
        return sign | (uint16_t)h;
    }
    // normal: rebias exponent, round the 13 dropped bits to nearest even
    uint32_t h = (abs - 0x38000000u) >> 13;
    const uint32_t rem = abs & 0x1fffu;
    h += (rem > 0x1000u) || (rem == 0x1000u && (h & 1u));
    return sign | (uint16_t)h;
}

float f16_bits_to_f32(uint16_t bits) {
    const uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    const uint32_t e = (bits >> 10) & 0x1fu;
    const uint32_t m = bits & 0x3ffu;
    float f;
    if (e == 0) {
        f = std::ldexp((float)m, -24);  // exact: m < 2^10
        uint32_t x;
        std::memcpy(&x, &f, 4);
        x |= sign;
        std::memcpy(&f, &x, 4);
        return f;
    }
    const uint32_t x = sign | (e == 31 ? (0x7f800000u | (m << 13)) : (((e + 112u) << 23) | (m << 13)));
    std::memcpy(&f, &x, 4);
    return f;
}

namespace {

// N(0,1) by the polar-free Box-Muller transform over SplitMix64 doubles; pairs cached.
struct Gaussian {
    uint64_t state;
    bool has_spare = false;
    double spare = 0.0;
    explicit Gaussian(uint64_t seed) : state(dcn_splitmix64_seed(seed)) {}
    double uniform() {  // [0, 1) with 53 random bits
        return (double)(dcn_splitmix64_next(&state) >> 11) * 0x1.0p-53;
    }
    double normal() {
        if (has_spare) {
            has_spare = false;
            return spare;
        }
        const double u1 = uniform();
        const double u2 = uniform();
        const double r = std::sqrt(-2.0 * std::log1p(-u1));
        const double t = 6.283185307179586 * u2;
        spare = r * std::sin(t);
        has_spare = true;
        return r * std::cos(t);
    }
};

struct ConfigSpec {
    dcn_shape shape;
    double flow_px;      // flow grid values ~ U(-flow_px, flow_px)
    double noise_sigma;  // offsets 10*tanh(N(0, sigma))
    double hard_mask;    // fraction of mask sites forced to sigmoid(+-20)
};

bool config_spec(int config, ConfigSpec* spec) {
    dcn_shape s{1, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16};
    switch (config) {
        case 1:
        case 2:
            *spec = ConfigSpec{s, 6.0, 1.0, 0.0};
            return true;
        case 3:
            s.batch = 16;
            *spec = ConfigSpec{s, 12.0, 1.0, 0.0};
            return true;
        case 5:
            s.input_height = s.output_height = 180;
            s.input_width = s.output_width = 320;
            *spec = ConfigSpec{s, 32.0, 2.0, 0.1};
            return true;
        default:
            return false;
    }
}

}  // namespace
}  // namespace dcn

extern "C" {

uint64_t dcn_splitmix64_seed(uint64_t seed) {
    // SeededGenerator.init (DeformConv.swift:171-173)
    return seed == 0 ? 0x9E3779B97F4A7C15ull : seed;
}

uint64_t dcn_splitmix64_next(uint64_t* state) {
    // SeededGenerator.next (DeformConv.swift:175-181)
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void dcn_seeded_floats(uint64_t* state, size_t count, float lo, float hi, float* out) {
    // Swift's BinaryFloatingPoint.random(in: ClosedRange, using:) for Float: a
    // significand-sized integer r in [0, 2^24] from next(upperBound: 2^24 + 1)
    // (Lemire's nearly divisionless method on UInt32 = low 32 bits of next()),
    // r == 2^24 returns the upper bound, otherwise delta * (r * 2^-24) + lo.
    const float delta = hi - lo;
    const uint32_t bound = (1u << 24) + 1u;
    for (size_t i = 0; i < count; ++i) {
        uint32_t random = (uint32_t)dcn_splitmix64_next(state);
        uint64_t m = (uint64_t)random * bound;
        if ((uint32_t)m < bound) {
            const uint32_t t = (0u - bound) % bound;
            while ((uint32_t)m < t) {
                random = (uint32_t)dcn_splitmix64_next(state);
                m = (uint64_t)random * bound;
            }
        }
        const uint32_t r = (uint32_t)(m >> 32);
        if (r == (1u << 24)) {
            out[i] = hi;
            continue;
        }
        const float unit = (float)r * 0x1.0p-24f;
        const float product = delta * unit;
        out[i] = product + lo;
    }
}

dcn_status dcn_config_shape(int config, dcn_shape* out) {
    if (!out) return DCN_INVALID_ARGUMENT;
    dcn::ConfigSpec spec;
    if (!dcn::config_spec(config, &spec)) return DCN_INVALID_SHAPE;
    *out = spec.shape;
    return DCN_OK;
}

dcn_status dcn_generate_config_inputs(int config, uint64_t seed, float* input, size_t input_count,
                                      float* offset, size_t offset_count, float* mask,
                                      size_t mask_count, float* weight, size_t weight_count,
                                      float* bias, size_t bias_count) {
    dcn::ConfigSpec spec;
    if (!dcn::config_spec(config, &spec)) return DCN_INVALID_SHAPE;
    dcn_counts c;
    if (dcn_shape_counts(&spec.shape, &c) != DCN_OK) return DCN_INVALID_SHAPE;
    if (input_count != c.input || offset_count != c.offset || mask_count != c.mask ||
        weight_count != c.weight || bias_count != c.bias)
        return DCN_INVALID_ARRAY_COUNT;
    if (!input || !offset || !mask || !weight || !bias) return DCN_INVALID_ARGUMENT;
    const dcn_shape& s = spec.shape;
    dcn::Gaussian rng(seed);
    for (size_t i = 0; i < c.input; ++i) input[i] = (float)rng.normal();
    // He-uniform bound sqrt(6 / fan_in), fan_in = Cin/groups * Kh * Kw.
    const double fan_in = (double)(s.input_channels / s.groups) * s.kernel_height * s.kernel_width;
    const double bound = std::sqrt(6.0 / fan_in);
    for (size_t i = 0; i < c.weight; ++i) weight[i] = (float)((2.0 * rng.uniform() - 1.0) * bound);
    for (size_t i = 0; i < c.bias; ++i) bias[i] = (float)((2.0 * rng.uniform() - 1.0) * 0.1);

    const int ho = s.output_height, wo = s.output_width;
    const size_t plane = (size_t)ho * wo;
    const size_t points = (size_t)s.offset_groups * c.kernel_area;  // (g, tap) pairs
    std::vector<float> flow_y(plane), flow_x(plane);
    for (int n = 0; n < s.batch; ++n) {
        // Smooth flow: an 8x8 grid per component, bilinearly upsampled (align_corners).
        double gy[64], gx[64];
        for (int i = 0; i < 64; ++i) gy[i] = (2.0 * rng.uniform() - 1.0) * spec.flow_px;
        for (int i = 0; i < 64; ++i) gx[i] = (2.0 * rng.uniform() - 1.0) * spec.flow_px;
        for (int oy = 0; oy < ho; ++oy) {
            const double sy = ho > 1 ? oy * 7.0 / (ho - 1) : 0.0;
            const int y0 = std::min((int)sy, 6);
            const double ty = sy - y0;
            for (int ox = 0; ox < wo; ++ox) {
                const double sx = wo > 1 ? ox * 7.0 / (wo - 1) : 0.0;
                const int x0 = std::min((int)sx, 6);
                const double tx = sx - x0;
                auto lerp2 = [&](const double* g) {
                    const double a = g[y0 * 8 + x0] * (1 - tx) + g[y0 * 8 + x0 + 1] * tx;
                    const double b = g[(y0 + 1) * 8 + x0] * (1 - tx) + g[(y0 + 1) * 8 + x0 + 1] * tx;
                    return a * (1 - ty) + b * ty;
                };
                flow_y[(size_t)oy * wo + ox] = (float)lerp2(gy);
                flow_x[(size_t)oy * wo + ox] = (float)lerp2(gx);
            }
        }
        float* off = offset + (size_t)n * 2 * points * plane;
        for (size_t ch = 0; ch < 2 * points; ++ch) {
            const std::vector<float>& flow = (ch % 2 == 0) ? flow_y : flow_x;  // dy, dx
            for (size_t p = 0; p < plane; ++p)
                off[ch * plane + p] =
                    (float)(10.0 * std::tanh(spec.noise_sigma * rng.normal()) + flow[p]);
        }
    }
    for (size_t i = 0; i < c.mask; ++i) {
        double z = rng.normal();
        if (spec.hard_mask > 0.0 && rng.uniform() < spec.hard_mask)
            z = rng.uniform() < 0.5 ? -20.0 : 20.0;
        mask[i] = (float)(1.0 / (1.0 + std::exp(-z)));
    }
    return DCN_OK;
}

uint16_t dcn_f32_to_f16(float value) { return dcn::f32_to_f16_bits(value); }
float dcn_f16_to_f32(uint16_t bits) { return dcn::f16_bits_to_f32(bits); }
void dcn_f32_to_f16_array(const float* in, uint16_t* out, size_t count) {
    for (size_t i = 0; i < count; ++i) out[i] = dcn::f32_to_f16_bits(in[i]);
}
void dcn_f16_to_f32_array(const uint16_t* in, float* out, size_t count) {
    for (size_t i = 0; i < count; ++i) out[i] = dcn::f16_bits_to_f32(in[i]);
}

double dcn_checksum_f32(const float* values, size_t count) {
    // MetalRunner.swift:332-337: stride 257, summed in Double
    double sum = 0.0;
    for (size_t i = 0; i < count; i += 257) sum += (double)values[i];
    return sum;
}

double dcn_checksum_f16(const uint16_t* values, size_t count) {
    double sum = 0.0;
    for (size_t i = 0; i < count; i += 257) sum += (double)dcn::f16_bits_to_f32(values[i]);
    return sum;
}

dcn_status dcn_compute_statistics(const double* samples, size_t count, dcn_statistics* out) {
    // BenchmarkStatistics.init (BenchmarkStatistics.swift:13-34)
    if (!samples || !out || count == 0) return DCN_INVALID_ARGUMENT;
    std::vector<double> v(samples, samples + count);
    for (double x : v)
        if (!std::isfinite(x)) return DCN_INVALID_ARGUMENT;
    std::sort(v.begin(), v.end());
    double total = 0.0;
    for (double x : v) total += x;
    const double mean = total / (double)count;
    double var = 0.0;
    for (double x : v) var += (x - mean) * (x - mean);
    var /= (double)count;
    auto percentile = [&](double fraction) {
        // BenchmarkStatistics.swift:36-43
        if (count < 2) return v[0];
        const double position = fraction * (double)(count - 1);
        const size_t lower = (size_t)std::floor(position);
        const size_t upper = (size_t)std::ceil(position);
        const double w = position - (double)lower;
        return v[lower] * (1 - w) + v[upper] * w;
    };
    out->minimum = v.front();
    out->maximum = v.back();
    out->median = (count % 2 == 0) ? (v[count / 2 - 1] + v[count / 2]) / 2 : v[count / 2];
    out->mean = mean;
    out->standard_deviation = std::sqrt(var);
    out->percentile10 = percentile(0.10);
    out->percentile90 = percentile(0.90);
    out->count = count;
    return DCN_OK;
}

}  // extern "C"

extern "C" {

dcn_status dcn_temporal_schedule(int frame_count, dcn_schedule_step* steps, size_t capacity,
                                 size_t* count) {
    if (frame_count <= 0) return DCN_INVALID_SHAPE;
    const size_t total = 4 * (size_t)frame_count;
    if (count) *count = total;
    if (!steps || capacity < total) return DCN_INVALID_ARGUMENT;
    size_t i = 0;
    for (int b = 0; b < 4; ++b) {
        const bool backward = b % 2 == 0;  // backward_1, forward_1, backward_2, forward_2
        auto frame_at = [&](int position) { return backward ? frame_count - 1 - position : position; };
        for (int p = 0; p < frame_count; ++p) {
            dcn_schedule_step& st = steps[i++];
            st.branch = b;
            st.position = p;
            st.frame = frame_at(p);
            st.flow_index = p == 0 ? -1 : (backward ? st.frame : st.frame - 1);
            st.second_order_frame = p > 1 ? frame_at(p - 2) : -1;
        }
    }
    return DCN_OK;
}

size_t dcn_schedule_persistent_bytes(int frame_count) {
    if (frame_count <= 0) return 0;
    const size_t fp16 = 2, t = (size_t)frame_count;
    const size_t lq = t * 3 * 256 * 256 * fp16;
    const size_t features = t * 5 * 64 * 64 * 64 * fp16;
    const size_t flows = 2 * (t - 1) * 2 * 64 * 64 * fp16;
    return lq + features + flows;
}

dcn_status dcn_temporal_chunk_ranges(int frame_count, int max_frames_per_chunk, int* starts,
                                     int* sizes, size_t capacity, size_t* count) {
    if (frame_count < 3 || max_frames_per_chunk < 3) return DCN_INVALID_SHAPE;
    const int requested = (frame_count + max_frames_per_chunk - 1) / max_frames_per_chunk;
    const int chunks = std::max(1, std::min(requested, frame_count / 3));
    if (count) *count = (size_t)chunks;
    if (!starts || !sizes || capacity < (size_t)chunks) return DCN_INVALID_ARGUMENT;
    const int base = frame_count / chunks, larger = frame_count % chunks;
    int start = 0;
    for (int i = 0; i < chunks; ++i) {
        const int size = base + (i < larger ? 1 : 0);
        starts[i] = start;
        sizes[i] = size;
        start += size;
    }
    return DCN_OK;
}

}  // extern "C"
