// Deterministic synthetic data: SplitMix64 streams and Box-Muller normals.
// A stream starts at seed ^ (stream+1)*0xD1B54A32D192ED03; each pair of
// outputs (a, b) gives u1 = ((a>>11)+1)*2^-53 in (0,1], u2 = (b>>11)*2^-53,
// r = sqrt(-2 ln u1), and the normals r*cos(2*pi*u2), r*sin(2*pi*u2) in
// double, scaled by stddev and rounded to float. Token ids are outputs
// modulo the vocabulary.
#pragma once
#include <cmath>
#include <cstddef>
#include <cstdint>

namespace miniprefix {
namespace synthetic {

inline std::uint64_t next(std::uint64_t& state) {
    std::uint64_t z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline std::uint64_t stream(std::uint64_t seed, std::uint64_t id) { return seed ^ ((id + 1ull) * 0xD1B54A32D192ED03ull); }

inline void normal(float* dst, std::size_t count, std::uint64_t seed, std::uint64_t id, double stddev) {
    std::uint64_t state = stream(seed, id);
    const double two_pi = 6.283185307179586476925286766559;
    std::size_t i = 0;
    while (i < count) {
        const std::uint64_t a = next(state), b = next(state);
        const double u1 = static_cast<double>((a >> 11) + 1) * 0x1.0p-53;
        const double u2 = static_cast<double>(b >> 11) * 0x1.0p-53;
        const double r = std::sqrt(-2.0 * std::log(u1)), theta = two_pi * u2;
        dst[i++] = static_cast<float>(stddev * (r * std::cos(theta)));
        if (i < count) dst[i++] = static_cast<float>(stddev * (r * std::sin(theta)));
    }
}

inline void tokens(std::int32_t* dst, std::size_t count, std::uint64_t seed, std::uint64_t id, std::int32_t vocabulary) {
    std::uint64_t state = stream(seed, id);
    for (std::size_t i = 0; i < count; ++i)
        dst[i] = static_cast<std::int32_t>(next(state) % static_cast<std::uint64_t>(vocabulary));
}

}  // namespace synthetic
}  // namespace miniprefix
