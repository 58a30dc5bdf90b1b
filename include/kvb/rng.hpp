// Library-independent random streams for workloads and block tables. The engine is
// std::mt19937_64, whose output sequence the C++ standard fixes; every mapping from its 64-bit
// draws to floats and ranges is explicit here, so a seed means the same numbers on any standard
// library (the reference's uniform_real_distribution / std::shuffle streams are
// implementation-defined, src/workload.hpp:38-39, src/reference.cpp:21).
#pragma once

#include <cmath>
#include <cstdint>
#include <random>

namespace kvb::rng {

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

// Independent stream `index` of kind `tag` under `seed`.
enum Tag : uint64_t { kQuery = 1, kKeyValue = 2, kAmplitude = 3 };
inline std::mt19937_64 stream(uint64_t seed, Tag tag, uint64_t index) {
    return std::mt19937_64(splitmix64(seed ^ splitmix64((uint64_t(tag) << 56) ^ index)));
}

// Uniform in (-1, 1): the top 24 bits of a draw, centred: (k + 0.5) * 2^-23 - 1.
inline float uniform_pm1(uint64_t x) { return float((double(x >> 40) + 0.5) * 0x1p-23 - 1.0); }

// Uniform integer in [0, n): high 64 bits of draw * n.
inline uint64_t below(uint64_t x, uint64_t n) { return uint64_t((unsigned __int128)x * n >> 64); }

// Two N(0,1) values from two draws (Box-Muller in fp64: u1 in (0, 1], u2 in [0, 1)).
inline void normal_pair(uint64_t a, uint64_t b, float& z0, float& z1) {
    const double u1 = (double(a >> 11) + 1.0) * 0x1p-53;
    const double u2 = double(b >> 11) * 0x1p-53;
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double th = 6.283185307179586476925 * u2;
    z0 = float(r * std::cos(th));
    z1 = float(r * std::sin(th));
}

}  // namespace kvb::rng
