// Deterministic streams for synthetic models and inputs: SplitMix64 exactly as the reference
// tests' SeededRandom (Tests/GemmaEmbedTests/KernelTests.swift:9-26), plus Box-Muller Gaussians.
#pragma once

#include <cmath>
#include <cstdint>
#include <string>

namespace ge {

// SplitMix64's output function (Steele, Lea, Flood 2014).
inline uint64_t splitmix_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct SeededRandom {
    uint64_t state;
    explicit SeededRandom(uint64_t seed) : state(seed + 0x9E3779B97F4A7C15ull) {}
    uint64_t next() {
        state += 0x9E3779B97F4A7C15ull;
        return splitmix_mix(state);
    }
    // Uniform integer in [lo, hi) by 32-bit multiply-shift of the high word.
    int64_t uniform_int(int64_t lo, int64_t hi) {
        const uint64_t span = uint64_t(hi - lo);
        return lo + int64_t(((next() >> 32) * span) >> 32);
    }
    // Uniform in (0, 1] and [0, 1) with 53-bit resolution.
    double open_unit() { return double((next() >> 11) + 1) * 0x1.0p-53; }
    double unit() { return double(next() >> 11) * 0x1.0p-53; }
    // One N(0, 1) draw per call (Box-Muller, cosine branch; two uniforms).
    double gaussian() {
        const double u1 = open_unit();
        const double u2 = unit();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586476925286766559 * u2);
    }
};

// FNV-1a 64 of a name, for per-tensor seeds.
inline uint64_t fnv1a64(const std::string& s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 0x100000001b3ull;
    }
    return h;
}

// Seed of one tensor's stream: mix(seed ^ fnv1a64(name)).
inline uint64_t tensor_seed(uint64_t seed, const std::string& name) { return splitmix_mix(seed ^ fnv1a64(name)); }

}  // namespace ge
