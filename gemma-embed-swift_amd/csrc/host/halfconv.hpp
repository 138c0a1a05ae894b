// Host-side IEEE binary16 and bfloat16 conversions (round to nearest, ties to even).
#pragma once

#include <cstdint>
#include <cstring>

namespace ge {

inline float half_to_float(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while (!(man & 0x400u));
            bits = sign | (uint32_t(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

inline uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return uint16_t(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0));
    if (a >= 0x477ff000u) return uint16_t(sign | 0x7c00u);
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return uint16_t(sign);
        const uint32_t e = a >> 23, m = (a & 0x7fffffu) | 0x800000u, shift = 126 - e;
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1))) q++;
        return uint16_t(sign | q);
    }
    uint32_t q = (((a >> 23) - 112) << 10) | ((a & 0x7fffffu) >> 13);
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return uint16_t(sign | q);
}

inline uint16_t float_to_bf16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return uint16_t((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return uint16_t(x >> 16);
}

inline float bf16_to_float(uint16_t b) {
    const uint32_t x = uint32_t(b) << 16;
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

}  // namespace ge
