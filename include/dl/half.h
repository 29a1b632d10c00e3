#pragma once
// bf16 storage codec: f32 -> bf16 rounds to nearest even and quiets NaN; bf16 -> f32 is an exact shift
// (reference include/dl/half.h:43-47,60-66).  The same integer rules run in the device kernels.

#include <cstdint>
#include <cstring>

namespace dl {

struct BFloat16 {
    std::uint16_t bits = 0;

    BFloat16() = default;
    explicit BFloat16(float value) : bits(encode(value)) {}
    explicit operator float() const { return decode(bits); }

    static std::uint16_t encode(float value) {
        std::uint32_t b;
        std::memcpy(&b, &value, 4);
        if ((b & 0x7fffffffu) > 0x7f800000u) return static_cast<std::uint16_t>((b >> 16) | 0x40u);
        return static_cast<std::uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
    }
    static float decode(std::uint16_t value) {
        const std::uint32_t b = static_cast<std::uint32_t>(value) << 16;
        float result;
        std::memcpy(&result, &b, 4);
        return result;
    }
};

} // namespace dl
