#pragma once
// Explicit-key randomness.  Mirrors include/dl/random.h:14-22,113-115 of the reference: a RandomKey selects
// the Philox4x32-10 round key (seed) and the high 64 counter bits (stream); the element number is the low
// 64 bits.  Integer outputs are identical on every device by construction.

#include "dl/tensor.h"

#include <array>

namespace dl {

struct RandomKey {
    std::uint64_t seed, stream = 0;
    bool operator==(const RandomKey&) const = default;
};

/// Derives a new key from a label; the input key is unchanged (reference src/core/random.cpp:14-18).
DL_API RandomKey fold_in(RandomKey key, std::uint64_t label) noexcept;
DL_API std::array<RandomKey, 2> split(RandomKey key) noexcept;
DL_API std::vector<RandomKey> split(RandomKey key, std::size_t count);

/// Keyed uniform [low, high) and standard normal, generated on `options.device`.
DL_API Tensor uniform(RandomKey key, Shape shape, double low, double high, TensorOptions options = {});
DL_API Tensor randn(RandomKey key, Shape shape, TensorOptions options = {});
/// scale * randn(key), rounded once to options.dtype (no reference counterpart: fuses randn and scale
/// for seeded weight synthesis of large models directly in device memory).
DL_API Tensor normal(RandomKey key, Shape shape, double scale, TensorOptions options = {});

} // namespace dl
