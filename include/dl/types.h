#pragma once
// Scalar types, devices and tensor options.  Mirrors include/dl/types.h:10-57 of the reference.  The
// accelerator keeps the reference's API spelling (DeviceType::cuda, Device::cuda(i), value 1) so that the
// reference's callers compile unchanged; in this library it names HIP device i.  `gpu` is an alias of the
// same value.

#include "dl/export.h"
#include "dl/half.h"

#include <cstddef>
#include <cstdint>
#include <vector>

namespace dl {

using Index = std::int64_t;
using Shape = std::vector<Index>;

enum class DType : std::uint8_t { f32, f64, i64, boolean, f16, bf16 };
enum class DeviceType : std::uint8_t { cpu, cuda, gpu = cuda };
enum class KeepDim { no, yes };

/// Where a storage lives.  The CPU device has index zero; `cuda(i)` (alias `gpu(i)`) is HIP device i.
struct Device {
    DeviceType type = DeviceType::cpu;
    int index = 0;

    static constexpr Device cpu() { return {}; }
    static constexpr Device cuda(int index = 0) { return {DeviceType::cuda, index}; }
    static constexpr Device gpu(int index = 0) { return cuda(index); }
    bool operator==(const Device&) const = default;
};

struct TensorOptions {
    DType dtype = DType::f32;
    Device device = Device::cpu();
    bool requires_grad = false;
};

/// Waits for the work already submitted to `device`; CPU work is complete on return.
DL_API void synchronize(Device device);

constexpr std::size_t element_size(DType dtype) {
    constexpr std::size_t sizes[] = {4, 8, 8, 1, 2, 2};
    return sizes[static_cast<std::size_t>(dtype)];
}

constexpr bool is_low_precision(DType dtype) { return dtype == DType::f16 || dtype == DType::bf16; }
constexpr bool is_floating(DType dtype) {
    return dtype == DType::f32 || dtype == DType::f64 || is_low_precision(dtype);
}
/// Low-precision storage computes and returns f32 (reference include/dl/types.h:44-46).
constexpr DType accumulation_dtype(DType dtype) { return is_low_precision(dtype) ? DType::f32 : dtype; }

template <class T> struct DTypeOf;
template <> struct DTypeOf<float> { static constexpr auto value = DType::f32; };
template <> struct DTypeOf<double> { static constexpr auto value = DType::f64; };
template <> struct DTypeOf<Index> { static constexpr auto value = DType::i64; };
template <> struct DTypeOf<bool> { static constexpr auto value = DType::boolean; };
template <> struct DTypeOf<BFloat16> { static constexpr auto value = DType::bf16; };
template <class T> inline constexpr DType dtype_of = DTypeOf<T>::value;

} // namespace dl
