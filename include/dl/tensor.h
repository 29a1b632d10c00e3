#pragma once
// Tensor handle.  Mirrors the subset of include/dl/tensor.h:17-141 (reference) that the decoder token loop
// uses: metadata, host round trips (item / to_vector / from_span), dtype casts, device moves and views.
// A copied handle shares identity; views build a new layout over the same storage.  Arithmetic on GPU
// tensors runs in this library's HIP kernels; CPU tensors hold host data (parameters before `to`,
// inputs, and results read back) and only support layout, cast and transfer operations.

#include "dl/types.h"

#include <memory>
#include <optional>
#include <span>
#include <utility>

namespace dl {
namespace detail {
struct TensorImpl;
struct TensorAccess;
} // namespace detail

class DL_API Tensor {
public:
    const Shape& shape() const;
    const Shape& strides() const;
    Index size(Index axis) const;
    Index ndim() const;
    Index numel() const;
    /// Element offset from the start of the storage; data() already includes it.
    Index storage_offset() const;
    DType dtype() const;
    Device device() const;
    bool is_contiguous() const;
    bool requires_grad() const;

    /// Address of the first logical element on the tensor's device.
    template <class T> const T* data() const { return static_cast<const T*>(raw_data()); }

    /// Converts a one-element tensor to T on the host (blocking device-to-host read).
    template <class T> T item() const {
        Tensor value = to(Device::cpu()).astype(dtype_of<T>);
        return *value.data<T>();
    }

    /// Logical row-major copy on the host.
    template <class T> std::vector<T> to_vector() const {
        if (numel() == 0) return {};
        Tensor dense = to(Device::cpu()).astype(dtype_of<T>).contiguous();
        auto first = dense.data<T>();
        return std::vector<T>(first, first + numel());
    }

    Tensor clone() const;
    Tensor detach() const;
    Tensor contiguous() const;
    Tensor astype(DType dtype) const;
    /// Same device returns this handle; otherwise a contiguous copy on `device`.
    Tensor to(Device device) const;

    Tensor view(Shape shape) const;
    Tensor reshape(Shape shape) const;
    Tensor transpose(Index first, Index second) const;
    Tensor unsqueeze(Index axis) const;
    Tensor squeeze(Index axis) const;
    Tensor flatten(Index first = 0, Index last = -1) const;
    Tensor slice(Index axis, Index start, Index stop, Index step = 1) const;
    Tensor select(Index axis, Index index) const;
    Tensor narrow(Index axis, Index start, Index length) const;

    bool defined() const { return impl_ != nullptr; }
    Tensor() = default;

private:
    explicit Tensor(std::shared_ptr<detail::TensorImpl> impl) : impl_(std::move(impl)) {}
    const void* raw_data() const;

    std::shared_ptr<detail::TensorImpl> impl_;
    friend struct detail::TensorAccess;
};

DL_API Tensor full(Shape shape, double value, TensorOptions options = {});
DL_API Tensor zeros(Shape shape, TensorOptions options = {});
DL_API Tensor ones(Shape shape, TensorOptions options = {});
DL_API Tensor empty(Shape shape, TensorOptions options = {});

namespace detail {
DL_API Tensor from_host(const void* data, Shape shape, DType dtype, bool requires_grad, Device device);
}

/// Copies contiguous host values into an independent tensor on `device`.
template <class T>
Tensor from_span(std::span<const T> values, Shape shape, bool requires_grad = false,
                 Device device = Device::cpu()) {
    return detail::from_host(values.data(), std::move(shape), dtype_of<T>, requires_grad, device);
}

} // namespace dl
