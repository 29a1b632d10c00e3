// Tensor internals: a storage plus a strided layout (shape, strides and offset in elements).
// Mirrors the reference's TensorData/Storage/Layout split (src/core/tensor_data.h:11-66, layout.h:36-48).
#pragma once

#include "core/device.h"
#include "dl/tensor.h"

#include <memory>

namespace dl::detail {

struct TensorImpl {
    std::shared_ptr<Storage> storage;
    Shape shape, strides;
    Index offset = 0;
    DType dtype = DType::f32;
    bool requires_grad = false;

    Index numel() const {
        Index n = 1;
        for (Index s : shape) n *= s;
        return n;
    }
    void* data() const {
        return static_cast<char*>(storage->data) + static_cast<std::ptrdiff_t>(offset) *
                                                       static_cast<std::ptrdiff_t>(element_size(dtype));
    }
    Device device() const { return storage->device; }
};

struct TensorAccess {
    static Tensor make(std::shared_ptr<TensorImpl> impl) { return Tensor(std::move(impl)); }
    static const std::shared_ptr<TensorImpl>& impl(const Tensor& t) { return t.impl_; }
};

Shape contiguous_strides(const Shape& shape);
/// A new contiguous tensor with uninitialised (host: zeroed) storage.
Tensor empty_tensor(const Shape& shape, DType dtype, Device device);
/// Mutable device/host address of the first element.
void* mutable_data(const Tensor& t);
int dlk_dtype(DType dtype);
/// Copies `source` (any layout, any dtype) into `target` (any layout, same shape, same device), converting
/// dtype.  GPU tensors copy with one kernel on the compute stream.
void copy_into(const Tensor& target, const Tensor& source);
/// Makes `tensor` refer to `value`'s storage and layout in place (identity kept for all handles).
void rebind(const Tensor& tensor, const Tensor& value);
std::string shape_string(const Shape& shape);
/// A counter that module weight loads and device moves advance (Module::load_state_dict, Module::to): caches
/// derived from parameter values (the repacked projection weights of the batched decode) are valid while it
/// stays where it was when they were built.  Writes through a raw data pointer do not advance it.
uint64_t parameter_epoch();
void advance_parameter_epoch();

} // namespace dl::detail
