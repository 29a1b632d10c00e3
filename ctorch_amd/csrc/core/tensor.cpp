// Tensor handle, views, casts and transfers (reference include/dl/tensor.h:17-141, src/core/tensor.cpp:11-84,
// src/core/layout.cpp:134-191).  GPU copies and casts run the strided copy kernel on the compute stream; host
// tensors use plain loops.
#include "core/tensor_impl.h"

#include <cstring>
#include <stdexcept>

namespace dl::detail {

Shape contiguous_strides(const Shape& shape) {
    Shape strides(shape.size());
    Index running = 1;
    for (std::size_t i = shape.size(); i-- > 0;) {
        strides[i] = running;
        running *= shape[i];
    }
    return strides;
}

std::string shape_string(const Shape& shape) {
    std::string out = "[";
    for (std::size_t i = 0; i < shape.size(); ++i) out += (i ? ", " : "") + std::to_string(shape[i]);
    return out + "]";
}

int dlk_dtype(DType dtype) {
    switch (dtype) {
    case DType::f32: return DLK_F32;
    case DType::f64: return DLK_F64;
    case DType::i64: return DLK_I64;
    case DType::boolean: return DLK_BOOL;
    case DType::bf16: return DLK_BF16;
    default: throw std::invalid_argument("f16 storage is not supported by this build");
    }
}

Tensor empty_tensor(const Shape& shape, DType dtype, Device device) {
    for (Index s : shape)
        if (s < 0) throw std::invalid_argument("tensor dimensions must be non-negative");
    auto impl = std::make_shared<TensorImpl>();
    impl->shape = shape;
    impl->strides = contiguous_strides(shape);
    impl->dtype = dtype;
    impl->storage = allocate_storage(static_cast<std::size_t>(impl->numel()) * element_size(dtype), device);
    return TensorAccess::make(std::move(impl));
}

void* mutable_data(const Tensor& t) { return TensorAccess::impl(t)->data(); }

namespace {

double host_load(const void* base, DType dtype, Index i) {
    switch (dtype) {
    case DType::f32: return static_cast<const float*>(base)[i];
    case DType::f64: return static_cast<const double*>(base)[i];
    case DType::i64: return static_cast<double>(static_cast<const Index*>(base)[i]);
    case DType::boolean: return static_cast<const bool*>(base)[i] ? 1.0 : 0.0;
    case DType::bf16: return BFloat16::decode(static_cast<const std::uint16_t*>(base)[i]);
    default: throw std::invalid_argument("unsupported dtype");
    }
}

void host_store(void* base, DType dtype, Index i, double v) {
    switch (dtype) {
    case DType::f32: static_cast<float*>(base)[i] = static_cast<float>(v); break;
    case DType::f64: static_cast<double*>(base)[i] = v; break;
    case DType::i64: static_cast<Index*>(base)[i] = static_cast<Index>(v); break;
    case DType::boolean: static_cast<bool*>(base)[i] = v != 0.0; break;
    case DType::bf16: static_cast<std::uint16_t*>(base)[i] = BFloat16::encode(static_cast<float>(v)); break;
    default: throw std::invalid_argument("unsupported dtype");
    }
}

void host_copy(const TensorImpl& dst, const TensorImpl& src) {
    const Index n = src.numel();
    const int rank = static_cast<int>(src.shape.size());
    const std::size_t es = element_size(src.dtype);
    std::vector<Index> index(static_cast<std::size_t>(rank), 0);
    char* dbase = static_cast<char*>(dst.storage->data);
    const char* sbase = static_cast<const char*>(src.storage->data);
    for (Index linear = 0; linear < n; ++linear) {
        Index so = src.offset, d = dst.offset;
        for (int a = 0; a < rank; ++a) {
            so += index[static_cast<std::size_t>(a)] * src.strides[static_cast<std::size_t>(a)];
            d += index[static_cast<std::size_t>(a)] * dst.strides[static_cast<std::size_t>(a)];
        }
        if (src.dtype == dst.dtype) {
            std::memcpy(dbase + d * static_cast<Index>(es), sbase + so * static_cast<Index>(es), es);
        } else if (src.dtype == DType::i64 && dst.dtype == DType::i64) {
            static_cast<Index*>(dst.storage->data)[d] = static_cast<const Index*>(src.storage->data)[so];
        } else {
            host_store(dbase, dst.dtype, d, host_load(sbase, src.dtype, so));
        }
        for (int a = rank - 1; a >= 0; --a) {
            if (++index[static_cast<std::size_t>(a)] < src.shape[static_cast<std::size_t>(a)]) break;
            index[static_cast<std::size_t>(a)] = 0;
        }
    }
}

bool dense(const TensorImpl& t) { return t.strides == contiguous_strides(t.shape); }

} // namespace

void copy_into(const Tensor& target, const Tensor& source) {
    const auto& dst = *TensorAccess::impl(target);
    const auto& src = *TensorAccess::impl(source);
    if (dst.shape != src.shape)
        throw std::invalid_argument("copy shape mismatch: " + shape_string(dst.shape) + " vs " + shape_string(src.shape));
    if (!(dst.device() == src.device())) throw std::invalid_argument("copy_into needs tensors on one device");
    if (src.numel() == 0) return;
    if (dst.device().type == DeviceType::cpu) {
        host_copy(dst, src);
        return;
    }
    GpuContext& context = gpu_context(dst.device().index);
    if (dst.dtype == src.dtype && dense(dst) && dense(src)) {
        hip_check(dlh_memcpy_async(dst.data(), src.data(), static_cast<std::size_t>(src.numel()) * element_size(src.dtype),
                                   DLH_DEVICE_TO_DEVICE, context.stream),
                  "copy");
        return;
    }
    hip_check(dlk_copy(src.data(), dlk_dtype(src.dtype), src.strides.data(), dst.data(), dlk_dtype(dst.dtype),
                       dst.strides.data(), src.shape.data(), static_cast<int>(src.shape.size()), context.stream),
              "copy kernel");
}

void rebind(const Tensor& tensor, const Tensor& value) {
    auto& impl = *TensorAccess::impl(tensor);
    const auto& source = *TensorAccess::impl(value);
    impl.storage = source.storage;
    impl.shape = source.shape;
    impl.strides = source.strides;
    impl.offset = source.offset;
    impl.dtype = source.dtype;
}

Tensor from_host(const void* data, Shape shape, DType dtype, bool requires_grad, Device device) {
    Tensor host = empty_tensor(shape, dtype, Device::cpu());
    const std::size_t bytes = static_cast<std::size_t>(TensorAccess::impl(host)->numel()) * element_size(dtype);
    if (bytes) std::memcpy(mutable_data(host), data, bytes);
    TensorAccess::impl(host)->requires_grad = requires_grad;
    if (device.type == DeviceType::cpu) return host;
    Tensor out = host.to(device);
    TensorAccess::impl(out)->requires_grad = requires_grad;
    return out;
}

} // namespace dl::detail

namespace dl {

using detail::TensorAccess;

namespace {
const detail::TensorImpl& get(const std::shared_ptr<detail::TensorImpl>& impl) {
    if (!impl) throw std::logic_error("undefined tensor");
    return *impl;
}
Index normalize_axis(Index axis, Index rank) {
    const Index a = axis < 0 ? axis + rank : axis;
    if (a < 0 || a >= rank) throw std::out_of_range("axis out of range");
    return a;
}
Tensor view_of(const detail::TensorImpl& base, Shape shape, Shape strides, Index offset) {
    auto impl = std::make_shared<detail::TensorImpl>();
    impl->storage = base.storage;
    impl->shape = std::move(shape);
    impl->strides = std::move(strides);
    impl->offset = offset;
    impl->dtype = base.dtype;
    impl->requires_grad = false;
    return TensorAccess::make(std::move(impl));
}
Shape resolve_shape(Shape shape, Index numel) {
    Index known = 1, infer = -1;
    for (std::size_t i = 0; i < shape.size(); ++i) {
        if (shape[i] == -1) {
            if (infer >= 0) throw std::invalid_argument("only one -1 is allowed in a shape");
            infer = static_cast<Index>(i);
        } else {
            known *= shape[i];
        }
    }
    if (infer >= 0) {
        if (known == 0 || numel % known != 0) throw std::invalid_argument("shape does not match the element count");
        shape[static_cast<std::size_t>(infer)] = numel / known;
    } else if (known != numel) {
        throw std::invalid_argument("shape does not match the element count");
    }
    return shape;
}
} // namespace

const Shape& Tensor::shape() const { return get(impl_).shape; }
const Shape& Tensor::strides() const { return get(impl_).strides; }
Index Tensor::size(Index axis) const { return shape()[static_cast<std::size_t>(normalize_axis(axis, ndim()))]; }
Index Tensor::ndim() const { return static_cast<Index>(shape().size()); }
Index Tensor::numel() const { return get(impl_).numel(); }
Index Tensor::storage_offset() const { return get(impl_).offset; }
DType Tensor::dtype() const { return get(impl_).dtype; }
Device Tensor::device() const { return get(impl_).device(); }
bool Tensor::is_contiguous() const { return get(impl_).strides == detail::contiguous_strides(shape()); }
bool Tensor::requires_grad() const { return get(impl_).requires_grad; }
const void* Tensor::raw_data() const { return get(impl_).data(); }

Tensor Tensor::clone() const {
    Tensor out = detail::empty_tensor(shape(), dtype(), device());
    detail::copy_into(out, *this);
    return out;
}
Tensor Tensor::detach() const {
    const auto& self = get(impl_);
    return view_of(self, self.shape, self.strides, self.offset);
}
Tensor Tensor::contiguous() const { return is_contiguous() ? *this : clone(); }

Tensor Tensor::astype(DType target) const {
    if (target == dtype()) return *this;
    Tensor out = detail::empty_tensor(shape(), target, device());
    detail::copy_into(out, *this);
    return out;
}

Tensor Tensor::to(Device target) const {
    if (target == device()) return *this;
    Tensor source = contiguous();
    const auto& src = get(TensorAccess::impl(source));
    Tensor out = detail::empty_tensor(src.shape, src.dtype, target);
    const std::size_t bytes = static_cast<std::size_t>(src.numel()) * element_size(src.dtype);
    if (bytes == 0) return out;
    if (target.type == DeviceType::gpu && src.device().type == DeviceType::cpu) {
        auto& context = detail::gpu_context(target.index);
        detail::hip_check(dlh_memcpy_async(detail::mutable_data(out), src.data(), bytes, DLH_HOST_TO_DEVICE,
                                           context.stream), "host to device copy");
        // the host source may be released as soon as this returns
        detail::hip_check(dlh_stream_synchronize(context.stream), "host to device copy");
    } else if (target.type == DeviceType::cpu && src.device().type == DeviceType::gpu) {
        auto& context = detail::gpu_context(src.device().index);
        detail::hip_check(dlh_memcpy_async(detail::mutable_data(out), src.data(), bytes, DLH_DEVICE_TO_HOST,
                                           context.stream), "device to host copy");
        detail::hip_check(dlh_stream_synchronize(context.stream), "device to host copy");
    } else {
        // GPU to GPU across devices: stage through the host
        return to(Device::cpu()).to(target);
    }
    return out;
}

Tensor Tensor::view(Shape new_shape) const {
    if (!is_contiguous()) throw std::invalid_argument("view needs a contiguous tensor; use reshape");
    const auto& self = get(impl_);
    Shape resolved = resolve_shape(std::move(new_shape), numel());
    Shape strides = detail::contiguous_strides(resolved);
    return view_of(self, std::move(resolved), std::move(strides), self.offset);
}

Tensor Tensor::reshape(Shape new_shape) const { return contiguous().view(std::move(new_shape)); }

Tensor Tensor::transpose(Index first, Index second) const {
    const auto& self = get(impl_);
    const Index a = normalize_axis(first, ndim()), b = normalize_axis(second, ndim());
    Shape shape = self.shape, strides = self.strides;
    std::swap(shape[static_cast<std::size_t>(a)], shape[static_cast<std::size_t>(b)]);
    std::swap(strides[static_cast<std::size_t>(a)], strides[static_cast<std::size_t>(b)]);
    return view_of(self, std::move(shape), std::move(strides), self.offset);
}

Tensor Tensor::unsqueeze(Index axis) const {
    const auto& self = get(impl_);
    const Index rank = ndim();
    const Index a = axis < 0 ? axis + rank + 1 : axis;
    if (a < 0 || a > rank) throw std::out_of_range("unsqueeze axis out of range");
    Shape shape = self.shape, strides = self.strides;
    const Index stride = a < rank ? self.strides[static_cast<std::size_t>(a)] * self.shape[static_cast<std::size_t>(a)] : 1;
    shape.insert(shape.begin() + a, 1);
    strides.insert(strides.begin() + a, stride);
    return view_of(self, std::move(shape), std::move(strides), self.offset);
}

Tensor Tensor::squeeze(Index axis) const {
    const auto& self = get(impl_);
    const Index a = normalize_axis(axis, ndim());
    if (self.shape[static_cast<std::size_t>(a)] != 1) return *this;
    Shape shape = self.shape, strides = self.strides;
    shape.erase(shape.begin() + a);
    strides.erase(strides.begin() + a);
    return view_of(self, std::move(shape), std::move(strides), self.offset);
}

Tensor Tensor::flatten(Index first, Index last) const {
    const Index rank = ndim();
    if (rank == 0) return reshape({1});
    const Index a = normalize_axis(first, rank), b = normalize_axis(last, rank);
    if (a > b) throw std::invalid_argument("flatten needs first <= last");
    Shape shape;
    for (Index i = 0; i < a; ++i) shape.push_back(this->shape()[static_cast<std::size_t>(i)]);
    Index merged = 1;
    for (Index i = a; i <= b; ++i) merged *= this->shape()[static_cast<std::size_t>(i)];
    shape.push_back(merged);
    for (Index i = b + 1; i < rank; ++i) shape.push_back(this->shape()[static_cast<std::size_t>(i)]);
    return reshape(std::move(shape));
}

Tensor Tensor::slice(Index axis, Index start, Index stop, Index step) const {
    const auto& self = get(impl_);
    const Index a = normalize_axis(axis, ndim());
    const Index size = self.shape[static_cast<std::size_t>(a)];
    if (step <= 0 || start < 0 || stop > size || start > stop) throw std::out_of_range("slice range out of bounds");
    Shape shape = self.shape, strides = self.strides;
    shape[static_cast<std::size_t>(a)] = (stop - start + step - 1) / step;
    strides[static_cast<std::size_t>(a)] *= step;
    return view_of(self, std::move(shape), std::move(strides), self.offset + start * self.strides[static_cast<std::size_t>(a)]);
}

Tensor Tensor::select(Index axis, Index index) const {
    const Index a = normalize_axis(axis, ndim());
    const Index size = shape()[static_cast<std::size_t>(a)];
    const Index i = index < 0 ? index + size : index;
    if (i < 0 || i >= size) throw std::out_of_range("select index out of range");
    return slice(a, i, i + 1).squeeze(a);
}

Tensor Tensor::narrow(Index axis, Index start, Index length) const {
    const Index a = normalize_axis(axis, ndim());
    const Index size = shape()[static_cast<std::size_t>(a)];
    const Index s = start < 0 ? start + size : start;
    if (length < 0 || s < 0 || s + length > size) throw std::out_of_range("narrow range out of bounds");
    return slice(a, s, s + length);
}

Tensor empty(Shape shape, TensorOptions options) { return detail::empty_tensor(shape, options.dtype, options.device); }

Tensor full(Shape shape, double value, TensorOptions options) {
    Tensor out = detail::empty_tensor(shape, options.dtype, options.device);
    const Index n = out.numel();
    if (options.device.type == DeviceType::cpu) {
        Tensor f64 = detail::empty_tensor(shape, DType::f64, Device::cpu());
        double* d = static_cast<double*>(detail::mutable_data(f64));
        for (Index i = 0; i < n; ++i) d[i] = value;
        detail::copy_into(out, f64);
    } else {
        auto& context = detail::gpu_context(options.device.index);
        detail::hip_check(dlk_fill(detail::mutable_data(out), detail::dlk_dtype(options.dtype), n, value, context.stream),
                          "fill");
    }
    detail::TensorAccess::impl(out)->requires_grad = options.requires_grad;
    return out;
}
Tensor zeros(Shape shape, TensorOptions options) { return full(std::move(shape), 0.0, options); }
Tensor ones(Shape shape, TensorOptions options) { return full(std::move(shape), 1.0, options); }

} // namespace dl
