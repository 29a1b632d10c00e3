// KV cache (reference src/nn/kv_cache.cpp:9-42).  Storage [.., capacity, D] is allocated by the first append (or
// by the fused decode path's reserve), appends copy along the second-to-last axis, key()/value() are narrow views
// and clear/truncate only move the length.  On a GPU the length is mirrored in an i64 device word that the
// fused kernels read (RoPE position, KV slot, attention length) and advance, so that a captured step needs no
// host-side arguments.
#include "nn/ops_internal.h"

#include <stdexcept>

namespace dl::nn {

using namespace dl::detail;

KVCache::KVCache(Index capacity) : capacity_(capacity) {
    if (capacity <= 0) throw std::invalid_argument("KV cache capacity must be positive");
}

void KVCache::sync_position() const {
    if (!position_) return;
    auto& context = gpu_context(position_->device().index);
    hip_check(dlk_fill(mutable_data(*position_), DLK_I64, 1, static_cast<double>(length_), context.stream),
              "KV cache length");
}

void KVCache::check_layout(Index batch, Index heads, Index head_dim, DType dtype, Device device) const {
    if (!key_) return;
    // the fused kernels write and read both tensors with the layer's shape and dtype: a cache whose key or
    // value storage (each taken from its own first append) differs must fail here, before any launch
    const Shape shape{batch, heads, capacity_, head_dim};
    auto differs = [&](const std::optional<Tensor>& storage) {
        return !storage || storage->shape() != shape || storage->dtype() != dtype || !(storage->device() == device);
    };
    if (differs(key_) || differs(value_) || (device.type == DeviceType::gpu && !position_))
        throw std::invalid_argument("KV cache shape, dtype or device changed");
}

void KVCache::reserve(Index batch, Index heads, Index head_dim, DType dtype, Device device) {
    check_layout(batch, heads, head_dim, dtype, device);
    if (key_) return;
    const Shape shape{batch, heads, capacity_, head_dim};
    key_ = empty_tensor(shape, dtype, device);
    value_ = empty_tensor(shape, dtype, device);
    if (device.type == DeviceType::gpu) {
        position_ = empty_tensor({1}, DType::i64, device);
        sync_position();
    }
}

void KVCache::append(const Tensor& key, const Tensor& value) {
    if (key.ndim() < 2 || value.ndim() != key.ndim()) throw std::invalid_argument("KV cache append needs [.., n, D]");
    const auto count = key.size(-2);
    if (count != value.size(-2) || count > capacity_ - length_)
        throw std::invalid_argument("KV cache append exceeds capacity or has unequal key/value lengths");
    // as in the reference: key and value storage each take their input's shape (capacity rows), dtype and device
    // on the first append, and a later append that differs in any of them throws
    auto storage_shape = [&](const Tensor& input) {
        Shape shape = input.shape();
        shape[shape.size() - 2] = capacity_;
        return shape;
    };
    if (!key_) {
        if (!(key.device() == value.device())) throw std::invalid_argument("KV cache shape, dtype or device changed");
        key_ = empty_tensor(storage_shape(key), key.dtype(), key.device());
        value_ = empty_tensor(storage_shape(value), value.dtype(), value.device());
        if (key.device().type == DeviceType::gpu) position_ = empty_tensor({1}, DType::i64, key.device());
    } else {
        auto differs = [&](const Tensor& input, const Tensor& storage) {
            return storage.shape() != storage_shape(input) || storage.dtype() != input.dtype() ||
                   !(storage.device() == input.device());
        };
        if (differs(key, *key_) || differs(value, *value_))
            throw std::invalid_argument("KV cache shape, dtype or device changed");
    }
    copy_into(key_->narrow(-2, length_, count), key);
    copy_into(value_->narrow(-2, length_, count), value);
    length_ += count;
    sync_position();
}

Tensor KVCache::key() const {
    if (!key_) throw std::logic_error("KV cache has no key tensor before its first append");
    return key_->narrow(-2, 0, length_);
}

Tensor KVCache::value() const {
    if (!value_) throw std::logic_error("KV cache has no value tensor before its first append");
    return value_->narrow(-2, 0, length_);
}

void KVCache::clear() {
    length_ = 0;
    sync_position();
}

void KVCache::truncate(Index length) {
    if (length < 0 || length > length_) throw std::out_of_range("KV cache truncation must keep an existing prefix");
    length_ = length;
    sync_position();
}

void* KVCache::key_data() const { return key_ ? mutable_data(*key_) : nullptr; }
void* KVCache::value_data() const { return value_ ? mutable_data(*value_) : nullptr; }
std::int64_t* KVCache::position_data() const {
    return position_ ? static_cast<std::int64_t*>(mutable_data(*position_)) : nullptr;
}

} // namespace dl::nn
