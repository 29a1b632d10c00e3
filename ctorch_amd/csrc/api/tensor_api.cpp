// Tensor, operator, randomness and device entries of <dl/c_api.h> (reference src/api/tensor.cpp:9-100,273,449,
// 465,581-586, src/api/statistics.cpp:16-22).
#include "api/common.h"
#include "core/tensor_impl.h"
#include "dl/autograd.h"
#include "dl/gpu.h"

#include <cstring>
#include <string>

using namespace dl::capi;

namespace dl::capi {
namespace {
thread_local std::string error_buffer;
}
void set_error(const char* message) noexcept {
    try {
        error_buffer.assign(message ? message : "");
        if (error_buffer.size() > 2047) error_buffer.resize(2047);
    } catch (...) {
    }
}
const char* error_text() noexcept { return error_buffer.c_str(); }
} // namespace dl::capi

extern "C" {

const char* dl_version(void) { return "ctorch-amd 0.1.0 (gfx950)"; }
const char* dl_last_error(void) { return error_text(); }
dl_tensor_options dl_default_tensor_options(void) { return {DL_F32, {DL_CPU, 0}, 0}; }

void dl_tensor_release(dl_tensor* tensor) { delete tensor; }

dl_status dl_tensor_retain(const dl_tensor* tensor, dl_tensor** output) {
    return make_handle(output, [&] { return require(tensor, "tensor").value; });
}

dl_tensor_info dl_tensor_get_info(const dl_tensor* tensor) {
    dl_tensor_info info{};
    if (!tensor || !tensor->value.defined()) return info;
    const auto& t = tensor->value;
    info.dtype = static_cast<dl_dtype>(t.dtype());
    info.device = convert(t.device());
    info.numel = t.numel();
    info.contiguous = t.is_contiguous();
    info.requires_grad = t.requires_grad();
    info.leaf = 1;
    return info;
}

dl_shape dl_tensor_shape(const dl_tensor* tensor) {
    if (!tensor) return {nullptr, 0};
    const auto& s = tensor->value.shape();
    return {s.data(), s.size()};
}

dl_shape dl_tensor_strides(const dl_tensor* tensor) {
    if (!tensor) return {nullptr, 0};
    const auto& s = tensor->value.strides();
    return {s.data(), s.size()};
}

const void* dl_tensor_data(const dl_tensor* tensor) { return tensor ? tensor->value.data<void>() : nullptr; }

size_t dl_tensor_nbytes(const dl_tensor* tensor) {
    return tensor ? static_cast<size_t>(tensor->value.numel()) * dl::element_size(tensor->value.dtype()) : 0;
}

dl_status dl_tensor_copy_to_host(const dl_tensor* tensor, void* destination) {
    return invoke([&] {
        const auto& t = require(tensor, "tensor").value;
        dl::Tensor host = t.to(dl::Device::cpu()).contiguous();
        const size_t bytes = static_cast<size_t>(host.numel()) * dl::element_size(host.dtype());
        if (bytes) std::memcpy(destination, host.data<void>(), bytes);
    });
}

dl_status dl_from_host(const void* data, dl_shape shape, dl_tensor_options options, dl_tensor** output) {
    return make_handle(output, [&] {
        const auto o = convert(options);
        return dl::detail::from_host(data, convert(shape), o.dtype, o.requires_grad, o.device);
    });
}

dl_status dl_full(dl_shape shape, double value, dl_tensor_options options, dl_tensor** output) {
    return make_handle(output, [&] { return dl::full(convert(shape), value, convert(options)); });
}
dl_status dl_zeros(dl_shape shape, dl_tensor_options options, dl_tensor** output) {
    return make_handle(output, [&] { return dl::zeros(convert(shape), convert(options)); });
}
dl_status dl_ones(dl_shape shape, dl_tensor_options options, dl_tensor** output) {
    return make_handle(output, [&] { return dl::ones(convert(shape), convert(options)); });
}

dl_status dl_clone(const dl_tensor* input, dl_tensor** output) {
    return make_handle(output, [&] { return require(input, "input").value.clone(); });
}
dl_status dl_contiguous(const dl_tensor* input, dl_tensor** output) {
    return make_handle(output, [&] { return require(input, "input").value.contiguous(); });
}
dl_status dl_astype(const dl_tensor* input, dl_dtype dtype, dl_tensor** output) {
    return make_handle(output, [&] { return require(input, "input").value.astype(convert(dtype)); });
}
dl_status dl_to(const dl_tensor* input, dl_device device, dl_tensor** output) {
    return make_handle(output, [&] { return require(input, "input").value.to(convert(device)); });
}
dl_status dl_reshape(const dl_tensor* input, dl_shape shape, dl_tensor** output) {
    return make_handle(output, [&] { return require(input, "input").value.reshape(convert(shape)); });
}
dl_status dl_select(const dl_tensor* input, int64_t axis, int64_t index, dl_tensor** output) {
    return make_handle(output, [&] { return require(input, "input").value.select(axis, index); });
}
dl_status dl_narrow(const dl_tensor* input, int64_t axis, int64_t start, int64_t length, dl_tensor** output) {
    return make_handle(output, [&] { return require(input, "input").value.narrow(axis, start, length); });
}

dl_status dl_argmax(const dl_tensor* input, int64_t axis, int32_t keepdim, dl_tensor** output) {
    return make_handle(output, [&] {
        return dl::argmax(require(input, "input").value, axis, keepdim ? dl::KeepDim::yes : dl::KeepDim::no);
    });
}
dl_status dl_linear(const dl_tensor* input, const dl_tensor* weight, const dl_tensor* bias, dl_tensor** output) {
    return make_handle(output, [&] {
        return dl::linear(require(input, "input").value, require(weight, "weight").value,
                          bias ? std::optional<dl::Tensor>{bias->value} : std::nullopt);
    });
}
dl_status dl_embedding(const dl_tensor* indices, const dl_tensor* weight, dl_tensor** output) {
    return make_handle(output, [&] {
        auto out = dl::embedding(require(indices, "indices").value, require(weight, "weight").value);
        dl::detail::check_device_errors(out.device(), "embedding");
        return out;
    });
}
dl_status dl_rms_norm(const dl_tensor* input, dl_shape normalized_shape, const dl_tensor* weight,
                      const double* epsilon, dl_tensor** output) {
    return make_handle(output, [&] {
        return dl::rms_norm(require(input, "input").value, convert(normalized_shape),
                            weight ? std::optional<dl::Tensor>{weight->value} : std::nullopt,
                            epsilon ? std::optional<double>{*epsilon} : std::nullopt);
    });
}

dl_status dl_synchronize(dl_device device) { return invoke([&] { dl::synchronize(convert(device)); }); }

dl_status dl_gpu_memory_get_stats(int32_t device, dl_gpu_memory_stats* output) {
    return invoke([&] {
        if (!output) throw std::invalid_argument("memory statistics output is null");
        const auto stats = dl::gpu::memory_stats(device);
        *output = {stats.used_bytes, stats.reserved_bytes, stats.peak_used_bytes, stats.peak_reserved_bytes,
                   stats.release_threshold};
    });
}

dl_status dl_gpu_memory_set_release_threshold(int32_t device, uint64_t bytes) {
    return invoke([&] { dl::gpu::set_memory_release_threshold(bytes, device); });
}

dl_status dl_gpu_memory_reset_peak_stats(int32_t device) {
    return invoke([&] { dl::gpu::reset_peak_memory_stats(device); });
}

dl_status dl_gpu_memory_release_unused(int32_t device) {
    return invoke([&] { dl::gpu::release_unused_memory(device); });
}

dl_status dl_cuda_memory_get_stats(int32_t device, dl_cuda_memory_stats* output) {
    return dl_gpu_memory_get_stats(device, output);
}
dl_status dl_cuda_memory_set_release_threshold(int32_t device, uint64_t bytes) {
    return dl_gpu_memory_set_release_threshold(device, bytes);
}
dl_status dl_cuda_memory_reset_peak_stats(int32_t device) { return dl_gpu_memory_reset_peak_stats(device); }
dl_status dl_cuda_memory_release_unused(int32_t device) { return dl_gpu_memory_release_unused(device); }

int32_t dl_grad_enabled(void) { return dl::is_grad_enabled() ? 1 : 0; }

dl_random_key dl_random_fold_in(dl_random_key key, uint64_t label) { return convert(dl::fold_in(convert(key), label)); }

void dl_random_split(dl_random_key key, size_t count, dl_random_key* outputs) {
    for (size_t i = 0; i < count; ++i) outputs[i] = convert(dl::fold_in(convert(key), i));
}

dl_status dl_uniform_with_key(dl_random_key key, dl_shape shape, double low, double high, dl_tensor_options options,
                              dl_tensor** output) {
    return make_handle(output, [&] { return dl::uniform(convert(key), convert(shape), low, high, convert(options)); });
}

dl_status dl_randn_with_key(dl_random_key key, dl_shape shape, dl_tensor_options options, dl_tensor** output) {
    return make_handle(output, [&] { return dl::randn(convert(key), convert(shape), convert(options)); });
}

} // extern "C"
