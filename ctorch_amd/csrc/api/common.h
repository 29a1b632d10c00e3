// C ABI plumbing (reference src/api/common.h:8-150, common.cpp:8-32): owned handles wrap C++ values, every
// status entry catches C++ exceptions into DL_ERROR plus thread-local text, and create/compute entries set
// their output slot to NULL before running.
#pragma once

#include "dl/generate_c_api.h"
#include "dl/decoder.h"
#include "nn/language_model.h"

#include <exception>
#include <memory>
#include <vector>

struct dl_tensor { dl::Tensor value; };
struct dl_module { std::shared_ptr<dl::nn::UnaryModule> value; };
struct dl_state { dl::StateDict value; };
struct dl_decoder_cache { std::vector<dl::nn::KVCache> value; };
struct dl_decoder_lm {
    std::shared_ptr<dl::nn::UnaryModule> embedding, decoder, head;
    std::unique_ptr<dl::detail::DecoderLM> value;
};
struct dl_timer {
    int device;
    dlh_event start, stop;
};

namespace dl::capi {

void set_error(const char* message) noexcept;
const char* error_text() noexcept;

template <class Function> dl_status invoke(Function&& function) noexcept {
    try {
        function();
        set_error("");
        return DL_OK;
    } catch (const std::exception& error) {
        set_error(error.what());
    } catch (...) {
        set_error("unknown C++ exception");
    }
    return DL_ERROR;
}

template <class Handle, class Function> dl_status make_handle(Handle** output, Function&& function) noexcept {
    if (!output) {
        set_error("output slot is NULL");
        return DL_ERROR;
    }
    *output = nullptr;
    return invoke([&] { *output = new Handle{function()}; });
}

inline Device convert(dl_device value) { return {static_cast<DeviceType>(value.type), value.index}; }
inline dl_device convert(Device value) { return {static_cast<dl_device_type>(value.type), value.index}; }
inline DType convert(dl_dtype value) { return static_cast<DType>(value); }
inline RandomKey convert(dl_random_key value) { return {value.seed, value.stream}; }
inline dl_random_key convert(RandomKey value) { return {value.seed, value.stream}; }
inline Shape convert(dl_shape value) { return value.size == 0 ? Shape{} : Shape(value.data, value.data + value.size); }
inline TensorOptions convert(dl_tensor_options value) {
    return {convert(value.dtype), convert(value.device), value.requires_grad != 0};
}

template <class T> T& require(T* handle, const char* what) {
    if (!handle) throw std::invalid_argument(std::string(what) + " is NULL");
    return *handle;
}

} // namespace dl::capi
