// Module and state entries of <dl/c_api.h> (reference src/api/module.cpp:31,44,167,201-216, src/api/state.cpp:66-80).
#include "api/common.h"
#include "dl/io.h"

#include <stdexcept>

using namespace dl::capi;

extern "C" {

void dl_module_release(dl_module* module) { delete module; }

dl_status dl_module_retain(const dl_module* module, dl_module** output) {
    return make_handle(output, [&] { return require(module, "module").value; });
}

dl_status dl_linear_create(int64_t input_features, int64_t output_features, int32_t bias, dl_tensor_options options,
                           dl_module** output) {
    return make_handle(output, [&] {
        return std::static_pointer_cast<dl::nn::UnaryModule>(
            std::make_shared<dl::nn::Linear>(input_features, output_features, bias != 0, convert(options)));
    });
}

dl_status dl_linear_from_tensors(const dl_tensor* weight, const dl_tensor* bias, dl_module** output) {
    return make_handle(output, [&] {
        return std::static_pointer_cast<dl::nn::UnaryModule>(std::make_shared<dl::nn::Linear>(
            require(weight, "weight").value, bias ? std::optional<dl::Tensor>{bias->value} : std::nullopt));
    });
}

dl_status dl_embedding_create(int64_t vocabulary, int64_t dimensions, dl_tensor_options options, dl_module** output) {
    return make_handle(output, [&] {
        return std::static_pointer_cast<dl::nn::UnaryModule>(
            std::make_shared<dl::nn::Embedding>(vocabulary, dimensions, convert(options)));
    });
}

dl_status dl_embedding_from_tensor(const dl_tensor* weight, dl_module** output) {
    return make_handle(output, [&] {
        return std::static_pointer_cast<dl::nn::UnaryModule>(
            std::make_shared<dl::nn::Embedding>(require(weight, "weight").value));
    });
}

dl_status dl_rms_norm_create(dl_shape normalized_shape, const double* epsilon, int32_t affine,
                             dl_tensor_options options, dl_module** output) {
    return make_handle(output, [&] {
        return std::static_pointer_cast<dl::nn::UnaryModule>(std::make_shared<dl::nn::RMSNorm>(
            convert(normalized_shape), epsilon ? std::optional<double>{*epsilon} : std::nullopt, affine != 0,
            convert(options)));
    });
}

dl_status dl_module_forward(dl_module* module, const dl_tensor* input, dl_tensor** output) {
    return make_handle(output, [&] {
        auto out = require(module, "module").value->forward(require(input, "input").value);
        return out;
    });
}

dl_status dl_module_to(dl_module* module, dl_device device) {
    return invoke([&] { require(module, "module").value->to(convert(device)); });
}

dl_status dl_module_parameters(const dl_module* module, dl_state** output) {
    return make_handle(output, [&] { return require(module, "module").value->named_parameters(); });
}

dl_status dl_module_state(const dl_module* module, dl_state** output) {
    return make_handle(output, [&] { return require(module, "module").value->state_dict(); });
}

dl_status dl_module_load_state(dl_module* module, const dl_state* state) {
    return invoke([&] { require(module, "module").value->load_state_dict(require(state, "state").value); });
}

void dl_state_release(dl_state* state) { delete state; }

size_t dl_state_size(const dl_state* state) { return state ? state->value.size() : 0; }

const char* dl_state_name(const dl_state* state, size_t index) {
    if (!state || index >= state->value.size()) return nullptr;
    return state->value[index].first.c_str();
}

dl_status dl_state_tensor(const dl_state* state, size_t index, dl_tensor** output) {
    return make_handle(output, [&] {
        const auto& s = require(state, "state").value;
        if (index >= s.size()) throw std::out_of_range("state index out of range");
        return s[index].second;
    });
}

dl_status dl_state_save(const char* path, const dl_state* state) {
    return invoke([&] {
        if (!path) throw std::invalid_argument("path must be non-NULL");
        dl::io::save(path, require(state, "state").value);
    });
}

dl_status dl_state_load(const char* path, dl_state** output) {
    return make_handle(output, [&] {
        if (!path) throw std::invalid_argument("path must be non-NULL");
        return dl::io::load(path);
    });
}

dl_status dl_state_create(const char* const* names, const dl_tensor* const* tensors, size_t count, dl_state** output) {
    return make_handle(output, [&] {
        dl::StateDict state;
        state.reserve(count);
        for (size_t i = 0; i < count; ++i) {
            if (!names[i] || !tensors[i]) throw std::invalid_argument("state entries must be non-NULL");
            state.emplace_back(names[i], tensors[i]->value);
        }
        return state;
    });
}

} // extern "C"
