// Linear, Embedding and RMSNorm (reference src/nn/layers.cpp:6-80).  Default initialisation follows the
// reference's distributions (Linear U(+-1/sqrt(in)), Embedding N(0, 1), RMSNorm ones) from a thread-local
// generator; exact initial values are not part of the contract (tests and benchmarks load or synthesise
// their weights).
#include "nn/ops_internal.h"

#include <cmath>
#include <limits>
#include <random>
#include <stdexcept>

namespace dl::nn {
namespace {

std::mt19937_64& generator() {
    thread_local std::mt19937_64 engine(0);
    return engine;
}

Tensor host_parameter(const Shape& shape, TensorOptions options, int kind, double bound) {
    if (options.device.type == DeviceType::gpu && kind != 2 &&
        (options.dtype == DType::f32 || options.dtype == DType::bf16)) {
        // device-side draw from a key taken from the thread's generator (large models initialise in HBM)
        const RandomKey key{generator()(), generator()()};
        TensorOptions o = options;
        o.requires_grad = false;
        return kind == 0 ? uniform(key, shape, -bound, bound, o) : normal(key, shape, 1.0, o);
    }
    Tensor host = detail::empty_tensor(shape, DType::f32, Device::cpu());
    float* data = static_cast<float*>(detail::mutable_data(host));
    const Index n = host.numel();
    if (kind == 0) {
        std::uniform_real_distribution<double> dist(-bound, bound);
        for (Index i = 0; i < n; ++i) data[i] = static_cast<float>(dist(generator()));
    } else if (kind == 1) {
        std::normal_distribution<double> dist(0.0, 1.0);
        for (Index i = 0; i < n; ++i) data[i] = static_cast<float>(dist(generator()));
    } else {
        for (Index i = 0; i < n; ++i) data[i] = 1.0f;
    }
    Tensor typed = host.astype(options.dtype);
    Tensor out = typed.to(options.device);
    if (out.dtype() == typed.dtype() && out.device() == typed.device()) out = out.clone();
    return out;
}

} // namespace

Linear::Linear(Index input_features, Index output_features, bool bias, TensorOptions options)
    : weight_(register_parameter("weight",
                                 host_parameter({output_features, input_features}, options, 0,
                                                1.0 / std::sqrt(static_cast<double>(std::max<Index>(1, input_features)))))) {
    if (bias)
        bias_ = register_parameter("bias", host_parameter({output_features}, options, 0,
                                                          1.0 / std::sqrt(static_cast<double>(std::max<Index>(1, input_features)))));
}

Linear::Linear(Tensor weight, std::optional<Tensor> bias) : weight_(register_parameter("weight", std::move(weight))) {
    if (weight_.ndim() != 2) throw std::invalid_argument("Linear weight must be [out, in]");
    if (bias) bias_ = register_parameter("bias", std::move(*bias));
}

Tensor Linear::forward(const Tensor& input) { return linear(input, weight_, bias_); }

Embedding::Embedding(Index vocabulary, Index dimensions, TensorOptions options)
    : weight_(register_parameter("weight", host_parameter({vocabulary, dimensions}, options, 1, 0.0))) {}

Embedding::Embedding(Tensor weight) : weight_(register_parameter("weight", std::move(weight))) {
    if (weight_.ndim() != 2) throw std::invalid_argument("Embedding weight must be [V, D]");
}

Tensor Embedding::forward(const Tensor& indices) { return embedding(indices, weight_); }

RMSNorm::RMSNorm(Shape normalized_shape, std::optional<double> epsilon, bool affine, TensorOptions options)
    : normalized_shape_(std::move(normalized_shape)), epsilon_(epsilon) {
    if (affine) weight_ = register_parameter("weight", host_parameter(normalized_shape_, options, 2, 0.0));
}

double RMSNorm::epsilon() const {
    return epsilon_ ? *epsilon_ : static_cast<double>(std::numeric_limits<float>::epsilon());
}

Tensor RMSNorm::forward(const Tensor& input) { return rms_norm(input, normalized_shape_, weight_, epsilon_); }

} // namespace dl::nn
