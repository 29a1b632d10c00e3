#pragma once
// Module tree.  Mirrors include/dl/nn.h:29-124,209-219,381-390 of the reference: registration of
// parameters / buffers / children, state_dict and load_state_dict by canonical dotted names in
// registration order, `to(device)` keeping parameter identity, and the Linear / Embedding / RMSNorm layers.

#include "dl/ops.h"

#include <string>
#include <string_view>

namespace dl {

using NamedTensor = std::pair<std::string, Tensor>;
using StateDict = std::vector<NamedTensor>;

namespace nn {

class DL_API Module {
public:
    virtual ~Module() = default;
    Module() = default;
    Module(const Module&) = delete;
    Module& operator=(const Module&) = delete;

    std::vector<Tensor> parameters() const;
    StateDict named_parameters() const;
    StateDict named_buffers() const;
    /// Parameters in registration order, then buffers; the tensors share this module's storage.
    StateDict state_dict() const;
    /// Writes same-name, same-shape values into the existing tensors (dtype is converted when the
    /// value is floating point; the device is the module's).
    void load_state_dict(std::span<const NamedTensor> state);
    /// Moves parameters and buffers, keeping tensor identity.
    void to(Device device);

    void train(bool enabled = true) { training_ = enabled; }
    void eval() { train(false); }
    bool is_training() const { return training_; }

protected:
    Tensor register_parameter(std::string name, Tensor value);
    Tensor register_buffer(std::string name, Tensor value);
    void register_module(std::string name, std::shared_ptr<Module> child);

    template <class Child, class... Args>
    std::shared_ptr<Child> add_module(std::string name, Args&&... args) {
        auto child = std::make_shared<Child>(std::forward<Args>(args)...);
        register_module(std::move(name), child);
        return child;
    }

private:
    void collect(bool buffers, const std::string& prefix, StateDict& out) const;
    void validate_name(std::string_view name) const;

    StateDict parameters_;
    StateDict buffers_;
    std::vector<std::pair<std::string, std::shared_ptr<Module>>> children_;
    bool training_ = true;
};

class DL_API UnaryModule : public Module {
public:
    virtual Tensor forward(const Tensor& input) = 0;
    Tensor operator()(const Tensor& input) { return forward(input); }
};

class DL_API Linear : public UnaryModule {
public:
    Linear(Index input_features, Index output_features, bool bias = true, TensorOptions options = {});
    Linear(Tensor weight, std::optional<Tensor> bias = std::nullopt);
    Tensor forward(const Tensor& input) override;
    const Tensor& weight() const { return weight_; }
    const std::optional<Tensor>& bias() const { return bias_; }

private:
    Tensor weight_;
    std::optional<Tensor> bias_;
};

class DL_API Embedding : public UnaryModule {
public:
    Embedding(Index vocabulary, Index dimensions, TensorOptions options = {});
    explicit Embedding(Tensor weight);
    Tensor forward(const Tensor& indices) override;
    const Tensor& weight() const { return weight_; }

private:
    Tensor weight_;
};

class DL_API RMSNorm : public UnaryModule {
public:
    explicit RMSNorm(Shape normalized_shape, std::optional<double> epsilon = std::nullopt, bool affine = true,
                     TensorOptions options = {});
    Tensor forward(const Tensor& input) override;
    const std::optional<Tensor>& weight() const { return weight_; }
    double epsilon() const;

private:
    Shape normalized_shape_;
    std::optional<double> epsilon_;
    std::optional<Tensor> weight_;
};

} // namespace nn
} // namespace dl
