// Module registry, named state and device moves (reference src/nn/module.cpp:37-201).  Traversal is depth-first
// in registration order (parameters of a module before its children), tensors are de-duplicated by identity
// and the canonical name of a shared tensor is the lexicographically smallest path.
#include "core/tensor_impl.h"
#include "dl/nn.h"

#include <algorithm>
#include <atomic>
#include <stdexcept>
#include <unordered_map>
#include <unordered_set>

namespace dl::detail {
namespace {
std::atomic<uint64_t> g_parameter_epoch{1};
}
uint64_t parameter_epoch() { return g_parameter_epoch.load(std::memory_order_acquire); }
void advance_parameter_epoch() { g_parameter_epoch.fetch_add(1, std::memory_order_acq_rel); }
} // namespace dl::detail

namespace dl::nn {

using detail::TensorAccess;

void Module::validate_name(std::string_view name) const {
    if (name.empty() || name.find('.') != std::string_view::npos)
        throw std::invalid_argument("module entry names must be non-empty and contain no '.'");
    auto taken = [&](const auto& list) {
        return std::any_of(list.begin(), list.end(), [&](const auto& entry) { return entry.first == name; });
    };
    if (taken(parameters_) || taken(buffers_) || taken(children_))
        throw std::invalid_argument("duplicate module entry name: " + std::string(name));
}

Tensor Module::register_parameter(std::string name, Tensor value) {
    validate_name(name);
    parameters_.emplace_back(std::move(name), value);
    return value;
}

Tensor Module::register_buffer(std::string name, Tensor value) {
    validate_name(name);
    buffers_.emplace_back(std::move(name), value);
    return value;
}

void Module::register_module(std::string name, std::shared_ptr<Module> child) {
    validate_name(name);
    children_.emplace_back(std::move(name), std::move(child));
}

void Module::collect(bool buffers, const std::string& prefix, StateDict& out) const {
    for (const auto& [name, tensor] : buffers ? buffers_ : parameters_) out.emplace_back(prefix + name, tensor);
    for (const auto& [name, child] : children_) child->collect(buffers, prefix + name + ".", out);
}

namespace {
StateDict unique_by_identity(StateDict all) {
    StateDict result;
    std::unordered_map<const void*, std::size_t> slots;
    for (auto& [name, tensor] : all) {
        const void* identity = TensorAccess::impl(tensor).get();
        auto [slot, inserted] = slots.emplace(identity, result.size());
        if (inserted) result.emplace_back(std::move(name), tensor);
        else result[slot->second].first = std::min(result[slot->second].first, name);
    }
    return result;
}
} // namespace

StateDict Module::named_parameters() const {
    StateDict all;
    collect(false, "", all);
    return unique_by_identity(std::move(all));
}

StateDict Module::named_buffers() const {
    StateDict all;
    collect(true, "", all);
    return unique_by_identity(std::move(all));
}

std::vector<Tensor> Module::parameters() const {
    std::vector<Tensor> out;
    for (auto& entry : named_parameters()) out.push_back(entry.second);
    return out;
}

StateDict Module::state_dict() const {
    auto result = named_parameters();
    for (auto& entry : named_buffers()) result.push_back(std::move(entry));
    return result;
}

void Module::load_state_dict(std::span<const NamedTensor> state) {
    std::unordered_map<std::string_view, const Tensor*> source;
    for (const auto& [name, tensor] : state) source.emplace(name, &tensor);
    auto destination = state_dict();
    std::unordered_set<const void*> target_storage;
    for (const auto& [name, tensor] : destination) target_storage.insert(TensorAccess::impl(tensor)->storage.get());
    // values that alias this module's storage are cloned first, so swaps load the values seen at call time
    std::vector<Tensor> values;
    values.reserve(destination.size());
    for (const auto& [name, tensor] : destination) {
        auto found = source.find(name);
        if (found == source.end()) throw std::invalid_argument("state is missing tensor: " + name);
        const Tensor& value = *found->second;
        if (value.shape() != tensor.shape())
            throw std::invalid_argument("state tensor shape differs: " + name + " " + detail::shape_string(value.shape()) +
                                        " vs " + detail::shape_string(tensor.shape()));
        if (is_floating(value.dtype()) != is_floating(tensor.dtype()))
            throw std::invalid_argument("state tensor dtype differs: " + name);
        const bool aliases = target_storage.count(TensorAccess::impl(value)->storage.get()) != 0;
        values.push_back(aliases ? value.clone() : value);
    }
    for (std::size_t i = 0; i < destination.size(); ++i) {
        const Tensor& target = destination[i].second;
        detail::copy_into(target, values[i].to(target.device()));
    }
    detail::advance_parameter_epoch();
}

void Module::to(Device device) {
    auto tensors = named_parameters();
    for (auto& entry : named_buffers()) tensors.push_back(std::move(entry));
    for (auto& [name, tensor] : tensors) {
        if (tensor.device() == device) continue;
        detail::rebind(tensor, tensor.to(device));
    }
    detail::advance_parameter_epoch();
}

} // namespace dl::nn
