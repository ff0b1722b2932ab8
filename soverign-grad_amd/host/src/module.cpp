// module.cpp -- parameter registry (interface of src/module.cpp:20-134).
#include "sovereigngrad/module.hpp"

#include <functional>
#include <stdexcept>

namespace sovereigngrad {
namespace nn {

void Module::train(bool mode) {
    training_ = mode;
    for (auto& kv : submodules_) kv.second->train(mode);
}

void Module::to(Device device) {
    for (auto& kv : parameters_) *kv.second = kv.second->to(device);
    for (auto& kv : submodules_) kv.second->to(device);
}

void Module::register_parameter(const std::string& name, Tensor& param) { parameters_[name] = &param; }

void Module::register_module(const std::string& name, std::shared_ptr<Module> module) {
    submodules_[name] = std::move(module);
}

std::vector<Tensor> Module::parameters() const {
    std::vector<Tensor> out;
    for (const auto& kv : named_parameters()) out.push_back(kv.second);
    return out;
}

// A name under a prefix: "prefix.name", or "name" alone for an empty prefix
// (src/module.cpp:66,70,97,102).
static std::string qualified(const std::string& prefix, const std::string& name) {
    return prefix.empty() ? name : prefix + "." + name;
}

std::vector<std::pair<std::string, Tensor>> Module::named_parameters(const std::string& prefix) const {
    std::vector<std::pair<std::string, Tensor>> out;
    for (const auto& kv : parameters_)
        if (kv.second && kv.second->is_defined()) out.emplace_back(qualified(prefix, kv.first), *kv.second);
    for (const auto& kv : submodules_) {
        if (!kv.second) continue;
        auto sub = kv.second->named_parameters(qualified(prefix, kv.first));
        out.insert(out.end(), sub.begin(), sub.end());
    }
    return out;
}

std::unordered_map<std::string, Tensor> Module::state_dict(const std::string& prefix) const {
    std::unordered_map<std::string, Tensor> out;
    for (const auto& kv : parameters_)
        if (kv.second && kv.second->is_defined()) out[qualified(prefix, kv.first)] = kv.second->clone();
    for (const auto& kv : submodules_) {
        if (!kv.second) continue;
        for (auto& e : kv.second->state_dict(qualified(prefix, kv.first))) out[e.first] = e.second;
    }
    return out;
}

void Module::load_state_dict(const std::unordered_map<std::string, Tensor>& sd, bool strict) {
    // Every defined parameter under its qualified name (src/module.cpp:114-134):
    // missing entries are an error when strict, shapes must match, and the
    // registered tensor is written in place (copy_from bumps its version, so a
    // quantized module repacks its device weight on the next forward).
    std::function<void(Module&, const std::string&)> load = [&](Module& m, const std::string& prefix) {
        for (auto& kv : m.parameters_) {
            if (!kv.second || !kv.second->is_defined()) continue;
            const std::string name = qualified(prefix, kv.first);
            auto it = sd.find(name);
            if (it == sd.end()) {
                if (strict) throw std::runtime_error("Missing parameter in state_dict: '" + name + "'");
                continue;
            }
            Tensor& dst = *kv.second;
            if (dst.shape() != it->second.shape())
                throw std::runtime_error("Shape mismatch for parameter '" + name + "': expected [" + dst.summary() +
                                         "] but got [" + it->second.summary() + "]");
            dst.copy_from(it->second);
        }
        for (auto& kv : m.submodules_)
            if (kv.second) load(*kv.second, qualified(prefix, kv.first));
    };
    load(*this, "");
}

}  // namespace nn
}  // namespace sovereigngrad
