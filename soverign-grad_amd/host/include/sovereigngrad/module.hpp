// module.hpp -- parameter registry with the reference's interface
// (include/sovereigngrad/module.hpp:12-48): named parameters, submodules,
// state_dict (clones) and a strict, shape-checked load_state_dict that writes
// into the registered tensors in place (src/module.cpp:94-134).
#pragma once

#include "sovereigngrad/tensor.hpp"

#include <memory>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace sovereigngrad {
namespace nn {

class Module {
public:
    Module() = default;
    virtual ~Module() = default;

    virtual void train(bool mode = true);
    void eval() { train(false); }
    bool is_training() const { return training_; }

    virtual void to(Device device);
    void cpu() { to(Device::CPU); }
    void cuda() { to(Device::CUDA); }

    virtual Tensor forward(const Tensor& input) { return input; }
    virtual Tensor operator()(const Tensor& input) { return forward(input); }

    void register_parameter(const std::string& name, Tensor& param);
    void register_module(const std::string& name, std::shared_ptr<Module> module);

    std::vector<Tensor> parameters() const;
    std::vector<std::pair<std::string, Tensor>> named_parameters(const std::string& prefix = "") const;

    std::unordered_map<std::string, Tensor> state_dict(const std::string& prefix = "") const;
    void load_state_dict(const std::unordered_map<std::string, Tensor>& state_dict, bool strict = true);

protected:
    bool training_ = true;
    std::unordered_map<std::string, Tensor*> parameters_;
    std::unordered_map<std::string, std::shared_ptr<Module>> submodules_;
};

}  // namespace nn
}  // namespace sovereigngrad
