// serialization.hpp -- the reference's ".sgrd" checkpoint format
// (include/sovereigngrad/serialization.hpp, src/serialization.cpp:11-101):
// "SGRD", u32 version 1, u32 count, then per tensor u32 name length, name,
// u32 rank, i64 dims, i64 numel, fp32 payload.  Quantized modules store their
// codes as fp32 "qdata", exactly as the reference does.
#pragma once

#include "sovereigngrad/module.hpp"
#include "sovereigngrad/tensor.hpp"

#include <string>
#include <unordered_map>

namespace sovereigngrad {
namespace serialization {

void save_checkpoint(const std::unordered_map<std::string, Tensor>& state_dict, const std::string& filepath);
std::unordered_map<std::string, Tensor> load_checkpoint(const std::string& filepath, Device device = Device::CPU);
void save_module(const nn::Module& module, const std::string& filepath);
void load_module(nn::Module& module, const std::string& filepath, bool strict = true);

}  // namespace serialization
}  // namespace sovereigngrad
