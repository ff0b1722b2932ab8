// safetensors.hpp -- SafeTensors files with the reference's interface
// (include/sovereigngrad/safetensors.hpp): an 8-byte little-endian header
// length, a JSON header {"name":{"dtype","shape","data_offsets"}}, then the
// payload.  Tensors are written as F32 with names sorted; F32, F16, I32 and I64
// payloads are read (and converted to fp32).
#pragma once

#include "sovereigngrad/module.hpp"
#include "sovereigngrad/tensor.hpp"

#include <string>
#include <unordered_map>
#include <vector>

namespace sovereigngrad {
namespace safetensors {

struct TensorMeta {
    std::string dtype;
    std::vector<int64_t> shape;
    size_t data_offset_start = 0;
    size_t data_offset_end = 0;
};

void save_file(const std::unordered_map<std::string, Tensor>& state_dict, const std::string& filepath);
std::unordered_map<std::string, Tensor> load_file(const std::string& filepath, Device device = Device::CPU);
void save_module(const nn::Module& module, const std::string& filepath);
void load_module(nn::Module& module, const std::string& filepath, bool strict = true);
std::unordered_map<std::string, TensorMeta> inspect_file(const std::string& filepath);

}  // namespace safetensors
}  // namespace sovereigngrad
