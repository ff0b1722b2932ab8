// nn.hpp -- the layers of the quantized path with the reference's interfaces
// (include/sovereigngrad/nn.hpp:17-38 Linear, :927-1001 QuantizedLinear and
// QuantizedLinear4Bit): same constructors, defaults, from_float factories,
// forward/operator() and parameter names ("weight"/"bias"; "qdata"/"scales"/
// "bias").  The quantized forward runs libsgq.so's fused GPU kernels.
#pragma once

#include "sovereigngrad/module.hpp"
#include "sovereigngrad/quantization.hpp"
#include "sovereigngrad/tensor.hpp"

#include <memory>

namespace sovereigngrad {
namespace nn {

class Linear : public Module {
public:
    Tensor W;  // [in, out]
    Tensor b;  // [1, out]
    Linear(int64_t in_features, int64_t out_features, Device device = Device::CPU);
    Tensor forward(const Tensor& x) override;
    Tensor operator()(const Tensor& x) override { return forward(x); }
};

class QuantizedLinear : public Module {
public:
    quantization::QuantizedTensor q_weight;
    Tensor bias;
    int64_t in_features;
    int64_t out_features;

    QuantizedLinear(int64_t in_features, int64_t out_features, Device device = Device::CPU);
    static std::shared_ptr<QuantizedLinear> from_float(const Linear& float_linear);
    Tensor forward(const Tensor& x) override;
    Tensor operator()(const Tensor& x) override { return forward(x); }

private:
    struct NoInit {};
    QuantizedLinear(NoInit, int64_t in_features, int64_t out_features);
    void register_all();
};

class QuantizedLinear4Bit : public Module {
public:
    quantization::QuantizedTensor q_weight;
    Tensor bias;
    int64_t in_features;
    int64_t out_features;
    int64_t group_size;

    QuantizedLinear4Bit(int64_t in_features, int64_t out_features, int64_t group_size = 32,
                        Device device = Device::CPU);
    static std::shared_ptr<QuantizedLinear4Bit> from_float(const Linear& float_linear, int64_t group_size = 32);
    Tensor forward(const Tensor& x) override;
    Tensor operator()(const Tensor& x) override { return forward(x); }

private:
    struct NoInit {};
    QuantizedLinear4Bit(NoInit, int64_t in_features, int64_t out_features, int64_t group_size);
    void register_all();
};

}  // namespace nn
}  // namespace sovereigngrad
