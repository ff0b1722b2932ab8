// nn.cpp -- Linear and the quantized linear layers (interfaces of
// include/sovereigngrad/nn.hpp:17-38 and :927-1001).
#include "sovereigngrad/nn.hpp"

#include <cmath>

namespace sovereigngrad {
namespace nn {

Linear::Linear(int64_t in_features, int64_t out_features, Device device) {
    const float std = std::sqrt(2.0f / (float)(in_features + out_features));
    W = Tensor::randn({in_features, out_features}, 0.0f, std, device, true);
    b = Tensor::zeros({1, out_features}, device, true);
    register_parameter("weight", W);
    register_parameter("bias", b);
}

Tensor Linear::forward(const Tensor& x) { return x.matmul(W) + b; }

QuantizedLinear::QuantizedLinear(int64_t in, int64_t out, Device device) : in_features(in), out_features(out) {
    const float std = std::sqrt(2.0f / (float)(in + out));
    Tensor W = Tensor::randn({in, out}, 0.0f, std, device, false);
    q_weight = quantization::quantize_int8(W, quantization::QuantizationScheme::PerChannelSymmetric);
    bias = Tensor::zeros({1, out}, device, false);
    register_all();
}

QuantizedLinear::QuantizedLinear(NoInit, int64_t in, int64_t out) : in_features(in), out_features(out) {}

void QuantizedLinear::register_all() {
    register_parameter("qdata", q_weight.qdata);
    register_parameter("scales", q_weight.scales);
    register_parameter("bias", bias);
}

std::shared_ptr<QuantizedLinear> QuantizedLinear::from_float(const Linear& fl) {
    std::shared_ptr<QuantizedLinear> ql(new QuantizedLinear(NoInit{}, fl.W.shape()[0], fl.W.shape()[1]));
    ql->q_weight = quantization::quantize_int8(fl.W, quantization::QuantizationScheme::PerChannelSymmetric);
    ql->bias = fl.b.clone();
    ql->register_all();
    return ql;
}

Tensor QuantizedLinear::forward(const Tensor& x) { return quantization::quantized_matmul_int8(x, q_weight, bias); }

QuantizedLinear4Bit::QuantizedLinear4Bit(int64_t in, int64_t out, int64_t gs, Device device)
    : in_features(in), out_features(out), group_size(gs) {
    const float std = std::sqrt(2.0f / (float)(in + out));
    Tensor W = Tensor::randn({in, out}, 0.0f, std, device, false);
    q_weight = quantization::quantize_int4(W, gs);
    bias = Tensor::zeros({1, out}, device, false);
    register_all();
}

QuantizedLinear4Bit::QuantizedLinear4Bit(NoInit, int64_t in, int64_t out, int64_t gs)
    : in_features(in), out_features(out), group_size(gs) {}

void QuantizedLinear4Bit::register_all() {
    register_parameter("qdata", q_weight.qdata);
    register_parameter("scales", q_weight.scales);
    register_parameter("bias", bias);
}

std::shared_ptr<QuantizedLinear4Bit> QuantizedLinear4Bit::from_float(const Linear& fl, int64_t gs) {
    std::shared_ptr<QuantizedLinear4Bit> ql(
        new QuantizedLinear4Bit(NoInit{}, fl.W.shape()[0], fl.W.shape()[1], gs));
    ql->q_weight = quantization::quantize_int4(fl.W, gs);
    ql->bias = fl.b.clone();
    ql->register_all();
    return ql;
}

Tensor QuantizedLinear4Bit::forward(const Tensor& x) {
    return quantization::quantized_matmul_int4(x, q_weight, bias);
}

}  // namespace nn
}  // namespace sovereigngrad
