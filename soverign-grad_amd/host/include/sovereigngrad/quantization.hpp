// quantization.hpp -- drop-in replacement of the reference's quantization API
// (include/sovereigngrad/quantization.hpp:11-37).  Same enum, struct fields,
// function names, signatures and defaults; every function runs its arithmetic
// in libsgq.so's gfx950 kernels.  Tensors on Device::CPU are moved to the GPU
// for the computation and results come back on the caller's device, as the
// reference returns them (src/quantization.cpp:40,73-74,110,156-157,186).
#pragma once

#include "sovereigngrad/tensor.hpp"

#include <cstdint>
#include <memory>
#include <mutex>
#include <vector>

namespace sovereigngrad {
namespace quantization {

enum class QuantizationScheme { PerTensorSymmetric, PerChannelSymmetric, GroupedAsymmetric };

// Device-resident packed form of a QuantizedTensor (see include/sgq.h):
// packed codes plus, for the strip-major INT4 layout, transposed scales.  It
// is derived from qdata/scales and rebuilt whenever either of them is
// replaced or written in place (their version counters change).
struct PackedWeight {
    std::mutex mu;
    std::shared_ptr<Storage> codes;  // GPU
    Tensor devscales;                // GPU (INT4 strip-major layout)
    Tensor scales_dev;               // GPU copy of the reference-layout scales
    uint64_t qdata_id = 0, scales_id = 0;  // TensorImpl ids of the qdata / scales it was built from
    uint64_t qdata_version = 0, scales_version = 0;
    bool valid = false;
};

struct QuantizedTensor {
    Tensor qdata;        // codes, one fp32 per weight, in the weight's shape (reference layout)
    Tensor scales;       // fp32 scales (1, rows, or ceil(numel/group_size))
    Tensor zero_points;  // unused (symmetric schemes), kept for interface compatibility
    QuantizationScheme scheme = QuantizationScheme::PerChannelSymmetric;
    std::vector<int64_t> original_shape;
    int64_t group_size = 0;
    int bits = 8;
    std::shared_ptr<PackedWeight> packed = std::make_shared<PackedWeight>();
};

// INT8 Quantization
QuantizedTensor quantize_int8(const Tensor& x, QuantizationScheme scheme = QuantizationScheme::PerChannelSymmetric);
Tensor dequantize_int8(const QuantizedTensor& qx);

// INT4 Quantization
QuantizedTensor quantize_int4(const Tensor& x, int64_t group_size = 32);
Tensor dequantize_int4(const QuantizedTensor& qx);

// The packed device form of q (built, or rebuilt after qdata/scales changed,
// on demand) for callers of the C ABI such as the LLaMA block decode step.
// The handle keeps the device buffers alive while it is held.
struct PackedHandle {
    std::shared_ptr<Storage> codes;
    Tensor devscales;  // INT4 strip-major layout
    Tensor scales;     // reference-layout scales on the GPU
};
PackedHandle packed_weight(const QuantizedTensor& q);

// Direct Low-Bit Matrix Multiplication: x[B,K] . deq(W[K,N]) (+ bias[1,N])
Tensor quantized_matmul_int8(const Tensor& x, const QuantizedTensor& q_weight, const Tensor& bias = Tensor());
Tensor quantized_matmul_int4(const Tensor& x, const QuantizedTensor& q_weight, const Tensor& bias = Tensor());

}  // namespace quantization
}  // namespace sovereigngrad
