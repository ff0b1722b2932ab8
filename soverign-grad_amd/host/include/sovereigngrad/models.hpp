// models.hpp -- the reference's LLaMABlock (include/sovereigngrad/models.hpp:
// 197-224) with every nn::Linear a QuantizedLinear4Bit, decoded one token per
// sequence with a key/value cache on the GPU.  Submodule and parameter names
// follow the reference block (norm1.weight, attn.q_proj.*, mlp.w_gate.*, ...),
// with each projection's qdata/scales/bias in place of weight/bias.
//
// The reference has no cache: NanoLLaMA::generate reruns the full sequence for
// every token (models.hpp:270-302).  decode() returns, for each sequence's new
// token, the row the reference's LLaMABlock::forward gives for that position.
#pragma once

#include "sovereigngrad/nn.hpp"

#include <cstdint>
#include <memory>
#include <vector>

namespace sovereigngrad {
namespace nn {

// RMSNorm's parameter (nn.hpp:67-85): weight [D] (ones), eps.
class RMSNorm : public Module {
public:
    Tensor weight;
    float eps;
    RMSNorm(int64_t normalized_shape, float eps = 1e-5f, Device device = Device::CPU);
    Tensor forward(const Tensor& x) override;  // rms_norm (src/ops.cpp:1532-1556) on the GPU
    Tensor operator()(const Tensor& x) override { return forward(x); }
};

// CausalSelfAttention's projections (nn.hpp:503-531), quantized.
class QuantizedCausalSelfAttention : public Module {
public:
    int64_t embed_dim, num_heads, head_dim;
    float scale;  // 1 / sqrt((float)(embed_dim / num_heads)), nn.hpp:518
    std::shared_ptr<QuantizedLinear4Bit> q_proj, k_proj, v_proj, out_proj;
    QuantizedCausalSelfAttention(int64_t embed_dim, int64_t num_heads, int64_t group_size = 32,
                                 Device device = Device::CPU);
};

// SwiGLU's projections (nn.hpp:135-149), quantized.
class QuantizedSwiGLU : public Module {
public:
    std::shared_ptr<QuantizedLinear4Bit> w_gate, w_up, w_down;
    QuantizedSwiGLU(int64_t in_features, int64_t hidden_features, int64_t group_size = 32,
                    Device device = Device::CPU);
};

}  // namespace nn

namespace models {

// Per-layer key/value cache, [B, max_tokens, D] fp32 each on the GPU.
struct KVCache {
    int64_t B, max_tokens, D;
    Tensor k, v;
    KVCache(int64_t B, int64_t max_tokens, int64_t D);
};

// Tokens already cached per sequence, shared by every layer of a step
// (host copy plus the device copy the kernels read).  A negative or
// out-of-range position marks a sequence that takes no part in the step.
class DecodePositions {
public:
    explicit DecodePositions(int64_t B);
    void set(const std::vector<int32_t>& pos);  // uploads
    void advance();                             // +1 for every active sequence, uploads
    const std::vector<int32_t>& host() const { return host_; }
    const int32_t* device() const { return static_cast<const int32_t*>(dev_->ptr); }
    int64_t max_len() const;  // 1 + the largest position (>= 1)

private:
    std::vector<int32_t> host_;
    std::shared_ptr<Storage> dev_;
};

class QuantizedLLaMABlock : public nn::Module {
public:
    std::shared_ptr<nn::RMSNorm> norm1, norm2;
    std::shared_ptr<nn::QuantizedCausalSelfAttention> attn;
    std::shared_ptr<nn::QuantizedSwiGLU> mlp;
    int64_t embed_dim, hidden_dim, group_size;

    QuantizedLLaMABlock(int64_t embed_dim, int64_t num_heads, int64_t hidden_dim, int64_t group_size = 32,
                        Device device = Device::CPU);

    // Quantizes float projections ([in, out] weights with [1, out] biases, as
    // QuantizedLinear4Bit::from_float, nn.hpp:984-992) in the order q, k, v,
    // out, gate, up, down; norm weights are copied.
    static std::shared_ptr<QuantizedLLaMABlock> from_float(const std::vector<const nn::Linear*>& projections,
                                                           const Tensor& norm1_weight, const Tensor& norm2_weight,
                                                           int64_t num_heads, int64_t group_size = 32);

    // x [B, D]: one new token per sequence.  Writes this token's key and value
    // at row pos[b] of the cache and returns the block output [B, D] on x's
    // device.  Sequences whose position is out of range get a NaN row.
    Tensor decode(const Tensor& x, KVCache& cache, const DecodePositions& pos);
};

}  // namespace models
}  // namespace sovereigngrad
