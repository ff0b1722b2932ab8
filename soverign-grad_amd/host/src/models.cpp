// models.cpp -- the quantized LLaMA block decode step over libsgq.so
// (sgq_llama_block_decode_int4, sgq_rms_norm).
#include "sovereigngrad/models.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <utility>
#include <stdexcept>

#include "hip_check.hpp"

namespace sovereigngrad {
namespace nn {

RMSNorm::RMSNorm(int64_t d, float e, Device device) : eps(e) {
    weight = Tensor::ones({d}, device, true);
    register_parameter("weight", weight);
}

Tensor RMSNorm::forward(const Tensor& x) {
    if (x.shape().size() < 2) throw std::runtime_error("RMSNorm requires at least 2D tensor!");  // ops.cpp:1533
    const int64_t D = x.shape().back();
    const Tensor xg = x.device() == Device::CUDA ? x : x.to(Device::CUDA);
    const Tensor wg = weight.device() == Device::CUDA ? weight : weight.to(Device::CUDA);
    Tensor out = Tensor::empty(x.shape(), Device::CUDA);
    SG_SGQ_CHECK(sgq_rms_norm(xg.data(), xg.numel() / D, D, wg.data(), eps, out.data(), nullptr));
    return x.device() == Device::CUDA ? out : out.to(x.device());
}

QuantizedCausalSelfAttention::QuantizedCausalSelfAttention(int64_t d, int64_t heads, int64_t gs, Device device)
    : embed_dim(d), num_heads(heads), head_dim(d / heads),
      scale(1.0f / std::sqrt((float)(d / heads))) {
    if (d % heads != 0) throw std::runtime_error("embed_dim must be divisible by num_heads!");  // nn.hpp:521-523
    q_proj = std::make_shared<QuantizedLinear4Bit>(d, d, gs, device);
    k_proj = std::make_shared<QuantizedLinear4Bit>(d, d, gs, device);
    v_proj = std::make_shared<QuantizedLinear4Bit>(d, d, gs, device);
    out_proj = std::make_shared<QuantizedLinear4Bit>(d, d, gs, device);
    register_module("q_proj", q_proj);
    register_module("k_proj", k_proj);
    register_module("v_proj", v_proj);
    register_module("out_proj", out_proj);
}

QuantizedSwiGLU::QuantizedSwiGLU(int64_t in, int64_t hidden, int64_t gs, Device device) {
    w_gate = std::make_shared<QuantizedLinear4Bit>(in, hidden, gs, device);
    w_up = std::make_shared<QuantizedLinear4Bit>(in, hidden, gs, device);
    w_down = std::make_shared<QuantizedLinear4Bit>(hidden, in, gs, device);
    register_module("w_gate", w_gate);
    register_module("w_up", w_up);
    register_module("w_down", w_down);
}

}  // namespace nn

namespace models {

KVCache::KVCache(int64_t b, int64_t mt, int64_t d) : B(b), max_tokens(mt), D(d) {
    k = Tensor::empty({b, mt, d}, Device::CUDA);
    v = Tensor::empty({b, mt, d}, Device::CUDA);
}

DecodePositions::DecodePositions(int64_t B) : host_(static_cast<size_t>(B), 0) {
    dev_ = std::make_shared<Storage>(static_cast<size_t>(B > 0 ? B : 1) * sizeof(int32_t), Device::CUDA, true);
}

void DecodePositions::set(const std::vector<int32_t>& pos) {
    if (pos.size() != host_.size()) throw std::runtime_error("DecodePositions: expected one position per sequence");
    host_ = pos;
    if (!host_.empty())
        SG_HIP_CHECK(hipMemcpy(dev_->ptr, host_.data(), host_.size() * sizeof(int32_t), hipMemcpyHostToDevice));
}

void DecodePositions::advance() {
    std::vector<int32_t> next = host_;
    for (auto& p : next)
        if (p >= 0) ++p;
    set(next);
}

int64_t DecodePositions::max_len() const {
    int32_t m = 0;
    for (int32_t p : host_) m = std::max(m, p);
    return (int64_t)m + 1;
}

QuantizedLLaMABlock::QuantizedLLaMABlock(int64_t d, int64_t heads, int64_t h, int64_t gs, Device device)
    : embed_dim(d), hidden_dim(h), group_size(gs) {
    norm1 = std::make_shared<nn::RMSNorm>(d, 1e-5f, device);
    attn = std::make_shared<nn::QuantizedCausalSelfAttention>(d, heads, gs, device);
    norm2 = std::make_shared<nn::RMSNorm>(d, 1e-5f, device);
    mlp = std::make_shared<nn::QuantizedSwiGLU>(d, h, gs, device);
    register_module("norm1", norm1);
    register_module("attn", attn);
    register_module("norm2", norm2);
    register_module("mlp", mlp);
}

std::shared_ptr<QuantizedLLaMABlock> QuantizedLLaMABlock::from_float(const std::vector<const nn::Linear*>& p,
                                                                     const Tensor& n1, const Tensor& n2,
                                                                     int64_t heads, int64_t gs) {
    if (p.size() != 7) throw std::runtime_error("from_float: expected q, k, v, out, gate, up, down");
    const int64_t D = p[0]->W.shape()[0], H = p[4]->W.shape()[1];
    auto blk = std::make_shared<QuantizedLLaMABlock>(D, heads, H, gs, p[0]->W.device());
    std::shared_ptr<nn::QuantizedLinear4Bit>* dst[7] = {&blk->attn->q_proj, &blk->attn->k_proj, &blk->attn->v_proj,
                                                       &blk->attn->out_proj, &blk->mlp->w_gate, &blk->mlp->w_up,
                                                       &blk->mlp->w_down};
    const char* names[7] = {"q_proj", "k_proj", "v_proj", "out_proj", "w_gate", "w_up", "w_down"};
    for (int i = 0; i < 7; ++i) {
        *dst[i] = nn::QuantizedLinear4Bit::from_float(*p[i], gs);
        (i < 4 ? static_cast<nn::Module*>(blk->attn.get()) : static_cast<nn::Module*>(blk->mlp.get()))
            ->register_module(names[i], *dst[i]);
    }
    blk->norm1->weight.copy_from(n1);
    blk->norm2->weight.copy_from(n2);
    return blk;
}

Tensor QuantizedLLaMABlock::decode(const Tensor& x, KVCache& cache, const DecodePositions& pos) {
    if (x.shape().size() != 2 || x.shape()[1] != embed_dim) throw std::runtime_error("decode: x must be [B, D]");
    const int64_t B = x.shape()[0];
    if (cache.B != B || cache.D != embed_dim) throw std::runtime_error("decode: cache shape does not match x");
    if ((int64_t)pos.host().size() != B) throw std::runtime_error("decode: one position per sequence");
    const int64_t max_len = std::min(pos.max_len(), cache.max_tokens);
    auto gpu = [](const Tensor& t) { return t.device() == Device::CUDA ? t : t.to(Device::CUDA); };
    const Tensor xg = gpu(x);
    const std::shared_ptr<nn::QuantizedLinear4Bit> lin[7] = {attn->q_proj, attn->k_proj, attn->v_proj, attn->out_proj,
                                                            mlp->w_gate, mlp->w_up, mlp->w_down};
    quantization::PackedHandle ph[7];
    Tensor bias[7];
    sgq_int4_linear* fields[7];
    sgq_llama_block_int4 blk;
    std::memset(&blk, 0, sizeof(blk));
    fields[0] = &blk.q, fields[1] = &blk.k, fields[2] = &blk.v, fields[3] = &blk.o;
    fields[4] = &blk.gate, fields[5] = &blk.up, fields[6] = &blk.down;
    for (int i = 0; i < 7; ++i) {
        if (lin[i]->group_size != group_size) throw std::runtime_error("decode: projections differ in group size");
        ph[i] = quantization::packed_weight(lin[i]->q_weight);
        if (!ph[i].devscales.defined()) throw std::runtime_error("decode: projection not in the tiled INT4 layout");
        if (lin[i]->bias.defined()) bias[i] = gpu(lin[i]->bias);
        *fields[i] = sgq_int4_linear{ph[i].codes->ptr, std::as_const(ph[i].devscales).data(),
                                     bias[i].defined() ? std::as_const(bias[i]).data() : nullptr};
    }
    const Tensor g1 = gpu(norm1->weight), g2 = gpu(norm2->weight);
    blk.D = embed_dim;
    blk.H = hidden_dim;
    blk.group_size = group_size;
    blk.eps = norm1->eps;
    blk.attn_scale = attn->scale;
    blk.norm1 = g1.data();
    blk.norm2 = g2.data();
    const int64_t wsb = sgq_llama_decode_workspace_bytes(B, embed_dim, hidden_dim, max_len);
    if (wsb < 0) throw std::runtime_error("decode: bad shape");
    Storage ws(static_cast<size_t>(wsb), Device::CUDA, false);
    Tensor out = Tensor::empty({B, embed_dim}, Device::CUDA);
    SG_SGQ_CHECK(sgq_llama_block_decode_int4(&blk, xg.data(), out.data(), B, cache.k.data(), cache.v.data(),
                                             cache.max_tokens, pos.device(), max_len, ws.ptr, wsb, nullptr));
    return x.device() == Device::CUDA ? out : out.to(x.device());
}

}  // namespace models
}  // namespace sovereigngrad
