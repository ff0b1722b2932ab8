// quantization.cpp -- the reference's quantization API (src/quantization.cpp:11-206)
// on top of libsgq.so.  The arithmetic runs in the gfx950 kernels; this file
// only manages tensors, devices and the packed device form of each weight.
#include "sovereigngrad/quantization.hpp"

#include <stdexcept>
#include <utility>

#include "hip_check.hpp"

namespace sovereigngrad {
namespace quantization {

namespace {

struct View2D {
    int64_t rows, cols;
};

// [rows, cols] view of a weight: rows = shape[0] (src/quantization.cpp:44-45);
// rank <= 1 tensors are one row.
View2D view2d(const std::vector<int64_t>& shape) {
    if (shape.size() >= 2) {
        int64_t cols = 1;
        for (size_t i = 1; i < shape.size(); ++i) cols *= shape[i];
        return {shape[0], cols};
    }
    return {1, shape.empty() ? 1 : shape[0]};
}

Tensor on_gpu(const Tensor& t) { return t.device() == Device::CPU ? t.to(Device::CUDA) : t; }
Tensor to_device(const Tensor& t, Device d) { return t.device() == d ? t : t.to(d); }

std::shared_ptr<Storage> gpu_bytes(int64_t bytes) {
    return std::make_shared<Storage>(static_cast<size_t>(bytes > 16 ? bytes : 16), Device::CUDA, false);
}

// dequantize_int8 takes the per-tensor branch for that scheme or a single
// scale (src/quantization.cpp:90).
int int8_branch(const QuantizedTensor& q) {
    return (q.scheme == QuantizationScheme::PerTensorSymmetric || q.scales.numel() == 1) ? SGQ_PER_TENSOR_SYMMETRIC
                                                                                          : SGQ_PER_CHANNEL_SYMMETRIC;
}

void record(PackedWeight& p, const QuantizedTensor& q) {
    p.qdata_id = q.qdata.id();
    p.scales_id = q.scales.id();
    p.qdata_version = q.qdata.version();
    p.scales_version = q.scales.version();
    p.valid = true;
}

// Device buffers of one packed weight, held by value so that a concurrent
// repack cannot free them while a forward uses them.
struct PackedView {
    std::shared_ptr<Storage> codes;
    Tensor devscales;
    Tensor scales_dev;
};

PackedView view_of(const PackedWeight& p) { return PackedView{p.codes, p.devscales, p.scales_dev}; }

// Returns the packed device form of q, rebuilding it from qdata/scales when
// they were replaced or written since it was built (e.g. by load_state_dict).
PackedView packed_of(const QuantizedTensor& q) {
    if (!q.packed) throw std::runtime_error("QuantizedTensor has no packed state");
    PackedWeight& p = *q.packed;
    std::lock_guard<std::mutex> lock(p.mu);
    if (p.valid && p.qdata_id == q.qdata.id() && p.scales_id == q.scales.id() &&
        p.qdata_version == q.qdata.version() && p.scales_version == q.scales.version())
        return view_of(p);
    if (!q.qdata.defined() || !q.scales.defined()) throw std::runtime_error("QuantizedTensor is empty");
    const View2D v = view2d(q.original_shape);
    const Tensor qg = on_gpu(q.qdata);
    Tensor sg = on_gpu(q.scales).clone();
    std::shared_ptr<Storage> ws;
    if (q.bits == 8) {
        auto codes = gpu_bytes(sgq_int8_packed_bytes(v.rows, v.cols));
        const int64_t wsb = sgq_quantize_workspace_bytes(8, v.rows, v.cols, 0);
        ws = gpu_bytes(wsb);
        SG_SGQ_CHECK(sgq_pack_int8(qg.data(), v.rows, v.cols, codes->ptr, ws->ptr, wsb, nullptr));
        p.codes = codes;
        p.devscales = Tensor();
    } else {
        auto codes = gpu_bytes(sgq_int4_packed_bytes(v.rows, v.cols, q.group_size));
        const int64_t nds = sgq_int4_devscale_count(v.rows, v.cols, q.group_size);
        Tensor ds = Tensor::empty({nds > 4 ? nds : 4}, Device::CUDA);
        const int64_t wsb = sgq_quantize_workspace_bytes(4, v.rows, v.cols, q.group_size);
        ws = gpu_bytes(wsb);
        SG_SGQ_CHECK(sgq_pack_int4(qg.data(), sg.data(), v.rows, v.cols, q.group_size, codes->ptr, ds.data(), ws->ptr,
                                   wsb, nullptr));
        p.codes = codes;
        p.devscales = ds;
    }
    p.scales_dev = sg;
    record(p, q);
    return view_of(p);
}

void check_linear_args(const Tensor& x, const QuantizedTensor& w, const Tensor& bias, View2D& v) {
    // The reference dequantizes to original_shape and calls matmul, which
    // needs 2-D operands with matching inner dimensions (src/ops.cpp:380-389).
    if (x.shape().size() != 2 || w.original_shape.size() != 2)
        throw std::runtime_error("matmul currently requires 2D tensors!");
    v = view2d(w.original_shape);
    if (x.shape()[1] != v.rows) throw std::runtime_error("Matrix inner dimensions must match for matmul!");
    if (bias.defined() && bias.numel() != v.cols)
        throw std::runtime_error("bias must hold out_features values ([1, out] or [out])");
}

}  // namespace

PackedHandle packed_weight(const QuantizedTensor& q) {
    const PackedView v = packed_of(q);
    return PackedHandle{v.codes, v.devscales, v.scales_dev};
}

QuantizedTensor quantize_int8(const Tensor& x, QuantizationScheme scheme) {
    const View2D v = view2d(x.shape());
    const int eff = (scheme == QuantizationScheme::PerTensorSymmetric || x.shape().size() < 2)
                        ? SGQ_PER_TENSOR_SYMMETRIC
                        : SGQ_PER_CHANNEL_SYMMETRIC;
    if (eff == SGQ_PER_CHANNEL_SYMMETRIC && v.rows == 0)
        throw std::runtime_error("quantize_int8: per-channel quantization of a tensor with no rows");
    const Tensor xg = on_gpu(x);
    QuantizedTensor r;
    r.original_shape = x.shape();
    r.scheme = scheme;
    r.bits = 8;
    r.group_size = x.numel();
    Tensor qd = Tensor::empty(x.shape(), Device::CUDA);
    Tensor sc = Tensor::empty({eff == SGQ_PER_TENSOR_SYMMETRIC ? 1 : v.rows}, Device::CUDA);
    auto codes = gpu_bytes(sgq_int8_packed_bytes(v.rows, v.cols));
    const int64_t wsb = sgq_quantize_workspace_bytes(8, v.rows, v.cols, 0);
    auto ws = gpu_bytes(wsb);
    SG_SGQ_CHECK(sgq_quantize_int8(xg.data(), v.rows, v.cols, eff, qd.data(), sc.data(), codes->ptr, ws->ptr, wsb,
                                   nullptr));
    r.qdata = to_device(qd, x.device());
    r.scales = to_device(sc, x.device());
    PackedWeight& p = *r.packed;
    p.codes = codes;
    p.scales_dev = sc;
    record(p, r);
    return r;
}

QuantizedTensor quantize_int4(const Tensor& x, int64_t group_size) {
    if (group_size <= 0) group_size = 32;  // src/quantization.cpp:118
    const View2D v = view2d(x.shape());
    const Tensor xg = on_gpu(x);
    QuantizedTensor r;
    r.original_shape = x.shape();
    r.scheme = QuantizationScheme::GroupedAsymmetric;
    r.bits = 4;
    r.group_size = group_size;
    const int64_t ngroups = sgq_int4_scale_count(v.rows, v.cols, group_size);
    Tensor qd = Tensor::empty(x.shape(), Device::CUDA);
    Tensor sc = Tensor::empty({ngroups}, Device::CUDA);
    auto codes = gpu_bytes(sgq_int4_packed_bytes(v.rows, v.cols, group_size));
    const int64_t nds = sgq_int4_devscale_count(v.rows, v.cols, group_size);
    Tensor ds = Tensor::empty({nds > 4 ? nds : 4}, Device::CUDA);
    const int64_t wsb = sgq_quantize_workspace_bytes(4, v.rows, v.cols, group_size);
    auto ws = gpu_bytes(wsb);
    SG_SGQ_CHECK(sgq_quantize_int4(xg.data(), v.rows, v.cols, group_size, qd.data(), sc.data(), codes->ptr, ds.data(),
                                   ws->ptr, wsb, nullptr));
    r.qdata = to_device(qd, x.device());
    r.scales = to_device(sc, x.device());
    PackedWeight& p = *r.packed;
    p.codes = codes;
    p.devscales = ds;
    p.scales_dev = sc;
    record(p, r);
    return r;
}

namespace {
Tensor dequantize_codes(const QuantizedTensor& qx, int bits, int branch) {
    const View2D v = view2d(qx.original_shape);
    const Tensor qg = on_gpu(qx.qdata);
    const Tensor sg = on_gpu(qx.scales);
    Tensor out = Tensor::empty(qx.original_shape, Device::CUDA);
    SG_SGQ_CHECK(sgq_dequantize_codes(qg.data(), sg.data(), bits, branch, v.rows, v.cols, qx.group_size, out.data(),
                                      nullptr));
    return to_device(out, qx.qdata.device());
}
}  // namespace

Tensor dequantize_int8(const QuantizedTensor& qx) { return dequantize_codes(qx, 8, int8_branch(qx)); }

Tensor dequantize_int4(const QuantizedTensor& qx) { return dequantize_codes(qx, 4, 0); }

Tensor quantized_matmul_int8(const Tensor& x, const QuantizedTensor& q_weight, const Tensor& bias) {
    View2D v{};
    check_linear_args(x, q_weight, bias, v);
    const PackedView p = packed_of(q_weight);
    const Tensor xg = on_gpu(x);
    const Tensor bg = bias.defined() ? on_gpu(bias) : Tensor();
    const int64_t M = x.shape()[0];
    Tensor y = Tensor::empty({M, v.cols}, Device::CUDA);
    // The workspace the library asks for (none for the current kernels), from
    // the device pool; stream order keeps a later reuse behind this launch.
    const int64_t wsb = sgq_linear_workspace_bytes(8, M, v.rows, v.cols);
    const std::shared_ptr<Storage> ws = wsb > 0 ? gpu_bytes(wsb) : nullptr;
    SG_SGQ_CHECK(sgq_linear_int8(xg.data(), M, v.rows, v.cols, p.codes->ptr, std::as_const(p.scales_dev).data(),
                                 int8_branch(q_weight),
                                 bg.defined() ? bg.data() : nullptr, y.data(), ws ? ws->ptr : nullptr, wsb, nullptr));
    return to_device(y, x.device());
}

Tensor quantized_matmul_int4(const Tensor& x, const QuantizedTensor& q_weight, const Tensor& bias) {
    View2D v{};
    check_linear_args(x, q_weight, bias, v);
    const PackedView p = packed_of(q_weight);
    const Tensor xg = on_gpu(x);
    const Tensor bg = bias.defined() ? on_gpu(bias) : Tensor();
    const int64_t M = x.shape()[0];
    Tensor y = Tensor::empty({M, v.cols}, Device::CUDA);
    const int64_t wsb = sgq_linear_workspace_bytes(4, M, v.rows, v.cols);
    const std::shared_ptr<Storage> ws = wsb > 0 ? gpu_bytes(wsb) : nullptr;
    SG_SGQ_CHECK(sgq_linear_int4(xg.data(), M, v.rows, v.cols, p.codes->ptr, std::as_const(p.scales_dev).data(),
                                 p.devscales.defined() ? std::as_const(p.devscales).data() : nullptr,
                                 q_weight.group_size,
                                 bg.defined() ? bg.data() : nullptr, y.data(), ws ? ws->ptr : nullptr, wsb, nullptr));
    return to_device(y, x.device());
}

}  // namespace quantization
}  // namespace sovereigngrad
