// tensor.cpp -- fp32 tensors on the host or the GPU (the subset of the
// reference's Tensor used by the quantized path; see tensor.hpp).
#include "sovereigngrad/tensor.hpp"

#include <cstdint>
#include <cmath>
#include <cstring>
#include <mutex>
#include <random>
#include <sstream>
#include <stdexcept>

#include "hip_check.hpp"

namespace sovereigngrad {

std::string dtype_to_string(DType d) {
    switch (d) {
        case DType::Float32: return "Float32";
        case DType::Float16: return "Float16";
        case DType::Int32: return "Int32";
        case DType::Int64: return "Int64";
    }
    return "Unknown";
}

int64_t compute_numel(const std::vector<int64_t>& shape) {
    int64_t n = 1;
    for (int64_t d : shape) {
        if (d < 0) throw std::runtime_error("negative dimension in tensor shape");
        if (d != 0 && n > INT64_MAX / d) throw std::runtime_error("tensor shape overflows int64 element count");
        n *= d;
    }
    return n;
}

Storage::Storage(size_t bytes, Device dev, bool zero_fill) : size(bytes), device(dev) {
    ptr = MemoryAllocator::instance().allocate(bytes, dev);
    if (zero_fill && ptr) {
        if (dev == Device::CPU)
            std::memset(ptr, 0, bytes);
        else
            SG_HIP_CHECK(hipMemset(ptr, 0, bytes));
    }
}

Storage::~Storage() { MemoryAllocator::instance().free(ptr, device); }

namespace {
std::atomic<uint64_t> g_next_impl_id{1};
}  // namespace

TensorImpl::TensorImpl(const std::vector<int64_t>& shp, Device dev, bool req, bool zero_fill)
    : shape(shp), device(dev), requires_grad(req), id(g_next_impl_id.fetch_add(1, std::memory_order_relaxed)) {
    storage = std::make_shared<Storage>(static_cast<size_t>(compute_numel(shp)) * sizeof(float), dev, zero_fill);
}

int64_t TensorImpl::numel() const { return compute_numel(shape); }

namespace {

std::mutex g_rng_mu;
std::mt19937_64& rng() {
    static std::mt19937_64 eng(std::random_device{}());
    return eng;
}

void copy_bytes(void* dst, Device ddev, const void* src, Device sdev, size_t bytes) {
    if (bytes == 0) return;
    if (ddev == Device::CPU && sdev == Device::CPU) {
        std::memcpy(dst, src, bytes);
        return;
    }
    hipMemcpyKind kind = ddev == Device::CPU ? hipMemcpyDeviceToHost
                         : (sdev == Device::CPU ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice);
    SG_HIP_CHECK(hipMemcpy(dst, src, bytes, kind));
}

Tensor from_host_values(const std::vector<float>& v, const std::vector<int64_t>& shape, Device dev, bool req) {
    if ((int64_t)v.size() != compute_numel(shape)) throw std::runtime_error("data size does not match shape");
    Tensor t(std::make_shared<TensorImpl>(shape, dev, req, false));
    copy_bytes(t.data(), dev, v.data(), Device::CPU, v.size() * sizeof(float));
    return t;
}

}  // namespace

Tensor::Tensor(const std::vector<int64_t>& shape, Device device, bool requires_grad)
    : impl(std::make_shared<TensorImpl>(shape, device, requires_grad, true)) {}

Tensor::Tensor(float scalar, Device device, bool requires_grad) {
    *this = from_host_values({scalar}, {1}, device, requires_grad);
}

Tensor::Tensor(const std::vector<float>& data, const std::vector<int64_t>& shape, Device device, bool requires_grad) {
    *this = from_host_values(data, shape, device, requires_grad);
}

Tensor Tensor::zeros(const std::vector<int64_t>& shape, Device device, bool requires_grad) {
    return Tensor(shape, device, requires_grad);
}

Tensor Tensor::ones(const std::vector<int64_t>& shape, Device device, bool requires_grad) {
    return full(shape, 1.0f, device, requires_grad);
}

Tensor Tensor::full(const std::vector<int64_t>& shape, float value, Device device, bool requires_grad) {
    return from_host_values(std::vector<float>((size_t)compute_numel(shape), value), shape, device, requires_grad);
}

Tensor Tensor::randn(const std::vector<int64_t>& shape, float mean, float std, Device device, bool requires_grad) {
    std::vector<float> v((size_t)compute_numel(shape));
    {
        std::lock_guard<std::mutex> lock(g_rng_mu);
        std::normal_distribution<float> dist(mean, std);
        for (auto& e : v) e = dist(rng());
    }
    return from_host_values(v, shape, device, requires_grad);
}

void Tensor::manual_seed(uint64_t seed) {
    std::lock_guard<std::mutex> lock(g_rng_mu);
    rng().seed(seed);
}

Tensor Tensor::empty(const std::vector<int64_t>& shape, Device device) {
    return Tensor(std::make_shared<TensorImpl>(shape, device, false, false));
}

Tensor Tensor::to(Device device) const {
    if (!impl) return Tensor();
    if (device == impl->device) return *this;
    Tensor t(std::make_shared<TensorImpl>(impl->shape, device, impl->requires_grad, false));
    copy_bytes(t.data(), device, data(), impl->device, (size_t)numel() * sizeof(float));
    return t;
}

Tensor Tensor::clone() const {
    if (!impl) return Tensor();
    Tensor t(std::make_shared<TensorImpl>(impl->shape, impl->device, impl->requires_grad, false));
    copy_bytes(t.data(), impl->device, data(), impl->device, (size_t)numel() * sizeof(float));
    return t;
}

void Tensor::copy_from(const Tensor& src) {
    if (!impl || !src.impl) throw std::runtime_error("copy_from on an undefined tensor");
    if (src.numel() != numel()) throw std::runtime_error("copy_from: element counts differ");
    copy_bytes(impl->data(), impl->device, src.data(), src.device(), (size_t)numel() * sizeof(float));
    impl->bump_version();  // one write, one version
}

Tensor Tensor::matmul(const Tensor& other) const {
    if (shape().size() != 2 || other.shape().size() != 2)
        throw std::runtime_error("matmul currently requires 2D tensors!");
    const int64_t M = shape()[0], K = shape()[1], N = other.shape()[1];
    if (other.shape()[0] != K) throw std::runtime_error("Matrix inner dimensions must match for matmul!");
    Tensor a = cpu(), b = other.cpu();
    Tensor out = Tensor::zeros({M, N}, Device::CPU);
    const float* pa = a.data();
    const float* pb = b.data();
    float* po = out.data();
    for (int64_t i = 0; i < M; ++i)
        for (int64_t k = 0; k < K; ++k) {
            const float aik = pa[i * K + k];
            for (int64_t j = 0; j < N; ++j) po[i * N + j] = std::fma(aik, pb[k * N + j], po[i * N + j]);
        }
    return out.to(device());
}

namespace {
Tensor elementwise(const Tensor& a, const Tensor& b, bool subtract) {
    const auto& sa = a.shape();
    const auto& sb = b.shape();
    const int64_t na = a.numel(), nb = b.numel();
    const bool same = na == nb;
    const int64_t cols = sa.empty() ? 1 : sa.back();
    const bool row_bcast = !same && nb == cols && (sb.size() <= 1 || compute_numel(sb) == sb.back());
    if (!same && !row_bcast && nb != 1) throw std::runtime_error("Incompatible shapes for elementwise op");
    Tensor ca = a.cpu(), cb = b.cpu();
    Tensor out = Tensor::empty(sa, Device::CPU);
    for (int64_t i = 0; i < na; ++i) {
        const float vb = same ? cb.data()[i] : (row_bcast ? cb.data()[i % cols] : cb.data()[0]);
        out.data()[i] = subtract ? ca.data()[i] - vb : ca.data()[i] + vb;
    }
    return out.to(a.device());
}
}  // namespace

Tensor Tensor::operator+(const Tensor& other) const { return elementwise(*this, other, false); }
Tensor Tensor::operator-(const Tensor& other) const { return elementwise(*this, other, true); }

float Tensor::item() const {
    if (numel() != 1) throw std::runtime_error("item() needs a one-element tensor");
    return cpu().data()[0];
}

float Tensor::get_element(const std::vector<int64_t>& indices) const {
    if (indices.size() != shape().size()) throw std::runtime_error("get_element: wrong number of indices");
    int64_t flat = 0;
    for (size_t i = 0; i < indices.size(); ++i) {
        if (indices[i] < 0 || indices[i] >= shape()[i]) throw std::runtime_error("get_element: index out of range");
        flat = flat * shape()[i] + indices[i];
    }
    float v = 0.0f;
    copy_bytes(&v, Device::CPU, data() + flat, device(), sizeof(float));
    return v;
}

std::string Tensor::summary() const {
    std::ostringstream ss;
    ss << "Tensor(shape=[";
    for (size_t i = 0; i < shape().size(); ++i) ss << (i ? ", " : "") << shape()[i];
    ss << "], device=" << device_to_string(device()) << ", dtype=" << dtype_to_string(dtype()) << ")";
    return ss.str();
}

}  // namespace sovereigngrad
