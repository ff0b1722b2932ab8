// tensor.hpp -- the subset of the reference's Tensor that the quantized
// inference path touches (include/sovereigngrad/tensor.hpp:34-206): fp32
// contiguous storage on the host or the GPU, factories, device transfer,
// clone, element access, a CPU matmul and elementwise add.  Autograd, views
// and the other ops are out of scope for this build.
#pragma once

#include "sovereigngrad/allocator.hpp"

#include <atomic>
#include <cstdint>
#include <initializer_list>
#include <memory>
#include <string>
#include <vector>

namespace sovereigngrad {

enum class DType { Float32, Float16, Int32, Int64 };

std::string dtype_to_string(DType d);

// Raw memory owned through the caching allocator; zero-filled on creation
// like the reference's Storage (src/tensor.cpp:33-42).
struct Storage {
    void* ptr = nullptr;
    size_t size = 0;  // bytes
    Device device = Device::CPU;
    Storage(size_t size, Device device, bool zero_fill = true);
    ~Storage();
    Storage(const Storage&) = delete;
    Storage& operator=(const Storage&) = delete;
};

struct TensorImpl {
    std::shared_ptr<Storage> storage;
    std::vector<int64_t> shape;
    Device device = Device::CPU;
    DType dtype = DType::Float32;
    bool requires_grad = false;
    // Bumped by every in-place write: copy_from (load_state_dict) and every
    // mutable data() access through Tensor.  Atomic: forwards on several host
    // threads read it while packing weights.
    std::atomic<uint64_t> version{0};
    // Unique for the life of the process (a new impl never reuses an old id,
    // even at the same address), so caches can key on it.
    const uint64_t id;

    TensorImpl(const std::vector<int64_t>& shape, Device device, bool requires_grad = false, bool zero_fill = true);
    float* data() { return storage ? static_cast<float*>(storage->ptr) : nullptr; }
    const float* data() const { return storage ? static_cast<const float*>(storage->ptr) : nullptr; }
    int64_t numel() const;
    void bump_version() { version.fetch_add(1, std::memory_order_acq_rel); }
};

class Tensor {
public:
    std::shared_ptr<TensorImpl> impl;

    Tensor() = default;
    explicit Tensor(std::shared_ptr<TensorImpl> i) : impl(std::move(i)) {}
    Tensor(const std::vector<int64_t>& shape, Device device = Device::CPU, bool requires_grad = false);
    Tensor(float scalar, Device device = Device::CPU, bool requires_grad = false);
    Tensor(const std::vector<float>& data, const std::vector<int64_t>& shape, Device device = Device::CPU,
           bool requires_grad = false);

    static Tensor zeros(const std::vector<int64_t>& shape, Device device = Device::CPU, bool requires_grad = false);
    static Tensor ones(const std::vector<int64_t>& shape, Device device = Device::CPU, bool requires_grad = false);
    static Tensor full(const std::vector<int64_t>& shape, float value, Device device = Device::CPU,
                       bool requires_grad = false);
    // N(mean, std) draws.  The reference seeds from std::random_device
    // (src/tensor.cpp:136-153); here the default engine is process-global and
    // reseedable with manual_seed for reproducible tests.
    static Tensor randn(const std::vector<int64_t>& shape, float mean = 0.0f, float std = 1.0f,
                        Device device = Device::CPU, bool requires_grad = false);
    static void manual_seed(uint64_t seed);
    // An uninitialised tensor (no zero fill) for outputs that are fully written.
    static Tensor empty(const std::vector<int64_t>& shape, Device device = Device::CPU);

    const std::vector<int64_t>& shape() const { return impl->shape; }
    Device device() const { return impl->device; }
    DType dtype() const { return impl ? impl->dtype : DType::Float32; }
    int64_t numel() const { return impl ? impl->numel() : 0; }
    bool is_contiguous() const { return true; }
    bool is_defined() const { return impl != nullptr; }
    bool defined() const { return impl != nullptr; }
    uint64_t version() const { return impl ? impl->version.load(std::memory_order_acquire) : 0; }
    uint64_t id() const { return impl ? impl->id : 0; }
    bool requires_grad() const { return impl && impl->requires_grad; }
    // Mutable access counts as a write: it bumps the version, so a quantized
    // layer whose qdata or scales are changed through it repacks its device
    // weight on the next forward (the reference re-reads qdata every call).
    float* data() {
        if (!impl) return nullptr;
        impl->bump_version();
        return impl->data();
    }
    const float* data() const { return impl ? impl->data() : nullptr; }

    Tensor to(Device device) const;
    Tensor cpu() const { return to(Device::CPU); }
    Tensor cuda() const { return to(Device::CUDA); }
    Tensor contiguous() const { return *this; }
    Tensor clone() const;
    // Copies src's elements into this tensor's storage (same numel; any devices)
    // and bumps the version.
    void copy_from(const Tensor& src);

    // y = this . other for 2-D fp32 tensors, computed on the host (the fp32
    // Linear layer is not part of the quantized path).
    Tensor matmul(const Tensor& other) const;
    // Elementwise add with the broadcasting the bias add needs ([M,N] + [1,N]).
    Tensor operator+(const Tensor& other) const;
    Tensor operator-(const Tensor& other) const;

    float item() const;
    float get_element(const std::vector<int64_t>& indices) const;
    std::string summary() const;
};

int64_t compute_numel(const std::vector<int64_t>& shape);

}  // namespace sovereigngrad
