// allocator.hpp -- caching allocator for host and MI355X device memory.
//
// Same interface as the reference's MemoryAllocator
// (include/sovereigngrad/allocator.hpp:28-69); the device side is a HIP pool
// instead of the CUDA one.  Differences, all deliberate:
//   * best-fit lookup is an ordered map (log n), not a linear scan, and freeing
//     merges only the freed block with its neighbours;
//   * block sizes are rounded up to 256 bytes, so every pointer handed out is
//     256-byte aligned (the packed-weight kernels need 16);
//   * running out of device memory first returns cached segments to the
//     driver and retries, then throws std::runtime_error -- it never calls
//     back into a locked accessor (the reference's OOM path deadlocks on its
//     own mutex, src/allocator.cpp:37,95,184).
//
// Stream order: a freed device block is cached at once and may be handed to
// the next allocate() while kernels that use it are still queued.  That is
// safe because every launch of the host layer goes to the default stream, in
// order, like the reference's CUDA path: work queued on the freed block runs
// before any work queued later on its new owner.  A caller that launches on
// other streams must synchronise them before freeing memory they use (the
// same contract as the reference's pool, which also reuses without events).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>

namespace sovereigngrad {

// CUDA is kept as the name of the accelerator enumerator so that code written
// against the reference compiles unchanged; GPU is the same device.
enum class Device { CPU, CUDA, GPU = CUDA };

inline std::string device_to_string(Device d) { return d == Device::CPU ? "CPU" : "CUDA"; }

class MemoryAllocator {
public:
    static MemoryAllocator& instance();

    // Allocate memory on the specified device (nullptr for 0 bytes).
    void* allocate(size_t bytes, Device device);
    // Return memory to the cache.
    void free(void* ptr, Device device);
    // Return every cached (free) segment to the OS / driver.
    void release_all();

    size_t active_allocations(Device device) const;
    size_t cached_allocations(Device device) const;
    size_t total_memory_allocated(Device device) const;  // bytes managed (active + cached)
    size_t peak_memory_allocated(Device device) const;   // peak bytes in use
    void reset_peak_memory_stats();
    std::string get_memory_summary(Device device) const;

    ~MemoryAllocator();
    MemoryAllocator(const MemoryAllocator&) = delete;
    MemoryAllocator& operator=(const MemoryAllocator&) = delete;

private:
    MemoryAllocator() = default;

    struct Block {
        char* ptr = nullptr;
        size_t size = 0;
        bool in_use = false;
        Block* prev = nullptr;  // neighbours inside the same segment
        Block* next = nullptr;
        char* segment = nullptr;  // base of the driver allocation
    };
    struct Pool {
        std::multimap<size_t, Block*> free_by_size;
        std::unordered_map<char*, Block*> by_ptr;  // every block, keyed by address
        size_t in_use_bytes = 0;
        size_t managed_bytes = 0;
        size_t peak_bytes = 0;
        size_t active_count = 0;
    };

    Pool& pool(Device d) { return d == Device::CPU ? cpu_ : gpu_; }
    const Pool& pool(Device d) const { return d == Device::CPU ? cpu_ : gpu_; }
    void* allocate_locked(size_t bytes, Device device);
    void release_free_segments_locked(Device device);
    void erase_free(Pool& p, Block* b);
    static char* raw_alloc(size_t bytes, Device device);
    static void raw_free(char* p, Device device);

    Pool cpu_, gpu_;
    mutable std::mutex mutex_;
};

}  // namespace sovereigngrad
