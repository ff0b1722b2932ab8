// allocator.cpp -- caching allocator with a HIP device pool.  See
// include/sovereigngrad/allocator.hpp for how it differs from the reference's
// (src/allocator.cpp:34-247).
#include "sovereigngrad/allocator.hpp"

#include <cstdlib>
#include <cstring>
#include <new>
#include <sstream>
#include <stdexcept>

#include "hip_check.hpp"

namespace sovereigngrad {

namespace {
constexpr size_t kAlign = 256;                 // every block starts 256-byte aligned
constexpr size_t kMinSplit = 1024;             // split a cached block when >= 1 KiB would remain
constexpr size_t kMinGpuSegment = 1u << 20;    // 1 MiB device segments (src/allocator.cpp:81)
constexpr size_t kMinCpuSegment = 4096;        // 4 KiB host segments
size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
}  // namespace

MemoryAllocator& MemoryAllocator::instance() {
    static MemoryAllocator* inst = new MemoryAllocator();  // never destroyed: outlives every Storage
    return *inst;
}

MemoryAllocator::~MemoryAllocator() { release_all(); }

char* MemoryAllocator::raw_alloc(size_t bytes, Device device) {
    if (device == Device::CPU) return static_cast<char*>(std::aligned_alloc(kAlign, round_up(bytes, kAlign)));
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();  // clear the sticky error of the failed allocation
        return nullptr;
    }
    return static_cast<char*>(p);
}

void MemoryAllocator::raw_free(char* p, Device device) {
    if (device == Device::CPU)
        std::free(p);
    else
        (void)hipFree(p);
}

void MemoryAllocator::erase_free(Pool& p, Block* b) {
    auto range = p.free_by_size.equal_range(b->size);
    for (auto it = range.first; it != range.second; ++it) {
        if (it->second == b) {
            p.free_by_size.erase(it);
            return;
        }
    }
}

void MemoryAllocator::release_free_segments_locked(Device device) {
    Pool& p = pool(device);
    for (auto it = p.free_by_size.begin(); it != p.free_by_size.end();) {
        Block* b = it->second;
        if (b->prev == nullptr && b->next == nullptr) {  // the whole segment is free
            it = p.free_by_size.erase(it);
            p.by_ptr.erase(b->ptr);
            p.managed_bytes -= b->size;
            raw_free(b->segment, device);
            delete b;
        } else {
            ++it;
        }
    }
}

void* MemoryAllocator::allocate_locked(size_t bytes, Device device) {
    Pool& p = pool(device);
    const size_t size = round_up(bytes, kAlign);
    Block* b = nullptr;
    auto it = p.free_by_size.lower_bound(size);  // best fit: smallest cached block that is large enough
    if (it != p.free_by_size.end()) {
        b = it->second;
        p.free_by_size.erase(it);
    } else {
        const size_t seg = std::max(size, device == Device::CPU ? kMinCpuSegment : kMinGpuSegment);
        char* raw = raw_alloc(seg, device);
        if (!raw) {
            release_free_segments_locked(device);  // give cached segments back and retry once
            raw = raw_alloc(seg, device);
        }
        if (!raw) {
            if (device == Device::CPU) throw std::bad_alloc();
            std::ostringstream ss;
            ss << "HIP allocator out of memory: requested " << seg << " bytes, active allocations: "
               << p.active_count << ", bytes in use: " << p.in_use_bytes << ", managed: " << p.managed_bytes;
            throw std::runtime_error(ss.str());
        }
        b = new Block{raw, seg, false, nullptr, nullptr, raw};
        p.by_ptr[raw] = b;
        p.managed_bytes += seg;
    }
    if (b->size - size >= kMinSplit) {
        Block* rest = new Block{b->ptr + size, b->size - size, false, b, b->next, b->segment};
        if (b->next) b->next->prev = rest;
        b->next = rest;
        b->size = size;
        p.by_ptr[rest->ptr] = rest;
        p.free_by_size.emplace(rest->size, rest);
    }
    b->in_use = true;
    p.in_use_bytes += b->size;
    p.active_count += 1;
    if (p.in_use_bytes > p.peak_bytes) p.peak_bytes = p.in_use_bytes;
    return b->ptr;
}

void* MemoryAllocator::allocate(size_t bytes, Device device) {
    if (bytes == 0) return nullptr;
    std::lock_guard<std::mutex> lock(mutex_);
    return allocate_locked(bytes, device);
}

void MemoryAllocator::free(void* ptr, Device device) {
    if (!ptr) return;
    std::lock_guard<std::mutex> lock(mutex_);
    Pool& p = pool(device);
    auto it = p.by_ptr.find(static_cast<char*>(ptr));
    if (it == p.by_ptr.end() || !it->second->in_use) return;  // unknown or already free: ignored
    Block* b = it->second;
    b->in_use = false;
    p.in_use_bytes -= b->size;
    p.active_count -= 1;
    // Merge with free neighbours of the same segment.
    if (b->next && !b->next->in_use) {
        Block* n = b->next;
        erase_free(p, n);
        p.by_ptr.erase(n->ptr);
        b->size += n->size;
        b->next = n->next;
        if (n->next) n->next->prev = b;
        delete n;
    }
    if (b->prev && !b->prev->in_use) {
        Block* pr = b->prev;
        erase_free(p, pr);
        p.by_ptr.erase(b->ptr);
        pr->size += b->size;
        pr->next = b->next;
        if (b->next) b->next->prev = pr;
        delete b;
        b = pr;
    }
    p.free_by_size.emplace(b->size, b);
}

void MemoryAllocator::release_all() {
    std::lock_guard<std::mutex> lock(mutex_);
    release_free_segments_locked(Device::CPU);
    release_free_segments_locked(Device::CUDA);
}

size_t MemoryAllocator::active_allocations(Device device) const {
    std::lock_guard<std::mutex> lock(mutex_);
    return pool(device).active_count;
}

size_t MemoryAllocator::cached_allocations(Device device) const {
    std::lock_guard<std::mutex> lock(mutex_);
    return pool(device).free_by_size.size();
}

size_t MemoryAllocator::total_memory_allocated(Device device) const {
    std::lock_guard<std::mutex> lock(mutex_);
    return pool(device).managed_bytes;
}

size_t MemoryAllocator::peak_memory_allocated(Device device) const {
    std::lock_guard<std::mutex> lock(mutex_);
    return pool(device).peak_bytes;
}

void MemoryAllocator::reset_peak_memory_stats() {
    std::lock_guard<std::mutex> lock(mutex_);
    cpu_.peak_bytes = cpu_.in_use_bytes;
    gpu_.peak_bytes = gpu_.in_use_bytes;
}

std::string MemoryAllocator::get_memory_summary(Device device) const {
    std::lock_guard<std::mutex> lock(mutex_);
    const Pool& p = pool(device);
    size_t cached_bytes = 0;
    for (const auto& kv : p.free_by_size) cached_bytes += kv.first;
    std::ostringstream ss;
    ss << "[" << device_to_string(device) << " Memory Summary] Active: " << p.in_use_bytes / 1024.0 << " KB ("
       << p.active_count << " blocks), Cached: " << cached_bytes / 1024.0 << " KB (" << p.free_by_size.size()
       << " blocks), Peak: " << p.peak_bytes / 1024.0 << " KB";
    return ss.str();
}

}  // namespace sovereigngrad
