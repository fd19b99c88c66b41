// Device memory for the C++ host API.  Same interface as the reference's
// MemoryPool / device_malloc / memcpy_* (include/cudeep/memory.cuh:13-45):
// a process-wide caching allocator keyed by exact size, mutex-protected,
// with allocated / cached byte counters.  The pool returns blocks of the
// current HIP device; with stream == nullptr the copies are synchronous.
#pragma once

#include <cstddef>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.hpp"
#include "error.hpp"

namespace cudeep {

class MemoryPool {
public:
    static MemoryPool& instance();

    void* allocate(size_t nbytes);
    void deallocate(void* ptr);
    // Kernel scratch of launches on the null stream (a separate exact-size
    // cache): a block returned while the launch that used it may still run
    // goes only to later null-stream launches, which the null stream orders
    // after it -- never to tensor storage, which may be written from a
    // non-blocking stream at once.
    void* allocate_scratch(size_t nbytes);
    void deallocate_scratch(void* ptr);
    void release_cached();
    size_t allocated_bytes() const { return allocated_bytes_; }
    size_t cached_bytes() const { return cached_bytes_; }

    MemoryPool(const MemoryPool&) = delete;
    MemoryPool& operator=(const MemoryPool&) = delete;

private:
    MemoryPool() = default;
    ~MemoryPool();

    // hipMalloc, retrying once after giving the cached blocks back.
    // Caller holds mutex_.
    void* device_alloc_locked(size_t nbytes);

    std::unordered_map<size_t, std::vector<void*>> free_blocks_;
    std::unordered_map<size_t, std::vector<void*>> free_scratch_;
    std::unordered_map<void*, size_t> scratch_blocks_;
    std::unordered_map<void*, size_t> allocated_blocks_;
    std::mutex mutex_;
    size_t allocated_bytes_ = 0;
    size_t cached_bytes_ = 0;
};

void* device_malloc(size_t nbytes);
void device_free(void* ptr);
void memcpy_h2d(void* dst, const void* src, size_t nbytes, hipStream_t stream = nullptr);
void memcpy_d2h(void* dst, const void* src, size_t nbytes, hipStream_t stream = nullptr);
void memcpy_d2d(void* dst, const void* src, size_t nbytes, hipStream_t stream = nullptr);

}  // namespace cudeep
