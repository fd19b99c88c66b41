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
    // Returns a block that work already enqueued on `stream` may still use:
    // the pool records an event there and hands the block out again only
    // once that event has completed, so a later user on any stream
    // (including non-blocking ones, which do not wait for the null stream)
    // cannot overwrite it while the earlier kernel runs.
    void deallocate_after(void* ptr, hipStream_t stream);
    void release_cached();
    size_t allocated_bytes() const { return allocated_bytes_; }
    size_t cached_bytes() const { return cached_bytes_; }

    MemoryPool(const MemoryPool&) = delete;
    MemoryPool& operator=(const MemoryPool&) = delete;

private:
    MemoryPool() = default;
    ~MemoryPool();

    struct Pending {
        void* ptr;
        size_t nbytes;
        hipEvent_t done;
    };
    // Moves pending blocks whose event has completed (all of them, after
    // waiting, when `wait`) to the free lists.  Caller holds mutex_.
    void reclaim_locked(bool wait);

    std::unordered_map<size_t, std::vector<void*>> free_blocks_;
    std::vector<Pending> pending_;
    std::vector<hipEvent_t> spare_events_;
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
