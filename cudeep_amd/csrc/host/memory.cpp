// MemoryPool and raw device memory helpers of the C++ host API
// (interface of the reference's src/memory.cu:7-97): exact-size caching
// allocator with a mutex and byte counters; synchronous copies when no
// stream is given.  The pool object lives until process exit and is never
// destroyed, so no hipFree runs after the HIP runtime has shut down.  Kernel
// scratch of null-stream launches has a cache of its own (allocate_scratch).
#include "../../../include/cudeep/memory.hpp"

namespace cudeep {

MemoryPool& MemoryPool::instance() {
    static MemoryPool* pool = new MemoryPool();
    return *pool;
}

MemoryPool::~MemoryPool() { release_cached(); }

void* MemoryPool::device_alloc_locked(size_t nbytes) {
    void* ptr = nullptr;
    hipError_t e = hipMalloc(&ptr, nbytes);
    if (e != hipSuccess) {
        // give both caches back to the runtime and retry once
        for (auto* cache : {&free_blocks_, &free_scratch_})
            for (auto& kv : *cache)
                for (void* p : kv.second) (void)hipFree(p);
        free_blocks_.clear();
        free_scratch_.clear();
        cached_bytes_ = 0;
        CUDEEP_CHECK_HIP(hipMalloc(&ptr, nbytes));
    }
    return ptr;
}

void* MemoryPool::allocate(size_t nbytes) {
    if (nbytes == 0) return nullptr;
    std::lock_guard<std::mutex> lock(mutex_);
    void* ptr = nullptr;
    auto it = free_blocks_.find(nbytes);
    if (it != free_blocks_.end() && !it->second.empty()) {
        ptr = it->second.back();
        it->second.pop_back();
        cached_bytes_ -= nbytes;
    } else {
        ptr = device_alloc_locked(nbytes);
    }
    allocated_blocks_[ptr] = nbytes;
    allocated_bytes_ += nbytes;
    return ptr;
}

void MemoryPool::deallocate(void* ptr) {
    if (!ptr) return;
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = allocated_blocks_.find(ptr);
    if (it == allocated_blocks_.end()) throw std::runtime_error("MemoryPool: unknown pointer");
    const size_t n = it->second;
    allocated_blocks_.erase(it);
    allocated_bytes_ -= n;
    free_blocks_[n].push_back(ptr);
    cached_bytes_ += n;
}

void* MemoryPool::allocate_scratch(size_t nbytes) {
    if (nbytes == 0) return nullptr;
    std::lock_guard<std::mutex> lock(mutex_);
    void* ptr = nullptr;
    auto it = free_scratch_.find(nbytes);
    if (it != free_scratch_.end() && !it->second.empty()) {
        ptr = it->second.back();
        it->second.pop_back();
        cached_bytes_ -= nbytes;
    } else {
        ptr = device_alloc_locked(nbytes);
    }
    scratch_blocks_[ptr] = nbytes;
    allocated_bytes_ += nbytes;
    return ptr;
}

void MemoryPool::deallocate_scratch(void* ptr) {
    if (!ptr) return;
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = scratch_blocks_.find(ptr);
    if (it == scratch_blocks_.end()) throw std::runtime_error("MemoryPool: unknown scratch pointer");
    const size_t n = it->second;
    scratch_blocks_.erase(it);
    allocated_bytes_ -= n;
    free_scratch_[n].push_back(ptr);
    cached_bytes_ += n;
}

void MemoryPool::release_cached() {
    std::lock_guard<std::mutex> lock(mutex_);
    for (auto* cache : {&free_blocks_, &free_scratch_})
        for (auto& kv : *cache)
            for (void* p : kv.second) (void)hipFree(p);
    free_blocks_.clear();
    free_scratch_.clear();
    cached_bytes_ = 0;
}

void* device_malloc(size_t nbytes) { return MemoryPool::instance().allocate(nbytes); }

void device_free(void* ptr) { MemoryPool::instance().deallocate(ptr); }

static void copy(void* dst, const void* src, size_t nbytes, hipMemcpyKind kind, hipStream_t s) {
    if (nbytes == 0) return;
    if (s) {
        CUDEEP_CHECK_HIP(hipMemcpyAsync(dst, src, nbytes, kind, s));
    } else {
        CUDEEP_CHECK_HIP(hipMemcpy(dst, src, nbytes, kind));
    }
}

void memcpy_h2d(void* dst, const void* src, size_t nbytes, hipStream_t stream) {
    copy(dst, src, nbytes, hipMemcpyHostToDevice, stream);
}

void memcpy_d2h(void* dst, const void* src, size_t nbytes, hipStream_t stream) {
    copy(dst, src, nbytes, hipMemcpyDeviceToHost, stream);
}

void memcpy_d2d(void* dst, const void* src, size_t nbytes, hipStream_t stream) {
    copy(dst, src, nbytes, hipMemcpyDeviceToDevice, stream);
}

}  // namespace cudeep
