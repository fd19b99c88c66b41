// MemoryPool and raw device memory helpers of the C++ host API
// (interface of the reference's src/memory.cu:7-97): exact-size caching
// allocator with a mutex and byte counters; synchronous copies when no
// stream is given.  The pool object lives until process exit and is never
// destroyed, so no hipFree runs after the HIP runtime has shut down.  Blocks
// returned with deallocate_after wait behind an event until the work that
// used them has finished.
#include "../../../include/cudeep/memory.hpp"

namespace cudeep {

MemoryPool& MemoryPool::instance() {
    static MemoryPool* pool = new MemoryPool();
    return *pool;
}

MemoryPool::~MemoryPool() { release_cached(); }

void MemoryPool::reclaim_locked(bool wait) {
    size_t kept = 0;
    for (Pending& p : pending_) {
        const hipError_t e = wait ? hipEventSynchronize(p.done) : hipEventQuery(p.done);
        if (e == hipErrorNotReady) {
            pending_[kept++] = p;
            continue;
        }
        CUDEEP_CHECK_HIP(e);
        free_blocks_[p.nbytes].push_back(p.ptr);
        spare_events_.push_back(p.done);
    }
    pending_.resize(kept);
}

void* MemoryPool::allocate(size_t nbytes) {
    if (nbytes == 0) return nullptr;
    std::lock_guard<std::mutex> lock(mutex_);
    if (!pending_.empty()) reclaim_locked(false);
    void* ptr = nullptr;
    auto it = free_blocks_.find(nbytes);
    if (it != free_blocks_.end() && !it->second.empty()) {
        ptr = it->second.back();
        it->second.pop_back();
        cached_bytes_ -= nbytes;
    } else {
        hipError_t e = hipMalloc(&ptr, nbytes);
        if (e != hipSuccess) {
            // give the cache (pending blocks too, once their users are done)
            // back to the runtime and retry once
            reclaim_locked(true);
            for (auto& kv : free_blocks_)
                for (void* p : kv.second) (void)hipFree(p);
            free_blocks_.clear();
            cached_bytes_ = 0;
            CUDEEP_CHECK_HIP(hipMalloc(&ptr, nbytes));
        }
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

void MemoryPool::deallocate_after(void* ptr, hipStream_t stream) {
    if (!ptr) return;
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = allocated_blocks_.find(ptr);
    if (it == allocated_blocks_.end()) throw std::runtime_error("MemoryPool: unknown pointer");
    const size_t n = it->second;
    hipEvent_t ev = nullptr;
    if (!spare_events_.empty()) {
        ev = spare_events_.back();
        spare_events_.pop_back();
    } else {
        CUDEEP_CHECK_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    }
    const hipError_t e = hipEventRecord(ev, stream);
    if (e != hipSuccess) {
        spare_events_.push_back(ev);
        CUDEEP_CHECK_HIP(e);
    }
    allocated_blocks_.erase(it);
    allocated_bytes_ -= n;
    pending_.push_back({ptr, n, ev});
    cached_bytes_ += n;
}

void MemoryPool::release_cached() {
    std::lock_guard<std::mutex> lock(mutex_);
    reclaim_locked(true);
    for (auto& kv : free_blocks_)
        for (void* p : kv.second) (void)hipFree(p);
    free_blocks_.clear();
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
