// RAII HIP stream / event (interface of include/cudeep/stream.cuh:8-44).
// Streams are created at the default priority.
#pragma once

#include "common.hpp"
#include "error.hpp"

namespace cudeep {

class Stream {
public:
    Stream();
    ~Stream();
    Stream(const Stream&) = delete;
    Stream& operator=(const Stream&) = delete;
    Stream(Stream&& other) noexcept;
    Stream& operator=(Stream&& other) noexcept;

    hipStream_t get() const { return stream_; }
    void synchronize();

    static Stream& default_stream();

private:
    explicit Stream(hipStream_t s, bool owns) : stream_(s), owns_(owns) {}
    hipStream_t stream_ = nullptr;
    bool owns_ = true;
};

class Event {
public:
    Event();
    ~Event();
    Event(const Event&) = delete;
    Event& operator=(const Event&) = delete;

    void record(hipStream_t stream = nullptr);
    void synchronize();
    float elapsed_ms(const Event& start) const;
    hipEvent_t get() const { return event_; }

private:
    hipEvent_t event_ = nullptr;
};

}  // namespace cudeep
